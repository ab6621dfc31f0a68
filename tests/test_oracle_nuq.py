"""Pins of the CPU oracle's nuq functions (no GPU).

Each oracle function is checked against something other than itself: the
reference's own known-answer tests, a torch library routine that the case
reduces to, or exhaustive enumeration with an independent numpy restatement.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

RNG = np.random.default_rng(1234)


def _h(x):
    return np.asarray(x, np.float16)


# ------------------------------------------------ reference known answers

def test_known_answer_round_to_nearest_pole():
    # src/kvquant/tests/test_nuq_roundtrip.py:25-31
    poles = [-1.0, -0.5, 0.0, 0.5, 1.0]
    got = [poles[O.nearest_code(v, poles)] for v in [0.1, 0.4, -0.6, 1.2]]
    assert got == [0.0, 0.5, -0.5, 1.0]


def test_known_answer_outlier_band():
    # src/kvquant/tests/test_nuq_roundtrip.py:34-39
    x = _h([[[-2.0, -0.4, 0.1, 0.7, 3.5]]])  # (T=1, H=1, D=5)
    poles = np.zeros((1, 5, 2), np.float32)
    _, _, m = O.pack_k(x, poles, np.ones((1, 5)), -np.ones((1, 5)))
    assert m.reshape(-1).tolist() == [1, 0, 0, 0, 1]


def test_known_answer_outliers_preserved():
    # src/kvquant/tests/test_nuq_roundtrip.py:65-75
    x = _h([-5.0, -0.3, 0.0, 0.4, 7.0]).reshape(1, 1, 5)
    poles = np.broadcast_to(np.array([-0.5, 0.0, 0.5], np.float32), (1, 5, 3)).copy()
    c, v, m = O.pack_k(x, poles, np.ones((1, 5)), -np.ones((1, 5)))
    out = O.h2f(O.unpack(c, v, m, poles, "k")).reshape(-1)
    assert out[0] == -5.0 and out[-1] == 7.0
    assert m.reshape(-1).tolist() == [1, 0, 0, 0, 1]
    assert out[1:4].tolist() == [-0.5, 0.0, 0.5]


def test_known_answer_planted_outlier():
    # src/kvquant/tests/test_triton_kernels.py:120-129
    x = RNG.standard_normal((16, 1, 32)).astype(np.float16)
    x[0, 0, 0] = 99.0
    q = np.quantile(x.astype(np.float32), [0.125, 0.375, 0.625, 0.875], axis=0)[:, 0, :].T
    poles = q[None].astype(np.float16).astype(np.float32)
    up = np.quantile(x.astype(np.float32), 0.99, axis=0).astype(np.float16).astype(np.float32)
    lo = np.quantile(x.astype(np.float32), 0.01, axis=0).astype(np.float16).astype(np.float32)
    c, v, m = O.pack_k(x, poles, up, lo)
    assert m[0, 0, 0] == 1 and O.h2f(v[0, 0, 0]) == 99.0
    assert O.h2f(O.unpack(c, v, m, poles, "k")[0, 0, 0]) == 99.0
    assert c.max() <= 3 and c.min() >= 0  # test_triton_kernels.py:74-81


# --------------------------------------------- torch library routine pins

@pytest.mark.parametrize("L", [4, 16])
def test_codes_equal_torch_argmin(L):
    """Codes are torch.argmin (first minimum) of fp32 |v - pole|."""
    T, H, D = 64, 4, 32
    x = RNG.standard_normal((T, H, D)).astype(np.float16)
    poles = np.sort(RNG.standard_normal((H, D, L)), axis=-1).astype(np.float16).astype(np.float32)
    up = np.full((H, D), 1.5, np.float32)
    c, v, m = O.pack_k(x, poles, up, -up)
    xt = torch.from_numpy(x.astype(np.float32))
    diff = (xt.unsqueeze(-1) - torch.from_numpy(poles).unsqueeze(0)).abs()
    assert np.array_equal(c, diff.argmin(dim=-1).numpy().astype(np.uint8))
    mt = (xt > 1.5) | (xt < -1.5)
    assert np.array_equal(m.astype(bool), mt.numpy())
    assert np.array_equal(v, np.where(m.astype(bool), x.view(np.uint16), 0))


def test_exact_ties_take_lower_level():
    poles = np.array([[[0.0, 1.0, 2.0, 3.0]]], np.float32)
    x = _h([[[0.5, 1.5, 2.5]]]).reshape(3, 1, 1)
    c, _, _ = O.pack_k(x, poles, np.full((1, 1), 9.0), np.full((1, 1), -9.0))
    assert c.reshape(-1).tolist() == [0, 1, 2]
    xt = torch.tensor([0.5, 1.5, 2.5])
    assert (xt[:, None] - torch.tensor([0.0, 1, 2, 3])).abs().argmin(-1).tolist() == [0, 1, 2]


def test_pack_v_clamps_position_rows():
    """Rows beyond the calibrated length reuse row T_cal-1 (compact_pool.py:467)."""
    T, H, D, Tt, L = 40, 2, 16, 8, 4
    x = RNG.standard_normal((T, H, D)).astype(np.float16)
    poles = np.sort(RNG.standard_normal((H, Tt, L)), axis=-1).astype(np.float32)
    up = RNG.uniform(1, 2, (H, Tt)).astype(np.float32)
    pos = np.arange(T) + 3
    c, v, m = O.pack_v(x, poles, up, -up, positions=pos)
    rows = np.minimum(pos, Tt - 1)
    pe = poles[:, rows].transpose(1, 0, 2)  # (T,H,L)
    xt = torch.from_numpy(x.astype(np.float32))
    ref = (xt.unsqueeze(-1) - torch.from_numpy(pe).unsqueeze(2)).abs().argmin(-1).numpy()
    assert np.array_equal(c, ref.astype(np.uint8))
    ue = up[:, rows].T[:, :, None]
    assert np.array_equal(m.astype(bool), (x.astype(np.float32) > ue) | (x.astype(np.float32) < -ue))


def test_roundtrip_error_bound():
    # src/kvquant/tests/test_triton_batched.py:136-151
    T, H, D, L = 256, 4, 32, 16
    x = RNG.standard_normal((T, H, D)).astype(np.float16)
    poles = np.sort(RNG.standard_normal((H, D, L)), axis=-1).astype(np.float16).astype(np.float32)
    sigma = np.abs(x.astype(np.float32)).mean()
    up = np.full((H, D), np.float16(sigma * 1.5), np.float32)
    c, v, m = O.pack_k(x, poles, up, -up)
    rec = O.h2f(O.unpack(c, v, m, poles, "k"))
    mb = m.astype(bool)
    assert np.array_equal(rec[mb], x.astype(np.float32)[mb])
    spacing = np.diff(poles, axis=-1).max()
    assert np.abs(rec - x.astype(np.float32))[~mb].max() <= spacing * 0.51


def test_nuq_py_fp16_semantics_match_torch_half_ops():
    """nuq.py forms |v - p| in fp16 for fp16 inputs: torch's own fp16 ops."""
    v = torch.randn(64, 32).half()
    p = torch.sort(torch.randn(64, 32, 16), dim=-1).values.half()
    up = torch.full((64, 32), 1.2).half()
    codes, recon, mask = O.nuq_py_semantics(v.numpy(), p.numpy(), up.numpy(), (-up).numpy())
    d = (v.unsqueeze(-1) - p).abs()
    assert np.array_equal(codes, d.argmin(-1).numpy())
    q = torch.gather(p, -1, d.argmin(-1, keepdim=True)).squeeze(-1)
    m = (v < -up) | (v > up)
    assert np.array_equal(mask, m.numpy())
    assert np.array_equal(recon.view(np.uint16), torch.where(m, v, q).numpy().view(np.uint16))


# ------------------------------------------- decision tables (exhaustive)

ALL_H = np.arange(65536, dtype=np.uint32).astype(np.uint16)
ALL_F = ALL_H.view(np.float16).astype(np.float32)


def _scan_all(poles):
    """First argmin of fp32 |x - p| for every fp16 x (numpy; NaN rows -> 0)."""
    with np.errstate(invalid="ignore"):
        d = np.abs(ALL_F[:, None] - np.asarray(poles, np.float32)[None, :])
    d = np.where(np.isnan(d), np.inf, d)
    return d.argmin(axis=1)


def _fast_all(t, L):
    """Independent numpy restatement of the fast path: count of breakpoints <= x."""
    bp = O.h2f(t["bp"][: L - 1])
    codes = (ALL_F[:, None] >= bp[None, :]).sum(axis=1)
    ok = (ALL_H & 0x7FFF) <= t["xsafe"]
    if not (t["flags"] & 1):
        ok[:] = False
    return codes, ok


def _tables_to_check():
    out = []
    for i in range(120):
        L = 16 if i % 2 else 4
        scale = 10.0 ** RNG.uniform(-3, 3)
        p = np.sort(RNG.standard_normal(L) * scale).astype(np.float16).astype(np.float32)
        out.append(p)
    out += [np.array(p, np.float32) for p in (
        [0, 0, 1, 1], [1, 1, 1, 1], [-65504, 0, 65504, 65504], [0.001, 0.0011, 0.0012, 0.0013],
        [-3, -2.99951171875, 0, 1e-7], [-1, 0, 0, 0, 1, 1, 1, 2, 2, 3, 3, 3, 4, 5, 6, 7],
        list(np.linspace(-1, 1, 16)), [5, 4, 3, 2],
    )]
    fp32 = np.sort(RNG.standard_normal((20, 16)), axis=1).astype(np.float32)  # fp32 poles
    out += list(fp32)
    return out


def test_fast_tables_exhaustive_c():
    for p in _tables_to_check():
        for up, lo in [(1.5, -1.5), (np.inf, -np.inf), (0.0, 0.0), (0.3333, -0.77777)]:
            bad, cov = O.check_table_exhaustive(p, up, lo)
            assert bad == 0, (p, up, lo)


def test_fast_tables_exhaustive_numpy_and_coverage():
    covered = []
    for p in _tables_to_check():
        L = p.size
        t = O.prep_tables(p[None], [1.0], [-1.0])[0]
        codes, ok = _fast_all(t, L)
        ref = _scan_all(p)
        assert np.array_equal(codes[ok], ref[ok]), p
        if np.all(np.diff(p) > 0) and np.min(np.diff(p)) > 1e-3:
            near = np.abs(ALL_F) <= 2 * np.abs(p).max() + 2
            covered.append(ok[near].mean())
    # well-spread tables: the fast path covers every input in the poles' range
    assert min(covered) == 1.0


def test_fast_tables_flag_unsafe_tables():
    bad_tables = [np.array([3.0, 2.0, 1.0, 0.0], np.float32),        # unsorted
                  np.array([0.0, np.nan, 1.0, 2.0], np.float32),     # NaN pole
                  np.array([0.0, 1.0, np.inf, np.inf], np.float32),  # inf pole
                  np.array([0.0, 2.0 ** -24, 2.0 ** -23, 1.0], np.float32)]  # gaps too small
    t = O.prep_tables(np.stack(bad_tables), np.ones(4), -np.ones(4))
    assert (t["flags"] & 1).tolist() == [0, 0, 0, 0]


def test_planted_breakpoint_error_is_caught():
    """Moving one breakpoint by a single fp16 step must break exhaustive equality."""
    p = np.sort(RNG.standard_normal(16)).astype(np.float16).astype(np.float32)
    t = O.prep_tables(p[None], [1.0], [-1.0])[0].copy()
    t["bp"][7] = np.uint16(int(t["bp"][7]) + 1) if t["bp"][7] < 0x8000 else np.uint16(int(t["bp"][7]) - 1)
    codes, ok = _fast_all(t, 16)
    assert not np.array_equal(codes[ok], _scan_all(p)[ok])


def test_threshold_canonicalisation():
    # outlier iff x < lo || x > up, on fp16 x, for fp32 thresholds
    for up, lo in [(0.1, -0.1), (0.0, 0.0), (np.inf, -np.inf), (1e9, -1e9), (-2.0, 3.0),
                   (np.nan, np.nan), (70000.0, -70000.0)]:
        t = O.prep_tables(np.zeros((1, 4), np.float32), [up], [lo])[0]
        fin = np.isfinite(ALL_F)
        got = (ALL_F < O.h2f(t["lo"])) | (ALL_F > O.h2f(t["up"]))
        with np.errstate(invalid="ignore"):
            ref = (ALL_F < np.float32(lo)) | (ALL_F > np.float32(up))
        assert np.array_equal(got[fin], ref[fin]), (up, lo)


# ------------------------------------------------ bit packing and CSR

def test_bitpack_known_answers():
    assert O.bitpack(np.array([[0, 1, 2, 3]]), 2).tolist() == [[0xE4]]
    assert O.bitpack(np.array([[1, 2]]), 4).tolist() == [[0x21]]
    assert O.bitpack(np.array([[15, 0, 3, 12]]), 4).tolist() == [[0x0F, 0xC3]]


@pytest.mark.parametrize("bits", [2, 4])
def test_bitpack_roundtrip(bits):
    c = RNG.integers(0, 1 << bits, (7, 3, 128)).astype(np.uint8)
    assert np.array_equal(O.bitunpack(O.bitpack(c, bits), bits, 128), c)


def test_csr_known_answer_and_roundtrip():
    m = np.array([[0, 1, 0, 1], [0, 0, 0, 0], [1, 0, 0, 0]], np.uint8)
    v = np.arange(12, dtype=np.float16).reshape(3, 4)
    rp, col, val = O.csr_encode(m, v)
    assert rp.tolist() == [0, 2, 2, 3]
    assert col.tolist() == [1, 3, 0]
    assert O.h2f(val).tolist() == [1.0, 3.0, 8.0]
    m2, v2 = O.csr_decode(rp, col, val, 3, 4)
    assert np.array_equal(m2, m)
    assert np.array_equal(O.h2f(v2)[m.astype(bool)], v.astype(np.float32)[m.astype(bool)])
