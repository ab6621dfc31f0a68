"""GPU parity of the calibration fit (hkv_kmeans_1d) and of the key / value
calibration built on it, against the oracle on the same inputs.

The fit is bit-exact to the oracle's restatement: the assignments are fp32
compares, the means float64 sums rounded to fp32 (the two sum in different
orders; the fp32 rounding of the mean hides that).  The calibration pipeline
(src/kvquant/calibration.py:126-188 with this build's subsample and fit) is
restated in numpy: quantiles by np.quantile, the same seeded permutation of
the sample axis (drawn by torch on the CPU), the first kmeans_subsample
in-threshold values, the oracle fit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(23)


def _ragged(sizes, dist):
    parts = [(RNG.standard_normal(n) if dist == "normal" else RNG.standard_t(3, n)).astype(np.float32)
             * np.float32(RNG.uniform(0.1, 10)) for n in sizes]
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    return parts, (np.concatenate(parts) if parts else np.zeros(0, np.float32)), off


@pytest.mark.parametrize("k,iters,dist", [(4, 50, "normal"), (16, 50, "t3"), (16, 0, "normal"),
                                          (1, 5, "t3"), (3, 20, "normal")])
def test_kmeans_vs_oracle(dev, k, iters, dist):
    from helix_kv.ops import kmeans_1d

    sizes = [0, 1, k - 1 if k > 1 else 0, k, 17, 100, 2000, 5000, 8192, 9000, 4096]
    parts, vals, off = _ragged(sizes, dist)
    got = kmeans_1d(torch.from_numpy(vals).to(dev), torch.from_numpy(off).to(dev), k, iters)
    got = got.cpu().numpy()
    for i, p in enumerate(parts):
        assert np.array_equal(got[i], O.kmeans_1d(p, k, iters)), (i, sizes[i])


@pytest.mark.parametrize("k,dist", [(4, "normal"), (16, "t3"), (1, "t3"), (3, "normal"), (16, "normal")])
def test_kmeans_optimal_vs_oracle(dev, k, dist):
    """hkv_kmeans_1d_optimal against the oracle's exhaustive DP: bit-exact
    centres for problems of every size class (empty, fewer than k, exactly k,
    up to the 6144-value limit, and past it: NaN), and values with ties."""
    from helix_kv.ops import kmeans_1d_optimal

    sizes = [0, 1, k - 1 if k > 1 else 0, k, 17, 100, 2000, 5000, 6144, 6145, 4096]
    parts, vals, off = _ragged(sizes, dist)
    # a problem with many ties: values on a coarse grid
    tie = (np.round(RNG.standard_normal(1500) * 4) / 4).astype(np.float32)
    parts.append(tie)
    vals = np.concatenate([vals, tie])
    off = np.concatenate([off, [off[-1] + tie.size]]).astype(np.int64)
    got = kmeans_1d_optimal(torch.from_numpy(vals).to(dev), torch.from_numpy(off).to(dev), k)
    got = got.cpu().numpy()
    for i, p in enumerate(parts):
        want = O.kmeans_optimal(p, k)
        if p.size > 6144:
            assert np.isnan(got[i]).all(), i
        else:
            assert np.array_equal(got[i], want), (i, p.size, got[i], want)


def _oracle_rows(X, cfg):
    n = X.shape[1]
    up = np.quantile(X, 1 - cfg.outlier_pct, axis=1)   # float32 rows, as the reference
    lo = np.quantile(X, cfg.outlier_pct, axis=1)
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(cfg.seed)).numpy()
    poles = []
    for r in range(X.shape[0]):
        x = X[r, perm]
        inside = x[(x >= lo[r]) & (x <= up[r])][: cfg.kmeans_subsample]
        if cfg.kmeans_fit == "optimal":
            poles.append(O.kmeans_optimal(inside, 2 ** cfg.num_bits))
        else:
            poles.append(O.kmeans_1d(inside, 2 ** cfg.num_bits, cfg.kmeans_iters))
    return np.stack(poles), up, lo


@pytest.mark.parametrize("bits", [2, 4])
def test_calibrate_keys_and_values_vs_oracle(dev, bits):
    from kvquant.calibration import CalibrationConfig, calibrate_keys, calibrate_values

    cfg = CalibrationConfig(num_bits=bits, kmeans_subsample=700, outlier_pct=0.01, seed=3)
    T, H, D = 2048, 2, 16
    K = (RNG.standard_t(3, (T, H, D)) * RNG.lognormal(0, 0.5, (1, H, D))).astype(np.float16)
    ks = calibrate_keys(torch.from_numpy(K).to(dev), cfg)
    X = K.astype(np.float32).transpose(1, 2, 0).reshape(H * D, T)
    poles, up, lo = _oracle_rows(X, cfg)
    assert np.array_equal(ks.upper_threshold.cpu().numpy(), up.reshape(H, D))
    assert np.array_equal(ks.lower_threshold.cpu().numpy(), lo.reshape(H, D))
    assert np.array_equal(ks.poles.cpu().numpy(), poles.reshape(H, D, -1))
    assert ks.num_bits == bits and ks.poles.shape == (H, D, 2 ** bits)

    Np, S = 4, 64
    V = RNG.standard_t(3, (Np, S, H, 32)).astype(np.float16)
    vs = calibrate_values(torch.from_numpy(V).to(dev), cfg)
    XV = V.astype(np.float32).transpose(2, 1, 0, 3).reshape(H * S, Np * 32)
    poles, up, lo = _oracle_rows(XV, cfg)
    assert np.array_equal(vs.upper_threshold.cpu().numpy(), up.reshape(H, S))
    assert np.array_equal(vs.lower_threshold.cpu().numpy(), lo.reshape(H, S))
    assert np.array_equal(vs.poles.cpu().numpy(), poles.reshape(H, S, -1))


def test_kmeans_errors(dev):
    from helix_kv.ops import kmeans_1d

    v = torch.zeros(8, device=dev)
    off = torch.tensor([0, 8], dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        kmeans_1d(v, off, 17)        # k > 16
    with pytest.raises(ValueError):
        kmeans_1d(v, off, 4, -1)     # negative steps


def test_calibrated_mixed_scales_pack_end_to_end(dev, tmp_path):
    """Calibration -> a spliced nuq2 / nuq4 KVScales -> .pt -> device tables ->
    pack_layer / unpack_layer of each layer, against the oracle's pack and
    compact encoding with each layer's own level count (fp32 scales, as
    calibration writes them)."""
    from kvquant.calibration import CalibrationConfig, calibrate_keys, calibrate_values
    from kvquant.packed import device_tables, pack_layer, unpack_layer
    from kvquant.scales import KVScales

    T, H, D = 512, 2, 128
    layers = []
    for bits in (2, 4):
        cfg = CalibrationConfig(num_bits=bits, kmeans_subsample=400, outlier_pct=0.02)
        K = torch.from_numpy(RNG.standard_t(3, (T, H, D)).astype(np.float16)).to(dev)
        V = torch.from_numpy(RNG.standard_t(3, (2, 64, H, D)).astype(np.float16)).to(dev)
        layers.append(KVScales([calibrate_keys(K, cfg).to("cpu")], [calibrate_values(V, cfg).to("cpu")],
                               num_bits=bits))
    mixed = KVScales(layers[0].per_layer_keys + layers[1].per_layer_keys,
                     layers[0].per_layer_values + layers[1].per_layer_values)
    p = tmp_path / "mixed.pt"
    mixed.save(str(p))
    tabs = device_tables(KVScales.load(str(p)), dev)
    for i, lt in enumerate(tabs):
        ks, vs = mixed.per_layer_keys[i], mixed.per_layer_values[i]
        bits = 2 if ks.poles.shape[-1] <= 4 else 4
        assert lt.k_bits == bits and lt.v_bits == bits
        x = RNG.standard_t(3, (300, H, D)).astype(np.float16)
        y = RNG.standard_t(3, (300, H, D)).astype(np.float16)
        ck, cv = pack_layer(torch.from_numpy(x).to(dev), torch.from_numpy(y).to(dev), lt)
        f = lambda t: t.float().numpy()
        wk = O.pack_k(x, f(ks.poles), f(ks.upper_threshold), f(ks.lower_threshold))
        wv = O.pack_v(y, f(vs.poles), f(vs.upper_threshold), f(vs.lower_threshold))
        for cc, w in ((ck, wk), (cv, wv)):
            pk, rp, col, val = O.pack_compact(*w, bits)
            assert np.array_equal(cc.packed.cpu().numpy(), pk)
            assert np.array_equal(cc.row_ptr.cpu().numpy(), rp)
            assert np.array_equal(cc.col.cpu().numpy(), col)
        ok, ov = unpack_layer(ck, cv, lt)
        assert np.array_equal(ok.cpu().view(torch.int16).numpy().view(np.uint16),
                              O.unpack(*wk, f(ks.poles), "k"))
        assert np.array_equal(ov.cpu().view(torch.int16).numpy().view(np.uint16),
                              O.unpack(*wv, f(vs.poles), "v"))
