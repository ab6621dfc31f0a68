"""The oracle reproduces the frozen vectors of tests/golden/ byte for byte
(regression pin; the vectors are written by tests/golden/make_golden.py)."""
from __future__ import annotations

from pathlib import Path

import numpy as np

import oracle as O

G = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(G / f"{name}.npz")  # allow_pickle=False by default


def test_golden_nuq():
    z = _load("nuq")
    f = lambda a: a.astype(np.float32)  # noqa: E731
    kc, kv, km = O.pack_k(z["x"], f(z["k_poles"]), f(z["k_upper"]), -f(z["k_upper"]))
    vc, vv, vm = O.pack_v(z["x"], f(z["v_poles"]), f(z["v_upper"]), -f(z["v_upper"]))
    for got, name in ((kc, "k_codes"), (kv, "k_outv"), (km, "k_outm"),
                      (vc, "v_codes"), (vv, "v_outv"), (vm, "v_outm")):
        assert np.array_equal(got, z[name]), name
    for got, name in zip(O.pack_compact(kc, kv, km, 4), ("k_packed", "k_row_ptr", "k_col", "k_val")):
        assert np.array_equal(got, z[name]), name
    for got, name in zip(O.pack_compact(vc, vv, vm, 2), ("v_packed", "v_row_ptr", "v_col", "v_val")):
        assert np.array_equal(got, z[name]), name
    assert z["k_outm"].any() and z["v_outm"].any()


def test_golden_quest():
    z = _load("quest")
    mn, mx = O.page_stats(z["K"])
    assert np.array_equal(mn, z["k_min"]) and np.array_equal(mx, z["k_max"])
    b = O.page_bound_group(z["q"].astype(np.float32), mn.astype(np.float32),
                           mx.astype(np.float32), int(z["group"]))
    assert np.array_equal(b, z["bound"])
    assert np.array_equal(O.topk_sinks(b, int(z["k"]), int(z["sinks"])), z["sel"])


def test_golden_decode():
    z, n = _load("decode"), _load("nuq")
    T, H, D = n["x"].shape
    kd = O.h2f(O.unpack(n["k_codes"], n["k_outv"], n["k_outm"], n["k_poles"].astype(np.float32), "k"))
    vd = O.h2f(O.unpack(n["v_codes"], n["v_outv"], n["v_outm"], n["v_poles"].astype(np.float32), "v"))
    P = -(-T // 16)
    pad = P * 16 - T
    Kp = np.concatenate([kd, np.zeros((pad, H, D), np.float32)]).reshape(P, 16, H, D)
    Vp = np.concatenate([vd, np.zeros((pad, H, D), np.float32)]).reshape(P, 16, H, D)
    g = int(z["group"])
    out = O.selected_attention(z["q"].astype(np.float64), Kp, Vp, z["sel"], lambda h: h // g,
                               num_tokens=T)
    assert np.array_equal(out, z["out"])
