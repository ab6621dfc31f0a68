"""Writes the frozen vectors in this folder (run from the repository root:
``python tests/golden/make_golden.py``).

The reference keeps no golden-vector files (its tests are seeded-random plus
known answers), so these vectors are produced by the oracle after it has been
pinned by those known answers and closed forms; they freeze small end-to-end
cases of every row of the path so that any later change of the oracle or of the
GPU path shows up as a byte difference:

* nuq.npz    -- K (per-channel, nuq4) and V (per-token, nuq2, clamped rows)
  of a (40, 2, 128) fp16 batch with outliers: codes, outlier values, masks,
  packed bytes and CSR;
* quest.npz  -- page stats of (32, 8, 2, 64) fp16 K, the group-summed bound
  of a (6, 64) query and the top 10 + 3 sinks;
* decode.npz -- float64 attention of a (14, 128) query (GQA 7:1) over two
  selected pages per KV head, one of them the partial last page, of nuq.npz's
  batch dequantised (K: its nuq4 per-channel codes, V: its nuq2 per-token
  codes, outliers exact).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle as O  # noqa: E402


def nuq(rng):
    T, H, D = 40, 2, 128
    x = (rng.standard_t(3, (T, H, D)) * 0.8).astype(np.float16)
    kp = np.sort(rng.standard_normal((H, D, 16)), -1).astype(np.float16)
    ku = np.full((H, D), 1.6, np.float16)
    vp = np.sort(rng.standard_normal((H, 24, 4)), -1).astype(np.float16)
    vu = np.full((H, 24), 1.4, np.float16)
    f = lambda a: a.astype(np.float32)  # noqa: E731
    kc, kv, km = O.pack_k(x, f(kp), f(ku), f(-ku))
    vc, vv, vm = O.pack_v(x, f(vp), f(vu), f(-vu))
    kpk, krp, kcol, kval = O.pack_compact(kc, kv, km, 4)
    vpk, vrp, vcol, vval = O.pack_compact(vc, vv, vm, 2)
    np.savez_compressed(HERE / "nuq.npz", x=x, k_poles=kp, k_upper=ku, v_poles=vp, v_upper=vu,
                        k_codes=kc, k_outv=kv, k_outm=km, v_codes=vc, v_outv=vv, v_outm=vm,
                        k_packed=kpk, k_row_ptr=krp, k_col=kcol, k_val=kval,
                        v_packed=vpk, v_row_ptr=vrp, v_col=vcol, v_val=vval)


def quest(rng):
    P, S, H, D, group = 32, 8, 2, 64, 3
    K = rng.standard_normal((P, S, H, D)).astype(np.float16)
    q = rng.standard_normal((H * group, D)).astype(np.float16)
    mn, mx = O.page_stats(K)
    bound = O.page_bound_group(q.astype(np.float32), mn.astype(np.float32), mx.astype(np.float32),
                               group)
    sel = O.topk_sinks(bound, 10, 3)
    np.savez_compressed(HERE / "quest.npz", K=K, q=q, k_min=mn, k_max=mx, bound=bound, sel=sel,
                        group=np.int64(group), k=np.int64(10), sinks=np.int64(3))


def decode(rng):
    z = np.load(HERE / "nuq.npz")
    T, H, D = z["x"].shape
    group = 7
    kd = O.h2f(O.unpack(z["k_codes"], z["k_outv"], z["k_outm"], z["k_poles"].astype(np.float32), "k"))
    vd = O.h2f(O.unpack(z["v_codes"], z["v_outv"], z["v_outm"], z["v_poles"].astype(np.float32), "v"))
    P = -(-T // 16)
    pad = P * 16 - T
    Kp = np.concatenate([kd, np.zeros((pad, H, D), np.float32)]).reshape(P, 16, H, D)
    Vp = np.concatenate([vd, np.zeros((pad, H, D), np.float32)]).reshape(P, 16, H, D)
    q = rng.standard_normal((H * group, D)).astype(np.float16)
    sel = np.array([[0, 1], [P - 1, P - 1]], np.int64)
    out = O.selected_attention(q.astype(np.float64), Kp, Vp, sel, lambda h: h // group,
                               num_tokens=T)
    np.savez_compressed(HERE / "decode.npz", q=q, sel=sel, group=np.int64(group), out=out)


if __name__ == "__main__":
    rng = np.random.default_rng(20260101)
    nuq(rng)
    quest(rng)
    decode(rng)
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)
