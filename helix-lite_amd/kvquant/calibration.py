"""nuq scale calibration on the GPU: the offline step that feeds the KV-cache path.

The reference calibrates on the CPU (src/kvquant/calibration.py:126-188).  For
every (KV head, channel) of K over all calibration tokens, and every (KV head,
position) of V over all prompts and channels, it takes
  - thresholds at the outlier_pct and 1 - outlier_pct quantiles (np.quantile,
    linear interpolation),
  - the values between them (inclusive),
  - at most kmeans_subsample of those, drawn at random,
  - a sklearn k-means with 2**num_bits clusters (_kmeans_1d, :106-123),
one problem at a time: about 17,000 fits per layer at the default config.

Here every problem of a layer runs at once: the quantiles from a per-row sort
(np.quantile's linear rule, in float32 as numpy computes it for the
reference's float32 rows), the in-threshold values
compacted on the device, and the fits in one launch of hkv_kmeans_1d.  Two
steps are this build's own and differ from the reference's:
  - the subsample keeps, per problem, the first kmeans_subsample in-threshold
    values in one seeded permutation of the sample axis (the reference draws
    rng.choice per problem);
  - the fit is the exact optimum of the k-means objective on the subsample
    (hkv_kmeans_1d_optimal: dynamic programming over the sorted values), so
    its inertia is never above that of sklearn's k-means++ with 3 restarts;
    kmeans_fit="lloyd" (or a subsample above 6144) takes kmeans_iters Lloyd
    steps from order statistics instead (hkv_kmeans_1d).
Model loading and the dataset (run_calibration) need network access and are
not part of this build.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from helix_kv.ops import kmeans_1d, kmeans_1d_optimal

from .scales import PerChannelScale, PerTokenScale


OPTIMAL_MAX = 6144  # the largest problem the exact fit takes


@dataclass
class CalibrationConfig:
    """The reference's fields (src/kvquant/calibration.py:45-59) plus the
    GPU fit: "optimal" (exact 1-D k-means by dynamic programming,
    hkv_kmeans_1d_optimal, for kmeans_subsample <= 6144) or "lloyd"
    (kmeans_iters Lloyd steps from order statistics, hkv_kmeans_1d)."""

    model_name: str = "Qwen/Qwen2.5-7B-Instruct-1M"
    num_prompts: int = 32
    seqlen: int = 4096
    num_bits: int = 2
    outlier_pct: float = 0.005
    first_few_fp16: int = 4
    cap_outliers: int = -1
    dataset: str = "wikitext"
    device: str = "cuda:0"
    seed: int = 0
    output_path: str = "scales/qwen2_5_7b_1m_nuq2.pt"
    kmeans_subsample: int = 5000
    log_every_n_layers: int = 1
    progress_log_path: str | None = None
    kmeans_iters: int = 50
    kmeans_fit: str = "optimal"


def row_quantiles(X: torch.Tensor, q: float) -> torch.Tensor:
    """Per row of X (R, n) fp32: the q-quantile exactly as np.quantile
    computes it for a float32 row (the reference's call,
    src/kvquant/calibration.py:141-142, :176-177), all in float32:
      position v = fl32(fl32(n - 1) * fl32(q)), i = floor(v), g = fl32(v - i);
      a, b = sorted[i], sorted[i + 1], d = fl32(b - a);
      result = fl32(a + fl32(d * g)) when g < 0.5, else fl32(b - fl32(d * fl32(1 - g)));
      v >= n - 1 gives the largest value."""
    import numpy as np

    n = int(X.shape[1])
    s = torch.sort(X.float(), dim=1).values
    v = np.float32(n - 1) * np.float32(q)
    if v >= np.float32(n - 1):
        return s[:, n - 1].clone()
    i = int(np.floor(v))
    g = np.float32(v - np.float32(i))
    a, b = s[:, i], s[:, i + 1]
    d = b - a
    if g >= np.float32(0.5):
        return b - d * float(np.float32(1) - g)
    return a + d * float(g)


def _fit_rows(X: torch.Tensor, cfg: CalibrationConfig):
    """X (R, n) fp32 on the GPU -> (poles (R, 2**bits), upper (R,), lower (R,))."""
    R, n = (int(x) for x in X.shape)
    up = row_quantiles(X, 1.0 - cfg.outlier_pct)
    lo = row_quantiles(X, cfg.outlier_pct)
    g = torch.Generator(device="cpu").manual_seed(int(cfg.seed))
    perm = torch.randperm(n, generator=g).to(X.device)
    Xp = X[:, perm]
    inside = (Xp >= lo[:, None]) & (Xp <= up[:, None])
    keep = inside & (torch.cumsum(inside.to(torch.int32), dim=1) <= int(cfg.kmeans_subsample))
    counts = keep.sum(dim=1)
    offsets = torch.zeros(R + 1, dtype=torch.int64, device=X.device)
    offsets[1:] = torch.cumsum(counts, dim=0)
    values = Xp[keep]
    k = 2 ** int(cfg.num_bits)
    if cfg.kmeans_fit == "optimal" and int(cfg.kmeans_subsample) <= OPTIMAL_MAX:
        poles = kmeans_1d_optimal(values, offsets, k)
    elif cfg.kmeans_fit in ("optimal", "lloyd"):
        poles = kmeans_1d(values, offsets, k, int(cfg.kmeans_iters))
    else:
        raise ValueError(f"kmeans_fit must be 'optimal' or 'lloyd', got {cfg.kmeans_fit!r}")
    return poles, up, lo


def calibrate_keys(K_concat: torch.Tensor, cfg: CalibrationConfig) -> PerChannelScale:
    """K_concat (total_tokens, H, D) -> per-channel scales: poles (H, D, L),
    thresholds (H, D), fp32 on K_concat's device (src/kvquant/calibration.py:126-156)."""
    T, H, D = (int(x) for x in K_concat.shape)
    X = K_concat.float().permute(1, 2, 0).reshape(H * D, T).contiguous()
    poles, up, lo = _fit_rows(X, cfg)
    L = int(poles.shape[1])
    return PerChannelScale(poles=poles.view(H, D, L), upper_threshold=up.view(H, D),
                           lower_threshold=lo.view(H, D), num_bits=int(cfg.num_bits))


def calibrate_values(V_stack: torch.Tensor, cfg: CalibrationConfig) -> PerTokenScale:
    """V_stack (num_prompts, seqlen, H, D) -> per-token scales: poles
    (H, seqlen, L), thresholds (H, seqlen); the samples of (h, t) are
    V_stack[:, t, h, :] over prompts and channels (src/kvquant/calibration.py:159-188)."""
    Np, S, H, D = (int(x) for x in V_stack.shape)
    X = V_stack.float().permute(2, 1, 0, 3).reshape(H * S, Np * D).contiguous()
    poles, up, lo = _fit_rows(X, cfg)
    L = int(poles.shape[1])
    return PerTokenScale(poles=poles.view(H, S, L), upper_threshold=up.view(H, S),
                         lower_threshold=lo.view(H, S), num_bits=int(cfg.num_bits))
