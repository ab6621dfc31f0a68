"""nuq (non-uniform) quantisation: the reference's CPU spec functions, on the GPU.

Drop-in for src/kvquant/nuq.py:22-156.  Same signatures and results,
including the dtype semantics of the spec: the difference ``values - poles`` is
formed in the promoted dtype of the two (for fp16 inputs it is rounded to fp16
before ``abs``/``argmin``, which can move ties relative to the fp32 kernels),
the first minimum wins, outliers are ``values < lower | values > upper``, and
``quantize_nuq`` returns ``where(mask, values, pole)`` in the promoted dtype.

The element-wise work runs in one broadcasting gfx950 kernel
(``hkv_nuq_quantize_generic`` / ``hkv_nuq_dequantize_generic``).  The two
optional ``find_outliers`` refinements the reference's own GPU kernels ignore
(``cap_outliers``, ``first_few_fp16``) are applied afterwards with the same
tensor operations as the spec (nuq.py:74-92), on the same device.
Tensors must live on the GPU.
"""
from __future__ import annotations

import ctypes

import torch

from helix_kv import _native as N

_MAXD = 6


def _float(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype in (torch.float16, torch.float32, torch.bfloat16) else t.float()


def _shape_arg(shape) -> "ctypes.Array":
    arr = (N._i64 * _MAXD)()
    for i, s in enumerate(shape):
        arr[i] = int(s)
    return arr


def _quantize(values, poles, upper=None, lower=None, want_codes=False, want_recon=True,
              want_mask=False, recon_dtype=None):
    N.require_gpu(values, poles, upper, lower)
    values = _float(values)
    poles = _float(poles)
    L = int(poles.shape[-1])
    shapes = [values.shape, poles.shape[:-1]]
    if upper is not None:
        upper, lower = _float(upper), _float(lower)
        shapes += [upper.shape, lower.shape]
    S = torch.broadcast_shapes(*shapes)
    if len(S) > _MAXD:
        raise ValueError(f"at most {_MAXD} broadcast dims supported, got {len(S)}")
    nd = len(S)
    v = values.expand(S)
    p = poles.expand(*S, L)
    cdt = torch.promote_types(values.dtype, poles.dtype)
    rdt = recon_dtype or cdt
    dev = values.device
    codes = torch.empty(S, dtype=torch.int64, device=dev) if want_codes else None
    recon = torch.empty(S, dtype=rdt, device=dev) if want_recon else None
    mask = torch.empty(S, dtype=torch.bool, device=dev) if want_mask else None
    dv, dp = N.desc(v, nd), N.desc(p, nd)
    du = dl = None
    if upper is not None:
        du, dl = N.desc(upper.expand(S), nd), N.desc(lower.expand(S), nd)
    st = N.lib().hkv_nuq_quantize_generic(
        nd, _shape_arg(S), dv, dp, int(p.stride(-1)), L,
        None if du is None else ctypes.byref(du), None if dl is None else ctypes.byref(dl),
        N.dtype_code(torch.empty(0, dtype=cdt)), N.ptr(codes), N.ptr(recon),
        N.dtype_code(torch.empty(0, dtype=rdt)), N.ptr(mask), N.stream_of(values))
    N.check(st, "hkv_nuq_quantize_generic", ValueError)
    return codes, recon, mask


def round_to_nearest_pole(values: torch.Tensor, poles: torch.Tensor) -> torch.Tensor:
    """Nearest pole per element (first minimum of |values - poles| in the
    promoted dtype), returned in the poles' dtype.  nuq.py:22-38."""
    _, recon, _ = _quantize(values, poles, recon_dtype=_float(poles).dtype)
    return recon


def nearest_pole_index(values: torch.Tensor, poles: torch.Tensor) -> torch.Tensor:
    """The int64 codes behind :func:`round_to_nearest_pole`."""
    codes, _, _ = _quantize(values, poles, want_codes=True, want_recon=False)
    return codes


def find_outliers(values: torch.Tensor, upper_threshold: torch.Tensor,
                  lower_threshold: torch.Tensor, cap_outliers: int = -1,
                  first_few_fp16: int = -1, seq_dim: int = -2) -> torch.Tensor:
    """Boolean outlier mask (values outside [lower, upper]).  nuq.py:41-94."""
    _, _, mask = _quantize(values, values.unsqueeze(-1), upper_threshold, lower_threshold,
                           want_recon=False, want_mask=True)
    if cap_outliers > 0:
        # keep the cap_outliers largest normalised deviations per row (nuq.py:74-87)
        zero_point = (upper_threshold + lower_threshold) / 2
        half_band = ((upper_threshold - lower_threshold) / 2).clamp(min=1e-8)
        magnitude = ((values - zero_point) / half_band).abs() * mask.to(values.dtype)
        keep = torch.topk(magnitude, k=cap_outliers, dim=-1).indices
        mask = torch.zeros_like(mask).scatter_(-1, keep, True)
    if first_few_fp16 > 0:
        idx = [slice(None)] * mask.dim()
        idx[seq_dim] = slice(0, first_few_fp16)
        mask[tuple(idx)] = True
    return mask


def quantize_nuq(values: torch.Tensor, poles: torch.Tensor, upper_threshold: torch.Tensor,
                 lower_threshold: torch.Tensor, cap_outliers: int = -1, first_few_fp16: int = -1,
                 seq_dim: int = -2) -> tuple[torch.Tensor, torch.Tensor]:
    """(reconstructed, outlier_mask): outliers keep their value, the rest their
    nearest pole.  nuq.py:97-132."""
    if cap_outliers <= 0 and first_few_fp16 <= 0:
        _, recon, mask = _quantize(values, poles, upper_threshold, lower_threshold,
                                   want_mask=True)
        return recon, mask
    mask = find_outliers(values, upper_threshold, lower_threshold, cap_outliers,
                         first_few_fp16, seq_dim)
    quantised = round_to_nearest_pole(values, poles)
    return torch.where(mask, values, quantised), mask


def dequantize_nuq(codes: torch.Tensor, outliers: torch.Tensor, outlier_mask: torch.Tensor,
                   poles: torch.Tensor, *, check_codes: bool = False) -> torch.Tensor:
    """where(mask, outliers, poles[code]) in the outliers' dtype.  nuq.py:135-156.

    Asynchronous, like the reference's gather (nuq.py:155-156).  A code
    outside [0, L) reads pole 0; with check_codes=True the call waits for the
    kernel and raises RuntimeError if any code was out of range (the
    reference's gather raises on such an index)."""
    N.require_gpu(codes, outliers, outlier_mask, poles)
    outliers = _float(outliers)
    poles = _float(poles)
    L = int(poles.shape[-1])
    S = torch.broadcast_shapes(codes.shape, outliers.shape, outlier_mask.shape, poles.shape[:-1])
    if len(S) > _MAXD:
        raise ValueError(f"at most {_MAXD} broadcast dims supported, got {len(S)}")
    nd = len(S)
    c = codes if codes.dtype in (torch.int64, torch.int32, torch.uint8) else codes.long()
    m = outlier_mask if outlier_mask.dtype in (torch.bool, torch.uint8) else outlier_mask.bool()
    p = poles.expand(*S, L)
    out = torch.empty(S, dtype=outliers.dtype, device=outliers.device)
    err = torch.zeros(1, dtype=torch.int32, device=outliers.device)
    st = N.lib().hkv_nuq_dequantize_generic(
        nd, _shape_arg(S), N.desc(c.expand(S), nd), N.desc(outliers.expand(S), nd),
        N.desc(m.expand(S), nd), N.desc(p, nd), int(p.stride(-1)), L, N.ptr(out),
        N.dtype_code(out), N.ptr(err), N.stream_of(outliers))
    N.check(st, "hkv_nuq_dequantize_generic", ValueError)
    if check_codes and int(err.item()):
        raise RuntimeError("dequantize_nuq: code index out of range")
    return out


__all__ = ["round_to_nearest_pole", "find_outliers", "quantize_nuq", "dequantize_nuq",
           "nearest_pole_index"]
