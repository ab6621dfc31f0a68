"""ctypes binding of libhelix_kv.so (the C ABI declared in include/helix_kv.h).

The library is built in-tree by ``helix-lite_amd/csrc/Makefile`` and loaded
from this directory.  There is no fallback: if the library is missing or a
tensor is not on a GPU, calls raise.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libhelix_kv.so"

HKV_OK = 0
HKV_ERR_ARG = 1
HKV_ERR_SHAPE = 2
HKV_ERR_DTYPE = 3
HKV_ERR_CAPACITY = 4
HKV_ERR_LAUNCH = 5
HKV_ERR_WORKSPACE = 6
HKV_ERR_SCRATCH = 7

DT_F16, DT_F32, DT_BF16, DT_I64, DT_U8, DT_I32 = 0, 1, 2, 3, 4, 5
TABLE_BYTES = 80

_DTYPE_CODE = {torch.float16: DT_F16, torch.float32: DT_F32, torch.bfloat16: DT_BF16,
               torch.int64: DT_I64, torch.uint8: DT_U8, torch.bool: DT_U8, torch.int32: DT_I32}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_sz = ctypes.c_size_t


class NuqScales(ctypes.Structure):
    """Mirror of ``hkv_nuq_scales``."""

    _fields_ = [
        ("tables", _p), ("poles", _p), ("upper", _p), ("lower", _p),
        ("poles_dtype", ctypes.c_int32), ("thr_dtype", ctypes.c_int32),
        ("levels", ctypes.c_int32), ("per_token", ctypes.c_int32),
        ("rows", _i64), ("positions", _p), ("pos_offset", _i64),
    ]


class PackItem(ctypes.Structure):
    """Mirror of ``hkv_pack_item``."""

    _fields_ = [
        ("values", _p), ("T", _i64), ("H", ctypes.c_int32), ("D", ctypes.c_int32),
        ("bits", ctypes.c_int32), ("reserved", ctypes.c_int32), ("scales", NuqScales),
        ("packed", _p), ("row_ptr", _p), ("col", _p), ("val", _p), ("capacity", _i64),
    ]


class UnpackItem(ctypes.Structure):
    """Mirror of ``hkv_unpack_item``."""

    _fields_ = [
        ("packed", _p), ("row_ptr", _p), ("col", _p), ("val", _p), ("capacity", _i64), ("T", _i64),
        ("H", ctypes.c_int32), ("D", ctypes.c_int32), ("bits", ctypes.c_int32),
        ("reserved", ctypes.c_int32), ("scales", NuqScales), ("out", _p),
    ]


class PagedSideDesc(ctypes.Structure):
    """Mirror of ``hkv_paged_side``."""

    _fields_ = [
        ("codes", _p), ("ocnt", _p), ("oent", _p), ("ovf", _p), ("ovf_ent", _p), ("ovf_next", _p),
        ("kmin", _p), ("kmax", _p), ("status", _p), ("num_blocks", _i64),
        ("heads", ctypes.c_int32), ("bits", ctypes.c_int32), ("cap", ctypes.c_int32),
        ("n_chunks", ctypes.c_int32),
    ]


class TensorDesc(ctypes.Structure):
    """Mirror of ``hkv_tensor_desc``."""

    _fields_ = [("data", _p), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("strides", _i64 * 6)]


_SIGS = {
    "hkv_version": ([], ctypes.c_char_p),
    "hkv_status_string": ([_i32], ctypes.c_char_p),
    "hkv_nuq_build_tables": ([_p, _i32, _p, _p, _i32, _i64, _i32, _p, _p], _i32),
    "hkv_nuq_pack_dense": ([_p, _i64, _i32, _i32, ctypes.POINTER(NuqScales), _p, _p, _p, _p], _i32),
    "hkv_nuq_unpack_dense": ([_p, _p, _p, _i64, _i32, _i32, ctypes.POINTER(NuqScales), _p, _p], _i32),
    "hkv_nuq_pack_compact_workspace_bytes": ([_i64, _i32, _i32], _sz),
    "hkv_nuq_pack_compact": ([_p, _i64, _i32, _i32, _i32, ctypes.POINTER(NuqScales), _p, _p, _p,
                              _p, _i64, _p, _sz, _p], _i32),
    "hkv_nuq_pack_compact_batch_workspace_bytes": ([ctypes.POINTER(PackItem), _i32], _sz),
    "hkv_nuq_pack_compact_batch": ([ctypes.POINTER(PackItem), _i32, _p, _sz, _p], _i32),
    "hkv_nuq_unpack_compact_batch": ([ctypes.POINTER(UnpackItem), _i32, _p], _i32),
    "hkv_nuq_unpack_compact": ([_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32,
                                ctypes.POINTER(NuqScales), _p, _p], _i32),
    "hkv_nuq_quantize_generic": ([_i32, ctypes.POINTER(_i64), ctypes.POINTER(TensorDesc),
                                  ctypes.POINTER(TensorDesc), _i64, _i32, ctypes.POINTER(TensorDesc),
                                  ctypes.POINTER(TensorDesc), _i32, _p, _p, _i32, _p, _p], _i32),
    "hkv_nuq_dequantize_generic": ([_i32, ctypes.POINTER(_i64), ctypes.POINTER(TensorDesc),
                                    ctypes.POINTER(TensorDesc), ctypes.POINTER(TensorDesc),
                                    ctypes.POINTER(TensorDesc), _i64, _i32, _p, _i32, _p, _p], _i32),
    "hkv_pool_write": ([_p, _i64, _i32, _i32, ctypes.POINTER(NuqScales), _p, _i64, _i32, _p, _p, _p,
                        _p, _p, _p], _i32),
    "hkv_pool_gather": ([_p, _p, _p, _i64, _i32, _i32, _i32, ctypes.POINTER(NuqScales), _p, _p, _i64,
                         _p, _p], _i32),
    "hkv_paged_write": ([_p, _i64, ctypes.POINTER(NuqScales), _p, ctypes.POINTER(PagedSideDesc), _p],
                        _i32),
    "hkv_paged_gather": ([ctypes.POINTER(PagedSideDesc), ctypes.POINTER(NuqScales), _p, _p, _i64, _p,
                          _p], _i32),
    "hkv_quest_select_paged": ([_p, _i32, _i32, ctypes.POINTER(PagedSideDesc), _p, _i64, _i64, _i64,
                                _p, _p, ctypes.POINTER(_i64), _p, _sz, _p], _i32),
    "hkv_paged_decode_attn": ([_p, _i32, _i64, _p, ctypes.POINTER(PagedSideDesc), _p,
                               ctypes.POINTER(PagedSideDesc), _p, _i64, _p, _i64, _i32,
                               ctypes.c_float, _p, _i32, _p, _sz, _p], _i32),
    "hkv_quest_page_stats": ([_p, _i32, _i64, _i32, _i32, _i32, _p, _p, _p], _i32),
    "hkv_quest_page_bound": ([_p, _i32, _i32, _p, _p, _i32, _i64, _i32, _i32, _p, _i32, _p], _i32),
    "hkv_quest_topk_workspace_bytes": ([_i64, _i32], _sz),
    "hkv_quest_topk": ([_p, _i32, _i64, _i32, _i64, _i64, _p, ctypes.POINTER(_i64), _p, _sz, _p], _i32),
    "hkv_quest_select_workspace_bytes": ([_i64, _i32], _sz),
    "hkv_quest_select": ([_p, _i32, _i32, _p, _p, _i32, _i64, _i32, _i32, _i64, _i64, _p, _p,
                          ctypes.POINTER(_i64), _p, _sz, _p], _i32),
    "hkv_quest_select_noalloc_max_workspace": ([], _sz),
    "hkv_quest_select_noalloc": ([_p, _i32, _i32, _p, _p, _i32, _i64, _i32, _i32, _i64, _i64, _p, _p,
                                  ctypes.POINTER(_i64), _p], _i32),
    "hkv_quest_page_stats_u8_workspace_bytes": ([_i32, _i32], _sz),
    "hkv_quest_page_stats_u8": ([_p, _p, _i32, _i64, _i32, _i32, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "hkv_quest_select_u8": ([_p, _i32, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i64, _i64, _p, _p,
                             ctypes.POINTER(_i64), _p, _sz, _p], _i32),
    "hkv_quest_select_blocks": ([_p, _i32, _i32, _p, _p, _i32, _i64, _i32, _p, _i64, _i64, _i64,
                                 _i64, _p, _p, _p, _p, _p, _p, _p], _i32),
    "hkv_decode_workspace_bytes": ([_i64, _i32, _i32], _sz),
    "hkv_decode_attn": ([_p, _i32, _i32, _i32, _i64,
                         _p, _p, _p, _p, _i64, _i32, _p,
                         _p, _p, _p, _p, _i64, _i32, _p, _i64,
                         _p, _i64, _i32, ctypes.c_float, _p, _i32, _p, _sz, _p], _i32),
    "hkv_decode_batch_workspace_bytes": ([_i32, ctypes.POINTER(_i64), _i32, _i32], _sz),
    "hkv_decode_attn_batch": ([_p, _i32, _i32, _i32, _i32, _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                               _p, _p, _p, _p, _i64, _i32, _p,
                               _p, _p, _p, _p, _i64, _i32, _p, _i64,
                               _p, ctypes.POINTER(_i64), _i32, ctypes.c_float, _p, _i32, _p, _sz, _p], _i32),
    "hkv_paged_decode_attn_batch": ([_p, _i32, _i32, ctypes.POINTER(_i64), _p, ctypes.POINTER(_i64),
                                     ctypes.POINTER(PagedSideDesc), _p, ctypes.POINTER(PagedSideDesc), _p,
                                     _i64, _p, ctypes.POINTER(_i64), _i32, ctypes.c_float, _p, _i32, _p,
                                     _sz, _p], _i32),
    "hkv_union_pages_workspace_bytes": ([_i64], _sz),
    "hkv_union_pages_ragged": ([_p, _i32, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _p, _p, _sz,
                                _p], _i32),
    "hkv_quest_select_ragged": ([_p, _i32, _i32, _i32, _p, _p, _i32, _i32, _i32,
                                 ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i64, _p, _p,
                                 ctypes.POINTER(_i64), _p], _i32),
    "hkv_quest_select_paged_ragged": ([_p, _i32, _i32, _i32, ctypes.POINTER(PagedSideDesc), _p,
                                       ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                       _i64, _p, _p, ctypes.POINTER(_i64), _p], _i32),
    "hkv_nuq_gather_pages": ([_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32,
                              ctypes.POINTER(NuqScales), _i32, _i32, ctypes.POINTER(_i64),
                              ctypes.POINTER(_i64), _p, _p, _p], _i32),
    "hkv_kmeans_1d": ([_p, _p, _i64, _i32, _i32, _p, _p], _i32),
    "hkv_kmeans_1d_optimal_workspace_bytes": ([], _sz),
    "hkv_kmeans_1d_optimal": ([_p, _p, _i64, _i32, _p, _p, _sz, _p], _i32),
    "hkv_selected_attention_workspace_bytes": ([_i64, _i32, _i32, _i32], _sz),
    "hkv_selected_attention": ([_p, _i32, _i32, _i32, _p, _p, _i32, _i64, _i32, _i32, _i32, _i32,
                                _p, _i64, _i32, _i32, ctypes.c_float, _p, _i32, _p, _sz, _p], _i32),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"helix_kv native library not found at {LIB_PATH}; build it with "
                        "`make -C helix-lite_amd/csrc` (or __graft_entry__.build())")
                L = ctypes.CDLL(str(LIB_PATH))
                for name, (args, res) in _SIGS.items():
                    fn = getattr(L, name)
                    fn.argtypes = args
                    fn.restype = res
                _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def check(status: int, what: str, exc: type[Exception] = RuntimeError) -> None:
    if status == HKV_OK:
        return
    msg = lib().hkv_status_string(status).decode()
    if status in (HKV_ERR_SHAPE, HKV_ERR_ARG, HKV_ERR_DTYPE):
        raise exc(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {status})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """hipStream_t of torch's current stream on t's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise AssertionError("helix_kv runs on the GPU: tensors must be on a CUDA (HIP) device")


# --------------------------------------------------------------- workspaces

_ws: dict[tuple, torch.Tensor] = {}
# Buffers replaced by larger ones.  They are never freed: a HIP graph captured
# while one of them was current keeps its raw address and writes to it on
# every replay, so handing that memory back to the caching allocator would
# let a replay corrupt whatever tensor received it next.
_ws_retired: list[torch.Tensor] = []


def workspace(kind: str, nbytes: int, device: torch.device) -> torch.Tensor:
    """A zero-initialised device scratch buffer reused across calls.

    One buffer per (kind, device, current stream); grown (and re-zeroed) when a
    larger one is needed.  Calls that share a buffer are ordered on that
    stream, which the kernels rely on.  A superseded buffer stays allocated
    for the life of the process (graphs captured earlier still address it).
    """
    dev = torch.device(device)
    key = (kind, dev.index, torch.cuda.current_stream(dev).cuda_stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _ws_retired.append(buf)
        buf = torch.zeros(max(int(nbytes), 64), dtype=torch.uint8, device=dev)
        _ws[key] = buf
    return buf


def desc(t: torch.Tensor, ndim: int) -> TensorDesc:
    """Descriptor of a view already expanded to a broadcast shape of ``ndim`` dims
    (a trailing level axis, if any, is not part of it)."""
    d = TensorDesc()
    d.data = t.data_ptr()
    d.dtype = dtype_code(t)
    st = list(t.stride())[:ndim]
    for i in range(6):
        d.strides[i] = st[i] if i < ndim else 0
    return d


_cus: dict[int, int] = {}


def num_cus(device=None) -> int:
    """Compute units of the (current) device, cached."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _cus:
        _cus[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _cus[idx]
