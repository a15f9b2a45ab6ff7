"""ctypes binding of the C ABI declared in include/omnimem_hip.h.

The library is loaded after ``torch`` so that its ``libamdhip64.so.7`` dependency resolves to the
HIP runtime torch already loaded (same SONAME): one runtime per process, so torch's streams and
device pointers are valid in our launches.  There is no fallback: if the library is missing the
import of any op raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the HIP library, see module docstring)

from .backend import NSABackendError

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_omnimem_hip.so")

OMM_F32, OMM_BF16, OMM_F16, OMM_FP8E4M3 = 0, 1, 2, 3
OMM_OK = 0

_DTYPE = {torch.float32: OMM_F32, torch.bfloat16: OMM_BF16, torch.float16: OMM_F16}


class View4(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("size", ctypes.c_int64 * 4),
                ("stride", ctypes.c_int64 * 4)]


class TopkMask(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "block_size", "group_size", "chunk_q", "chunk_k", "blocks_per_chunk", "q_chunk_offset",
        "q_half", "k_half", "ex_win", "ex_sink", "causal", "tf_mask", "prog_excl")]


class PagedKV(ctypes.Structure):
    _fields_ = [
        ("pool_k", ctypes.c_void_p), ("pool_v", ctypes.c_void_p),
        ("scale_k", ctypes.c_void_p), ("scale_v", ctypes.c_void_p),
        ("host_k", ctypes.c_void_p), ("host_v", ctypes.c_void_p),
        ("host_scale_k", ctypes.c_void_p), ("host_scale_v", ctypes.c_void_p),
        ("unit_table", ctypes.c_void_p), ("stamp", ctypes.c_void_p), ("reads", ctypes.c_void_p),
        ("num_heads", ctypes.c_int32), ("max_chunks", ctypes.c_int32),
        ("n_chunks", ctypes.c_int32), ("chunk_len", ctypes.c_int32),
        ("page_tokens", ctypes.c_int32), ("pages_per_chunk", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("n_slots", ctypes.c_int32), ("n_host_slots", ctypes.c_int32),
        ("page_seen", ctypes.c_void_p),
        ("qk_fp8", ctypes.c_int32),
        ("touches", ctypes.c_void_p),
        ("stage_k", ctypes.c_void_p), ("stage_v", ctypes.c_void_p),
        ("stage_scale_k", ctypes.c_void_p), ("stage_scale_v", ctypes.c_void_p),
        ("stage_map_epoch", ctypes.c_void_p), ("stage_map_slot", ctypes.c_void_p),
        ("stage_counter", ctypes.c_void_p), ("stage_slots", ctypes.c_int32),
    ]


_vp, _i32, _i64, _f32, _sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
_V = ctypes.POINTER(View4)
_M = ctypes.POINTER(TopkMask)
_P = ctypes.POINTER(PagedKV)

# Every entry point of include/omnimem_hip.h: name -> (restype, argtypes).
PROTOTYPES = {
    "omm_last_error": (ctypes.c_char_p, []),
    "omm_abi_version": (_i32, []),
    "omm_host_alloc": (_i32, [_sz, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "omm_host_free": (_i32, [_vp]),
    "omm_block_pool": (_i32, [_V, _V, _i32, _i32, _vp]),
    "omm_topk_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "omm_topk": (_i32, [_V, _V, _i32, _i32, _f32, _M, _vp, _vp, _sz, _vp]),
    "omm_paged_stage": (_i32, [_P, _V, _i32, _vp]),
    "omm_copy_units_async": (_i32, [_vp] * 8 + [_vp, _vp, _i32, _i32, _i32, _i64, _i64, _vp]),
    "omm_topk_fused_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32]),
    "omm_topk_fused": (_i32, [_V, _V, _i32, _i32, _i32, _f32, _M, _vp, _vp, _sz, _vp]),
    "omm_topk_fused_debug": (_i32, [_V, _V, _i32, _i32, _i32, _f32, _M, _vp, _vp, _vp, _sz, _vp]),
    "omm_topk_fused_noalloc_max_bytes": (_sz, []),
    "omm_topk_fused_noalloc": (_i32, [_V, _V, _i32, _i32, _i32, _f32, _M, _vp, _vp]),
    "omm_topk_from_scores": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _M, _vp, _vp, _sz, _vp]),
    "omm_sel_fwd": (_i32, [_V, _V, _V, _V, _i32, _i32, _i32, _i32, _i32, _f32, _V, _vp, _vp]),
    "omm_sel_fwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i32, _i32]),
    "omm_sel_fwd_ws": (_i32, [_V, _V, _V, _V, _i32, _i32, _i32, _i32, _i32, _f32, _V, _vp, _vp, _sz,
                              _vp]),
    "omm_sel_fwd_gated": (_i32, [_V, _V, _V, _V, _i32, _i32, _i32, _i32, _f32, _V, _V, _V, _V, _vp,
                                 _vp]),
    "omm_sel_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i32, _i32, _i64]),
    "omm_sel_bwd": (_i32, [_V, _V, _V, _V, _V, _vp, _V, _i32, _i32, _i32, _i32, _i32, _f32, _V, _V,
                           _V, _vp, _sz, _vp]),
    "omm_sel_fwd_ptr": (_i32, [_V, _vp, _vp, _vp, _i64, _i32, _i32, _i64, _i64, _f32, _V, _vp,
                               _vp]),
    "omm_build_ptr_table": (_i32, [_V, _vp, _vp, _i64, _i64, _i32, _vp, _i64, _i32, _i64, _vp,
                                   _vp, _vp]),
    "omm_sel_bwd_ptr_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i32, _i32, _i64, _i32]),
    "omm_sel_bwd_ptr": (_i32, [_V, _V, _vp, _V, _V, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                               _vp, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64,
                               _i64, _f32, _i32, _V, _vp, _vp, _sz, _vp]),
    "omm_paged_append": (_i32, [_P, _V, _V, _i32, _i32, _V, _V, _i32, _vp]),
    "omm_paged_append_ring": (_i32, [_P, _V, _V, _i32, _i32, _V, _V, _V, _V, _i32, _vp]),
    "omm_sel_fwd_paged": (_i32, [_V, _V, _P, _i32, _f32, _V, _vp, _i32, _vp]),
    "omm_sel_fwd_paged_gated": (_i32, [_V, _V, _P, _i32, _f32, _V, _V, _V, _V, _vp, _i32, _vp]),
    "omm_copy_units": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32,
                              _i64, _i64, _vp]),
    "omm_gather_publish_clear": (_i32, [_vp, _i64, _i64, _i64, ctypes.POINTER(_i64), _vp]),
    "omm_block_range": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                               _i32, _i32, _i32, _vp]),
    "omm_dedup_run": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                             _vp]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NSABackendError(
                        f"the gfx950 HIP library {LIB_PATH} is not built; run "
                        "`python -c 'import __graft_entry__ as g; g.build()'` (or "
                        "`python -m omnimem_amd.build`) first")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in PROTOTYPES.items():
                    fn = getattr(handle, name, None)
                    if fn is None:
                        continue  # reported by missing_symbols() and when called
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def missing_symbols() -> list:
    """Entry points of the header that the loaded library does not export."""
    return [n for n in PROTOTYPES if getattr(lib(), n, None) is None]


def last_error() -> str:
    msg = lib().omm_last_error()
    return msg.decode(errors="replace") if msg else ""


def call(name: str, *args, error: type = NSABackendError) -> None:
    """Call an entry point; a non-zero status raises ``error`` with the library's message."""
    fn = getattr(lib(), name, None)
    if fn is None:
        raise NSABackendError(f"{name} is not exported by {LIB_PATH}")
    rc = fn(*args)
    if rc != OMM_OK:
        raise error(f"{name}: {last_error()} (status {rc})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE[t.dtype]
    except KeyError:
        raise NSABackendError(f"unsupported dtype {t.dtype} (expected bfloat16, float16 or float32)")


def view4(t: torch.Tensor) -> View4:
    if t.dim() != 4:
        raise NSABackendError(f"expected a 4-D tensor, got shape {tuple(t.shape)}")
    v = View4()
    v.data = t.data_ptr() if t.numel() else 0
    for i in range(4):
        v.size[i] = t.shape[i]
        v.stride[i] = t.stride(i)
    return v


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of t's device (respects ``torch.cuda.stream``)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_cuda(*pairs) -> None:
    dev = None
    for t, name in pairs:
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise NSABackendError(f"{name} must be a GPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise NSABackendError(f"{name} on {t.device} but expected {dev}")


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
