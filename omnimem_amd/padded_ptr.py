"""Pointer-table selection attention and the block-store entry, with the reference signatures.

Reference: src/omnimem/nsa/ops/selection/padded_ptr/_dispatch.py:14-93 (``build_ptr_table``,
``launch_ptr_fwd``), wrapper.py:458-553 (``selection_attention_padded_ptr_fast``),
block_wrapper.py:15-89 (``selection_attention_block_store``) and cuda_backend/ops.py:123-141
(``sel_fwd_ptr``).  The K/V blocks are reached through raw int64 byte addresses exactly as
there; the paged cache of ``omnimem_amd.block_cache`` is served by ``selection_attention_paged``
(int32 unit slots, no raw addresses, fp8 pages).
"""
from __future__ import annotations

from typing import Any, Dict, Optional, Sequence, Tuple

import torch

from . import _lib, ops
from .backend import NSABackendError, get_backend

__all__ = ["build_ptr_table", "launch_ptr_fwd", "selection_attention_padded_ptr_fast",
           "selection_attention_block_store", "selection_attention_paged"]


@torch.compiler.disable()
def build_ptr_table(block_indices: torch.Tensor, block_base_ptrs_k: torch.Tensor,
                    block_base_ptrs_v: torch.Tensor, n_blocks_per_head: torch.Tensor,
                    batch_stride: int, blocks_per_chunk: int = 0, in_chunk_block_bytes: int = 0,
                    backend: Optional[str] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """int64 [B, MG, H, T] K and V byte addresses of every selected block (0 = skip), via
    ``torch.ops.omnimem_nsa.build_ptr_table``.  Raw addresses make this an eager boundary, as in
    the reference (cuda_backend/ops.py:74)."""
    get_backend() if backend is None else None
    return ops.op("build_ptr_table")(block_indices, block_base_ptrs_k, block_base_ptrs_v,
                                     n_blocks_per_head, int(batch_stride), int(blocks_per_chunk),
                                     int(in_chunk_block_bytes))


def _build_ptr_table_impl(block_indices, block_base_ptrs_k, block_base_ptrs_v, n_blocks_per_head,
                          batch_stride, blocks_per_chunk, in_chunk_block_bytes):
    _lib.require_cuda((block_indices, "block_indices"), (block_base_ptrs_k, "block_base_ptrs_k"),
                      (block_base_ptrs_v, "block_base_ptrs_v"),
                      (n_blocks_per_head, "n_blocks_per_head"))
    if block_indices.dim() != 4 or block_indices.dtype != torch.int32:
        raise NSABackendError("build_ptr_table: block_indices must be int32 [B, MG, H, T]")
    if block_base_ptrs_k.dim() != 2 or block_base_ptrs_k.shape != block_base_ptrs_v.shape:
        raise NSABackendError("build_ptr_table: base tables must be [H, max_chunks] and agree")
    if block_base_ptrs_k.dtype != torch.int64 or block_base_ptrs_v.dtype != torch.int64:
        raise NSABackendError("build_ptr_table: base tables must be int64 byte addresses")
    if block_base_ptrs_k.stride() != block_base_ptrs_v.stride():
        raise NSABackendError("build_ptr_table: base_k / base_v must share strides")
    H = block_indices.shape[2]
    if block_base_ptrs_k.shape[0] != H or n_blocks_per_head.shape != (H,):
        raise NSABackendError("build_ptr_table: base tables and n_blocks_per_head need H rows")
    if n_blocks_per_head.dtype != torch.int32 or not n_blocks_per_head.is_contiguous():
        raise NSABackendError("build_ptr_table: n_blocks_per_head must be contiguous int32 [H]")
    if blocks_per_chunk < 0 or (blocks_per_chunk > 0 and in_chunk_block_bytes <= 0):
        raise NSABackendError("build_ptr_table: blocks_per_chunk >= 0 and in_chunk_block_bytes "
                              "> 0 for a chunk-level base table")
    ptr_k = torch.empty(block_indices.shape, dtype=torch.int64, device=block_indices.device)
    ptr_v = torch.empty_like(ptr_k)
    if ptr_k.numel() == 0:
        return ptr_k, ptr_v
    _lib.call("omm_build_ptr_table", _lib.view4(block_indices), block_base_ptrs_k.data_ptr(),
              block_base_ptrs_v.data_ptr(), block_base_ptrs_k.stride(0),
              block_base_ptrs_k.stride(1), block_base_ptrs_k.shape[1],
              n_blocks_per_head.data_ptr(), int(batch_stride), int(blocks_per_chunk),
              int(in_chunk_block_bytes), ptr_k.data_ptr(), ptr_v.data_ptr(),
              _lib.stream_of(block_indices))
    return ptr_k, ptr_v


@torch.compiler.disable()
def launch_ptr_fwd(q: torch.Tensor, ptr_table_k: torch.Tensor, ptr_table_v: torch.Tensor,
                   block_size: int, group_size: int, stride_bn: int, stride_bd: int,
                   softmax_scale: float, return_lse: bool, input_precision: str = "tf32",
                   owners: Sequence[torch.Tensor] = (), backend: Optional[str] = None):
    """Pointer forward via ``torch.ops.omnimem_nsa.sel_fwd_ptr``: returns (out, lse or None).
    bf16 storage only, as the reference."""
    out, lse = ops.op("sel_fwd_ptr")(q, ptr_table_k, ptr_table_v, int(block_size),
                                     int(group_size), int(stride_bn), int(stride_bd),
                                     float(softmax_scale), str(input_precision), list(owners))
    return out, (lse if return_lse else None)


def _sel_fwd_ptr_impl(q, ptr_table_k, ptr_table_v, block_size, group_size, stride_bn, stride_bd,
                      softmax_scale, input_precision, owners):
    _lib.require_cuda((q, "q"), (ptr_table_k, "ptr_table_k"), (ptr_table_v, "ptr_table_v"))
    for o in owners:
        if isinstance(o, torch.Tensor) and o.dtype != torch.bfloat16:
            raise NSABackendError(
                f"pointer selection attention requires bf16 K/V storage, got {o.dtype}")
    if q.dtype != torch.bfloat16:
        raise NSABackendError(f"pointer selection attention requires bf16 q, got {q.dtype}")
    B, M, H, D = q.shape
    G = int(group_size)
    assert M % G == 0, f"selection attention requires M ({M}) divisible by group_size ({G})"
    if ptr_table_k.shape != ptr_table_v.shape or ptr_table_k.shape[:3] != (B, M // G, H):
        raise NSABackendError("launch_ptr_fwd: pointer tables must be [B, M/G, H, T]")
    if ptr_table_k.stride() != ptr_table_v.stride():
        raise NSABackendError("launch_ptr_fwd: pointer tables must share strides")
    out = torch.empty_like(q)
    lse = torch.empty((B, H, M), dtype=torch.float32, device=q.device)
    strides = (_lib.ctypes.c_int64 * 4)(*ptr_table_k.stride())
    _lib.call("omm_sel_fwd_ptr", _lib.view4(q), ptr_table_k.data_ptr(), ptr_table_v.data_ptr(),
              strides, ptr_table_k.shape[-1], int(block_size), G, int(stride_bn),
              int(stride_bd), float(softmax_scale), _lib.view4(out),
              lse.data_ptr() if lse.numel() else None, _lib.stream_of(q))
    return out, lse


def selection_attention_padded_ptr_fast(
    q: torch.Tensor,
    block_indices: torch.Tensor,
    block_size: int,
    group_size: int,
    chunk_len: int,
    chunk_base_ptrs_k: torch.Tensor,
    chunk_base_ptrs_v: torch.Tensor,
    n_chunks_per_head: torch.Tensor,
    chunk_strides: Dict[str, Any],
    softmax_scale: Optional[float] = None,
    return_lse: bool = False,
    input_precision: str = "tf32",
    verify_complete: bool = False,
    kv_cache=None,
    layer_idx: Optional[int] = None,
):
    """Selection attention over per-head chunk storage addressed by base pointers
    (wrapper.py:458-553).  Chunk base address 0 means "not resident": the block is skipped.

    With a ``PagedKVCache`` as ``kv_cache`` the call is served by the paged kernel instead (the
    base tables are then not needed), which also reaches host-resident units."""
    from .block_cache import PagedKVCache
    if isinstance(kv_cache, PagedKVCache):
        return selection_attention_paged(q, block_indices, block_size, group_size, kv_cache,
                                         layer_idx, softmax_scale, return_lse)
    B, M, H, D = q.shape
    G = group_size
    MG = M // G
    T = block_indices.shape[-1]
    assert q.is_cuda and q.dtype == torch.bfloat16
    assert M % G == 0
    assert block_indices.shape == (B, MG, H, T)
    assert block_indices.dtype == torch.int32
    assert chunk_base_ptrs_k.dtype == torch.int64 and chunk_base_ptrs_v.dtype == torch.int64
    assert chunk_base_ptrs_k.shape[0] == H
    assert n_chunks_per_head.dtype == torch.int32 and n_chunks_per_head.shape == (H,)
    assert chunk_len % block_size == 0
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    blocks_per_chunk = chunk_len // block_size
    n_global_blocks = (n_chunks_per_head * blocks_per_chunk).to(torch.int32)
    in_chunk_block_bytes = block_size * int(chunk_strides["token_stride_bytes"])
    ptr_k, ptr_v = build_ptr_table(block_indices, chunk_base_ptrs_k, chunk_base_ptrs_v,
                                   n_global_blocks, int(chunk_strides["batch_stride_bytes"]),
                                   blocks_per_chunk, in_chunk_block_bytes)
    out, lse = launch_ptr_fwd(q, ptr_k, ptr_v, block_size, G, int(chunk_strides["stride_bn"]),
                              int(chunk_strides["stride_bd"]), softmax_scale, return_lse,
                              input_precision)
    return (out, lse) if return_lse else out


def selection_attention_paged(q: torch.Tensor, block_indices: torch.Tensor, block_size: int,
                              group_size: int, kv_cache, layer_idx: int,
                              softmax_scale: Optional[float] = None, return_lse: bool = False):
    """Selection attention over ``PagedKVCache`` pages (bf16 or fp8), touching their LRU stamps."""
    if block_size != kv_cache.P:
        raise NSABackendError(f"block_size {block_size} != cache page size {kv_cache.P}")
    if torch.is_grad_enabled() and q.requires_grad:
        raise RuntimeError("the paged KV cache is inference-only: call under torch.no_grad()")
    return kv_cache.select(q, block_indices, layer_idx, group_size, softmax_scale, return_lse)


def selection_attention_block_store(q: torch.Tensor, block_indices: torch.Tensor,
                                    block_size: int, group_size: int, kv_cache, layer_idx: int,
                                    softmax_scale: Optional[float] = None,
                                    return_lse: bool = False, input_precision: str = "tf32"):
    """block_wrapper.py:15-89: B == 1, bf16, no grad.

    ``kv_cache.block_store`` follows the reference's store protocol (``prepare_selection``,
    ``table_views`` -> (addr_k, addr_v, n_valid) int64 [H, MB] / int32 [H],
    ``release_selection``, ``pool_k`` / ``pool_v``); a ``PagedKVCache`` (as ``kv_cache`` or as its
    ``block_store``) is served by the paged kernel."""
    from .block_cache import PagedKVCache
    B, M, H, D = q.shape
    G = group_size
    MG = M // G
    T = block_indices.shape[-1]
    assert B == 1, f"the block KV store requires batch size 1, got B={B}"
    assert q.is_cuda and q.dtype == torch.bfloat16, \
        f"block-store selection attention needs bf16 GPU queries, got {q.dtype}"
    assert block_indices.shape == (B, MG, H, T), \
        f"block_indices {tuple(block_indices.shape)} != {(B, MG, H, T)}"
    assert block_indices.dtype == torch.int32
    if torch.is_grad_enabled():
        raise RuntimeError(
            "the block KV cache is inference-only: selection_attention_block_store was called "
            "with grad enabled.  Wrap the forward in torch.no_grad()")
    store = kv_cache if isinstance(kv_cache, PagedKVCache) else getattr(kv_cache, "block_store", None)
    if isinstance(store, PagedKVCache):
        return selection_attention_paged(q, block_indices, block_size, group_size, store,
                                         layer_idx, softmax_scale, return_lse)
    assert store is not None, "selection_attention_block_store needs a configured store"
    assert store.block_tokens == block_size and store.head_dim == D and store.num_heads == H, (
        f"store geometry (bt={store.block_tokens}, D={store.head_dim}, H={store.num_heads}) != "
        f"({block_size}, {D}, {H})")
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    lease = store.prepare_selection(layer_idx, block_indices)
    try:
        addr_k, addr_v, n_valid = store.table_views(layer_idx)
        ptr_k, ptr_v = build_ptr_table(block_indices, addr_k, addr_v, n_valid, 0, 0)
        out, lse = launch_ptr_fwd(q, ptr_k, ptr_v, block_size, G, D, 1, softmax_scale,
                                  return_lse, input_precision,
                                  owners=(store.pool_k[layer_idx], store.pool_v[layer_idx]))
    finally:
        store.release_selection(lease)
    return (out, lse) if return_lse else out
