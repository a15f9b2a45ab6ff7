"""Pointer-table selection attention and the block-store entry, with the reference signatures.

Reference: src/omnimem/nsa/ops/selection/padded_ptr/_dispatch.py:14-115 (``build_ptr_table``,
``launch_ptr_fwd``, ``launch_ptr_bwd``), wrapper.py:458-553
(``selection_attention_padded_ptr_fast``), autograd.py:38-300 (the training entries
``selection_attention_padded_ptr_train`` / ``_train_fast``), block_wrapper.py:15-89
(``selection_attention_block_store``) and cuda_backend/ops.py:123-184 (``sel_fwd_ptr``,
``sel_bwd_ptr``).  The K/V blocks are reached through raw int64 byte addresses exactly as
there; the paged cache of ``omnimem_amd.block_cache`` is served by ``selection_attention_paged``
(int32 unit slots, no raw addresses, fp8 pages).
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib, ops
from .backend import NSABackendError, get_backend, resolve_backend

__all__ = ["build_ptr_table", "launch_ptr_fwd", "launch_ptr_bwd",
           "selection_attention_padded_ptr_fast", "selection_attention_padded_ptr_train",
           "selection_attention_padded_ptr_train_fast", "selection_attention_block_store",
           "selection_attention_paged"]


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


@torch.compiler.disable()
def launch_ptr_bwd(*, q: torch.Tensor, out: torch.Tensor, lse: torch.Tensor, d_out: torch.Tensor,
                   block_indices: torch.Tensor, ptr_table_k: torch.Tensor,
                   ptr_table_v: torch.Tensor, block_base_ptrs_k: torch.Tensor,
                   block_base_ptrs_v: torch.Tensor, block_base_ptrs_dk: torch.Tensor,
                   block_base_ptrs_dv: torch.Tensor, n_blocks_per_head: torch.Tensor,
                   block_size: int, group_size: int, batch_stride_kv_bytes: int,
                   batch_stride_dkv_bytes: int, stride_bn: int, stride_bd: int,
                   stride_dbn: Optional[int] = None, stride_dbd: Optional[int] = None,
                   blocks_per_chunk: int = 0, in_chunk_block_bytes_kv: int = 0,
                   in_chunk_block_bytes_dkv: int = 0, softmax_scale: Optional[float] = None,
                   input_precision: str = "tf32", backend: Optional[str] = None,
                   compute_dkv: bool = True, owners: Sequence[torch.Tensor] = (),
                   grad_buffers: Sequence[torch.Tensor] = ()) -> Tuple[torch.Tensor, torch.Tensor]:
    """Pointer backward via ``torch.ops.omnimem_nsa.sel_bwd_ptr``: returns ``(dq, delta)``.

    dK / dV are stored into the fp32 scratch blocks that ``block_base_ptrs_dk`` / ``_dv`` address
    (``grad_buffers`` names those tensors for the op's alias annotation); ``compute_dkv=False``
    computes dq alone.  Arguments as in the reference's ``selection_attention_padded_ptr_bwd``
    (padded_ptr/kernels/select_bwd.py:564-590): ``stride_dbn`` / ``stride_dbd`` default to
    ``stride_bn`` / ``stride_bd``, an empty ``n_blocks_per_head`` means no per-head bound."""
    resolve_backend(backend)
    D = q.shape[-1]
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    return ops.op("sel_bwd_ptr")(
        q, out, lse, d_out, block_indices, ptr_table_k, ptr_table_v, block_base_ptrs_k,
        block_base_ptrs_v, block_base_ptrs_dk, block_base_ptrs_dv, n_blocks_per_head,
        int(block_size), int(group_size), int(batch_stride_kv_bytes), int(batch_stride_dkv_bytes),
        int(stride_bn), int(stride_bd), int(stride_bn if stride_dbn is None else stride_dbn),
        int(stride_bd if stride_dbd is None else stride_dbd), int(blocks_per_chunk),
        int(in_chunk_block_bytes_kv), int(in_chunk_block_bytes_dkv), scale, str(input_precision),
        bool(compute_dkv), list(owners), list(grad_buffers))


def _sel_bwd_ptr_impl(q, out, lse, d_out, block_indices, ptr_k, ptr_v, base_k, base_v, base_dk,
                      base_dv, n_blocks_per_head, block_size, group_size, batch_stride_kv_bytes,
                      batch_stride_dkv_bytes, stride_bn, stride_bd, stride_dbn, stride_dbd,
                      blocks_per_chunk, in_chunk_block_bytes_kv, in_chunk_block_bytes_dkv, scale,
                      compute_dkv, grad_buffers):
    _lib.require_cuda((q, "q"), (out, "out"), (lse, "lse"), (d_out, "d_out"),
                      (block_indices, "block_indices"), (ptr_k, "ptr_table_k"),
                      (ptr_v, "ptr_table_v"))
    if q.dtype != torch.bfloat16:
        raise NSABackendError(f"sel_bwd_ptr: q must be bfloat16, got {q.dtype}")
    if d_out.dtype != q.dtype:
        d_out = d_out.to(q.dtype)
    if out.dtype != q.dtype:
        raise NSABackendError("sel_bwd_ptr: out must have q's dtype")
    for g in grad_buffers:
        if isinstance(g, torch.Tensor) and g.dtype != torch.float32:
            raise NSABackendError(f"pointer dK/dV scratch must be float32, got {g.dtype}")
    if lse.dtype != torch.float32:
        raise NSABackendError("sel_bwd_ptr: lse must be fp32 [B, H, M]")
    lse = lse.contiguous()
    if block_indices.dtype != torch.int32 or block_indices.dim() != 4:
        raise NSABackendError("sel_bwd_ptr: block_indices must be int32 [B, MG, H, T]")
    if ptr_k.dtype != torch.int64 or ptr_v.dtype != torch.int64:
        raise NSABackendError("sel_bwd_ptr: ptr tables must be int64 byte addresses")
    if ptr_k.shape != block_indices.shape or ptr_v.shape != ptr_k.shape or \
            ptr_v.stride() != ptr_k.stride():
        raise NSABackendError("sel_bwd_ptr: ptr_k / ptr_v must match block_indices' shape and "
                              "share strides")
    B, M, H, D = q.shape
    T = block_indices.shape[-1]
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    delta = torch.empty((B, H, M), dtype=torch.float32, device=q.device)
    if B == 0 or M == 0 or H == 0:
        return dq, delta
    nb = None
    max_base = 0
    base_args = (None,) * 5
    if compute_dkv:
        tabs = (base_k, base_v, base_dk, base_dv)
        _lib.require_cuda(*((t, n) for t, n in zip(tabs, ("base_k", "base_v", "base_dk", "base_dv"))))
        if any(t.dtype != torch.int64 or t.dim() != 2 or t.shape != base_k.shape or
               t.stride() != base_k.stride() for t in tabs) or base_k.shape[0] != H:
            raise NSABackendError("sel_bwd_ptr: base_k / base_v / base_dk / base_dv must be int64 "
                                  "[H, MAXB] with one shape and one set of strides")
        if n_blocks_per_head.numel():
            if n_blocks_per_head.dtype != torch.int32 or n_blocks_per_head.shape != (H,):
                raise NSABackendError("sel_bwd_ptr: n_blocks_per_head must be int32 [H]")
            _lib.require_cuda((n_blocks_per_head, "n_blocks_per_head"))
            nb = n_blocks_per_head.contiguous()
        max_base = base_k.shape[1]
        strides = (_lib.ctypes.c_int64 * 2)(*base_k.stride())
        base_args = (base_k.data_ptr(), base_v.data_ptr(), base_dk.data_ptr(), base_dv.data_ptr(),
                     strides)
    ws = _lib.workspace(_lib.lib().omm_sel_bwd_ptr_workspace_bytes(
        B, M, H, max_base, int(blocks_per_chunk), int(group_size), T, int(bool(compute_dkv))),
        q.device)
    pstr = (_lib.ctypes.c_int64 * 4)(*ptr_k.stride())
    _lib.call("omm_sel_bwd_ptr", _lib.view4(q), _lib.view4(out), lse.data_ptr(),
              _lib.view4(d_out), _lib.view4(block_indices), ptr_k.data_ptr(), ptr_v.data_ptr(),
              pstr, *base_args, max_base, None if nb is None else nb.data_ptr(), int(block_size),
              int(group_size), int(batch_stride_kv_bytes), int(batch_stride_dkv_bytes),
              int(stride_bn), int(stride_bd), int(stride_dbn), int(stride_dbd),
              int(blocks_per_chunk), int(in_chunk_block_bytes_kv), int(in_chunk_block_bytes_dkv),
              float(scale), int(bool(compute_dkv)), _lib.view4(dq), delta.data_ptr(),
              ws.data_ptr(), ws.numel(), _lib.stream_of(q))
    return dq, delta


def _base_table(chunks: Sequence[torch.Tensor], per_head: Sequence[int], width: int,
                device) -> torch.Tensor:
    """int64 [H, width]: entry (h, c) is the address of chunk c of head h in the head-major list
    ``chunks`` (0 for chunks that are not on the GPU, and past a head's count)."""
    table = torch.zeros((len(per_head), max(width, 1)), dtype=torch.int64)
    i = 0
    for h, n in enumerate(per_head):
        for c in range(n):
            t = chunks[i]
            table[h, c] = t.data_ptr() if t.is_cuda else 0
            i += 1
    return table.to(device, non_blocking=True)


class _PaddedPtrTrainFn(torch.autograd.Function):
    """Pointer-table selection attention with gradients for q and for every K / V chunk tensor.

    The chunks arrive as autograd inputs (``*chunks`` = the head-major K chunks, then the V
    chunks, each [B, chunk_len, D] bf16), so their gradients flow back to them; the address tables
    are rebuilt from these tensors on every call (reference autograd.py:38-200).  The backward
    stores dK / dV into one zeroed fp32 buffer holding every chunk and rounds it to bf16 once."""

    @staticmethod
    def forward(ctx, q, block_indices, n_chunks_per_head, meta, *chunks):
        per_head = list(meta["n_chunks_per_head_list"])
        n_k = sum(per_head)
        width = int(meta["max_chunks"])
        bs, G, bpc = int(meta["block_size"]), int(meta["group_size"]), int(meta["blocks_per_chunk"])
        st = meta["chunk_strides"]
        base_k = _base_table(chunks[:n_k], per_head, width, q.device)
        base_v = _base_table(chunks[n_k:], per_head, width, q.device)
        n_blocks = (n_chunks_per_head.to(torch.int32) * bpc).to(torch.int32)
        ptr_k, ptr_v = build_ptr_table(block_indices, base_k, base_v, n_blocks,
                                       int(st["batch_stride_bytes"]), bpc,
                                       bs * int(st["token_stride_bytes"]))
        out, lse = launch_ptr_fwd(q, ptr_k, ptr_v, bs, G, int(st["stride_bn"]),
                                  int(st["stride_bd"]), float(meta["softmax_scale"]), True,
                                  meta.get("input_precision", "tf32"), owners=chunks)
        ctx.save_for_backward(q, out, lse, block_indices, ptr_k, ptr_v, base_k, base_v, n_blocks,
                              *chunks)
        ctx.meta = meta
        return out

    @staticmethod
    def backward(ctx, d_out):
        q, out, lse, block_indices, ptr_k, ptr_v, base_k, base_v, n_blocks, *chunks = \
            ctx.saved_tensors
        meta = ctx.meta
        per_head = list(meta["n_chunks_per_head_list"])
        n_k = sum(per_head)
        st = meta["chunk_strides"]
        bs, bpc = int(meta["block_size"]), int(meta["blocks_per_chunk"])
        shapes = {tuple(c.shape) for c in chunks}
        if len(shapes) != 1:
            raise NSABackendError(f"pointer training path: K/V chunks must share one shape, got "
                                  f"{sorted(shapes)}")
        cshape = chunks[0].shape  # [B, chunk_len, D]
        scratch = torch.zeros((2, n_k) + tuple(cshape), dtype=torch.float32, device=q.device)
        dks, dvs = scratch[0].unbind(0), scratch[1].unbind(0)
        width = base_k.shape[1]
        base_dk = _base_table(dks, per_head, width, q.device)
        base_dv = _base_table(dvs, per_head, width, q.device)
        # a chunk that is not on the GPU has base 0: it is skipped and gets no gradient
        base_dk.masked_fill_(base_k == 0, 0)
        base_dv.masked_fill_(base_v == 0, 0)
        e32 = 4
        dq, _ = launch_ptr_bwd(
            q=q, out=out, lse=lse, d_out=d_out.contiguous(), block_indices=block_indices,
            ptr_table_k=ptr_k, ptr_table_v=ptr_v, block_base_ptrs_k=base_k,
            block_base_ptrs_v=base_v, block_base_ptrs_dk=base_dk, block_base_ptrs_dv=base_dv,
            n_blocks_per_head=n_blocks, block_size=bs, group_size=int(meta["group_size"]),
            batch_stride_kv_bytes=int(st["batch_stride_bytes"]),
            batch_stride_dkv_bytes=dks[0].stride(0) * e32, stride_bn=int(st["stride_bn"]),
            stride_bd=int(st["stride_bd"]), stride_dbn=dks[0].stride(1),
            stride_dbd=dks[0].stride(2), blocks_per_chunk=bpc,
            in_chunk_block_bytes_kv=bs * int(st["token_stride_bytes"]),
            in_chunk_block_bytes_dkv=bs * dks[0].stride(1) * e32,
            softmax_scale=float(meta["softmax_scale"]),
            input_precision=meta.get("input_precision", "tf32"), owners=chunks,
            grad_buffers=(scratch,))
        grads = scratch.to(chunks[0].dtype)
        dk = [g if c.is_cuda else None for g, c in zip(grads[0].unbind(0), chunks[:n_k])]
        dv = [g if c.is_cuda else None for g, c in zip(grads[1].unbind(0), chunks[n_k:])]
        return (dq, None, None, None, *dk, *dv)


def selection_attention_padded_ptr_train_fast(
        q: torch.Tensor, block_indices: torch.Tensor, block_size: int, group_size: int,
        chunk_len: int, max_chunks: int, n_chunks_per_head: torch.Tensor,
        chunk_strides: Dict[str, Any], k_chunks_flat: Tuple[torch.Tensor, ...],
        v_chunks_flat: Tuple[torch.Tensor, ...], n_chunks_per_head_list: List[int],
        softmax_scale: Optional[float] = None, input_precision: str = "tf32") -> torch.Tensor:
    """Training forward over head-major chunk lists (autograd.py:203-240): gradients reach ``q``
    and every tensor of ``k_chunks_flat`` / ``v_chunks_flat`` ([B, chunk_len, D] bf16, head h's
    chunks at positions sum(n_chunks_per_head_list[:h]) ...)."""
    D = q.shape[-1]
    if len(k_chunks_flat) != sum(n_chunks_per_head_list) or \
            len(v_chunks_flat) != len(k_chunks_flat):
        raise NSABackendError("k_chunks_flat / v_chunks_flat must hold sum(n_chunks_per_head_list) "
                              "chunks each")
    if chunk_len % block_size:
        raise NSABackendError(f"chunk_len {chunk_len} is not a multiple of block_size {block_size}")
    meta = {"block_size": int(block_size), "group_size": int(group_size),
            "chunk_len": int(chunk_len), "chunk_strides": dict(chunk_strides),
            "softmax_scale": D ** -0.5 if softmax_scale is None else float(softmax_scale),
            "input_precision": input_precision, "blocks_per_chunk": chunk_len // block_size,
            "n_chunks_per_head_list": [int(n) for n in n_chunks_per_head_list],
            "max_chunks": int(max_chunks)}
    return _PaddedPtrTrainFn.apply(q, block_indices, n_chunks_per_head, meta, *k_chunks_flat,
                                   *v_chunks_flat)


def selection_attention_padded_ptr_train(
        q: torch.Tensor, k_chunks: List[List[torch.Tensor]], v_chunks: List[List[torch.Tensor]],
        block_indices: torch.Tensor, block_size: int, group_size: int, chunk_len: int,
        softmax_scale: Optional[float] = None, input_precision: str = "tf32",
        strict: bool = True) -> torch.Tensor:
    """Training forward over per-head lists of chunk tensors (autograd.py:243-300): the address
    tables are built from the lists on each call.  A chunk that a selected block lives in must be
    on the GPU (``strict``; else it is skipped and gets no gradient)."""
    H = len(k_chunks)
    per_head = [len(k_chunks[h]) for h in range(H)]
    if [len(v) for v in v_chunks] != per_head:
        raise NSABackendError("k_chunks and v_chunks must hold the same chunks per head")
    bpc = chunk_len // block_size
    ids = block_indices.detach().to("cpu", torch.int64)
    sample = None
    for h in range(H):
        sel = ids[:, :, h, :]
        cids = torch.unique(sel[(sel >= 0) & (sel < per_head[h] * bpc)] // bpc).tolist()
        for c in cids:
            kc, vc = k_chunks[h][c], v_chunks[h][c]
            if not (kc.is_cuda and vc.is_cuda):
                if strict:
                    raise RuntimeError(
                        f"k/v_chunks[{h}][{c}] is not on the GPU: move it there before "
                        "selection_attention_padded_ptr_train, or pass strict=False to skip it")
                continue
            if kc.dtype != torch.bfloat16 or vc.dtype != torch.bfloat16:
                raise NSABackendError(f"pointer selection attention requires bf16 K/V storage, "
                                      f"got {kc.dtype} / {vc.dtype} for head {h}, chunk {c}")
            if sample is None:
                sample = kc
    if sample is None:
        raise AssertionError("no GPU-resident chunk is selected by block_indices")
    if not sample.is_contiguous():
        raise NSABackendError("chunk tensors must be contiguous [B, chunk_len, D]")
    e = sample.element_size()
    strides = {"batch_stride_bytes": sample.stride(0) * e,
               "token_stride_bytes": sample.stride(1) * e,
               "stride_bn": sample.stride(1), "stride_bd": sample.stride(2),
               "chunk_len": chunk_len}
    n_chunks = torch.tensor(per_head, dtype=torch.int32, device=q.device)
    k_flat = tuple(c for h in range(H) for c in k_chunks[h])
    v_flat = tuple(c for h in range(H) for c in v_chunks[h])
    return selection_attention_padded_ptr_train_fast(
        q, block_indices, block_size, group_size, chunk_len, max(per_head), n_chunks, strides,
        k_flat, v_flat, per_head, softmax_scale, input_precision)


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
