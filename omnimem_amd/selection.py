"""Dense selection attention with the reference's Python signature.

Reference: src/omnimem/nsa/ops/selection/__init__.py:12-100 (facade and validation),
cuda_backend/ops.py:90-117 (op adapters) and cuda_backend/autograd.py:9-45 (autograd wiring:
the forward saves q, k, v, ids, out and lse; the backward returns dq, dk, dv).  The backward
runs on gfx950 MFMA for bf16 / f16 with head dim 64 or 128, and on fp32 VALU kernels for fp32
and every other head dim up to 256.
Extension: ``M % group_size`` need not be 0 (the last query group may be ragged).
"""
from __future__ import annotations

import math
import os
from typing import Optional, Tuple

import torch

from . import _lib, ops
from .backend import NSABackendError, get_backend

__all__ = ["selection_attention", "sel_fwd", "sel_fwd_gated", "sel_bwd", "dense_attention"]


def _debug_checks_enabled() -> bool:
    return os.environ.get("OMNIMEM_NSA_DEBUG", "0") not in ("", "0", "false", "False")


def _validate_common(q, k, v, block_indices, block_size, chunk_size, group_size, causal):
    """Argument checks of the reference facade (nsa/ops/selection/__init__.py:16-44)."""
    B, M, H, D = q.shape
    N = k.shape[1]
    G = group_size
    assert k.shape == (B, N, H, D), f"expected k {(B, N, H, D)}, got {tuple(k.shape)}"
    assert v.shape == (B, N, H, D), f"expected v {(B, N, H, D)}, got {tuple(v.shape)}"
    assert D >= 16, f"expected D >= 16, but got {D}"
    MG = -(-M // G)
    assert block_indices.dim() == 4 and block_indices.shape[:3] == (B, MG, H), (
        f"Expected block_indices {(B, MG, H, '*')}, got {tuple(block_indices.shape)}")
    if chunk_size <= 0:
        raise ValueError(f"chunk_size must be > 0, got {chunk_size}")
    if block_indices.shape[-1] == 0:
        raise ValueError("top_idx last dim T must be > 0")
    num_blocks = math.ceil(N / block_size)
    # One host sync per call, as in the reference; the op-level sel_fwd() skips it.  A traced
    # graph cannot branch on tensor values, so there the same check runs as an op of the graph
    # and raises the same ValueError when the graph runs.
    if torch.compiler.is_compiling():
        ops.op("check_block_ids")(block_indices.new_empty((1,)), block_indices, num_blocks)
    else:
        ops.check_block_ids_now(block_indices, num_blocks)
    return num_blocks


def _debug_check_unique(block_indices):
    ids = block_indices.to(torch.int64)
    sorted_ids, _ = ids.sort(dim=-1)
    dup = (sorted_ids[..., 1:] == sorted_ids[..., :-1]) & (sorted_ids[..., 1:] >= 0)
    if dup.any():
        raise ValueError("duplicate valid block ids within a row are not allowed (OMNIMEM_NSA_DEBUG)")


def _grad_needed(*ts) -> bool:
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad
                                           for t in ts)


def _check_bwd_supported(q):
    if q.shape[-1] > 256:
        raise NotImplementedError(
            f"selection attention backward supports head dims up to 256 (got {q.shape[-1]}); "
            "call under torch.no_grad() or detach the inputs")


def sel_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
            block_size: int, chunk_size: int, scale: float, causal: bool, group_size: int,
            allow_tf32: bool = True, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Op-level adapter (counterpart of ``omnimem_nsa::sel_fwd``): returns (out, lse [B,H,M] f32).

    No host synchronisation; ids outside [0, ceil(N/block_size)) are skipped by the kernel.
    Without ``out`` / ``lse`` the call goes through ``torch.ops.omnimem_nsa.sel_fwd``."""
    if out is None and lse is None:
        return ops.op("sel_fwd")(q, k, v, block_indices, int(block_size), int(chunk_size),
                                 float(scale), bool(causal), int(group_size), bool(allow_tf32))
    return _sel_fwd_impl(q, k, v, block_indices, block_size, chunk_size, scale, causal,
                         group_size, out, lse)


def _sel_fwd_impl(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
                  block_size: int, chunk_size: int, scale: float, causal: bool, group_size: int,
                  out: Optional[torch.Tensor] = None,
                  lse: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    _lib.require_cuda((q, "q"), (k, "k"), (v, "v"), (block_indices, "block_indices"))
    if not (q.dtype == k.dtype == v.dtype):
        raise NSABackendError(f"sel_fwd: q/k/v must share one dtype, got {q.dtype}/{k.dtype}/{v.dtype}")
    if block_indices.dtype != torch.int32:
        block_indices = block_indices.to(torch.int32)
    B, M, H, D = q.shape
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty((B, H, M), dtype=torch.float32, device=q.device)
    # fp32 calls with few items per CU split into equal runs and merge through a workspace
    ws_bytes = _lib.lib().omm_sel_fwd_workspace_bytes(
        B, M, H, D, block_indices.shape[-1], _lib.dtype_code(q), int(group_size))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=q.device) if ws_bytes else None
    _lib.call("omm_sel_fwd_ws", _lib.view4(q), _lib.view4(k), _lib.view4(v),
              _lib.view4(block_indices), _lib.dtype_code(q), int(block_size), int(chunk_size),
              int(bool(causal)), int(group_size), float(scale), _lib.view4(out),
              lse.data_ptr() if lse.numel() else None,
              ws.data_ptr() if ws is not None else None, ws_bytes, _lib.stream_of(q))
    return out, lse


def sel_fwd_gated(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
                  block_size: int, chunk_size: int, scale: float, causal: bool, group_size: int,
                  gates: torch.Tensor, o_cmp: torch.Tensor, o_swa: torch.Tensor,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``sel_fwd`` with the NSA branch mix in the kernel's epilogue (bf16): returns
    ``g[..., 0] * o_cmp + g[..., 1] * o_slc + g[..., 2] * o_swa`` computed in fp32 from the
    unrounded selection output o_slc and rounded once, as the full-sequence branch of
    causal_wan_nsa_model.py:391-458 combines them (:541-546).  gates: bf16 [B, M, H, 3] after the
    clamp and sigmoid; o_cmp / o_swa: bf16 like q; ``out`` must not overlap them."""
    _lib.require_cuda((q, "q"), (k, "k"), (v, "v"), (block_indices, "block_indices"),
                      (gates, "gates"), (o_cmp, "o_cmp"), (o_swa, "o_swa"))
    for name, t in (("q", q), ("k", k), ("v", v), ("gates", gates), ("o_cmp", o_cmp),
                    ("o_swa", o_swa)):
        if t.dtype != torch.bfloat16:
            raise NSABackendError(f"sel_fwd_gated: {name} must be bf16, got {t.dtype}")
    if block_indices.dtype != torch.int32:
        block_indices = block_indices.to(torch.int32)
    if out is None:
        out = torch.empty_like(q)
    _lib.call("omm_sel_fwd_gated", _lib.view4(q), _lib.view4(k), _lib.view4(v),
              _lib.view4(block_indices), int(block_size), int(chunk_size), int(bool(causal)),
              int(group_size), float(scale), _lib.view4(gates), _lib.view4(o_cmp),
              _lib.view4(o_swa), _lib.view4(out), None, _lib.stream_of(q))
    return out


def sel_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
            out: torch.Tensor, lse: torch.Tensor, d_out: torch.Tensor, block_size: int,
            chunk_size: int, scale: float, causal: bool, group_size: int,
            allow_tf32: bool = True) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Op-level adapter (counterpart of ``omnimem_nsa::sel_bwd``): returns (dq, dk, dv) in the
    q / k / v dtypes.  No host synchronisation.  ``allow_tf32`` is accepted for signature
    compatibility: 16-bit inputs use 16-bit MFMA operands with fp32 accumulation, fp32 inputs
    full fp32 arithmetic.  Runs as ``torch.ops.omnimem_nsa.sel_bwd``."""
    return ops.op("sel_bwd")(q, k, v, block_indices, out, lse, d_out, int(block_size),
                             int(chunk_size), float(scale), bool(causal), int(group_size),
                             bool(allow_tf32))


def _sel_bwd_impl(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
                  out: torch.Tensor, lse: torch.Tensor, d_out: torch.Tensor, block_size: int,
                  chunk_size: int, scale: float, causal: bool,
                  group_size: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    _lib.require_cuda((q, "q"), (k, "k"), (v, "v"), (block_indices, "block_indices"),
                      (out, "out"), (lse, "lse"), (d_out, "d_out"))
    if not (q.dtype == k.dtype == v.dtype == out.dtype == d_out.dtype):
        raise NSABackendError("sel_bwd: q/k/v/out/d_out must share one dtype")
    if lse.dtype != torch.float32 or not lse.is_contiguous():
        raise NSABackendError("sel_bwd: lse must be contiguous fp32 [B, H, M]")
    if block_indices.dtype != torch.int32:
        block_indices = block_indices.to(torch.int32)
    B, M, H, D = q.shape
    N = k.shape[1]
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    if B == 0 or M == 0 or H == 0:
        return dq, dk.zero_(), dv.zero_()
    T = block_indices.shape[-1]
    ws = _lib.workspace(_lib.lib().omm_sel_bwd_workspace_bytes(B, M, H, N, int(block_size),
                                                               int(group_size), T), q.device)
    _lib.call("omm_sel_bwd", _lib.view4(q), _lib.view4(k), _lib.view4(v),
              _lib.view4(block_indices), _lib.view4(out), lse.data_ptr(), _lib.view4(d_out),
              _lib.dtype_code(q), int(block_size), int(chunk_size), int(bool(causal)),
              int(group_size), float(scale), _lib.view4(dq), _lib.view4(dk), _lib.view4(dv),
              ws.data_ptr(), ws.numel(), _lib.stream_of(q))
    return dq, dk, dv


class SelectionAttentionFn(torch.autograd.Function):
    """Autograd wiring of the reference's SelectionAttentionCUDA (cuda_backend/autograd.py:9-45)."""

    @staticmethod
    def forward(ctx, q, k, v, block_indices, block_size, chunk_size=1, softmax_scale=None,
                causal=False, return_lse=False, allow_tf32=True, bwd_method='auto',
                group_size=1):
        if softmax_scale is None:
            softmax_scale = 1.0 / (q.shape[-1] ** 0.5)
        out, lse = sel_fwd(q, k, v, block_indices, block_size, chunk_size, softmax_scale, causal,
                           group_size, allow_tf32)
        ctx.save_for_backward(q, k, v, block_indices, out, lse)
        ctx.args = (block_size, chunk_size, softmax_scale, causal, group_size, allow_tf32)
        if return_lse:
            ctx.mark_non_differentiable(lse)
            return out, lse
        return out

    @staticmethod
    def backward(ctx, *grad_outputs):
        q, k, v, block_indices, out, lse = ctx.saved_tensors
        block_size, chunk_size, scale, causal, group_size, allow_tf32 = ctx.args
        dq, dk, dv = sel_bwd(q, k, v, block_indices, out, lse, grad_outputs[0], block_size,
                             chunk_size, scale, causal, group_size, allow_tf32)
        return dq, dk, dv, None, None, None, None, None, None, None, None, None


def selection_attention(
        q, k, v,
        block_indices,
        block_count,
        block_size,
        chunk_size=1,
        scale=None,
        variant='two-pass',
        causal=False,
        return_lse=False,
        allow_tf32=True,
        bwd_method='auto',
        group_size=1,
):
    """Selection attention forward, q [B,M,H,D], k/v [B,N,H,D], block_indices [B,M/G,H,T].

    Same arguments, validation and result as the reference (nsa/ops/selection/__init__.py:56);
    returns out (q dtype) or (out, lse [B,H,M] fp32) with ``return_lse``."""
    if variant not in ('one-pass', 'two-pass'):
        raise ValueError(f"Invalid variant: {variant!r}, expected 'one-pass' or 'two-pass'")
    if group_size < 1:
        raise ValueError(f"Invalid group_size: {group_size}, expected >= 1")
    if variant == 'one-pass':
        raise NotImplementedError(f"{variant=} is not supported")
    if bwd_method not in ('auto', 'mask', 'inverted'):
        raise ValueError(f"Unknown bwd_method '{bwd_method}', expected 'auto', 'inverted' or 'mask'")
    get_backend()
    _validate_common(q, k, v, block_indices, block_size, chunk_size, group_size, causal)
    if not torch.compiler.is_compiling() and _debug_checks_enabled():
        _debug_check_unique(block_indices)
    if block_indices.dtype != torch.int32:
        block_indices = block_indices.to(torch.int32)
    sc = scale if scale is not None else q.shape[-1] ** -0.5
    if _grad_needed(q, k, v):
        _check_bwd_supported(q)
        return SelectionAttentionFn.apply(q, k, v, block_indices, block_size, chunk_size, sc,
                                          causal, return_lse, allow_tf32, bwd_method, group_size)
    out, lse = sel_fwd(q, k, v, block_indices, block_size, chunk_size, sc, causal, group_size,
                       allow_tf32)
    return (out, lse) if return_lse else out


_ALL_BLOCKS = {}


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    scale: Optional[float] = None, return_lse: bool = False,
                    out: Optional[torch.Tensor] = None):
    """Full (non-causal) softmax attention of q [B, M, H, D] over k, v [B, N, H, D], computed by
    the selection kernel with every 64-token block listed for every 128-query group.

    This is the AR driver's compressed-history branch (o_cmp over the pooled keys,
    models/transformers/causal_wan_nsa_model.py:506) and window branch (o_swa,
    :508), which the reference runs through flash attention.  The block list is one
    ``arange`` broadcast with stride 0 over groups and heads, so a call allocates nothing but
    the output.  Returns out (q's layout) or (out, lse [B, H, M] fp32)."""
    _lib.require_cuda((q, "q"), (k, "k"), (v, "v"))
    B, M, H, D = q.shape
    N = k.shape[1]
    if k.shape != (B, N, H, D) or v.shape != (B, N, H, D):
        raise NSABackendError(f"dense_attention: expected k, v {(B, N, H, D)}, got "
                              f"{tuple(k.shape)} / {tuple(v.shape)}")
    # 128-query groups: the kernel then runs 4-wave workgroups that share each K/V tile between
    # two 64-query halves (the same blocks are listed for every group, so the result does not
    # depend on the grouping)
    G, BS = 128, 64
    T = max(1, -(-N // BS))
    key = (q.device, T)
    ar = _ALL_BLOCKS.get(key)
    if ar is None:
        ar = torch.arange(T, dtype=torch.int32, device=q.device)
        _ALL_BLOCKS[key] = ar
    ids = ar.view(1, 1, 1, T).expand(B, -(-M // G), H, T)
    o, lse = sel_fwd(q, k, v, ids, BS, 1, D ** -0.5 if scale is None else scale, False, G,
                     out=out,
                     lse=None if return_lse else torch.empty(0, device=q.device))
    return (o, lse) if return_lse else o
