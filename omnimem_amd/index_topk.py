"""Top-k block selection with the reference's Python signatures.

Reference: src/omnimem/nsa/ops/index_topk.py:43-176 (facade), cuda_backend/ops.py:55-70 (op
adapter).  Differences, all extensions that leave the reference's accepted inputs unchanged:

* ``T % group_size`` and ``chunk_size % group_size`` need not be 0: the last query group may be
  ragged (pooled over its own tokens) and a group belongs to the chunk of its first token, the
  rule the selection kernel already uses (cuda_backend/csrc/selection_fwd.cu:218).
* ``blocks_per_chunk > 0`` selects chunk-aligned key blocks (block c lies in chunk
  c // blocks_per_chunk), the page layout of the paged KV cache.
* ``allow_tf32`` and ``bt_chunk`` are accepted and ignored.  Scores are fp32 sums of exact
  products: MFMA dot products for bf16 / f16 inputs with head dim 64 or 128 and top-k <= 16 (the
  role of the reference's TF32 WMMA), fmaf over d ascending otherwise.
* Top-k up to 128 follows the reference's path-A ordering (cuda_backend/csrc/topk.cu:584,
  648-660); 129 to 4096 its path-B ordering (topk.cu:741-807: raw order codes, so -0 below +0
  and visible -inf / NaN scores ranked, hidden blocks last as -1).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib, ops
from .backend import NSABackendError, get_backend

__all__ = [
    "parallel_nsa_topk",
    "parallel_nsa_topk_grouped_heads",
    "should_use_selection_attention",
    "block_pool",
    "topk",
    "topk_from_scores",
]


def block_pool(x: torch.Tensor, group: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Mean of each run of ``group`` consecutive tokens of x [B, T, H, D] (ragged tail allowed).

    The HIP replacement of ``x.view(B, T//g, g, H, D).mean(2)`` in x's dtype
    (``torch.ops.omnimem_nsa.block_pool``; with ``out`` the result is written in place)."""
    if out is None:
        return ops.op("block_pool")(x, int(group))
    return _block_pool_impl(x, group, out)


def _block_pool_impl(x: torch.Tensor, group: int, out: Optional[torch.Tensor] = None):
    _lib.require_cuda((x, "x"))
    B, T, H, D = x.shape
    MG = -(-T // group) if T else 0
    if out is None:
        out = torch.empty((B, MG, H, D), dtype=x.dtype, device=x.device)
    _lib.call("omm_block_pool", _lib.view4(x), _lib.view4(out), _lib.dtype_code(x), int(group),
              _lib.stream_of(x))
    return out


def _mask(block_size, group_size, chunk_q, chunk_k, causal, ex_win, ex_sink, prog_excl, tf_mask,
          q_chunk_offset, q_half, k_half, blocks_per_chunk) -> _lib.TopkMask:
    m = _lib.TopkMask()
    m.block_size, m.group_size = int(block_size), int(group_size)
    m.chunk_q, m.chunk_k = int(chunk_q), int(chunk_k)
    m.blocks_per_chunk = int(blocks_per_chunk)
    m.q_chunk_offset = int(q_chunk_offset)
    m.q_half, m.k_half = int(q_half), int(k_half)
    m.ex_win, m.ex_sink = int(ex_win), int(ex_sink)
    m.causal, m.tf_mask, m.prog_excl = int(bool(causal)), int(bool(tf_mask)), int(bool(prog_excl))
    return m


_INT32_MAX = 2 ** 31 - 1


def _check_int(name: str, v, lo: int = 0) -> int:
    v = int(v)
    if v < lo or v > _INT32_MAX:
        raise NSABackendError(f"{name}={v} out of the supported range [{lo}, {_INT32_MAX}]")
    return v


def topk(q: torch.Tensor, k: torch.Tensor, topk: int, scale: float, block_size: int,
         chunk_size: int, chunk_size_k: int, causal: bool, ex_win: int = 0, ex_sink: int = 0,
         prog_excl: bool = False, tf_mask: bool = False, q_chunk_offset: int = 0,
         allow_tf32: bool = True, group_size: int = 1, blocks_per_chunk: int = 0) -> torch.Tensor:
    """Op-level adapter, the counterpart of ``omnimem_nsa::topk`` (cuda_backend/ops.py:55-70).

    q: pooled rows [B, MG, H, D]; ``chunk_size`` counts rows as in the reference op, so the token
    chunk of the query side is chunk_size * group_size.  With the reference's arguments only
    (``group_size`` 1, ``blocks_per_chunk`` 0) the call goes through the registered
    ``torch.ops.omnimem_nsa.topk``."""
    if int(group_size) == 1 and int(blocks_per_chunk) == 0:
        return ops.op("topk")(q, k, int(topk), float(scale), int(block_size), int(chunk_size),
                              int(chunk_size_k), bool(causal), int(ex_win), int(ex_sink),
                              bool(prog_excl), bool(tf_mask), int(q_chunk_offset),
                              bool(allow_tf32))
    return _topk_impl(q, k, topk, scale, block_size, chunk_size, chunk_size_k, causal, ex_win,
                      ex_sink, prog_excl, tf_mask, q_chunk_offset, allow_tf32, group_size,
                      blocks_per_chunk)


def _topk_impl(q: torch.Tensor, k: torch.Tensor, topk: int, scale: float, block_size: int,
               chunk_size: int, chunk_size_k: int, causal: bool, ex_win: int = 0,
               ex_sink: int = 0, prog_excl: bool = False, tf_mask: bool = False,
               q_chunk_offset: int = 0, allow_tf32: bool = True, group_size: int = 1,
               blocks_per_chunk: int = 0) -> torch.Tensor:
    for name, v in (("block_size", block_size), ("chunk_size", chunk_size),
                    ("chunk_size_k", chunk_size_k), ("ex_win", ex_win), ("ex_sink", ex_sink),
                    ("q_chunk_offset", q_chunk_offset)):
        _check_int(name, v)
    _lib.require_cuda((q, "q"), (k, "k"))
    if q.dim() != 4 or k.dim() != 4:
        raise NSABackendError("topk: expected q [B,MG,H,D] and k [B,NC,H,D]")
    if q.dtype != k.dtype:
        raise NSABackendError(f"topk: q and k must share a dtype, got {q.dtype} vs {k.dtype}")
    B, MG, H, _ = q.shape
    NC = k.shape[1]
    q_half = MG // (2 * chunk_size) if tf_mask else 0
    k_half = (NC * block_size) // (2 * chunk_size_k) if tf_mask else 0
    m = _mask(block_size, group_size, int(chunk_size) * int(group_size), chunk_size_k, causal,
              ex_win, ex_sink, prog_excl, tf_mask, q_chunk_offset, q_half, k_half,
              blocks_per_chunk)
    out = torch.empty((B, MG, H, int(topk)), dtype=torch.int32, device=q.device)
    ws_n = _lib.lib().omm_topk_workspace_bytes(B, MG, H, NC, int(topk))
    ws = _lib.workspace(ws_n, q.device)
    _lib.call("omm_topk", _lib.view4(q), _lib.view4(k), _lib.dtype_code(q), int(topk),
              float(scale), m, out.data_ptr() if out.numel() else None, ws.data_ptr(), ws_n,
              _lib.stream_of(q))
    return out


def topk_from_scores(scores: torch.Tensor, topk: int, block_size: int, chunk_size: int,
                     chunk_size_k: int, causal: bool, ex_win: int = 0, ex_sink: int = 0,
                     prog_excl: bool = False, tf_mask: bool = False, q_chunk_offset: int = 0,
                     group_size: int = 1, blocks_per_chunk: int = 0) -> torch.Tensor:
    """Selection only: fp32 scores [B, MG, H, NC] (already scaled) -> int32 [B, MG, H, topk]."""
    _lib.require_cuda((scores, "scores"))
    if scores.dtype != torch.float32 or scores.dim() != 4:
        raise NSABackendError("topk_from_scores: scores must be fp32 [B, MG, H, NC]")
    scores = scores.contiguous()
    B, MG, H, NC = scores.shape
    q_half = MG // (2 * chunk_size) if tf_mask else 0
    k_half = (NC * block_size) // (2 * chunk_size_k) if tf_mask else 0
    m = _mask(block_size, group_size, int(chunk_size) * int(group_size), chunk_size_k, causal,
              ex_win, ex_sink, prog_excl, tf_mask, q_chunk_offset, q_half, k_half,
              blocks_per_chunk)
    out = torch.empty((B, MG, H, int(topk)), dtype=torch.int32, device=scores.device)
    ws_n = _lib.lib().omm_topk_workspace_bytes(B, MG, H, NC, int(topk))
    ws = _lib.workspace(ws_n, scores.device)
    _lib.call("omm_topk_from_scores", scores.data_ptr(), B, MG, H, NC, int(topk), m,
              out.data_ptr() if out.numel() else None, ws.data_ptr(), ws_n,
              _lib.stream_of(scores))
    return out


def parallel_nsa_topk(
        q: torch.Tensor,       # [B, T, H, K]
        k: torch.Tensor,       # [B, TC, H, K]
        block_counts: int,
        block_size: int = 64,
        scale: Optional[float] = None,
        chunk_size: int = 64,
        causal: bool = True,
        bt_chunk: int = 512,
        allow_tf32: bool = True,
        group_size: int = 1,
        exclude_window_chunks: int = 0,
        exclude_sink_chunks: int = 0,
        progressive_exclude: bool = False,
        tf_mask: bool = False,
        q_chunk_offset: int = 0,
        blocks_per_chunk: int = 0,
) -> torch.Tensor:
    """Top-``block_counts`` compressed-key blocks per query group: int32 [B, ceil(T/G), H, S].

    Same arguments and result as the reference (nsa/ops/index_topk.py:43-105); -1 marks slots
    with no visible block.  Query-group pooling, scoring and selection run in one HIP call."""
    get_backend()
    assert not (tf_mask and q_chunk_offset), \
        "tf_mask assumes a full [clean|noisy] layout; q_chunk_offset must be 0"
    _lib.require_cuda((q, "q"), (k, "k"))
    if q.dim() != 4 or k.dim() != 4:
        raise NSABackendError("parallel_nsa_topk: expected q [B,T,H,K] and k [B,TC,H,K]")
    if q.dtype != k.dtype:
        raise NSABackendError(f"topk: q and k must share a dtype, got {q.dtype} vs {k.dtype}")
    B, T, H, K = q.shape
    G = int(group_size)
    if G < 1:
        raise ValueError(f"group_size must be >= 1, got {G}")
    MG = -(-T // G)
    NC = k.shape[1]
    if tf_mask:
        assert chunk_size % G == 0 and T % G == 0, "tf_mask requires G | chunk_size and G | T"
        rows = chunk_size // G
        assert MG % (2 * rows) == 0, (
            f"tf_mask=True requires T ({MG}) divisible by 2*chunk_size ({2 * rows}); "
            f"Q must be laid out as [clean | noisy] with equal halves.")
        kchunk_blocks = chunk_size // block_size
        assert NC % (2 * kchunk_blocks) == 0, (
            f"tf_mask=True requires TC ({NC}) divisible by 2 * (chunk_size_k/block_size) "
            f"({2 * kchunk_blocks}); K layout must be [clean | noisy] with equal halves.")
    for name, v in (("block_size", block_size), ("chunk_size", chunk_size),
                    ("exclude_window_chunks", exclude_window_chunks),
                    ("exclude_sink_chunks", exclude_sink_chunks),
                    ("q_chunk_offset", q_chunk_offset)):
        _check_int(name, v)
    sc = scale if scale is not None else K ** -0.5
    return ops.op("topk_fused")(q, k, int(block_counts), float(sc), int(block_size),
                                int(chunk_size), bool(causal), int(exclude_window_chunks),
                                int(exclude_sink_chunks), bool(progressive_exclude),
                                bool(tf_mask), int(q_chunk_offset), G, int(blocks_per_chunk))


def _topk_fused_impl(q: torch.Tensor, k: torch.Tensor, S: int, sc: float, block_size: int,
                     chunk_size: int, causal: bool, ex_win: int, ex_sink: int, prog_excl: bool,
                     tf_mask: bool, q_chunk_offset: int, G: int,
                     blocks_per_chunk: int) -> torch.Tensor:
    """``torch.ops.omnimem_nsa.topk_fused`` on the GPU: query pooling + scores + top-k in one
    C-ABI call (``chunk_size`` in tokens on both sides)."""
    _lib.require_cuda((q, "q"), (k, "k"))
    B, T, H, K = q.shape
    MG = -(-T // G)
    NC = k.shape[1]
    q_half = (MG * G) // (2 * chunk_size) if tf_mask else 0
    k_half = (NC * block_size) // (2 * chunk_size) if tf_mask else 0
    m = _mask(block_size, G, chunk_size, chunk_size, causal, ex_win, ex_sink, prog_excl, tf_mask,
              q_chunk_offset, q_half, k_half, blocks_per_chunk)
    out = torch.empty((B, MG, H, S), dtype=torch.int32, device=q.device)
    dt = _lib.dtype_code(q)
    ws_n = _lib.lib().omm_topk_fused_workspace_bytes(B, T, H, K, NC, G, S, dt)
    ws = _lib.workspace(ws_n, q.device)
    _lib.call("omm_topk_fused", _lib.view4(q), _lib.view4(k), dt, G, S, float(sc), m,
              out.data_ptr() if out.numel() else None, ws.data_ptr(), ws_n, _lib.stream_of(q))
    return out


def parallel_nsa_topk_with_scores(q: torch.Tensor, k: torch.Tensor, block_counts: int,
                                  block_size: int = 64, scale: Optional[float] = None,
                                  chunk_size: int = 64, causal: bool = True, group_size: int = 1,
                                  exclude_window_chunks: int = 0, exclude_sink_chunks: int = 0,
                                  progressive_exclude: bool = False, tf_mask: bool = False,
                                  q_chunk_offset: int = 0, blocks_per_chunk: int = 0):
    """Inspection hook: ``parallel_nsa_topk``'s indices together with the fp32 block scores its
    selection ran on ([B, ceil(T/G), H, TC]; NaN where a row's columns were not scored because
    the mask hides them).  bf16 / f16 inputs with head dim 64 or 128 (the MFMA path)."""
    _lib.require_cuda((q, "q"), (k, "k"))
    B, T, H, K = q.shape
    G = int(group_size)
    MG = -(-T // G)
    NC = k.shape[1]
    sc = scale if scale is not None else K ** -0.5
    q_half = (MG * G) // (2 * chunk_size) if tf_mask else 0
    k_half = (NC * block_size) // (2 * chunk_size) if tf_mask else 0
    m = _mask(block_size, G, chunk_size, chunk_size, causal, exclude_window_chunks,
              exclude_sink_chunks, progressive_exclude, tf_mask, q_chunk_offset, q_half, k_half,
              blocks_per_chunk)
    S = int(block_counts)
    out = torch.empty((B, MG, H, S), dtype=torch.int32, device=q.device)
    scores = torch.full((B, MG, H, NC), float("nan"), dtype=torch.float32, device=q.device)
    dt = _lib.dtype_code(q)
    ws_n = _lib.lib().omm_topk_fused_workspace_bytes(B, T, H, K, NC, G, S, dt)
    ws = _lib.workspace(ws_n, q.device)
    _lib.call("omm_topk_fused_debug", _lib.view4(q), _lib.view4(k), dt, G, S, float(sc), m,
              out.data_ptr() if out.numel() else None, scores.data_ptr(), ws.data_ptr(), ws_n,
              _lib.stream_of(q))
    return out, scores


def parallel_nsa_topk_grouped_heads(
    q: torch.Tensor,           # [B, T, H, K]
    k: torch.Tensor,           # [B, TC, H, K]
    num_kv_head_groups: int,
    block_counts: int,
    block_size: int,
    chunk_size: int,
    causal: bool = False,
    group_size: int = 1,
    tf_mask=False,
    **topk_kwargs,
) -> torch.Tensor:
    """GQA-style head pooling, then ``parallel_nsa_topk``; indices broadcast back to H heads.

    Reference: nsa/ops/index_topk.py:108-162 (head pool first, then query pool; both in the
    input dtype).  Head pooling runs on the same HIP pooling kernel over the head axis."""
    B, T, H, K = q.shape
    TC = k.shape[1]
    assert H % num_kv_head_groups == 0
    if num_kv_head_groups == H:
        return parallel_nsa_topk(q=q, k=k, block_counts=block_counts, block_size=block_size,
                                 chunk_size=chunk_size, causal=causal, group_size=group_size,
                                 tf_mask=tf_mask, **topk_kwargs)
    hpg = H // num_kv_head_groups

    def head_pool(x: torch.Tensor, n: int) -> torch.Tensor:
        # [B, n, H, K] viewed as [B*n, H, 1, K]; pool runs of hpg consecutive heads
        xv = x.reshape(B * n, H, 1, K)
        return block_pool(xv, hpg).reshape(B, n, num_kv_head_groups, K)

    qg = head_pool(q, T)
    kg = head_pool(k, TC)
    idx = parallel_nsa_topk(q=qg, k=kg, block_counts=block_counts, block_size=block_size,
                            chunk_size=chunk_size, causal=causal, group_size=group_size,
                            tf_mask=tf_mask, **topk_kwargs)
    return (idx.unsqueeze(-2).expand(-1, -1, -1, hpg, -1)
            .reshape(idx.shape[0], idx.shape[1], H, idx.shape[-1]))


def should_use_selection_attention(seq_len, chunk_size, exclude_window_chunks, exclude_sink_chunks,
                                   causal=True):
    """Host-only gate, as nsa/ops/index_topk.py:165-176."""
    total_chunks = math.ceil(seq_len / chunk_size)
    if causal:
        max_visible = total_chunks
        excluded = min(exclude_sink_chunks, max_visible) + min(exclude_window_chunks, max_visible)
        return max_visible - excluded > 0
    excluded = exclude_window_chunks + exclude_sink_chunks
    return total_chunks - excluded > 0
