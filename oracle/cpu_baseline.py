"""CPU baseline of the NSA selection path -- TEST INFRASTRUCTURE ONLY.

Only ``bench.py``'s ``cpu_baseline`` leg and ``tests/`` use this module, to time (and check) the
reference's PyTorch CPU formulation beside the HIP path.  The product package ``omnimem_amd``
never imports it.

It restates, in torch on the CPU, the reference's naive path:

* ``select_attention_chunked`` follows ``select_attention_torch_chunk``
  (src/omnimem/nsa/naive/select_attention.py:53-149): permute to [B, H, ., .] (:85), for each
  32-query chunk (:88) gather the selected K/V token rows into [B, H, q, S*BS, D] (:117-124),
  fp32 einsum with the scale folded into q (:126-130), chunk-causal mask on token positions
  (:131-135), online softmax over kv sub-chunks (:137-144), normalise and cast (:146).
  Token ids come from ``inflate_indices`` (src/omnimem/nsa/naive/index_selection.py:155-166).
  Two departures, both required by inputs the reference path cannot take: ids of -1 and token
  ids >= N (the partial last block) are masked to -inf instead of being gathered (the reference
  would index out of range), and a row with no visible token returns 0 (the CUDA kernel's
  convention, cuda_backend/csrc/selection_fwd.cu:3) instead of NaN.
* ``topk_scores`` follows ``index_selection_topk`` (nsa/naive/index_selection.py:6-54):
  ``q @ k_cmp^T * scale``, chunk-causal mask on (q // chunk, (k * bs) // chunk), ``torch.topk``;
  ties are then re-ordered to (score desc, id asc) by a stable sort, the rule of the CUDA op.
"""
from __future__ import annotations

import torch


def inflate_indices(top_idx: torch.Tensor, block_size: int) -> torch.Tensor:
    """[B, M, H, T] block ids -> [B, M, H, T*block_size] token ids (-1 blocks stay negative)."""
    B, M, H, T = top_idx.shape
    off = torch.arange(block_size, dtype=top_idx.dtype)
    tok = top_idx.unsqueeze(-1) * block_size + off
    tok = torch.where(top_idx.unsqueeze(-1) < 0, torch.full_like(tok, -1), tok)
    return tok.reshape(B, M, H, T * block_size)


def select_attention_chunked(q, k, v, token_idx, scale=None, causal=False, chunk_size=None,
                             q_chunk_size: int = 32, kv_chunk_size=None):
    """q [B, M, H, D], k/v [B, N, H, D], token_idx int64 [B, M, H, S] -> out [B, M, H, D]."""
    B, M, H, D = q.shape
    N = k.shape[1]
    S = token_idx.shape[-1]
    if kv_chunk_size is None:
        kv_chunk_size = S
    if scale is None:
        scale = D ** -0.5
    q, k, v, token_idx = (x.permute(0, 2, 1, 3).contiguous() for x in (q, k, v, token_idx))
    out = torch.empty_like(q)
    for q0 in range(0, M, q_chunk_size):
        q1 = min(q0 + q_chunk_size, M)
        nq = q1 - q0
        qc = q[:, :, q0:q1].to(torch.float32) * scale
        idx_q = token_idx[:, :, q0:q1]
        m_i = torch.full((B, H, nq), -torch.inf)
        l_i = torch.zeros((B, H, nq))
        o_i = torch.zeros((B, H, nq, D))
        for s0 in range(0, S, kv_chunk_size):
            s1 = min(s0 + kv_chunk_size, S)
            tok = idx_q[..., s0:s1]
            ok = (tok >= 0) & (tok < N)
            safe = torch.where(ok, tok, torch.zeros_like(tok))
            gidx = safe.unsqueeze(-1).expand(-1, -1, -1, -1, D)
            sk = torch.gather(k.unsqueeze(2).expand(-1, -1, nq, -1, -1), 3, gidx).to(torch.float32)
            sv = torch.gather(v.unsqueeze(2).expand(-1, -1, nq, -1, -1), 3, gidx).to(torch.float32)
            qk = torch.einsum("bhqd,bhqkd->bhqk", qc, sk)
            if causal:
                qpos = torch.arange(q0, q1).view(1, 1, -1, 1)
                ok = ok & ((tok // chunk_size) <= (qpos // chunk_size))
            qk = qk.masked_fill(~ok, float("-inf"))
            m_new = torch.maximum(m_i, qk.max(dim=-1).values)
            m_safe = torch.where(torch.isinf(m_new), torch.zeros_like(m_new), m_new)
            alpha = torch.exp(m_i - m_safe)
            p = torch.exp(qk - m_safe.unsqueeze(-1))
            l_i = l_i * alpha + p.sum(-1)
            o_i = o_i * alpha.unsqueeze(-1) + torch.einsum("bhqk,bhqkd->bhqd", p, sv)
            m_i = m_new
        den = torch.where(l_i > 0, l_i, torch.ones_like(l_i))
        out[:, :, q0:q1] = (o_i / den.unsqueeze(-1)).to(q.dtype)
    return out.permute(0, 2, 1, 3).contiguous()


def topk_scores(q, k_cmp, block_count: int, scale=None, causal=False, chunk_size=None,
                block_size=None, group_size: int = 1) -> torch.Tensor:
    """q [B, T, H, D] (already pooled by group_size), k_cmp [B, TC, H, D] -> int32 [B, T, H, S].

    chunk_size counts tokens; pooled row g lies in chunk (g * group_size) // chunk_size."""
    B, T, H, D = q.shape
    TC = k_cmp.shape[1]
    if scale is None:
        scale = D ** -0.5
    qh, kh = (x.permute(0, 2, 1, 3).to(torch.float32) for x in (q, k_cmp))
    score = (qh @ kh.transpose(-2, -1)) * scale
    if causal:
        qi = torch.arange(T).view(1, 1, -1, 1)
        ki = torch.arange(TC).view(1, 1, 1, -1)
        score = score.masked_fill(((qi * group_size) // chunk_size) < ((ki * block_size) // chunk_size),
                                  float("-inf"))
    score = score.permute(0, 2, 1, 3)
    val, idx = torch.topk(score, block_count, dim=-1)
    # (score desc, id asc): stable sort by id, then by score
    idx, order = torch.sort(idx, dim=-1)
    val = torch.gather(val, -1, order)
    val, order = torch.sort(val, dim=-1, descending=True, stable=True)
    idx = torch.gather(idx, -1, order)
    return torch.where(torch.isinf(val), torch.full_like(idx, -1), idx).to(torch.int32)
