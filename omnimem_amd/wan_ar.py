"""Wan2.1-shaped causal NSA DiT for autoregressive (AR) chunk generation over the paged cache.

This is the caller counterpart of the selection path: random-init weights of the Wan2.1-T2V-1.3B
shape (30 blocks, dim 1536, 12 heads x 128, FFN 8960, 512 text tokens), the NSA self-attention
of the reference's AR inference branch, and the AR loop of its pipeline:

* block: src/omnimem/models/transformers/causal_wan_nsa_model.py:626-700
  (``CausalWanNSAttentionBlock``: adaLN modulation, self-attention, cross-attention, FFN);
* NSA self-attention, AR branch (block_mask None): :354-386 and :461-552 -- q/k/v projections,
  RMSNorm on q and k, rotary embedding, sigmoid gates from ``g_proj`` clamped to [-10, 10],
  K/V block compression into the cache, compressed attention over the pooled history, sliding
  window attention over the last ``window`` chunks, top-k + selection attention over the cache
  (:182-239: ``causal=False``, ``chunk_size`` = chunk tokens, ``q_chunk_offset`` = chunk id,
  window exclusion with progressive gating), gate combine, output projection;
* AR loop: src/omnimem/pipelines/pipeline_wan_causal.py:350-474 -- per chunk, 4 denoise forwards
  and 1 context forward (t = 0) that rewrite the chunk's cache entries, then the offload flush.

What stays PyTorch-ROCm (dense, off the selection path): the linear layers (hipBLASLt), the
norms and the cross-attention.  The compressed attention runs on the selection kernel
(``dense_attention``: every pooled block listed for every query group), and so does the window
attention (``PagedKVCache.window_attention``: the window's pages read in place, or a dense ring
for an fp8 cache).
Rotary embedding is a plain interleaved rotation over the head dim with per-position angles (the
reference's 3-axis frequency split and token reorder only permute which angles a token gets).
The scheduler arithmetic between denoise steps is one axpy: timing does not depend on it.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .block_cache import PagedKVCache
from .index_topk import parallel_nsa_topk
from .selection import dense_attention

__all__ = ["WanARConfig", "WanNSAAR"]


@dataclass
class WanARConfig:
    layers: int = 30
    dim: int = 1536
    ffn_dim: int = 8960
    heads: int = 12
    text_len: int = 512
    text_dim: int = 4096
    freq_dim: int = 256
    in_dim: int = 16                 # latent channels
    patch: int = 4                   # 1 x 2 x 2 patch
    frame_tokens: int = 1560         # 30 x 52 latent patches per frame (480 x 832 video)
    frames_per_chunk: int = 3
    page_tokens: int = 64            # selection block (BASELINE: 64)
    group_size: int = 64             # queries sharing one top-k row
    topk: int = 16
    exclude_window_chunks: int = 3
    exclude_sink_chunks: int = 0
    progressive_exclude: bool = True
    window_chunks: int = 3           # sliding-window attention span, in chunks
    denoise_steps: int = 4
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads

    @property
    def chunk_tokens(self) -> int:
        return self.frame_tokens * self.frames_per_chunk


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w


def _ln(x: torch.Tensor, eps: float, w=None, b=None) -> torch.Tensor:
    return F.layer_norm(x.float(), (x.shape[-1],), w, b, eps).to(x.dtype)


class _Block:
    """Weights of one NSA block (random init, seeded)."""

    def __init__(self, cfg: WanARConfig, gen: torch.Generator, device, dtype):
        d, f = cfg.dim, cfg.ffn_dim

        def lin(o, i):
            w = torch.randn((o, i), generator=gen) * (1.0 / math.sqrt(i))
            return w.to(device=device, dtype=dtype), torch.zeros(o, device=device, dtype=dtype)

        self.q, self.k, self.v, self.o = lin(d, d), lin(d, d), lin(d, d), lin(d, d)
        self.norm_q = torch.ones(d, device=device, dtype=dtype)
        self.norm_k = torch.ones(d, device=device, dtype=dtype)
        gw = torch.randn((3 * cfg.heads, d), generator=gen) * 1e-3
        self.g = (gw.to(device=device, dtype=dtype), torch.zeros(3 * cfg.heads, device=device, dtype=dtype))
        self.cq, self.ck, self.cv, self.co = lin(d, d), lin(d, d), lin(d, d), lin(d, d)
        self.cnorm_q = torch.ones(d, device=device, dtype=dtype)
        self.cnorm_k = torch.ones(d, device=device, dtype=dtype)
        self.norm3_w = torch.ones(d, device=device, dtype=torch.float32)
        self.norm3_b = torch.zeros(d, device=device, dtype=torch.float32)
        self.f1, self.f2 = lin(f, d), lin(d, f)
        self.modulation = (torch.randn((1, 6, d), generator=gen) / math.sqrt(d)).to(device)


class WanNSABase:
    """Random-init Wan2.1-1.3B-shaped DiT weights (seeded) and the pieces every driver shares:
    patch / text / time embeddings, rotary embedding, the block (adaLN modulation,
    self-attention, cross-attention, FFN; causal_wan_nsa_model.py:626-700) and a per-category
    event-timer breakdown (``timers``).  Subclasses supply the self-attention branch."""

    def __init__(self, cfg: WanARConfig, device="cuda", seed: int = 0, dtype=torch.bfloat16):
        self.cfg = cfg
        self.device, self.dtype = torch.device(device), dtype
        gen = torch.Generator().manual_seed(seed)
        self.blocks = [_Block(cfg, gen, self.device, dtype) for _ in range(cfg.layers)]
        d = cfg.dim

        def lin(o, i):
            return ((torch.randn((o, i), generator=gen) / math.sqrt(i)).to(self.device, dtype),
                    torch.zeros(o, device=self.device, dtype=dtype))

        self.patch_in = lin(d, cfg.in_dim * cfg.patch)
        self.text1, self.text2 = lin(d, cfg.text_dim), lin(d, d)
        self.time1, self.time2 = lin(d, cfg.freq_dim), lin(d, d)
        self.time_proj = lin(6 * d, d)
        self.head = lin(cfg.in_dim * cfg.patch, d)
        self.head_mod = (torch.randn((1, 2, d), generator=gen) / math.sqrt(d)).to(self.device)
        ctx = torch.randn((1, cfg.text_len, cfg.text_dim), generator=gen).to(self.device, dtype)
        self.context = F.linear(F.gelu(F.linear(ctx, *self.text1), approximate="tanh"), *self.text2)
        # cross-attention K/V of the (fixed) prompt, once per block
        H, hd = cfg.heads, cfg.head_dim
        self.ctx_kv = []
        for blk in self.blocks:
            ck = _rms(F.linear(self.context, *blk.ck), blk.cnorm_k, cfg.eps)
            cv = F.linear(self.context, *blk.cv)
            self.ctx_kv.append((ck.view(1, -1, H, hd).transpose(1, 2).contiguous(),
                                cv.view(1, -1, H, hd).transpose(1, 2).contiguous()))
        half = hd // 2
        self.inv_freq = 1.0 / (10000 ** (torch.arange(half, device=self.device, dtype=torch.float64) / half))
        self.timers: Optional[Dict[str, List]] = None
        # set to a dict to record one layer's attention inputs and branch outputs (tests)
        self.trace: Optional[Dict[str, torch.Tensor]] = None
        self.trace_layer = 0
        self._rope_tab: Dict = {}

    # ------------------------------------------------------------------ pieces
    def _tic(self, name):
        if self.timers is None:
            return None
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return (name, e)

    def _toc(self, tok):
        if tok is None:
            return
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.timers.setdefault(tok[0], []).append((tok[1], e))

    def _rope(self, x: torch.Tensor, start: int) -> torch.Tensor:
        """x [1, S, H, D]: rotate interleaved pairs by angle pos * inv_freq (complex multiply in
        fp32; the angle table of a chunk is built once, in fp64)."""
        S = x.shape[1]
        key = (start, S)
        rot = self._rope_tab.get(key)
        if rot is None:
            pos = torch.arange(start, start + S, device=x.device, dtype=torch.float64)
            ang = torch.outer(pos, self.inv_freq)
            rot = torch.polar(torch.ones_like(ang), ang).to(torch.complex64)[None, :, None, :]
            self._rope_tab = {key: rot}  # one chunk at a time
        xc = torch.view_as_complex(x.float().unflatten(-1, (-1, 2)).contiguous())
        return torch.view_as_real(xc * rot).flatten(-2).to(x.dtype)

    def _time_embed(self, t: float) -> torch.Tensor:
        cfg = self.cfg
        half = cfg.freq_dim // 2
        pos = torch.tensor([t], device=self.device, dtype=torch.float64)
        sinus = torch.outer(pos, torch.pow(10000, -torch.arange(half, device=self.device).double() / half))
        emb = torch.cat([sinus.cos(), sinus.sin()], 1).to(self.dtype)
        e = F.linear(F.silu(F.linear(emb, *self.time1)), *self.time2)
        e0 = F.linear(F.silu(e), *self.time_proj).float().view(1, 6, cfg.dim)
        return e, e0

    def _qkvg(self, blk: _Block, x: torch.Tensor):
        """q, k, v [1, S, H, hd] (RMSNorm on q and k) and the sigmoid gates [1, S, H, 3]
        (causal_wan_nsa_model.py:369-386)."""
        cfg = self.cfg
        S, H, hd = x.shape[1], cfg.heads, cfg.head_dim
        q = _rms(F.linear(x, *blk.q), blk.norm_q, cfg.eps).view(1, S, H, hd)
        k = _rms(F.linear(x, *blk.k), blk.norm_k, cfg.eps).view(1, S, H, hd)
        v = F.linear(x, *blk.v).view(1, S, H, hd)
        g = torch.clamp(F.linear(x, *blk.g), -10.0, 10.0).view(1, S, H, 3).sigmoid()
        return q, k, v, g

    def _embed(self, latents: torch.Tensor, t: float):
        x = F.linear(latents, *self.patch_in)
        e, e0 = self._time_embed(t)
        return x, e, e0

    def _head_out(self, x: torch.Tensor, e: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        m = (self.head_mod + e.float().unsqueeze(1)).unbind(1)
        return F.linear((_ln(x, cfg.eps).float() * (1 + m[1]) + m[0]).to(x.dtype), *self.head)

    def _block(self, layer: int, x: torch.Tensor, e0: torch.Tensor, ctx) -> torch.Tensor:
        cfg, blk = self.cfg, self.blocks[layer]
        e = (blk.modulation + e0).unbind(1)
        tk = self._tic("norm")
        h = (_ln(x, cfg.eps).float() * (1 + e[1]) + e[0]).to(x.dtype)
        self._toc(tk)
        x = x + (self._self_attn(blk, layer, h, ctx).float() * e[2]).to(x.dtype)
        tk = self._tic("cross_ffn")
        S, H, hd = x.shape[1], cfg.heads, cfg.head_dim
        hq = _ln(x, cfg.eps, blk.norm3_w, blk.norm3_b)
        cq = _rms(F.linear(hq, *blk.cq), blk.cnorm_q, cfg.eps).view(1, S, H, hd).transpose(1, 2)
        ck, cv = self.ctx_kv[layer]
        co = F.scaled_dot_product_attention(cq, ck, cv).transpose(1, 2).flatten(2)
        x = x + F.linear(co, *blk.co)
        h = (_ln(x, cfg.eps).float() * (1 + e[4]) + e[3]).to(x.dtype)
        y = F.linear(F.gelu(F.linear(h, *blk.f1), approximate="tanh"), *blk.f2)
        x = x + (y.float() * e[5]).to(x.dtype)
        self._toc(tk)
        return x


class WanNSAAR(WanNSABase):
    """AR generation over a ``PagedKVCache`` (bf16 or fp8 pages).

    ``step(cid)`` runs one AR chunk (denoise forwards + context forward + flush); ``prefill``
    fills chunks 0..n-1 of every layer with seeded random keys / values without running the
    model, so a long-history cache is reached in seconds.  ``timers`` (category -> list of event
    pairs) collects a per-category time breakdown when set."""

    def __init__(self, cfg: WanARConfig, cache: PagedKVCache, device="cuda", seed: int = 0,
                 dtype=torch.bfloat16):
        super().__init__(cfg, device, seed, dtype)
        self.cache = cache
        assert cache.L == cfg.layers and cache.H == cfg.heads and cache.D == cfg.head_dim
        assert cache.chunk_len == cfg.chunk_tokens and cache.P == cfg.page_tokens
        # stage each selection's host-resident pages into HBM on a side stream (prefetch)
        self.prefetch = True

    def _self_attn(self, blk: _Block, layer: int, x: torch.Tensor, cid: int) -> torch.Tensor:
        cfg, cache = self.cfg, self.cache
        tk = self._tic("linear")
        q, k, v, g = self._qkvg(blk, x)
        self._toc(tk)
        tk = self._tic("rope")
        start = cid * cfg.chunk_tokens
        q = self._rope(q, start)
        k = self._rope(k, start)
        self._toc(tk)
        tk = self._tic("cache_append")
        cache.append(layer, k, v, cid)                 # paged K/V + pooled K/V of the chunk
        self._toc(tk)
        # top-k first, so that the host-resident pages it selects are staged into HBM on a side
        # stream while the compressed and window branches run
        tk = self._tic("topk")
        k_cmp, v_cmp = cache.cmp_history(layer)
        ids = parallel_nsa_topk(q, k_cmp, cfg.topk, block_size=cfg.page_tokens,
                                chunk_size=cfg.chunk_tokens, causal=False,
                                group_size=cfg.group_size,
                                exclude_window_chunks=cfg.exclude_window_chunks,
                                exclude_sink_chunks=cfg.exclude_sink_chunks,
                                progressive_exclude=cfg.progressive_exclude,
                                q_chunk_offset=cid, blocks_per_chunk=cache.ppc)
        staged = cache.prefetch(ids, layer) if self.prefetch else None
        self._toc(tk)
        tk = self._tic("attn_cmp")
        o_cmp = dense_attention(q, k_cmp, v_cmp)       # over the pooled history
        self._toc(tk)
        tk = self._tic("attn_swa")
        o_swa = cache.window_attention(q, layer)        # over the window chunks
        self._toc(tk)
        tk = self._tic("sel_attn")
        # selection with the branch mix g_cmp*o_cmp + g_slc*o_slc + g_swa*o_swa in its epilogue
        o = cache.select(q, ids, layer, cfg.group_size, gates=g, o_cmp=o_cmp, o_swa=o_swa,
                         prefetch=staged)
        self._toc(tk)
        if self.trace is not None and layer == self.trace_layer:
            self.trace.update(q=q.clone(), g=g.clone(), ids=ids.clone(), o_cmp=o_cmp.clone(),
                              o_swa=o_swa.clone(), o=o.clone())
        tk = self._tic("linear")
        out = F.linear(o.flatten(2), *blk.o)
        self._toc(tk)
        return out

    @torch.no_grad()
    def forward(self, latents: torch.Tensor, t: float, cid: int) -> torch.Tensor:
        """latents: [1, chunk_tokens, in_dim * patch] patchified latents of chunk ``cid``."""
        cfg = self.cfg
        x, e, e0 = self._embed(latents, t)
        # fused attention kernels only: an unsupported shape raises instead of taking the
        # batched-matmul math path
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            for layer in range(cfg.layers):
                x = self._block(layer, x, e0, cid)
        return self._head_out(x, e)

    @torch.no_grad()
    def step(self, cid: int, noise: torch.Tensor) -> dict:
        """One AR chunk: denoise forwards at t = 1000 .. 250, a context forward at t = 0 on the
        result (both rewrite chunk ``cid`` of every layer), then the cache flush."""
        cfg = self.cfg
        x = noise
        ts = [1000.0 * (1 - i / cfg.denoise_steps) for i in range(cfg.denoise_steps)]
        for i, t in enumerate(ts):
            pred = self.forward(x, t, cid)
            dt = (ts[i + 1] if i + 1 < len(ts) else 0.0) - t
            x = x + pred * (dt / 1000.0)
        self.forward(x, 0.0, cid)
        tk = self._tic("flush")
        st = self.cache.flush()
        self._toc(tk)
        return st

    @torch.no_grad()
    def prefill(self, n_chunks: int, seed: int = 1, student_t: bool = False):
        """Chunks 0..n_chunks-1 of every layer from seeded random K/V (N(0,1), or Student-t with
        4 degrees of freedom), flushing after each chunk like the AR loop and waiting for each
        flush's copies before the next chunk's appends."""
        cfg, cache = self.cfg, self.cache
        g = torch.Generator(device=self.device).manual_seed(seed)
        shape = (1, cfg.chunk_tokens, cfg.heads, cfg.head_dim)
        for cid in range(n_chunks):
            for layer in range(cfg.layers):
                if student_t:
                    # t(4) = N(0,1) / sqrt(chi2(4) / 4), chi2(4) = -2 ln(u1 u2)
                    z = torch.randn((2,) + shape, generator=g, device=self.device)
                    u = torch.rand((2, 2) + shape, generator=g, device=self.device).clamp_min_(1e-12)
                    chi = -2.0 * torch.log(u[:, 0] * u[:, 1])
                    kv = (z / torch.sqrt(chi / 4.0)).to(self.dtype)
                else:
                    kv = torch.randn((2,) + shape, generator=g, device=self.device).to(self.dtype)
                cache.append(layer, kv[0], kv[1], cid)
            cache.flush()
            # a flush's copies run beside the next chunk's work; here that is only the next
            # chunk's appends, so let them land first
            torch.cuda.synchronize(self.device)
