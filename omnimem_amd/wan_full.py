"""Full-sequence causal NSA forward of the Wan2.1-1.3B shape.

The caller counterpart of the dense selection path: the random-init Wan block of ``wan_ar``
(``WanNSABase``: 30 blocks, dim 1536, 12 heads x 128, RMSNorm on q and k, cross-attention, FFN)
with the full-sequence branch of the reference's NSA self-attention
(src/omnimem/models/transformers/causal_wan_nsa_model.py:391-458), run over one whole clip of
``frames`` latent frames (21 for an 81-frame 480x832 clip: 32760 tokens):

* rotary embedding of q and k (positions 0..S-1; the reference's 3-axis split and token
  reorder only permute which angles a token gets);
* K and V block compression (64-token mean pooling, ``block_pool``; the last block pools its 56
  valid tokens);
* compressed attention o_cmp over the pooled rows, block-causal by chunk: a query of chunk c sees
  pooled row j when (64 j) // chunk <= c (the flex mask of ``create_cmp_block``,
  src/omnimem/models/flex_attention_utils.py:45-47 with kv_stride 64), one dense call per chunk
  over its visible prefix;
* sliding-window attention o_swa over the chunks c - window + 1 .. c (block-causal by chunk, the
  window block mask), one dense call per chunk;
* top-k selection with the causal chunk mask (``parallel_nsa_topk``, groups of 64 queries) and
  selection attention causal by chunk -- the config-3 hot path -- with the sigmoid-gated mix
  g_cmp o_cmp + g_slc o_slc + g_swa o_swa in its epilogue (``sel_fwd_gated``);
* the output projection.

``forward(latents, t)`` returns the head output; ``timers`` (as in ``WanNSAAR``) break the time
down by category, and ``sel_events`` collects one event pair per selection call (the gated one:
the mix is part of its epilogue) so that the selection kernel's own time can be summed over the
30 layers.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .index_topk import block_pool, parallel_nsa_topk
from .selection import dense_attention, sel_fwd, sel_fwd_gated
from .wan_ar import WanARConfig, WanNSABase, _Block

__all__ = ["WanNSAFull"]


class WanNSAFull(WanNSABase):
    """Full-sequence NSA forward over ``frames`` latent frames (module docstring)."""

    def __init__(self, cfg: WanARConfig, frames: int = 21, device="cuda", seed: int = 0,
                 dtype=torch.bfloat16):
        super().__init__(cfg, device, seed, dtype)
        self.frames = int(frames)
        self.tokens = self.frames * cfg.frame_tokens
        # (start event, end event) of every selection-attention call of the last forward
        # and the block ids of those calls (for their useful-FLOP count)
        self.sel_events: Optional[List[Tuple[torch.cuda.Event, torch.cuda.Event]]] = None
        self.sel_ids: List[torch.Tensor] = []

    def _chunk_ranges(self, S: int):
        C = self.cfg.chunk_tokens
        return [(c, c * C, min((c + 1) * C, S)) for c in range(-(-S // C))]

    def _self_attn(self, blk: _Block, layer: int, x: torch.Tensor, _ctx) -> torch.Tensor:
        cfg = self.cfg
        S = x.shape[1]
        C, BS, G = cfg.chunk_tokens, cfg.page_tokens, cfg.group_size
        scale = cfg.head_dim ** -0.5
        tk = self._tic("linear")
        q, k, v, g = self._qkvg(blk, x)
        self._toc(tk)
        tk = self._tic("rope")
        q = self._rope(q, 0)
        k = self._rope(k, 0)
        self._toc(tk)
        tk = self._tic("pool")
        k_cmp = block_pool(k, BS)
        v_cmp = block_pool(v, BS)
        self._toc(tk)
        tk = self._tic("topk")
        ids = parallel_nsa_topk(q, k_cmp, cfg.topk, block_size=BS, chunk_size=C, causal=True,
                                group_size=G)
        self._toc(tk)
        tk = self._tic("attn_cmp")
        o_cmp = torch.empty_like(q)
        n_cmp = k_cmp.shape[1]
        for c, a, b in self._chunk_ranges(S):
            vis = min(n_cmp, ((c + 1) * C - 1) // BS + 1)  # pooled rows j with 64 j // C <= c
            dense_attention(q[:, a:b], k_cmp[:, :vis], v_cmp[:, :vis], scale=scale,
                            out=o_cmp[:, a:b])
        self._toc(tk)
        tk = self._tic("attn_swa")
        o_swa = torch.empty_like(q)
        W = max(1, cfg.window_chunks)
        for c, a, b in self._chunk_ranges(S):
            lo = max(0, c - W + 1) * C
            dense_attention(q[:, a:b], k[:, lo:b], v[:, lo:b], scale=scale, out=o_swa[:, a:b])
        self._toc(tk)
        tk = self._tic("sel_attn")
        ev = None
        if self.sel_events is not None:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        # selection with the branch mix in its epilogue
        o = sel_fwd_gated(q, k, v, ids, BS, C, scale, True, G, g, o_cmp, o_swa)
        if ev is not None:
            ev[1].record()
            self.sel_events.append(ev)
            self.sel_ids.append(ids)
        self._toc(tk)
        if self.trace is not None and layer == self.trace_layer:
            o_slc, _ = sel_fwd(q, k, v, ids, BS, C, scale, True, G)  # the branch alone
            self.trace.update(q=q.clone(), k=k.clone(), v=v.clone(), g=g.clone(),
                              ids=ids.clone(), o_cmp=o_cmp.clone(), o_swa=o_swa.clone(),
                              o_slc=o_slc, o=o.clone())
        tk = self._tic("linear")
        out = F.linear(o.flatten(2), *blk.o)
        self._toc(tk)
        return out

    @torch.no_grad()
    def forward(self, latents: torch.Tensor, t: float) -> torch.Tensor:
        """latents: [1, tokens, in_dim * patch] patchified latents of the whole clip."""
        cfg = self.cfg
        if latents.shape[1] != self.tokens:
            raise ValueError(f"expected {self.tokens} tokens, got {latents.shape[1]}")
        x, e, e0 = self._embed(latents, t)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            for layer in range(cfg.layers):
                x = self._block(layer, x, e0, None)
        return self._head_out(x, e)
