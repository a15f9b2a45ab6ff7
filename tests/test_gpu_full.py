"""The full-sequence (config 3) driver on a small Wan-shaped model, branch by branch against the
float64 oracle (causal_wan_nsa_model.py:391-458): compressed attention block-causal by chunk
over the pooled keys, sliding-window attention over the last chunks, top-k under the causal chunk
mask (the MFMA parity check on the kernel's own scores), selection attention causal by chunk, and
the gated mix.  Two chunks of 1560 tokens plus a ragged third, so the partial last chunk, the
partial last pooled block and chunk-crossing pooled blocks are all exercised."""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O

pytestmark = pytest.mark.gpu


def _close(name, got, want, mx=2e-2, mean=1e-3):
    g = got.double().cpu().numpy() if isinstance(got, torch.Tensor) else got
    err = np.abs(g - want)
    assert err.max() <= mx, f"{name}: max-abs {err.max():.3e}"
    assert err.mean() <= mean, f"{name}: mean-abs {err.mean():.3e}"


def _masked_attn(q, k, v, scale, allowed):
    """float64 attention per head, q [M, H, D], k / v [N, H, D], allowed [M, N] bool."""
    s = np.einsum("mhd,nhd->hmn", q, k) * scale
    s = np.where(allowed[None], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    return np.einsum("hmn,nhd->mhd", p / p.sum(-1, keepdims=True), v)


def test_full_sequence_layer_branches_match_oracle():
    from tests._topk_checks import check_mfma_topk
    from omnimem_amd.wan_ar import WanARConfig
    from omnimem_amd.wan_full import WanNSAFull
    cfg = WanARConfig(layers=2, dim=256, ffn_dim=512, heads=2, text_len=16, text_dim=64,
                      freq_dim=32, frame_tokens=520, frames_per_chunk=3, page_tokens=64,
                      group_size=64, topk=8, window_chunks=2)
    frames = 7  # 3640 tokens: chunks of 1560, 1560 and 520
    model = WanNSAFull(cfg, frames=frames, seed=11)
    g = torch.Generator(device="cuda").manual_seed(12)
    x = torch.randn((1, model.tokens, cfg.in_dim * cfg.patch), generator=g,
                    device="cuda").to(torch.bfloat16)
    model.trace, model.trace_layer = {}, 1
    out = model.forward(x, 500.0)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    tr = model.trace
    S, C, BS, G, D = model.tokens, cfg.chunk_tokens, cfg.page_tokens, cfg.group_size, cfg.head_dim
    scale = D ** -0.5
    q, k, v = (tr[n][0].double().cpu().numpy() for n in ("q", "k", "v"))
    tq, tkc = np.arange(S), np.arange(S)
    # pooled keys / values, as block_pool computes them (checked bit-exact elsewhere)
    kc = O.pool_mean(tr["k"].float().cpu().numpy(), BS, "bf16")[0].astype(np.float64)
    vc = O.pool_mean(tr["v"].float().cpu().numpy(), BS, "bf16")[0].astype(np.float64)
    j = np.arange(kc.shape[0])
    o_cmp = _masked_attn(q, kc, vc, scale, (j[None, :] * BS) // C <= (tq[:, None] // C))
    _close("o_cmp", tr["o_cmp"][0], o_cmp)
    W = cfg.window_chunks
    qc, kcid = tq[:, None] // C, tkc[None, :] // C
    o_swa = _masked_attn(q, k, v, scale, (kcid <= qc) & (kcid > qc - W))
    _close("o_swa", tr["o_swa"][0], o_swa)
    mask = O.Mask(block_size=BS, group_size=G, chunk_q=C, chunk_k=C, causal=1)
    check_mfma_topk(tr["q"], torch.from_numpy(kc[None]).to(torch.bfloat16).cuda(), cfg.topk,
                    mask, scale, G, got=tr["ids"].cpu().numpy(), block_size=BS, chunk_size=C,
                    causal=True)
    ids = tr["ids"].cpu().numpy()
    o_slc, _ = O.selection_attention(q[None], k[None], v[None], ids, G, scale,
                                     O.dense_block_tokens(S, BS, C, True), chunk_size=C,
                                     causal=True)
    _close("o_slc", tr["o_slc"][0], o_slc[0])
    gt = tr["g"][0].double().cpu().numpy()
    mix = gt[..., 0:1] * o_cmp + gt[..., 1:2] * o_slc[0] + gt[..., 2:3] * o_swa
    _close("mix", tr["o"][0], mix)
