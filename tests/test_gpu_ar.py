"""End-to-end AR driver checks on a small Wan-shaped model.

The selection path must give the same model output whatever the cache residency: two drivers
with identical seeds, one with every unit in HBM and one whose HBM pool forces evictions to the
host pool (read there directly by the paged kernel), must produce bit-identical latents.  The
second cache must actually have moved units, and its LRU bookkeeping must balance.

One AR forward's layer is also checked branch by branch against the float64 oracle
(oracle/nsa_oracle.py): the compressed attention over every pooled row, the window attention,
the top-k over the pooled history (the MFMA parity check of tests/_topk_checks.py), the
selection attention over the selected pages and the gated mix of the three
(causal_wan_nsa_model.py:496-546).
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O

pytestmark = pytest.mark.gpu


def _cfg():
    from omnimem_amd.wan_ar import WanARConfig
    return WanARConfig(layers=2, dim=256, ffn_dim=512, heads=2, text_len=16, text_dim=64,
                       freq_dim=32, frame_tokens=520, frames_per_chunk=3, page_tokens=64,
                       group_size=64, topk=8, exclude_window_chunks=1, window_chunks=1,
                       denoise_steps=2)


def _run(hbm_slots, dtype=torch.bfloat16, history=5, steps=2):
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.wan_ar import WanNSAAR
    cfg = _cfg()
    n = history + steps + 1
    cache = PagedKVCache(cfg.layers, cfg.heads, cfg.head_dim, max_chunks=n,
                         chunk_len=cfg.chunk_tokens, page_tokens=cfg.page_tokens, dtype=dtype,
                         hbm_slots=hbm_slots, window_chunks=cfg.window_chunks,
                         keep_window_kv=(dtype == "fp8"))
    model = WanNSAAR(cfg, cache, seed=3)
    model.prefill(history, seed=4, student_t=(dtype == "fp8"))
    g = torch.Generator(device="cuda").manual_seed(5)
    outs = []
    for cid in range(history, history + steps):
        x = torch.randn((1, cfg.chunk_tokens, cfg.in_dim * cfg.patch), generator=g,
                        device="cuda").to(torch.bfloat16)
        model.step(cid, x)
        outs.append(model.forward(x, 500.0, cid))
    torch.cuda.synchronize()
    return outs, cache


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
def test_ar_output_independent_of_residency(dtype):
    cfg = _cfg()
    full = cfg.layers * cfg.heads * 8
    a, ca = _run(full, dtype)
    assert ca.stats["evicted_units"] == 0
    # room for 3 chunks per (layer, head): synchronous flushes; for 5: asynchronous ones
    for per_head, asyn in ((3, False), (5, True)):
        b, cb = _run(cfg.layers * cfg.heads * per_head, dtype)
        assert cb._async_ok() == asyn
        assert cb.stats["evicted_units"] > 0
        assert cb.stats["misses"] > 0
        for x, y in zip(a, b):
            assert torch.isfinite(x.float()).all()
            assert torch.equal(x, y), per_head
        # every written unit is in exactly one pool
        for l in range(cfg.layers):
            for h in range(cfg.heads):
                for c in range(cb.n_chunks[l]):
                    assert cb.where(l, h, c) in ("hbm", "host")
        cb.close()
    ca.close()


def _close(name, got, want, mx=2e-2, mean=1e-3, rel=0.0):
    """max-abs <= mx + rel * max|want| (rel covers bf16 roundings of large values), and mean-abs
    <= mean."""
    g = got.double().cpu().numpy() if isinstance(got, torch.Tensor) else got
    err = np.abs(g - want)
    bound = mx + rel * np.abs(want).max()
    assert err.max() <= bound, f"{name}: max-abs {err.max():.3e} > {bound:.3e}"
    assert err.mean() <= mean, f"{name}: mean-abs {err.mean():.3e}"


def _cache_kv(cache, layer, n):
    """K and V of chunks 0..n-1 as float64 [tokens, H, D], the values the selection kernel
    computes with: bf16 pages as stored, fp8 pages as code * page scale."""
    if not cache.fp8:
        k = torch.cat([cache._gather_chunk(layer, "k", c) for c in range(n)], 0)
        v = torch.cat([cache._gather_chunk(layer, "v", c) for c in range(n)], 0)
        return k.double().cpu().numpy(), v.double().cpu().numpy()
    C, H, D = cache.chunk_len, cache.H, cache.D
    out = [np.zeros((n * C, H, D)), np.zeros((n * C, H, D))]
    for c in range(n):
        for h in range(H):
            kc, vc, sk, sv = cache.read_unit(layer, h, c)
            for i, (codes, sc) in enumerate(((kc, sk), (vc, sv))):
                deq = O.dequantize_pages(codes.numpy(), sc.numpy()[:, None, None])
                out[i][c * C:(c + 1) * C, h] = deq.reshape(-1, D)[:C]
    return out[0], out[1]


def _dense_attn(q, k, v, scale):
    """float64 softmax attention per head: q [M, H, D], k / v [N, H, D]."""
    s = np.einsum("mhd,nhd->hmn", q, k) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    return np.einsum("hmn,nhd->mhd", p / p.sum(-1, keepdims=True), v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
def test_ar_layer_branches_match_oracle(dtype):
    from tests._topk_checks import check_mfma_topk
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.wan_ar import WanNSAAR
    cfg = _cfg()
    history = 4
    cid = history
    cache = PagedKVCache(cfg.layers, cfg.heads, cfg.head_dim, max_chunks=cid + 2,
                         chunk_len=cfg.chunk_tokens, page_tokens=cfg.page_tokens, dtype=dtype,
                         hbm_slots=cfg.layers * cfg.heads * (cid + 2),
                         window_chunks=cfg.window_chunks, keep_window_kv=(dtype == "fp8"))
    model = WanNSAAR(cfg, cache, seed=3)
    model.prefill(history, seed=4, student_t=(dtype == "fp8"))
    g = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn((1, cfg.chunk_tokens, cfg.in_dim * cfg.patch), generator=g,
                    device="cuda").to(torch.bfloat16)
    model.trace, model.trace_layer = {}, 1
    model.forward(x, 500.0, cid)
    torch.cuda.synchronize()
    tr = model.trace
    layer, C, P, G, D = 1, cfg.chunk_tokens, cfg.page_tokens, cfg.group_size, cfg.head_dim
    scale = D ** -0.5
    q = tr["q"][0].double().cpu().numpy()
    # the cache's own K / V (fp8 pages dequantised) and pooled history, as the kernels read them
    kd, vd = _cache_kv(cache, layer, cid + 1)
    kc, vc = cache.cmp_history(layer)
    # compressed attention over every pooled row of the history
    o_cmp = _dense_attn(q, kc[0].double().cpu().numpy(), vc[0].double().cpu().numpy(), scale)
    _close("o_cmp", tr["o_cmp"][0], o_cmp)
    # window attention over the last window_chunks chunks (here the current one): the pages of a
    # bf16 cache, the dense bf16 ring an fp8 cache keeps beside its pages
    if dtype == "fp8":
        wk, wv = cache.window_kv(layer)
        wk, wv = wk[0].double().cpu().numpy(), wv[0].double().cpu().numpy()
    else:
        w0 = (cid + 1 - cfg.window_chunks) * C
        wk, wv = kd[w0:], vd[w0:]
    o_swa = _dense_attn(q, wk, wv, scale)
    _close("o_swa", tr["o_swa"][0], o_swa)
    # top-k: the driver's call, checked on the kernel's own scores plus the fp32 score bound
    kw = dict(block_size=P, chunk_size=C, causal=False,
              exclude_window_chunks=cfg.exclude_window_chunks, exclude_sink_chunks=0,
              progressive_exclude=cfg.progressive_exclude, q_chunk_offset=cid,
              blocks_per_chunk=cache.ppc)
    mask = O.Mask(block_size=P, group_size=G, chunk_q=C, chunk_k=C, blocks_per_chunk=cache.ppc,
                  q_chunk_offset=cid, ex_win=cfg.exclude_window_chunks, causal=0, prog_excl=1)
    check_mfma_topk(tr["q"], kc, cfg.topk, mask, scale, G, got=tr["ids"].cpu().numpy(), **kw)
    # selection attention over the selected pages, then the gated mix in float64
    ids = tr["ids"].cpu().numpy()
    o_slc, _ = O.selection_attention(q[None], kd[None], vd[None], ids, G, scale,
                                     O.paged_block_tokens(C, P, cid + 1))
    gt = tr["g"][0].double().cpu().numpy()
    mix = gt[..., 0:1] * o_cmp + gt[..., 1:2] * o_slc[0] + gt[..., 2:3] * o_swa
    # an fp8 cache rounds o_slc to bf16 before its mix pass: two roundings of the output scale
    _close("mix", tr["o"][0], mix, rel=2.0 ** -7 if dtype == "fp8" else 0.0)
    cache.close()
