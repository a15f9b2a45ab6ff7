"""Configs 4 and 5 at their stated state, checked against the float64 oracle.

The cache is the one ``bench.py`` times: Wan2.1-1.3B shapes (30 layers, 12 heads x 128), 4680-token
chunks of 64-token pages, 80 chunks prefilled (374,400 tokens per layer) under a 48 GB HBM
budget, so that about a third of the bf16 units live in the host pool (config 4); config 5 is the
fp8-e4m3 cache over Student-t(4) keys and values, with bf16 and with fp8 (quantised query rows)
Q K^T.  One AR step runs (4 denoise forwards, the context forward and the flush), then one more
forward of the next chunk records a middle layer's attention inputs and outputs.

For three query groups (the first, a middle one and the ragged last) and all 12 heads, the
branches of causal_wan_nsa_model.py:496-546 are recomputed in float64 from the cache's own
contents (``read_unit`` of the selected units only, fp8 pages as code * page scale): the
compressed attention over every pooled row, the window attention over the last three chunks,
the selection attention over the 16 selected pages, and the gated mix of the three.  The bf16
case must select host-resident units among those checked.

Tolerances: 2e-2 max-abs and 1e-3 mean-abs (the bf16 bar).  Student-t(4) values make outputs of
magnitude up to about 10, whose own rounding to bf16 is up to 2^-8 of their size (about 2^-9.5
on average), so the fp8 cases add 2^-8 * max|want| to the max-abs bound and 2^-8 * mean|want| to
the mean-abs bound of each branch (2^-7 for the mix, which an fp8 cache computes from the
rounded o_slc).
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O

pytestmark = pytest.mark.gpu

HISTORY, LAYER, GROUPS = 80, 17, (0, 36, 73)


def _f64(t):
    return t.double().cpu().numpy()


def _attn(q, k, v, scale):
    """float64 softmax attention of q [m, D] over k / v [n, D]."""
    s = q @ k.T * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p / p.sum(-1, keepdims=True)) @ v


def _close(name, got, want, mx=2e-2, mean=1e-3, rel=0.0):
    err = np.abs(got - want)
    bound = mx + rel * np.abs(want).max()
    assert err.max() <= bound, f"{name}: max-abs {err.max():.3e} > {bound:.3e}"
    mbound = mean + rel * np.abs(want).mean()
    assert err.mean() <= mbound, f"{name}: mean-abs {err.mean():.3e} > {mbound:.3e}"


class _Units:
    """K / V of one (layer, head, chunk) unit as float64 [chunk_len, D], read once each: bf16
    pages as stored, fp8 pages as code * page scale (what the kernels compute with)."""

    def __init__(self, cache, layer):
        self.cache, self.layer, self.memo = cache, layer, {}

    def __call__(self, h, c):
        key = (h, c)
        if key not in self.memo:
            cache = self.cache
            C, D = cache.chunk_len, cache.D
            parts = cache.read_unit(self.layer, h, c)
            if cache.fp8:
                kc, vc, sk, sv = parts
                k = O.dequantize_pages(kc.numpy(), sk.numpy()[:, None, None])
                v = O.dequantize_pages(vc.numpy(), sv.numpy()[:, None, None])
            else:
                k, v = parts[0].float().numpy(), parts[1].float().numpy()
            self.memo[key] = (k.reshape(-1, D)[:C].astype(np.float64),
                              v.reshape(-1, D)[:C].astype(np.float64))
        return self.memo[key]


def _quantized_row(x: np.ndarray) -> np.ndarray:
    """e4m3 image of one query row with the page rule (scale amax / 448, nearest even)."""
    c, sc = O.quantize_pages(x.astype(np.float32)[None, :], 1)
    return O.dequantize_pages(c, sc)[0].astype(np.float64)


@pytest.mark.parametrize("variant", ["bf16", "fp8", "fp8_qk8"])
def test_ar_stated_state_branches_match_oracle(variant):
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.wan_ar import WanARConfig, WanNSAAR
    cfg = WanARConfig()
    fp8 = variant != "bf16"
    cache = PagedKVCache(cfg.layers, cfg.heads, cfg.head_dim, max_chunks=HISTORY + 3,
                         chunk_len=cfg.chunk_tokens, page_tokens=cfg.page_tokens,
                         dtype="fp8" if fp8 else torch.bfloat16, hbm_budget_bytes=int(48e9),
                         window_chunks=cfg.window_chunks, keep_window_kv=fp8,
                         qk_fp8=variant == "fp8_qk8")
    model = WanNSAAR(cfg, cache, seed=4)
    model.prefill(HISTORY, seed=5, student_t=fp8)
    gen = torch.Generator(device="cuda").manual_seed(6)
    noise = lambda: torch.randn((1, cfg.chunk_tokens, cfg.in_dim * cfg.patch), generator=gen,
                                device="cuda").to(torch.bfloat16)
    model.step(HISTORY, noise())
    cid = HISTORY + 1
    model.trace, model.trace_layer = {}, LAYER
    model.forward(noise(), 500.0, cid)
    tr = model.trace
    # o_slc alone: the same selection without the mix (no residency change before a flush)
    o_slc_gpu = cache.select(tr["q"], tr["ids"], LAYER, cfg.group_size)
    torch.cuda.synchronize()
    print(f"{variant}: cache of {cache.n_slots} HBM / {cache.n_host} host unit slots, "
          f"{int((cache._table_h <= -2).sum())} units on the host", flush=True)

    C, P, G, D, H = cfg.chunk_tokens, cfg.page_tokens, cfg.group_size, cfg.head_dim, cfg.heads
    scale = D ** -0.5
    ppc = cache.ppc
    units = _Units(cache, LAYER)
    q, ids = _f64(tr["q"][0]), tr["ids"][0].cpu().numpy()
    gates = _f64(tr["g"][0])
    got_slc, got_mix = _f64(o_slc_gpu[0]), _f64(tr["o"][0])
    got_cmp, got_swa = _f64(tr["o_cmp"][0]), _f64(tr["o_swa"][0])
    kc, vc = (_f64(t[0]) for t in cache.cmp_history(LAYER))
    win = list(range(cid + 1 - cfg.window_chunks, cid + 1))
    if fp8:
        wk, wv = (_f64(t[0]) for t in cache.window_kv(LAYER))  # ring slots, any chunk order
    where = {"hbm": 0, "host": 0}
    rel = 2.0 ** -8 if fp8 else 0.0
    for g in GROUPS:
        m0, m1 = g * G, min((g + 1) * G, C)
        for h in range(H):
            qr = q[m0:m1, h]
            # compressed branch: every pooled row of chunks 0..cid
            o_cmp = _attn(qr, kc[:, h], vc[:, h], scale)
            _close(f"o_cmp g{g} h{h}", got_cmp[m0:m1, h], o_cmp, rel=rel)
            # window branch: the last three chunks' tokens (pages of a bf16 cache, the dense
            # ring of an fp8 cache)
            if fp8:
                o_swa = _attn(qr, wk[:, h], wv[:, h], scale)
            else:
                ks, vs = zip(*(units(h, c) for c in win))
                o_swa = _attn(qr, np.concatenate(ks), np.concatenate(vs), scale)
            _close(f"o_swa g{g} h{h}", got_swa[m0:m1, h], o_swa, rel=rel)
            # selection branch over the listed pages
            kk, vv = [], []
            for bid in ids[g, h]:
                if bid < 0:
                    continue
                c, p = divmod(int(bid), ppc)
                assert c <= cid - cfg.exclude_window_chunks, (g, h, bid)
                where[cache.where(LAYER, h, c)] += 1
                n = min(P, C - p * P)
                uk, uv = units(h, c)
                kk.append(uk[p * P:p * P + n])
                vv.append(uv[p * P:p * P + n])
            assert len(kk) == cfg.topk
            qs = np.stack([_quantized_row(r) for r in qr]) if variant == "fp8_qk8" else qr
            o_slc = _attn(qs, np.concatenate(kk), np.concatenate(vv), scale)
            _close(f"o_slc g{g} h{h}", got_slc[m0:m1, h], o_slc, rel=rel)
            gt = gates[m0:m1, h]
            mix = gt[:, 0:1] * o_cmp + gt[:, 1:2] * o_slc + gt[:, 2:3] * o_swa
            # an fp8 cache rounds o_slc to bf16 before its mix pass
            _close(f"mix g{g} h{h}", got_mix[m0:m1, h], mix, rel=2 * rel)
    print(f"{variant}: selected units checked: {where}", flush=True)
    if not fp8:
        assert where["host"] > 0, "no checked selection read a host-resident unit"
    del model
    cache.close()
