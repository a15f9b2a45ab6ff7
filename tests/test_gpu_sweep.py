"""Seeded random sweep over the selection path's argument space, each case against the oracle.

Every case draws its shape and options from its own seed, so a failure names a reproducible
configuration: the selection forward (dtypes, head dims 64 / 96 / 128, group sizes up to 192,
block sizes 16..100, ragged tails, chunk-causal masks, -1 / out-of-range / duplicate ids,
negative scales) against the float64 oracle at the BASELINE tolerances; its backward against the
oracle's exact gradient; the gated dense selection (branch mix in the epilogue); the paged cache's selection (bf16 / fp8 pages, host-resident units);
the top-k selection from given scores (ties, -0, -inf, NaN) for topk 1..600 against the oracle's
rule (path A to 128, path B past it); the fused pool + score + top-k call (MFMA and fmaf
paths, causal and AR window masks); the cache appends, bit-exact (pages, fp8 codes and
scales, pooled rows, the window ring); the window attention over pages or the ring; and random
sequences of appends, flushes, evictions, rewrites and snapshot / restore on a small cache, whose
selections (with or without staging its host pages first) must equal an all-HBM cache's bit for bit.
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
FWD_TOL = {torch.bfloat16: (2e-2, 1e-3), torch.float16: (2e-2, 1e-3), torch.float32: (1e-4, 1e-5)}
BWD_TOL = {torch.bfloat16: (2e-2, 5e-3), torch.float16: (2e-2, 5e-3), torch.float32: (1e-4, 1e-5)}
DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _case(seed, max_m, max_n, max_t):
    r = np.random.default_rng(seed)
    dtype = DTYPES[r.integers(0, 3)]
    D = int(r.choice([64, 128, 128, 64, 96]))
    H = int(r.integers(1, 4))
    G = int(r.choice([16, 30, 64, 64, 100, 128, 192]))
    BS = int(r.choice([16, 32, 64, 64, 100]))
    M = int(r.integers(1, max_m + 1))
    N = int(r.integers(BS // 2 + 1, max_n + 1))
    nb = -(-N // BS)
    T = int(r.integers(1, min(max_t, nb + 2) + 1))
    causal = bool(r.integers(0, 2))
    chunk = int(r.integers(BS, max(BS + 1, N))) if causal else 1
    minus = float(r.choice([0.0, 0.1, 0.3]))
    dup = bool(r.integers(0, 2))
    sgn = float(r.choice([1.0, 1.0, -1.0]))
    B = int(r.choice([1, 1, 2]))
    return dict(dtype=dtype, B=B, D=D, H=H, G=G, BS=BS, M=M, N=N, nb=nb, T=T, causal=causal,
                chunk=chunk, minus=minus, dup=dup, scale=sgn * D ** -0.5)


def _inputs(c, seed):
    gen = torch.Generator().manual_seed(seed)
    B, M, N, H, D, dt = c["B"], c["M"], c["N"], c["H"], c["D"], c["dtype"]
    q = (torch.randn((B, M, H, D), generator=gen) * D ** -0.25).to(dt)
    k = (torch.randn((B, N, H, D), generator=gen) * D ** -0.25).to(dt)
    v = torch.randn((B, N, H, D), generator=gen).to(dt)
    MG = -(-M // c["G"])
    ids = torch.randint(-1, c["nb"], (B, MG, H, c["T"]), generator=gen, dtype=torch.int32)
    ids[torch.rand(ids.shape, generator=gen) < c["minus"]] = -1
    if c["dup"] and c["T"] > 1:
        ids[..., 1] = ids[..., 0]
    return q, k, v, ids


def _desc(c):
    return ", ".join(f"{k}={v}" for k, v in c.items())


@pytest.mark.parametrize("seed", range(48))
def test_sel_fwd_sweep(seed):
    from omnimem_amd.selection import sel_fwd
    c = _case(7000 + seed, 400, 1500, 12)
    q, k, v, ids = _inputs(c, seed)
    out, lse = sel_fwd(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), c["BS"], c["chunk"],
                       c["scale"], c["causal"], c["G"])
    want_o, want_l = O.selection_attention(
        q.float().numpy(), k.float().numpy(), v.float().numpy(), ids.numpy(), c["G"], c["scale"],
        O.dense_block_tokens(c["N"], c["BS"], c["chunk"], c["causal"]), chunk_size=c["chunk"],
        causal=c["causal"])
    o = out.float().cpu().numpy().astype(np.float64)
    l = lse.cpu().numpy().astype(np.float64)
    mx, mean = FWD_TOL[c["dtype"]]
    err = np.abs(o - want_o)
    assert err.max() <= mx and err.mean() <= mean, (
        f"{_desc(c)}: max-abs {err.max():.3e}, mean-abs {err.mean():.3e}")
    assert np.array_equal(np.isneginf(l), np.isneginf(want_l)), _desc(c)
    fin = ~np.isneginf(want_l)
    if fin.any():
        assert np.abs(l[fin] - want_l[fin]).max() <= 1e-3, _desc(c)


@pytest.mark.parametrize("seed", range(24))
def test_sel_bwd_sweep(seed):
    from omnimem_amd.selection import sel_bwd, sel_fwd
    c = _case(8000 + seed, 256, 800, 8)
    q, k, v, ids = _inputs(c, seed)
    qd, kd, vd, idd = (x.to(DEV) for x in (q, k, v, ids))
    out, lse = sel_fwd(qd, kd, vd, idd, c["BS"], c["chunk"], c["scale"], c["causal"], c["G"])
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(seed + 1)).to(c["dtype"])
    dq, dk, dv = sel_bwd(qd, kd, vd, idd, out, lse, do.to(DEV), c["BS"], c["chunk"], c["scale"],
                         c["causal"], c["G"])
    want = O.selection_attention_bwd(
        q.double().numpy(), k.double().numpy(), v.double().numpy(), ids.numpy(),
        out.double().cpu().numpy(), lse.double().cpu().numpy(), do.double().numpy(), c["G"],
        c["scale"], O.dense_block_tokens(c["N"], c["BS"], c["chunk"], c["causal"]),
        chunk_size=c["chunk"], causal=c["causal"])
    mx, mean = BWD_TOL[c["dtype"]]
    for name, got, w in (("dq", dq, want[0]), ("dk", dk, want[1]), ("dv", dv, want[2])):
        g = got.float().cpu().numpy().astype(np.float64)
        if not np.abs(w).max() > 0:
            assert not np.abs(g).max() > 0, f"{name}: {_desc(c)}"
            continue
        err = np.abs(g - w)
        assert err.max() <= mx * np.abs(w).max(), f"{name} max-abs {err.max():.3e}: {_desc(c)}"
        assert err.mean() <= mean * np.abs(w).mean(), f"{name} mean-abs {err.mean():.3e}: {_desc(c)}"


@pytest.mark.parametrize("seed", range(48))
def test_topk_from_scores_sweep(seed):
    from omnimem_amd.index_topk import topk_from_scores
    r = np.random.default_rng(9000 + seed)
    r2 = np.random.default_rng(19000 + seed)
    MG, H, NC = int(r.integers(1, 101)), int(r.integers(1, 4)), int(r.integers(1, 3001))
    topk = int(r.choice([int(r.integers(1, 17)), int(r.integers(17, 65)),
                         int(r.integers(65, 129)), int(r.integers(129, 601))]))
    bs = int(r.choice([16, 30, 64]))
    chunk = int(bs * r.integers(1, 6))
    causal = bool(r.integers(0, 2))
    ex_win = int(r.integers(0, 3)) if not causal else 0
    G = int(r2.choice([1, 1, 4, 16]))  # query tokens per row: the row chunk is chunk // G rows
    mk = dict(block_size=bs, group_size=G, chunk_q=chunk * G, chunk_k=chunk, causal=int(causal),
              ex_win=ex_win, prog_excl=int(ex_win > 0), q_chunk_offset=int(r.integers(0, 3)) if ex_win else 0)
    s = r.integers(-20, 20, size=(1, MG, H, NC)).astype(np.float32) * 0.125
    s[r.random(s.shape) < 0.02] = -0.0
    s[r.random(s.shape) < 0.01] = -np.inf
    s[r.random(s.shape) < 0.005] = np.nan
    got = topk_from_scores(torch.from_numpy(s).to(DEV), topk, bs, chunk, chunk, causal,
                           ex_win=ex_win, prog_excl=bool(mk["prog_excl"]),
                           q_chunk_offset=mk["q_chunk_offset"], group_size=G).cpu().numpy()
    om = O.Mask(**mk)
    want = O.topk_select(s, topk, om) if topk <= 128 else O.topk_select_large(s, topk, om)
    np.testing.assert_array_equal(got, want, err_msg=f"MG={MG} H={H} NC={NC} topk={topk} {mk}")


def _e4m3_rows(q: torch.Tensor) -> np.ndarray:
    """q [1, M, H, D] quantised to e4m3 per (query, head) row with the page rule (scale amax /
    448, round to nearest even), as codes * scale: what the fp8 Q K^T kernel multiplies."""
    x = q.float().numpy()
    out = np.empty_like(x)
    for m in range(x.shape[1]):
        for h in range(x.shape[2]):
            c, sc = O.quantize_pages(x[0, m, h][None, :], 1)
            out[0, m, h] = O.dequantize_pages(c, sc)[0]
    return out


@pytest.mark.parametrize("seed", range(24))
def test_paged_selection_sweep(seed):
    """The paged cache (bf16 or fp8 pages, fp8 Q K^T, 16..64-token pages, ragged chunk tails,
    head dims 64 / 128, groups up to 128, negative scales, some units on the host, with or
    without the gated branch mix) against the float64 oracle on the values the kernel computes
    with (fp8: codes times page scales; fp8 Q K^T: the queries' e4m3 image too)."""
    from omnimem_amd.block_cache import PagedKVCache
    r = np.random.default_rng(9500 + seed)
    dtype = [torch.bfloat16, "fp8"][int(r.integers(0, 2))]
    H, D = int(r.integers(1, 4)), int(r.choice([64, 128]))
    fp8 = dtype == "fp8"
    qk8 = fp8 and bool(r.integers(0, 2))
    P = int(r.choice([16, 32, 64]))
    C = int(r.integers(P, 701))
    n = int(r.integers(1, 5))
    G = int(r.choice([16, 64, 128]))
    M = int(r.integers(1, 401))
    scale = float(r.choice([1.0, 1.0, -1.0])) * D ** -0.5
    gated = bool(r.integers(0, 2))
    host = bool(r.integers(0, 2))
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         qk_fp8=qk8, hbm_slots=H * n, host_slots=H * n, window_chunks=0)
    g = torch.Generator().manual_seed(seed)
    ks = [(torch.randn((1, C, H, D), generator=g) * 0.3).to(torch.bfloat16) for _ in range(n)]
    vs = [torch.randn((1, C, H, D), generator=g).to(torch.bfloat16) for _ in range(n)]
    for cid in range(n):
        cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
    if host:
        cache.evict_all()  # every unit read from the host pool
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    MG, npages = -(-M // G), n * cache.ppc
    T = int(r.integers(1, min(20, npages) + 1))
    ids = torch.randint(-1, npages, (1, MG, H, T), generator=g, dtype=torch.int32)
    kw = {}
    if gated:
        gates = torch.sigmoid(torch.randn((1, M, H, 3), generator=g) * 2).to(torch.bfloat16)
        o_cmp = torch.randn((1, M, H, D), generator=g).to(torch.bfloat16)
        o_swa = torch.randn((1, M, H, D), generator=g).to(torch.bfloat16)
        kw = dict(gates=gates.to(DEV), o_cmp=o_cmp.to(DEV), o_swa=o_swa.to(DEV))
    out, lse = cache.select(q.to(DEV), ids.to(DEV), 0, G, softmax_scale=scale, return_lse=True,
                            **kw)
    if fp8:
        kk = np.zeros((1, n * C, H, D), np.float32)
        vv = np.zeros_like(kk)
        for cid in range(n):
            for h in range(H):
                kc, vc, sk, sv = cache.read_unit(0, h, cid)
                for codes, sc, dst in ((kc, sk, kk), (vc, sv, vv)):
                    deq = O.dequantize_pages(codes.numpy(), sc.numpy()[:, None, None])
                    dst[0, cid * C:(cid + 1) * C, h] = deq.reshape(-1, D)[:C]
    else:
        kk = torch.cat(ks, 1).float().numpy()
        vv = torch.cat(vs, 1).float().numpy()
    qq = _e4m3_rows(q) if qk8 else q.float().numpy()
    want_o, want_l = O.selection_attention(qq, kk, vv, ids.numpy(), G, scale,
                                           O.paged_block_tokens(C, P, n))
    mx, mean = 2e-2, 1e-3
    if gated:  # the mix is O(1): its bf16 rounding alone is about 1e-3 mean-abs
        gg = gates.float().numpy().astype(np.float64)
        want_o = (gg[..., 0:1] * o_cmp.float().numpy() + gg[..., 1:2] * want_o
                  + gg[..., 2:3] * o_swa.float().numpy())
        mx, mean = 4e-2, 3e-3
    desc = (f"dtype={dtype} qk8={qk8} H={H} D={D} P={P} C={C} n={n} G={G} M={M} T={T} "
            f"scale={scale:.4f} gated={gated} host={host}")
    o = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(o - want_o)
    assert err.max() <= mx and err.mean() <= mean, (
        f"{desc}: max-abs {err.max():.3e}, mean-abs {err.mean():.3e}")
    l = lse.cpu().numpy().astype(np.float64)
    assert np.array_equal(np.isneginf(l), np.isneginf(want_l)), desc
    fin = ~np.isneginf(want_l)
    if fin.any():
        assert np.abs(l[fin] - want_l[fin]).max() <= 1e-3, desc
    cache.close()


@pytest.mark.parametrize("seed", range(16))
def test_fused_topk_sweep(seed):
    """parallel_nsa_topk on random shapes: bf16 / f16 at head dims 64 / 128 with topk <= 16 (the
    MFMA path: indices equal the oracle's rule on the kernel's own scores, scores within the fp32
    summation bound) and fp32 or topk up to 200 (the fmaf chain: bit-exact against the oracle's
    scores, path A to 128, path B past it); causal chunks, the AR window exclusion, ragged tails."""
    from _topk_checks import check_mfma_topk
    from omnimem_amd.index_topk import parallel_nsa_topk
    r = np.random.default_rng(9700 + seed)
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(r.integers(0, 3))]
    D = int(r.choice([64, 128]))
    H = int(r.integers(1, 4))
    G = int(r.choice([16, 32, 64]))
    T = int(r.integers(1, 3001))
    NC = int(r.integers(1, 1201))
    topk = int(r.choice([int(r.integers(1, 17)), int(r.integers(1, 17)), int(r.integers(17, 201))]))
    chunk = int(G * r.integers(1, 8))
    causal = bool(r.integers(0, 2))
    exw = 0 if causal else int(r.integers(0, 3))
    qoff = int(r.integers(0, 4)) if exw else 0
    bpc = int(r.integers(1, 40)) if exw else 0
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((1, T, H, D), generator=g).to(dtype)
    k = torch.randn((1, NC, H, D), generator=g).to(dtype)
    kw = dict(block_size=64, chunk_size=chunk, causal=causal, exclude_window_chunks=exw,
              progressive_exclude=exw > 0, q_chunk_offset=qoff, blocks_per_chunk=bpc)
    mask = O.Mask(block_size=64, group_size=G, chunk_q=chunk, chunk_k=chunk, blocks_per_chunk=bpc,
                  q_chunk_offset=qoff, ex_win=exw, causal=int(causal), prog_excl=int(exw > 0))
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), topk, group_size=G, **kw).cpu().numpy()
    desc = f"dtype={dtype} D={D} H={H} G={G} T={T} NC={NC} topk={topk} {kw}"
    if dtype != torch.float32 and topk <= 16:
        check_mfma_topk(q.to(DEV), k.to(DEV), topk, mask, D ** -0.5, G, got=got, **kw)
        return
    dt = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype]
    scores = O.block_scores(O.pool_mean(q.float().numpy(), G, dt), k.float().numpy(), D ** -0.5)
    want = (O.topk_select(scores, topk, mask) if topk <= 128
            else O.topk_select_large(scores, topk, mask))
    np.testing.assert_array_equal(got, want, err_msg=desc)


@pytest.mark.parametrize("seed", range(16))
def test_paged_append_sweep(seed):
    """Cache appends over random geometries (heads, head dims 64 / 96 / 128, pages of 16..100
    tokens, chunk lengths with ragged last pages, bf16 or fp8 pages, a window ring or none),
    bit-exact: page bytes (bf16) or e4m3 codes and per-page scales (fp8), the pooled K / V rows
    of each page, and the ring slot's copy of the chunk."""
    from omnimem_amd.block_cache import PagedKVCache
    r = np.random.default_rng(9900 + seed)
    dtype = [torch.bfloat16, "fp8"][int(r.integers(0, 2))]
    H, D = int(r.integers(1, 5)), int(r.choice([64, 96, 128]))
    P = int(r.choice([16, 30, 64, 64, 100]))
    C = int(r.integers(P, 1201))
    n = int(r.integers(1, 4))
    ring = bool(r.integers(0, 2))
    fp8 = dtype == "fp8"
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         hbm_slots=H * n, host_slots=H * n, window_chunks=n if ring else 0,
                         keep_window_kv=ring)
    g = torch.Generator().manual_seed(seed)
    ppc = cache.ppc
    desc = f"dtype={dtype} H={H} D={D} P={P} C={C} n={n} ring={ring}"
    for cid in range(n):
        k = (torch.randn((1, C, H, D), generator=g) * 2.0).to(torch.bfloat16)
        v = torch.randn((1, C, H, D), generator=g).to(torch.bfloat16)
        cache.append(0, k.to(DEV), v.to(DEV), cid)
        kc_all, vc_all = cache.cmp_history(0)
        for x, pooled in ((k, kc_all), (v, vc_all)):
            want = O.pool_mean(x.float().numpy(), P, "bf16")
            got = pooled[:, cid * ppc:(cid + 1) * ppc].float().cpu().numpy()
            np.testing.assert_array_equal(got, want, err_msg=f"pooled, {desc}")
        for h in range(H):
            unit = cache.read_unit(0, h, cid)
            for j, x in enumerate((k, v)):
                rows = np.zeros((ppc * P, D), np.float32)
                rows[:C] = x[0, :, h].float().numpy()
                pages = rows.reshape(ppc, P, D)
                if not fp8:
                    np.testing.assert_array_equal(unit[j].float().numpy(), pages,
                                                  err_msg=f"pages h{h}, {desc}")
                    continue
                codes, scales = unit[j].numpy(), unit[2 + j].numpy()
                for p in range(ppc):
                    want_c, want_s = O.quantize_pages(pages[p], min(P, C - p * P))
                    np.testing.assert_array_equal(codes[p], want_c, err_msg=f"h{h} p{p}, {desc}")
                    assert np.float32(scales[p]) == want_s, (h, p, desc)
        if ring:
            w = cid % cache.window
            assert torch.equal(cache.win_k[0][w].cpu(), k[0]), desc
            assert torch.equal(cache.win_v[0][w].cpu(), v[0]), desc
    cache.close()


@pytest.mark.parametrize("seed", range(12))
def test_sel_fwd_gated_sweep(seed):
    """Dense selection with the NSA branch mix in its epilogue (bf16) over random shapes, against
    g0 o_cmp + g1 o_slc + g2 o_swa from the float64 oracle's o_slc."""
    from omnimem_amd.selection import sel_fwd_gated
    c = _case(9300 + seed, 400, 1500, 12)
    c["dtype"] = torch.bfloat16
    if c["D"] not in (64, 128):  # the gated epilogue is on the MFMA paths only
        c["D"], c["scale"] = 128, (1.0 if c["scale"] > 0 else -1.0) * 128 ** -0.5
    q, k, v, ids = _inputs(c, seed)
    gen = torch.Generator().manual_seed(seed + 100)
    B, M, H, D = c["B"], c["M"], c["H"], c["D"]
    oc = torch.randn((B, M, H, D), generator=gen).to(torch.bfloat16)
    ow = torch.randn((B, M, H, D), generator=gen).to(torch.bfloat16)
    g = torch.sigmoid(torch.randn((B, M, H, 3), generator=gen) * 2).to(torch.bfloat16)
    out = sel_fwd_gated(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), c["BS"], c["chunk"],
                        c["scale"], c["causal"], c["G"], g.to(DEV), oc.to(DEV), ow.to(DEV))
    slc, _ = O.selection_attention(
        q.float().numpy(), k.float().numpy(), v.float().numpy(), ids.numpy(), c["G"], c["scale"],
        O.dense_block_tokens(c["N"], c["BS"], c["chunk"], c["causal"]), chunk_size=c["chunk"],
        causal=c["causal"])
    gg = g.double().numpy()
    want = gg[..., 0:1] * oc.double().numpy() + gg[..., 1:2] * slc + gg[..., 2:3] * ow.double().numpy()
    err = np.abs(out.double().cpu().numpy() - want)
    # the mix is O(1) (o_cmp, o_swa ~ N(0, 1)): its bf16 rounding alone is about 1e-3 mean-abs
    assert err.max() <= 4e-2 and err.mean() <= 3e-3, (
        f"{_desc(c)}: max-abs {err.max():.3e}, mean-abs {err.mean():.3e}")


@pytest.mark.parametrize("seed", range(12))
def test_window_attention_sweep(seed):
    """Sliding-window attention over the paged cache (pages read in place, or the dense bf16 ring)
    on random geometries against float64 softmax attention over every token of the last W chunks
    (all of them while fewer than W exist)."""
    from omnimem_amd.block_cache import PagedKVCache
    r = np.random.default_rng(9800 + seed)
    dtype = [torch.bfloat16, "fp8"][int(r.integers(0, 2))]
    H, D = int(r.integers(1, 4)), int(r.choice([64, 128]))
    P = int(r.choice([16, 32, 64]))
    C = int(r.integers(P, 501))
    n = int(r.integers(1, 6))
    W = int(r.integers(1, 4))
    ring = bool(r.integers(0, 2))
    M = int(r.integers(1, 301))
    fp8 = dtype == "fp8"
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         window_chunks=W, keep_window_kv=ring)
    g = torch.Generator().manual_seed(seed)
    ks = [(torch.randn((1, C, H, D), generator=g) * 0.3).to(torch.bfloat16) for _ in range(n)]
    vs = [torch.randn((1, C, H, D), generator=g).to(torch.bfloat16) for _ in range(n)]
    for cid in range(n):
        cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    with torch.no_grad():
        out = cache.window_attention(q.to(DEV), 0)
    first = max(0, n - W)
    if fp8 and not ring:  # pages hold codes: the kernel computes with codes times page scales
        kk = np.zeros((1, (n - first) * C, H, D), np.float32)
        vv = np.zeros_like(kk)
        for i, cid in enumerate(range(first, n)):
            for h in range(H):
                kc, vc, sk, sv = cache.read_unit(0, h, cid)
                for codes, sc, dst in ((kc, sk, kk), (vc, sv, vv)):
                    deq = O.dequantize_pages(codes.numpy(), sc.numpy()[:, None, None])
                    dst[0, i * C:(i + 1) * C, h] = deq.reshape(-1, D)[:C]
    else:
        kk = torch.cat(ks[first:], 1).float().numpy()
        vv = torch.cat(vs[first:], 1).float().numpy()
    Nw = kk.shape[1]
    ids = np.broadcast_to(np.arange(-(-Nw // 64), dtype=np.int32), (1, -(-M // 64), H, -(-Nw // 64)))
    want_o, _ = O.selection_attention(q.float().numpy(), kk, vv, ids, 64, D ** -0.5,
                                      O.dense_block_tokens(Nw, 64, 1, False))
    o = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(o - want_o)
    desc = f"dtype={dtype} ring={ring} H={H} D={D} P={P} C={C} n={n} W={W} M={M}"
    assert err.max() <= 2e-2 and err.mean() <= 1e-3, (
        f"{desc}: max-abs {err.max():.3e}, mean-abs {err.mean():.3e}")
    cache.close()


# (12, 3): a pool one chunk tighter, where making room for an append evicted units of the chunk
# being written (regression case of the append fix)
@pytest.mark.parametrize("seed,slack", [(s, 4) for s in range(48)] + [(12, 3)])
def test_cache_residency_sequence_sweep(seed, slack):
    """A random sequence of cache operations on two caches fed the same data: one with every unit
    in HBM, one whose small HBM pool forces evictions and promotions (asynchronous flushes, moves
    pending across appends), plus evict_all, rewrites of earlier chunks, snapshot / rewrite /
    restore or discard of a chunk range, flushes without a reservation and a reset.  After every step the two caches' selections must be bit-identical:
    where a unit sits never changes what the kernel reads."""
    from omnimem_amd.block_cache import PagedKVCache
    r = np.random.default_rng(9600 + seed)
    dtype = [torch.bfloat16, "fp8"][int(r.integers(0, 2))]
    L, H = int(r.integers(1, 3)), int(r.integers(1, 3))
    D = int(r.choice([64, 128]))
    P = int(r.choice([32, 64]))
    C = int(r.integers(P, 400))
    n = int(r.integers(4, 8))
    W = int(r.integers(0, 3))
    G, M = 64, int(r.integers(1, 200))
    fp8 = dtype == "fp8"
    units = L * H * n
    mk = lambda slots: PagedKVCache(L, H, D, max_chunks=n, chunk_len=C, page_tokens=P,
                                    dtype=dtype, hbm_slots=slots, host_slots=2 * units,
                                    window_chunks=W, keep_window_kv=fp8 and W > 0)
    # the small pool holds the window's protected units, the two reserved next chunks of an
    # asynchronous flush and the chunk a snapshot keeps while it is rewritten
    full, small = mk(2 * units), mk(L * H * int(r.integers(W + slack, max(W + slack + 1, n))))
    g = torch.Generator().manual_seed(seed)
    desc = f"dtype={dtype} L={L} H={H} D={D} P={P} C={C} n={n} W={W} small={small.n_slots}"

    def write(l, c):
        k = (torch.randn((1, C, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
        v = torch.randn((1, C, H, D), generator=g).to(torch.bfloat16).to(DEV)
        full.append(l, k, v, c)
        small.append(l, k, v, c)

    def compare(nc, step):
        for l in range(L):
            q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
            ids = r.integers(-1, nc * small.ppc, size=(1, -(-M // G), H, int(r.integers(1, 12))))
            ids = torch.from_numpy(ids.astype(np.int32)).to(DEV)
            a, la = full.select(q, ids, l, G, return_lse=True)
            # the small cache stages its host pages first half of the time (prefetch)
            pf = small.prefetch(ids, l) if r.random() < 0.5 else None
            b, lb = small.select(q, ids, l, G, return_lse=True, prefetch=pf)
            torch.cuda.synchronize()
            assert torch.equal(a, b) and torch.equal(la, lb), f"{step} (prefetch {pf is not None}): {desc}"

    # the pinned regression case runs its original sequence; the others also discard snapshots
    # and flush without a reservation (drawn from a second generator)
    extra, r2 = slack != 3, np.random.default_rng(19600 + seed)
    snap = None
    for cid in range(n):
        for l in range(L):
            write(l, cid)
        compare(cid + 1, f"append {cid}")
        full.flush()
        small.flush()
        compare(cid + 1, f"flush {cid}")
        x = r.random()
        if x < 0.25 and cid > 0:  # rewrite an earlier chunk (its units may be moving)
            c = int(r.integers(0, cid))
            for l in range(L):
                write(l, c)
            compare(cid + 1, f"rewrite {c}")
        elif x < 0.4:
            small.evict_all()
            compare(cid + 1, "evict_all")
        elif x < 0.6 and snap is None and cid >= 1:
            lo = int(r.integers(0, cid))
            snap = (full.snapshot_chunks(lo, cid + 1), small.snapshot_chunks(lo, cid + 1), lo, cid)
            for l in range(L):
                write(l, lo)
            compare(cid + 1, f"snapshot + rewrite {lo}")
        elif snap is not None:
            if not extra or r2.random() < 0.7:
                full.restore_chunks(snap[0])
                small.restore_chunks(snap[1])
                compare(cid + 1, f"restore {snap[2]}..{snap[3]}")
            else:
                full.discard_snapshot(snap[0])
                small.discard_snapshot(snap[1])
                compare(cid + 1, f"discard {snap[2]}..{snap[3]}")
            snap = None
        if extra and r2.random() < 0.2:  # a flush that reserves nothing for the next chunk
            full.flush(reserve_next_chunk=False)
            small.flush(reserve_next_chunk=False)
            compare(cid + 1, f"flush without reservation {cid}")
    if snap is not None:
        full.discard_snapshot(snap[0])
        small.discard_snapshot(snap[1])
    # after a reset both caches start over and must agree again
    full.reset()
    small.reset()
    for l in range(L):
        write(l, 0)
    compare(1, "after reset")
    full.close()
    small.close()
