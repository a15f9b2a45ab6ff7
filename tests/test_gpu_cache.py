"""GPU parity of the block KV cache path: reference pointer tables, the paged cache (append,
fused block compression, fp8 pages, paged selection, evict / promote, LRU), and the reference's
block-store kernels K1 / K2 / K3.

Bit-exact: addresses, cache bytes (bf16 pages, fp8 codes and scales), pooled keys / values,
residency moves, dedup keys.  Attention: float64 oracle within the bf16 tolerances
(2e-2 max-abs, 1e-3 mean-abs), and bit-exact invariance under residency changes.
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O
from oracle.lru_model import ReferenceLRU

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check_attn(out, lse, want_o, want_l, mx=2e-2, mean=1e-3):
    o = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(o - want_o)
    assert err.max() <= mx, f"max-abs {err.max():.3e}"
    assert err.mean() <= mean, f"mean-abs {err.mean():.3e}"
    if lse is not None:
        l = lse.cpu().numpy().astype(np.float64)
        assert np.array_equal(np.isneginf(l), np.isneginf(want_l))
        fin = ~np.isneginf(want_l)
        if fin.any():
            assert np.abs(l[fin] - want_l[fin]).max() <= 1e-3


# ------------------------------------------------------------------ pointer tables (reference)
def test_build_ptr_table_matches_address_rule():
    from omnimem_amd.padded_ptr import build_ptr_table
    rng = np.random.default_rng(0)
    B, MG, H, T, MC, bpc = 2, 5, 3, 7, 6, 4
    ids = rng.integers(-2, MC * bpc + 3, size=(B, MG, H, T)).astype(np.int32)
    base_k = rng.integers(1, 2 ** 40, size=(H, MC)).astype(np.int64) * 256
    base_v = rng.integers(1, 2 ** 40, size=(H, MC)).astype(np.int64) * 256
    base_k[1, 2] = 0
    base_v[2, 0] = 0
    nblk = np.array([MC * bpc, 3 * bpc, MC * bpc - 1], np.int32)
    bstride, icb = 1 << 20, 4096
    pk, pv = build_ptr_table(torch.from_numpy(ids).to(DEV), torch.from_numpy(base_k).to(DEV),
                             torch.from_numpy(base_v).to(DEV), torch.from_numpy(nblk).to(DEV),
                             bstride, bpc, icb)
    want_k = np.zeros_like(ids, dtype=np.int64)
    want_v = np.zeros_like(ids, dtype=np.int64)
    for b, g, h, t in np.ndindex(*ids.shape):
        bid = int(ids[b, g, h, t])
        if bid < 0 or bid >= nblk[h]:
            continue
        cid, loc = divmod(bid, bpc)
        if cid >= MC:
            continue
        d = b * bstride + loc * icb
        want_k[b, g, h, t] = base_k[h, cid] + d if base_k[h, cid] else 0
        want_v[b, g, h, t] = base_v[h, cid] + d if base_v[h, cid] else 0
    np.testing.assert_array_equal(pk.cpu().numpy(), want_k)
    np.testing.assert_array_equal(pv.cpu().numpy(), want_v)


@pytest.mark.parametrize("G", [15, 150])  # 150: 4-wave workgroups (3 subgroups of a group)
def test_padded_ptr_fast_reference_geometry(G):
    """The reference's AR shape (30-token blocks, groups of 15, 4680-token chunks) over
    per-head chunk tensors addressed by base pointers; a non-resident chunk (base 0) is skipped."""
    from omnimem_amd.padded_ptr import selection_attention_padded_ptr_fast
    g = torch.Generator().manual_seed(1)
    H, D, C, BS, T, n_chunks = 2, 128, 4680, 30, 8, 3
    chunks_k = [[(torch.randn((1, C, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
                 for _ in range(n_chunks)] for _ in range(H)]
    chunks_v = [[torch.randn((1, C, D), generator=g).to(torch.bfloat16).to(DEV)
                 for _ in range(n_chunks)] for _ in range(H)]
    base_k = torch.tensor([[t.data_ptr() for t in row] for row in chunks_k], dtype=torch.int64)
    base_v = torch.tensor([[t.data_ptr() for t in row] for row in chunks_v], dtype=torch.int64)
    base_k[1, 0] = 0  # head 1, chunk 0 is "on the CPU"
    M = 150
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    bpc = C // BS
    ids = torch.stack([torch.randperm(n_chunks * bpc, generator=g)[:T] for _ in range(M // G * H)])
    ids = ids.view(1, M // G, H, T).to(torch.int32)
    strides = {"batch_stride_bytes": C * D * 2, "token_stride_bytes": D * 2, "stride_bn": D,
               "stride_bd": 1, "chunk_len": C}
    out, lse = selection_attention_padded_ptr_fast(
        q.to(DEV), ids.to(DEV), BS, G, C, base_k.to(DEV), base_v.to(DEV),
        torch.full((H,), n_chunks, dtype=torch.int32, device=DEV), strides, return_lse=True)
    k = torch.stack([torch.cat([c[0] for c in row]) for row in chunks_k], 1)[None].float().cpu()
    v = torch.stack([torch.cat([c[0] for c in row]) for row in chunks_v], 1)[None].float().cpu()
    ids_np = ids.numpy().copy()
    # the skipped chunk contributes nothing: drop its blocks from head 1 in the oracle
    ids_np[:, :, 1][ids_np[:, :, 1] // bpc == 0] = -1
    want_o, want_l = O.selection_attention(q.float().numpy(), k.numpy(), v.numpy(), ids_np, G,
                                           D ** -0.5, O.dense_block_tokens(n_chunks * C, BS, 1, False))
    _check_attn(out, lse, want_o, want_l)


@pytest.mark.parametrize("shift,G", [(1, 15), (4, 150), (3, 15)])
def test_padded_ptr_fast_misaligned_bases(shift, G):
    """Chunk bases that are only 2- or 8-byte aligned (views `shift` elements into their
    allocations), as the reference's pointer contract allows (csrc/ptr_table.cu:32-49): the
    device detects each block's misalignment and copies it with 2-byte loads; results must match
    the oracle exactly as for aligned bases.  Head 1 mixes aligned and misaligned chunks."""
    from omnimem_amd.padded_ptr import selection_attention_padded_ptr_fast
    g = torch.Generator().manual_seed(7 + shift)
    H, D, C, BS, T, n_chunks = 2, 128, 4680, 30, 8, 3

    def chunk(i, scale):
        x = (torch.randn((1, C * D + 8), generator=g) * scale).to(torch.bfloat16).to(DEV)
        off = shift if i % 2 == 0 else 0
        return x[:, off:off + C * D].view(1, C, D)

    chunks_k = [[chunk(h + c, 0.3) for c in range(n_chunks)] for h in range(H)]
    chunks_v = [[chunk(h + c + 1, 1.0) for c in range(n_chunks)] for h in range(H)]
    base_k = torch.tensor([[t.data_ptr() for t in row] for row in chunks_k], dtype=torch.int64)
    base_v = torch.tensor([[t.data_ptr() for t in row] for row in chunks_v], dtype=torch.int64)
    assert ((base_k % 16) != 0).any() and ((base_v % 16) != 0).any()
    M = 150
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    bpc = C // BS
    ids = torch.stack([torch.randperm(n_chunks * bpc, generator=g)[:T] for _ in range(M // G * H)])
    ids = ids.view(1, M // G, H, T).to(torch.int32)
    strides = {"batch_stride_bytes": C * D * 2, "token_stride_bytes": D * 2, "stride_bn": D,
               "stride_bd": 1, "chunk_len": C}
    out, lse = selection_attention_padded_ptr_fast(
        q.to(DEV), ids.to(DEV), BS, G, C, base_k.to(DEV), base_v.to(DEV),
        torch.full((H,), n_chunks, dtype=torch.int32, device=DEV), strides, return_lse=True)
    k = torch.stack([torch.cat([c[0] for c in row]) for row in chunks_k], 1)[None].float().cpu()
    v = torch.stack([torch.cat([c[0] for c in row]) for row in chunks_v], 1)[None].float().cpu()
    want_o, want_l = O.selection_attention(q.float().numpy(), k.numpy(), v.numpy(), ids.numpy(),
                                           G, D ** -0.5,
                                           O.dense_block_tokens(n_chunks * C, BS, 1, False))
    _check_attn(out, lse, want_o, want_l)


# ------------------------------------------------------------------ paged cache
def _chunk(g, S, H, D, scale=1.0, t_dist=False):
    if t_dist:
        x = torch.distributions.StudentT(4.0).sample((1, S, H, D))
    else:
        x = torch.randn((1, S, H, D), generator=g)
    return (x * scale).to(torch.bfloat16)


def _pages(x: np.ndarray, C: int, P: int):
    """[S, D] chunk (S <= C) -> [ppc, P, D] pages with zero padding."""
    ppc = -(-C // P)
    out = np.zeros((ppc * P, x.shape[-1]), np.float32)
    out[:x.shape[0]] = x
    return out.reshape(ppc, P, -1)


def test_paged_append_rejects_partial_chunks():
    """Whole chunks only: a shorter write would leave page slots that attention reads (every
    page of a written chunk counts min(page_tokens, chunk_len - p*page_tokens) tokens)."""
    from omnimem_amd.backend import BlockKVBackendError
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(4000)
    H, D, C, P = 2, 128, 4680, 64
    cache = PagedKVCache(1, H, D, max_chunks=2, chunk_len=C, page_tokens=P, hbm_slots=4,
                         window_chunks=0)
    k = _chunk(g, 4000, H, D).to(DEV)
    with pytest.raises(BlockKVBackendError, match="whole chunks"):
        cache.append(0, k, k, 0)
    kv = cache.layer_view(0)
    from omnimem_amd import _lib
    import ctypes
    with pytest.raises(BlockKVBackendError, match="whole chunks"):
        _lib.call("omm_paged_append", ctypes.byref(kv), _lib.view4(k), _lib.view4(k), 0, 4000,
                  None, None, 0, _lib.stream_of(k), error=BlockKVBackendError)


# (heads, head dim, page tokens): pages of at most 64 tokens take the 4-wave staged kernel
# (partial head groups: 3 of 4 heads, 5 of 8), longer pages the one-wave kernel
APPEND_GEOMS = [(3, 128, 64), (5, 64, 30), (2, 128, 96)]


@pytest.mark.parametrize("H,D,P", APPEND_GEOMS)
def test_paged_append_bf16_bitexact_and_pooled(H, D, P):
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.index_topk import block_pool
    S = 4680
    g = torch.Generator().manual_seed(S + P)
    C = 4680
    cache = PagedKVCache(1, H, D, max_chunks=4, chunk_len=C, page_tokens=P, hbm_slots=12,
                         window_chunks=0)
    k, v = _chunk(g, S, H, D), _chunk(g, S, H, D)
    cache.append(0, k.to(DEV), v.to(DEV), 2)
    for h in range(H):
        kk, vv = cache.read_unit(0, h, 2)
        np.testing.assert_array_equal(kk.float().numpy(), _pages(k[0, :, h].float().numpy(), C, P))
        np.testing.assert_array_equal(vv.float().numpy(), _pages(v[0, :, h].float().numpy(), C, P))
    kc, vc = cache.cmp_history(0)
    ppc = cache.ppc
    got_k = kc[:, 2 * ppc:3 * ppc].float().cpu().numpy()
    got_v = vc[:, 2 * ppc:3 * ppc].float().cpu().numpy()
    nfull = -(-S // P)
    np.testing.assert_array_equal(got_k[:, :nfull], O.pool_mean(k.float().numpy(), P, "bf16"))
    np.testing.assert_array_equal(got_v[:, :nfull], O.pool_mean(v.float().numpy(), P, "bf16"))
    assert not got_k[:, nfull:].any()
    # the fused pool equals the standalone block pool kernel
    np.testing.assert_array_equal(got_k[:, :nfull], block_pool(k.to(DEV), P).float().cpu().numpy())


@pytest.mark.parametrize("H,D,P", [(2, 128, 64), (3, 64, 30), (2, 128, 80)])
def test_paged_append_fp8_codes_and_scales_bitexact(H, D, P):
    from omnimem_amd.block_cache import PagedKVCache
    torch.manual_seed(7 + P)
    C = 4680
    cache = PagedKVCache(1, H, D, max_chunks=2, chunk_len=C, page_tokens=P, dtype="fp8",
                         hbm_slots=4, window_chunks=0)
    k, v = _chunk(None, C, H, D, 3.0, True), _chunk(None, C, H, D, 2.0, True)
    k[0, 128:192, 1] = 0  # page 2 of head 1 all zero: scale 1, codes 0
    cache.append(0, k.to(DEV), v.to(DEV), 0)
    for h in range(H):
        kc, vc, sk, sv = cache.read_unit(0, h, 0)
        for x, codes, sc in ((k, kc, sk), (v, vc, sv)):
            pages = _pages(x[0, :, h].float().numpy(), C, P)
            for p in range(cache.ppc):
                valid = min(P, C - p * P)
                want_c, want_s = O.quantize_pages(pages[p], valid)
                np.testing.assert_array_equal(codes[p].numpy(), want_c, err_msg=f"h{h} p{p}")
                assert np.float32(sc[p].item()) == want_s, (h, p)


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
@pytest.mark.parametrize("H,D,P", [(3, 128, 64), (2, 64, 30), (2, 128, 80)])
def test_paged_append_ring_copy(dtype, H, D, P):
    """The window ring slot an fp8 cache keeps (written by the append kernel from its registers
    for head dim 64 / 128 and pages of <= 64 tokens, by a copy kernel otherwise) holds k / v bit
    for bit, and the pages, scales and pooled rows equal those of a cache without the ring."""
    from omnimem_amd.block_cache import PagedKVCache
    torch.manual_seed(11 + P)
    C, W = 4680, 2
    kw = dict(max_chunks=4, chunk_len=C, page_tokens=P, dtype=dtype, hbm_slots=4 * H,
              window_chunks=W)
    ring = PagedKVCache(1, H, D, keep_window_kv=True, **kw)
    plain = PagedKVCache(1, H, D, keep_window_kv=False, **kw)
    for cid in range(3):
        k, v = _chunk(None, C, H, D, 2.0, True).to(DEV), _chunk(None, C, H, D, 1.5, True).to(DEV)
        ring.append(0, k, v, cid)
        plain.append(0, k, v, cid)
        assert torch.equal(ring.win_k[0][cid % W], k[0]) and torch.equal(ring.win_v[0][cid % W], v[0])
    for cid in range(3):
        for h in range(H):
            for a, b in zip(ring.read_unit(0, h, cid), plain.read_unit(0, h, cid)):
                assert torch.equal(a, b), (cid, h)
    for a, b in zip(ring.cmp_history(0), plain.cmp_history(0)):
        assert torch.equal(a, b)


def test_paged_append_ring_without_unit_slots():
    """Heads whose unit slot is not allocated (table entry -1) skip their pages but still get
    the ring copy; a ring view overlapping the input is rejected."""
    import ctypes
    from omnimem_amd import _lib
    from omnimem_amd.backend import BlockKVBackendError
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(12)
    H, D, C, P = 2, 128, 4680, 64
    cache = PagedKVCache(1, H, D, max_chunks=2, chunk_len=C, page_tokens=P, dtype="fp8",
                         hbm_slots=2, window_chunks=1, keep_window_kv=True)
    k, v = _chunk(g, C, H, D).to(DEV), _chunk(g, C, H, D).to(DEV)
    rk, rv = torch.zeros_like(k), torch.zeros_like(v)
    pool_before = cache.pool_k.clone()
    kv = cache.layer_view(0)  # nothing written: every unit slot is -1
    _lib.call("omm_paged_append_ring", ctypes.byref(kv), _lib.view4(k), _lib.view4(v), 0, C,
              None, None, _lib.view4(rk), _lib.view4(rv), 0, _lib.stream_of(k),
              error=BlockKVBackendError)
    torch.cuda.synchronize()
    assert torch.equal(rk, k) and torch.equal(rv, v)
    assert torch.equal(cache.pool_k, pool_before)
    with pytest.raises(BlockKVBackendError, match="overlaps"):
        _lib.call("omm_paged_append_ring", ctypes.byref(kv), _lib.view4(k), _lib.view4(v), 0, C,
                  None, None, _lib.view4(k), None, 0, _lib.stream_of(k), error=BlockKVBackendError)


def _paged_oracle_inputs(chunks_k, chunks_v, fp8_cache=None, layer=0):
    """Concatenate chunk tensors [1, C, H, D] into the oracle's [1, n*C, H, D]; for an fp8
    cache, the dequantised values the kernel computes with (code * page scale in fp32: the kernel
    widens the codes to bf16 exactly and applies the scales to the scores and to p)."""
    if fp8_cache is None:
        return (torch.cat(chunks_k, 1).float().numpy(), torch.cat(chunks_v, 1).float().numpy())
    c = fp8_cache
    n = len(chunks_k)
    H, D, C = c.H, c.D, c.chunk_len
    out_k = np.zeros((1, n * C, H, D), np.float32)
    out_v = np.zeros_like(out_k)
    for cid in range(n):
        for h in range(H):
            kc, vc, sk, sv = c.read_unit(layer, h, cid)
            for codes, sc, dst in ((kc, sk, out_k), (vc, sv, out_v)):
                deq = O.dequantize_pages(codes.numpy(), sc.numpy()[:, None, None])
                deq = deq.reshape(-1, D)[:C]
                dst[0, cid * C:(cid + 1) * C, h] = deq
    return out_k, out_v


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
@pytest.mark.parametrize("G", [64, 128])  # 128: 4-wave workgroups over two 64-query halves
def test_paged_selection_matches_oracle_and_is_residency_invariant(dtype, G):
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.padded_ptr import selection_attention_paged
    torch.manual_seed(11)
    g = torch.Generator().manual_seed(11)
    H, D, C, P, T, n = 3, 128, 4680, 64, 16, 4
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         hbm_slots=H * n, host_slots=H * n, window_chunks=0)
    fp8 = dtype == "fp8"
    ks = [_chunk(g, C, H, D, 0.3, fp8) for _ in range(n)]
    vs = [_chunk(g, C, H, D, 1.0, fp8) for _ in range(n)]
    for cid in range(n):
        cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
    M = C
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    MG = -(-M // G)
    ppc = cache.ppc
    ids = torch.stack([torch.randperm(n * ppc, generator=g)[:T] for _ in range(MG * H)])
    ids = ids.view(1, MG, H, T).to(torch.int32)
    ids[0, 3, 1, :5] = -1
    ids[0, 5, 0, 0] = n * ppc + 3  # a page of a chunk that does not exist yet: skipped
    qd, idd = q.to(DEV), ids.to(DEV)
    with torch.no_grad():
        out, lse = selection_attention_paged(qd, idd, P, G, cache, 0, return_lse=True)
    kk, vv = _paged_oracle_inputs(ks, vs, cache if fp8 else None)
    want_o, want_l = O.selection_attention(q.float().numpy(), kk, vv, ids.numpy(), G, D ** -0.5,
                                           O.paged_block_tokens(C, P, n))
    _check_attn(out, lse, want_o, want_l)
    # move every unit to the host pool: the kernel reads it there, bit for bit the same
    cache.evict_all()
    assert all(cache.where(0, h, c) == "host" for h in range(H) for c in range(n))
    out2, lse2 = cache.select(qd, idd, 0, G, return_lse=True)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    # evicted bytes come back bit-exact after a promote
    before = [cache.read_unit(0, h, c) for h in range(H) for c in range(n)]
    cache.flush(reserve_next_chunk=False)
    after = [cache.read_unit(0, h, c) for h in range(H) for c in range(n)]
    assert all(cache.where(0, h, c) == "hbm" for h in range(H) for c in range(n))
    for a, b in zip(before, after):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    out3 = cache.select(qd, idd, 0, G)
    assert torch.equal(out, out3)


@pytest.mark.parametrize("qk8", [False, True])
def test_paged_selection_fp8_scale_extremes(qk8):
    """fp8 pages whose scales span the float range: the kernel folds s_k into the exponent scale
    and s_v into p as 2^(log2 s_v) with the row sum divided by s_v, so a zero V chunk (scale 1,
    all codes 0), a tiny chunk (values ~1e-30) and a large one (values ~1e30 in V, K kept
    moderate so the scores stay finite) must all match the float64 oracle on code * scale."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(91 + int(qk8))
    torch.manual_seed(91)
    H, D, C, P, T, n = 2, 128, 4680, 64, 16, 3
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype="fp8",
                         qk_fp8=qk8, hbm_slots=H * n, host_slots=H * n, window_chunks=0)
    ks = [_chunk(g, C, H, D, 0.3), _chunk(g, C, H, D, 1e-30), _chunk(g, C, H, D, 0.3)]
    vs = [torch.zeros((1, C, H, D), dtype=torch.bfloat16), _chunk(g, C, H, D, 1e-30),
          _chunk(g, C, H, D, 1e30)]
    for cid in range(n):
        cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
    _, _, sk, sv = cache.read_unit(0, 0, 1)
    assert float(sk.max()) < 1e-29 and float(cache.read_unit(0, 0, 0)[3].min()) == 1.0
    M, G = 700, 64
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    MG = -(-M // G)
    ids = torch.stack([torch.randperm(n * cache.ppc, generator=g)[:T] for _ in range(MG * H)])
    ids = ids.view(1, MG, H, T).to(torch.int32)
    out, lse = cache.select(q.to(DEV), ids.to(DEV), 0, G, return_lse=True)
    kk, vv = _fp8_cache_images(cache, n)
    qq = _quantized_rows(q) if qk8 else q.float().numpy()
    want_o, want_l = O.selection_attention(qq, kk, vv, ids.numpy(), G, D ** -0.5,
                                           O.paged_block_tokens(C, P, n))
    # outputs reach 1e30 where large-V pages are selected: compare relative to each row's scale
    o = out.float().cpu().numpy().astype(np.float64)
    scale = np.maximum(np.abs(want_o).max(-1, keepdims=True), 1e-300)
    err = np.abs(o - want_o) / scale
    assert np.isfinite(o).all()
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
    l = lse.cpu().numpy().astype(np.float64)
    assert np.abs(l - want_l).max() <= 1e-3


def _quantized_rows(q: torch.Tensor) -> np.ndarray:
    """The e4m3 image of q [1, M, H, D] quantised per (query, head) row with the page rule
    (scale amax / 448, round to nearest even): codes * scale, fp32."""
    x = q.float().numpy()
    out = np.empty_like(x)
    for m in range(x.shape[1]):
        for h in range(x.shape[2]):
            c, sc = O.quantize_pages(x[0, m, h][None, :], 1)
            out[0, m, h] = O.dequantize_pages(c, sc)[0]
    return out


def _fp8_cache_images(cache, n):
    """K and V as the kernels compute with them: codes * page scale in fp32 (the codes are
    widened exactly and the scales applied to the scores and to p)."""
    H, D, C = cache.H, cache.D, cache.chunk_len
    kk = np.zeros((1, n * C, H, D), np.float32)
    vv = np.zeros_like(kk)
    for cid in range(n):
        for h in range(H):
            kc, vc, sk, sv = cache.read_unit(0, h, cid)
            k = O.dequantize_pages(kc.numpy(), sk.numpy()[:, None, None]).reshape(-1, D)[:C]
            v = O.dequantize_pages(vc.numpy(), sv.numpy()[:, None, None]).reshape(-1, D)[:C]
            kk[0, cid * C:(cid + 1) * C, h] = k
            vv[0, cid * C:(cid + 1) * C, h] = v
    return kk, vv


@pytest.mark.parametrize("D,G,sign", [(128, 64, 1.0), (64, 128, 1.0), (128, 64, -1.0)])
def test_paged_selection_fp8_qk_matches_oracle(D, G, sign):
    """The fp8 Q K^T variant (qk_fp8): queries quantised to e4m3 per query row, K page codes on
    fp8 MFMA.  Checked against the float64 oracle run on the quantised queries and the
    dequantised K and V, at the bf16 tolerances; a
    negative scale exercises the codes' sign flip."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(int(D + G + (sign < 0)))
    torch.manual_seed(D + G)
    H, C, P, T, n = 3, 4680, 64, 16, 3
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype="fp8",
                         qk_fp8=True, hbm_slots=H * n, host_slots=H * n, window_chunks=0)
    ks = [_chunk(g, C, H, D, 0.3, True) for _ in range(n)]
    vs = [_chunk(g, C, H, D, 1.0, True) for _ in range(n)]
    for cid in range(n):
        cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
    M = 1000
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    MG = -(-M // G)
    ids = torch.stack([torch.randperm(n * cache.ppc, generator=g)[:T] for _ in range(MG * H)])
    ids = ids.view(1, MG, H, T).to(torch.int32)
    ids[0, 2, 1, :5] = -1
    scale = sign * D ** -0.5
    out, lse = cache.select(q.to(DEV), ids.to(DEV), 0, G, softmax_scale=scale, return_lse=True)
    kk, vv = _fp8_cache_images(cache, n)
    want_o, want_l = O.selection_attention(_quantized_rows(q), kk, vv, ids.numpy(), G, scale,
                                           O.paged_block_tokens(C, P, n))
    _check_attn(out, lse, want_o, want_l)


@pytest.mark.parametrize("dtype,qk8,G", [(torch.bfloat16, False, 64), (torch.bfloat16, False, 128),
                                         ("fp8", False, 64), ("fp8", True, 64)])
def test_gated_selection_mix_matches_float64(dtype, qk8, G):
    """The NSA branch mix fused into the selection epilogue (causal_wan_nsa_model.py:541-546):
    out = g0 * o_cmp + g1 * o_slc + g2 * o_swa against float64, with o_slc from the float64
    oracle on the cache's values; the bf16 tolerances of attention outputs.  The plain
    selection of the same call must equal the gated one with gates (0, 1, 0)."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(77 + G)
    torch.manual_seed(77)
    H, D, C, P, T, n = 3, 128, 4680, 64, 16, 3
    fp8 = dtype == "fp8"
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         qk_fp8=qk8, hbm_slots=H * n, host_slots=H * n, window_chunks=0)
    ks = [_chunk(g, C, H, D, 0.3, fp8) for _ in range(n)]
    vs = [_chunk(g, C, H, D, 1.0, fp8) for _ in range(n)]
    for cid in range(n):
        cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
    M = 1500
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    MG = -(-M // G)
    ids = torch.stack([torch.randperm(n * cache.ppc, generator=g)[:T] for _ in range(MG * H)])
    ids = ids.view(1, MG, H, T).to(torch.int32)
    gates = torch.sigmoid(torch.randn((1, M, H, 3), generator=g) * 2).to(torch.bfloat16)
    o_cmp = torch.randn((1, M, H, D), generator=g).to(torch.bfloat16)
    o_swa = torch.randn((1, M, H, D), generator=g).to(torch.bfloat16)
    qd, idd = q.to(DEV), ids.to(DEV)
    mix, lse = cache.select(qd, idd, 0, G, gates=gates.to(DEV), o_cmp=o_cmp.to(DEV),
                            o_swa=o_swa.to(DEV), return_lse=True)
    if fp8:
        kk, vv = _fp8_cache_images(cache, n)
        qq = _quantized_rows(q) if qk8 else q.float().numpy()
    else:
        kk, vv = torch.cat(ks, 1).float().numpy(), torch.cat(vs, 1).float().numpy()
        qq = q.float().numpy()
    o_slc, want_l = O.selection_attention(qq, kk, vv, ids.numpy(), G, D ** -0.5,
                                          O.paged_block_tokens(C, P, n))
    gg = gates.float().numpy().astype(np.float64)
    want = (gg[..., 0:1] * o_cmp.float().numpy() + gg[..., 1:2] * o_slc
            + gg[..., 2:3] * o_swa.float().numpy())
    # the mix is O(1) (o_cmp, o_swa ~ N(0, 1)): its bf16 rounding alone is about 1e-3 mean-abs
    _check_attn(mix, lse, want, want_l, mx=4e-2, mean=3e-3)
    one = torch.zeros_like(gates)
    one[..., 1] = 1.0
    plain = cache.select(qd, idd, 0, G)
    via_gate = cache.select(qd, idd, 0, G, gates=one.to(DEV), o_cmp=o_cmp.to(DEV),
                            o_swa=o_swa.to(DEV))
    assert torch.equal(plain, via_gate)


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
def test_gated_selection_output_aliasing(dtype):
    """out may be the very view o_cmp is on a bf16 cache (the fused epilogue reads each element
    before writing it) and gives the same mix; an fp8 cache (two passes) rejects it, and both
    reject a partial overlap."""
    from omnimem_amd.backend import BlockKVBackendError
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(5)
    H, D, C, P, T, n, G, M = 2, 128, 512, 64, 4, 2, 64, 256
    fp8 = dtype == "fp8"
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         window_chunks=0)
    for cid in range(n):
        cache.append(0, _chunk(g, C, H, D, 0.3, fp8).to(DEV), _chunk(g, C, H, D, 1.0, fp8).to(DEV),
                     cid)
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    ids = torch.stack([torch.randperm(n * cache.ppc, generator=g)[:T] for _ in range(M // G * H)])
    ids = ids.view(1, M // G, H, T).to(torch.int32).to(DEV)
    gates = torch.sigmoid(torch.randn((1, M, H, 3), generator=g)).to(torch.bfloat16).to(DEV)
    o_cmp = torch.randn((1, M, H, D), generator=g).to(torch.bfloat16).to(DEV)
    o_swa = torch.randn((1, M, H, D), generator=g).to(torch.bfloat16).to(DEV)
    want = cache.select(q, ids, 0, G, gates=gates, o_cmp=o_cmp, o_swa=o_swa)
    if fp8:
        with pytest.raises(BlockKVBackendError, match="overlaps"):
            cache.select(q, ids, 0, G, gates=gates, o_cmp=o_cmp, o_swa=o_swa, out=o_cmp)
    else:
        alias = o_cmp.clone()
        got = cache.select(q, ids, 0, G, gates=gates, o_cmp=alias, o_swa=o_swa, out=alias)
        assert got.data_ptr() == alias.data_ptr() and torch.equal(got, want)
    buf = torch.zeros((1, M + 1, H, D), dtype=torch.bfloat16, device=DEV)
    buf[:, :M] = o_swa
    with pytest.raises(BlockKVBackendError, match="overlaps"):
        cache.select(q, ids, 0, G, gates=gates, o_cmp=o_cmp, o_swa=buf[:, :M], out=buf[:, 1:])
    cache.close()


def test_fp8_quantisation_error_against_bf16_cache():
    """Config 5's error budget, per variant: selection-attention output over
    Student-t(4) K/V against float64 on the original bf16 values, for the bf16 cache, the fp8
    cache with bf16 queries, and the fp8 cache with fp8 queries (qk_fp8).  The fp8 cache errors
    are the quantisation's; the test bounds them and prints them."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(55)
    torch.manual_seed(55)
    H, D, C, P, T, n, G = 4, 128, 4680, 64, 16, 3, 64
    ks = [_chunk(g, C, H, D, 1.0, True) for _ in range(n)]
    vs = [_chunk(g, C, H, D, 1.0, True) for _ in range(n)]
    M = 2048
    q = torch.randn((1, M, H, D), generator=g).to(torch.bfloat16)
    MG = M // G
    ids = torch.stack([torch.randperm(n * -(-C // P), generator=g)[:T] for _ in range(MG * H)])
    ids = ids.view(1, MG, H, T).to(torch.int32)
    ref, _ = O.selection_attention(q.float().numpy(), torch.cat(ks, 1).float().numpy(),
                                   torch.cat(vs, 1).float().numpy(), ids.numpy(), G, D ** -0.5,
                                   O.paged_block_tokens(C, P, n))
    errs = {}
    for name, kw in (("bf16", dict(dtype=torch.bfloat16)), ("fp8", dict(dtype="fp8")),
                     ("fp8_qk", dict(dtype="fp8", qk_fp8=True))):
        cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P,
                             hbm_slots=H * n, host_slots=H * n, window_chunks=0, **kw)
        for cid in range(n):
            cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
        out = cache.select(q.to(DEV), ids.to(DEV), 0, G).float().cpu().numpy()
        d = np.abs(out.astype(np.float64) - ref)
        rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
        errs[name] = (float(d.max()), float(d.mean()), float(rel))
        cache.close()
    print("selection output error vs float64 on bf16 K/V (max-abs, mean-abs, rel-L2):", errs)
    assert errs["bf16"][2] < 5e-3
    assert errs["fp8"][2] < 0.06 and errs["fp8_qk"][2] < 0.08
    assert errs["fp8_qk"][2] >= errs["fp8"][2] * 0.9  # quantising q adds error, not removes it


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
def test_window_attention_reads_pages_in_place(dtype):
    """SWA over the paged cache (window_attention without the dense ring) against float64
    softmax attention over every token of the last 3 chunks: ragged chunks (300 tokens = 4 full
    pages + 44), a window that covers part of the history, and for bf16 the dense-ring path on
    the same data, which must agree with it."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(13)
    H, D, C, P, n, W, M = 2, 128, 300, 64, 5, 3, 200
    fp8 = dtype == "fp8"
    caches = [PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                           window_chunks=W, keep_window_kv=keep)
              for keep in ((False, True) if not fp8 else (False,))]
    ks = [_chunk(g, C, H, D, 0.3, fp8) for _ in range(n)]
    vs = [_chunk(g, C, H, D, 1.0, fp8) for _ in range(n)]
    for cache in caches:
        for cid in range(n):
            cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    with torch.no_grad():
        outs = [c.window_attention(q.to(DEV), 0) for c in caches]
    torch.cuda.synchronize()
    kk, vv = _paged_oracle_inputs(ks, vs, caches[0] if fp8 else None)
    kk, vv = kk[:, (n - W) * C:], vv[:, (n - W) * C:]
    ids = np.broadcast_to(np.arange(W * caches[0].ppc, dtype=np.int32), (1, -(-M // 64), H, W * caches[0].ppc))
    want_o, _ = O.selection_attention(q.float().numpy(), kk, vv, ids, 64, D ** -0.5,
                                      O.paged_block_tokens(C, P, W))
    for out in outs:
        _check_attn(out, None, want_o, None)
    if len(outs) == 2:
        assert (outs[0].float() - outs[1].float()).abs().max().item() <= 1e-2


def test_mmcache_adapters_and_chunk_metadata_feed_the_pointer_path():
    """Reference call sites unchanged: get_chunk_metadata -> selection_attention_padded_ptr_fast
    without a cache (the pointer kernels; reference geometry, 30-token blocks dividing the chunk)
    agrees with the paged kernel and the float64 oracle, including after units move to the host
    pool (mapped addresses); flush_offload / preallocate_offload_buffer / lru_touch_per_head
    exist with the reference's signatures."""
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.padded_ptr import selection_attention_padded_ptr_fast
    g = torch.Generator().manual_seed(17)
    H, D, C, P, G, T, n = 2, 128, 120, 30, 15, 6, 4
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, window_chunks=0,
                         hbm_slots=H * n, host_slots=H * n)
    assert cache.preallocate_offload_buffer(torch.empty(1, C, D), 4) is None
    ks = [_chunk(g, C, H, D, 0.3) for _ in range(n)]
    vs = [_chunk(g, C, H, D, 1.0) for _ in range(n)]
    for cid in range(n):
        cache.update_cache("k_cache", ks[cid].to(DEV), 0, cid * C)
        cache.update_cache("v_cache", vs[cid].to(DEV), 0, cid * C)
    cache.lru_touch_per_head(0, "k_cache", 1, 2)
    M = 90
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(n * cache.ppc, generator=g)[:T] for _ in range(M // G * H)])
    ids = ids.view(1, M // G, H, T).to(torch.int32)
    want_o, want_l = O.selection_attention(q.float().numpy(), *_paged_oracle_inputs(ks, vs),
                                           ids.numpy(), G, D ** -0.5, O.paged_block_tokens(C, P, n))
    qd, idd = q.to(DEV), ids.to(DEV)
    for step in ("hbm", "host"):
        if step == "host":
            cache.evict_all()
        pk, nk, st = cache.get_chunk_metadata(0, "k_cache")
        pv, _, _ = cache.get_chunk_metadata(0, "v_cache")
        assert st["chunk_len"] == C and st["stride_bn"] == D
        with torch.no_grad():
            out, lse = selection_attention_padded_ptr_fast(qd, idd, P, G, C, pk, pv, nk, st,
                                                           return_lse=True)
            ref = cache.select(qd, idd, 0, G)
        _check_attn(out, lse, want_o, want_l)
        assert (out.float() - ref.float()).abs().max().item() <= 1e-2
    cache.flush_offload()


def test_lru_residency_matches_reference_model():
    """lru_max_size per (layer, head), no sink / window: after every flush the HBM-resident
    chunks are exactly the reference LRU's (models/cache.py:673-699, :1032-1142)."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(5)
    L, H, D, C, P, G, T, n, cap = 2, 3, 64, 640, 64, 64, 6, 7, 3
    cache = PagedKVCache(L, H, D, max_chunks=n, chunk_len=C, page_tokens=P, hbm_slots=L * H * n,
                         host_slots=L * H * n, lru_max_size=cap, window_chunks=0,
                         keep_window_kv=False)
    model = ReferenceLRU(L, H, cap)
    ppc = cache.ppc
    rng = np.random.default_rng(5)
    q = torch.randn((1, C, H, D), generator=g).to(torch.bfloat16).to(DEV)
    for cid in range(n):
        for l in range(L):
            k = torch.randn((1, C, H, D), generator=g).to(torch.bfloat16).to(DEV)
            cache.append(l, k, k, cid)
            model.write(l, cid)
            for _ in range(2):
                ids = rng.integers(0, (cid + 1) * ppc, size=(1, C // G, H, T)).astype(np.int32)
                cache.select(q, torch.from_numpy(ids).to(DEV), l, G)
                model.select(l, ids, ppc, n)
        cache.flush(reserve_next_chunk=False)
        model.flush()
        got = {(l, h, c) for l in range(L) for h in range(H) for c in range(cid + 1)
               if cache.where(l, h, c) == "hbm"}
        assert got == model.resident(), f"after chunk {cid}"


def test_budget_flush_keeps_window_and_most_recent():
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(6)
    L, H, D, C, P, n, slots = 1, 2, 64, 256, 64, 8, 10
    cache = PagedKVCache(L, H, D, max_chunks=n, chunk_len=C, page_tokens=P, hbm_slots=slots,
                         window_chunks=2, sink_chunks=1, keep_window_kv=False)
    for cid in range(n):
        k = torch.randn((1, C, H, D), generator=g).to(torch.bfloat16).to(DEV)
        cache.append(0, k, k, cid)
        st = cache.flush()
        resident = [(h, c) for h in range(H) for c in range(cid + 1) if cache.where(0, h, c) == "hbm"]
        assert len(resident) + H <= slots  # the next chunk's slots are reserved
        for h in range(H):
            assert cache.where(0, h, 0) == "hbm"                   # sink
            for c in range(max(0, cid - 1), cid + 1):
                assert cache.where(0, h, c) == "hbm"               # window
        assert st["evicted_units"] >= 0
    assert cache.stats["evicted_units"] > 0


# ------------------------------------------------------------------ K1 / K2 / K3
def test_block_kv_warmup_known_answers():
    from omnimem_amd import block_kv_ops
    assert block_kv_ops.warmup(DEV) > 0


def test_dedup_matches_numpy_unique():
    from omnimem_amd.block_kv_ops import DeviceBlockDedup
    rng = np.random.default_rng(8)
    H, T, bpc, n_chunks = 12, 16, 74, 80
    mb = bpc * n_chunks
    ids = rng.integers(-1, mb + 5, size=(1, 74, H, T)).astype(np.int32)
    dd = DeviceBlockDedup(H, mb, T, cap=20000, device=DEV, blocks_per_chunk=bpc)
    for rep in range(2):
        keys, n, overflow = dd.unique_keys(torch.from_numpy(ids).to(DEV))
        want = set()
        for (b, g, h, t), bid in np.ndenumerate(ids):
            if 0 <= bid < mb:
                cid, loc = divmod(int(bid), bpc)
                want.add((cid * H + h) * bpc + loc)
        assert n == len(want) and not overflow
        np.testing.assert_array_equal(np.asarray(keys), np.array(sorted(want), np.int32))
        ids = rng.integers(-1, mb, size=ids.shape).astype(np.int32)
    small = DeviceBlockDedup(H, mb, T, cap=10, device=DEV, blocks_per_chunk=bpc)
    keys, n, overflow = small.unique_keys(torch.from_numpy(ids).to(DEV))
    assert overflow and n > 10 and len(keys) == 10


def test_gather_publish_clear_and_block_range():
    from omnimem_amd.block_kv_ops import (clear_block_range, gather_publish_clear,
                                          register_block_range, table_entry_addresses)
    g = torch.Generator().manual_seed(9)
    BT, D = 64, 128
    src = torch.randn((3, BT, D), generator=g).to(torch.bfloat16).pin_memory()  # host sources
    src_v = torch.randn((3, BT, D), generator=g).to(torch.bfloat16).pin_memory()
    dst = torch.zeros((3, BT, D), dtype=torch.bfloat16, device=DEV)
    dst_v = torch.zeros_like(dst)
    table = torch.full((2, 1, 8), 7, dtype=torch.int64, device=DEV)
    pub_k = table_entry_addresses(table, 0, [0, 1, 2])
    pub_v = table_entry_addresses(table, 1, [0, 1, 2])
    clear = table_entry_addresses(table, 0, [5, 6])
    desc = torch.tensor([src[i].data_ptr() for i in range(3)] + [src_v[i].data_ptr() for i in range(3)]
                        + [dst[i].data_ptr() for i in range(3)] + [dst_v[i].data_ptr() for i in range(3)]
                        + list(pub_k) + list(pub_v) + list(clear), dtype=torch.int64, device=DEV)
    assert gather_publish_clear(desc, 3, 2, BT, D, dst) == 4
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), src) and torch.equal(dst_v.cpu(), src_v)
    t = table.cpu()
    assert t[0, 0, :3].tolist() == [dst[i].data_ptr() for i in range(3)]
    assert t[1, 0, :3].tolist() == [dst_v[i].data_ptr() for i in range(3)]
    assert t[0, 0, 5:7].tolist() == [0, 0] and t[0, 0, 7].item() == 7
    tab = torch.zeros((2, 3, 10), dtype=torch.int64, device=DEV)
    nv = torch.zeros(3, dtype=torch.int32, device=DEV)
    register_block_range(tab, nv, 2, 5, 1 << 30, 1 << 31, 4096, 64, 7)
    t = tab.cpu()
    for h in range(3):
        assert t[0, h, 2:7].tolist() == [(1 << 30) + h * 4096 + j * 64 for j in range(5)]
        assert t[1, h, 2:7].tolist() == [(1 << 31) + h * 4096 + j * 64 for j in range(5)]
        assert t[:, h, :2].abs().sum() == 0 and t[:, h, 7:].abs().sum() == 0
    assert nv.tolist() == [7, 7, 7]
    clear_block_range(tab, nv, 3, 2, -1, which="k")
    t = tab.cpu()
    assert t[0, :, 3:5].abs().sum() == 0 and t[1, :, 3:5].abs().sum() > 0 and nv.tolist() == [7] * 3


def test_block_store_entry_uses_paged_cache():
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.padded_ptr import selection_attention_block_store, selection_attention_paged
    g = torch.Generator().manual_seed(12)
    H, D, C, P = 2, 128, 1024, 64
    cache = PagedKVCache(1, H, D, max_chunks=2, chunk_len=C, page_tokens=P, window_chunks=0)
    for cid in range(2):
        k = torch.randn((1, C, H, D), generator=g).to(torch.bfloat16).to(DEV)
        cache.append(0, k, k, cid)
    q = torch.randn((1, 128, H, D), generator=g).to(torch.bfloat16).to(DEV)
    ids = torch.randint(0, 32, (1, 2, H, 4), generator=g).to(torch.int32).to(DEV)
    with torch.no_grad():
        a = selection_attention_block_store(q, ids, P, 64, cache, 0)
        b = selection_attention_paged(q, ids, P, 64, cache, 0)
    assert torch.equal(a, b)
    with pytest.raises(RuntimeError):
        selection_attention_block_store(q, ids, P, 64, cache, 0)  # grad enabled


@pytest.mark.parametrize("dtype,stage_slots", [(torch.bfloat16, 8192), (torch.bfloat16, 5),
                                               ("fp8", 8192), ("fp8", 5)])
def test_prefetch_staging_is_bit_identical(dtype, stage_slots):
    """Selection with the host-resident pages staged into HBM first (prefetch on a side stream,
    omm_paged_stage) gives exactly the output and LSE of reading them in place over the host
    link, also when the staging pool holds fewer pages than the call lists (the rest are read in
    place); both match the float64 oracle.  The map must have staged host pages only, each
    distinct page once."""
    from omnimem_amd.backend import BlockKVBackendError
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(91)
    H, D, C, P, T, n, G, M = 3, 128, 1000, 64, 8, 4, 64, 700
    fp8 = dtype == "fp8"
    cache = PagedKVCache(1, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         hbm_slots=H * 2, host_slots=H * n, window_chunks=0,
                         stage_slots=stage_slots)
    ks = [_chunk(g, C, H, D, 0.3, fp8) for _ in range(n)]
    vs = [_chunk(g, C, H, D, 1.0, fp8) for _ in range(n)]
    for cid in range(n):
        cache.append(0, ks[cid].to(DEV), vs[cid].to(DEV), cid)
        cache.flush()
    host = [(h, c) for h in range(H) for c in range(n) if cache.where(0, h, c) == "host"]
    assert host, "no unit moved to the host pool"
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    MG = -(-M // G)
    ids = torch.stack([torch.randperm(n * cache.ppc, generator=g)[:T] for _ in range(MG * H)])
    ids = ids.view(1, MG, H, T).to(torch.int32).to(DEV)
    plain, plain_l = cache.select(q, ids, 0, G, return_lse=True)
    handle = cache.prefetch(ids, 0)
    assert handle["event"] is not None
    staged, staged_l = cache.select(q, ids, 0, G, return_lse=True, prefetch=handle)
    torch.cuda.synchronize()
    assert torch.equal(plain, staged) and torch.equal(plain_l, staged_l)
    # the map: every host page listed is stamped with the call's epoch, once, within the pool
    ep = cache._stage_epoch.cpu().numpy()
    sl = cache._stage_slot.cpu().numpy()
    want = set()
    for (_, gg, h, t), bid in np.ndenumerate(ids.cpu().numpy()):
        c, p = divmod(int(bid), cache.ppc)
        if cache.where(0, h, c) == "host":
            want.add((h, c, p))
    got = {tuple(x) for x in np.argwhere(ep == handle["epoch"])}
    assert got == want
    slots = sorted(int(sl[x]) for x in got if sl[x] >= 0)
    assert len(slots) == min(len(want), stage_slots)
    assert slots == list(range(len(slots)))          # each slot used once
    assert int(cache._stage_counter.item()) == len(want)
    # and against the float64 oracle
    if fp8:
        kk, vv = _fp8_cache_images(cache, n)
    else:
        kk, vv = torch.cat(ks, 1).float().numpy(), torch.cat(vs, 1).float().numpy()
    want_o, want_l = O.selection_attention(q.float().cpu().numpy(), kk, vv, ids.cpu().numpy(),
                                           G, D ** -0.5, O.paged_block_tokens(C, P, n))
    _check_attn(staged, staged_l, want_o, want_l)
    # one prefetch outstanding at a time, consumed by the matching select only
    h2 = cache.prefetch(ids, 0)
    with pytest.raises(BlockKVBackendError):
        cache.prefetch(ids, 0)
    with pytest.raises(BlockKVBackendError):
        cache.select(q, ids.clone(), 0, G, prefetch=h2)
    cache.close()


def _slots_balance(cache):
    """Every HBM / host slot is in the table, held by a snapshot, or free, exactly once."""
    held = [s for sn in cache._snaps for s in sn["units"].values() if s is not None]
    t = cache._table_h
    hbm = sorted(t[t >= 0].tolist() + [s for s in held if s >= 0] + list(cache._free_hbm))
    host = sorted((-2 - t[t <= -2]).tolist() + [-2 - s for s in held if s <= -2]
                  + list(cache._free_host))
    assert hbm == list(range(cache.n_slots))
    assert host == list(range(cache.n_host))


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
def test_snapshot_restore_chunks(dtype):
    """Prompt-switch snapshots (pipeline_wan_causal.py:33-57, 369-396): chunks [1, 3) are
    snapshotted, a flush may move them, they are rewritten (new slots, copy on write) and read
    back as the new data; restore_chunks brings back every byte, scale and pooled row of the old
    version while later chunks keep their new data; discard_snapshot keeps the new data; slots
    stay balanced throughout, overlapping snapshots are refused, and the restored cache's
    selection matches the float64 oracle on the old values."""
    from omnimem_amd.backend import BlockKVBackendError
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(61)
    L, H, D, C, P, n = 2, 2, 128, 500, 64, 6
    fp8 = dtype == "fp8"
    # the host pool has room for every unit: slots a snapshot holds are spare capacity
    cache = PagedKVCache(L, H, D, max_chunks=n, chunk_len=C, page_tokens=P, dtype=dtype,
                         hbm_slots=L * H * 3, host_slots=L * H * n, window_chunks=1,
                         keep_window_kv=fp8)
    data = {}
    def write(l, c, tag):
        k = _chunk(g, C, H, D, 0.3, fp8)
        v = _chunk(g, C, H, D, 1.0, fp8)
        data[(l, c, tag)] = (k, v)
        cache.append(l, k.to(DEV), v.to(DEV), c)
    for c in range(5):
        for l in range(L):
            write(l, c, "old")
        cache.flush()
    assert any(cache.where(l, h, c) == "host" for l in range(L) for h in range(H) for c in range(5))
    units = lambda lo, hi: {(l, h, c): cache.read_unit(l, h, c) for l in range(L)
                            for h in range(H) for c in range(lo, hi)}
    same = lambda a, b: all(torch.equal(x, y) for x, y in zip(a, b))
    before = units(0, 5)
    pooled = [(cache.k_cmp[l].clone(), cache.v_cmp[l].clone()) for l in range(L)]
    snap = cache.snapshot_chunks(1, 3)
    with pytest.raises(BlockKVBackendError, match="overlap"):
        cache.snapshot_chunks(2, 4)
    cache.flush()                      # may move the snapshotted units before their rewrite
    _slots_balance(cache)
    for c in (1, 2):
        for l in range(L):
            write(l, c, "new")
    for l in range(L):
        write(l, 5, "new")
    cache.flush()
    _slots_balance(cache)
    after = units(0, 6)
    for (l, h, c), parts in after.items():
        if c in (1, 2):
            assert not same(parts, before[(l, h, c)]), "rewrite did not take effect"
        elif c < 5:
            assert same(parts, before[(l, h, c)])
    cache.restore_chunks(snap, 1)
    _slots_balance(cache)
    with pytest.raises(BlockKVBackendError):
        cache.restore_chunks(snap, 1)
    restored = units(0, 6)
    for (l, h, c), parts in restored.items():
        assert same(parts, before[(l, h, c)] if c < 5 else after[(l, h, c)]), (l, h, c)
    for l in range(L):
        rows = slice(0, 5 * cache.ppc)
        assert torch.equal(cache.k_cmp[l][:, rows], pooled[l][0][:, rows])
        assert torch.equal(cache.v_cmp[l][:, rows], pooled[l][1][:, rows])
    # selection over the restored layer 0 against float64 on the old values of chunks 0..4
    M, G, T = 300, 64, 6
    q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(5 * cache.ppc, generator=g)[:T]
                       for _ in range(-(-M // G) * H)]).view(1, -1, H, T).to(torch.int32)
    got, lse = cache.select(q.to(DEV), ids.to(DEV), 0, G, return_lse=True)
    if fp8:
        kk = np.zeros((1, 5 * C, H, D), np.float32)
        vv = np.zeros_like(kk)
        for c in range(5):
            for h in range(H):
                kc, vc, sk, sv = restored[(0, h, c)]
                kk[0, c * C:(c + 1) * C, h] = O.dequantize_pages(
                    kc.numpy(), sk.numpy()[:, None, None]).reshape(-1, D)[:C]
                vv[0, c * C:(c + 1) * C, h] = O.dequantize_pages(
                    vc.numpy(), sv.numpy()[:, None, None]).reshape(-1, D)[:C]
    else:
        kk = torch.cat([data[(0, c, "old")][0] for c in range(5)], 1).float().numpy()
        vv = torch.cat([data[(0, c, "old")][1] for c in range(5)], 1).float().numpy()
    want_o, want_l = O.selection_attention(q.float().numpy(), kk, vv, ids.numpy(), G, D ** -0.5,
                                           O.paged_block_tokens(C, P, 5))
    _check_attn(got, lse, want_o, want_l)
    # discard: the rewrite stays, the old slots are freed
    snap2 = cache.snapshot_chunks(3, 5)
    for l in range(L):
        write(l, 3, "newer")
    cache.discard_snapshot(snap2)
    _slots_balance(cache)
    for l in range(L):
        for h in range(H):
            assert not same(cache.read_unit(l, h, 3), before[(l, h, 3)])
    cache.close()


@pytest.mark.parametrize("dtype", [torch.bfloat16, "fp8"])
def test_async_flush_matches_resident_cache(dtype):
    """Asynchronous flush (byte budget): a flush enqueues its moves on the move stream and the
    next flush commits them.  Selections before and after each commit return exactly what an
    all-HBM cache returns, ``read_unit`` reads the pool serving the unit, slots balance once
    committed, and an append that rewrites a chunk still moving commits first and lands."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(71)
    L, H, D, C, P, n, W, G, T, M = 2, 2, 128, 500, 64, 9, 1, 64, 6, 200
    fp8 = dtype == "fp8"
    mk = lambda slots: PagedKVCache(L, H, D, max_chunks=n, chunk_len=C, page_tokens=P,
                                    dtype=dtype, hbm_slots=slots, window_chunks=W,
                                    keep_window_kv=False)
    full, small = mk(L * H * n), mk(L * H * 5)
    assert small._async_ok()
    rng = np.random.default_rng(7)

    def write(l, c):
        k, v = _chunk(g, C, H, D, 0.3, fp8).to(DEV), _chunk(g, C, H, D, 1.0, fp8).to(DEV)
        full.append(l, k, v, c)
        small.append(l, k, v, c)

    def compare(cid):
        for l in range(L):
            q = (torch.randn((1, M, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
            ids = rng.integers(0, (cid + 1) * small.ppc, size=(1, -(-M // G), H, T))
            ids = torch.from_numpy(ids.astype(np.int32)).to(DEV)
            a, la = full.select(q, ids, l, G, return_lse=True)
            b, lb = small.select(q, ids, l, G, return_lse=True)
            torch.cuda.synchronize()
            assert torch.equal(a, b) and torch.equal(la, lb), (cid, l)

    pending = 0
    for cid in range(n - 1):
        for l in range(L):
            write(l, cid)
        compare(cid)
        full.flush()
        st = small.flush()
        if st["evicted_units"] or st["promoted_units"]:
            assert small._moves is not None
            pending += 1
            moving = sorted(u for u, _, _ in small._moves[1])
            for (l, h, c) in moving[:2]:    # served by the source slot until committed
                same = zip(full.read_unit(l, h, c), small.read_unit(l, h, c))
                assert all(torch.equal(x, y) for x, y in same), (l, h, c)
        compare(cid)
    assert pending > 0 and small.stats["evicted_units"] > 0
    assert any(small.where(l, h, c) == "host" for l in range(L) for h in range(H)
               for c in range(n))
    # rewrite a chunk whose units are still moving: the append commits the moves first
    assert small._moves is not None
    (l, _, c), _, _ = small._moves[1][0]
    k, v = _chunk(g, C, H, D, 0.3, fp8).to(DEV), _chunk(g, C, H, D, 1.0, fp8).to(DEV)
    full.append(l, k, v, c)
    small.append(l, k, v, c)
    assert small._moves is None
    compare(n - 2)
    _slots_balance(small)
    for l, h, c in [(a, b, x) for a in range(L) for b in range(H) for x in range(n - 1)]:
        same = zip(full.read_unit(l, h, c), small.read_unit(l, h, c))
        assert all(torch.equal(x, y) for x, y in same), (l, h, c)
    full.close()
    small.close()


def test_async_flush_pending_moves_with_snapshots_reset_and_evict_all():
    """Operations that meet an asynchronous flush's pending moves commit them first: a snapshot
    taken while units are moving, its restore after further flushes, evict_all, and reset; the
    bytes read back stay those written, and slots balance after each step."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(83)
    L, H, D, C, P, n, W = 2, 2, 128, 500, 64, 9, 1
    cache = PagedKVCache(L, H, D, max_chunks=n, chunk_len=C, page_tokens=P, hbm_slots=L * H * 5,
                         host_slots=L * H * n, window_chunks=W, keep_window_kv=False)
    assert cache._async_ok()
    data = {}

    def write(l, c):
        k, v = _chunk(g, C, H, D, 0.3), _chunk(g, C, H, D, 1.0)
        data[(l, c)] = (k, v)
        cache.append(l, k.to(DEV), v.to(DEV), c)

    def check(upto):
        for l in range(L):
            for c in range(upto):
                k, v = data[(l, c)]
                for h in range(H):
                    uk, uv = cache.read_unit(l, h, c)[:2]
                    want_k = _pages(k[0, :, h].float().numpy(), C, P)
                    want_v = _pages(v[0, :, h].float().numpy(), C, P)
                    assert np.array_equal(uk.float().numpy().reshape(want_k.shape), want_k), (l, h, c)
                    assert np.array_equal(uv.float().numpy().reshape(want_v.shape), want_v), (l, h, c)

    for c in range(6):
        for l in range(L):
            write(l, c)
        cache.flush()
    assert cache._moves is not None            # this flush's evictions are still pending
    snap = cache.snapshot_chunks(1, 3)         # commits them first
    assert cache._moves is None
    _slots_balance(cache)
    old = {key: data[key] for key in data if key[1] in (1, 2)}
    for c in (1, 2):                           # rewrite the snapshotted chunks
        for l in range(L):
            write(l, c)
    for l in range(L):
        write(l, 6)
    cache.flush()
    assert cache._moves is not None
    cache.restore_chunks(snap, 1)              # commits, then restores
    assert cache._moves is None
    data.update(old)
    _slots_balance(cache)
    check(7)
    cache.flush()
    cache.evict_all()                          # commits, then moves everything to the host
    assert cache._moves is None
    assert all(cache.where(l, h, c) == "host" for l in range(L) for h in range(H) for c in range(7))
    _slots_balance(cache)
    check(7)
    for l in range(L):
        write(l, 7)
    cache.flush()
    cache.reset()                              # waits for any copies in flight, forgets all
    assert cache._moves is None and all(nc == 0 for nc in cache.n_chunks)
    _slots_balance(cache)
    cache.close()
