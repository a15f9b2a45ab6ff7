"""The reference's AR self-attention call sequence runs unchanged against ``MMCache`` (the paged
cache behind the reference constructor), and every value it returns is checked against the
oracle.

The sequence is restated from models/transformers/causal_wan_nsa_model.py:461-511 (the AR branch,
``block_mask is None``) and :182-239 (``slc_attention_padded_ptr``); the cache is built with the
keyword arguments of pipelines/pipeline_wan_causal.py:235-316.  Geometry: the reference's own
30-token blocks and 15-query groups, 240-token chunks, a 2-chunk window with one sink chunk and
an LRU of 2 chunks per head, so units move to the host pool and the selection reads them there.
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O
from _topk_checks import check_mfma_topk

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, D, S, BS, G, TOPK, WIN, SINK, EXW = 2, 128, 240, 30, 15, 4, 2, 1, 2


def _attention(q, k, v):
    """The model's ``attention`` (flash attention in the reference): full softmax attention."""
    from omnimem_amd.selection import dense_attention
    return dense_attention(q, k, v)


def _ar_layer(kv_cache, q, k, v, layer_idx, start_id, num_selected_blocks):
    """causal_wan_nsa_model.py:471-511 and :182-239, restated (no gates, no projections)."""
    from omnimem_amd.index_topk import parallel_nsa_topk_grouped_heads
    from omnimem_amd.padded_ptr import selection_attention_padded_ptr_fast
    b, s, n, d = q.shape
    q_chunk_offset = start_id // s
    roped_key_cmp = kv_cache.update_cache(
        name='k_cmp_cache', hidden_state=k.view(b, s // BS, BS, n, d).mean(2),
        layer_idx=layer_idx, start_id=start_id // BS)
    v_cmp = kv_cache.update_cache(
        name='v_cmp_cache', hidden_state=v.view(b, s // BS, BS, n, d).mean(2),
        layer_idx=layer_idx, start_id=start_id // BS)
    roped_key_swa = kv_cache.update_cache(name='k_cache', hidden_state=k, layer_idx=layer_idx,
                                          start_id=start_id)
    v_swa = kv_cache.update_cache(name='v_cache', hidden_state=v, layer_idx=layer_idx,
                                  start_id=start_id)
    o_cmp = _attention(q, roped_key_cmp, v_cmp)
    o_swa = _attention(q, roped_key_swa, v_swa)
    # slc_attention_padded_ptr: with progressive_exclude=True the reference skips the
    # should_use_selection_attention gate and always selects
    block_indices = parallel_nsa_topk_grouped_heads(
        q=q, k=roped_key_cmp, num_kv_head_groups=n, block_counts=num_selected_blocks,
        block_size=BS, chunk_size=s, causal=False, group_size=G, exclude_window_chunks=EXW,
        exclude_sink_chunks=0, progressive_exclude=True,
        q_chunk_offset=q_chunk_offset).to(torch.int32).contiguous()
    ptrs_k, n_chunks_k, strides = kv_cache.get_chunk_metadata(layer_idx, 'k_cache')
    ptrs_v, _, _ = kv_cache.get_chunk_metadata(layer_idx, 'v_cache')
    o_slc = selection_attention_padded_ptr_fast(
        q=q, block_indices=block_indices, block_size=BS, group_size=G,
        chunk_len=strides['chunk_len'], chunk_base_ptrs_k=ptrs_k, chunk_base_ptrs_v=ptrs_v,
        n_chunks_per_head=n_chunks_k, chunk_strides=strides,
        verify_complete=kv_cache._has_cpu_chunks, kv_cache=kv_cache, layer_idx=layer_idx)
    return roped_key_cmp, v_cmp, roped_key_swa, v_swa, o_cmp, o_swa, o_slc, block_indices


def _make_cache(n_chunks, lru_max_size=2):
    from omnimem_amd.block_cache import MMCache
    total = n_chunks * S
    shape, cshape = (1, total, H, D), (1, total // BS, H, D)
    kwargs = dict(
        config=dict(cache_type=["k_cache", "v_cache", "k_cmp_cache", "v_cmp_cache"],
                    k_cache={}, v_cache={}, k_cmp_cache={}, v_cmp_cache={}),
        seq_dim=1,
        available_shape=dict(k_cache=shape, v_cache=shape, k_cmp_cache=cshape,
                             v_cmp_cache=cshape),
        device=DEV, dtype=torch.bfloat16,
        block_seqlen_config=dict(k_cache=S, v_cache=S, k_cmp_cache=S // BS, v_cmp_cache=S // BS),
        window_config=dict(k_cache=WIN, v_cache=WIN, k_cmp_cache=None, v_cmp_cache=None),
        sink_config=dict(k_cache=SINK, v_cache=SINK, k_cmp_cache=None, v_cmp_cache=None),
        num_layers=1, per_head_types=None, chunk_per_head_types={'k_cache', 'v_cache'},
        num_heads=H, kv_block_size=BS)
    return MMCache(**kwargs, lru_max_size=lru_max_size)


def _tol(got, want, mx=2e-2, mean=1e-3, what=""):
    err = np.abs(got.float().cpu().numpy().astype(np.float64) - want)
    assert err.max() <= mx, f"{what}: max-abs {err.max():.3e}"
    assert err.mean() <= mean, f"{what}: mean-abs {err.mean():.3e}"


def _dense_ref(q, k, v):
    """float64 softmax attention of q over all of k / v ([1, M, H, D])."""
    q, k, v = (x.float().cpu().numpy().astype(np.float64) for x in (q, k, v))
    s = np.einsum("bmhd,bnhd->bhmn", q, k) * D ** -0.5
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhmn,bnhd->bmhd", p, v)


def test_reference_ar_sequence_against_mmcache():
    n_chunks = 7
    cache = _make_cache(n_chunks)
    g = torch.Generator().manual_seed(21)
    ks, vs, kc = [], [], []
    saw_host = False
    for cid in range(n_chunks):
        k = (torch.randn((1, S, H, D), generator=g) * 0.3).to(torch.bfloat16)
        v = torch.randn((1, S, H, D), generator=g).to(torch.bfloat16)
        ks.append(k)
        vs.append(v)
        for fwd in range(2):  # the AR loop rewrites a chunk on every denoise forward
            q = (torch.randn((1, S, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
            with torch.no_grad():
                (k_cmp, v_cmp, k_swa, v_swa, o_cmp, o_swa, o_slc,
                 ids) = _ar_layer(cache, q, k.to(DEV), v.to(DEV), 0, cid * S, TOPK)
            # pooled history = the caller's pooled chunks, all of them (kv_cmp has no window)
            kpool = k.to(DEV).view(1, S // BS, BS, H, D).mean(2).cpu()
            if fwd == 0:
                kc.append(kpool)
            want_kc = torch.cat(kc, 1)
            assert torch.equal(k_cmp.cpu(), want_kc)
            assert v_cmp.shape == want_kc.shape
            # window = sink chunk 0 + the last WIN chunks, ascending
            keep = sorted(set(range(min(SINK, cid + 1))) |
                          set(range(max(SINK, cid + 1 - WIN), cid + 1)))
            assert torch.equal(k_swa.cpu(), torch.cat([ks[c] for c in keep], 1))
            assert torch.equal(v_swa.cpu(), torch.cat([vs[c] for c in keep], 1))
            _tol(o_cmp, _dense_ref(q, k_cmp, v_cmp), what="o_cmp")
            _tol(o_swa, _dense_ref(q, k_swa, v_swa), what="o_swa")
            # top-k: the oracle's selection rule on the kernel's scores of the same inputs
            mask = O.Mask(block_size=BS, group_size=G, chunk_q=S, chunk_k=S,
                          q_chunk_offset=cid, ex_win=EXW, causal=0, prog_excl=1)
            check_mfma_topk(q, k_cmp, TOPK, mask, D ** -0.5, G, got=ids.cpu().numpy(),
                            block_size=BS, chunk_size=S, causal=False, exclude_window_chunks=EXW,
                            progressive_exclude=True, q_chunk_offset=cid)
            k_all = torch.cat(ks, 1).float().numpy()
            v_all = torch.cat(vs, 1).float().numpy()
            want_o, _ = O.selection_attention(q.float().cpu().numpy(), k_all, v_all,
                                              ids.cpu().numpy(), G, D ** -0.5,
                                              O.paged_block_tokens(S, BS, cid + 1))
            _tol(o_slc, want_o, what=f"o_slc chunk {cid}")
        cache.flush_offload()
        saw_host = saw_host or cache._has_cpu_chunks
    assert saw_host, "the LRU never moved a unit to the host pool"
    assert cache.block_seqlens["k_cmp_cache"] == S // BS


def test_pipeline_chunk_protocol_and_lru_hit_rate():
    """The pipeline's per-chunk cache protocol (pipeline_wan_causal.py:300-306, 404-406, 420-475)
    and the model's entry checks (causal_wan_nsa_model.py:783-784) run against ``MMCache``:
    ``reset``; per chunk ``lru_reset_stats``, then forwards (a denoise and the context forward),
    each asserting ``available_type`` and running the layer's four ``update_cache`` calls and
    the selection, then ``flush_offload`` and ``lru_hit_rate_overall``.  The hit rate must be
    the reference's (models/cache.py:673-716): per selection call, each distinct (head, chunk)
    unit it reads is one access, a hit when that unit is resident on the GPU; counted here from
    the call's block ids and the cache's residency at the time of the call."""
    n_chunks = 7
    cache = _make_cache(n_chunks)
    cache.reset()
    g = torch.Generator().manual_seed(33)
    ppc = S // BS
    saw_miss = False
    for cid in range(n_chunks):
        cache.lru_reset_stats()
        assert cache.lru_hit_rate_overall() == 0.0
        hits = total = 0
        k = (torch.randn((1, S, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
        v = torch.randn((1, S, H, D), generator=g).to(torch.bfloat16).to(DEV)
        for fwd in range(2):
            assert 'k_cmp_cache' in cache.available_type
            assert 'v_cmp_cache' in cache.available_type
            q = (torch.randn((1, S, H, D), generator=g) * 0.3).to(torch.bfloat16).to(DEV)
            with torch.no_grad():
                ids = _ar_layer(cache, q, k, v, 0, cid * S, TOPK)[-1]
            units = {(h, int(b) // ppc) for (_, _, h, _), b in np.ndenumerate(ids.cpu().numpy())
                     if b >= 0 and int(b) // ppc <= cid}
            for h, c in units:
                where = cache.where(0, h, c)
                assert where in ("hbm", "host")
                hits += where == "hbm"
                saw_miss = saw_miss or where == "host"
            total += len(units)
            # accesses not yet flushed are already counted
            want = hits / total if total else 0.0
            assert abs(cache.lru_hit_rate_overall() - want) < 1e-12
        cache.flush_offload()
        want = hits / total if total else 0.0
        assert abs(cache.lru_hit_rate_overall() - want) < 1e-12, (cid, hits, total)
    assert saw_miss, "no selection read a host-resident unit"
    # the model-level checks reject a cache without the pooled names only through the assert;
    # the adapter adds them even when config['cache_type'] omits them
    from omnimem_amd.block_cache import MMCache
    c2 = MMCache(config=dict(cache_type=["k_cache", "v_cache"]), seq_dim=1,
                 available_shape=dict(k_cache=(1, 480, 2, 128)), device=DEV,
                 block_seqlen_config=dict(k_cache=240), num_layers=1, num_heads=2,
                 kv_block_size=30)
    assert c2.available_type[:2] == ["k_cache", "v_cache"]
    assert {"k_cmp_cache", "v_cmp_cache"} <= set(c2.available_type)
    c2.close()
    cache.close()


def test_mmcache_constructor_rejections():
    from omnimem_amd.backend import BlockKVBackendError
    from omnimem_amd.block_cache import MMCache
    base = dict(config=dict(cache_type=["k_cache", "v_cache"]), seq_dim=1,
                available_shape=dict(k_cache=(1, 480, 2, 128)), device=DEV,
                block_seqlen_config=dict(k_cache=240), num_layers=1, num_heads=2,
                kv_block_size=30)
    MMCache(**base)
    with pytest.raises(BlockKVBackendError):
        MMCache(**{**base, "seq_dim": 2})
    with pytest.raises(BlockKVBackendError):
        MMCache(**{**base, "available_shape": dict(k_cache=(2, 480, 2, 128))})
    with pytest.raises(BlockKVBackendError):
        MMCache(**{**base, "block_seqlen_config": dict(k_cache=240, k_cmp_cache=7)})
    with pytest.raises(BlockKVBackendError):
        MMCache(**{**base, "config": dict(cache_type=["k_cache"])})


def test_update_cache_window_without_sinks_and_fp8_ring():
    """window 2 / no sink on a bf16 cache read from pages, and an fp8 cache whose window comes
    from its bf16 ring: update_cache returns the window chunks ascending in both."""
    from omnimem_amd.block_cache import PagedKVCache
    g = torch.Generator().manual_seed(3)
    for dtype, ring in ((torch.bfloat16, False), ("fp8", True)):
        cache = PagedKVCache(1, H, D, max_chunks=5, chunk_len=S, page_tokens=BS, dtype=dtype,
                             window_chunks=2, keep_window_kv=ring)
        ks = []
        for cid in range(5):
            k = torch.randn((1, S, H, D), generator=g).to(torch.bfloat16)
            ks.append(k)
            got_k = cache.update_cache("k_cache", k.to(DEV), 0, cid * S)
            got_v = cache.update_cache("v_cache", k.to(DEV), 0, cid * S)
            want = torch.cat(ks[max(0, cid - 1):cid + 1], 1)
            assert torch.equal(got_k.cpu(), want) and torch.equal(got_v.cpu(), want)
