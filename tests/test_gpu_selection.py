"""GPU parity of dense selection attention against the float64 oracle.

Tolerances (BASELINE): bf16/f16 max-abs 2e-2 and mean-abs 1e-3; fp32 1e-4.  Cases cover the
reference's edge rules (cuda_backend/csrc/common.cuh:158-190, :327-332; selection_fwd.cu:1-3):
partial last blocks, chunk-causal prefixes, -1 and out-of-range ids, duplicate ids (counted
twice), groups larger than 64, blocks longer than 64 tokens, the reference's own shape
(30-token blocks, groups of 15) and BASELINE configs 1 and 3.
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.bfloat16: (2e-2, 1e-3), torch.float16: (2e-2, 1e-3), torch.float32: (1e-4, 1e-5)}


def _ids(gen, B, MG, H, T, nblocks, minus=0.0, dup=False):
    ids = torch.empty((B, MG, H, T), dtype=torch.int32)
    for b in range(B):
        for g in range(MG):
            for h in range(H):
                ids[b, g, h] = torch.randperm(max(nblocks, T), generator=gen)[:T].to(torch.int32)
    if minus:
        ids[torch.rand(ids.shape, generator=gen) < minus] = -1
    if dup:
        ids[..., 1] = ids[..., 0]
    return ids


def _check(out, lse, want_o, want_l, dtype, rows=None):
    o = out.float().cpu().numpy().astype(np.float64)
    l = lse.cpu().numpy().astype(np.float64)
    if rows is not None:
        o, want_o = o[:, rows], want_o[:, rows]
        l, want_l = l[:, :, rows], want_l[:, :, rows]
    mx, mean = TOL[dtype]
    err = np.abs(o - want_o)
    assert err.max() <= mx, f"max-abs {err.max():.3e} > {mx}"
    assert err.mean() <= mean, f"mean-abs {err.mean():.3e} > {mean}"
    both_inf = np.isneginf(l) & np.isneginf(want_l)
    assert np.array_equal(np.isneginf(l), np.isneginf(want_l))
    if (~both_inf).any():
        assert np.abs(l[~both_inf] - want_l[~both_inf]).max() <= 1e-3


CASES = [
    # M, N, H, D, G, BS, T, causal, chunk, minus, dup
    (256, 512, 2, 128, 64, 64, 4, False, 1, 0.0, False),
    (300, 700, 3, 128, 15, 30, 8, True, 600, 0.1, False),
    (200, 333, 2, 128, 100, 100, 3, True, 150, 0.0, False),
    (64, 256, 2, 128, 1, 64, 2, False, 1, 0.0, False),
    (130, 256, 2, 64, 64, 32, 5, False, 1, 0.2, True),
    (90, 180, 1, 96, 30, 16, 6, True, 60, 0.0, False),
    (128, 64, 1, 128, 64, 64, 3, False, 1, 1.0, False),  # every id -1: O = 0, lse = -inf
    # groups of more than 64 queries: 4-wave workgroups covering two 64-query subgroups (the
    # second workgroup of a 192-query group has one empty subgroup)
    (400, 512, 2, 128, 192, 64, 5, True, 256, 0.1, False),
    (300, 384, 2, 64, 128, 64, 4, False, 1, 0.0, True),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", CASES)
def test_sel_fwd_matches_oracle(dtype, case):
    from omnimem_amd.selection import sel_fwd
    M, N, H, D, G, BS, T, causal, chunk, minus, dup = case
    gen = torch.Generator().manual_seed(M * 31 + N + G)
    q = (torch.randn((1, M, H, D), generator=gen) * D ** -0.25).to(dtype)
    k = (torch.randn((1, N, H, D), generator=gen) * D ** -0.25).to(dtype)
    v = torch.randn((1, N, H, D), generator=gen).to(dtype)
    MG = -(-M // G)
    nb = -(-N // BS)
    ids = _ids(gen, 1, MG, H, T, nb + 2, minus, dup)  # a few ids past the end too
    out, lse = sel_fwd(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), BS, chunk, D ** -0.5, causal, G)
    want_o, want_l = O.selection_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                           ids.numpy(), G, D ** -0.5,
                                           O.dense_block_tokens(N, BS, chunk, causal),
                                           chunk_size=chunk, causal=causal)
    _check(out, lse, want_o, want_l, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("scale", [-0.09, 0.0, 8.0])
def test_sel_fwd_scale_values(scale, dtype):
    """A negative scale (the MFMA paths negate Q), a zero scale (uniform weights over the
    visible tokens, VALU path) and a large one (the running max is raised on later tiles), with a
    partial last block so masked keys are present; bf16 and fp32 (the fp32 MFMA kernel)."""
    from omnimem_amd.selection import sel_fwd
    M, N, H, D, G, BS, T = 130, 300, 2, 128, 64, 64, 5
    gen = torch.Generator().manual_seed(11)
    q = (torch.randn((1, M, H, D), generator=gen) * D ** -0.25).to(dtype)
    k = (torch.randn((1, N, H, D), generator=gen) * D ** -0.25).to(dtype)
    v = torch.randn((1, N, H, D), generator=gen).to(dtype)
    ids = _ids(gen, 1, -(-M // G), H, T, 5)
    out, lse = sel_fwd(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), BS, 1, scale, False, G)
    want_o, want_l = O.selection_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                           ids.numpy(), G, scale, O.dense_block_tokens(N, BS, 1, False))
    _check(out, lse, want_o, want_l, dtype)


SPLIT_CASES = [
    # M, N, H, D, G, BS, T, causal, chunk, minus, dup[, B]
    (1560, 4680, 12, 128, 64, 64, 16, False, 1560, 0.0, False),  # config 1 shape, 300 items
    (500, 1000, 3, 128, 64, 64, 6, True, 250, 0.1, False, 2),  # two batches: item order b, h, g
    (64, 512, 1, 128, 64, 64, 3, False, 1, 0.0, False),    # one item: 3 runs of one slot each
    (64, 512, 1, 128, 64, 64, 7, True, 256, 0.5, True),    # runs with no live slot, duplicates
    (300, 700, 3, 128, 15, 30, 8, True, 600, 0.1, False),  # reference geometry, ragged groups
    (130, 256, 2, 64, 48, 32, 5, False, 1, 0.2, True),     # head dim 64, groups of 48
    (128, 64, 1, 128, 64, 64, 5, False, 1, 1.0, False),    # every id -1 across the runs
    (2000, 2048, 4, 128, 64, 64, 9, True, 512, 0.0, False),  # 128 items over 512 runs
]


def _sel_fwd_raw(q, k, v, ids, BS, chunk, scale, causal, G, ws):
    """omm_sel_fwd (ws None) or omm_sel_fwd_ws through the C-ABI; returns (out, lse)."""
    from omnimem_amd import _lib
    B, M, H, D = q.shape
    out = torch.empty_like(q)
    lse = torch.empty((B, H, M), dtype=torch.float32, device=q.device)
    args = [_lib.view4(q), _lib.view4(k), _lib.view4(v), _lib.view4(ids), _lib.dtype_code(q), BS,
            chunk, int(causal), G, scale, _lib.view4(out), lse.data_ptr()]
    if ws is None:
        _lib.call("omm_sel_fwd", *args, _lib.stream_of(q))
    else:
        _lib.call("omm_sel_fwd_ws", *args, ws.data_ptr(), ws.numel(), _lib.stream_of(q))
    return out, lse


@pytest.mark.parametrize("case", SPLIT_CASES)
def test_sel_fwd_f32_split_matches_oracle_and_unsplit(case):
    """fp32 calls with few items per CU split their selected blocks into equal runs (one per
    workgroup) and merge the split items' records in a second pass.  Both the split call (its
    workspace filled with NaN first: nothing in it may be read before it is written) and the
    unsplit omm_sel_fwd are checked against the float64 oracle at the fp32 bar, and against each
    other (same arithmetic per piece, merged in another order)."""
    from omnimem_amd import _lib
    M, N, H, D, G, BS, T, causal, chunk, minus, dup = case[:11]
    B = case[11] if len(case) > 11 else 1
    gen = torch.Generator().manual_seed(M + 7 * N + T)
    q = torch.randn((B, M, H, D), generator=gen) * D ** -0.25
    k = torch.randn((B, N, H, D), generator=gen) * D ** -0.25
    v = torch.randn((B, N, H, D), generator=gen)
    MG = -(-M // G)
    ids = _ids(gen, B, MG, H, T, -(-N // BS) + 1, minus, dup)
    nbytes = _lib.lib().omm_sel_fwd_workspace_bytes(B, M, H, D, T, _lib.OMM_F32, G)
    assert nbytes > 0, "few items per CU: the call must split"
    ws = torch.full((nbytes // 4,), float("nan"), device=DEV)
    qd, kd, vd, idd = q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV)
    o_s, l_s = _sel_fwd_raw(qd, kd, vd, idd, BS, chunk, D ** -0.5, causal, G, ws)
    o_p, l_p = _sel_fwd_raw(qd, kd, vd, idd, BS, chunk, D ** -0.5, causal, G, None)
    want_o, want_l = O.selection_attention(q.numpy(), k.numpy(), v.numpy(), ids.numpy(), G,
                                           D ** -0.5, O.dense_block_tokens(N, BS, chunk, causal),
                                           chunk_size=chunk, causal=causal)
    _check(o_s, l_s, want_o, want_l, torch.float32)
    _check(o_p, l_p, want_o, want_l, torch.float32)
    assert (o_s - o_p).abs().max().item() <= 1e-5
    fin = torch.isfinite(l_p)
    assert torch.equal(fin, torch.isfinite(l_s))
    assert (l_s[fin] - l_p[fin]).abs().max().item() <= 1e-5 if fin.any() else True
    # a second call reuses the workspace as the first left it
    o_2, l_2 = _sel_fwd_raw(qd, kd, vd, idd, BS, chunk, D ** -0.5, causal, G, ws)
    assert torch.equal(o_2, o_s) and torch.equal(l_2, l_s)


def test_sel_fwd_f32_split_policy():
    """The split needs fp32, head dim 64 / 128, groups of at most 64 and fewer than 4 items per
    CU; a workspace that is too small (or none) runs the unsplit kernel."""
    from omnimem_amd import _lib
    L = _lib.lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert L.omm_sel_fwd_workspace_bytes(1, 1560, 12, 128, 16, _lib.OMM_F32, 64) > 0
    assert L.omm_sel_fwd_workspace_bytes(1, 1560, 12, 128, 16, _lib.OMM_BF16, 64) == 0
    assert L.omm_sel_fwd_workspace_bytes(1, 1560, 12, 96, 16, _lib.OMM_F32, 64) == 0
    assert L.omm_sel_fwd_workspace_bytes(1, 1560, 12, 128, 16, _lib.OMM_F32, 128) == 0
    assert L.omm_sel_fwd_workspace_bytes(1, 64 * 4 * cus, 1, 128, 16, _lib.OMM_F32, 64) == 0
    assert L.omm_sel_fwd_workspace_bytes(1, 64 * (4 * cus - 1), 1, 128, 16, _lib.OMM_F32, 64) > 0
    # too small a workspace: the unsplit path, same result as omm_sel_fwd bit for bit
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn((1, L_, 2, 128), generator=gen).div_(128 ** 0.5).to(DEV)
               for L_ in (256, 512, 512))
    ids = _ids(gen, 1, 4, 2, 4, 8).to(DEV)
    small = torch.empty((1024,), dtype=torch.uint8, device=DEV)
    o_a, l_a = _sel_fwd_raw(q, k, v, ids, 64, 1, 128 ** -0.5, False, 64, small)
    o_b, l_b = _sel_fwd_raw(q, k, v, ids, 64, 1, 128 ** -0.5, False, 64, None)
    assert torch.equal(o_a, o_b) and torch.equal(l_a, l_b)
    with pytest.raises(Exception, match="16-byte aligned"):
        _lib.call("omm_sel_fwd_ws", _lib.view4(q), _lib.view4(k), _lib.view4(v), _lib.view4(ids),
                  _lib.OMM_F32, 64, 1, 0, 64, 128 ** -0.5, _lib.view4(o_a), l_a.data_ptr(),
                  small.data_ptr() + 4, 1020, _lib.stream_of(q))


def test_sel_fwd_strided_views():
    from omnimem_amd.selection import sel_fwd
    gen = torch.Generator().manual_seed(9)
    qkv = torch.randn((1, 512, 3, 4, 128), generator=gen).to(torch.bfloat16)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]  # interleaved, as a fused qkv projection
    ids = _ids(gen, 1, 8, 4, 4, 8)
    out, lse = sel_fwd(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), 64, 1, 128 ** -0.5, False, 64)
    want_o, want_l = O.selection_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                           ids.numpy(), 64, 128 ** -0.5,
                                           O.dense_block_tokens(512, 64, 1, False))
    _check(out, lse, want_o, want_l, torch.bfloat16)


@pytest.mark.parametrize("causal", [True, False])
def test_config1_fp32_full_size(causal):
    """fp32, q [1,1560,12,128], k/v [1,4680,12,128] ~ N(0,1)/sqrt(128),
    64-token blocks, groups of 64, top-16 over 1560-token frame chunks.

    causal=True is the dense op's frame-chunk mask with the queries as frame 0
    (selection_fwd.cu:218, common.cuh:327-332): every group sees frame-0 keys only, so 25 of the
    74 blocks are candidates and block 24 (tokens 1536..1599) is cut at token 1560.
    causal=False reads the queries as the last frame, so all three frames are candidates.
    The top-k indices are checked bit for bit against the oracle on the same pooled inputs
    before the attention is checked against the float64 oracle."""
    from omnimem_amd.index_topk import parallel_nsa_topk, block_pool
    from omnimem_amd.selection import selection_attention
    gen = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn((1, L, 12, 128), generator=gen) / 128 ** 0.5 for L in (1560, 4680, 4680))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc = block_pool(kd, 64)
    np.testing.assert_array_equal(kc.cpu().numpy(), O.pool_mean(k.numpy(), 64, "f32"))
    ids = parallel_nsa_topk(qd, kc, 16, block_size=64, chunk_size=1560, causal=causal,
                            group_size=64)
    want_ids = O.topk(O.pool_mean(q.numpy(), 64, "f32"), O.pool_mean(k.numpy(), 64, "f32"), 16,
                      128 ** -0.5, O.Mask(block_size=64, group_size=64, chunk_q=1560,
                                          chunk_k=1560, causal=int(causal)))
    got_ids = ids.cpu().numpy()
    np.testing.assert_array_equal(got_ids, want_ids)
    if causal:
        assert got_ids.max() <= 24 and (got_ids >= 0).all()  # frame 0 only, 25 candidates
    else:
        assert got_ids.max() > 24  # later frames are selected
    out, lse = selection_attention(qd, kd, vd, ids, 16, 64, chunk_size=1560, causal=causal,
                                   return_lse=True, group_size=64)
    want_o, want_l = O.selection_attention(q.numpy(), k.numpy(), v.numpy(), got_ids, 64,
                                           128 ** -0.5,
                                           O.dense_block_tokens(4680, 64, 1560, causal),
                                           chunk_size=1560, causal=causal)
    _check(out, lse, want_o, want_l, torch.float32)


def test_config3_layer_bf16_sampled_groups():
    """BASELINE config 3 shape for one layer: M = N = 32760, 12 heads, groups of 64, top-16,
    causal by 4680-token chunks; checked on a sample of 24 query groups (all heads)."""
    from omnimem_amd.index_topk import parallel_nsa_topk, block_pool
    from omnimem_amd.selection import sel_fwd
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn((1, 32760, 12, 128), generator=gen).to(torch.bfloat16) for _ in range(3))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    ids = parallel_nsa_topk(qd, block_pool(kd, 64), 16, block_size=64, chunk_size=4680,
                            causal=True, group_size=64)
    out, lse = sel_fwd(qd, kd, vd, ids, 64, 4680, 128 ** -0.5, True, 64)
    groups = sorted(set([0, 72, 73, 511] + torch.randint(0, 512, (20,), generator=gen).tolist()))
    want_o, want_l = O.selection_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                           ids.cpu().numpy(), 64, 128 ** -0.5,
                                           O.dense_block_tokens(32760, 64, 4680, True),
                                           chunk_size=4680, causal=True, groups=groups)
    rows = np.concatenate([np.arange(g * 64, min(32760, g * 64 + 64)) for g in groups])
    _check(out, lse, want_o, want_l, torch.bfloat16, rows=rows)


def test_selection_attention_facade_validation():
    from omnimem_amd.selection import selection_attention
    q = torch.zeros((1, 64, 1, 16), device=DEV, dtype=torch.bfloat16)
    ids = torch.full((1, 1, 1, 2), 5, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        selection_attention(q, q, q, ids, 2, 64, group_size=64)  # id 5 >= 1 block
    o = selection_attention(q.requires_grad_(), q, q, ids.clamp(max=0), 2, 64, group_size=64)
    assert o.grad_fn is not None  # the backward is wired (head dim 16 runs the VALU kernels)


@pytest.mark.parametrize("M,N,H", [(130, 300, 2), (64, 64, 1), (300, 1500, 3), (1, 70, 1)])
def test_dense_attention_matches_oracle(M, N, H):
    """dense_attention (every block listed; the AR driver's window and compressed-history
    branches) against plain softmax attention in float64, ragged M and N included."""
    from omnimem_amd.selection import dense_attention
    D = 128
    gen = torch.Generator().manual_seed(M * 7 + N)
    q = (torch.randn((1, M, H, D), generator=gen) * D ** -0.25).to(torch.bfloat16)
    k = (torch.randn((1, N, H, D), generator=gen) * D ** -0.25).to(torch.bfloat16)
    v = torch.randn((1, N, H, D), generator=gen).to(torch.bfloat16)
    out, lse = dense_attention(q.to(DEV), k.to(DEV), v.to(DEV), return_lse=True)
    T = -(-N // 64)
    ids = np.broadcast_to(np.arange(T, dtype=np.int32), (1, -(-M // 64), H, T))
    want_o, want_l = O.selection_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                           ids, 64, D ** -0.5, O.dense_block_tokens(N, 64, 1, False))
    _check(out, lse, want_o, want_l, torch.bfloat16)


def test_dense_attention_window_shape_sampled():
    """AR window shape (one chunk of 4680 queries over 3 chunks of keys), sampled query groups."""
    from omnimem_amd.selection import dense_attention
    M, N, H, D = 4680, 3 * 4680, 2, 128
    gen = torch.Generator().manual_seed(5)
    q = (torch.randn((1, M, H, D), generator=gen) * D ** -0.25).to(torch.bfloat16)
    k = (torch.randn((1, N, H, D), generator=gen) * D ** -0.25).to(torch.bfloat16)
    v = torch.randn((1, N, H, D), generator=gen).to(torch.bfloat16)
    out, lse = dense_attention(q.to(DEV), k.to(DEV), v.to(DEV), return_lse=True)
    T = -(-N // 64)
    groups = [0, 37, 73]
    ids = np.broadcast_to(np.arange(T, dtype=np.int32), (1, -(-M // 64), H, T))
    want_o, want_l = O.selection_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                           ids, 64, D ** -0.5, O.dense_block_tokens(N, 64, 1, False),
                                           groups=groups)
    rows = np.concatenate([np.arange(g * 64, min(M, g * 64 + 64)) for g in groups])
    _check(out, lse, want_o, want_l, torch.bfloat16, rows=rows)


def test_empty_shapes():
    """Degenerate sizes through the facades (the reference's early returns): no queries, no key
    blocks (every id -1, top-k all -1), and no keys at all (out 0, lse -inf)."""
    from omnimem_amd.index_topk import block_pool, parallel_nsa_topk
    from omnimem_amd.selection import sel_fwd
    H, D = 2, 128
    g = torch.Generator().manual_seed(5)
    # no queries: empty ids, empty out / lse
    q0 = torch.empty((1, 0, H, D), dtype=torch.bfloat16, device=DEV)
    k = torch.randn((1, 256, H, D), generator=g).to(torch.bfloat16).to(DEV)
    kc = block_pool(k, 64)
    ids0 = parallel_nsa_topk(q0, kc, 4, block_size=64, chunk_size=64, causal=False, group_size=64)
    assert tuple(ids0.shape) == (1, 0, H, 4)
    out0, lse0 = sel_fwd(q0, k, k, ids0, 64, 1, D ** -0.5, False, 64)
    assert out0.numel() == 0 and lse0.numel() == 0
    # pooling of zero tokens
    assert block_pool(q0, 64).shape[1] == 0
    # no key blocks: every slot -1
    q = torch.randn((1, 128, H, D), generator=g).to(torch.bfloat16).to(DEV)
    kc0 = torch.empty((1, 0, H, D), dtype=torch.bfloat16, device=DEV)
    ids = parallel_nsa_topk(q, kc0, 4, block_size=64, chunk_size=64, causal=False, group_size=64)
    assert tuple(ids.shape) == (1, 2, H, 4) and bool((ids == -1).all())
    # no keys: ids past the end select nothing, so out is 0 and lse -inf
    k0 = torch.empty((1, 0, H, D), dtype=torch.bfloat16, device=DEV)
    ids_any = torch.zeros((1, 2, H, 4), dtype=torch.int32, device=DEV)
    out, lse = sel_fwd(q, k0, k0, ids_any, 64, 1, D ** -0.5, False, 64)
    assert bool((out == 0).all()) and bool(torch.isneginf(lse).all())


@pytest.mark.parametrize("case", [
    # M, N, H, D, G, BS, T, causal, chunk
    (300, 700, 3, 128, 64, 64, 6, True, 256),   # 2-wave DMA kernel, ragged last group
    (400, 512, 2, 128, 192, 64, 5, True, 256),  # 4-wave DMA kernel (two subgroups)
    (130, 256, 2, 64, 64, 32, 5, False, 1),     # head dim 64
])
def test_sel_fwd_gated_mix_matches_float64(case):
    """Dense selection with the NSA branch mix in its epilogue (causal_wan_nsa_model.py:541-546):
    out = g0 o_cmp + g1 o_slc + g2 o_swa against float64 from the oracle's o_slc, at the bf16
    tolerances."""
    from omnimem_amd.selection import sel_fwd_gated
    M, N, H, D, G, BS, T, causal, chunk = case
    gen = torch.Generator().manual_seed(M + 7 * N)
    dt = torch.bfloat16
    q = (torch.randn((1, M, H, D), generator=gen) * D ** -0.25).to(dt)
    k = (torch.randn((1, N, H, D), generator=gen) * D ** -0.25).to(dt)
    v = torch.randn((1, N, H, D), generator=gen).to(dt)
    oc = torch.randn((1, M, H, D), generator=gen).to(dt)
    ow = torch.randn((1, M, H, D), generator=gen).to(dt)
    g = torch.sigmoid(torch.randn((1, M, H, 3), generator=gen)).to(dt)
    ids = _ids(gen, 1, -(-M // G), H, T, -(-N // BS))
    out = sel_fwd_gated(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), BS, chunk, D ** -0.5, causal,
                        G, g.to(DEV), oc.to(DEV), ow.to(DEV))
    want_slc, _ = O.selection_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                        ids.numpy(), G, D ** -0.5,
                                        O.dense_block_tokens(N, BS, chunk, causal),
                                        chunk_size=chunk, causal=causal)
    gg = g.double().numpy()
    want = (gg[..., 0:1] * oc.double().numpy() + gg[..., 1:2] * want_slc
            + gg[..., 2:3] * ow.double().numpy())
    err = np.abs(out.double().cpu().numpy() - want)
    assert err.max() <= 2e-2, f"max-abs {err.max():.3e}"
    assert err.mean() <= 1e-3, f"mean-abs {err.mean():.3e}"


def test_sel_fwd_gated_rejects_overlap_and_bad_inputs():
    """out may not be or overlap o_cmp / o_swa (the fallback kernel mixes in a second pass after
    writing out); the gated call is bf16 only, with gates [B, M, H, 3]."""
    from omnimem_amd.backend import NSABackendError
    from omnimem_amd.selection import sel_fwd_gated
    M, N, H, D, G, BS = 128, 256, 2, 128, 64, 64
    dt = torch.bfloat16
    q = torch.randn((1, M, H, D), device=DEV).to(dt)
    k = torch.randn((1, N, H, D), device=DEV).to(dt)
    oc, ow = torch.randn_like(q), torch.randn_like(q)
    g = torch.rand((1, M, H, 3), device=DEV).to(dt)
    ids = torch.zeros((1, 2, H, 2), dtype=torch.int32, device=DEV)
    ids[..., 1] = 1

    def call(q_=q, g_=g, oc_=oc, ow_=ow, out=None):
        return sel_fwd_gated(q_, k.to(q_.dtype), k.to(q_.dtype), ids, BS, 1, D ** -0.5, False, G,
                             g_, oc_, ow_, out=out)

    buf = torch.empty((1, M + 1, H, D), dtype=dt, device=DEV)
    for kw in ({"out": oc}, {"out": ow}, {"oc_": buf[:, :M], "out": buf[:, 1:]}):
        with pytest.raises(NSABackendError, match="overlap"):
            call(**kw)
    with pytest.raises(NSABackendError, match="bf16"):
        call(q_=q.float())
    with pytest.raises(NSABackendError, match="gates"):
        call(g_=torch.rand((1, M, H, 2), device=DEV).to(dt))
    assert torch.isfinite(call().float()).all()
