"""GPU parity of block compression, query pooling and top-k against the CPU oracle.

Bit-exact: pooled values; block indices of the exact-order path (fp32, or strides / head dims
off the MFMA path) against the oracle's own fmaf scores; block indices of the MFMA path (bf16 /
f16, head dim 64 or 128) against the oracle's selection on the kernel's own scores, whose
accuracy is bounded separately (tests/_topk_checks.py).  Cases follow the reference's mask modes
(cuda_backend/csrc/topk.cu:36-97) and BASELINE config 2 at full size.
"""
import zlib

import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O
from _topk_checks import check_mfma_topk

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _bf16(shape, gen, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16)


def _img(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,group", [(256, 64), (70, 64), (4680, 64), (300, 15), (5, 1),
                                     (32768, 64), (130, 130)])
def test_block_pool_bitexact(dtype, T, group):
    """Small launches run the 4-wave kernel (rows staged in LDS), large ones (32768 tokens:
    1,024 rows x 1 column slice) the one-wave kernel; group 130 takes two 64-token runs, the
    second of 2 tokens."""
    from omnimem_amd.index_topk import block_pool
    g = torch.Generator().manual_seed(T * 7 + group)
    x = torch.randn((2, T, 3, 128), generator=g).to(dtype)
    got = block_pool(x.to(DEV), group).cpu()
    dt = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype]
    want = O.pool_mean(_img(x), group, dt)
    np.testing.assert_array_equal(got.float().numpy(), want)


def test_block_pool_strided_input():
    from omnimem_amd.index_topk import block_pool
    g = torch.Generator().manual_seed(3)
    base = torch.randn((1, 128, 4, 2, 64), generator=g).to(torch.bfloat16)
    x = base[:, :, :, 1, :]  # non-contiguous head stride
    got = block_pool(x.to(DEV), 30).cpu()
    np.testing.assert_array_equal(got.float().numpy(), O.pool_mean(_img(x), 30, "bf16"))


def _scores_case(seed, B, MG, H, NC, ties=True):
    rng = np.random.default_rng(seed)
    if ties:
        s = rng.integers(-20, 20, size=(B, MG, H, NC)).astype(np.float32) * 0.125
        s[rng.random(s.shape) < 0.02] = -0.0
    else:
        s = rng.standard_normal((B, MG, H, NC)).astype(np.float32)
    s[rng.random(s.shape) < 0.01] = -np.inf
    s[rng.random(s.shape) < 0.005] = np.nan
    return s


MASKS = {
    "causal": dict(block_size=64, group_size=64, chunk_q=256, chunk_k=256, causal=1),
    "causal_ragged": dict(block_size=64, group_size=64, chunk_q=4680, chunk_k=4680, causal=1),
    "ar_awe": dict(block_size=64, group_size=64, chunk_q=4680, chunk_k=4680, blocks_per_chunk=74,
                   q_chunk_offset=5, ex_win=3, causal=0, prog_excl=1),
    "sink_win": dict(block_size=30, group_size=15, chunk_q=4680, chunk_k=4680, ex_sink=1, ex_win=2,
                     causal=1, prog_excl=1),
    "noncausal": dict(block_size=64, group_size=1, chunk_q=64, chunk_k=64, causal=0),
}


@pytest.mark.parametrize("mask", list(MASKS))
@pytest.mark.parametrize("topk", [1, 16, 64, 65, 100, 128])
@pytest.mark.parametrize("NC", [37, 512, 5850])
def test_topk_from_scores_bitexact(mask, topk, NC):
    """topk up to 128 (the reference's path A range, topk.cu:584, 648-660): past 64 the
    survivor threshold comes from every lane's two largest keys; rows with fewer visible blocks
    than topk pad with -1."""
    from omnimem_amd.index_topk import topk_from_scores
    mk = MASKS[mask]
    B, MG, H = 1, 74, 3
    s = _scores_case(zlib.crc32(f"{mask}/{topk}/{NC}".encode()) & 0xFFFF, B, MG, H, NC)
    G = mk["group_size"]
    got = topk_from_scores(torch.from_numpy(s).to(DEV), topk, mk["block_size"], mk["chunk_q"] // G
                           if mk["chunk_q"] % G == 0 else mk["chunk_q"], mk["chunk_k"],
                           bool(mk["causal"]), ex_win=mk.get("ex_win", 0),
                           ex_sink=mk.get("ex_sink", 0), prog_excl=bool(mk.get("prog_excl", 0)),
                           q_chunk_offset=mk.get("q_chunk_offset", 0), group_size=G
                           if mk["chunk_q"] % G == 0 else 1,
                           blocks_per_chunk=mk.get("blocks_per_chunk", 0)).cpu().numpy()
    om = O.Mask(**mk)
    if mk["chunk_q"] % G != 0:
        om.group_size = 1
    want = O.topk_select(s, topk, om)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("topk", [96, 128])
def test_parallel_nsa_topk_fused_large_topk_bitexact(dtype, topk):
    """Fused pooling + scoring + top-k with 64 < topk <= 128: off the MFMA path (topk > 16), so
    the scores are the fmaf chain and the indices are bit-exact against the oracle's scores;
    the AR mask over 80 cached chunks (split spans and the merge) and a causal case."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(topk)
    B, H, D = 1, 2, 128
    for T, NC, chunk, causal, qoff, exw in ((4680, 5920, 4680, False, 80, 3),
                                            (2048, 128, 512, True, 0, 0)):
        q = torch.randn((B, T, H, D), generator=g).to(dtype)
        k = torch.randn((B, NC, H, D), generator=g).to(dtype)
        bpc = 74 if not causal else 0
        got = parallel_nsa_topk(q.to(DEV), k.to(DEV), topk, block_size=64, chunk_size=chunk,
                                causal=causal, exclude_window_chunks=exw,
                                progressive_exclude=not causal, q_chunk_offset=qoff,
                                blocks_per_chunk=bpc, group_size=64).cpu().numpy()
        mask = O.Mask(block_size=64, group_size=64, chunk_q=chunk, chunk_k=chunk,
                      blocks_per_chunk=bpc, q_chunk_offset=qoff, ex_win=exw,
                      causal=int(causal), prog_excl=int(not causal))
        dt = "bf16" if dtype == torch.bfloat16 else "f32"
        want = O.topk(O.pool_mean(_img(q), 64, dt), _img(k), topk, D ** -0.5, mask)
        np.testing.assert_array_equal(got, want)
        if causal:
            assert (got[:, :8] == -1).any()  # early rows see fewer than topk blocks


def test_topk_above_cap_rejected():
    from omnimem_amd.backend import NSABackendError
    from omnimem_amd.index_topk import parallel_nsa_topk
    q = torch.zeros((1, 128, 1, 64), device=DEV)
    k = torch.zeros((1, 300, 1, 64), device=DEV)
    with pytest.raises(NSABackendError, match="4096"):
        parallel_nsa_topk(q, k, 4097, block_size=64, chunk_size=64, causal=False, group_size=64)


@pytest.mark.parametrize("mask", list(MASKS))
@pytest.mark.parametrize("topk", [129, 300])
@pytest.mark.parametrize("NC", [37, 512, 5850])
def test_topk_from_scores_above_128_bitexact(mask, topk, NC):
    """topk past 128 follows the reference's path B (topk.cu:741-807): raw order codes, so -0,
    -inf and NaN scores of visible blocks are ranked; hidden blocks give -1; -1 past NC."""
    from omnimem_amd.index_topk import topk_from_scores
    mk = MASKS[mask]
    B, MG, H = 1, 74, 3
    s = _scores_case(zlib.crc32(f"large/{mask}/{topk}/{NC}".encode()) & 0xFFFF, B, MG, H, NC)
    G = mk["group_size"]
    got = topk_from_scores(torch.from_numpy(s).to(DEV), topk, mk["block_size"], mk["chunk_q"] // G
                           if mk["chunk_q"] % G == 0 else mk["chunk_q"], mk["chunk_k"],
                           bool(mk["causal"]), ex_win=mk.get("ex_win", 0),
                           ex_sink=mk.get("ex_sink", 0), prog_excl=bool(mk.get("prog_excl", 0)),
                           q_chunk_offset=mk.get("q_chunk_offset", 0), group_size=G
                           if mk["chunk_q"] % G == 0 else 1,
                           blocks_per_chunk=mk.get("blocks_per_chunk", 0)).cpu().numpy()
    om = O.Mask(**mk)
    if mk["chunk_q"] % G != 0:
        om.group_size = 1
    np.testing.assert_array_equal(got, O.topk_select_large(s, topk, om))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("topk", [129, 700])
def test_parallel_nsa_topk_fused_above_128_bitexact(dtype, topk):
    """Fused pooling + scoring with topk past 128: the scores of every row go to the workspace
    (the fmaf chain, across split column spans for the 5920-block AR history) and one
    workgroup per row selects; bit-exact against the oracle's scores under path B's rule.  On
    these finite scores the first 128 ids equal the topk = 128 call's."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(topk)
    B, H, D = 1, 2, 128
    for T, NC, chunk, causal, qoff, exw in ((4680, 5920, 4680, False, 80, 3),
                                            (2048, 600, 512, True, 0, 0)):
        q = torch.randn((B, T, H, D), generator=g).to(dtype)
        k = torch.randn((B, NC, H, D), generator=g).to(dtype)
        bpc = 74 if not causal else 0
        kw = dict(block_size=64, chunk_size=chunk, causal=causal, exclude_window_chunks=exw,
                  progressive_exclude=not causal, q_chunk_offset=qoff, blocks_per_chunk=bpc,
                  group_size=64)
        got = parallel_nsa_topk(q.to(DEV), k.to(DEV), topk, **kw).cpu().numpy()
        mask = O.Mask(block_size=64, group_size=64, chunk_q=chunk, chunk_k=chunk,
                      blocks_per_chunk=bpc, q_chunk_offset=qoff, ex_win=exw,
                      causal=int(causal), prog_excl=int(not causal))
        dt = "bf16" if dtype == torch.bfloat16 else "f32"
        scores = O.block_scores(O.pool_mean(_img(q), 64, dt), _img(k), D ** -0.5)
        np.testing.assert_array_equal(got, O.topk_select_large(scores, topk, mask))
        small = parallel_nsa_topk(q.to(DEV), k.to(DEV), 128, **kw).cpu().numpy()
        np.testing.assert_array_equal(got[..., :128], small)


def test_topk_pooled_op_above_128_bitexact():
    """The pooled-rows op (omm_topk) with topk past 128: top-200 of 300 visible blocks, and a
    causal case whose rows see at most 10 blocks and pad with -1."""
    from omnimem_amd.index_topk import topk as topk_op
    g = torch.Generator().manual_seed(5)
    B, MG, H, D, NC = 2, 40, 3, 64, 300
    q = torch.randn((B, MG, H, D), generator=g)
    k = torch.randn((B, NC, H, D), generator=g)
    scores = O.block_scores(_img(q), _img(k), 0.125)
    for causal, cq, ck in ((False, 64, 64), (True, 8, 128)):
        got = topk_op(q.to(DEV), k.to(DEV), 200, 0.125, 64, cq, ck, causal).cpu().numpy()
        mask = O.Mask(block_size=64, group_size=1, chunk_q=cq, chunk_k=ck, causal=int(causal))
        np.testing.assert_array_equal(got, O.topk_select_large(scores, 200, mask))
        if causal:
            assert (got[..., 10:] == -1).all() and (got[..., :2] >= 0).all()
        else:
            assert (got >= 0).all()


def test_topk_tf_mask_bitexact():
    from omnimem_amd.index_topk import topk_from_scores
    B, H, chunk, bs = 1, 2, 64, 16
    MG, NC = 8 * chunk, 8 * chunk // bs
    s = _scores_case(77, B, MG, H, NC)
    got = topk_from_scores(torch.from_numpy(s).to(DEV), 16, bs, chunk, chunk, True,
                           tf_mask=True).cpu().numpy()
    want = O.topk_select(s, 16, O.Mask(block_size=bs, group_size=1, chunk_q=chunk, chunk_k=chunk,
                                       causal=1, tf_mask=1, q_half=4, k_half=4))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,NC,G,chunk,causal,qoff,exw", [
    (1024, 16, 64, 256, True, 0, 0),
    (4680, 592, 64, 4680, False, 7, 3),      # AR step: one chunk of queries vs 8 cached chunks
    (3000, 100, 30, 600, True, 0, 1),
])
def test_parallel_nsa_topk_fused_bitexact(dtype, T, NC, G, chunk, causal, qoff, exw):
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(T + NC)
    B, H, D = 1, 4, 128
    q = torch.randn((B, T, H, D), generator=g).to(dtype)
    k = torch.randn((B, NC, H, D), generator=g).to(dtype)
    bpc = 74 if not causal else 0
    kw = dict(block_size=64, chunk_size=chunk, causal=causal, exclude_window_chunks=exw,
              progressive_exclude=not causal, q_chunk_offset=qoff, blocks_per_chunk=bpc)
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 16, group_size=G, **kw).cpu().numpy()
    mask = O.Mask(block_size=64, group_size=G, chunk_q=chunk, chunk_k=chunk,
                  blocks_per_chunk=bpc, q_chunk_offset=qoff, ex_win=exw,
                  causal=int(causal), prog_excl=int(not causal))
    if dtype == torch.bfloat16:  # MFMA path
        check_mfma_topk(q.to(DEV), k.to(DEV), 16, mask, D ** -0.5, G, got=got, **kw)
        return
    qp = O.pool_mean(_img(q), G, "f32")
    want = O.topk(qp, _img(k), 16, D ** -0.5, mask)
    np.testing.assert_array_equal(got, want)


def test_topk_config2_full_size_bitexact():
    """q [1,32768,12,128] bf16 pooled by 64, k_cmp [1,512,12,128], top-16,
    chunk 4680 tokens, causal."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(2)
    q = torch.randn((1, 32768, 12, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 512, 12, 128), generator=g).to(torch.bfloat16)
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 16, block_size=64, chunk_size=4680,
                            causal=True, group_size=64).cpu().numpy()
    mask = O.Mask(block_size=64, group_size=64, chunk_q=4680, chunk_k=4680, causal=1)
    check_mfma_topk(q.to(DEV), k.to(DEV), 16, mask, 128 ** -0.5, 64, got=got, block_size=64,
                    chunk_size=4680, causal=True)
    assert (got >= 0).all()  # every group sees >= 73 blocks


def test_grouped_heads_broadcast():
    from omnimem_amd.index_topk import parallel_nsa_topk_grouped_heads
    g = torch.Generator().manual_seed(5)
    q = torch.randn((1, 512, 4, 64), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 32, 4, 64), generator=g).to(torch.bfloat16)
    got = parallel_nsa_topk_grouped_heads(q.to(DEV), k.to(DEV), 2, 8, 16, 128, causal=True,
                                          group_size=16).cpu().numpy()
    # head pool (pairs of heads) then query pool, both rounded to bf16
    qh = O.round_to(_img(q).reshape(1, 512, 2, 2, 64).astype(np.float32).sum(3) / 2, "bf16")
    kh = O.round_to(_img(k).reshape(1, 32, 2, 2, 64).astype(np.float32).sum(3) / 2, "bf16")
    mask = O.Mask(block_size=16, group_size=16, chunk_q=128, chunk_k=128, causal=1)
    qh_t = torch.from_numpy(qh).to(torch.bfloat16).to(DEV)
    kh_t = torch.from_numpy(kh).to(torch.bfloat16).to(DEV)
    want = check_mfma_topk(qh_t, kh_t, 8, mask, 64 ** -0.5, 16, block_size=16, chunk_size=128,
                           causal=True)
    np.testing.assert_array_equal(got[:, :, 0::2], want)
    np.testing.assert_array_equal(got[:, :, 1::2], want)


def test_topk_fused_config3_ragged_tail_bitexact():
    """Config 3 shape: T = 32760 (last group 56 tokens) pooled inside the top-k kernel."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(33)
    q = torch.randn((1, 32760, 12, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 512, 12, 128), generator=g).to(torch.bfloat16)
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 16, block_size=64, chunk_size=4680,
                            causal=True, group_size=64).cpu().numpy()
    mask = O.Mask(block_size=64, group_size=64, chunk_q=4680, chunk_k=4680, causal=1)
    check_mfma_topk(q.to(DEV), k.to(DEV), 16, mask, 128 ** -0.5, 64, got=got, block_size=64,
                    chunk_size=4680, causal=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_topk_fused_many_heads_bitexact(dtype):
    """64 heads x 4 row tiles: the single-pass fused kernel, every element type."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(34)
    q = torch.randn((1, 4096, 64, 64), generator=g).to(dtype)
    k = torch.randn((1, 200, 64, 64), generator=g).to(dtype)
    kw = dict(block_size=32, chunk_size=1024, causal=True, exclude_sink_chunks=1,
              exclude_window_chunks=1)
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 8, group_size=64, **kw).cpu().numpy()
    mask = O.Mask(block_size=32, group_size=64, chunk_q=1024, chunk_k=1024, causal=1,
                  ex_sink=1, ex_win=1)
    if dtype != torch.float32:  # MFMA path
        check_mfma_topk(q.to(DEV), k.to(DEV), 8, mask, 64 ** -0.5, 64, got=got, **kw)
        return
    want = O.topk(O.pool_mean(_img(q), 64, "f32"), _img(k), 8, 64 ** -0.5, mask)
    np.testing.assert_array_equal(got, want)


def test_topk_strided_inputs_scalar_staging_bitexact():
    """Non-unit dim strides on q and k: element-wise staging paths."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(35)
    qb = torch.randn((1, 640, 3, 96, 2), generator=g).to(torch.bfloat16)
    kb = torch.randn((1, 50, 3, 96, 2), generator=g).to(torch.bfloat16)
    q, k = qb[..., 0], kb[..., 1]
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 6, block_size=16, chunk_size=160,
                            causal=True, group_size=20).cpu().numpy()
    want = O.topk(O.pool_mean(_img(q), 20, "bf16"), _img(k), 6, 96 ** -0.5,
                  O.Mask(block_size=16, group_size=20, chunk_q=160, chunk_k=160, causal=1))
    np.testing.assert_array_equal(got, want)


def test_topk_prepooled_op_long_history_split_merge():
    """Pre-pooled op with a long history: column splits + merge (AR shape, 80 cached chunks)."""
    from omnimem_amd.index_topk import topk
    g = torch.Generator().manual_seed(36)
    q = torch.randn((1, 74, 12, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 80 * 74, 12, 128), generator=g).to(torch.bfloat16)
    # chunk_size counts pooled rows (74 rows = one 4680-token chunk of queries, chunk 80)
    got = topk(q.to(DEV), k.to(DEV), 16, 128 ** -0.5, 64, 74, 4680, False, ex_win=3,
               prog_excl=True, q_chunk_offset=80, group_size=64,
               blocks_per_chunk=74).cpu().numpy()
    # the same rows through the scores hook: one row per "token" (group 1), 74-row query chunks;
    # keys in chunk-aligned pages of 74
    mask = O.Mask(block_size=64, group_size=1, chunk_q=74, chunk_k=74, blocks_per_chunk=74,
                  q_chunk_offset=80, ex_win=3, causal=0, prog_excl=1)
    check_mfma_topk(q.to(DEV), k.to(DEV), 16, mask, 128 ** -0.5, 1, got=got, block_size=64,
                    chunk_size=74, causal=False, exclude_window_chunks=3, progressive_exclude=True,
                    q_chunk_offset=80, blocks_per_chunk=74)


def test_topk_fused_massive_ties_bitexact():
    """Score ties far beyond the survivor buffer (keys of heads 0-1 all zero: every score is 0,
    the top-16 are the 16 lowest visible ids; heads 2-7 keys in {-1, 0, 1} / 8): rows with more
    than 64 survivors take the one-row fallback."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(37)
    q = torch.randn((1, 32768, 8, 128), generator=g).to(torch.bfloat16)
    k = (torch.randint(-1, 2, (1, 512, 8, 128), generator=g).float() / 8).to(torch.bfloat16)
    k[:, :, :2] = 0
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 16, block_size=64, chunk_size=4680,
                            causal=True, group_size=64).cpu().numpy()
    mask = O.Mask(block_size=64, group_size=64, chunk_q=4680, chunk_k=4680, causal=1)
    check_mfma_topk(q.to(DEV), k.to(DEV), 16, mask, 128 ** -0.5, 64, got=got, block_size=64,
                    chunk_size=4680, causal=True)
    assert (got[:, :, :2] == np.arange(16)).all()  # all-zero scores: the lowest ids


# Mask modes on the MFMA path's four-rows-per-wave selection, whose visibility is a pair of
# column intervals per row (one visible run, plus a noisy row's own noisy chunk under tf_mask or
# the chunks past a non-causal exclusion window).  Each case is (T, NC, H, D, G, topk, facade
# keyword arguments); together they take spans of 4, 8 and 12 column steps, the fused and the
# pool-to-workspace kernels, column splits with the merge, and every interval shape.
MFMA_MASK_CASES = {
    "tf": (1024, 64, 2, 64, 16, 8, dict(block_size=16, chunk_size=128, causal=True,
                                        tf_mask=True)),
    "tf_sink_win_prog": (2048, 128, 2, 128, 16, 16,
                         dict(block_size=16, chunk_size=128, causal=True, tf_mask=True,
                              exclude_sink_chunks=1, exclude_window_chunks=2,
                              progressive_exclude=True)),
    "sink_win_causal": (3000, 100, 2, 128, 30, 16,
                        dict(block_size=30, chunk_size=600, causal=True, exclude_sink_chunks=1,
                             exclude_window_chunks=2, progressive_exclude=True)),
    "window_two_runs": (2048, 128, 2, 64, 16, 16,
                        dict(block_size=16, chunk_size=256, causal=False,
                             exclude_window_chunks=2)),
    "window_two_runs_offset": (4680, 740, 3, 128, 64, 16,
                               dict(block_size=64, chunk_size=4680, causal=False,
                                    exclude_window_chunks=2, q_chunk_offset=4,
                                    blocks_per_chunk=74)),
    "noncausal_jm12_fused": (4096, 700, 16, 64, 16, 16,
                             dict(block_size=64, chunk_size=4096, causal=False)),
    "noncausal_split_merge": (300, 2000, 2, 128, 1, 16,
                              dict(block_size=64, chunk_size=300, causal=False)),
    "causal_ragged_small_topk": (4680, 512, 4, 128, 64, 3,
                                 dict(block_size=64, chunk_size=4680, causal=True)),
}


def _oracle_mask(T, NC, G, kw):
    chunk = kw["chunk_size"]
    bs = kw["block_size"]
    tf = bool(kw.get("tf_mask", False))
    MG = -(-T // G)
    return O.Mask(block_size=bs, group_size=G, chunk_q=chunk, chunk_k=chunk,
                  blocks_per_chunk=kw.get("blocks_per_chunk", 0),
                  q_chunk_offset=kw.get("q_chunk_offset", 0),
                  q_half=(MG * G) // (2 * chunk) if tf else 0,
                  k_half=(NC * bs) // (2 * chunk) if tf else 0,
                  ex_win=kw.get("exclude_window_chunks", 0),
                  ex_sink=kw.get("exclude_sink_chunks", 0), causal=int(kw["causal"]),
                  tf_mask=int(tf), prog_excl=int(kw.get("progressive_exclude", False)))


@pytest.mark.parametrize("case", list(MFMA_MASK_CASES))
def test_mfma_selection_mask_modes(case):
    from omnimem_amd.index_topk import parallel_nsa_topk
    T, NC, H, D, G, topk, kw = MFMA_MASK_CASES[case]
    g = torch.Generator().manual_seed(zlib.crc32(case.encode()) & 0xFFFF)
    q = _bf16((1, T, H, D), g)
    k = _bf16((1, NC, H, D), g)
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), topk, group_size=G, **kw).cpu().numpy()
    check_mfma_topk(q.to(DEV), k.to(DEV), topk, _oracle_mask(T, NC, G, kw), D ** -0.5, G,
                    got=got, **kw)


def test_mfma_selection_nan_and_inf_scores():
    """Keys holding NaN or +-inf give NaN / +-inf scores: NaN and -inf are never selected, +inf
    wins (cuda_backend/csrc/topk.cu:36-102).  The selection keeps NaN out of its running maxima
    through v_med3_f32's NaN rule; this pins that on the device."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(91)
    T, NC, H, D, G = 2048, 300, 2, 128, 16
    q = _bf16((1, T, H, D), g)
    k = _bf16((1, NC, H, D), g)
    k[0, 5::7, 0, 3] = float("nan")
    k[0, 11::13, 1, 0] = float("inf")
    k[0, 2::17, :, 1] = float("-inf")
    kw = dict(block_size=16, chunk_size=T, causal=False)
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 16, group_size=G, **kw).cpu().numpy()
    mask = _oracle_mask(T, NC, G, kw)
    # the score bound of check_mfma_topk is meaningless for non-finite scores: compare the
    # indices with the oracle's selection on the kernel's own scores only
    from omnimem_amd.index_topk import parallel_nsa_topk_with_scores
    ids, sc = parallel_nsa_topk_with_scores(q.to(DEV), k.to(DEV), 16, group_size=G, **kw)
    sc = sc.cpu().numpy()
    assert np.isnan(sc).any() and np.isposinf(sc).any() and np.isneginf(sc).any()
    np.testing.assert_array_equal(ids.cpu().numpy(), got)
    np.testing.assert_array_equal(got, O.topk_select(sc, 16, mask))


def test_ar_shape_fused_topk_80_chunks():
    """The call the AR driver makes at 80 cached chunks (omnimem_amd/wan_ar.py, reference
    causal_wan_nsa_model.py:496-505): one 4680-token chunk of full-resolution bf16 queries
    (groups of 64, ragged last group) against 5920 pooled keys (74 per chunk), window of 3 chunks
    excluded progressively, q_chunk_offset 80.  This takes the pool-to-workspace kernel, the
    column-split MFMA kernel and the merge; checked against the oracle's selection on the
    kernel's scores and the fp32 score bound."""
    from omnimem_amd.index_topk import parallel_nsa_topk
    g = torch.Generator().manual_seed(80)
    q = _bf16((1, 4680, 12, 128), g)
    k = _bf16((1, 80 * 74, 12, 128), g)
    kw = dict(block_size=64, chunk_size=4680, causal=False, exclude_window_chunks=3,
              exclude_sink_chunks=0, progressive_exclude=True, q_chunk_offset=80,
              blocks_per_chunk=74)
    got = parallel_nsa_topk(q.to(DEV), k.to(DEV), 16, group_size=64, **kw).cpu().numpy()
    mask = O.Mask(block_size=64, group_size=64, chunk_q=4680, chunk_k=4680, blocks_per_chunk=74,
                  q_chunk_offset=80, ex_win=3, causal=0, prog_excl=1)
    check_mfma_topk(q.to(DEV), k.to(DEV), 16, mask, 128 ** -0.5, 64, got=got, **kw)
    assert (got >= 0).all() and got.max() < 78 * 74  # the window chunks 78, 79 are excluded
