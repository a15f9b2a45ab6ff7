"""GPU parity of the dense selection-attention backward against the float64 oracle.

The oracle's backward (oracle.nsa_oracle.selection_attention_bwd, pinned in tests/test_oracle.py by
finite differences and by torch autograd) is fed the same bf16/f16 inputs and the GPU forward's
own (out, lse), so the comparison isolates the backward kernels.  Tolerance, per gradient tensor
g with oracle value r: max|g - r| <= 2e-2 * max|r| and mean|g - r| <= 5e-3 * mean|r| (16-bit
MFMA operands for P and dS, fp32 accumulation, one rounding of the result to the input dtype);
fp32 inputs (full fp32 VALU arithmetic, BASELINE's fp32 bar): 1e-4 * max|r| and 1e-5 * mean|r|.
Head dims other than 64 / 128, fp32 and non-unit dim strides run the VALU kernels.

Cases follow the forward's (reference rules: cuda_backend/csrc/selection_bwd.cu:18-306,
inverted_index.cu:13-34, bwd_common.cuh:33-60): partial tail blocks, chunk-causal prefixes, -1
and out-of-range ids, duplicated ids (counted twice), groups longer than 64 queries, blocks
longer than 64 tokens, the reference's own geometry (30-token blocks, groups of 15), rows that
see nothing, head dim 64, and BASELINE config 3 at full size.
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


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


TOL = {torch.bfloat16: (2e-2, 5e-3), torch.float16: (2e-2, 5e-3), torch.float32: (1e-4, 1e-5)}


def _close(name, got, want, mx=2e-2, mean=5e-3):
    g = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(g - want)
    scale_max = max(np.abs(want).max(), 1e-30)
    scale_mean = max(np.abs(want).mean(), 1e-30)
    assert err.max() <= mx * scale_max, f"{name}: max-abs {err.max():.3e} > {mx} x {scale_max:.3e}"
    assert err.mean() <= mean * scale_mean, (
        f"{name}: mean-abs {err.mean():.3e} > {mean} x {scale_mean:.3e}")


def _run(q, k, v, ids, G, BS, causal, chunk, dtype, scale=None, seed=0):
    from omnimem_amd.selection import sel_fwd, sel_bwd
    D = q.shape[-1]
    scale = D ** -0.5 if scale is None else scale
    qd, kd, vd, idd = (x.to(DEV) for x in (q, k, v, ids))
    out, lse = sel_fwd(qd, kd, vd, idd, BS, chunk, scale, causal, G)
    gen = torch.Generator().manual_seed(seed + 1)
    do = torch.randn(q.shape, generator=gen).to(dtype)
    dq, dk, dv = sel_bwd(qd, kd, vd, idd, out, lse, do.to(DEV), BS, chunk, scale, causal, G)
    torch.cuda.synchronize()
    return out, lse, do, dq, dk, dv, scale


CASES = [
    # M, N, H, D, G, BS, T, causal, chunk, minus, dup
    (256, 512, 2, 128, 64, 64, 4, False, 1, 0.0, False),
    (300, 700, 3, 128, 15, 30, 8, True, 600, 0.1, False),
    (200, 333, 2, 128, 100, 100, 3, True, 150, 0.0, False),
    (64, 256, 2, 128, 1, 64, 2, False, 1, 0.0, False),
    (130, 256, 2, 64, 64, 32, 5, False, 1, 0.2, True),
    (192, 640, 2, 128, 64, 64, 6, True, 128, 0.0, False),
    (128, 64, 1, 128, 64, 64, 3, False, 1, 1.0, False),  # every id -1: all gradients 0
]


CASES_VALU = [
    # M, N, H, D, G, BS, T, causal, chunk, minus, dup
    (256, 512, 2, 128, 64, 64, 4, False, 1, 0.0, False),
    (300, 700, 3, 128, 15, 30, 8, True, 600, 0.1, False),
    (200, 333, 2, 96, 100, 100, 3, True, 150, 0.0, True),
    (90, 180, 1, 200, 30, 16, 6, True, 60, 0.2, False),
]


@pytest.mark.parametrize("case", CASES, ids=[f"case{i}" for i in range(len(CASES))])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sel_bwd_matches_oracle(case, dtype):
    M, N, H, D, G, BS, T, causal, chunk, minus, dup = case
    gen = torch.Generator().manual_seed(hash(case) % 1000)
    q, k, v = (torch.randn((1, L, H, D), generator=gen).to(dtype) for L in (M, N, N))
    MG = -(-M // G)
    ids = _ids(gen, 1, MG, H, T, -(-N // BS), minus, dup)
    out, lse, do, dq, dk, dv, scale = _run(q, k, v, ids, G, BS, causal, chunk, dtype)
    want = O.selection_attention_bwd(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                     ids.numpy(), out.double().cpu().numpy(),
                                     lse.double().cpu().numpy(), do.double().numpy(), G, scale,
                                     O.dense_block_tokens(N, BS, chunk, causal), chunk_size=chunk,
                                     causal=causal)
    if minus == 1.0:
        for t in (dq, dk, dv):
            assert torch.count_nonzero(t) == 0
        return
    for name, got, w in (("dq", dq, want[0]), ("dk", dk, want[1]), ("dv", dv, want[2])):
        _close(name, got, w)


# fp32 everywhere; bf16 only at head dims the MFMA kernels do not take (bf16 at 64 / 128 runs
# the MFMA kernels, covered by test_sel_bwd_matches_oracle)
VALU_PARAMS = [pytest.param(case, dt, id=f"valu{i}-{'f32' if dt == torch.float32 else 'bf16'}")
               for i, case in enumerate(CASES_VALU) for dt in (torch.float32, torch.bfloat16)
               if not (dt == torch.bfloat16 and case[3] in (64, 128))]


@pytest.mark.parametrize("case,dtype", VALU_PARAMS)
def test_sel_bwd_valu_matches_oracle(case, dtype):
    """fp32 everywhere, and bf16 at head dims the MFMA kernels do not take (96, 200)."""
    M, N, H, D, G, BS, T, causal, chunk, minus, dup = case
    gen = torch.Generator().manual_seed(hash(case) % 997)
    q, k, v = (torch.randn((1, L, H, D), generator=gen).to(dtype) for L in (M, N, N))
    ids = _ids(gen, 1, -(-M // G), H, T, -(-N // BS), minus, dup)
    out, lse, do, dq, dk, dv, scale = _run(q, k, v, ids, G, BS, causal, chunk, dtype)
    want = O.selection_attention_bwd(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                     ids.numpy(), out.double().cpu().numpy(),
                                     lse.double().cpu().numpy(), do.double().numpy(), G, scale,
                                     O.dense_block_tokens(N, BS, chunk, causal), chunk_size=chunk,
                                     causal=causal)
    mx, mean = TOL[dtype]
    for name, got, w in (("dq", dq, want[0]), ("dk", dk, want[1]), ("dv", dv, want[2])):
        _close(name, got, w, mx, mean)


def test_sel_bwd_strided_views():
    """q / k / v / d_out as non-contiguous views: dim stride 2 (VALU kernels) and head-major
    layouts with unit dim stride (MFMA kernels)."""
    from omnimem_amd.selection import sel_fwd, sel_bwd
    dtype = torch.bfloat16
    M, N, H, D, G, BS, T = 128, 320, 2, 128, 64, 64, 3
    gen = torch.Generator().manual_seed(21)
    ids = _ids(gen, 1, M // G, H, T, N // BS)
    for mode in ("dim_stride_2", "head_major"):
        if mode == "dim_stride_2":
            src = [torch.randn((1, L, H, 2 * D), generator=gen).to(dtype) for L in (M, N, N, M)]
            host = [x[..., ::2] for x in src]
            dev = [x.to(DEV)[..., ::2] for x in src]
        else:
            src = [torch.randn((1, H, L, D), generator=gen).to(dtype) for L in (M, N, N, M)]
            host = [x.transpose(1, 2) for x in src]
            dev = [x.to(DEV).transpose(1, 2) for x in src]
        assert dev[0].stride(-1) == (2 if mode == "dim_stride_2" else 1)
        q, k, v, do = host
        qd, kd, vd, dod = dev
        out, lse = sel_fwd(qd, kd, vd, ids.to(DEV), BS, 1, D ** -0.5, False, G)
        dq, dk, dv = sel_bwd(qd, kd, vd, ids.to(DEV), out, lse, dod, BS, 1, D ** -0.5, False, G)
        want = O.selection_attention_bwd(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                         ids.numpy(), out.double().cpu().numpy(),
                                         lse.double().cpu().numpy(), do.double().numpy(), G,
                                         D ** -0.5, O.dense_block_tokens(N, BS, 1, False))
        for name, got, w in (("dq", dq, want[0]), ("dk", dk, want[1]), ("dv", dv, want[2])):
            _close(f"{name} ({mode})", got, w)


def test_sel_bwd_config1_fp32_full_size():
    """BASELINE config 1 (fp32, q [1,1560,12,128], k/v [1,4680,12,128] ~ N(0,1)/sqrt(128),
    64-token blocks, groups of 64, top-16 from our top-k): every gradient of every head."""
    from omnimem_amd.index_topk import parallel_nsa_topk, block_pool
    gen = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn((1, L, 12, 128), generator=gen) / 128 ** 0.5 for L in (1560, 4680, 4680))
    kd = k.to(DEV)
    ids = parallel_nsa_topk(q.to(DEV), block_pool(kd, 64), 16, block_size=64, chunk_size=1560,
                            causal=False, group_size=64).cpu()
    out, lse, do, dq, dk, dv, scale = _run(q, k, v, ids, 64, 64, False, 1560, torch.float32)
    want = O.selection_attention_bwd(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                     ids.numpy(), out.double().cpu().numpy(),
                                     lse.double().cpu().numpy(), do.double().numpy(), 64, scale,
                                     O.dense_block_tokens(4680, 64, 1560, False))
    for name, got, w in (("dq", dq, want[0]), ("dk", dk, want[1]), ("dv", dv, want[2])):
        _close(name, got, w, *TOL[torch.float32])


def test_sel_bwd_negative_scale_and_determinism():
    """A negative scale flips every score; two runs give identical bits (the block -> group
    buckets are filled in (group, slot) order, not in arrival order)."""
    dtype = torch.bfloat16
    M, N, H, D, G, BS, T = 256, 1024, 2, 128, 64, 64, 8
    gen = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn((1, L, H, D), generator=gen).to(dtype) for L in (M, N, N))
    ids = _ids(gen, 1, M // G, H, T, N // BS)
    out, lse, do, dq, dk, dv, scale = _run(q, k, v, ids, G, BS, False, 1, dtype, scale=-0.05)
    want = O.selection_attention_bwd(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                     ids.numpy(), out.double().cpu().numpy(),
                                     lse.double().cpu().numpy(), do.double().numpy(), G, scale,
                                     O.dense_block_tokens(N, BS, 1, False))
    for name, got, w in (("dq", dq, want[0]), ("dk", dk, want[1]), ("dv", dv, want[2])):
        _close(name, got, w)
    _, _, _, dq2, dk2, dv2, _ = _run(q, k, v, ids, G, BS, False, 1, dtype, scale=-0.05)
    for a, b2 in ((dq, dq2), (dk, dk2), (dv, dv2)):
        assert torch.equal(a, b2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_sel_bwd_negative_scale_partial_blocks(dtype, D):
    """A negative scale with a partial last block (N = 343: block 5 holds 23 tokens) and a
    causal chunk that ends inside a block: the dQ kernel's masked keys must get P = 0 whichever
    sign the scale has (regression: masking the scores with -inf before the negative scale
    turned them into +inf)."""
    M, N, H, G, BS, T = 207, 343, 2, 64, 64, 5
    gen = torch.Generator().manual_seed(D + 3)
    q, k, v = (torch.randn((1, L, H, D), generator=gen).to(dtype) for L in (M, N, N))
    ids = _ids(gen, 1, -(-M // G), H, T, -(-N // BS), 0.1)
    for causal, chunk in ((False, 1), (True, 150)):
        out, lse, do, dq, dk, dv, scale = _run(q, k, v, ids, G, BS, causal, chunk, dtype,
                                               scale=-D ** -0.5)
        want = O.selection_attention_bwd(q.double().numpy(), k.double().numpy(),
                                         v.double().numpy(), ids.numpy(),
                                         out.double().cpu().numpy(), lse.double().cpu().numpy(),
                                         do.double().numpy(), G, scale,
                                         O.dense_block_tokens(N, BS, chunk, causal),
                                         chunk_size=chunk, causal=causal)
        for name, got, w in (("dq", dq, want[0]), ("dk", dk, want[1]), ("dv", dv, want[2])):
            assert torch.isfinite(got).all(), name
            _close(name, got, w)


def test_selection_attention_autograd_matches_exact_gradient():
    """Facade with requires_grad: loss.backward() through the autograd function, against the
    oracle's gradient of its own exact forward."""
    from omnimem_amd.selection import selection_attention
    dtype = torch.bfloat16
    M, N, H, D, G, BS, T, C = 320, 960, 2, 128, 64, 64, 5, 320
    gen = torch.Generator().manual_seed(12)
    q, k, v = (torch.randn((1, L, H, D), generator=gen).to(dtype) for L in (M, N, N))
    ids = _ids(gen, 1, M // G, H, T, N // BS, 0.1)
    w = torch.randn(q.shape, generator=gen).to(dtype)
    qd, kd, vd = (x.to(DEV).requires_grad_() for x in (q, k, v))
    o = selection_attention(qd, kd, vd, ids.to(DEV), T, BS, chunk_size=C, causal=True,
                            group_size=G)
    (o.float() * w.to(DEV).float()).sum().backward()
    fwd = O.selection_attention(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                ids.numpy(), G, D ** -0.5, O.dense_block_tokens(N, BS, C, True),
                                chunk_size=C, causal=True)
    want = O.selection_attention_bwd(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                     ids.numpy(), fwd[0], fwd[1], w.double().numpy(), G, D ** -0.5,
                                     O.dense_block_tokens(N, BS, C, True), chunk_size=C,
                                     causal=True)
    for name, t, wg in (("dq", qd, want[0]), ("dk", kd, want[1]), ("dv", vd, want[2])):
        assert t.grad is not None and t.grad.dtype == dtype
        _close(name, t.grad, wg)


def test_sel_bwd_config3_full_size():
    """BASELINE config 3 layer shape (M = N = 32760, 12 heads, groups and blocks of 64, top-16,
    causal by 4680-token chunks, ids from the fused top-k): all gradients of two sampled heads
    against the oracle, and for every head the column sums the mathematics fixes
    (sum_j dk_j = 0, sum_j dv_j = sum of d_out over the queries that see a token)."""
    from omnimem_amd.index_topk import parallel_nsa_topk, block_pool
    dtype = torch.bfloat16
    M = N = 32760
    H, D, G, BS, C = 12, 128, 64, 64, 4680
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn((1, M, H, D), generator=gen).to(dtype) for _ in range(3))
    kd = k.to(DEV)
    ids = parallel_nsa_topk(q.to(DEV), block_pool(kd, 64), 16, block_size=64, chunk_size=C,
                            causal=True, group_size=G).cpu()
    out, lse, do, dq, dk, dv, scale = _run(q, k, v, ids, G, BS, True, C, dtype, seed=3)
    dk64 = dk.double()
    assert dk64.sum(dim=1).abs().max().item() <= 2e-2 * dk64.abs().sum(dim=1).max().item()
    seen = torch.isfinite(lse).transpose(1, 2)[..., None].to(DEV)          # [1, M, H, 1]
    want_sum = (do.to(DEV).double() * seen).sum(dim=1)
    got_sum = dv.double().sum(dim=1)
    assert (got_sum - want_sum).abs().max().item() <= 2e-2 * want_sum.abs().max().item()
    for h in (0, 7):
        sl = slice(h, h + 1)
        want = O.selection_attention_bwd(
            q[:, :, sl].double().numpy(), k[:, :, sl].double().numpy(),
            v[:, :, sl].double().numpy(), ids[:, :, sl].numpy(),
            out[:, :, sl].double().cpu().numpy(), lse[:, sl].double().cpu().numpy(),
            do[:, :, sl].double().numpy(), G, scale, O.dense_block_tokens(N, BS, C, True),
            chunk_size=C, causal=True)
        for name, got, w in (("dq", dq[:, :, sl], want[0]), ("dk", dk[:, :, sl], want[1]),
                             ("dv", dv[:, :, sl], want[2])):
            _close(f"{name}[h={h}]", got, w)


def test_sel_bwd_rejects_unsupported():
    from omnimem_amd.backend import NSABackendError
    from omnimem_amd.selection import sel_bwd
    q = torch.zeros((1, 64, 1, 300), device=DEV, dtype=torch.bfloat16)
    ids = torch.zeros((1, 1, 1, 1), device=DEV, dtype=torch.int32)
    lse = torch.zeros((1, 1, 64), device=DEV)
    with pytest.raises(NSABackendError, match="head dim"):
        sel_bwd(q, q, q, ids, q, lse, q, 64, 1, 0.1, False, 64)
