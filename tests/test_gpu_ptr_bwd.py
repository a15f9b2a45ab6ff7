"""GPU parity of the pointer-table selection backward (``sel_bwd_ptr``) against the float64 oracle.

The K / V blocks live in per-head chunk tensors [B, chunk_len, D] reached through int64 base
tables, as in the reference's padded-pointer training path (cuda_backend/csrc/
selection_bwd.cu:1409-1529, padded_ptr/kernels/select_bwd.py:564-711, padded_ptr/autograd.py).
The oracle (oracle.nsa_oracle.selection_attention_bwd, pinned in tests/test_oracle.py by finite
differences and torch autograd) runs on the equivalent dense layout: head h's chunk c holds dense
tokens [c*chunk_len, (c+1)*chunk_len), so block id bid is dense tokens [bid*bs, bid*bs + bs).  Ids
a head cannot resolve (negative, at or past its n_blocks bound, or in a chunk whose base is 0) are
-1 for the oracle.  It is fed the same bf16 inputs and the GPU forward's own (out, lse), so the
comparison isolates the backward kernels.

Tolerances as for the dense backward: per gradient tensor g with oracle value r, max|g - r| <=
2e-2 * max|r| and mean|g - r| <= 5e-3 * mean|r| (16-bit MFMA operands for P and dS, fp32
accumulation); delta (fp32 dot products of bf16 rows) within 1e-5 * max|delta|.  Write rules
checked exactly: every block a head resolves is stored (0 when no group lists it), nothing is
written for a block it cannot resolve, and compute_dkv=False writes no scratch at all.
"""
import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
SENTINEL = 7.0


def _close(name, got, want, mx=2e-2, mean=5e-3):
    g = np.asarray(got, dtype=np.float64)
    err = np.abs(g - want)
    scale_max = max(np.abs(want).max(), 1e-30)
    scale_mean = max(np.abs(want).mean(), 1e-30)
    assert err.max() <= mx * scale_max, f"{name}: max-abs {err.max():.3e} > {mx} x {scale_max:.3e}"
    assert err.mean() <= mean * scale_mean, (
        f"{name}: mean-abs {err.mean():.3e} > {mean} x {scale_mean:.3e}")


def _chunk(gen, B, C, D, scale, shift=0, dtype=torch.bfloat16):
    """[B, C, D] chunk on the GPU; shift > 0 makes it a view `shift` elements into a larger
    allocation (a base address that is only 2-byte aligned when shift is odd)."""
    x = (torch.randn((B * C * D + 8,), generator=gen) * scale).to(dtype).to(DEV)
    return x[shift:shift + B * C * D].view(B, C, D)


class Setup:
    """Per-head chunks, base tables, ids and the forward of one case."""

    def __init__(self, seed, B, M, H, D, G, BS, C, T, n_chunks, shift=0, dk_shift=0,
                 missing=(), minus=0.1, beyond=True, dup=False, block_level=False):
        gen = torch.Generator().manual_seed(seed)
        self.B, self.M, self.H, self.D, self.G, self.BS, self.C, self.T = B, M, H, D, G, BS, C, T
        self.n_chunks = list(n_chunks)
        self.maxc = max(self.n_chunks)
        self.bpc = C // BS
        self.block_level = block_level
        self.k = [[_chunk(gen, B, C, D, 0.3, shift if (h + c) % 2 == 0 else 0)
                   for c in range(self.n_chunks[h])] for h in range(H)]
        self.v = [[_chunk(gen, B, C, D, 1.0, shift if (h + c) % 2 == 1 else 0)
                   for c in range(self.n_chunks[h])] for h in range(H)]
        self.missing = set(missing)  # (h, c) pairs whose base is 0
        # fp32 dK / dV scratch, pre-filled with a sentinel
        self.dk = [[_chunk(gen, B, C, D, 0.0, dk_shift, torch.float32).fill_(SENTINEL)
                    for c in range(self.n_chunks[h])] for h in range(H)]
        self.dv = [[_chunk(gen, B, C, D, 0.0, dk_shift, torch.float32).fill_(SENTINEL)
                    for c in range(self.n_chunks[h])] for h in range(H)]
        MG = -(-M // G)
        hi = self.maxc * self.bpc + (self.bpc if beyond else 0)
        ids = torch.randint(-1 if minus else 0, hi, (B, MG, H, T), generator=gen,
                            dtype=torch.int32)
        if minus:
            ids[torch.rand(ids.shape, generator=gen) < minus] = -1
        if dup:
            ids[..., 1] = ids[..., 0]
        self.ids = ids
        self.nblk = torch.tensor([n * self.bpc for n in self.n_chunks], dtype=torch.int32)
        self.q = (torch.randn((B, M, H, D), generator=gen) * 0.3).to(torch.bfloat16)
        self.do = torch.randn((B, M, H, D), generator=gen).to(torch.bfloat16)
        self.scale = D ** -0.5

    def table(self, chunks):
        """[H, width] addresses: chunk level (width maxc), or block level (width maxc*bpc, one
        entry per block, blocks_per_chunk = 0)."""
        if self.block_level:
            t = torch.zeros((self.H, self.maxc * self.bpc), dtype=torch.int64)
            for h in range(self.H):
                for c, x in enumerate(chunks[h]):
                    if (h, c) in self.missing:
                        continue
                    for j in range(self.bpc):
                        t[h, c * self.bpc + j] = x[0, j * self.BS].data_ptr()
        else:
            t = torch.zeros((self.H, self.maxc), dtype=torch.int64)
            for h in range(self.H):
                for c, x in enumerate(chunks[h]):
                    if (h, c) not in self.missing:
                        t[h, c] = x.data_ptr()
        return t.to(DEV)

    def bases(self):
        return self.table(self.k), self.table(self.v), self.table(self.dk), self.table(self.dv)

    def geometry(self):
        """(blocks_per_chunk, batch bytes kv / dkv, in-chunk block bytes kv / dkv)."""
        if self.block_level:
            return 0, self.C * self.D * 2, self.C * self.D * 4, 0, 0
        return (self.bpc, self.C * self.D * 2, self.C * self.D * 4, self.BS * self.D * 2,
                self.BS * self.D * 4)

    def oracle_ids(self):
        """-1 for every id its head cannot resolve."""
        ids = self.ids.numpy().copy()
        for h in range(self.H):
            x = ids[:, :, h]
            bad = (x < 0) | (x >= self.nblk[h].item())
            for (hh, c) in self.missing:
                if hh == h:
                    bad |= (x // self.bpc) == c
            x[bad] = -1
        return ids

    def dense(self, chunks):
        out = torch.zeros((self.B, self.maxc * self.C, self.H, self.D), dtype=torch.float64)
        for h in range(self.H):
            for c, x in enumerate(chunks[h]):
                out[:, c * self.C:(c + 1) * self.C, h] = x.double().cpu()
        return out.numpy()


def _forward(s, base_k, base_v, nb):
    from omnimem_amd.padded_ptr import build_ptr_table, launch_ptr_fwd
    bpc, bkv, _, icb, _ = s.geometry()
    pk, pv = build_ptr_table(s.ids.to(DEV), base_k, base_v, nb, bkv, bpc, icb)
    out, lse = launch_ptr_fwd(s.q.to(DEV), pk, pv, s.BS, s.G, s.D, 1, s.scale, True)
    return pk, pv, out, lse


def _backward(s, pk, pv, out, lse, bases, nb, compute_dkv=True):
    from omnimem_amd.padded_ptr import launch_ptr_bwd
    bpc, bkv, bdkv, icb, icbd = s.geometry()
    bk, bv, bdk, bdv = bases
    dq, delta = launch_ptr_bwd(
        q=s.q.to(DEV), out=out, lse=lse, d_out=s.do.to(DEV), block_indices=s.ids.to(DEV),
        ptr_table_k=pk, ptr_table_v=pv, block_base_ptrs_k=bk, block_base_ptrs_v=bv,
        block_base_ptrs_dk=bdk, block_base_ptrs_dv=bdv, n_blocks_per_head=nb,
        block_size=s.BS, group_size=s.G, batch_stride_kv_bytes=bkv,
        batch_stride_dkv_bytes=bdkv, stride_bn=s.D, stride_bd=1, stride_dbn=s.D, stride_dbd=1,
        blocks_per_chunk=bpc, in_chunk_block_bytes_kv=icb, in_chunk_block_bytes_dkv=icbd,
        softmax_scale=s.scale, compute_dkv=compute_dkv)
    torch.cuda.synchronize()
    return dq, delta


def _check(s, out, lse, dq, delta):
    ids_o = s.oracle_ids()
    N = s.maxc * s.C
    want = O.selection_attention_bwd(s.q.double().numpy(), s.dense(s.k), s.dense(s.v), ids_o,
                                     out.double().cpu().numpy(), lse.double().cpu().numpy(),
                                     s.do.double().numpy(), s.G, s.scale,
                                     O.dense_block_tokens(N, s.BS, 1, False))
    _close("dq", dq.double().cpu().numpy(), want[0])
    d = delta.double().cpu().numpy()
    assert np.abs(d - want[3]).max() <= 1e-5 * max(np.abs(want[3]).max(), 1e-30)
    for name, scratch, w in (("dk", s.dk, want[1]), ("dv", s.dv, want[2])):
        got = np.zeros_like(w)
        for h in range(s.H):
            for c in range(s.n_chunks[h]):
                x = scratch[h][c].double().cpu().numpy()
                if (h, c) in s.missing:
                    assert np.all(x == SENTINEL), f"{name}: unresolvable chunk ({h}, {c}) written"
                    continue
                assert not np.any(x == SENTINEL), f"{name}: chunk ({h}, {c}) not fully stored"
                got[:, c * s.C:(c + 1) * s.C, h] = x
        _close(name, got, w)


CASES = [
    # seed, B, M, H, D, G, BS, C, T, n_chunks, shift, dk_shift, missing, dup, block_level
    (1, 1, 150, 2, 128, 15, 30, 4680, 8, (3, 2), 0, 0, (), False, False),    # reference AR shape
    (2, 1, 300, 2, 128, 150, 30, 1560, 8, (2, 3), 0, 0, ((1, 0),), True, False),  # 4-wave groups
    (3, 2, 256, 2, 64, 64, 64, 512, 4, (2, 2), 0, 0, (), False, False),       # D 64, B 2
    (4, 1, 120, 2, 128, 15, 30, 480, 6, (2, 1), 1, 1, ((0, 1),), False, False),  # misaligned
    (5, 1, 128, 3, 96, 32, 32, 256, 5, (2, 2, 1), 0, 0, (), True, False),    # VALU (D 96)
    (6, 1, 64, 2, 128, 64, 16, 128, 6, (2, 2), 0, 0, ((1, 1),), False, True),  # block-level bases
]


@pytest.mark.parametrize("case", CASES, ids=[f"case{c[0]}" for c in CASES])
def test_sel_bwd_ptr_matches_oracle(case):
    seed, B, M, H, D, G, BS, C, T, n_chunks, shift, dk_shift, missing, dup, blk = case
    print(f"sel_bwd_ptr case {case}", flush=True)
    s = Setup(seed, B, M, H, D, G, BS, C, T, n_chunks, shift, dk_shift, missing, dup=dup,
              block_level=blk)
    bases = s.bases()
    nb = s.nblk.to(DEV)
    pk, pv, out, lse = _forward(s, bases[0], bases[1], nb)
    dq, delta = _backward(s, pk, pv, out, lse, bases, nb)
    _check(s, out, lse, dq, delta)


@pytest.mark.parametrize("seed", range(16))
def test_sel_bwd_ptr_sweep(seed):
    """Seeded random geometries for the pointer path, forward and backward: batch 1 or 2, head
    dims 64 / 96 / 128, groups of 8..150 queries, 16..64-token blocks, ragged chunk counts per
    head, 2-byte aligned bases, unresolvable chunks, ids past a head's bound, duplicates, chunk-
    or block-level base tables."""
    r = np.random.default_rng(4400 + seed)
    B, H = int(r.integers(1, 3)), int(r.integers(1, 4))
    D = int(r.choice([64, 128, 128, 96]))
    G = int(r.choice([8, 15, 32, 64, 150]))
    BS = int(r.choice([16, 30, 32, 64]))
    C = BS * int(r.integers(1, 9))
    n_chunks = tuple(int(x) for x in r.integers(1, 4, size=H))
    M = G * int(r.integers(1, max(2, 320 // G) + 1))  # the pointer path takes whole groups
    T = int(r.integers(1, 9))
    shift, dk_shift = int(r.integers(0, 2)), int(r.integers(0, 2))
    missing = tuple((h, c) for h in range(H) for c in range(n_chunks[h]) if r.random() < 0.15)
    dup, blk = bool(r.integers(0, 2)) and T > 1, bool(r.integers(0, 2))
    case = (seed, B, M, H, D, G, BS, C, T, n_chunks, shift, dk_shift, missing, dup, blk)
    print(f"sel_bwd_ptr sweep case {case}", flush=True)
    s = Setup(4400 + seed, B, M, H, D, G, BS, C, T, n_chunks, shift, dk_shift, missing, dup=dup,
              block_level=blk)
    bases = s.bases()
    nb = s.nblk.to(DEV)
    pk, pv, out, lse = _forward(s, bases[0], bases[1], nb)
    dq, delta = _backward(s, pk, pv, out, lse, bases, nb)
    _check(s, out, lse, dq, delta)


def test_sel_bwd_ptr_dq_only_and_unbounded():
    """compute_dkv=False gives the same dq and writes no scratch; an empty n_blocks_per_head
    drops the per-head bound of the dK / dV index (every id below the table's width reaches its
    block), as the reference's optional bound."""
    s = Setup(11, 1, 150, 2, 128, 15, 30, 1560, 8, (2, 2), beyond=False)
    bases = s.bases()
    nb = s.nblk.to(DEV)
    pk, pv, out, lse = _forward(s, bases[0], bases[1], nb)
    dq0, delta0 = _backward(s, pk, pv, out, lse, bases, nb, compute_dkv=False)
    for h in range(s.H):
        for c in range(s.n_chunks[h]):
            assert torch.all(s.dk[h][c] == SENTINEL) and torch.all(s.dv[h][c] == SENTINEL)
    dq1, delta1 = _backward(s, pk, pv, out, lse, bases, torch.empty(0, dtype=torch.int32,
                                                                     device=DEV))
    assert torch.equal(dq0, dq1) and torch.equal(delta0, delta1)
    _check(s, out, lse, dq1, delta1)


def test_sel_bwd_ptr_rows_without_keys():
    """A group whose every id is -1 has lse = -inf: dq is 0 for its rows and it adds nothing to
    dK / dV."""
    s = Setup(12, 1, 120, 2, 128, 15, 30, 480, 4, (2, 2), minus=0.0)
    s.ids[:, 3] = -1
    bases = s.bases()
    nb = s.nblk.to(DEV)
    pk, pv, out, lse = _forward(s, bases[0], bases[1], nb)
    dq, delta = _backward(s, pk, pv, out, lse, bases, nb)
    assert torch.count_nonzero(dq[:, 45:60]) == 0
    _check(s, out, lse, dq, delta)


def test_padded_ptr_train_gradients_match_oracle():
    """selection_attention_padded_ptr_train (lists of chunk tensors) and _train_fast: gradients of
    q and of every K / V chunk tensor against the float64 oracle, on the reference AR geometry."""
    from omnimem_amd.padded_ptr import (selection_attention_padded_ptr_train,
                                        selection_attention_padded_ptr_train_fast)
    gen = torch.Generator().manual_seed(21)
    B, M, H, D, G, BS, C, T = 1, 150, 2, 128, 15, 30, 1560, 8
    n_chunks = [3, 2]
    bpc = C // BS
    k = [[(torch.randn((B, C, D), generator=gen) * 0.3).to(torch.bfloat16).to(DEV).requires_grad_()
          for _ in range(n)] for n in n_chunks]
    v = [[torch.randn((B, C, D), generator=gen).to(torch.bfloat16).to(DEV).requires_grad_()
          for _ in range(n)] for n in n_chunks]
    q = (torch.randn((B, M, H, D), generator=gen) * 0.3).to(torch.bfloat16).to(DEV)
    q.requires_grad_()
    ids = torch.randint(0, max(n_chunks) * bpc, (B, M // G, H, T), generator=gen,
                        dtype=torch.int32)
    do = torch.randn((B, M, H, D), generator=gen).to(torch.bfloat16)

    out = selection_attention_padded_ptr_train(q, k, v, ids.to(DEV), BS, G, C)
    out.backward(do.to(DEV))
    grads = [q.grad.clone()] + [x.grad.clone() for row in k for x in row] + \
            [x.grad.clone() for row in v for x in row]

    for t in [q] + [x for row in k + v for x in row]:
        t.grad = None
    strides = {"batch_stride_bytes": C * D * 2, "token_stride_bytes": D * 2, "stride_bn": D,
               "stride_bd": 1, "chunk_len": C}
    out2 = selection_attention_padded_ptr_train_fast(
        q, ids.to(DEV), BS, G, C, max(n_chunks),
        torch.tensor(n_chunks, dtype=torch.int32, device=DEV), strides,
        tuple(x for row in k for x in row), tuple(x for row in v for x in row), n_chunks)
    out2.backward(do.to(DEV))
    assert torch.equal(out, out2)
    grads2 = [q.grad] + [x.grad for row in k for x in row] + [x.grad for row in v for x in row]
    for a, b in zip(grads, grads2):
        assert torch.equal(a, b)

    # oracle on the dense layout; head 1 has 2 chunks, so its ids >= 2 * bpc select nothing
    ids_o = ids.numpy().copy()
    for h in range(H):
        x = ids_o[:, :, h]
        x[x >= n_chunks[h] * bpc] = -1
    N = max(n_chunks) * C

    def dense(chunks):
        d = torch.zeros((B, N, H, D), dtype=torch.float64)
        for h, row in enumerate(chunks):
            for c, x in enumerate(row):
                d[:, c * C:(c + 1) * C, h] = x.detach().double().cpu()
        return d.numpy()

    kd, vd = dense(k), dense(v)
    want_o, want_l = O.selection_attention(q.detach().double().cpu().numpy(), kd, vd, ids_o, G,
                                           D ** -0.5, O.dense_block_tokens(N, BS, 1, False))
    _close("out", out.detach().double().cpu().numpy(), want_o)
    want = O.selection_attention_bwd(q.detach().double().cpu().numpy(), kd, vd, ids_o,
                                     out.detach().double().cpu().numpy(), want_l,
                                     do.double().numpy(), G, D ** -0.5,
                                     O.dense_block_tokens(N, BS, 1, False))
    _close("dq", grads[0].double().cpu().numpy(), want[0])
    i = 1
    for name, w in (("dk", want[1]), ("dv", want[2])):
        got = np.zeros_like(w)
        for h in range(H):
            for c in range(n_chunks[h]):
                got[:, c * C:(c + 1) * C, h] = grads[i].double().cpu().numpy()
                i += 1
        _close(name, got, w)


def test_sel_bwd_ptr_rejects_bad_arguments():
    from omnimem_amd.backend import NSABackendError
    s = Setup(31, 1, 60, 2, 128, 15, 30, 480, 4, (1, 1))
    bases = s.bases()
    nb = s.nblk.to(DEV)
    pk, pv, out, lse = _forward(s, bases[0], bases[1], nb)
    bk, bv, bdk, bdv = bases
    with pytest.raises(NSABackendError):  # base tables of different shapes
        _backward(s, pk, pv, out, lse, (bk, bv, bdk[:, :0], bdv), nb)
    with pytest.raises(NSABackendError):  # n_blocks_per_head of the wrong length
        _backward(s, pk, pv, out, lse, bases, nb[:1])
    with pytest.raises(NSABackendError):  # fp16 queries
        from omnimem_amd.padded_ptr import launch_ptr_bwd
        launch_ptr_bwd(q=s.q.half().to(DEV), out=out, lse=lse, d_out=s.do.to(DEV),
                       block_indices=s.ids.to(DEV), ptr_table_k=pk, ptr_table_v=pv,
                       block_base_ptrs_k=bk, block_base_ptrs_v=bv, block_base_ptrs_dk=bdk,
                       block_base_ptrs_dv=bdv, n_blocks_per_head=nb, block_size=30,
                       group_size=15, batch_stride_kv_bytes=0, batch_stride_dkv_bytes=0,
                       stride_bn=128, stride_bd=1)
