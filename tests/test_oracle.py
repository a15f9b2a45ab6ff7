"""Pins of the CPU oracle against checks that do not restate it (CPU only).

Each oracle function is compared with something independent of its own formula: torch's
conversions, float64 linear algebra, closed forms of the visibility rule, the reference naive
implementation's mask formulation (nsa/naive/index_selection.py:28-36), brute-force sorting with
numpy's lexsort, and textbook attention via torch SDPA in float64.
"""
import math

import numpy as np
import pytest
import torch

from oracle import nsa_oracle as O


# ---------------------------------------------------------------- conversions
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-40, -1e-40, 3.4e38, np.inf, -np.inf], np.float32)])
    # halfway cases: bf16 mantissa boundary + exactly half an ulp
    base = rng.standard_normal(2000).astype(np.float32)
    half = (O.f32_to_bf16(base).astype(np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, half])
    ours = O.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)


def test_e4m3_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = O.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    both_nan = np.isnan(ours) & np.isnan(ref)
    np.testing.assert_array_equal(ours[~both_nan], ref[~both_nan])
    assert both_nan.sum() == 2  # 0x7f and 0xff


def test_e4m3_encode_matches_torch_within_range():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-448, 448, 50000), rng.standard_normal(50000) * 1e-2,
                        rng.standard_normal(50000) * 3]).astype(np.float32)
    # every representable value and every midpoint between neighbours (tie cases)
    vals = np.sort(np.unique(O.e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8))))
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, vals, -vals, mids, -mids]).astype(np.float32)
    ours = O.e4m3_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, ref)


def test_e4m3_encode_saturates():
    x = np.array([448.0, 449.0, 464.0, 470.0, 1e6, np.inf, -1e6, -np.inf], np.float32)
    got = O.e4m3_encode(x)
    assert list(got[:6]) == [0x7E] * 6 and list(got[6:]) == [0xFE, 0xFE]
    assert O.e4m3_encode(np.array([np.nan], np.float32))[0] & 0x7F == 0x7F


# ---------------------------------------------------------------- pooling
def test_pool_mean_exact_on_integers():
    # small integers: every fp32 partial sum is exact, so the result is the exact mean, rounded
    rng = np.random.default_rng(2)
    x = rng.integers(-64, 64, size=(2, 200, 3, 8)).astype(np.float32)
    for g, dt in ((64, "bf16"), (15, "f32"), (30, "f16")):
        got = O.pool_mean(x, g, dt)
        T = x.shape[1]
        for j in range(got.shape[1]):
            seg = x[:, j * g:min((j + 1) * g, T)].astype(np.float64)
            exact = seg.mean(axis=1)
            np.testing.assert_array_equal(got[:, j], O.round_to(exact.astype(np.float32), dt))


def test_pool_mean_close_to_torch_bf16_mean():
    rng = np.random.default_rng(3)
    x = O.round_to(rng.standard_normal((1, 256, 4, 64)).astype(np.float32), "bf16")
    got = O.pool_mean(x, 64, "bf16")
    ref = torch.from_numpy(x).to(torch.bfloat16).view(1, 4, 64, 4, 64).mean(2).float().numpy()
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - ref) <= ulp)


def test_pool_mean_ragged_tail_counts_valid_tokens():
    x = np.full((1, 70, 2, 4), 3.0, np.float32)  # 64 + 6 tokens
    got = O.pool_mean(x, 64, "f32")
    np.testing.assert_array_equal(got, np.full((1, 2, 2, 4), 3.0, np.float32))


# ---------------------------------------------------------------- scores
def test_block_scores_exact_on_small_integers():
    rng = np.random.default_rng(4)
    q = rng.integers(-8, 8, size=(1, 5, 2, 128)).astype(np.float32)
    k = rng.integers(-8, 8, size=(1, 7, 2, 128)).astype(np.float32)
    got = O.block_scores(q, k, 0.25)
    ref = np.einsum("bghd,bchd->bghc", q.astype(np.float64), k.astype(np.float64)) * 0.25
    np.testing.assert_array_equal(got, ref.astype(np.float32))


def test_block_scores_close_to_float64():
    rng = np.random.default_rng(5)
    q = O.round_to(rng.standard_normal((2, 9, 3, 128)).astype(np.float32), "bf16")
    k = O.round_to(rng.standard_normal((2, 11, 3, 128)).astype(np.float32), "bf16")
    got = O.block_scores(q, k, 128 ** -0.5)
    ref = np.einsum("bghd,bchd->bghc", q.astype(np.float64), k.astype(np.float64)) * 128 ** -0.5
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-5)


# ---------------------------------------------------------------- visibility
def test_causal_mask_matches_naive_reference_formulation():
    # nsa/naive/index_selection.py:28-36: q_chunk = q // chunk; k_chunk = (k * bs) // chunk
    for bs, chunk, MG, NC in ((64, 256, 40, 40), (30, 4680, 400, 600), (64, 4680, 200, 150)):
        m = O.Mask(block_size=bs, group_size=1, chunk_q=chunk, chunk_k=chunk, causal=1)
        vis = O.visible_matrix(m, MG, NC)
        qi = np.arange(MG)[:, None]
        ki = np.arange(NC)[None, :]
        np.testing.assert_array_equal(vis, (qi // chunk) >= ((ki * bs) // chunk))


def test_grouped_rows_use_first_token_chunk():
    # G | chunk: row g is in chunk g // (chunk / G) (the reference divides chunk_size by G)
    m = O.Mask(block_size=64, group_size=15, chunk_q=4680, chunk_k=4680, causal=1)
    vis = O.visible_matrix(m, 1000, 300)
    rows_per_chunk = 4680 // 15
    for g in (0, 311, 312, 623, 624, 999):
        qc = g // rows_per_chunk
        kc = (np.arange(300) * 64) // 4680
        np.testing.assert_array_equal(vis[g], kc <= qc)


def test_ar_window_exclusion_closed_form():
    # AR selection (causal=False, q_chunk_offset, AWE 3, progressive): from q_cid >= 3 every
    # block except chunks within distance 2 of the query chunk; before that, everything.
    bpc, n_chunks = 74, 12
    for qoff in range(0, 10):
        m = O.Mask(block_size=64, group_size=64, chunk_q=4680, chunk_k=4680, blocks_per_chunk=bpc,
                   q_chunk_offset=qoff, ex_win=3, causal=0, prog_excl=1)
        vis = O.visible_matrix(m, 74, bpc * n_chunks)
        kc = np.arange(bpc * n_chunks) // bpc
        want = np.ones_like(kc, dtype=bool) if qoff < 3 else np.abs(kc - qoff) >= 3
        for g in range(74):
            np.testing.assert_array_equal(vis[g], want)


def test_sink_exclusion_closed_form():
    m = O.Mask(block_size=64, group_size=1, chunk_q=256, chunk_k=256, ex_sink=1, causal=1)
    vis = O.visible_matrix(m, 32, 32)  # 4 blocks per chunk
    for g in range(32):
        qc = g // 256
        kc = (np.arange(32) * 64) // 256
        np.testing.assert_array_equal(vis[g], (kc <= qc) & (kc >= 1))


def test_teacher_forcing_four_cases_closed_form():
    # 4 clean chunks then 4 noisy chunks on both sides; chunk = 4 blocks, G = 1, BS = chunk/4
    chunk, bs = 64, 16
    MG = 8 * chunk
    NC = 8 * chunk // bs
    m = O.Mask(block_size=bs, group_size=1, chunk_q=chunk, chunk_k=chunk, causal=1, tf_mask=1,
               q_half=4, k_half=4)
    vis = O.visible_matrix(m, MG, NC)
    for g in range(0, MG, 7):
        qc = g // chunk
        for c in range(NC):
            kc = (c * bs) // chunk
            if qc < 4:
                want = kc < 4 and kc <= qc                      # clean sees earlier/same clean
            else:
                want = (kc < 4 and kc < qc - 4) or (kc == qc)   # noisy: strictly earlier clean + own
            assert vis[g, c] == want, (g, c)


# ---------------------------------------------------------------- selection
def _brute_topk(scores, vis, topk):
    out = np.full(scores.shape[:-1] + (topk,), -1, np.int32)
    for idx in np.ndindex(*scores.shape[:-1]):
        s = scores[idx].astype(np.float32)
        ids = np.arange(s.shape[0])
        ok = vis[idx[1]] & (s > -np.inf)  # NaN compares False
        s2 = np.where(s == 0, 0.0, s)     # -0 == +0
        order = np.lexsort((ids[ok], -s2[ok].astype(np.float64)))
        sel = ids[ok][order][:topk]
        out[idx][:len(sel)] = sel
    return out


@pytest.mark.parametrize("topk", [1, 5, 16, 64])
def test_topk_select_matches_lexsort(topk):
    rng = np.random.default_rng(10 + topk)
    B, MG, H, NC = 2, 37, 3, 300
    s = rng.integers(-6, 6, size=(B, MG, H, NC)).astype(np.float32) * 0.5  # many ties
    s[rng.random(s.shape) < 0.02] = -0.0
    s[rng.random(s.shape) < 0.02] = -np.inf
    s[rng.random(s.shape) < 0.01] = np.nan
    m = O.Mask(block_size=16, group_size=4, chunk_q=64, chunk_k=64, causal=1)
    got = O.topk_select(s, topk, m)
    want = _brute_topk(s, O.visible_matrix(m, MG, NC), topk)
    np.testing.assert_array_equal(got, want)


def test_topk_all_equal_scores_gives_lowest_ids():
    s = np.zeros((1, 3, 2, 50), np.float32)
    m = O.Mask(block_size=1, group_size=1, chunk_q=1, chunk_k=1, causal=0)
    got = O.topk_select(s, 16, m)
    assert (got == np.arange(16)).all()


def test_topk_fewer_visible_than_k_pads_minus_one():
    s = np.random.default_rng(0).standard_normal((1, 2, 1, 10)).astype(np.float32)
    m = O.Mask(block_size=64, group_size=64, chunk_q=192, chunk_k=192, causal=1)
    got = O.topk_select(s, 8, m)  # row 0: chunk 0 -> blocks 0..2 visible only
    assert sorted(got[0, 0, 0, :3].tolist()) == [0, 1, 2] and (got[0, 0, 0, 3:] == -1).all()


def test_topk_select_large_known_answer():
    """Past topk = 128 the reference ranks raw order codes (topk.cu:163-166) with hidden columns
    as key 0 / value -1, sorted stably (topk.cu:741-807).  Row 6 of a causal mask with one-column
    chunks sees columns 0..6; the expected order is read off those rules: +NaN (code 0xffc00000)
    first, then 2.0, 1.0, +0 above -0, -inf (code 0x007fffff), then the code-0 tie in column
    order: the visible -NaN 0xffffffff (column 6) and the hidden column 7, which gives -1, then
    -1 past NC."""
    m = O.Mask(block_size=1, group_size=1, chunk_q=1, chunk_k=1, causal=1)
    s = np.zeros((1, 8, 1, 8), np.float32)
    row = np.array([1.0, 0.0, -np.inf, -0.0, 0.0, 2.0, 0.0, 5.0], np.float32)
    bits = row.view(np.uint32)
    bits[1] = 0x7FC00000  # +NaN
    bits[6] = 0xFFFFFFFF  # -NaN with every mantissa bit set: code 0
    s[0, 6, 0] = row
    got = O.topk_select_large(s, 10, m)[0, 6, 0]
    np.testing.assert_array_equal(got, [1, 5, 0, 4, 3, 2, 6, -1, -1, -1])


@pytest.mark.parametrize("topk", [5, 60, 400])
def test_topk_select_large_agrees_with_the_small_rule_on_finite_scores(topk):
    """On finite scores without -0 both rules order by (score desc, id asc) over the visible
    columns: the numpy sort of path B and the C qsort of path A agree wherever the row has at
    least topk visible columns, and path B pads with -1 (hidden columns) where it has fewer."""
    rng = np.random.default_rng(20 + topk)
    B, MG, H, NC = 1, 37, 2, 300
    s = rng.integers(-6, 6, size=(B, MG, H, NC)).astype(np.float32) * 0.5  # many ties
    s[s == 0] = 0.25
    m = O.Mask(block_size=16, group_size=4, chunk_q=64, chunk_k=64, causal=1)
    np.testing.assert_array_equal(O.topk_select_large(s, topk, m), O.topk_select(s, topk, m))


# ---------------------------------------------------------------- attention
def _sdpa64(q, k, v, mask):
    qt, kt, vt = (torch.from_numpy(np.asarray(a, np.float64)) for a in (q, k, v))
    return torch.nn.functional.scaled_dot_product_attention(
        qt[None], kt[None], vt[None], attn_mask=torch.from_numpy(mask)[None]).numpy()[0]


def test_selection_single_block_is_plain_attention():
    rng = np.random.default_rng(20)
    B, M, N, H, D, BS = 1, 8, 256, 2, 32, 64
    q, k, v = (rng.standard_normal((B, L, H, D)) for L in (M, N, N))
    ids = np.full((B, M, H, 1), 2, np.int32)
    out, lse = O.selection_attention(q, k, v, ids, 1, D ** -0.5,
                                     O.dense_block_tokens(N, BS, 1, False))
    for h in range(H):
        ref = _sdpa64(q[0, :, h], k[0, 128:192, h], v[0, 128:192, h], np.ones((M, 64), bool))
        np.testing.assert_allclose(out[0, :, h], ref, atol=1e-12)
        s = (q[0, :, h] @ k[0, 128:192, h].T) * D ** -0.5
        np.testing.assert_allclose(lse[0, h], np.log(np.exp(s).sum(1)), atol=1e-12)


def test_selection_causal_partial_blocks_match_masked_sdpa():
    rng = np.random.default_rng(21)
    B, M, N, H, D, BS, C, G = 1, 100, 100, 1, 16, 16, 40, 10
    q, k, v = (rng.standard_normal((B, L, H, D)) for L in (M, N, N))
    MG = M // G
    ids = np.stack([rng.permutation(7)[:4] for _ in range(MG)]).astype(np.int32)[None, :, None]
    out, _ = O.selection_attention(q, k, v, ids, G, D ** -0.5,
                                   O.dense_block_tokens(N, BS, C, True), chunk_size=C, causal=True)
    for g in range(MG):
        qc = (g * G) // C
        allowed = np.zeros(N, bool)
        for bid in ids[0, g, 0]:
            t = np.arange(bid * BS, min(N, bid * BS + BS))
            allowed[t[(t // C) <= qc]] = True
        rows = slice(g * G, (g + 1) * G)
        if not allowed.any():
            assert np.all(out[0, rows, 0] == 0)
            continue
        mask = np.broadcast_to(allowed, (G, N)).copy()
        ref = _sdpa64(q[0, rows, 0], k[0, :, 0], v[0, :, 0], mask)
        np.testing.assert_allclose(out[0, rows, 0], ref, atol=1e-12)


def test_selection_no_visible_token_gives_zero_and_neg_inf():
    q = np.ones((1, 4, 1, 16))
    k = v = np.ones((1, 64, 1, 16))
    ids = np.full((1, 1, 1, 3), -1, np.int32)
    out, lse = O.selection_attention(q, k, v, ids, 4, 0.25, O.dense_block_tokens(64, 64, 1, False))
    assert np.all(out == 0) and np.all(np.isneginf(lse))


def _bwd_case(seed):
    """Tiny causal case with a ragged last group, a partial tail block, -1 and out-of-range ids,
    a duplicated id and a group whose blocks are all invisible."""
    rng = np.random.default_rng(seed)
    B, M, N, H, D, BS, C, G = 1, 11, 22, 2, 4, 4, 8, 3
    q, k, v = (rng.standard_normal((B, L, H, D)) for L in (M, N, N))
    MG = -(-M // G)
    ids = rng.integers(0, 6, size=(B, MG, H, 3)).astype(np.int32)
    ids[0, 1, 0] = [0, 0, 1]        # duplicate: counted twice
    ids[0, 2, 1, 2] = -1
    ids[0, 3, 0, 1] = 9             # out of range: skipped
    ids[0, 0, 1] = [5, 4, 3]        # group 0 (chunk 0) sees none of these
    return q, k, v, ids, dict(group_size=G, scale=-0.7,
                              block_tokens=O.dense_block_tokens(N, BS, C, True), chunk_size=C,
                              causal=True)


def test_selection_bwd_matches_finite_differences():
    q, k, v, ids, kw = _bwd_case(30)
    w = np.random.default_rng(31).standard_normal(q.shape)

    def loss(q_, k_, v_):
        return float((O.selection_attention(q_, k_, v_, ids, **kw)[0] * w).sum())

    out, lse = O.selection_attention(q, k, v, ids, **kw)
    assert np.isneginf(lse[0, 1, 0:3]).all()   # the invisible group really is empty
    dq, dk, dv, _ = O.selection_attention_bwd(q, k, v, ids, out, lse, w, **kw)
    eps = 1e-6
    for x, g in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(x)
        for i in np.ndindex(x.shape):
            x0 = x[i]
            x[i] = x0 + eps
            lp = loss(q, k, v)
            x[i] = x0 - eps
            lm = loss(q, k, v)
            x[i] = x0
            num[i] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(g, num, atol=1e-7, rtol=1e-6)
    assert np.abs(dk).sum() > 0 and np.abs(dq).sum() > 0


def test_selection_bwd_matches_torch_autograd_of_masked_softmax():
    """Same gradients from torch autograd (float64) of a per-group masked softmax attention."""
    rng = np.random.default_rng(32)
    B, M, N, H, D, BS, C, G = 1, 40, 50, 2, 8, 8, 20, 5
    q, k, v = (rng.standard_normal((B, L, H, D)) for L in (M, N, N))
    MG = M // G
    ids = np.stack([np.stack([rng.permutation(7)[:3] for _ in range(H)]) for _ in range(MG)])
    ids = ids.astype(np.int32)[None]
    scale = 0.3
    kw = dict(group_size=G, scale=scale, block_tokens=O.dense_block_tokens(N, BS, C, True),
              chunk_size=C, causal=True)
    out, lse = O.selection_attention(q, k, v, ids, **kw)
    w = rng.standard_normal(q.shape)
    dq, dk, dv, _ = O.selection_attention_bwd(q, k, v, ids, out, lse, w, **kw)

    qt, kt, vt = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    total = 0.0
    for g in range(MG):
        for h in range(H):
            allowed = np.zeros(N, bool)
            for bid in ids[0, g, h]:
                t = np.arange(bid * BS, min(N, bid * BS + BS))
                allowed[t[(t // C) <= (g * G) // C]] = True
            if not allowed.any():
                continue
            rows = slice(g * G, (g + 1) * G)
            s = (qt[0, rows, h] @ kt[0, :, h].T) * scale
            s = s.masked_fill(~torch.from_numpy(allowed)[None], float("-inf"))
            o = torch.softmax(s, dim=-1) @ vt[0, :, h]
            total = total + (o * torch.from_numpy(w[0, rows, h])).sum()
    total.backward()
    for mine, t in ((dq, qt), (dk, kt), (dv, vt)):
        np.testing.assert_allclose(mine, t.grad.numpy(), atol=1e-12)


def test_selection_bwd_column_sums():
    """sum_j dS_mj = 0 for every query (delta is the P-weighted mean of dP), so dk sums to 0
    over keys; P rows sum to 1, so dv sums to the d_out of the queries that see a token."""
    q, k, v, ids, kw = _bwd_case(33)
    out, lse = O.selection_attention(q, k, v, ids, **kw)
    w = np.random.default_rng(34).standard_normal(q.shape)
    _, dk, dv, delta = O.selection_attention_bwd(q, k, v, ids, out, lse, w, **kw)
    np.testing.assert_allclose(dk.sum(axis=1), 0.0, atol=1e-12)
    seen = np.isfinite(lse).transpose(0, 2, 1)[..., None]           # [B, M, H, 1]
    np.testing.assert_allclose(dv.sum(axis=1), (w * seen).sum(axis=1), atol=1e-12)
    np.testing.assert_allclose(delta, np.einsum("bmhd,bmhd->bhm", out, w), atol=0)


def test_quantize_pages_error_bound_and_amax():
    rng = np.random.default_rng(22)
    x = (rng.standard_t(4, size=(64, 128)) * 3).astype(np.float32)
    codes, scale = O.quantize_pages(x, 64)
    xh = O.dequantize_pages(codes, scale)
    amax = np.abs(x).max()
    assert math.isclose(float(scale), float(amax) / 448.0, rel_tol=1e-6)
    assert np.abs(xh).max() <= np.float32(448.0) * scale * (1 + 1e-6)
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 in the normal range, abs error <= half
    # the subnormal step (2^-10 * scale) below it
    err = np.abs(xh - x)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, 2.0 ** -10 * scale) * (1 + 1e-5)
    assert np.all(err <= bound)


def test_quantize_zero_page():
    codes, scale = O.quantize_pages(np.zeros((64, 8), np.float32), 64)
    assert scale == 1.0 and not codes.any()


# ---------------------------------------------------------------- CPU baseline formulation
def test_cpu_baseline_chunked_matches_float64_oracle():
    """The timed CPU baseline (reference naive formulation, fp32) agrees with the float64
    oracle, including -1 ids, a partial last block and the chunk-causal mask."""
    from oracle import cpu_baseline as CB
    rng = np.random.default_rng(30)
    B, M, N, H, D, BS, G, C, T = 1, 96, 200, 2, 32, 16, 32, 64, 5
    q, k, v = (rng.standard_normal((B, L, H, D)).astype(np.float32) for L in (M, N, N))
    MG = M // G
    ids = np.stack([rng.permutation(13)[:T] for _ in range(MG * H)]).astype(np.int32)
    ids = ids.reshape(B, MG, H, T)
    ids[0, 1, 0, 2] = -1
    want, _ = O.selection_attention(q, k, v, ids, G, D ** -0.5, O.dense_block_tokens(N, BS, C, True),
                                    chunk_size=C, causal=True)
    # the naive path masks per token position; the kernel masks by the group's chunk, so check
    # groups that do not straddle a chunk boundary (G divides C here)
    tok = CB.inflate_indices(torch.from_numpy(ids).long(), BS)
    tok = tok.repeat_interleave(G, dim=1)
    got = CB.select_attention_chunked(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                      tok, scale=D ** -0.5, causal=True, chunk_size=C).numpy()
    np.testing.assert_allclose(got, want, atol=2e-5)


def test_cpu_baseline_topk_matches_oracle_without_ties():
    from oracle import cpu_baseline as CB
    rng = np.random.default_rng(31)
    q = rng.standard_normal((1, 20, 2, 64)).astype(np.float32)
    k = rng.standard_normal((1, 30, 2, 64)).astype(np.float32)
    got = CB.topk_scores(torch.from_numpy(q), torch.from_numpy(k), 8, causal=True, chunk_size=256,
                         block_size=64, group_size=64).numpy()
    want = O.topk(q, k, 8, 64 ** -0.5, O.Mask(block_size=64, group_size=64, chunk_q=256,
                                              chunk_k=256, causal=1))
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------- reference LRU model
def test_reference_lru_model_matches_closed_form():
    """An LRU of capacity C holds the C most recently touched distinct keys; the model's
    per-(layer, head) OrderedDict must agree with that closed form on random touch streams."""
    from oracle.lru_model import ReferenceLRU, lru_contents_bruteforce
    rng = np.random.default_rng(40)
    for cap in (1, 3, 7):
        m = ReferenceLRU(1, 2, cap)
        streams = {0: [], 1: []}
        for _ in range(300):
            h, c = int(rng.integers(0, 2)), int(rng.integers(0, 12))
            m.touch(0, h, c)
            streams[h].append(c)
        for h in (0, 1):
            assert list(m.lru[(0, h)].keys()) == lru_contents_bruteforce(streams[h], cap)


def test_reference_lru_flush_offloads_marked_outside_lru_and_window():
    from oracle.lru_model import ReferenceLRU
    m = ReferenceLRU(1, 1, 2, window=1, sink=1)
    for c in range(5):
        m.write(0, c)
    m.flush()
    # LRU = {3, 4}; sink chunk 0 and window chunk 4 protected; 1, 2 offloaded
    assert m.resident() == {(0, 0, 0), (0, 0, 3), (0, 0, 4)}
