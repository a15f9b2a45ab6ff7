"""CPU oracle of the NSA selection path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker of (or the CPU baseline beside) the HIP path.  The product
package ``omnimem_amd`` never imports it.

What it restates, with the reference lines it follows (paths under src/omnimem/ of
wuyushuwys/OmniMem):

* ``pool_mean``            -- mean pooling of consecutive tokens in the input dtype
                              (models/transformers/causal_wan_nsa_model.py:408;
                              nsa/ops/index_topk.py:76): fp32 sum in ascending token order, one
                              division by the count, one round-to-nearest-even.
* ``block_scores``         -- fp32 q.k * scale (nsa/ops/index_topk.py:99; topk.cu:389), with the
                              fixed fmaf order of nsa_oracle.c.
* ``topk_select``          -- visibility (cuda_backend/csrc/topk.cu:36-97) and ordering
                              (topk.cu:3,100-102; ops.h:11-12), in nsa_oracle.c.
* ``topk_select_large``    -- the rule past topk = 128 (path B, topk.cu:741-807): raw order codes,
                              hidden columns as key 0 / value -1, a stable descending sort.
* ``selection_attention``  -- dense selection attention (cuda_backend/csrc/common.cuh:158-190,
                              :327-332; selection_fwd.cu:1-3,218) as a float64 softmax over the
                              gathered token set; duplicated ids count twice, as in the kernel.
* ``selection_attention_bwd`` -- its backward from (out, lse, d_out): delta, P recomputed from
                              LSE, dS, dQ, dK, dV (cuda_backend/csrc/selection_bwd.cu:18-306).
* ``e4m3_encode/decode``   -- OCP fp8 e4m3fn with round-to-nearest-even and saturation (new: the
                              reference has no fp8 cache).
* ``quantize_pages``       -- per (page, head) amax/448 scaling of the fp8 cache.

How each is pinned independently of itself is in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, fields

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libnsa_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile nsa_oracle.c with gcc into oracle/_build/ (plain IEEE fp32, no contraction)."""
    src = os.path.join(_HERE, "nsa_oracle.c")
    if not force and os.path.exists(_LIB_PATH) and os.path.getmtime(_LIB_PATH) >= os.path.getmtime(src):
        return _LIB_PATH
    os.makedirs(os.path.dirname(_LIB_PATH), exist_ok=True)
    tmp = _LIB_PATH + f".tmp{os.getpid()}"
    subprocess.check_call(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
                           "-std=c11", src, "-o", tmp, "-lm"])
    os.replace(tmp, _LIB_PATH)
    return _LIB_PATH


class _Mask(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "block_size", "group_size", "chunk_q", "chunk_k", "blocks_per_chunk", "q_chunk_offset",
        "q_half", "k_half", "ex_win", "ex_sink", "causal", "tf_mask", "prog_excl")]


@dataclass
class Mask:
    """Token-level visibility parameters; same meaning as omm_topk_mask."""
    block_size: int = 64
    group_size: int = 1
    chunk_q: int = 64
    chunk_k: int = 64
    blocks_per_chunk: int = 0
    q_chunk_offset: int = 0
    q_half: int = 0
    k_half: int = 0
    ex_win: int = 0
    ex_sink: int = 0
    causal: int = 1
    tf_mask: int = 0
    prog_excl: int = 0

    def c(self) -> _Mask:
        return _Mask(*[int(getattr(self, f.name)) for f in fields(self)])


def lib():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(build())
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        i64 = ctypes.c_int64
        _lib.orc_scores.argtypes = [f32p, f32p, i64, i64, i64, i64, i64, ctypes.c_float, f32p]
        _lib.orc_topk.argtypes = [f32p, i64, i64, i64, i64, ctypes.c_int32,
                                  ctypes.POINTER(_Mask), i32p]
        _lib.orc_visible_matrix.argtypes = [ctypes.POINTER(_Mask), i64, i64,
                                            ctypes.POINTER(ctypes.c_uint8)]
    return _lib


def _ptr(a: np.ndarray, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


# ---------------------------------------------------------------------------------------------
# element conversions
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bf16 bits (quiet NaN kept)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    return np.where(nan, ((u >> 16) | np.uint32(0x40)).astype(np.uint16), r)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values rounded (RNE) to dtype and returned as their exact fp32 images."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "bf16":
        return bf16_to_f32(f32_to_bf16(x))
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    raise ValueError(dtype)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e.astype(np.float64) - 10))
    v = np.where((c & 0x7F) == 0x7F, np.nan, v)
    return (sign * v).astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn code, round-to-nearest-even, saturating at 448, NaN -> 0x7f."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = np.abs(x).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        sub = np.rint(a * np.float32(512.0)).astype(np.int64)
        e = ((a.view(np.uint32) >> 23) & 0xFF).astype(np.int64) - 127
        scale = np.exp2((3 - e).astype(np.float64)).astype(np.float32)
        m = np.rint(a * scale).astype(np.float64)
        norm = ((e + 7) << 3) + np.nan_to_num(m, nan=0, posinf=0).astype(np.int64) - 8
    code = np.where(a < np.float32(0.015625), sub, norm)
    code = np.where(a >= np.float32(480.0), 0x7E, code)
    code = np.minimum(code, 0x7E).astype(np.uint8)
    code = np.where(np.isnan(x), np.uint8(0x7F), code)
    return (code | sign).astype(np.uint8)


# ---------------------------------------------------------------------------------------------
# pooling and scores
def pool_mean(x: np.ndarray, group: int, dtype: str) -> np.ndarray:
    """x: fp32 image [B, T, H, D] of dtype elements -> pooled fp32 image [B, ceil(T/g), H, D]."""
    x = np.asarray(x, dtype=np.float32)
    B, T, H, D = x.shape
    MG = -(-T // group)
    out = np.empty((B, MG, H, D), dtype=np.float32)
    for j in range(MG):
        t0, t1 = j * group, min((j + 1) * group, T)
        acc = np.zeros((B, H, D), dtype=np.float32)
        for t in range(t0, t1):
            acc = (acc + x[:, t]).astype(np.float32)
        out[:, j] = acc / np.float32(t1 - t0)
    return round_to(out, dtype)


def block_scores(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """q [B, MG, H, D], k [B, NC, H, D] fp32 images -> fp32 scores [B, MG, H, NC]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    B, MG, H, D = q.shape
    NC = k.shape[1]
    out = np.empty((B, MG, H, NC), dtype=np.float32)
    lib().orc_scores(_ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), B, MG, H, NC, D,
                     ctypes.c_float(scale), _ptr(out, ctypes.c_float))
    return out


def topk_select(scores: np.ndarray, topk: int, mask: Mask) -> np.ndarray:
    s = np.ascontiguousarray(scores, dtype=np.float32)
    B, MG, H, NC = s.shape
    out = np.empty((B, MG, H, topk), dtype=np.int32)
    m = mask.c()
    lib().orc_topk(_ptr(s, ctypes.c_float), B, MG, H, NC, topk, ctypes.byref(m),
                   _ptr(out, ctypes.c_int32))
    return out


def topk_select_large(scores: np.ndarray, topk: int, mask: Mask) -> np.ndarray:
    """The reference's rule past topk = 128 (path B, cuda_backend/csrc/topk.cu:741-807): per row,
    key f32_to_ord(score) (topk.cu:163-166) for a visible column and 0 for a hidden one, whose
    value is -1 (:549-559); a stable descending sort of the keys (CUB segmented radix sort, so
    equal keys keep ascending column order); the first topk values, -1 past NC (:563-581).  The
    raw order code ranks +0 above -0 and ranks visible -inf and NaN scores as well."""
    s = np.ascontiguousarray(scores, dtype=np.float32)
    B, MG, H, NC = s.shape
    vis = visible_matrix(mask, MG, NC)[None, :, None, :]
    u = s.view(np.uint32)
    code = np.where((u & np.uint32(0x80000000)) != 0, ~u, u | np.uint32(0x80000000))
    code = np.where(vis, code, np.uint32(0)).astype(np.int64)
    val = np.broadcast_to(np.where(vis, np.arange(NC, dtype=np.int32), np.int32(-1)), s.shape)
    order = np.argsort(-code, axis=-1, kind="stable")
    ranked = np.take_along_axis(val, order, axis=-1)
    out = np.full((B, MG, H, topk), -1, dtype=np.int32)
    n = min(topk, NC)
    out[..., :n] = ranked[..., :n]
    return out


def visible_matrix(mask: Mask, MG: int, NC: int) -> np.ndarray:
    out = np.empty((MG, NC), dtype=np.uint8)
    m = mask.c()
    lib().orc_visible_matrix(ctypes.byref(m), MG, NC, _ptr(out, ctypes.c_uint8))
    return out.astype(bool)


def topk(q: np.ndarray, k: np.ndarray, topk_n: int, scale: float, mask: Mask) -> np.ndarray:
    return topk_select(block_scores(q, k, scale), topk_n, mask)


# ---------------------------------------------------------------------------------------------
# selection attention
def dense_block_tokens(N: int, block_size: int, chunk_size: int, causal: bool):
    """Token range of block id for the dense layout (common.cuh:173-187, :327-332)."""
    def tokens(bid: int, q_chunk: int):
        if bid < 0:
            return None
        t0 = bid * block_size
        if t0 >= N:
            return None
        if causal and t0 // chunk_size > q_chunk:
            return None
        n = min(block_size, N - t0)
        if causal:
            n = min(n, (q_chunk + 1) * chunk_size - t0)
        return (t0, n) if n > 0 else None
    return tokens


def paged_block_tokens(chunk_len: int, page_tokens: int, n_chunks: int):
    """Chunk-aligned pages: page p of chunk c is id c*ppc + p and covers tokens
    c*chunk_len + p*page_tokens ... (min(page_tokens, chunk_len - p*page_tokens) of them)."""
    ppc = -(-chunk_len // page_tokens)

    def tokens(bid: int, q_chunk: int):
        if bid < 0:
            return None
        c, p = divmod(bid, ppc)
        if c >= n_chunks:
            return None
        return (c * chunk_len + p * page_tokens, min(page_tokens, chunk_len - p * page_tokens))
    return tokens


def selection_attention(q, k, v, ids, group_size: int, scale: float, block_tokens,
                        chunk_size: int = 1, causal: bool = False, groups=None):
    """float64 reference: q [B, M, H, D], k/v [B, N, H, D], ids [B, MG, H, T].

    block_tokens(bid, q_chunk) -> (t0, n) or None.  Returns (out [B, M, H, D], lse [B, H, M]);
    with ``groups`` only those query groups are computed (the rest stay 0 / -inf)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, M, H, D = q.shape
    G = group_size
    MG = ids.shape[1]
    out = np.zeros((B, M, H, D), dtype=np.float64)
    lse = np.full((B, H, M), -np.inf, dtype=np.float64)
    for b in range(B):
        for g in (range(MG) if groups is None else groups):
            m0, m1 = g * G, min((g + 1) * G, M)
            if m0 >= M:
                continue
            q_chunk = (g * G) // chunk_size if causal else 0
            for h in range(H):
                toks = []
                for bid in ids[b, g, h]:
                    r = block_tokens(int(bid), q_chunk)
                    if r is not None:
                        toks.extend(range(r[0], r[0] + r[1]))
                if not toks:
                    continue
                idx = np.asarray(toks, dtype=np.int64)
                kk, vv = k[b, idx, h], v[b, idx, h]
                s = (q[b, m0:m1, h] @ kk.T) * scale
                mx = s.max(axis=1, keepdims=True)
                p = np.exp(s - mx)
                den = p.sum(axis=1, keepdims=True)
                out[b, m0:m1, h] = (p @ vv) / den
                lse[b, h, m0:m1] = (mx + np.log(den))[:, 0]
    return out, lse


def selection_attention_bwd(q, k, v, ids, out, lse, d_out, group_size: int, scale: float,
                            block_tokens, chunk_size: int = 1, causal: bool = False,
                            groups=None):
    """float64 backward of ``selection_attention`` from the forward's (out, lse), as the
    reference's dQ and dK/dV kernels define it (cuda_backend/csrc/selection_bwd.cu:18-163,
    :164-306; bwd_common.cuh:33-60):

        delta_m = sum_d out[m, d] * d_out[m, d]
        P_mj    = exp(q_m . k_j * scale - lse_m)        (0 when lse_m = -inf)
        dS_mj   = P_mj * (d_out_m . v_j - delta_m) * scale
        dq_m    = sum_j dS_mj k_j,   dk_j += sum_m dS_mj q_m,   dv_j += sum_m P_mj d_out_m

    over the tokens each query group selects (a duplicated id contributes twice, as in the
    forward).  Returns (dq, dk, dv, delta [B, H, M]); tokens no group selects get 0."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    out = np.asarray(out, dtype=np.float64)
    d_out = np.asarray(d_out, dtype=np.float64)
    lse = np.asarray(lse, dtype=np.float64)
    B, M, H, D = q.shape
    G = group_size
    MG = ids.shape[1]
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    delta = np.einsum("bmhd,bmhd->bhm", out, d_out)
    for b in range(B):
        for g in (range(MG) if groups is None else groups):
            m0, m1 = g * G, min((g + 1) * G, M)
            if m0 >= M:
                continue
            q_chunk = (g * G) // chunk_size if causal else 0
            for h in range(H):
                toks = []
                for bid in ids[b, g, h]:
                    r = block_tokens(int(bid), q_chunk)
                    if r is not None:
                        toks.extend(range(r[0], r[0] + r[1]))
                if not toks:
                    continue
                idx = np.asarray(toks, dtype=np.int64)
                kk, vv = k[b, idx, h], v[b, idx, h]
                qq, do = q[b, m0:m1, h], d_out[b, m0:m1, h]
                l = lse[b, h, m0:m1][:, None]
                fin = np.isfinite(l)
                p = np.where(fin, np.exp((qq @ kk.T) * scale - np.where(fin, l, 0.0)), 0.0)
                ds = p * ((do @ vv.T) - delta[b, h, m0:m1][:, None]) * scale
                dq[b, m0:m1, h] = ds @ kk
                np.add.at(dk[b, :, h], idx, ds.T @ qq)
                np.add.at(dv[b, :, h], idx, p.T @ do)
    return dq, dk, dv, delta


# ---------------------------------------------------------------------------------------------
# fp8 pages
def quantize_pages(x: np.ndarray, valid: int):
    """x: fp32 [P, D] page (rows >= valid are ignored and stored as 0) -> (codes, scale).

    scale = amax/448 (1 when amax == 0); codes = e4m3(clamp(x * (448/amax), +-448))."""
    x = np.asarray(x, dtype=np.float32).copy()
    x[valid:] = 0.0
    amax = np.float32(np.abs(x).max()) if x.size else np.float32(0)
    if amax > 0:
        scale = np.float32(amax / np.float32(448.0))
        inv = np.float32(np.float32(448.0) / amax)
    else:
        scale = np.float32(1.0)
        inv = np.float32(1.0)
    y = np.clip((x * inv).astype(np.float32), np.float32(-448.0), np.float32(448.0))
    return e4m3_encode(y), scale


def dequantize_pages(codes: np.ndarray, scale) -> np.ndarray:
    return (e4m3_decode(codes) * np.float32(scale)).astype(np.float32)
