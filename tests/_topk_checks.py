"""Parity check of the MFMA top-k path (bf16 / f16, head dim 64 or 128).

The kernel's block scores are fp32 sums of exact bf16 / f16 products in the MFMA's order (the
reference scores with TF32 WMMA, also an fp32 sum of exact products in its hardware's order), so
the parity target is the one BASELINE states: the indices equal the reference selection rule
(cuda_backend/csrc/topk.cu:3,36-102: visibility, score desc, id asc, -1 padding) applied to the
identical fp32 scores.  The check therefore:

1. reads the scores the selection ran on (``parallel_nsa_topk_with_scores``) and requires the
   indices to equal ``oracle.topk_select`` on them, bit for bit;
2. requires every visible score to lie within the fp32 summation bound of the float64 dot product
   of the oracle-pooled query row and the key: |s - s64| <= (D + 2) 2^-24 sum_d |q_d k_d| |scale|
   + 2^-24 |s64|.  Any order of fp32 additions of D exact products meets it; a wrong pooled row
   (one bf16 ulp off), a dropped product or a wrong scale does not.
"""
import numpy as np
import torch

from oracle import nsa_oracle as O


def _img(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def check_mfma_topk(q, k, topk, mask: "O.Mask", scale, group_size, got=None, **facade):
    """q [B, T, H, D] (full resolution), k [B, NC, H, D] on the GPU; ``facade`` holds the
    parallel_nsa_topk keyword arguments that produce ``mask``.  ``got``: indices returned by the
    product call, which must equal the hook's."""
    from omnimem_amd.index_topk import parallel_nsa_topk_with_scores
    ids, scores = parallel_nsa_topk_with_scores(q, k, topk, scale=scale, group_size=group_size,
                                                **facade)
    ids = ids.cpu().numpy()
    sc = scores.cpu().numpy()
    if got is not None:
        np.testing.assert_array_equal(np.asarray(got), ids)
    want = O.topk_select(sc, topk, mask)
    np.testing.assert_array_equal(ids, want)
    dt = {torch.bfloat16: "bf16", torch.float16: "f16"}[q.dtype]
    qp = O.pool_mean(_img(q), group_size, dt).astype(np.float64)
    kk = _img(k).astype(np.float64)
    s64 = np.einsum("bghd,bchd->bghc", qp, kk) * scale
    a64 = np.einsum("bghd,bchd->bghc", np.abs(qp), np.abs(kk)) * abs(scale)
    D = q.shape[-1]
    vis = O.visible_matrix(mask, qp.shape[1], kk.shape[1])[None, :, None, :]
    vis = np.broadcast_to(vis, sc.shape)
    bound = (D + 2) * 2.0 ** -24 * a64 + 2.0 ** -24 * np.abs(s64) + 1e-30
    err = np.abs(sc.astype(np.float64) - s64)
    bad = vis & ~(err <= bound)
    assert not bad.any(), (f"{int(bad.sum())} visible scores outside the fp32 bound; worst "
                           f"{float(np.max(np.where(vis, err / bound, 0))):.3g}x")
    return ids
