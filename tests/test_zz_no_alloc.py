"""The allocation-free top-k entry point (omm_topk_fused_noalloc) against omm_topk_fused, both
called through the C ABI: identical indices on two calls in a row, the second smaller, so the
second reuses the per-GPU scratch array the first left filled."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _mask(G, chunk, qoff, exw, bpc):
    from omnimem_amd.index_topk import _mask
    return _mask(64, G, chunk, chunk, False, exw, 0, True, False, qoff, 0, 0, bpc)


def _both(q, k, G, topk, chunk, qoff, exw, bpc):
    from omnimem_amd import _lib
    B, T, H, D = q.shape
    NC = k.shape[1]
    MG = -(-T // G)
    dt = _lib.dtype_code(q)
    m = _mask(G, chunk, qoff, exw, bpc)
    ref = torch.full((B, MG, H, topk), -7, dtype=torch.int32, device=DEV)
    got = torch.full_like(ref, -7)
    ws_n = _lib.lib().omm_topk_fused_workspace_bytes(B, T, H, D, NC, G, topk, dt)
    assert 0 < ws_n <= _lib.lib().omm_topk_fused_noalloc_max_bytes()  # the scratch path runs
    ws = torch.empty(ws_n, dtype=torch.uint8, device=DEV)
    s = _lib.stream_of(q)
    _lib.call("omm_topk_fused", _lib.view4(q), _lib.view4(k), dt, G, topk, 0.088, m,
              ref.data_ptr(), ws.data_ptr(), ws_n, s)
    _lib.call("omm_topk_fused_noalloc", _lib.view4(q), _lib.view4(k), dt, G, topk, 0.088, m,
              got.data_ptr(), s)
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


def test_noalloc_matches_workspace_entry_twice():
    g = torch.Generator().manual_seed(41)
    # AR shape: one 4680-token chunk of queries over 40 cached chunks of 74 pages
    q = torch.randn((1, 4680, 12, 128), generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn((1, 40 * 74, 12, 128), generator=g).to(torch.bfloat16).to(DEV)
    ref, got = _both(q, k, 64, 16, 4680, 40, 3, 74)
    np.testing.assert_array_equal(got, ref)
    assert (ref >= 0).all()
    # smaller second call: fewer heads, rows and columns
    q2 = torch.randn((1, 1000, 3, 128), generator=g).to(torch.bfloat16).to(DEV)
    k2 = torch.randn((1, 600, 3, 128), generator=g).to(torch.bfloat16).to(DEV)
    ref2, got2 = _both(q2, k2, 64, 8, 1000, 5, 1, 100)
    np.testing.assert_array_equal(got2, ref2)


def test_noalloc_rejects_calls_beyond_the_scratch():
    from omnimem_amd import _lib
    from omnimem_amd.backend import NSABackendError
    cap = _lib.lib().omm_topk_fused_noalloc_max_bytes()
    # pooled rows alone exceed the scratch: 1 x (8 MiB / 2 + 64) groups x 1 head x 1 dim
    T = cap // 2 + 64
    q = torch.zeros((1, T, 1, 8), dtype=torch.bfloat16, device=DEV)
    k = torch.zeros((1, 64, 1, 8), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((1, T, 1, 4), dtype=torch.int32, device=DEV)
    with pytest.raises(NSABackendError, match="static"):
        _lib.call("omm_topk_fused_noalloc", _lib.view4(q), _lib.view4(k), _lib.dtype_code(q), 1,
                  4, 1.0, _mask(1, 64, 0, 0, 0), out.data_ptr(), _lib.stream_of(q))
