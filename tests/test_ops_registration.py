"""The selection-path operators are registered with torch.library (namespace ``omnimem_nsa``) and
the reference-signature facades trace under torch.compile with no graph break (CPU only: fake
CUDA tensors, shape-only kernels).

Reference: the schemas of cuda_backend/csrc/bindings.cpp:7-36 and the fake kernels of
cuda_backend/ops.py:191-235.
"""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from omnimem_amd import ops

# The reference's schemas (cuda_backend/csrc/bindings.cpp:8-35), as written there.
REFERENCE_SCHEMAS = {
    "topk": "topk(Tensor q, Tensor k, int topk, float scale, int block_size, int chunk_size, "
            "int chunk_size_k, bool causal, int ex_win, int ex_sink, bool prog_excl, "
            "bool tf_mask, int q_chunk_offset, bool allow_tf32) -> Tensor",
    "build_ptr_table": "build_ptr_table(Tensor block_indices, Tensor base_k, Tensor base_v, "
                       "Tensor n_blocks_per_head, int batch_stride, int blocks_per_chunk, "
                       "int in_chunk_block_bytes) -> (Tensor, Tensor)",
    "sel_fwd": "sel_fwd(Tensor q, Tensor k, Tensor v, Tensor block_indices, int block_size, "
               "int chunk_size, float scale, bool causal, int group_size, bool allow_tf32) "
               "-> (Tensor, Tensor)",
    "sel_fwd_ptr": "sel_fwd_ptr(Tensor q, Tensor ptr_k, Tensor ptr_v, int block_size, "
                   "int group_size, int stride_bn, int stride_bd, float scale, "
                   "str input_precision, Tensor[] owners) -> (Tensor, Tensor)",
    "sel_bwd": "sel_bwd(Tensor q, Tensor k, Tensor v, Tensor block_indices, Tensor out, "
               "Tensor lse, Tensor d_out, int block_size, int chunk_size, float scale, "
               "bool causal, int group_size, bool allow_tf32) -> (Tensor, Tensor, Tensor)",
    "sel_bwd_ptr": "sel_bwd_ptr(Tensor q, Tensor out, Tensor lse, Tensor d_out, "
                   "Tensor block_indices, Tensor ptr_k, Tensor ptr_v, Tensor base_k, "
                   "Tensor base_v, Tensor base_dk, Tensor base_dv, Tensor n_blocks_per_head, "
                   "int block_size, int group_size, int batch_stride_kv_bytes, "
                   "int batch_stride_dkv_bytes, int stride_bn, int stride_bd, int stride_dbn, "
                   "int stride_dbd, int blocks_per_chunk, int in_chunk_block_bytes_kv, "
                   "int in_chunk_block_bytes_dkv, float scale, str input_precision, "
                   "bool compute_dkv, Tensor[] owners, Tensor(a!)[] grad_buffers) "
                   "-> (Tensor, Tensor)",
}


def _norm(schema: str) -> str:
    return " ".join(schema.replace("omnimem_nsa::", "").split())


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_reference_schemas_registered(name):
    got = str(ops.op(name).default._schema)
    assert _norm(got) == _norm(REFERENCE_SCHEMAS[name])


def _fake_inputs(fm, M=1024, N=1024, H=4, D=128, dtype=torch.bfloat16, grad=False):
    with fm:
        q, k, v = (torch.empty((1, L, H, D), dtype=dtype, device="cuda") for L in (M, N, N))
    if grad:
        for t in (q, k, v):
            t.requires_grad_(True)
    return q, k, v


def _layer(q, k, v):
    from omnimem_amd.index_topk import block_pool, parallel_nsa_topk
    from omnimem_amd.selection import selection_attention
    kc = block_pool(k, 64)
    ids = parallel_nsa_topk(q, kc, 4, block_size=64, chunk_size=256, causal=True, group_size=64)
    return selection_attention(q, k, v, ids, 4, 64, chunk_size=256, causal=True, group_size=64)


def test_facades_trace_without_graph_break():
    """block_pool -> parallel_nsa_topk -> selection_attention compiles as one graph."""
    torch._dynamo.reset()
    fm = FakeTensorMode()
    q, k, v = _fake_inputs(fm)
    compiled = torch.compile(_layer, backend="eager", fullgraph=True)
    with fm:
        out = compiled(q, k, v)
    assert out.shape == q.shape and out.dtype == q.dtype and out.device.type == "cuda"


def test_facades_trace_with_gradients():
    """With inputs that require grad, the autograd Function wrapping sel_fwd / sel_bwd traces in
    the same single graph and its output is differentiable.  (Running the backward needs a real
    device context for the autograd engine; sel_bwd's fake is checked directly below.)"""
    torch._dynamo.reset()
    fm = FakeTensorMode()
    q, k, v = _fake_inputs(fm, M=512, N=512, H=2, grad=True)

    def step(q, k, v):
        return _layer(q, k, v).float().sum()

    compiled = torch.compile(step, backend="eager", fullgraph=True)
    with fm:
        loss = compiled(q, k, v)
    assert loss.requires_grad and loss.grad_fn is not None


def test_fake_shapes_of_every_op():
    fm = FakeTensorMode()
    with fm:
        q = torch.empty((2, 300, 3, 64), dtype=torch.bfloat16, device="cuda")
        kc = torch.empty((2, 40, 3, 64), dtype=torch.bfloat16, device="cuda")
        ids = ops.op("topk_fused")(q, kc, 8, 0.125, 16, 120, True, 0, 0, False, False, 0, 64, 0)
        assert ids.shape == (2, 5, 3, 8) and ids.dtype == torch.int32
        pooled = ops.op("block_pool")(q, 64)
        assert pooled.shape == (2, 5, 3, 64) and pooled.dtype == torch.bfloat16
        rows = ops.op("topk")(pooled, kc, 8, 0.125, 16, 2, 120, True, 0, 0, False, False, 0, True)
        assert rows.shape == (2, 5, 3, 8)
        out, lse = ops.op("sel_fwd")(q, q, q, ids, 64, 120, 0.125, True, 64, True)
        assert out.shape == q.shape and lse.shape == (2, 3, 300) and lse.dtype == torch.float32
        dq, dk, dv = ops.op("sel_bwd")(q, q, q, ids, out, lse, out, 64, 120, 0.125, True, 64, True)
        assert dq.shape == dk.shape == dv.shape == q.shape and dq.is_contiguous()
        base = torch.empty((3, 4), dtype=torch.int64, device="cuda")
        nb = torch.empty((3,), dtype=torch.int32, device="cuda")
        pk, pv = ops.op("build_ptr_table")(ids, base, base, nb, 0, 0, 0)
        assert pk.shape == ids.shape and pk.dtype == torch.int64 and pv.dtype == torch.int64
        o2, l2 = ops.op("sel_fwd_ptr")(q[:, :256], pk[:, :4], pv[:, :4], 64, 64, 64, 1, 0.125,
                                       "tf32", [])
        assert o2.shape == (2, 256, 3, 64) and l2.shape == (2, 3, 256)
        scratch = torch.empty((2, 4, 30, 64), dtype=torch.float32, device="cuda")
        dq2, delta = ops.op("sel_bwd_ptr")(q[:, :256], o2, l2, o2, ids[:, :4], pk[:, :4],
                                           pv[:, :4], base, base, base, base, nb, 30, 64,
                                           0, 0, 64, 1, 64, 1, 4, 0, 0, 0.125, "tf32", True, [],
                                           [scratch])
        assert dq2.shape == (2, 256, 3, 64) and dq2.dtype == torch.bfloat16
        assert delta.shape == (2, 3, 256) and delta.dtype == torch.float32


def test_namespace_owned_by_another_library_falls_back():
    """With ``omnimem_nsa`` already defined by another library (the reference's extension in a
    side-by-side run), importing this package still works: its ops go to ``omnimem_amd_nsa``,
    with the same schemas, and the other library's namespace is left alone."""
    import subprocess
    import sys
    code = (
        "import torch, warnings\n"
        "other = torch.library.Library('omnimem_nsa', 'DEF')\n"
        "other.define('topk(Tensor q) -> Tensor')\n"
        "with warnings.catch_warnings(record=True) as w:\n"
        "    warnings.simplefilter('always')\n"
        "    from omnimem_amd import ops\n"
        "assert ops.NAMESPACE == 'omnimem_amd_nsa', ops.NAMESPACE\n"
        "assert any('owned by another library' in str(x.message) for x in w)\n"
        "assert str(torch.ops.omnimem_nsa.topk.default._schema) == 'omnimem_nsa::topk(Tensor q) -> Tensor'\n"
        "s = str(ops.op('sel_fwd').default._schema)\n"
        "assert s.startswith('omnimem_amd_nsa::sel_fwd(Tensor q, Tensor k'), s\n"
        "from omnimem_amd.selection import selection_attention\n"
        "print('ok')\n")
    root = __import__("os").path.dirname(__import__("os").path.dirname(__file__))
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr


def test_traced_id_check_raises_like_eager():
    """An out-of-range block id raises the same ValueError whether the facade's checks run
    eagerly or inside a compiled graph (fullgraph: the check is an op of the graph, not a
    break), and in-range ids pass both ways."""
    from omnimem_amd.selection import _validate_common
    q = torch.zeros((1, 128, 2, 64))
    k = v = torch.zeros((1, 256, 2, 64))

    def check(ids):
        return _validate_common(q, k, v, ids, 64, 64, 64, False)

    torch._dynamo.reset()
    compiled = torch.compile(check, backend="eager", fullgraph=True)
    good = torch.tensor([0, 3, -1, 2], dtype=torch.int32).view(1, 1, 1, 4).expand(1, 2, 2, 4)
    bad = good.clone()
    bad[0, 1, 1, 0] = 4  # 256 keys of 64-token blocks: ids 0..3
    for fn in (check, compiled):
        assert fn(good) == 4
        with pytest.raises(ValueError, match="top_idx out of range"):
            fn(bad)
