"""torch.library registration of the selection-path operators, namespace ``omnimem_nsa``.

The reference registers its CUDA kernels as ``torch.ops.omnimem_nsa.*`` (schemas:
cuda_backend/csrc/bindings.cpp:7-36) and gives each a shape-only fake so ``torch.compile`` can
trace through them (cuda_backend/ops.py:191-235).  The schemas below are the reference's, so a
caller of ``torch.ops.omnimem_nsa.topk`` / ``sel_fwd`` / ``sel_bwd`` / ``build_ptr_table`` /
``sel_fwd_ptr`` / ``sel_bwd_ptr`` runs unchanged.  Two more ops are this build's: ``topk_fused``
(query-group pooling, scoring and selection in one call, what ``parallel_nsa_topk`` runs) and
``block_pool`` (the K block compression), so that the facades trace as a chain of registered ops.

The CUDA-key implementations are the C-ABI calls of ``index_topk``, ``selection`` and
``padded_ptr`` (ctypes on the current stream, no host synchronisation); they raise
``NSABackendError`` on a bad argument, as the reference's adapters do.  The fakes compute
output shapes, dtypes and layouts only.  Importing this module registers everything once.

If another library already owns the ``omnimem_nsa`` namespace (the reference's extension loaded
in the same process, e.g. for a side-by-side parity run), the ops are registered under
``omnimem_amd_nsa`` instead and ``NAMESPACE`` names it: the reference's ops stay the reference's,
and the facades of this package call their own through ``op()``.
"""
from __future__ import annotations

import warnings

import torch

REFERENCE_NAMESPACE = "omnimem_nsa"
FALLBACK_NAMESPACE = "omnimem_amd_nsa"

SCHEMAS = {
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
    # this build's additions
    "topk_fused": "topk_fused(Tensor q, Tensor k, int topk, float scale, int block_size, "
                  "int chunk_size, bool causal, int ex_win, int ex_sink, bool prog_excl, "
                  "bool tf_mask, int q_chunk_offset, int group_size, int blocks_per_chunk) "
                  "-> Tensor",
    "block_pool": "block_pool(Tensor x, int group) -> Tensor",
    # range check of selection block ids inside a traced graph (an op that mutates its sink is
    # never dropped as dead code); raises ValueError when run, like the eager facade
    "check_block_ids": "check_block_ids(Tensor(a!) sink, Tensor block_indices, int num_blocks) "
                       "-> ()",
}


# ---- CUDA-key implementations (C-ABI calls) ------------------------------------------------
def _topk_cuda(q, k, topk, scale, block_size, chunk_size, chunk_size_k, causal, ex_win, ex_sink,
               prog_excl, tf_mask, q_chunk_offset, allow_tf32):
    from .index_topk import _topk_impl
    return _topk_impl(q, k, topk, scale, block_size, chunk_size, chunk_size_k, causal, ex_win,
                      ex_sink, prog_excl, tf_mask, q_chunk_offset, allow_tf32)


def _topk_fused_cuda(q, k, topk, scale, block_size, chunk_size, causal, ex_win, ex_sink,
                     prog_excl, tf_mask, q_chunk_offset, group_size, blocks_per_chunk):
    from .index_topk import _topk_fused_impl
    return _topk_fused_impl(q, k, topk, scale, block_size, chunk_size, causal, ex_win, ex_sink,
                            prog_excl, tf_mask, q_chunk_offset, group_size, blocks_per_chunk)


def _block_pool_cuda(x, group):
    from .index_topk import _block_pool_impl
    return _block_pool_impl(x, group)


def check_block_ids_now(block_indices, num_blocks):
    """The reference facade's id range check (nsa/ops/selection/__init__.py:36-42): one host
    synchronisation, ValueError for a valid id >= num_blocks."""
    valid_mask = block_indices >= 0
    if valid_mask.any() and torch.any(block_indices[valid_mask] >= num_blocks):
        raise ValueError(
            f"top_idx out of range: expected in [-1, {num_blocks - 1}] "
            f"but got [{block_indices.min()}, {block_indices.max()}]")


def _check_block_ids_impl(sink, block_indices, num_blocks):
    check_block_ids_now(block_indices, num_blocks)


def _check_block_ids_fake(sink, block_indices, num_blocks):
    return None


def _sel_fwd_cuda(q, k, v, block_indices, block_size, chunk_size, scale, causal, group_size,
                  allow_tf32):
    from .selection import _sel_fwd_impl
    return _sel_fwd_impl(q, k, v, block_indices, block_size, chunk_size, scale, causal,
                         group_size)


def _sel_bwd_cuda(q, k, v, block_indices, out, lse, d_out, block_size, chunk_size, scale, causal,
                  group_size, allow_tf32):
    from .selection import _sel_bwd_impl
    return _sel_bwd_impl(q, k, v, block_indices, out, lse, d_out, block_size, chunk_size, scale,
                         causal, group_size)


def _build_ptr_table_cuda(block_indices, base_k, base_v, n_blocks_per_head, batch_stride,
                          blocks_per_chunk, in_chunk_block_bytes):
    from .padded_ptr import _build_ptr_table_impl
    return _build_ptr_table_impl(block_indices, base_k, base_v, n_blocks_per_head, batch_stride,
                                 blocks_per_chunk, in_chunk_block_bytes)


def _sel_fwd_ptr_cuda(q, ptr_k, ptr_v, block_size, group_size, stride_bn, stride_bd, scale,
                      input_precision, owners):
    from .padded_ptr import _sel_fwd_ptr_impl
    return _sel_fwd_ptr_impl(q, ptr_k, ptr_v, block_size, group_size, stride_bn, stride_bd,
                             scale, input_precision, owners)


def _sel_bwd_ptr_cuda(q, out, lse, d_out, block_indices, ptr_k, ptr_v, base_k, base_v, base_dk,
                      base_dv, n_blocks_per_head, block_size, group_size, batch_stride_kv_bytes,
                      batch_stride_dkv_bytes, stride_bn, stride_bd, stride_dbn, stride_dbd,
                      blocks_per_chunk, in_chunk_block_bytes_kv, in_chunk_block_bytes_dkv, scale,
                      input_precision, compute_dkv, owners, grad_buffers):
    from .padded_ptr import _sel_bwd_ptr_impl
    return _sel_bwd_ptr_impl(q, out, lse, d_out, block_indices, ptr_k, ptr_v, base_k, base_v,
                             base_dk, base_dv, n_blocks_per_head, block_size, group_size,
                             batch_stride_kv_bytes, batch_stride_dkv_bytes, stride_bn, stride_bd,
                             stride_dbn, stride_dbd, blocks_per_chunk, in_chunk_block_bytes_kv,
                             in_chunk_block_bytes_dkv, scale, compute_dkv, grad_buffers)


# ---- fakes (shapes only) ------------------------------------------------------------------
def _topk_fake(q, k, topk, scale, block_size, chunk_size, chunk_size_k, causal, ex_win, ex_sink,
               prog_excl, tf_mask, q_chunk_offset, allow_tf32):
    B, MG, H, _ = q.shape
    return q.new_empty((B, MG, H, topk), dtype=torch.int32)


def _topk_fused_fake(q, k, topk, scale, block_size, chunk_size, causal, ex_win, ex_sink,
                     prog_excl, tf_mask, q_chunk_offset, group_size, blocks_per_chunk):
    B, T, H, _ = q.shape
    return q.new_empty((B, -(-T // group_size), H, topk), dtype=torch.int32)


def _block_pool_fake(x, group):
    B, T, H, D = x.shape
    return x.new_empty((B, -(-T // group), H, D))


def _sel_fwd_fake(q, k, v, block_indices, block_size, chunk_size, scale, causal, group_size,
                  allow_tf32):
    B, M, H, _ = q.shape
    return torch.empty_like(q), q.new_empty((B, H, M), dtype=torch.float32)


def _sel_bwd_fake(q, k, v, block_indices, out, lse, d_out, block_size, chunk_size, scale, causal,
                  group_size, allow_tf32):
    # dq, dk and dv are fresh contiguous buffers
    return q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape)


def _build_ptr_table_fake(block_indices, base_k, base_v, n_blocks_per_head, batch_stride,
                          blocks_per_chunk, in_chunk_block_bytes):
    shape = block_indices.shape
    return (block_indices.new_empty(shape, dtype=torch.int64),
            block_indices.new_empty(shape, dtype=torch.int64))


def _sel_fwd_ptr_fake(q, ptr_k, ptr_v, block_size, group_size, stride_bn, stride_bd, scale,
                      input_precision, owners):
    B, M, H, _ = q.shape
    return torch.empty_like(q), q.new_empty((B, H, M), dtype=torch.float32)


def _sel_bwd_ptr_fake(q, out, lse, d_out, block_indices, ptr_k, ptr_v, base_k, base_v, base_dk,
                      base_dv, n_blocks_per_head, block_size, group_size, batch_stride_kv_bytes,
                      batch_stride_dkv_bytes, stride_bn, stride_bd, stride_dbn, stride_dbd,
                      blocks_per_chunk, in_chunk_block_bytes_kv, in_chunk_block_bytes_dkv, scale,
                      input_precision, compute_dkv, owners, grad_buffers):
    # dq and delta are fresh contiguous buffers; dK / dV go to grad_buffers in place
    B, M, H, _ = q.shape
    return q.new_empty(q.shape), q.new_empty((B, H, M), dtype=torch.float32)


_IMPLS = {
    "topk": (_topk_cuda, _topk_fake),
    "topk_fused": (_topk_fused_cuda, _topk_fused_fake),
    "block_pool": (_block_pool_cuda, _block_pool_fake),
    "sel_fwd": (_sel_fwd_cuda, _sel_fwd_fake),
    "sel_bwd": (_sel_bwd_cuda, _sel_bwd_fake),
    "build_ptr_table": (_build_ptr_table_cuda, _build_ptr_table_fake),
    "sel_fwd_ptr": (_sel_fwd_ptr_cuda, _sel_fwd_ptr_fake),
    "sel_bwd_ptr": (_sel_bwd_ptr_cuda, _sel_bwd_ptr_fake),
    "check_block_ids": (_check_block_ids_impl, _check_block_ids_fake),
}
# keys each op is implemented for (the range check also runs on CPU tensors)
_KEYS = {"check_block_ids": ("CUDA", "CPU")}


def _define_library():
    """DEF library of the first namespace no other library owns."""
    for ns in (REFERENCE_NAMESPACE, FALLBACK_NAMESPACE):
        try:
            lib = torch.library.Library(ns, "DEF")
        except RuntimeError:
            continue
        if ns != REFERENCE_NAMESPACE:
            warnings.warn(f"torch.ops.{REFERENCE_NAMESPACE} is owned by another library (the "
                          f"reference extension?); this package's ops are torch.ops.{ns}.*",
                          RuntimeWarning, stacklevel=3)
        return ns, lib
    from .backend import NSABackendError
    raise NSABackendError(f"cannot register operators: namespaces {REFERENCE_NAMESPACE} and "
                          f"{FALLBACK_NAMESPACE} are both owned by other libraries")


NAMESPACE, _LIBRARY = _define_library()
for _name, _schema in SCHEMAS.items():
    _LIBRARY.define(_schema)
    _real, _fake = _IMPLS[_name]
    for _key in _KEYS.get(_name, ("CUDA",)):
        _LIBRARY.impl(_name, _real, _key)
    torch.library.register_fake(f"{NAMESPACE}::{_name}", _fake, lib=_LIBRARY)
del _name, _schema, _real, _fake, _key


def op(name: str):
    """The registered ``torch.ops.<NAMESPACE>.<name>`` overload packet."""
    return getattr(getattr(torch.ops, NAMESPACE), name)
