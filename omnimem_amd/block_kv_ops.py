"""Block-store kernels K1 / K2 / K3 behind the reference's Python facades.

Reference: src/omnimem/nsa/ops/selection/padded_ptr/kernels/block_kv_kernels.py:49-139
(``register_block_range``, ``clear_block_range``, ``gather_publish_clear``,
``table_entry_addresses``), kernels/block_kv_dedup.py:17-108 (``DeviceBlockDedup``) and
cuda_backend/block_kv_ops.py:76-114 (``warmup``).  Contracts: cuda_backend/csrc/block_kv_ops.h.
Every call enqueues on the current stream of its tensors' device and never synchronises, except
``DeviceBlockDedup.wait`` (its one host wait).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

from . import _lib
from .backend import BlockKVBackendError, resolve_block_kv_backend

__all__ = ["register_block_range", "clear_block_range", "gather_publish_clear",
           "table_entry_addresses", "DeviceBlockDedup", "warmup"]

_CLR_BLOCK = 256   # K1 clear entries per workgroup
_SCAN_BLOCK = 1024  # K3 keys per tile


def _check_table(table: torch.Tensor, n_valid: torch.Tensor):
    if not (table.dtype == torch.int64 and table.is_cuda and table.is_contiguous()):
        raise BlockKVBackendError("table must be a contiguous int64 GPU tensor")
    if table.dim() != 3 or table.shape[0] != 2:
        raise BlockKVBackendError(f"table must be [2, H, MB], got {tuple(table.shape)}")
    if not (n_valid.dtype == torch.int32 and n_valid.is_cuda and n_valid.shape == (table.shape[1],)
            and n_valid.is_contiguous()):
        raise BlockKVBackendError(f"n_valid must be contiguous int32 [H={table.shape[1]}]")


def _range(table, n_valid, first_bid, n_blocks, k_base, v_base, head_stride, block_bytes,
           n_valid_value, write_k, write_v, clear):
    _, H, MB = table.shape
    _lib.call("omm_block_range", table.data_ptr(), n_valid.data_ptr(), H, MB, int(first_bid),
              int(n_blocks), int(k_base), int(v_base), int(head_stride), int(block_bytes),
              int(n_valid_value), int(bool(write_k)), int(bool(write_v)), int(bool(clear)),
              _lib.stream_of(table), error=BlockKVBackendError)


def register_block_range(table: torch.Tensor, n_valid: torch.Tensor, first_bid: int,
                         n_blocks: int, k_base: int, v_base: int, head_stride_bytes: int,
                         block_bytes: int, n_valid_value: int,
                         backend: Optional[str] = None) -> None:
    """table[name, h, first_bid + j] = base_name + h*head_stride + j*block_bytes; base 0 skips."""
    resolve_block_kv_backend(backend)
    _check_table(table, n_valid)
    _, H, MB = table.shape
    first_bid, n_blocks = int(first_bid), int(n_blocks)
    if not (0 <= first_bid and first_bid + n_blocks <= MB):
        raise BlockKVBackendError(f"block range [{first_bid}, {first_bid + n_blocks}) outside [0, {MB})")
    if n_blocks <= 0:
        if int(n_valid_value) >= 0:
            n_valid.fill_(int(n_valid_value))
        return
    if int(k_base) == 0 and int(v_base) == 0:
        raise BlockKVBackendError("nothing to register")
    _range(table, n_valid, first_bid, n_blocks, k_base, v_base, head_stride_bytes, block_bytes,
           n_valid_value, int(k_base) != 0, int(v_base) != 0, False)


def clear_block_range(table: torch.Tensor, n_valid: torch.Tensor, first_bid: int, n_blocks: int,
                      n_valid_value: int, which: str = "kv",
                      backend: Optional[str] = None) -> None:
    """Zero table[rows, :, first_bid:first_bid + n_blocks] and set n_valid (< 0 leaves it)."""
    resolve_block_kv_backend(backend)
    _check_table(table, n_valid)
    _, H, MB = table.shape
    if which not in ("k", "v", "kv"):
        raise BlockKVBackendError(f"which must be 'k', 'v' or 'kv', got {which!r}")
    first_bid, n_blocks = int(first_bid), int(n_blocks)
    if not (0 <= first_bid and first_bid + n_blocks <= MB):
        raise BlockKVBackendError(f"block range [{first_bid}, {first_bid + n_blocks}) outside [0, {MB})")
    if n_blocks <= 0:
        if int(n_valid_value) >= 0:
            n_valid.fill_(int(n_valid_value))
        return
    _range(table, n_valid, first_bid, n_blocks, 0, 0, 0, 0, n_valid_value, "k" in which,
           "v" in which, True)


def table_entry_addresses(table: torch.Tensor, name_idx, keys):
    """Byte addresses of table[name_idx, key // MB, key % MB] for flat int64 keys h*MB + bid."""
    _, H, MB = table.shape
    if isinstance(keys, torch.Tensor):
        keys = keys.to(torch.int64)
    else:
        keys = np.asarray(keys, dtype=np.int64)
    return table.data_ptr() + (name_idx * H * MB + keys) * 8


def gather_publish_clear(desc: torch.Tensor, n_fetch: int, n_clear: int, block_tokens: int,
                         head_dim: int, typed: torch.Tensor, num_warps: int = 1,
                         wide: Optional[bool] = None, backend: Optional[str] = None) -> int:
    """K1 over the int64 descriptor (sources may be pinned host memory); returns workgroups
    launched, n_fetch + ceil(n_clear / 256).  ``num_warps`` / ``wide`` are accepted for
    signature compatibility: the kernel always runs 256 lanes and picks 16-byte copies when
    size and alignment allow."""
    resolve_block_kv_backend(backend)
    n_fetch, n_clear = int(n_fetch), int(n_clear)
    if n_fetch == 0 and n_clear == 0:
        return 0
    if not (desc.dtype == torch.int64 and desc.is_cuda and desc.is_contiguous()):
        raise BlockKVBackendError("desc must be a contiguous int64 GPU tensor")
    if desc.numel() < 6 * n_fetch + n_clear:
        raise BlockKVBackendError(
            f"descriptor holds {desc.numel()} elements, need {6 * n_fetch + n_clear}")
    if typed.element_size() != 2:
        raise BlockKVBackendError(
            f"the gather kernel supports 16-bit KV dtypes only, got {typed.dtype}")
    block_bytes = int(block_tokens) * int(head_dim) * 2
    if wide and block_bytes % 8:
        raise BlockKVBackendError(f"wide copy needs block_bytes ({block_bytes}) to be a multiple of 8")
    ctas = ctypes.c_int64(0)
    _lib.call("omm_gather_publish_clear", desc.data_ptr(), n_fetch, n_clear, block_bytes,
              ctypes.byref(ctas), _lib.stream_of(desc), error=BlockKVBackendError)
    return int(ctas.value)


class DeviceBlockDedup:
    """Fixed-capacity device dedup; unique_keys returns (keys int32 view, n_unique, overflow)."""

    def __init__(self, heads: int, mb: int, blocks_per_group: int, cap: int, device, *,
                 blocks_per_chunk: int, backend: Optional[str] = None):
        self.H, self.MB, self.T = int(heads), int(mb), int(blocks_per_group)
        self.bpc = int(blocks_per_chunk)
        if not (self.bpc > 0 and self.MB % self.bpc == 0):
            raise BlockKVBackendError(
                f"blocks_per_chunk {self.bpc} must divide MB {self.MB} for the key to be a bijection")
        self.n_keys = self.H * self.MB
        self.cap = int(cap)
        self.backend = resolve_block_kv_backend(backend)
        self.stamp = torch.full((self.n_keys,), -1, dtype=torch.int32, device=device)
        self.device = self.stamp.device
        self.n_tiles = -(-self.n_keys // _SCAN_BLOCK)
        if self.n_tiles > 2 ** 15:
            raise BlockKVBackendError("too many keys for the single-workgroup scan")
        self.counts = torch.zeros(self.n_tiles, dtype=torch.int32, device=self.device)
        self.offsets = torch.zeros(self.n_tiles, dtype=torch.int32, device=self.device)
        self.out = torch.zeros(1 + self.cap, dtype=torch.int32, device=self.device)
        self.pinned = torch.empty(1 + self.cap, dtype=torch.int32, pin_memory=True)
        self._pin_np = self.pinned.numpy()
        self.event = torch.cuda.Event()
        self.epoch = 0
        self.launches = 0
        self.d2h_bytes = 0
        self._in_flight = False

    @property
    def d2h_bytes_per_call(self) -> int:
        return self.pinned.numel() * 4

    def device_bytes(self) -> int:
        return sum(t.numel() * t.element_size()
                   for t in (self.stamp, self.counts, self.offsets, self.out))

    def enqueue(self, block_indices: torch.Tensor) -> None:
        if self._in_flight:
            raise RuntimeError("DeviceBlockDedup.enqueue() called again before the previous "
                               "enqueue's wait(); at most one call may be in flight")
        if not (block_indices.dtype == torch.int32 and block_indices.is_cuda
                and block_indices.is_contiguous()):
            raise BlockKVBackendError("block_indices must be a contiguous int32 GPU tensor")
        if block_indices.shape[-2] != self.H or block_indices.shape[-1] != self.T:
            raise BlockKVBackendError(
                f"expected [..., H={self.H}, T={self.T}], got {tuple(block_indices.shape)}")
        if block_indices.device != self.device:
            raise BlockKVBackendError(
                f"block_indices live on {block_indices.device}, the dedup buffers on {self.device}")
        self._in_flight = True
        self.epoch += 1
        if self.epoch >= 2 ** 31 - 1:
            self.stamp.fill_(-1)
            self.epoch = 1
        flat = block_indices.view(-1)
        _lib.call("omm_dedup_run", flat.data_ptr(), flat.numel(), self.stamp.data_ptr(),
                  self.counts.data_ptr(), self.offsets.data_ptr(), self.out.data_ptr(),
                  self.epoch, self.MB, self.H, self.T, self.bpc, self.cap,
                  _lib.stream_of(flat), error=BlockKVBackendError)
        self.pinned.copy_(self.out, non_blocking=True)
        self.event.record(torch.cuda.current_stream(self.device))
        self.launches += 4
        self.d2h_bytes += self.d2h_bytes_per_call

    def wait(self):
        try:
            self.event.synchronize()
        finally:
            self._in_flight = False
        n = int(self._pin_np[0])
        return self._pin_np[1:1 + min(n, self.cap)], n, n > self.cap

    def unique_keys(self, block_indices: torch.Tensor):
        self.enqueue(block_indices)
        return self.wait()


_warmed: set = set()


def warmup(device) -> int:
    """Launch K1, K2 and K3 once on tiny private tensors (the reference's warm-up known answers,
    cuda_backend/block_kv_ops.py:93-111); idempotent per device.  Returns launches issued."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    device = torch.device(device.type, index)
    if (device.type, index) in _warmed:
        return 0
    n = 0
    with torch.cuda.device(device):
        src = torch.ones(2, 16, dtype=torch.int16, device=device)
        dst = torch.zeros(2, 16, dtype=torch.int16, device=device)
        table = torch.full((4,), -1, dtype=torch.int64, device=device)
        a = table.data_ptr()
        desc = torch.tensor([src[0].data_ptr(), src[1].data_ptr(), dst[0].data_ptr(),
                             dst[1].data_ptr(), a, a + 8, a + 16, a + 24], dtype=torch.int64,
                            device=device)
        n += int(gather_publish_clear(desc, 1, 2, 16, 1, src) > 0)
        tab = torch.zeros(2, 1, 4, dtype=torch.int64, device=device)
        nv = torch.zeros(1, dtype=torch.int32, device=device)
        register_block_range(tab, nv, 0, 4, 4096, 8192, 64, 16, 4)
        clear_block_range(tab, nv, 0, 4, -1)
        n += 2
        dd = DeviceBlockDedup(1, 4, 4, 4, device, blocks_per_chunk=4)
        ids = torch.tensor([[[[0, -1, 3, 3]]]], dtype=torch.int32, device=device)
        keys, count, overflow = dd.unique_keys(ids)
        if count != 2 or list(keys) != [0, 3] or overflow:
            raise BlockKVBackendError(f"K3 warm-up known answer failed: {list(keys)}, {count}")
        n += 4
        torch.cuda.current_stream(device).synchronize()
    _warmed.add((device.type, index))
    return n
