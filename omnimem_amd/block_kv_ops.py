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
    """Distinct selected (head, block) keys of a block-index tensor, found on the device.

    The kernel (``omm_dedup_run``; contract of K3, cuda_backend/csrc/block_kv_ops.h:25-31)
    marks every valid entry's key with this call's epoch in a persistent stamp array, counts the
    marked keys per 1024-key tile, scans the counts and writes ``[n, key_0 < key_1 < ...]``.
    Entry e of the flattened ``[..., H, T]`` indices is head ``(e // T) % H``; block
    ``bid = cid * blocks_per_chunk + loc`` gives key ``(cid * H + h) * blocks_per_chunk + loc``,
    the chunk-major order of a per-head chunk store.

    All device state is one int32 allocation ``[stamps | tile counts | tile offsets | result]``;
    the result lands in one pinned host buffer.  ``enqueue`` launches and starts that copy,
    ``wait`` is the one host wait and returns ``(keys, n_unique, overflow)`` with ``keys`` a view
    of at most ``cap`` ascending keys.  Because the landing buffer is reused, a second
    ``enqueue`` before ``wait`` raises ``RuntimeError``.  Stamps start at 0 and epochs at 1; when
    the epoch would leave int32 the stamps are cleared and counting restarts.
    """

    _TILE = _SCAN_BLOCK

    def __init__(self, heads: int, mb: int, blocks_per_group: int, cap: int, device, *,
                 blocks_per_chunk: int, backend: Optional[str] = None):
        self.backend = resolve_block_kv_backend(backend)
        self.H, self.MB, self.T = int(heads), int(mb), int(blocks_per_group)
        self.bpc, self.cap = int(blocks_per_chunk), int(cap)
        if min(self.H, self.MB, self.T) <= 0 or self.cap < 0:
            raise BlockKVBackendError(
                f"dedup geometry must be positive: heads={self.H}, mb={self.MB}, "
                f"blocks_per_group={self.T}, cap={self.cap}")
        if self.bpc <= 0 or self.MB % self.bpc:
            raise BlockKVBackendError(
                f"blocks_per_chunk={self.bpc} must be positive and divide mb={self.MB}: the key "
                "(cid * heads + h) * blocks_per_chunk + loc is then a bijection")
        self.n_keys = self.H * self.MB
        self.n_tiles = -(-self.n_keys // self._TILE)
        if self.n_tiles > 2 ** 15:
            raise BlockKVBackendError(f"{self.n_keys} keys exceed the single-workgroup scan")
        nt = self.n_tiles
        self._state = torch.zeros(self.n_keys + 2 * nt + 1 + self.cap, dtype=torch.int32,
                                  device=device)
        self.device = self._state.device
        self._stamps = self._state[:self.n_keys]
        self._tile_counts = self._state[self.n_keys:self.n_keys + nt]
        self._tile_offsets = self._state[self.n_keys + nt:self.n_keys + 2 * nt]
        self._result = self._state[self.n_keys + 2 * nt:]
        self._landing = torch.empty(1 + self.cap, dtype=torch.int32, pin_memory=True)
        self._landed = torch.cuda.Event()
        self._epoch = 0
        self._pending = False
        self.calls = 0

    @property
    def d2h_bytes_per_call(self) -> int:
        """Bytes one call copies to the host: the count plus ``cap`` key slots."""
        return 4 * (1 + self.cap)

    def device_bytes(self) -> int:
        return self._state.numel() * 4

    def _next_epoch(self) -> int:
        if self._epoch == 2 ** 31 - 1:
            self._stamps.zero_()
            self._epoch = 0
        self._epoch += 1
        return self._epoch

    def enqueue(self, block_indices: torch.Tensor) -> None:
        """Launch the dedup of ``block_indices`` (contiguous int32 [..., H, T] on this device)
        and the copy of its result to the host, on the current stream.  No host wait."""
        if self._pending:
            raise RuntimeError("DeviceBlockDedup: wait() for the pending call before enqueueing "
                               "another (the host landing buffer is shared)")
        t = block_indices
        if not (isinstance(t, torch.Tensor) and t.dtype == torch.int32 and t.is_cuda
                and t.is_contiguous()):
            raise BlockKVBackendError("block_indices must be a contiguous int32 GPU tensor")
        if t.dim() < 2 or tuple(t.shape[-2:]) != (self.H, self.T):
            raise BlockKVBackendError(
                f"block_indices must end in [H={self.H}, T={self.T}], got {tuple(t.shape)}")
        if t.device != self.device:
            raise BlockKVBackendError(f"block_indices on {t.device}, dedup state on {self.device}")
        epoch = self._next_epoch()
        _lib.call("omm_dedup_run", t.data_ptr() if t.numel() else None, t.numel(),
                  self._stamps.data_ptr(), self._tile_counts.data_ptr(),
                  self._tile_offsets.data_ptr(), self._result.data_ptr(), epoch, self.MB, self.H,
                  self.T, self.bpc, self.cap, _lib.stream_of(t), error=BlockKVBackendError)
        self._landing.copy_(self._result, non_blocking=True)
        self._landed.record(torch.cuda.current_stream(self.device))
        self._pending = True
        self.calls += 1

    def wait(self):
        """Block until the pending call's result is on the host: (keys, n_unique, overflow)."""
        if not self._pending:
            raise RuntimeError("DeviceBlockDedup.wait() without a pending enqueue()")
        self._pending = False
        self._landed.synchronize()
        view = self._landing.numpy()
        n = int(view[0])
        return view[1:1 + min(n, self.cap)], n, n > self.cap

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
