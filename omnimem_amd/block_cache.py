"""Paged block KV cache for the NSA selection path (HBM pool + pinned host pool, LRU by bytes).

Reference: ``MMCache`` (src/omnimem/models/cache.py:7-1149), chunk_per_head storage
(:478-502), ptr tables (:227-347), LRU (:646-741), offload (:970-1142) and the reload path of
``_touch_lru_and_detect_missing`` (nsa/ops/selection/padded_ptr/wrapper.py:253-362).

Layout.  A *unit* is one (layer, head, chunk): ``pages_per_chunk`` pages of ``page_tokens``
tokens x ``head_dim`` values, contiguous (chunk-aligned pages; the last page of a 4680-token chunk
holds 8 valid tokens when pages are 64 tokens).  Units live in one HBM pool shared by every layer
(``hbm_slots`` units each for K and V) or in a device-mapped pinned host pool that the attention
kernel reads directly, so a unit that is not in HBM is never a miss that stalls the stream: it is
read over the host link page by page.  ``unit_table[layer]`` (int32 [H, max_chunks], on the
device) maps a unit to its slot: s >= 0 HBM, s <= -2 host slot -2-s, -1 never written.

Residency.  Every append and every selection call stamps the units it touches with an epoch,
and the selection kernel counts the pages it reads per unit, on the device (no host
synchronisation, unlike the reference's ``unique().cpu()`` per call).  At a chunk boundary
``flush()`` reads stamps and counts once and moves units between the pools in batched copies.
With ``lru_max_size`` (the reference's count, models/cache.py:673-699) each (layer, head) keeps its
most recent units by (epoch, chunk id), the order in which the reference's OrderedDict sees
them.  With a byte budget the policy is cost-based, because a host unit is read page by page:
units are evicted only to make room (coldest first: lowest heat, then least recent), and a host
unit is promoted only when its heat, a moving average of its page reads per interval, exceeds
the pages a swap would move.  Sink and window chunks always stay in HBM.  Under the byte budget
a flush only enqueues its copies, on a stream of their own (the copy engines), and the next
flush commits them; until then a moving unit is read from its source slot.

Host pages.  A selection reads a host-resident page over the host link, in place; or, after
``prefetch(ids, layer)``, from an HBM staging pool that a side stream fills with each distinct
host page the call lists, once, while the caller's other work runs (``omm_paged_stage``).

Streams.  Every method enqueues on the current stream of ``device`` (``prefetch`` and an
asynchronous ``flush`` also on the cache's side streams, ordered by events); use one stream per
cache.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _lib
from .backend import BlockKVBackendError

__all__ = ["PagedKVCache"]


class _UploadRing:
    """Pinned staging for asynchronous host -> device copies of small int32 arrays (unit
    tables, slot indices).  Each of the ``n`` buffers is rewritten only after an event says its
    previous copy has left, so no upload synchronises the stream."""

    def __init__(self, n: int, elems: int):
        self.bufs = [torch.empty(max(1, int(elems)), dtype=torch.int32).pin_memory()
                     for _ in range(n)]
        self.events = [None] * n
        self.i = 0

    def upload(self, src: np.ndarray, dst: torch.Tensor):
        """dst (device int32, contiguous) <- src (host), enqueued on the current stream."""
        j = self.i
        self.i = (j + 1) % len(self.bufs)
        if self.events[j] is not None:
            self.events[j].synchronize()
        n = src.size
        buf = self.bufs[j][:n]
        buf.numpy()[...] = src.reshape(-1)
        dst.view(-1)[:n].copy_(buf, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.events[j] = ev


class _HostPool:
    """Pinned, device-mapped host memory (omm_host_alloc), viewable from torch on the CPU."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.host = ctypes.c_void_p()
        self.dev = ctypes.c_void_p()
        if self.nbytes:
            _lib.call("omm_host_alloc", self.nbytes, ctypes.byref(self.host), ctypes.byref(self.dev),
                      error=BlockKVBackendError)

    @property
    def dev_ptr(self) -> int:
        return int(self.dev.value or 0)

    def cpu_view(self) -> torch.Tensor:
        if not self.nbytes:
            return torch.empty(0, dtype=torch.uint8)
        buf = (ctypes.c_uint8 * self.nbytes).from_address(self.host.value)
        return torch.frombuffer(buf, dtype=torch.uint8)

    def free(self):
        if self.host.value:
            _lib.call("omm_host_free", self.host, error=BlockKVBackendError)
            self.host = ctypes.c_void_p()
            self.dev = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PagedKVCache:
    """HBM + host paged KV cache of ``num_layers`` layers (see the module docstring).

    dtype: ``torch.bfloat16`` or ``"fp8"`` (OCP e4m3fn codes with one fp32 scale per
    (page, head) for K and for V).  Capacity: ``hbm_slots`` units per pool, or derived from
    ``hbm_budget_bytes`` (K + V + scales).  ``host_slots`` defaults to the units the HBM pool
    cannot hold plus one chunk of every layer and head (the slack a flush reserves).
    ``qk_fp8`` (fp8 caches): the selection quantises the queries to e4m3 per query row and runs
    Q K^T on fp8 MFMA with the K page codes, instead of widening the K codes to bf16 for the
    bf16 MFMA (the page scales apply to the scores either way).
    ``async_flush`` (byte-budget policy only): a flush enqueues its evictions and promotions on
    a stream of their own (copy engines) and returns; the moves are committed -- the unit table switched
    and the source slots freed -- at the next flush, or earlier when an operation needs them.
    Until then every moving unit is read from its source slot, which nothing rewrites.  The
    plan then keeps two chunks of slots free instead of one (the next chunk's, and the one the
    pending evictions release).
    """

    def __init__(self, num_layers: int, num_heads: int, head_dim: int, max_chunks: int,
                 chunk_len: int = 4680, page_tokens: int = 64, dtype=torch.bfloat16,
                 hbm_budget_bytes: Optional[int] = None, hbm_slots: Optional[int] = None,
                 host_slots: Optional[int] = None, lru_max_size: int = 0,
                 window_chunks: Optional[int] = 3, sink_chunks: int = 0,
                 keep_window_kv: bool = True, qk_fp8: bool = False,
                 stage_slots: int = 8192, async_flush: bool = True, device="cuda"):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise BlockKVBackendError("PagedKVCache lives on a GPU")
        self.L, self.H, self.D = int(num_layers), int(num_heads), int(head_dim)
        self.max_chunks = int(max_chunks)
        self.chunk_len, self.P = int(chunk_len), int(page_tokens)
        self.ppc = -(-self.chunk_len // self.P)
        self.fp8 = dtype == "fp8" or dtype == torch.float8_e4m3fn
        if not self.fp8 and dtype != torch.bfloat16:
            raise BlockKVBackendError(f"cache dtype must be bfloat16 or fp8, got {dtype}")
        if qk_fp8 and not self.fp8:
            raise BlockKVBackendError("qk_fp8 needs an fp8 cache")
        self.qk_fp8 = bool(qk_fp8)
        self.elem = 1 if self.fp8 else 2
        self.unit_elems = self.ppc * self.P * self.D
        self.unit_bytes = self.unit_elems * self.elem
        self.scale_bytes = self.ppc * 4 if self.fp8 else 0
        per_slot = 2 * (self.unit_bytes + self.scale_bytes)
        total_units = self.L * self.H * self.max_chunks
        if hbm_slots is None:
            if hbm_budget_bytes is None:
                hbm_slots = total_units
            else:
                hbm_slots = int(hbm_budget_bytes) // per_slot
        self.n_slots = int(min(hbm_slots, total_units))
        if self.n_slots < self.L * self.H:
            raise BlockKVBackendError(
                f"HBM pool of {self.n_slots} units cannot hold one chunk of every layer and head "
                f"({self.L * self.H} units)")
        self.lru_max_size = int(lru_max_size)
        if host_slots is None:
            if self.lru_max_size > 0:
                # the per-head count, not the pool, bounds residency: any unit may be evicted
                # (the reference preallocates a pinned slot per chunk, models/cache.py:970-1016)
                host_slots = total_units
            else:
                # every unit the HBM pool cannot hold, plus the chunk reserved at a flush and the
                # chunk of slots an asynchronous flush keeps free for its evictions to land in
                host_slots = min(total_units, total_units - self.n_slots + 2 * self.L * self.H)
        self.n_host = int(host_slots)
        self.hbm_budget_bytes = self.n_slots * per_slot
        # window None: the sink + window view is every chunk, and no chunk is protected from
        # eviction (the reference's rule without a window, models/cache.py:1060-1068)
        self.window = None if window_chunks is None else int(window_chunks)
        self.sink = int(sink_chunks)

        store = torch.uint8 if self.fp8 else torch.bfloat16
        shape = (self.n_slots, self.ppc, self.P, self.D)
        self.pool_k = torch.zeros(shape, dtype=store, device=self.device)
        self.pool_v = torch.zeros(shape, dtype=store, device=self.device)
        if self.fp8:
            self.scale_k = torch.ones((self.n_slots, self.ppc), dtype=torch.float32, device=self.device)
            self.scale_v = torch.ones_like(self.scale_k)
        else:
            self.scale_k = self.scale_v = None
        self._host_k = _HostPool(self.n_host * self.unit_bytes)
        self._host_v = _HostPool(self.n_host * self.unit_bytes)
        self._host_sk = _HostPool(self.n_host * self.scale_bytes)
        self._host_sv = _HostPool(self.n_host * self.scale_bytes)
        # HBM staging of the host-resident pages one selection call reads (``prefetch``)
        self.stage_slots = int(stage_slots) if self.n_host else 0
        ns = max(1, self.stage_slots)
        self._stage_k = torch.empty((ns, self.P, self.D), dtype=store, device=self.device)
        self._stage_v = torch.empty_like(self._stage_k)
        self._stage_sk = (torch.empty(ns, dtype=torch.float32, device=self.device)
                          if self.fp8 else None)
        self._stage_sv = torch.empty_like(self._stage_sk) if self.fp8 else None
        self._stage_epoch = torch.zeros((self.H, self.max_chunks, self.ppc), dtype=torch.int32,
                                        device=self.device)
        self._stage_slot = torch.full_like(self._stage_epoch, -1)
        self._stage_counter = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._side = None  # side stream of the staging and flush copies (created on first use)
        self._stage_pending = None
        # byte-budget policy: a flush enqueues its moves on the side stream and commits them
        # (table switch, source slots freed) at the next flush or whenever the host needs them
        self.async_flush = bool(async_flush) and self.lru_max_size == 0
        self._moves = None
        self._mover = None

        H, MC, L = self.H, self.max_chunks, self.L
        # one allocation each for every layer (the per-layer lists are views), so that a flush
        # reads all counters back with one synchronisation and a table upload is one copy
        self._unit_all = torch.full((L, H, MC), -1, dtype=torch.int32, device=self.device)
        self._stamp_all = torch.zeros((L, H, MC), dtype=torch.int32, device=self.device)
        self._reads_all = torch.zeros((L, H, MC), dtype=torch.int32, device=self.device)
        self._seen_all = torch.zeros((L, H, MC, self.ppc), dtype=torch.uint8, device=self.device)
        # per-call unit accesses (the reference's LRU access count, models/cache.py:673-699)
        self._touch_all = torch.zeros((L, H, MC), dtype=torch.int32, device=self.device)
        self.unit_table = list(self._unit_all.unbind(0))
        self.stamp = list(self._stamp_all.unbind(0))
        self.reads = list(self._reads_all.unbind(0))
        self.seen = list(self._seen_all.unbind(0))
        self.touches = list(self._touch_all.unbind(0))
        self._h_stamp = torch.empty((L, H, MC), dtype=torch.int32).pin_memory()
        self._h_reads = torch.empty((L, H, MC), dtype=torch.int32).pin_memory()
        self._h_pages = torch.empty((L, H, MC), dtype=torch.int32).pin_memory()
        self._h_touch = torch.empty((L, H, MC), dtype=torch.int32).pin_memory()
        self._ring = _UploadRing(8, max(L * H * MC, 2 * (self.n_slots + self.n_host)))
        self._d_idx = torch.empty(2 * (self.n_slots + self.n_host), dtype=torch.int32,
                                  device=self.device)
        ncb = MC * self.ppc
        self.k_cmp = [torch.zeros((1, ncb, H, self.D), dtype=torch.bfloat16, device=self.device)
                      for _ in range(self.L)]
        self.v_cmp = [torch.zeros_like(self.k_cmp[0]) for _ in range(self.L)]
        self.keep_window_kv = bool(keep_window_kv) and bool(self.window)
        if self.keep_window_kv:
            wshape = (self.window, self.chunk_len, H, self.D)
            self.win_k = [torch.zeros(wshape, dtype=torch.bfloat16, device=self.device)
                          for _ in range(self.L)]
            self.win_v = [torch.zeros_like(self.win_k[0]) for _ in range(self.L)]
        self._win_ids: Dict[tuple, torch.Tensor] = {}
        # update_cache('k_cmp_cache' / 'v_cmp_cache') hands in the caller's pooled rows; from
        # then on the append kernel leaves the pooled rows to the caller.  The pooled history
        # has its own window (None = all chunks, the reference pipeline's kv_cmp setting).
        self._pooled_by_caller = False
        self.cmp_window: Optional[int] = None
        self.cmp_sink = 0
        self._table_h = np.full((self.L, H, MC), -1, dtype=np.int32)
        self.n_chunks = [0] * self.L
        self._epoch = 0
        self._flush_epoch = 0
        self._staged_k: Dict[int, Tuple[torch.Tensor, int]] = {}
        self.reset()

    # ---------------------------------------------------------------- bookkeeping
    def reset(self):
        """Forget every chunk (pools keep their memory), as MMCache.reset (models/cache.py:771)."""
        if getattr(self, "_moves", None) is not None:
            self._moves[0].synchronize()  # copies in flight must land before slots are reused
        self._moves = None
        self._free_hbm = list(range(self.n_slots - 1, -1, -1))
        self._free_host = list(range(self.n_host - 1, -1, -1))
        self._table_h.fill(-1)
        self._heat = np.zeros(self._table_h.shape, dtype=np.float64)
        self._heat_init = np.zeros(self._table_h.shape, dtype=bool)
        self._unit_all.fill_(-1)
        self._stamp_all.zero_()
        self._reads_all.zero_()
        self._seen_all.zero_()
        self._touch_all.zero_()
        # staging-map entries carry the epoch of the call that staged them; epochs restart
        self._stage_epoch.zero_()
        self._stage_pending = None
        self._snaps = []
        self.n_chunks = [0] * self.L
        self._staged_k.clear()
        self._epoch = 0
        self._flush_epoch = 0
        # hits / misses: per-call unit accesses (a selection call reading a unit counts once)
        # served from HBM / from the host pool, the reference's LRU hit and (non-cold) miss
        # counts; *_units_touched: distinct units read between two flushes
        self.stats = {"hits": 0, "misses": 0, "hbm_units_touched": 0, "host_units_touched": 0,
                      "evicted_units": 0, "promoted_units": 0,
                      "evicted_bytes": 0, "promoted_bytes": 0, "flushes": 0,
                      "hbm_page_reads": 0, "host_page_reads": 0,
                      "hbm_pages_unique": 0, "host_pages_unique": 0}

    def next_epoch(self) -> int:
        self._epoch += 1
        if self._epoch >= 2 ** 31 - 1:
            raise BlockKVBackendError("epoch counter exhausted; call reset()")
        return self._epoch

    def _upload_table(self, layer: Optional[int] = None):
        """Device unit table of one layer (or all) from the host's, asynchronously."""
        if layer is None:
            self._ring.upload(self._table_h, self._unit_all)
        else:
            self._ring.upload(self._table_h[layer], self.unit_table[layer])

    def layer_view(self, layer: int) -> _lib.PagedKV:
        """The omm_paged_kv struct of one layer."""
        kv = _lib.PagedKV()
        kv.pool_k, kv.pool_v = self.pool_k.data_ptr(), self.pool_v.data_ptr()
        if self.fp8:
            kv.scale_k, kv.scale_v = self.scale_k.data_ptr(), self.scale_v.data_ptr()
            kv.host_scale_k, kv.host_scale_v = self._host_sk.dev_ptr, self._host_sv.dev_ptr
        kv.host_k, kv.host_v = self._host_k.dev_ptr, self._host_v.dev_ptr
        kv.unit_table = self.unit_table[layer].data_ptr()
        kv.stamp = self.stamp[layer].data_ptr()
        kv.reads = self.reads[layer].data_ptr()
        kv.page_seen = self.seen[layer].data_ptr()
        kv.touches = self.touches[layer].data_ptr()
        kv.num_heads, kv.max_chunks, kv.n_chunks = self.H, self.max_chunks, self.n_chunks[layer]
        kv.chunk_len, kv.page_tokens, kv.pages_per_chunk = self.chunk_len, self.P, self.ppc
        kv.head_dim = self.D
        kv.dtype = _lib.OMM_FP8E4M3 if self.fp8 else _lib.OMM_BF16
        kv.n_slots, kv.n_host_slots = self.n_slots, self.n_host
        kv.qk_fp8 = 1 if self.qk_fp8 else 0
        if self.stage_slots:
            kv.stage_k, kv.stage_v = self._stage_k.data_ptr(), self._stage_v.data_ptr()
            if self.fp8:
                kv.stage_scale_k = self._stage_sk.data_ptr()
                kv.stage_scale_v = self._stage_sv.data_ptr()
            kv.stage_map_epoch = self._stage_epoch.data_ptr()
            kv.stage_map_slot = self._stage_slot.data_ptr()
            kv.stage_counter = self._stage_counter.data_ptr()
            kv.stage_slots = self.stage_slots
        return kv

    # ---------------------------------------------------------------- append
    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, cid: int):
        """Write chunk ``cid`` (k, v: bf16 [1, chunk_len, H, D]) of one layer.

        Rewriting a chunk (the reference's 4 denoise + 1 context forwards per AR chunk) reuses its
        units.  Also writes the pooled keys / values of its pages (``k_cmp`` / ``v_cmp``)."""
        _lib.require_cuda((k, "k"), (v, "v"))
        if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise BlockKVBackendError("append expects bf16 keys and values")
        if not (0 <= cid < self.max_chunks):
            raise BlockKVBackendError(f"chunk id {cid} outside [0, {self.max_chunks})")
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != 1 or k.shape[2:] != (self.H, self.D):
            raise BlockKVBackendError(f"k / v must be [1, S, {self.H}, {self.D}], got "
                                      f"{tuple(k.shape)} / {tuple(v.shape)}")
        S = k.shape[1]
        if S != self.chunk_len:
            # attention reads every page of a written chunk with the token counts chunk_len
            # fixes, so a shorter write would expose unwritten slots
            raise BlockKVBackendError(f"{S} tokens for a chunk of {self.chunk_len} (whole chunks "
                                      "only)")
        if k.stride(3) != 1 or k.stride(1) % 8 or k.stride(2) % 8 or k.data_ptr() % 16:
            k = k.contiguous()
        if v.stride(3) != 1 or v.stride(1) % 8 or v.stride(2) % 8 or v.data_ptr() % 16:
            v = v.contiguous()
        if self._pending_in(layer, cid):
            self._commit()  # a unit of this chunk is moving: its copy must read the old data
        row = self._table_h[layer, :, cid]
        for sn in self._snaps:  # a snapshot keeps the version it saw: write to a new slot
            for h in range(self.H):
                u = (layer, h, cid)
                if u in sn["units"] and sn["units"][u] is None and row[h] != -1:
                    sn["units"][u] = int(row[h])
                    row[h] = -1
        if (row < 0).any():
            # making room may evict units of this very chunk (row is a view of the table), which
            # then need a slot too: repeat until the free list covers every unit to place (at
            # most H rounds; _make_room raises when it cannot free enough)
            need = int((row < 0).sum())
            while len(self._free_hbm) < need:
                self._make_room(need)
                need = int((row < 0).sum())
            changed = False
            for h in np.nonzero(row < 0)[0]:
                if row[h] <= -2:  # host-resident unit being rewritten: bring it home
                    self._free_host.append(-2 - int(row[h]))
                row[h] = self._free_hbm.pop()
                changed = True
            if changed:
                self._upload_table(layer)
        self.n_chunks[layer] = max(self.n_chunks[layer], cid + 1)
        kv = self.layer_view(layer)
        pool_k = pool_v = None
        if not self._pooled_by_caller:
            pool_k, pool_v = _lib.view4(self.k_cmp[layer]), _lib.view4(self.v_cmp[layer])
        ring_k = ring_v = None
        if self.keep_window_kv:  # the window ring's slot, written by the append kernel
            w = cid % self.window
            ring_k = _lib.view4(self.win_k[layer][w:w + 1, :S])
            ring_v = _lib.view4(self.win_v[layer][w:w + 1, :S])
        _lib.call("omm_paged_append_ring", ctypes.byref(kv), _lib.view4(k), _lib.view4(v),
                  int(cid), int(S), pool_k, pool_v, ring_k, ring_v, self.next_epoch(),
                  _lib.stream_of(k), error=BlockKVBackendError)

    @staticmethod
    def _window_chunks(n_valid: int, window: Optional[int], sink: int):
        """Chunk ids of the sink + window view of chunks 0..n_valid-1, ascending: all of them
        without a window; else the first ``sink`` chunks and the last ``window`` (the window
        never reaches into the sinks), as MMCache._resolve_window_range (models/cache.py:557-570)."""
        if window is None:
            return list(range(n_valid))
        s = min(int(sink), n_valid)
        start = max(s, n_valid - int(window))
        return list(range(s)) + list(range(start, n_valid))

    def _gather_chunk(self, layer: int, which: str, cid: int) -> torch.Tensor:
        """Chunk ``cid`` of every head as bf16 [chunk_len, H, D], read from the pools (fp8 pages
        dequantised with their scales; host-resident units copied over the host link)."""
        slots = self._table_h[layer, :, cid]
        if (slots == -1).any():
            raise BlockKVBackendError(f"chunk {cid} of layer {layer} was never written")
        pool = self.pool_k if which == "k" else self.pool_v
        scales = self.scale_k if which == "k" else self.scale_v
        rows = []
        for h, s in enumerate(slots.tolist()):
            if s >= 0:
                unit = pool[s]
                sc = scales[s] if self.fp8 else None
            else:
                hs, ub = -2 - s, self.unit_bytes
                host = (self._host_k if which == "k" else self._host_v).cpu_view()
                torch.cuda.current_stream(self.device).synchronize()  # pending moves land first
                unit = host[hs * ub:(hs + 1) * ub].view(pool.dtype).view(pool.shape[1:]).to(
                    self.device)
                sc = None
                if self.fp8:
                    sb = self.scale_bytes
                    hsc = (self._host_sk if which == "k" else self._host_sv).cpu_view()
                    sc = hsc[hs * sb:(hs + 1) * sb].view(torch.float32).to(self.device)
            if self.fp8:
                unit = (unit.view(torch.float8_e4m3fn).float() * sc[:, None, None]).to(
                    torch.bfloat16)
            rows.append(unit.reshape(self.ppc * self.P, self.D)[:self.chunk_len])
        return torch.stack(rows, dim=1)

    def _window_tokens(self, layer: int, which: str, cid: int, current: torch.Tensor):
        """Sink + window K or V up to chunk ``cid`` as [1, tokens, H, D], chunks ascending;
        chunk ``cid`` itself is ``current`` (the caller's tensor)."""
        parts = []
        for c in self._window_chunks(cid + 1, self.window, self.sink):
            if c == cid:
                parts.append(current[0])
            elif self.keep_window_kv and cid - c < self.window:  # keep_window_kv: window > 0
                ring = self.win_k[layer] if which == "k" else self.win_v[layer]
                parts.append(ring[c % self.window])
            else:
                parts.append(self._gather_chunk(layer, which, c))
        if not parts:  # a zero-chunk window: an empty view
            return current.new_empty((1, 0) + tuple(current.shape[2:]))
        return parts[0].unsqueeze(0) if len(parts) == 1 else torch.cat(parts, 0).unsqueeze(0)

    def _write_pooled(self, name: str, hidden_state: torch.Tensor, layer_idx: int, start: int):
        rows = self.k_cmp[layer_idx] if name == "k_cmp_cache" else self.v_cmp[layer_idx]
        n = hidden_state.shape[1]
        if hidden_state.dim() != 4 or hidden_state.shape[0] != 1 or n != self.ppc or \
                tuple(hidden_state.shape[2:]) != (self.H, self.D):
            raise BlockKVBackendError(
                f"{name} takes one chunk's pooled rows [1, {self.ppc}, {self.H}, {self.D}], got "
                f"{tuple(hidden_state.shape)}")
        if start % self.ppc:
            raise BlockKVBackendError(f"{name}: start_id {start} is not a chunk boundary")
        cid = start // self.ppc
        if not (0 <= cid < self.max_chunks):
            raise BlockKVBackendError(f"chunk id {cid} outside [0, {self.max_chunks})")
        self._pooled_by_caller = True
        rows[:, start:start + n].copy_(hidden_state)
        keep = self._window_chunks(cid + 1, self.cmp_window, self.cmp_sink)
        if keep == list(range(keep[0], keep[-1] + 1)):  # one contiguous range: a view
            return rows[:, keep[0] * self.ppc:(keep[-1] + 1) * self.ppc]
        return torch.cat([rows[:, c * self.ppc:(c + 1) * self.ppc] for c in keep], 1)

    def update_cache(self, name: str, hidden_state: torch.Tensor, layer_idx: int, start_id):
        """The reference's ``MMCache.update_cache`` (models/cache.py:439-522) for the four cache
        names of the NSA model's AR branch (causal_wan_nsa_model.py:479-504):

        * ``'k_cmp_cache'`` / ``'v_cmp_cache'`` (``start_id`` in pooled rows): store one chunk's
          pooled keys / values and return the pooled history ([1, rows, H, D]; all chunks unless
          ``cmp_window`` is set), a view valid until the next write of this layer;
        * ``'k_cache'`` (``start_id`` in tokens): take the chunk's keys and return the sink +
          window keys ([1, tokens, H, D], chunks ascending, this chunk last);
        * ``'v_cache'``: write the chunk (keys and values) into its pages and return the sink +
          window values the same way.

        Chunks are whole (``chunk_len`` tokens).  ``start_id`` may be a tensor (read once)."""
        start = int(start_id.item()) if isinstance(start_id, torch.Tensor) else int(start_id)
        if name in ("k_cmp_cache", "v_cmp_cache"):
            return self._write_pooled(name, hidden_state, layer_idx, start)
        if name not in ("k_cache", "v_cache"):
            raise BlockKVBackendError(f"unknown cache name {name!r} (expected 'k_cache', "
                                      "'v_cache', 'k_cmp_cache' or 'v_cmp_cache')")
        if start % self.chunk_len:
            raise BlockKVBackendError(f"{name}: start_id {start} is not a chunk boundary")
        cid = start // self.chunk_len
        if name == "k_cache":
            if not (0 <= cid < self.max_chunks):
                raise BlockKVBackendError(f"chunk id {cid} outside [0, {self.max_chunks})")
            self._staged_k[layer_idx] = (hidden_state, cid)
            if self.keep_window_kv:
                self.win_k[layer_idx][cid % self.window].copy_(hidden_state[0])
            return self._window_tokens(layer_idx, "k", cid, hidden_state)
        if layer_idx not in self._staged_k or self._staged_k[layer_idx][1] != cid:
            raise BlockKVBackendError("update_cache('v_cache') needs the matching 'k_cache' first")
        k, _ = self._staged_k.pop(layer_idx)
        self.append(layer_idx, k, hidden_state, cid)
        return self._window_tokens(layer_idx, "v", cid, hidden_state)

    @property
    def _has_cpu_chunks(self) -> bool:
        """Whether any unit lives in the host pool (the reference's flag, models/cache.py:66)."""
        return bool((self._table_h <= -2).any())

    @property
    def block_seqlens(self) -> Dict[str, int]:
        """Tokens (pooled rows for the cmp names) per chunk, as MMCache.block_seqlens."""
        return {"k_cache": self.chunk_len, "v_cache": self.chunk_len,
                "k_cmp_cache": self.ppc, "v_cmp_cache": self.ppc}

    def window_kv(self, layer: int, upto: Optional[int] = None):
        """K and V of the last ``window_chunks`` chunks as [1, tokens, H, D] (chunk order need not
        be ascending: attention over the window is permutation invariant)."""
        if not self.keep_window_kv:
            raise BlockKVBackendError("window K/V are not kept (keep_window_kv=False)")
        n = self.n_chunks[layer] if upto is None else upto
        w = min(n, self.window)
        L = self.chunk_len
        return (self.win_k[layer][:w].reshape(1, w * L, self.H, self.D),
                self.win_v[layer][:w].reshape(1, w * L, self.H, self.D))

    def window_attention(self, q: torch.Tensor, layer: int, softmax_scale: Optional[float] = None,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Sliding-window attention (the reference's SWA branch, causal_wan_nsa_model.py:508, whose
        K/V are the sink + window chunks update_cache returns, models/cache.py:576-588): softmax
        attention of q (bf16 [1, M, H, D]) over every token of the first ``sink_chunks`` and the
        last ``window_chunks`` chunks written.

        With ``keep_window_kv`` and no sinks the dense ring is read (``window_kv``); otherwise
        the pages of those chunks are read in place by the paged selection kernel, every page
        listed for every query group (sink and window units are protected from eviction, and a
        host-resident page would still be read).  The paged read neither stamps the LRU nor
        counts page reads.  An fp8 cache with sinks gathers the dequantised pages first."""
        from .selection import dense_attention
        n = self.n_chunks[layer]
        chunks = self._window_chunks(n, self.window, self.sink)
        if self.keep_window_kv and (self.sink == 0 or self.fp8):
            if self.sink == 0:
                wk, wv = self.window_kv(layer)
            else:
                wk = torch.cat([self._gather_chunk(layer, "k", c) for c in chunks], 0)[None]
                wv = torch.cat([self._gather_chunk(layer, "v", c) for c in chunks], 0)[None]
            return dense_attention(q, wk, wv, scale=softmax_scale, out=out)
        _lib.require_cuda((q, "q"))
        if q.dtype != torch.bfloat16:
            raise BlockKVBackendError(f"window attention needs bf16 queries, got {q.dtype}")
        B, M, H, D = q.shape
        if out is None:
            out = torch.empty_like(q)
        if not chunks:
            return out.zero_()
        G = 128  # every group lists the same pages: 128-query groups share each K/V tile
        T = len(chunks) * self.ppc
        key = (q.device, tuple(chunks))
        ids = self._win_ids.get(key)
        if ids is None:
            ids = torch.cat([torch.arange(c * self.ppc, (c + 1) * self.ppc, dtype=torch.int32)
                             for c in chunks]).to(q.device)
            self._win_ids = {key: ids}
        ids4 = ids.view(1, 1, 1, T).expand(B, -(-M // G), H, T)
        kv = self.layer_view(layer)
        kv.stamp = None
        kv.reads = None
        kv.page_seen = None
        kv.touches = None
        kv.stage_map_epoch = None
        scale = softmax_scale if softmax_scale is not None else D ** -0.5
        _lib.call("omm_sel_fwd_paged", _lib.view4(q), _lib.view4(ids4), ctypes.byref(kv), G,
                  float(scale), _lib.view4(out), None, 0, _lib.stream_of(q),
                  error=BlockKVBackendError)
        return out

    def cmp_history(self, layer: int):
        """Pooled keys / values of every page written so far: [1, n_chunks*ppc, H, D] each."""
        n = self.n_chunks[layer] * self.ppc
        return self.k_cmp[layer][:, :n], self.v_cmp[layer][:, :n]

    # ---------------------------------------------------------------- selection
    def prefetch(self, block_indices: torch.Tensor, layer: int):
        """Start staging the host-resident pages a ``select`` with these ids will read: one
        ``omm_paged_stage`` on a side stream (default priority), ordered after the work already
        enqueued on the current stream (the top-k that produced the ids), copying each distinct
        host page once into the HBM staging pool.  Returns the handle to pass to ``select``,
        which then waits for the copies and reads those pages from HBM.  Work enqueued on the
        current stream in between (the compressed and window branches) overlaps the copies.
        One prefetch may be outstanding per cache; ids of another layer or call must not be
        selected with this handle."""
        if self._stage_pending is not None:
            raise BlockKVBackendError("a prefetch is already outstanding; select() it first")
        _lib.require_cuda((block_indices, "block_indices"))
        if block_indices.dtype != torch.int32:
            block_indices = block_indices.to(torch.int32)
        epoch = self.next_epoch()
        handle = {"epoch": epoch, "layer": layer, "event": None, "ids": block_indices}
        if self.stage_slots and bool((self._table_h[layer] <= -2).any()):
            main = torch.cuda.current_stream(self.device)
            if self._side is None:
                self._side = torch.cuda.Stream(device=self.device)
            self._side.wait_stream(main)
            block_indices.record_stream(self._side)
            kv = self.layer_view(layer)
            with torch.cuda.stream(self._side):
                _lib.call("omm_paged_stage", ctypes.byref(kv), _lib.view4(block_indices),
                          epoch, _lib.stream_of(block_indices), error=BlockKVBackendError)
                ev = torch.cuda.Event()
                ev.record(self._side)
            handle["event"] = ev
        self._stage_pending = handle
        return handle

    def select(self, q: torch.Tensor, block_indices: torch.Tensor, layer: int, group_size: int,
               softmax_scale: Optional[float] = None, return_lse: bool = False,
               out: Optional[torch.Tensor] = None, gates: Optional[torch.Tensor] = None,
               o_cmp: Optional[torch.Tensor] = None, o_swa: Optional[torch.Tensor] = None,
               prefetch: Optional[dict] = None):
        """Selection attention of q (bf16 [1, M, H, D]) over the pages listed in block_indices
        (int32 [1, ceil(M/G), H, T], page id = chunk * pages_per_chunk + page).

        With ``gates`` (bf16 [1, M, H, 3], after the sigmoid) and the other two branch outputs
        ``o_cmp`` / ``o_swa`` the kernel writes the NSA branch mix g0*o_cmp + g1*o_slc + g2*o_swa
        (causal_wan_nsa_model.py:541-546) instead of o_slc, in one fp32 pass.  ``prefetch``: the
        handle of ``prefetch(block_indices, layer)``; staged pages are then read from HBM (the
        result is bit-identical either way)."""
        _lib.require_cuda((q, "q"), (block_indices, "block_indices"))
        if q.dtype != torch.bfloat16:
            raise BlockKVBackendError(f"paged selection needs bf16 queries, got {q.dtype}")
        if block_indices.dtype != torch.int32:
            block_indices = block_indices.to(torch.int32)
        if prefetch is not None:
            if prefetch is not self._stage_pending or prefetch["layer"] != layer or \
                    prefetch["ids"].data_ptr() != block_indices.data_ptr():
                raise BlockKVBackendError("prefetch handle does not match this select (layer, "
                                          "ids) or was already used")
            self._stage_pending = None
            if prefetch["event"] is not None:
                torch.cuda.current_stream(self.device).wait_event(prefetch["event"])
            epoch = prefetch["epoch"]
        else:
            epoch = self.next_epoch()
        B, M, H, D = q.shape
        scale = softmax_scale if softmax_scale is not None else D ** -0.5
        if out is None:
            out = torch.empty_like(q)
        lse = torch.empty((B, H, M), dtype=torch.float32, device=q.device) if return_lse else None
        kv = self.layer_view(layer)
        if gates is not None:
            if o_cmp is None or o_swa is None:
                raise BlockKVBackendError("the gated selection needs o_cmp and o_swa")
            for t, name in ((gates, "gates"), (o_cmp, "o_cmp"), (o_swa, "o_swa")):
                if t.dtype != torch.bfloat16 or not t.is_cuda:
                    raise BlockKVBackendError(f"{name} must be a bf16 CUDA tensor")
            _lib.call("omm_sel_fwd_paged_gated", _lib.view4(q), _lib.view4(block_indices),
                      ctypes.byref(kv), int(group_size), float(scale), _lib.view4(gates),
                      _lib.view4(o_cmp), _lib.view4(o_swa), _lib.view4(out),
                      lse.data_ptr() if lse is not None else None, epoch,
                      _lib.stream_of(q), error=BlockKVBackendError)
        else:
            _lib.call("omm_sel_fwd_paged", _lib.view4(q), _lib.view4(block_indices),
                      ctypes.byref(kv), int(group_size), float(scale), _lib.view4(out),
                      lse.data_ptr() if lse is not None else None, epoch,
                      _lib.stream_of(q), error=BlockKVBackendError)
        return (out, lse) if return_lse else out

    # ---------------------------------------------------------------- residency
    def _protected(self) -> np.ndarray:
        mask = np.zeros((self.L, self.H, self.max_chunks), dtype=bool)
        c = np.arange(self.max_chunks)
        for l in range(self.L):
            n = self.n_chunks[l]
            if self.window is None:
                continue
            prot = (c < min(self.sink, n)) | ((c >= max(0, n - self.window)) & (c < n))
            mask[l, :, :] = prot[None, :]
        return mask

    def _cap(self, reserve: int) -> int:
        """HBM slots the residency plan may fill: all of them but the reserve and those held by
        snapshots (``snapshot_chunks``) for units rewritten since."""
        held = sum(1 for sn in self._snaps for st in sn["units"].values()
                   if st is not None and st >= 0)
        return self.n_slots - reserve - held

    def head_capacity(self, reserve: int = 0) -> int:
        """HBM units each (layer, head) may keep: ``lru_max_size`` (the reference's count), or an
        equal share of the budget left after ``reserve`` slots (the next chunk's)."""
        if self.lru_max_size > 0:
            return self.lru_max_size
        return max(1, self._cap(reserve) // (self.L * self.H))

    def _plan(self, st: np.ndarray, reserve: int, rd: Optional[np.ndarray] = None):
        if self.lru_max_size > 0 or rd is None:
            return self._plan_lru(st, reserve)
        return self._plan_cost(st, rd, reserve)

    def _plan_lru(self, st: np.ndarray, reserve: int):
        """Desired HBM set: per (layer, head), its sink / window units, then its most recent
        (epoch, chunk) units up to ``head_capacity()``."""
        written = self._table_h != -1
        prot = self._protected() & written
        # rank key: later epoch first, then larger chunk id (the reference's touch order)
        key = st * (1 << 20) + np.arange(self.max_chunks)[None, None, :]
        key = np.where(written & ~prot, key, -1)
        cap = self.head_capacity(reserve)
        room = np.maximum(0, cap - prot.sum(-1))                          # [L, H]
        order = np.argsort(-key, axis=-1, kind="stable")                  # most recent first
        rank = np.empty_like(order)
        np.put_along_axis(rank, order, np.arange(self.max_chunks)[None, None, :].repeat(
            self.L, 0).repeat(self.H, 1), axis=-1)
        desired = prot | ((key >= 0) & (rank < room[..., None]))
        total = int(desired.sum())
        if total > self._cap(reserve):
            raise BlockKVBackendError(
                f"{total} units wanted in HBM exceed the {self._cap(reserve)} slots left after "
                f"reserving {reserve} for the next chunk (lower lru_max_size or raise the budget)")
        return desired

    def _plan_cost(self, st: np.ndarray, rd: np.ndarray, reserve: int):
        """Budget policy: keep what is resident, evict the coldest units only to make room, and
        swap a host unit in when its page reads beat a resident unit's by more than the pages a
        swap moves (two units each way).  ``rd``: the units' heat, a moving average of page reads
        per flush interval (``_update_heat``)."""
        written = self._table_h != -1
        prot = (self._protected() & written).reshape(-1)
        res = (self._table_h >= 0).reshape(-1)
        host = (self._table_h <= -2).reshape(-1)
        reads = rd.reshape(-1).astype(np.float64)
        stamp = st.reshape(-1)
        chunk = np.broadcast_to(np.arange(self.max_chunks), st.shape).reshape(-1)
        desired = res | prot
        cap = self._cap(reserve)
        # coldest first: fewest pages read, then oldest touch, then oldest chunk (two stable
        # sorts: by the packed (touch, chunk) key, then by reads)
        def cold(idx):
            idx = idx[np.argsort(stamp[idx] * (1 << 20) + chunk[idx], kind="stable")]
            return idx[np.argsort(reads[idx], kind="stable")]
        movable = cold(np.flatnonzero(desired & ~prot))
        over = int(desired.sum()) - cap
        if over > 0:
            if over > movable.size:
                raise BlockKVBackendError(
                    f"{int(prot.sum())} sink / window units exceed the {cap} HBM slots left after "
                    f"reserving {reserve}")
            desired[movable[:over]] = False
            movable = movable[over:]
        hot = np.flatnonzero(host & ~desired & (reads > 0))
        hot = hot[np.argsort(-reads[hot], kind="stable")]
        unit_pages = self.ppc
        # free slots first, hottest first, for units read more than a promotion moves
        free = cap - int(desired.sum())
        i = min(max(0, free), int(np.argmin(np.append(reads[hot] > unit_pages, False))))
        desired[hot[:i]] = True
        # then swaps, hottest host unit against coldest resident one, while the reads gained
        # beat the pages moved (both lists sorted, so the swaps that pay are a prefix)
        k = min(hot.size - i, movable.size)
        pays = reads[hot[i:i + k]] > reads[movable[:k]] + 2 * unit_pages
        j = int(np.argmin(np.append(pays, False)))
        desired[hot[i:i + j]] = True
        desired[movable[:j]] = False
        return desired.reshape(self._table_h.shape)

    def _take_slots(self, layer_units, to_host: bool):
        """Host side of one batch of moves: reassign the units' slots in the host table and the
        free lists; returns (src slots, dst slots)."""
        src, dst = [], []
        for (l, h, c) in layer_units:
            s = int(self._table_h[l, h, c])
            if to_host:
                d = self._free_host.pop()
                src.append(s)
                dst.append(d)
                self._table_h[l, h, c] = -2 - d
                self._free_hbm.append(s)
            else:
                hs = -2 - s
                d = self._free_hbm.pop()
                src.append(hs)
                dst.append(d)
                self._table_h[l, h, c] = d
                self._free_host.append(hs)
        return src, dst

    def _copy_batches(self, batches):
        """Enqueue the copies of planned batches [(to_host, src, dst)]: one upload of every
        batch's slot indices, then one omm_copy_units launch per batch.  Nothing synchronises:
        the copies and the index upload are ordered on the stream before any later kernel."""
        if not batches:
            return
        idx = np.concatenate([np.asarray(sd, dtype=np.int32) for _, src, dst in batches
                              for sd in (src, dst)])
        self._ring.upload(idx, self._d_idx)
        hk, hv = self._host_k.dev_ptr, self._host_v.dev_ptr
        pk, pv = self.pool_k.data_ptr(), self.pool_v.data_ptr()
        if self.fp8:
            hsk, hsv = self._host_sk.dev_ptr, self._host_sv.dev_ptr
            psk, psv = self.scale_k.data_ptr(), self.scale_v.data_ptr()
        else:
            hsk = hsv = psk = psv = None
        base = self._d_idx.data_ptr()
        off = 0
        for to_host, src, dst in batches:
            n = len(src)
            if to_host:
                args = (pk, hk, pv, hv, psk, hsk, psv, hsv)
                limits = (self.n_slots, self.n_host)
            else:
                args = (hk, pk, hv, pv, hsk, psk, hsv, psv)
                limits = (self.n_host, self.n_slots)
            _lib.call("omm_copy_units", *args, base + 4 * off, base + 4 * (off + n), n, *limits,
                      self.unit_bytes, self.scale_bytes, _lib.stream_of(self.pool_k),
                      error=BlockKVBackendError)
            off += 2 * n

    def _apply(self, desired: np.ndarray, st: Optional[np.ndarray] = None):
        """Move units so that HBM holds exactly the desired written units.  Evictions and
        promotions alternate in batches bounded by the free slots of the receiving pool (a
        promotion frees a host slot, an eviction an HBM slot), so a full host pool never
        blocks a swap; the least recent units leave first, the most recent arrive first.
        ``st``: host copy of the stamps (read back when needed and not given)."""
        resident = self._table_h >= 0
        on_host = self._table_h <= -2
        evict = np.argwhere(resident & ~desired)
        promote = np.argwhere(on_host & desired)
        if len(evict) > 1 or len(promote) > 1:
            if st is None:
                st = self._counts()[0]
            key = lambda u: st[u[:, 0], u[:, 1], u[:, 2]] * (1 << 20) + u[:, 2]
            if len(evict) > 1:
                evict = evict[np.argsort(key(evict), kind="stable")]
            if len(promote) > 1:
                promote = promote[np.argsort(-key(promote), kind="stable")]
        evict = [tuple(u) for u in evict]
        promote = [tuple(u) for u in promote]
        n_ev = n_pr = 0
        batches = []
        while evict or promote:
            ne = min(len(evict), len(self._free_host))
            if ne:
                batches.append((True,) + self._take_slots(evict[:ne], to_host=True))
                evict, n_ev = evict[ne:], n_ev + ne
            npr = min(len(promote), len(self._free_hbm))
            if npr:
                batches.append((False,) + self._take_slots(promote[:npr], to_host=False))
                promote, n_pr = promote[npr:], n_pr + npr
            if ne == 0 and npr == 0:
                raise BlockKVBackendError(
                    f"no free slot to swap through ({len(evict)} evictions, {len(promote)} "
                    f"promotions pending)")
        self._copy_batches(batches)
        if batches:
            self._upload_table()
        unit = 2 * (self.unit_bytes + self.scale_bytes)
        self.stats["evicted_units"] += n_ev
        self.stats["promoted_units"] += n_pr
        self.stats["evicted_bytes"] += n_ev * unit
        self.stats["promoted_bytes"] += n_pr * unit
        return n_ev, n_pr

    def _move_stream(self) -> torch.cuda.Stream:
        """Stream of an asynchronous flush's copies (default priority), apart from the staging
        stream so that a prefetch never queues behind a flush's evictions."""
        if self._mover is None:
            self._mover = torch.cuda.Stream(device=self.device)
        return self._mover

    def _pick_moves(self, desired: np.ndarray, st: np.ndarray, keep_free: int):
        """The moves an asynchronous flush makes towards ``desired``: evictions, least recent
        first, as many as there are free host slots; promotions, most recent first, into the
        free HBM slots beyond the ``keep_free`` the caller reserves next.  A move that finds no
        free slot waits for a later flush (a pending move frees its source only when
        committed).  Returns (evict, promote) as [n, 3] (layer, head, chunk) arrays."""
        evict = np.argwhere((self._table_h >= 0) & ~desired)
        promote = np.argwhere((self._table_h <= -2) & desired)
        key = lambda u: st[u[:, 0], u[:, 1], u[:, 2]] * (1 << 20) + u[:, 2]
        evict = evict[np.argsort(key(evict), kind="stable")][:len(self._free_host)]
        room = max(0, len(self._free_hbm) - keep_free)
        promote = promote[np.argsort(-key(promote), kind="stable")][:room]
        return evict, promote

    def _apply_async(self, evict: np.ndarray, promote: np.ndarray):
        """Enqueue the moves of ``_pick_moves`` on the move stream and leave them pending
        (``_commit``).  Within a batch the units are paired with destination slots in
        source-slot order, so that units adjacent in both pools go in one copy."""
        if len(evict) == 0 and len(promote) == 0:
            return 0, 0
        moves = []
        main = torch.cuda.current_stream(self.device)
        side = self._move_stream()
        side.wait_stream(main)  # the units' last writes (appends) come first
        hk, hv = self._host_k.host.value, self._host_v.host.value
        pk, pv = self.pool_k.data_ptr(), self.pool_v.data_ptr()
        if self.fp8:
            hsk, hsv = self._host_sk.host.value, self._host_sv.host.value
            psk, psv = self.scale_k.data_ptr(), self.scale_v.data_ptr()
        else:
            hsk = hsv = psk = psv = None
        for units, to_host in ((evict, True), (promote, False)):
            if len(units) == 0:
                continue
            src = self._table_h[units[:, 0], units[:, 1], units[:, 2]].astype(np.int64)
            if not to_host:
                src = -2 - src
            order = np.argsort(src, kind="stable")
            units, src = units[order], src[order]
            free = self._free_host if to_host else self._free_hbm
            free.sort(reverse=True)  # pops ascend: consecutive destinations where possible
            dst = np.array([free.pop() for _ in range(len(units))], dtype=np.int64)
            for (l, h, c), a, b in zip(units.tolist(), src.tolist(), dst.tolist()):
                # (unit, table entry once committed, slot released then)
                moves.append(((l, h, c), -2 - b if to_host else b, a if to_host else -2 - a))
            if to_host:
                args = (pk, hk, pv, hv, psk, hsk, psv, hsv)
                limits = (self.n_slots, self.n_host)
            else:
                args = (hk, pk, hv, pv, hsk, psk, hsv, psv)
                limits = (self.n_host, self.n_slots)
            s32, d32 = src.astype(np.int32), dst.astype(np.int32)
            _lib.call("omm_copy_units_async", *args, s32.ctypes.data, d32.ctypes.data,
                      len(units), *limits, self.unit_bytes, self.scale_bytes, side.cuda_stream,
                      error=BlockKVBackendError)
        ev = torch.cuda.Event()
        ev.record(side)
        self._moves = (ev, moves, {(l, c) for (l, _, c), _, _ in moves})
        n_ev, n_pr = len(evict), len(promote)
        unit = 2 * (self.unit_bytes + self.scale_bytes)
        self.stats["evicted_units"] += n_ev
        self.stats["promoted_units"] += n_pr
        self.stats["evicted_bytes"] += n_ev * unit
        self.stats["promoted_bytes"] += n_pr * unit
        return n_ev, n_pr

    def _commit(self, upload: bool = True) -> bool:
        """Commit the pending moves of an asynchronous flush: the current stream waits for
        their copies, the unit table switches to the destination slots and the source slots
        return to the free lists (work enqueued from now on may reuse them).  Returns whether
        the table changed (uploaded unless ``upload`` is false)."""
        if self._moves is None:
            return False
        ev, moves, _ = self._moves
        self._moves = None
        torch.cuda.current_stream(self.device).wait_event(ev)
        for (l, h, c), entry, old in moves:
            self._table_h[l, h, c] = entry
            self._release_slot(old)
        if upload:
            self._upload_table()
        return True

    def _pending_in(self, layer: int, cid: int) -> bool:
        return self._moves is not None and (layer, cid) in self._moves[2]

    def _counts(self):
        """Host copies of every layer's stamps, page-read counts, distinct pages read per unit
        (summed on the device) and per-call unit accesses (one synchronisation); the arrays are
        reused by the next call."""
        self._h_stamp.copy_(self._stamp_all, non_blocking=True)
        self._h_reads.copy_(self._reads_all, non_blocking=True)
        self._h_pages.copy_(self._seen_all.sum(-1, dtype=torch.int32), non_blocking=True)
        self._h_touch.copy_(self._touch_all, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        return (self._h_stamp.numpy().astype(np.int64), self._h_reads.numpy(),
                self._h_pages.numpy(), self._h_touch.numpy())

    def _update_heat(self, rd: np.ndarray, written: np.ndarray):
        """Heat of every unit: an exponential moving average (weight HEAT_ALPHA) of its page
        reads per flush interval, over the intervals in which it could be selected (written and
        outside the sink / window, which the top-k excludes).  A unit that becomes selectable
        starts from the mean heat of the others, so leaving the window (zero reads until then)
        does not make it look cold, and one interval's random fluctuations do not trigger swaps."""
        eligible = written & ~self._protected()
        new = eligible & ~self._heat_init
        if new.any():
            old = eligible & self._heat_init
            prior = float(self._heat[old].mean()) if old.any() else float(rd[new].mean())
            self._heat[new] = prior
            self._heat_init |= new
        a = self.HEAT_ALPHA
        self._heat[eligible] = (1.0 - a) * self._heat[eligible] + a * rd[eligible]

    HEAT_ALPHA = 0.25

    def _async_ok(self) -> bool:
        """Asynchronous flushes apply when some unit may have to leave HBM (the pool is smaller
        than every chunk of every layer and head) and there is room for the protected (sink +
        window) units besides the two chunks of slots they keep free."""
        if not self.async_flush or self.n_slots >= self.L * self.H * self.max_chunks:
            return False
        prot = (0 if self.window is None else self.window) + self.sink
        return self.n_slots >= (prot + 3) * self.L * self.H

    def _make_room(self, need: int):
        self._commit()
        st, rd, _, _ = self._counts()
        desired = self._plan(st, reserve=need, rd=self._heat)
        self._apply(desired, st)
        if len(self._free_hbm) < need:
            raise BlockKVBackendError(f"cannot free {need} HBM slots")

    def flush(self, reserve_next_chunk: bool = True) -> dict:
        """Chunk-boundary residency update (MMCache.flush_offload, models/cache.py:1032): one
        read of the stamps and page counts, then batched evict / promote copies enqueued without
        synchronising: on the current stream, or (``async_flush``) on the cache's move stream,
        committed by the next flush.  With ``reserve_next_chunk`` the HBM slots of the next chunk of every
        layer and head are assigned here, so the appends of the next AR step never touch the
        host.  Returns this flush's counts: per-call unit accesses served from HBM (hits) and
        from the host pool (misses), distinct units touched per pool, page listings (a page read
        by k selections counts k times) and unique pages read per pool.  The pool serving a
        unit's reads changes only here (and in an append that finds no free slot, which a
        flush's reservation prevents, or one that rewrites a moving unit), so the pool a unit
        sits in now is the pool its accesses since the last flush used."""
        st, rd, pages, tc = self._counts()
        touched = st > self._flush_epoch
        written = self._table_h != -1
        res, host = self._table_h >= 0, self._table_h <= -2
        hbm_units = int((touched & res).sum())
        host_units = int((touched & host).sum())
        hits, misses = int(tc[res].sum()), int(tc[host].sum())
        hbm_reads, host_reads = int(rd[res].sum()), int(rd[host].sum())
        hbm_unique, host_unique = int(pages[res].sum()), int(pages[host].sum())
        self.stats["hits"] += hits
        self.stats["misses"] += misses
        self.stats["hbm_units_touched"] += hbm_units
        self.stats["host_units_touched"] += host_units
        self.stats["hbm_page_reads"] += hbm_reads
        self.stats["host_page_reads"] += host_reads
        self.stats["hbm_pages_unique"] += hbm_unique
        self.stats["host_pages_unique"] += host_unique
        # the previous flush's moves: their units were read from the source slots until now
        changed = self._commit(upload=False)
        LH = self.L * self.H
        asyn = self._async_ok() and reserve_next_chunk
        reserve = (2 * LH if asyn else LH) if reserve_next_chunk else 0
        self._update_heat(rd, written)
        if (self.lru_max_size == 0 and not bool((self._table_h <= -2).any())
                and int((self._table_h >= 0).sum()) <= self._cap(reserve)):
            # byte budget, nothing on the host and room for everything: the cost plan keeps
            # exactly the resident set
            desired = self._table_h >= 0
        else:
            desired = self._plan(st, reserve=reserve, rd=self._heat) & written
        if asyn:
            moves = self._pick_moves(desired, st, keep_free=LH)
        else:
            if changed:
                self._upload_table()
                changed = False
            ev, pr = self._apply(desired, st)
        if reserve_next_chunk:
            for l in range(self.L):
                c = self.n_chunks[l]
                if c >= self.max_chunks:
                    continue
                row = self._table_h[l, :, c]
                # slots short (snapshots holding some): the append makes room itself
                for h in np.nonzero(row == -1)[0]:
                    if not self._free_hbm:
                        break
                    row[h] = self._free_hbm.pop()
                    changed = True
        if changed:
            self._upload_table()
        self._reads_all.zero_()
        self._seen_all.zero_()
        self._touch_all.zero_()
        if asyn:
            # last: a copy engine busy with the moves would hold up copies enqueued after them
            # on the current stream (the table uploads above)
            ev, pr = self._apply_async(*moves)
        self._flush_epoch = self._epoch
        self.stats["flushes"] += 1
        return {"hits": hits, "misses": misses, "hbm_units_touched": hbm_units,
                "host_units_touched": host_units, "evicted_units": ev, "promoted_units": pr,
                "hbm_page_reads": hbm_reads, "host_page_reads": host_reads,
                "hbm_pages_unique": hbm_unique, "host_pages_unique": host_unique}

    def flush_offload(self, layer_idx: Optional[int] = None) -> dict:
        """MMCache-compatible name of ``flush`` (models/cache.py:1032).  Residency is planned for
        all layers at once, so ``layer_idx`` is accepted and ignored."""
        return self.flush()

    def preallocate_offload_buffer(self, sample: torch.Tensor, max_entries_per_call: int,
                                   segment_cids: int = 10):
        """MMCache-compatible no-op (models/cache.py:970): the pinned host pool is sized when
        the cache is built."""
        return None

    def lru_touch_per_head(self, layer_idx: int, name: str, head: int, cid: int):
        """MMCache-compatible LRU touch (models/cache.py:673): stamps unit (head, cid) with a
        new epoch, as the selection kernel does for every unit it reads."""
        if name not in ("k_cache", "v_cache"):
            raise BlockKVBackendError(f"unknown cache name {name!r}")
        if self._table_h[layer_idx, int(head), int(cid)] == -1:
            return  # never written: nothing to keep (a selection skips such units too)
        self.stamp[layer_idx][int(head), int(cid)] = self.next_epoch()
        self.touches[layer_idx][int(head), int(cid)] += 1

    def get_chunk_metadata(self, layer_idx: int, name: str):
        """MMCache-compatible chunk table (models/cache.py:340-347): (int64 [H, max_chunks] byte
        address of each (head, chunk) unit or 0 when unwritten, int32 [H] chunks per head, the
        strides dict of ``selection_attention_padded_ptr_fast``).  Host-resident units get their
        device-mapped host address, which the pointer kernels read in place.  A unit is
        ``pages_per_chunk * page_tokens`` rows of ``head_dim`` bf16; when ``page_tokens`` divides
        ``chunk_len`` (the reference's 30-token blocks of 4680-token chunks) this is the
        reference's per-head chunk layout.  The addresses are valid until the next ``flush``."""
        if name not in ("k_cache", "v_cache"):
            raise BlockKVBackendError(f"unknown cache name {name!r}")
        if self.fp8:
            raise BlockKVBackendError("pointer-table metadata is bf16-only (the reference's "
                                      "pointer kernels read bf16 blocks)")
        pool = self.pool_k if name == "k_cache" else self.pool_v
        host = (self._host_k if name == "k_cache" else self._host_v).dev_ptr
        s = self.unit_table[layer_idx].to(torch.int64)
        ub = self.unit_bytes
        ptrs = torch.where(s >= 0, pool.data_ptr() + s * ub,
                           torch.where(s <= -2, host + (-2 - s) * ub, torch.zeros_like(s)))
        n = torch.full((self.H,), self.n_chunks[layer_idx], dtype=torch.int32, device=self.device)
        strides = {"batch_stride_bytes": ub, "token_stride_bytes": self.D * 2,
                   "stride_bn": self.D, "stride_bd": 1, "chunk_len": self.chunk_len}
        return ptrs, n, strides

    def lru_hit_rate_overall(self) -> float:
        """Hits over accesses since the last ``lru_reset_stats`` (models/cache.py:713-716): an
        access is one selection call (or ``lru_touch_per_head``) reading a (layer, head, chunk)
        unit, a hit when the unit is in HBM.  Accesses since the last flush are read from the
        device counters (one synchronisation).  The reference also counts no access for a
        chunk that is on the GPU but not yet in its LRU (a "cold miss"); here every HBM-resident
        unit is in the resident set, so such accesses count as hits."""
        tc = self._touch_all.cpu().numpy()
        hits = self.stats["hits"] + int(tc[self._table_h >= 0].sum())
        tot = hits + self.stats["misses"] + int(tc[self._table_h <= -2].sum())
        return hits / tot if tot else 0.0

    def lru_reset_stats(self):
        """Zero the access counts behind ``lru_hit_rate_overall`` (models/cache.py:718-727);
        residency, stamps and the other statistics are kept."""
        self.stats["hits"] = 0
        self.stats["misses"] = 0
        self._touch_all.zero_()

    # ---------------------------------------------------------------- snapshots
    def snapshot_chunks(self, chunk_start: int, chunk_end: int) -> dict:
        """Keep chunks [chunk_start, chunk_end) of every layer as they are now, for
        ``restore_chunks``: the pipeline's prompt switch re-encodes the last chunks with the new
        prompt and then puts the older ones back (``_snapshot_chunks`` / ``_restore_chunks``,
        pipelines/pipeline_wan_causal.py:33-57, 369-396).  Copy-on-write per unit: nothing is
        copied now; the first rewrite of a snapshotted unit goes to a new slot and the snapshot
        holds the old one (which no flush moves) until it is restored or discarded.  The pooled
        rows of the range (and, for an fp8 cache, its chunks in the dense window ring) are
        cloned.  A rewrite needs a free HBM slot per snapshotted unit, and the slots a snapshot
        holds are unavailable to residency until it is restored or discarded: size the pools
        (``hbm_slots`` / ``host_slots``) with that room."""
        self._commit()
        a, b = max(0, int(chunk_start)), min(self.max_chunks, int(chunk_end))
        for sn in self._snaps:
            if sn["range"][0] < b and a < sn["range"][1]:
                raise BlockKVBackendError(f"chunks [{a}, {b}) overlap an active snapshot of "
                                          f"{list(sn['range'])}")
        units = {}
        for l in range(self.L):
            for c in range(a, b):
                for h in range(self.H):
                    if self._table_h[l, h, c] != -1:
                        units[(l, h, c)] = None  # shared with the table until rewritten
        rows = slice(a * self.ppc, b * self.ppc)
        snap = {"range": (a, b), "units": units,
                "k_cmp": [t[:, rows].clone() for t in self.k_cmp],
                "v_cmp": [t[:, rows].clone() for t in self.v_cmp], "ring": {}}
        if self.keep_window_kv:
            for l in range(self.L):
                n = self.n_chunks[l]
                for c in range(max(a, n - self.window), min(b, n)):
                    w = c % self.window
                    snap["ring"][(l, c)] = (self.win_k[l][w].clone(), self.win_v[l][w].clone())
        self._snaps.append(snap)
        return snap

    def _release_slot(self, s: int):
        if s >= 0:
            self._free_hbm.append(s)
        elif s <= -2:
            self._free_host.append(-2 - s)

    def restore_chunks(self, snapshot: dict, chunk_start: Optional[int] = None):
        """Put the snapshotted chunks back: units rewritten since the snapshot get their old
        slot again (the newer version's slot is freed), untouched units stay as they are, and
        the pooled rows (and ring entries) are copied back.  ``chunk_start`` must be the
        snapshot's first chunk when given (the reference helper's argument)."""
        self._active_snapshot(snapshot)
        self._commit()  # a pending move of a rewritten unit would re-point it after the restore
        a, b = snapshot["range"]
        if chunk_start is not None and int(chunk_start) != a:
            raise BlockKVBackendError(f"snapshot starts at chunk {a}, not {chunk_start}")
        for (l, h, c), old in snapshot["units"].items():
            if old is None:
                continue
            self._release_slot(int(self._table_h[l, h, c]))
            self._table_h[l, h, c] = old
        self._snaps = [sn for sn in self._snaps if sn is not snapshot]
        rows = slice(a * self.ppc, b * self.ppc)
        for l in range(self.L):
            self.k_cmp[l][:, rows].copy_(snapshot["k_cmp"][l])
            self.v_cmp[l][:, rows].copy_(snapshot["v_cmp"][l])
        for (l, c), (wk, wv) in snapshot["ring"].items():
            self.win_k[l][c % self.window].copy_(wk)
            self.win_v[l][c % self.window].copy_(wv)
        self._upload_table()

    def discard_snapshot(self, snapshot: dict):
        """Drop a snapshot without restoring it; the slots it held are freed."""
        self._active_snapshot(snapshot)
        self._commit()
        for old in snapshot["units"].values():
            if old is not None:
                self._release_slot(old)
        self._snaps = [sn for sn in self._snaps if sn is not snapshot]

    def _active_snapshot(self, snapshot: dict):
        if not any(sn is snapshot for sn in self._snaps):
            raise BlockKVBackendError("snapshot already restored or discarded")

    # ---------------------------------------------------------------- inspection (tests)
    def read_unit(self, layer: int, head: int, cid: int):
        """(K, V[, scale_k, scale_v]) of one unit as CPU tensors, from the pool that serves its
        reads now (``where``)."""
        s = int(self._table_h[layer, head, cid])
        if s == -1:
            raise BlockKVBackendError("unit never written")
        torch.cuda.current_stream(self.device).synchronize()
        store = torch.uint8 if self.fp8 else torch.bfloat16
        shape = (self.ppc, self.P, self.D)
        if s >= 0:
            k, v = self.pool_k[s].cpu(), self.pool_v[s].cpu()
            sc = (self.scale_k[s].cpu(), self.scale_v[s].cpu()) if self.fp8 else ()
        else:
            hs = -2 - s
            ub = self.unit_bytes
            k = self._host_k.cpu_view()[hs * ub:(hs + 1) * ub].clone().view(store).view(shape)
            v = self._host_v.cpu_view()[hs * ub:(hs + 1) * ub].clone().view(store).view(shape)
            sc = ()
            if self.fp8:
                sb = self.scale_bytes
                sc = (self._host_sk.cpu_view()[hs * sb:(hs + 1) * sb].clone().view(torch.float32),
                      self._host_sv.cpu_view()[hs * sb:(hs + 1) * sb].clone().view(torch.float32))
        return (k, v) + tuple(sc)

    def where(self, layer: int, head: int, cid: int) -> str:
        """Pool that serves the unit's reads now: a unit an asynchronous flush is moving is
        read from its source slot until the move is committed."""
        s = int(self._table_h[layer, head, cid])
        return "none" if s == -1 else ("hbm" if s >= 0 else "host")

    def evict_all(self):
        """Move every unit to the host pool (failure-injection / parity tests)."""
        self._commit()
        desired = np.zeros_like(self._table_h, dtype=bool)
        self._apply(desired)

    def close(self):
        if self._moves is not None:
            self._moves[0].synchronize()
            self._moves = None
        for p in (self._host_k, self._host_v, self._host_sk, self._host_sv):
            p.free()


class MMCache(PagedKVCache):
    """``PagedKVCache`` behind the reference's ``MMCache`` constructor (models/cache.py:44-60),
    so the pipeline's cache construction (pipelines/pipeline_wan_causal.py:235-316) runs as is.

    Mapping of the reference's arguments:

    * ``config["cache_type"]`` must name ``k_cache`` and ``v_cache`` (``k_cmp_cache`` /
      ``v_cmp_cache`` are optional: the pooled history lives in every paged cache);
    * ``seq_dim`` must be 1; ``available_shape["k_cache"]`` is ``(B, tokens, H, D)`` with B = 1
      (the paged cache serves one sequence); ``max_chunks = ceil(tokens / chunk)``;
    * ``block_seqlen_config["k_cache"]`` is the chunk length in tokens, and
      ``block_seqlen_config["k_cmp_cache"]`` (if given) must equal the pages per chunk;
    * ``kv_block_size`` is the page size (the selection block; 64 when the reference passes 0);
    * ``window_config`` / ``sink_config`` give the window and sink chunks of ``k_cache`` and of
      ``k_cmp_cache`` (None: no window, every chunk is returned);
    * ``lru_max_size`` keeps the reference's per-(layer, head) chunk count; ``hbm_budget_bytes``
      (keyword only) replaces it with a byte budget;
    * ``dtype``, ``per_head_types``, ``chunk_per_head_types``, ``chunk_buffer_types`` are
      accepted: storage is always per-head chunk pages, in bf16, or fp8 e4m3 with
      ``cache_dtype="fp8"`` (keyword only).
    """

    def __init__(self, config, seq_dim, available_shape, device="cuda", dtype=torch.float32,
                 block_seqlen_config=None, window_config=None, sink_config=None,
                 num_layers=None, lru_max_size=10, per_head_types=None,
                 chunk_per_head_types=None, chunk_buffer_types=None, num_heads=None,
                 kv_block_size=0, *, hbm_budget_bytes: Optional[int] = None,
                 cache_dtype=torch.bfloat16, keep_window_kv: bool = False):
        types = set(config.get("cache_type", ()))
        if not {"k_cache", "v_cache"} <= types:
            raise BlockKVBackendError(f"MMCache over pages needs 'k_cache' and 'v_cache' in "
                                      f"config['cache_type'], got {sorted(types)}")
        if seq_dim != 1:
            raise BlockKVBackendError(f"the paged cache stores [B, tokens, H, D]: seq_dim must be "
                                      f"1, got {seq_dim}")
        if num_layers is None:
            raise BlockKVBackendError("num_layers is required")
        blk = dict(block_seqlen_config or {})
        if "k_cache" not in blk:
            raise BlockKVBackendError("block_seqlen_config['k_cache'] (the chunk length) is "
                                      "required: the paged cache is chunked")
        shape = tuple(available_shape["k_cache"])
        if len(shape) != 4 or shape[0] != 1:
            raise BlockKVBackendError(f"available_shape['k_cache'] must be (1, tokens, H, D), got "
                                      f"{shape}")
        H = int(num_heads) if num_heads else int(shape[2])
        if H != shape[2]:
            raise BlockKVBackendError(f"num_heads {H} != available_shape heads {shape[2]}")
        chunk = int(blk["k_cache"])
        page = int(kv_block_size) if kv_block_size else 64
        win = dict(window_config or {})
        sink = dict(sink_config or {})
        window = win.get("k_cache")
        max_chunks = -(-int(shape[1]) // chunk)
        super().__init__(int(num_layers), H, int(shape[3]), max_chunks=max_chunks,
                         chunk_len=chunk, page_tokens=page, dtype=cache_dtype,
                         hbm_budget_bytes=hbm_budget_bytes,
                         lru_max_size=0 if hbm_budget_bytes is not None else int(lru_max_size),
                         window_chunks=None if window is None else int(window),
                         sink_chunks=int(sink.get("k_cache") or 0),
                         keep_window_kv=keep_window_kv, device=device)
        cmp_rows = blk.get("k_cmp_cache")
        if cmp_rows is not None and int(cmp_rows) != self.ppc:
            raise BlockKVBackendError(
                f"block_seqlen_config['k_cmp_cache'] = {cmp_rows} pooled rows per chunk, but "
                f"{chunk}-token chunks of {page}-token blocks have {self.ppc}")
        cw = win.get("k_cmp_cache")
        self.cmp_window = None if cw is None else int(cw)
        self.cmp_sink = int(sink.get("k_cmp_cache") or 0)
        self.config = config
        # the reference's attribute (models/cache.py:63), which CausalWanNSAModel.forward checks
        # for the pooled names (causal_wan_nsa_model.py:783-784); every paged cache serves them
        self.available_type = list(config["cache_type"]) + [
            t for t in ("k_cmp_cache", "v_cmp_cache") if t not in types]
        self.seq_dim = seq_dim
        self.dtype = dtype
        self.num_heads = H
        self.num_layers = int(num_layers)
        self.kv_block_size = page
