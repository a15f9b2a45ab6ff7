"""CPU model of the reference's per-(layer, head) chunk LRU -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` import this module, as the checker of ``omnimem_amd.block_cache``'s residency.

Restates ``MMCache.lru_touch_per_head`` (src/omnimem/models/cache.py:673-699): one OrderedDict
of chunk ids per (layer, 'k_cache', head) with capacity ``lru_max_size``; a touch of a present id
moves it to the end, a touch of a new id when full pops the oldest (marking it for offload,
:1018-1030) and appends the new one.  Touch order: ``update_cache('k_cache', ...)`` touches the
written chunk of every head (:499-501); a selection call touches the unique (head, chunk) keys of
its block indices in ascending key order h * max_chunks + cid (wrapper.py:268-291).
``flush_offload`` (:1032-1142) then offloads marked chunks that are not back in the LRU and are
neither sink nor window chunks.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Dict, Iterable, Set, Tuple

import numpy as np


class ReferenceLRU:
    def __init__(self, num_layers: int, num_heads: int, lru_max_size: int, window: int = 0,
                 sink: int = 0):
        self.L, self.H, self.C = num_layers, num_heads, lru_max_size
        self.window, self.sink = window, sink
        self.lru: Dict[Tuple[int, int], OrderedDict] = {
            (l, h): OrderedDict() for l in range(num_layers) for h in range(num_heads)}
        self.marked: Set[Tuple[int, int, int]] = set()
        self.on_gpu: Set[Tuple[int, int, int]] = set()
        self.n_chunks = [0] * num_layers

    def touch(self, l: int, h: int, cid: int):
        lru = self.lru[(l, h)]
        if cid in lru:
            lru.move_to_end(cid)
            return
        if len(lru) >= self.C:
            old, _ = lru.popitem(last=False)
            self.marked.add((l, h, old))
        lru[cid] = None

    def write(self, l: int, cid: int):
        self.n_chunks[l] = max(self.n_chunks[l], cid + 1)
        for h in range(self.H):
            self.on_gpu.add((l, h, cid))
            self.touch(l, h, cid)

    def select(self, l: int, block_indices: np.ndarray, pages_per_chunk: int, max_chunks: int):
        """block_indices: [1, MG, H, T] page ids of layer l."""
        ids = np.asarray(block_indices)
        H = ids.shape[2]
        keys = set()
        for h in range(H):
            for bid in ids[:, :, h, :].reshape(-1):
                if bid >= 0:
                    keys.add(h * max_chunks + int(bid) // pages_per_chunk)
        for key in sorted(keys):
            h, cid = divmod(key, max_chunks)
            if (l, h, cid) not in self.on_gpu:
                self.on_gpu.add((l, h, cid))  # the reference reloads a missing chunk
            self.touch(l, h, cid)

    def flush(self):
        for (l, h, cid) in sorted(self.marked):
            if (l, h, cid) not in self.on_gpu:
                continue
            n = self.n_chunks[l]
            if self.window and (cid < self.sink or cid >= max(self.sink, n - self.window)):
                continue
            if cid in self.lru[(l, h)]:
                continue
            self.on_gpu.discard((l, h, cid))
        self.marked.clear()

    def resident(self) -> Set[Tuple[int, int, int]]:
        return set(self.on_gpu)


def lru_contents_bruteforce(touches: Iterable[int], capacity: int) -> list:
    """The ``capacity`` most recently touched distinct keys, oldest first (closed form of an LRU)."""
    seen = []
    for t in touches:
        if t in seen:
            seen.remove(t)
        seen.append(t)
    return seen[-capacity:] if capacity > 0 else []
