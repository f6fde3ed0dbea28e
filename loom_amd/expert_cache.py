"""Host mirror of Loom's expert cache (src/engine/expert_cache.zig) over the
HBM tier of ``libloomhip``: ``ExpertCache`` keeps the reference's names
(``pin``, ``get``, ``stats``, ``Stats.hitRate``, ``pinnedCount``), with the
cache in HBM and the backing store in pinned host memory (``HostBuffer``),
and ``moe_layer`` runs a routed MoE layer whose experts are read through it
(src/engine/moe.zig:97-124).

Errors follow the seam: hard failures raise ``LoomHipError``; a failed fill
aborts its reservation (Lru.abort) before raising, as ExpertCache.get does.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import EcStats, LoomHipError, MoeLayerEcDesc, check, lib
from .backend import _ptr, _stream


class HostBuffer:
    """Pinned host memory (``loomhip_host_alloc``) viewed as a uint8 array."""

    def __init__(self, nbytes: int):
        p = lib().loomhip_host_alloc(nbytes)
        if not p:
            raise LoomHipError(f"pinned host allocation of {nbytes} bytes failed")
        self.ptr, self.nbytes = p, nbytes
        self.array = np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(p))

    def free(self):
        if self.ptr:
            self.array = None
            lib().loomhip_host_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class Stats:
    """expert_cache.zig:18-36 (disk_misses = the host-copy misses)."""

    pin_hits: int
    lru_hits: int
    disk_misses: int
    bytes_read: int
    warmup_reads: int
    warmup_bytes: int

    def accesses(self) -> int:
        return self.pin_hits + self.lru_hits + self.disk_misses

    def hitRate(self) -> float:  # noqa: N802 -- the reference's name
        a = self.accesses()
        return 0.0 if a == 0 else (self.pin_hits + self.lru_hits) / a


class ExpertCache:
    """``capacity`` LRU slots plus ``pin_slots`` pinned ones of ``slot_bytes``
    in HBM for expert ids [0, n_ids)."""

    def __init__(self, capacity: int, slot_bytes: int, n_ids: int, pin_slots: int = 0):
        h = C.c_void_p()
        check(lib().loomhip_ec_create(capacity, pin_slots, slot_bytes, n_ids, C.byref(h)), "ec_create")
        self.h = h
        self.capacity, self.pin_slots, self.slot_bytes, self.n_ids = capacity, pin_slots, slot_bytes, n_ids
        self._sources = {}
        self._pinned = set()

    def close(self):
        if self.h:
            lib().loomhip_ec_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_source(self, expert_id: int, host: HostBuffer, offset: int = 0, length: int | None = None):
        """Expert ``expert_id``'s backing block: ``length`` bytes of ``host``
        from ``offset`` (the manifest entry readBlock reads)."""
        n = host.nbytes - offset if length is None else length
        check(lib().loomhip_ec_set_source(self.h, expert_id, host.ptr + offset, n), "ec_set_source")
        self._sources[expert_id] = host  # keep the buffer alive

    def pin(self, ids) -> None:
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        check(lib().loomhip_ec_pin(self.h, a.ctypes.data, a.size), "ec_pin")
        self._pinned.update(int(i) for i in a)

    def pinnedCount(self) -> int:  # noqa: N802
        return len(self._pinned)

    def get(self, expert_id: int, stream=None) -> int:
        """Device address of the block (ExpertCache.get)."""
        out = C.c_void_p()
        check(lib().loomhip_ec_get(self.h, expert_id, stream if stream is not None else _stream(),
                                   C.byref(out)), "ec_get")
        return int(out.value)

    def release(self, stream=None) -> None:
        check(lib().loomhip_ec_release(self.h, stream if stream is not None else _stream()), "ec_release")

    def prefetch(self, ids) -> None:
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        check(lib().loomhip_ec_prefetch(self.h, a.ctypes.data, a.size), "ec_prefetch")

    @property
    def stats(self) -> Stats:
        s = EcStats()
        check(lib().loomhip_ec_get_stats(self.h, C.byref(s)), "ec_stats")
        return Stats(s.pin_hits, s.lru_hits, s.misses, s.bytes_read, s.warmup_reads, s.warmup_bytes)

    def access_counts(self) -> np.ndarray:
        out = np.zeros(self.n_ids, np.uint64)
        check(lib().loomhip_ec_access_counts(self.h, out.ctypes.data, self.n_ids), "ec_access_counts")
        return out

    def clear(self) -> None:
        check(lib().loomhip_ec_clear(self.h), "ec_clear")

    def moe_layer(self, desc: MoeLayerEcDesc, normed, out, n_tok: int, want_ids: bool = False):
        """One routed MoE layer with its experts read through the cache:
        ``normed``/``out`` are device tensors [n_tok][dim]; returns (ids,
        gates) as numpy arrays when ``want_ids``."""
        ids = gates = None
        pi = pg = None
        if want_ids:
            ids = np.zeros((n_tok, desc.n_used), np.uint32)
            gates = np.zeros((n_tok, desc.n_used), np.float32)
            pi, pg = ids.ctypes.data, gates.ctypes.data
        check(lib().loomhip_moe_layer_cached(C.byref(desc), self.h, _ptr(normed), n_tok, _ptr(out), pi, pg,
                                             _stream()), "moe_layer_cached")
        return ids, gates


__all__ = ["ExpertCache", "HostBuffer", "Stats"]
