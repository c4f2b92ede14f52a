"""The expert cache policy (host only, no device): ingot_expert_cache_* against
the reference's own test of ExpertCache,
batched_slots_remain_pinned_during_prefetch_and_failed_reads_stay_invalid
(src/weights.rs:99-203): three slots, experts 0..2 loaded into slots 0..2, hits
on 0 and 1, expert 3 replacing the least recently used unpinned slot while 0
and 1 are pinned, "no reusable expert slot" with every slot pinned (slots
unchanged), a hit with every slot pinned, a failed read leaving its slot empty,
and the counters (3 hits, 4 misses)."""
import ctypes as C

import numpy as np
import pytest

from ingot_amd import _native as N


class Cache:
    def __init__(self, slots):
        self.lib = N.moe_lib()
        self.n = slots
        self.h = self.lib.ingot_expert_cache_create(slots)
        assert self.h

    def hit(self, e):
        return self.lib.ingot_expert_cache_hit(self.h, e)

    def slot(self, e, pinned=(), read_ok=True):
        """ExpertCache::slot: claim, read (commit on success). Returns the slot,
        or None for "no reusable expert slot" / a failed read."""
        pin = (C.c_uint32 * max(1, len(pinned)))(*pinned)
        load = C.c_int()
        s = self.lib.ingot_expert_cache_claim(self.h, e, pin, len(pinned), C.byref(load))
        if s < 0:
            return None
        if load.value:
            if not read_ok:
                return None
            assert self.lib.ingot_expert_cache_commit(self.h, s, e) == 0
        return s

    def state(self):
        ids = np.zeros(self.n, np.int64)
        hits, misses = C.c_uint64(), C.c_uint64()
        assert self.lib.ingot_expert_cache_state(self.h, ids.ctypes.data, C.byref(hits), C.byref(misses)) == 0
        return list(ids), hits.value, misses.value

    def close(self):
        self.lib.ingot_expert_cache_destroy(self.h)


def test_reference_cache_sequence():
    c = Cache(3)
    for expert in range(3):
        assert c.slot(expert) == expert
    assert c.hit(0) == 0
    assert c.hit(1) == 1
    # expert 3 while slots 0 and 1 are read by a batch: the least recently used
    # unpinned slot is 2
    assert c.slot(3, pinned=[0, 1]) == 2
    before = c.state()[0]
    assert c.slot(2, pinned=[0, 1, 2]) is None  # no reusable expert slot
    assert c.state()[0] == before
    assert c.slot(0, pinned=[0, 1, 2]) == 0  # a hit needs no free slot
    # a failed read of expert 2 (slot 2 again the only unpinned one) leaves it empty
    assert c.slot(2, pinned=[0, 1], read_ok=False) is None
    ids, hits, misses = c.state()
    assert ids[2] == -1
    assert c.hit(2) == -1 and c.hit(3) == -1
    assert (hits, misses) == (3, 4)
    c.close()


def test_lru_order_and_empty_slots_first():
    """Empty slots are taken first (lowest index); then the least recently used."""
    c = Cache(4)
    assert [c.slot(e) for e in (10, 11, 12)] == [0, 1, 2]
    assert c.slot(13) == 3
    assert c.hit(10) == 0  # 11 is now the least recently used
    assert c.slot(14) == 1
    assert c.slot(15, pinned=[2]) == 3  # 12 (slot 2) is older but pinned: 13 goes
    ids, hits, misses = c.state()
    assert ids == [10, 14, 12, 15] and (hits, misses) == (1, 6)
    c.close()


def test_create_rejects_zero_slots():
    assert not N.moe_lib().ingot_expert_cache_create(0)


def test_cached_layer_entry_points_exported():
    lib = N.moe_lib()
    for name in ("ingot_layer_create_cached", "ingot_layer_cache_stats"):
        assert getattr(lib, name)
