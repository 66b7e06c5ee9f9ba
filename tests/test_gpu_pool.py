"""Pool watermarks and preserve marks of the buffer table (the reference
backend's buf_pool.c:9-183 as its realize loop uses them,
src/schedule/realize.c:296-310, :326-340, :420-450), through the C-ABI.

  * rollback: unpreserved buffers since the watermark are parked and the next
    same-size allocations recycle their storage; preserved ones keep their
    bytes; a JIT-pinned one survives; older buffers are untouched;
  * ids: a rolled-back or recycled id is dead (refcount 0, no bytes) even
    after its slot is reused by a new buffer (the generation check);
  * arena blocks are freed outright, never parked; views since the mark are
    freed and release their parent;
  * clear_preserved_arena_views drops the mark of a view and of a parent
    allocated since the mark, not of an older parent;
  * free_unpreserved_all parks every live unmarked owning buffer (checked in
    a process of its own: the sweep is table-wide);
  * 10^5 realize-shaped cycles (allocate, mark the result, roll back, clear)
    keep the live device bytes flat and the slot table bounded."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _alloc(L, n, fill=None):
    bid = L.thvm_hip_buf_alloc(n)
    assert bid, L.thvm_hip_last_error()
    if fill is not None:
        a = np.full(n, fill, np.uint8)
        assert L.thvm_hip_buf_write(bid, a.ctypes.data, n) == 0
    return bid


def _read(L, bid, n):
    a = np.empty(n, np.uint8)
    assert L.thvm_hip_buf_read(bid, a.ctypes.data, n) == 0, L.thvm_hip_last_error()
    return a


def test_rollback_preserve_and_stale_ids(hip):
    L = hip.lib()
    _say("case: pool rollback semantics")
    old = _alloc(L, 4096, 7)                     # before the watermark
    wm = L.thvm_hip_buf_pool_begin()
    a, b, c = _alloc(L, 4096, 1), _alloc(L, 8192, 2), _alloc(L, 4096, 3)
    pinned = _alloc(L, 1024, 4)
    L.thvm_hip_buf_jit_pin(pinned)
    v = L.thvm_hip_buf_view(b, 256, 512)
    assert v and L.thvm_hip_buf_refcount(b) == 2
    arena = L.thvm_hip_buf_arena_alloc(1 << 20)
    assert arena
    live0 = L.thvm_hip_mem_live_bytes()
    L.thvm_hip_buf_mark_preserved(c)
    L.thvm_hip_buf_pool_rollback_with_preserve(wm)
    # preserved, pinned and older buffers keep their bytes; the rest are dead ids
    assert np.all(_read(L, c, 4096) == 3) and np.all(_read(L, old, 4096) == 7)
    assert np.all(_read(L, pinned, 1024) == 4)
    for dead in (a, b, v, arena):
        assert L.thvm_hip_buf_refcount(dead) == 0 and L.thvm_hip_buf_nbytes(dead) == 0
    # the arena's megabyte went back to the device; a and b sit parked
    assert L.thvm_hip_mem_live_bytes() == live0 - (1 << 20)
    # same-size allocations recycle the parked blocks (no new device bytes),
    # read as zeros, and get ids that differ from every dead one
    a2, b2 = _alloc(L, 4096), _alloc(L, 8192)
    assert L.thvm_hip_mem_live_bytes() == live0 - (1 << 20)
    assert np.all(_read(L, a2, 4096) == 0) and np.all(_read(L, b2, 8192) == 0)
    assert len({a2, b2} & {a, b, v, arena}) == 0
    # the dead ids stay dead although their slots are reused
    for dead in (a, b, v, arena):
        assert L.thvm_hip_buf_nbytes(dead) == 0
        assert L.thvm_hip_buf_read(dead, None, 0) == -1
    L.thvm_hip_buf_clear_preserved(wm)
    L.thvm_hip_buf_jit_unpin(pinned)
    for x in (old, c, pinned, a2, b2):
        L.thvm_hip_buf_free(x)


def test_arena_views_and_clear_marks(hip):
    L = hip.lib()
    _say("case: arena views, clear marks")
    weight = _alloc(L, 4096, 9)                  # an older parent a view reads
    wm = L.thvm_hip_buf_pool_begin()
    arena = L.thvm_hip_buf_arena_alloc(65536)
    av = L.thvm_hip_buf_view(arena, 0, 1024)
    wv = L.thvm_hip_buf_view(weight, 1024, 1024)
    for x in (arena, av, wv, weight):
        L.thvm_hip_buf_mark_preserved(x)
    L.thvm_hip_buf_clear_preserved_arena_views(wm)
    L.thvm_hip_buf_pool_rollback_with_preserve(wm)
    # the arena and its view lost their marks and died; the older weight kept
    # its mark and its bytes (its view since the mark died, releasing it)
    assert L.thvm_hip_buf_nbytes(arena) == 0 and L.thvm_hip_buf_nbytes(av) == 0
    assert L.thvm_hip_buf_nbytes(wv) == 0
    assert np.all(_read(L, weight, 4096) == 9) and L.thvm_hip_buf_refcount(weight) == 1
    L.thvm_hip_buf_clear_preserved(wm)
    L.thvm_hip_buf_free(weight)


_SWEEP_CHILD = """
import sys
sys.path[:0] = [{root!r}, {tests!r}]
import numpy as np
import thvm_amd
import test_gpu_pool as T
thvm_amd.init()
L = thvm_amd.lib()
keep, drop, older = T._alloc(L, 2048, 5), T._alloc(L, 2048, 6), T._alloc(L, 4096, 8)
pinned = T._alloc(L, 512, 1)
L.thvm_hip_buf_jit_pin(pinned)
v = L.thvm_hip_buf_view(older, 0, 256)
L.thvm_hip_buf_mark_preserved(keep)
freed = L.thvm_hip_buf_free_unpreserved_all()
assert freed == 2048 + 4096, freed
assert L.thvm_hip_buf_nbytes(drop) == 0 and L.thvm_hip_buf_nbytes(older) == 0
assert np.all(T._read(L, keep, 2048) == 5) and np.all(T._read(L, pinned, 512) == 1)
live = L.thvm_hip_mem_live_bytes()
again = T._alloc(L, 4096)
assert L.thvm_hip_mem_live_bytes() == live      # the parked block came back
thvm_amd.shutdown()
print("sweep child ok", flush=True)
"""


def test_free_unpreserved_all_in_a_fresh_process(hip):
    """The sweep is table-wide, so it runs in a process of its own (here it
    would reclaim other tests' live buffers)."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    _say("case: table-wide sweep (child process)")
    code = _SWEEP_CHILD.format(root=str(root), tests=str(root / "tests"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    _say(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "sweep child ok" in r.stdout


def test_hundred_thousand_cycles_stay_flat(hip):
    """A realize loop: per cycle a few transients and a view, the result
    marked preserved, rollback, marks cleared, the previous result released."""
    L = hip.lib()
    _say("case: 1e5 alloc/rollback cycles")
    prev = 0
    live = slots = None
    hw0 = L.thvm_hip_buf_slot_highwater()
    for i in range(100_000):
        wm = L.thvm_hip_buf_pool_begin()
        t1 = L.thvm_hip_buf_alloc(4096)
        t2 = L.thvm_hip_buf_alloc(65536)
        v = L.thvm_hip_buf_view(t2, 4096, 4096)
        res = L.thvm_hip_buf_alloc(1024)
        assert t1 and t2 and v and res, L.thvm_hip_last_error()
        L.thvm_hip_buf_mark_preserved(res)
        L.thvm_hip_buf_pool_rollback_with_preserve(wm)
        L.thvm_hip_buf_clear_preserved(wm)
        if prev:
            L.thvm_hip_buf_decref(prev)      # the previous result's last holder lets go
        prev = res
        if i == 10:
            live, slots = L.thvm_hip_mem_live_bytes(), L.thvm_hip_buf_slots_used()
        elif i > 10 and i % 10_000 == 0:
            assert L.thvm_hip_mem_live_bytes() == live, i
            assert L.thvm_hip_buf_slots_used() == slots, i
            _say(f"  cycle {i}: live {L.thvm_hip_mem_live_bytes()} B, slots {L.thvm_hip_buf_slots_used()}, "
                 f"highwater {L.thvm_hip_buf_slot_highwater()}")
    assert L.thvm_hip_mem_live_bytes() == live
    # ~4 buffer deaths per cycle: a slot retires after 2^14 of its own, so the
    # table grew by about 4e5 / 2^14 = 25 slots, not by 4e5
    assert L.thvm_hip_buf_slot_highwater() - hw0 < 64
    L.thvm_hip_buf_free(prev)
