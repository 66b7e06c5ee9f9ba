"""The drop-in boundary under the reference's own replay loop.

jit_replay (reference src/jit/capture.c:2687-2884) opens a graph capture on
a miss (graph_capture_begin, :2733), then, op by op, zeroes recycled outputs
(Backend.buf_zero, :2779-2780), dispatches kernels (dispatch_kernel) and
runs KV ASSIGNs through tensor_assign, which calls Backend.buf_copy_at
(src/tensor/assign.c:89-94) -- all inside the capture -- then
graph_capture_end_and_launch(slot) (:2873-2879); later replays hit the graph
(graph_replay, :2716) and jit_capture_drop invalidates it (:734-736).

These tests call the C-ABI hooks in exactly that order and check the
outputs of the first launch and of a replay at new inputs.  The ASSIGN row
is covered both ways: buf_copy_at with a host offset (frozen into the graph,
as the reference's CUDA graph freezes it) and buf_copy_row, whose row index
is read on the device, so a replay appends at the current row."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SRC_ADDONE = """extern "C" __global__ void addone(const float *x, float *y) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 8) y[i] = x[i] + 1.0f;
}"""


def say(*a):
    print(*a, flush=True)


def up(hip, a):
    return hip.Buffer.from_numpy(np.ascontiguousarray(a))


def test_graph_hooks_in_jit_replay_order(hip):
    say("case: graph hooks in jit_replay order (zero, dispatch, copy_at, copy_row)")
    L = hip.lib()
    g, b = (1, 1, 1), (8, 1, 1)
    xv = np.arange(8, dtype=np.float32)
    x, out = up(hip, xv), hip.Buffer(32)
    hip.dispatch("addone", SRC_ADDONE, [x, out], grid=g, block=b, outs=(1,))   # program cached
    rows, rb = 8, 16
    cache = hip.Buffer(rows * rb)
    kv_fixed = up(hip, np.arange(4, dtype=np.float32) + 100)
    kv_row = up(hip, np.arange(4, dtype=np.float32) + 200)
    length = up(hip, np.array([3], np.int32))
    out.write(np.full(8, 7, np.float32))          # stale bytes buf_zero must clear
    slot = 5
    probe = np.zeros(8, np.float32)
    assert L.thvm_hip_graph_capture_begin() == 0
    try:
        assert L.thvm_hip_buf_read(out.id, probe.ctypes.data, 32) == -1   # host transfer refused
        L.thvm_hip_buf_zero(out.id)
        hip.dispatch("addone", SRC_ADDONE, [x, out], grid=g, block=b, outs=(1,))
        assert L.thvm_hip_buf_copy_at(cache.id, 1 * rb, kv_fixed.id, 16) == 0
        assert L.thvm_hip_buf_copy_row(cache.id, 0, rb, length.id, 0, kv_row.id, 16) == 0
    finally:
        rc = L.thvm_hip_graph_capture_end_and_launch(slot)
    assert rc == 0, hip.last_error()
    got = cache.read(np.float32).reshape(rows, 4)
    assert np.array_equal(out.read(np.float32), xv + 1)
    assert np.array_equal(got[1], np.arange(4) + 100) and np.array_equal(got[3], np.arange(4) + 200)
    assert not got[[0, 2, 4, 5, 6, 7]].any()

    # replay (a graph hit) at new inputs and a new device row
    x.write(xv * 10)
    kv_fixed.write(np.arange(4, dtype=np.float32) + 300)
    kv_row.write(np.arange(4, dtype=np.float32) + 400)
    length.write(np.array([5], np.int32))
    out.write(np.full(8, -1, np.float32))
    assert L.thvm_hip_graph_replay(slot) == 0
    got = cache.read(np.float32).reshape(rows, 4)
    assert np.array_equal(out.read(np.float32), xv * 10 + 1)
    assert np.array_equal(got[1], np.arange(4) + 300)          # host offset: frozen row
    assert np.array_equal(got[5], np.arange(4) + 400)          # device row: the current one
    assert np.array_equal(got[3], np.arange(4) + 200)          # earlier append kept
    L.thvm_hip_graph_invalidate(slot)
    assert L.thvm_hip_graph_replay(slot) == -1


def test_buf_zero_and_copies_any_alignment(hip):
    """buf_zero is a fill kernel and copies of any alignment are copy
    kernels: only the addressed bytes change."""
    say("case: buf_zero / buf_copy_at / buf_copy_row on unaligned views")
    L = hip.lib()
    n = (1 << 20) + 77
    base = (np.arange(n) % 251 + 1).astype(np.uint8)
    parent = up(hip, base)
    v = L.thvm_hip_buf_view(parent.id, 3, 1000003)
    assert v != 0
    L.thvm_hip_buf_zero(v)
    got = parent.read(np.uint8)
    want = base.copy()
    want[3:3 + 1000003] = 0
    assert np.array_equal(got, want)
    L.thvm_hip_buf_decref(v)
    # unaligned copy inside a capture (a kernel node), then launched
    src = up(hip, np.arange(37, dtype=np.uint8) + 1)
    assert L.thvm_hip_graph_capture_begin() == 0
    try:
        assert L.thvm_hip_buf_copy_at(parent.id, 5, src.id, 37) == 0
    finally:
        assert L.thvm_hip_graph_capture_end_and_launch(7) == 0
    want[5:42] = np.arange(37) + 1
    assert np.array_equal(parent.read(np.uint8), want)
    L.thvm_hip_graph_invalidate(7)
    # a device row outside the destination writes nothing
    row = up(hip, np.array([1 << 30], np.int32))
    assert L.thvm_hip_buf_copy_row(parent.id, 0, 4096, row.id, 0, src.id, 37) == 0
    row.write(np.array([-2], np.int32))
    assert L.thvm_hip_buf_copy_row(parent.id, 0, 4096, row.id, 0, src.id, 37) == 0
    assert np.array_equal(parent.read(np.uint8), want)
    # in range: row 2 of 4096-byte rows at base 9
    row.write(np.array([2], np.int32))
    assert L.thvm_hip_buf_copy_row(parent.id, 9, 4096, row.id, 0, src.id, 37) == 0
    want[9 + 8192:9 + 8192 + 37] = np.arange(37) + 1
    assert np.array_equal(parent.read(np.uint8), want)
    # host-checked errors: a misaligned row index offset, a base past the end
    assert L.thvm_hip_buf_copy_row(parent.id, 0, 16, row.id, 2, src.id, 4) == -1
    assert L.thvm_hip_buf_copy_row(parent.id, n, 16, row.id, 0, src.id, 4) == -1
