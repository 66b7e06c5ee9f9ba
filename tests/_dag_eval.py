"""A plain numpy evaluator of renderer rows (the ThvmUop layout of
include/thvm_hip.h: op, dtype, src0..3, arg0..3 with the reference's UOP_*
and DT_* numbers).  Test infrastructure: it pins the meaning of the captured
reference DAGs (tests/golden/ref_lifted_kernels.npz) against the
reference's own outputs, independently of the HIP renderer.

Semantics: every RANGE not bound by a REDUCE is a parallel axis; a node's
value is an array over the axes it depends on (one array dimension per
axis, size 1 where it does not); REDUCE sums or maxes its axes away;
INDEX_E reads its buffer at the index (0 outside); STORE writes the value at
the index for every point of the parallel axes.  Float nodes round to
float32 after each operation; integers are int64 with C division."""
import numpy as np

CONST, ADD, MUL, NEG, RECIP, EXP2, LOG2, SQRT, CMPLT, REDUCE = 2, 9, 10, 11, 12, 13, 14, 15, 16, 17
CMPEQ, LOAD, CAST, BITCAST, RANGE, INDEX_E = 20, 21, 23, 24, 25, 26
IADD, ISUB, IMUL, IDIV, IMOD, ILT, IAND, IWHERE, BUFFER, STORE = 27, 28, 29, 30, 31, 32, 33, 34, 36, 37
IOR, IXOR, ISHL, ISHR, SIN = 41, 42, 44, 51, 55
FLOATS = {11: np.float16, 12: None, 13: np.float32, 14: np.float64}
NP_OF = {13: np.float32, 11: np.float16, 5: np.int32, 6: np.uint32, 7: np.int64, 0: np.uint8}


def _isf(dt):
    return dt in FLOATS


def _bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def decode_slot(raw: np.ndarray, dt: int) -> np.ndarray:
    if dt == 12:
        return _bf16_to_f32(raw.view(np.uint16))
    return raw.view(NP_OF[dt]).astype(np.float64 if _isf(dt) else np.int64)


def evaluate(rows: np.ndarray, slots: dict) -> np.ndarray:
    """rows [n, 10] int64; slots {slot: decoded 1-D array} for the inputs;
    returns the output buffer (slot 0) as float64 / int64, sized by the
    BUFFER row's element count."""
    n = len(rows)
    ranges = {}                            # node -> (axis id, extent)
    red_axes = set()
    for i, r in enumerate(rows):
        if r[0] == RANGE:
            ranges[i] = (int(r[6]), int(r[8]))
        if r[0] == REDUCE:
            for k in (3, 4, 5):
                if r[k] >= 0:
                    red_axes.add(int(r[k]))
    order = sorted(ranges, key=lambda i: ranges[i][0])
    dim = {node: d for d, node in enumerate(order)}
    nd = len(order)
    val = {}

    def shape_for(node):
        s = [1] * nd
        s[dim[node]] = ranges[node][1]
        return s

    def f32(x):
        return np.asarray(x, np.float64).astype(np.float32).astype(np.float64)

    def ev(i):
        if i in val:
            return val[i]
        r = rows[i]
        op, dt, s = int(r[0]), int(r[1]), [int(x) for x in r[2:6]]
        a = [int(x) for x in r[6:10]]
        fl = _isf(dt)
        if op == CONST:
            bits = np.array([a[0] & 0xFFFFFFFF], np.uint32)
            iv = a[0] & 0xFFFFFFFF
            v = bits.view(np.float32).astype(np.float64)[0] if fl else np.int64(iv - (1 << 32) if iv >= 1 << 31 else iv)
            out = np.full([1] * nd, v)
        elif op == RANGE:
            out = np.arange(ranges[i][1], dtype=np.int64).reshape(shape_for(i))
        elif op == BUFFER:
            out = None
        elif op == INDEX_E:
            buf = slots[int(rows[s[0]][6])]
            idx = np.broadcast_to(ev(s[1]), np.broadcast_shapes(np.shape(ev(s[1])), [1] * nd)).astype(np.int64)
            ok = (idx >= 0) & (idx < len(buf))
            out = np.where(ok, buf[np.clip(idx, 0, len(buf) - 1)], 0)
        elif op == LOAD:
            out = ev(s[0])
        elif op == REDUCE:
            x = ev(s[0])
            axes = tuple(dim[k] for k in s[1:] if k >= 0)
            x = np.broadcast_to(x, np.broadcast_shapes(np.shape(x), tuple(
                ranges[node][1] if d in axes else 1 for d, node in enumerate(order))))
            out = x.sum(axis=axes, keepdims=True) if a[0] == 0 else x.max(axis=axes, keepdims=True)
            out = f32(out) if fl else out
        elif op in (ADD, MUL, IADD, ISUB, IMUL, IAND, IOR, IXOR, ISHL, ISHR, IDIV, IMOD):
            x, y = ev(s[0]), ev(s[1])
            if op in (ADD, IADD):
                out = x + y
            elif op == ISUB:
                out = x - y
            elif op in (MUL, IMUL):
                out = x * y
            elif op == IAND:
                out = x.astype(np.int64) & y.astype(np.int64)
            elif op == IOR:
                out = x.astype(np.int64) | y.astype(np.int64)
            elif op == IXOR:
                out = x.astype(np.int64) ^ y.astype(np.int64)
            elif op == ISHL:
                out = x.astype(np.int64) << y.astype(np.int64)
            elif op == ISHR:
                out = x.astype(np.int64) >> y.astype(np.int64)
            elif op == IDIV:
                out = np.trunc(x / y).astype(np.int64)
            else:
                out = np.fmod(x, y).astype(np.int64)
            out = f32(out) if fl else out
        elif op in (NEG, RECIP, EXP2, LOG2, SQRT, SIN):
            x = ev(s[0])
            out = {NEG: lambda v: -v, RECIP: lambda v: 1.0 / v, EXP2: np.exp2, LOG2: np.log2,
                   SQRT: np.sqrt, SIN: np.sin}[op](x)
            out = f32(out) if fl else out
        elif op in (CMPLT, ILT, CMPEQ):
            x, y = ev(s[0]), ev(s[1])
            out = ((x == y) if op == CMPEQ else (x < y)).astype(np.float64 if fl else np.int64)
        elif op == IWHERE:
            c, x, y = ev(s[0]), ev(s[1]), ev(s[2])
            out = np.where(c != 0, x, y)
        elif op == CAST:
            x = ev(s[0])
            out = f32(x) if fl else np.trunc(x).astype(np.int64)
        else:
            raise NotImplementedError(f"row {i}: op {op}")
        val[i] = out
        return out

    root = rows[n - 1]
    assert root[0] == STORE
    out_rows = int(rows[int(root[2])][7])
    addr = ev(int(root[3]))
    v = ev(int(root[4]))
    full = np.broadcast_shapes(np.shape(addr), np.shape(v), tuple(
        1 if node in red_axes else ranges[node][1] for node in order))
    addr = np.broadcast_to(addr, full).reshape(-1)
    v = np.broadcast_to(v, full).reshape(-1)
    out = np.zeros(out_rows, np.float64)
    ok = (addr >= 0) & (addr < out_rows)
    out[addr[ok]] = v[ok]
    return out
