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
float32 after each operation, whatever their type, and a CAST into fp16 or
bf16 narrows to that type (through f32, round to nearest even), as does the
STORE into an fp16 / bf16 buffer: the reference CPU path's semantics
(src/backend/cpu/uop_walk.c:272-293, the walker that realizes non-f32
kernels).  Integers are int64 with C division.  A RANGE whose src0 is a
DEFINE_VAR row (a symbolic extent) runs to the variable's bound value
(`vars[arg0]`); only the outputs its points write are defined."""
import numpy as np

CONST, ADD, MUL, NEG, RECIP, EXP2, LOG2, SQRT, CMPLT, REDUCE = 2, 9, 10, 11, 12, 13, 14, 15, 16, 17
DEFINE_VAR = 18
CMPEQ, LOAD, CAST, BITCAST, RANGE, INDEX_E = 20, 21, 23, 24, 25, 26
IADD, ISUB, IMUL, IDIV, IMOD, ILT, IAND, IWHERE, BUFFER, STORE = 27, 28, 29, 30, 31, 32, 33, 34, 36, 37
IOR, IXOR, ISHL, ISHR, SIN = 41, 42, 44, 51, 55
FLOATS = {9: None, 11: np.float16, 12: None, 13: np.float32, 14: np.float64}
NP_OF = {13: np.float32, 11: np.float16, 5: np.int32, 6: np.uint32, 7: np.int64, 0: np.uint8}


def _isf(dt):
    return dt in FLOATS


def _bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def narrow(x, dt):
    """x (float64 values) stored in float dtype dt and read back: f32 first,
    then fp16 / bf16 round to nearest even (NaN kept), fp8 e4m3 by the
    kernel-store narrowing (saturating)."""
    f = np.asarray(x, np.float64).astype(np.float32)
    if dt == 9:                  # fp8 e4m3 through the oracle's kernel-store narrowing
        import _oracle as O
        return O.decode(O.encode(f, 9), 9).astype(np.float64)
    if dt == 11:
        return f.astype(np.float16).astype(np.float64)
    if dt == 12:
        u = f.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
        r = np.where(np.isnan(f), f.view(np.uint32) | 0x00400000, r).astype(np.uint32)
        return r.view(np.float32).astype(np.float64)
    return f.astype(np.float64)


def decode_slot(raw: np.ndarray, dt: int) -> np.ndarray:
    if dt == 9:
        import _oracle as O
        return O.decode(raw.view(np.uint8), 9).astype(np.float64)
    if dt == 12:
        return _bf16_to_f32(raw.view(np.uint16))
    return raw.view(NP_OF[dt]).astype(np.float64 if _isf(dt) else np.int64)


def evaluate(rows: np.ndarray, slots: dict, vars=(), written=False, narrow_every_op=False):
    """rows [n, 10] int64; slots {slot: decoded 1-D array} for the inputs;
    vars: the bound values of the DEFINE_VAR rows' variables.  Returns the
    output buffer (slot 0) as float64 / int64, sized by the BUFFER row's
    element count, narrowed to its dtype -- and with written=True also the
    mask of the elements the STORE wrote.  narrow_every_op: the other
    semantics, every fp16 / bf16 op's value narrowed to its type (a
    contrast for the tests, not the reference's)."""
    n = len(rows)
    ranges = {}                            # node -> (axis id, extent)
    red_axes = set()
    for i, r in enumerate(rows):
        if r[0] == RANGE:
            ext = int(r[8])
            if r[2] >= 0:                  # symbolic: the variable's bound value
                vr = rows[int(r[2])]
                assert vr[0] == DEFINE_VAR, f"row {i}: extent expression op {vr[0]}"
                ext = int(vars[int(vr[6])])
            ranges[i] = (int(r[6]), ext)
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

    def f32(x, dt=13):
        if narrow_every_op and dt in (11, 12):
            return narrow(x, dt)
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
        elif op == DEFINE_VAR:
            out = np.full([1] * nd, np.int64(vars[a[0]]))
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
            out = f32(out, dt) if fl else out
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
            out = f32(out, dt) if fl else out
        elif op in (NEG, RECIP, EXP2, LOG2, SQRT, SIN):
            x = ev(s[0])
            out = {NEG: lambda v: -v, RECIP: lambda v: 1.0 / v, EXP2: np.exp2, LOG2: np.log2,
                   SQRT: np.sqrt, SIN: np.sin}[op](x)
            out = f32(out, dt) if fl else out
        elif op in (CMPLT, ILT, CMPEQ):
            x, y = ev(s[0]), ev(s[1])
            out = ((x == y) if op == CMPEQ else (x < y)).astype(np.float64 if fl else np.int64)
        elif op == IWHERE:
            c, x, y = ev(s[0]), ev(s[1]), ev(s[2])
            out = np.where(c != 0, x, y)
        elif op == CAST:
            x = ev(s[0])
            out = narrow(x, dt) if fl else np.trunc(x).astype(np.int64)
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
    odt = int(rows[int(root[2])][1])
    if _isf(odt):
        out = narrow(out, odt)
    if written:
        mask = np.zeros(out_rows, bool)
        mask[addr[ok]] = True
        return out, mask
    return out
