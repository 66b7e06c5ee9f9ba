"""thvm_amd.tensor -- the lazy Tensor / TinyJit / Variable / Device host for
DEV=hip.

Mirrors the reference's Python host surface for the decode path
(py/thvm/tensor.py, py/thvm/_misc.py:172-245 TinyJit, py/thvm/device.py:28-41
Device, bench/gpt2/thvm_gpt2.py the GPT-2 driver it serves): tensors built
from numpy, lazy elementwise / reduce / movement ops, ``realize``,
``numpy``/``tolist``, ``assign`` into KV-cache slices, symbolic
``Variable.bind`` lengths, and ``TinyJit`` capture on the second call with
replay afterwards.

How a realize runs on MI355X:
  * the lazy graph is cut into kernels at reductions that cannot fuse (a
    reduce read through a broadcast or inside another reduce), at
    matmuls and at ``contiguous``; elementwise and movement ops fuse into the
    kernel that reads them (movement ops become index arithmetic);
  * ``x @ W.T`` with a contiguous weight and a small row count runs the
    hand-written gfx950 GEMV / MFMA builtin (bias fused); every other kernel
    is a lifted uop DAG that the library's renderer target turns into HIP
    source (compiled by hiprtc, cached by source);
  * symbolic lengths live in a device int32 buffer that kernels read, so a
    TinyJit graph replays correctly at every bound value; buffers of a
    symbolic shape are laid out at the variable's maximum.
There is no CPU fallback: every kernel runs through libthvm_hip.so."""
from __future__ import annotations

import math
import os
import struct
from typing import Optional, Sequence, Union

import numpy as np

import thvm_amd as _hip

# reference op numbers (src/thvm.h:302-512), axis types (:686-692), reduce
# kinds (:515-516)
U_CONST, U_ADD, U_MUL, U_NEG, U_RECIP, U_EXP2, U_LOG2, U_SQRT, U_CMPLT = 2, 9, 10, 11, 12, 13, 14, 15, 16
U_REDUCE, U_DEFINE_VAR, U_CMPEQ, U_LOAD, U_CAST, U_RANGE, U_INDEX_E = 17, 18, 20, 21, 23, 25, 26
U_IADD, U_ISUB, U_IMUL, U_IDIV, U_IMOD, U_ILT, U_IAND, U_IWHERE = 27, 28, 29, 30, 31, 32, 33, 34
U_BUFFER, U_STORE, U_IXOR, U_SIN = 36, 37, 42, 55
U_IOR, U_ISHL, U_ISHR = 41, 44, 51
KAX_REDUCE, KAX_GLOBAL = 1, 5
REDUCE_SUM, REDUCE_MAX = 0, 1


# --------------------------------------------------------------------------- dtypes
class DType:
    __slots__ = ("name", "id", "itemsize", "np")

    def __init__(self, name: str, id_: int, itemsize: int, npt):
        self.name, self.id, self.itemsize, self.np = name, id_, itemsize, npt

    def __repr__(self):
        return f"dtypes.{self.name}"


class dtypes:
    bool = DType("bool", 0, 1, np.bool_)
    uint8 = DType("uint8", 2, 1, np.uint8)
    uint32 = DType("uint", 6, 4, np.uint32)
    int32 = DType("int", 5, 4, np.int32)
    float16 = DType("half", 11, 2, np.float16)
    bfloat16 = DType("bfloat16", 12, 2, np.uint16)
    float32 = DType("float", 13, 4, np.float32)
    half = float16
    float = float32
    int = int32
    default_float = float32
    default_int = int32

    @staticmethod
    def is_float(dt: DType) -> bool:
        return dt.id in (11, 12, 13)

    @staticmethod
    def from_np(d) -> DType:
        d = np.dtype(d)
        for t in (dtypes.float32, dtypes.float16, dtypes.int32, dtypes.bool, dtypes.uint8, dtypes.uint32):
            if np.dtype(t.np) == d:
                return t
        if d == np.float64:
            return dtypes.float32
        if d == np.int64:
            return dtypes.int32
        raise TypeError(f"no device dtype for numpy {d}")


def _promote(a: DType, b: DType) -> DType:
    if a.id == b.id:
        return a
    fa, fb = dtypes.is_float(a), dtypes.is_float(b)
    if fa and fb:
        return dtypes.float32 if 13 in (a.id, b.id) else a
    if fa or fb:
        return a if fa else b
    return dtypes.int32


# --------------------------------------------------------------------------- symbolic ints
class Variable:
    """A symbolic int (reference py/thvm Variable / tinygrad UOp.variable):
    ``Variable(name, min, max).bind(v)``.  Variables of one name share one
    slot of the device variable buffer."""
    _slots: dict = {}

    def __init__(self, name: str, min_val: int, max_val: int):
        self.name, self.min, self.max = name, int(min_val), int(max_val)
        if name not in Variable._slots:
            if len(Variable._slots) >= 64:
                raise RuntimeError("more than 64 variable names")
            Variable._slots[name] = len(Variable._slots)
        self.slot = Variable._slots[name]
        self.val: Optional[int] = None

    def bind(self, val: int) -> "Variable":
        val = int(val)
        if not self.min <= val <= self.max:
            raise ValueError(f"{self.name}={val} outside [{self.min}, {self.max}]")
        self.val = val
        _VARS[self.name] = self
        return self

    def unbind(self):
        return self, self.val

    def _s(self) -> "Sym":
        return Sym({self.name: (self, 1)}, 0)

    def __add__(self, o): return self._s() + o
    __radd__ = __add__
    def __sub__(self, o): return self._s() - o
    def __mul__(self, o): return self._s() * o
    __rmul__ = __mul__

    def __repr__(self):
        return f"Variable({self.name}={self.val}, [{self.min},{self.max}])"


_VARS: dict = {}        # name -> the Variable bound most recently


class Sym:
    """c + sum(k_v * v): the affine symbolic ints the decode path needs."""
    __slots__ = ("terms", "c")

    def __init__(self, terms: dict, c: int):
        self.terms = {k: v for k, v in terms.items() if v[1] != 0}
        self.c = int(c)

    def __add__(self, o):
        if isinstance(o, Variable):
            o = o._s()
        if isinstance(o, Sym):
            t = dict(self.terms)
            for k, (v, m) in o.terms.items():
                t[k] = (v, t[k][1] + m) if k in t else (v, m)
            return _simp(Sym(t, self.c + o.c))
        return _simp(Sym(self.terms, self.c + int(o)))
    __radd__ = __add__

    def __sub__(self, o):
        return self + (-1) * o if isinstance(o, (Sym, Variable)) else self + (-int(o))

    def __rsub__(self, o):
        return (-1) * self + o

    def __mul__(self, o):
        if isinstance(o, (Sym, Variable)):
            raise NotImplementedError("symbolic * symbolic")
        o = int(o)
        return _simp(Sym({k: (v, m * o) for k, (v, m) in self.terms.items()}, self.c * o))
    __rmul__ = __mul__

    @property
    def vmax(self) -> int:
        return self.c + sum(m * (v.max if m > 0 else v.min) for v, m in self.terms.values())

    @property
    def vmin(self) -> int:
        return self.c + sum(m * (v.min if m > 0 else v.max) for v, m in self.terms.values())

    @property
    def val(self) -> int:
        return self.c + sum(m * _VARS.get(k, v).val for k, (v, m) in self.terms.items())

    def key(self):
        return (tuple(sorted((k, m) for k, (_, m) in self.terms.items())), self.c)

    def __eq__(self, o):
        if isinstance(o, Variable):
            o = o._s()
        return isinstance(o, Sym) and self.key() == o.key()

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return " + ".join([f"{m}*{k}" for k, (_, m) in self.terms.items()] + [str(self.c)])


def _simp(s: Sym):
    return s.c if not s.terms else s


def _sym(x):
    return x._s() if isinstance(x, Variable) else x


def smax(x) -> int:
    x = _sym(x)
    return x.vmax if isinstance(x, Sym) else int(x)


def sval(x) -> int:
    x = _sym(x)
    return x.val if isinstance(x, Sym) else int(x)


def _prod(xs):
    r = 1
    for x in xs:
        r = r * x
    return r


def _eq(a, b) -> bool:
    a, b = _sym(a), _sym(b)
    if isinstance(a, Sym) or isinstance(b, Sym):
        return isinstance(a, Sym) and isinstance(b, Sym) and a == b
    return int(a) == int(b)


# --------------------------------------------------------------------------- device
class _Device:
    """Device selection from ``DEV`` (reference py/thvm/device.py:28-41):
    this host serves ``HIP`` (one device, index 0)."""
    DEFAULT = "HIP"

    def canonicalize(self, d: Optional[str]) -> str:
        d = (d or self.DEFAULT).upper().split(":")[0]
        if d not in ("HIP", "GPU", "AMD"):
            raise RuntimeError(f"device {d}: this host runs on HIP only")
        return "HIP"

    def __getitem__(self, d):
        self.canonicalize(d)
        _ensure_init()
        return self


Device = _Device()
_INIT = False


def _ensure_init():
    global _INIT
    if not _INIT:
        _hip.device_from_env()
        _hip.init()
        _INIT = True


# --------------------------------------------------------------------------- buffers
class RBuf:
    """One device allocation owned by the host (freed with its last user)."""
    __slots__ = ("b", "nbytes", "__weakref__")

    def __init__(self, nbytes: int):
        _ensure_init()
        self.b = _hip.Buffer(max(int(nbytes), 16))
        self.nbytes = int(nbytes)

    @property
    def id(self) -> int:
        return self.b.id

    def __del__(self):
        try:
            if self.b.id:
                self.b.free()
        except Exception:
            pass


class _KV:
    """The device int32[64] that kernels read variable values from."""
    buf: Optional[RBuf] = None
    host = np.zeros(64, np.int32)
    dirty = True

    @classmethod
    def get(cls) -> RBuf:
        if cls.buf is None:
            cls.buf = RBuf(64 * 4)
            cls.dirty = True
        return cls.buf

    @classmethod
    def sync(cls):
        b = cls.get()
        new = cls.host.copy()
        for name, v in _VARS.items():
            if v.val is not None:
                new[v.slot] = v.val
        if cls.dirty or not np.array_equal(new, cls.host):
            cls.host = new
            b.b.write(new)
            cls.dirty = False


_CAPTURE: Optional[list] = None   # buffers a TinyJit capture must keep alive


# --------------------------------------------------------------------------- lazy graph
class LNode:
    """A lazy value: op over sources, or a realized buffer (op 'BUF')."""
    __slots__ = ("op", "srcs", "arg", "shape", "dtype", "rb", "strides", "offset", "__weakref__")

    def __init__(self, op, srcs, arg, shape, dtype):
        self.op, self.srcs, self.arg = op, tuple(srcs), arg
        self.shape, self.dtype = tuple(shape), dtype
        self.rb, self.strides, self.offset = None, None, 0

    def make_buf(self, rb: RBuf, strides, offset=0):
        self.op, self.srcs, self.arg = "BUF", (), None
        self.rb, self.strides, self.offset = rb, tuple(strides), offset


def _cstrides(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc *= smax(s)
    return tuple(reversed(st))


VIEW_OPS = ("RESHAPE", "PERMUTE", "EXPAND", "SHRINK", "PAD")


# --------------------------------------------------------------------------- kernel builder
class _KB:
    """Builds one kernel's lifted uop DAG (ThvmUop rows)."""

    def __init__(self):
        self.nodes: list = []
        self.memo: dict = {}
        self.cval: dict = {}
        self.slots: dict = {}
        self.bufs: list = []
        self.axis = 0
        self.memo_lower: dict = {}

    def add(self, op, dt, srcs=(), args=()):
        key = (op, dt, tuple(srcs), tuple(int(a) for a in args))
        if key in self.memo:
            return self.memo[key]
        self.nodes.append(key)
        i = len(self.nodes) - 1
        self.memo[key] = i
        return i

    # ---- constants and index arithmetic (int32, folded) ----
    def i(self, v: int) -> int:
        idx = self.add(U_CONST, 5, (), (int(v),))
        self.cval[idx] = int(v)
        return idx

    def const(self, v, dt: DType) -> int:
        if dtypes.is_float(dt):
            bits = struct.unpack("<I", struct.pack("<f", float(v)))[0]
            return self.add(U_CONST, dt.id, (), (bits,))
        if dt.id == 0:
            return self.add(U_CONST, 0, (), (1 if v else 0,))
        idx = self.add(U_CONST, dt.id, (), (int(v),))
        if dt.id == 5:
            self.cval[idx] = int(v)
        return idx

    def sym(self, x) -> int:
        x = _sym(x)
        if not isinstance(x, Sym):
            return self.i(int(x))
        r = self.i(x.c)
        for _, (v, m) in sorted(x.terms.items()):
            dv = self.add(U_DEFINE_VAR, 5, (), (v.slot, v.min, v.max))
            r = self.iadd(r, self.imul(dv, self.i(m)))
        return r

    def iadd(self, a, b):
        ca, cb = self.cval.get(a), self.cval.get(b)
        if ca is not None and cb is not None:
            return self.i(ca + cb)
        if ca == 0:
            return b
        if cb == 0:
            return a
        return self.add(U_IADD, 5, (a, b))

    def isub(self, a, b):
        cb = self.cval.get(b)
        if cb is not None:
            return self.iadd(a, self.i(-cb))
        return self.add(U_ISUB, 5, (a, b))

    def imul(self, a, b):
        ca, cb = self.cval.get(a), self.cval.get(b)
        if ca is not None and cb is not None:
            return self.i(ca * cb)
        if ca == 0 or cb == 0:
            return self.i(0)
        if ca == 1:
            return b
        if cb == 1:
            return a
        return self.add(U_IMUL, 5, (a, b))

    def idiv(self, a, b):
        ca, cb = self.cval.get(a), self.cval.get(b)
        if cb == 1:
            return a
        if ca is not None and cb is not None:
            return self.i(int(ca / cb))
        return self.add(U_IDIV, 5, (a, b))

    def imod(self, a, b):
        ca, cb = self.cval.get(a), self.cval.get(b)
        if cb == 1:
            return self.i(0)
        if ca is not None and cb is not None:
            return self.i(ca % cb)
        return self.add(U_IMOD, 5, (a, b))

    def ilt(self, a, b):
        ca, cb = self.cval.get(a), self.cval.get(b)
        if ca is not None and cb is not None:
            return self.i(1 if ca < cb else 0)
        return self.add(U_ILT, 5, (a, b))

    def iand(self, a, b):
        ca, cb = self.cval.get(a), self.cval.get(b)
        if ca == 1:
            return b
        if cb == 1:
            return a
        return self.add(U_IAND, 5, (a, b))

    def buffer(self, rb: RBuf, dt: DType, slot: Optional[int] = None) -> int:
        key = id(rb)
        if key not in self.slots:
            s = len(self.bufs) if slot is None else slot
            self.slots[key] = s
            if s == len(self.bufs):
                self.bufs.append(rb)
            else:
                self.bufs[s] = rb
        cap = rb.nbytes // dt.itemsize if rb.nbytes else 0
        return self.add(U_BUFFER, dt.id, (), (self.slots[key], cap))

    def rng(self, extent, kind) -> int:
        ax = self.axis
        self.axis += 1
        extent = _sym(extent)
        if isinstance(extent, Sym):
            return self.add(U_RANGE, 5, (self.sym(extent),), (ax, kind, 0))
        return self.add(U_RANGE, 5, (), (ax, kind, int(extent)))

    # ---- values ----
    def cast(self, v: int, dt: DType) -> int:
        if self.nodes[v][1] == dt.id:
            return v
        return self.add(U_CAST, dt.id, (v,))

    def load(self, n: LNode, idx) -> int:
        addr = self.i(n.offset)
        for ix, s, st in zip(idx, n.shape, n.strides):
            if _eq(s, 1):
                continue
            addr = self.iadd(addr, self.imul(ix, self.i(st)))
        b = self.buffer(n.rb, n.dtype)
        return self.add(U_LOAD, n.dtype.id, (self.add(U_INDEX_E, 5, (b, addr)),))

    def view_idx(self, n: LNode, idx):
        """index of n's source element that n's element `idx` reads, and the
        validity (PAD) -- None when always valid."""
        src = n.srcs[0]
        if n.op == "PERMUTE":
            out = [None] * len(idx)
            for i, p in enumerate(n.arg):
                out[p] = idx[i]
            return out, None
        if n.op == "EXPAND":
            return [self.i(0) if _eq(s, 1) and not _eq(ns, 1) else ix
                    for ix, s, ns in zip(idx, src.shape, n.shape)], None
        if n.op == "SHRINK":
            return [self.iadd(ix, self.sym(b)) for ix, (b, _) in zip(idx, n.arg)], None
        if n.op == "PAD":
            valid, out = None, []
            for ix, (pb, _), s in zip(idx, n.arg, src.shape):
                if pb == 0 and _eq(s, n.shape[len(out)]):
                    out.append(ix)
                    continue
                lo = self.add(U_IXOR, 5, (self.ilt(ix, self.i(pb)), self.i(1)))
                hi = self.ilt(ix, self.iadd(self.sym(s), self.i(pb)))
                v = self.iand(lo, hi)
                valid = v if valid is None else self.iand(valid, v)
                out.append(self.isub(ix, self.i(pb)))
            if valid is not None:
                out = [self.add(U_IWHERE, 5, (valid, o, self.i(0))) for o in out]
            return out, valid
        if n.op == "RESHAPE":
            return self.reshape_idx(src.shape, n.shape, idx), None
        raise AssertionError(n.op)

    def reshape_idx(self, sshape, nshape, idx):
        sn = [i for i, s in enumerate(sshape) if not _eq(s, 1)]
        nn = [i for i, s in enumerate(nshape) if not _eq(s, 1)]
        if len(sn) == len(nn) and all(_eq(sshape[a], nshape[b]) for a, b in zip(sn, nn)):
            out = [self.i(0)] * len(sshape)
            for a, b in zip(sn, nn):
                out[a] = idx[b]
            return out
        flat = self.i(0)
        for ix, st in zip(idx, _sym_cstrides(nshape)):
            flat = self.iadd(flat, self.imul(ix, self.sym(st)))
        out = []
        for s, st in zip(sshape, _sym_cstrides(sshape)):
            out.append(self.imod(self.idiv(flat, self.sym(st)), self.sym(s)) if not _eq(s, 1) else self.i(0))
        return out

    def lower(self, n: LNode, idx) -> int:
        key = (id(n), tuple(idx))
        if key in self.memo_lower:
            return self.memo_lower[key]
        v = self._lower(n, list(idx))
        self.memo_lower[key] = v
        return v

    def _lower(self, n: LNode, idx) -> int:
        op = n.op
        if op == "BUF":
            return self.load(n, idx)
        if op == "CONST":
            return self.const(n.arg, n.dtype)
        if op == "ARANGE":
            start, step = n.arg
            v = self.iadd(self.i(start), self.imul(idx[-1], self.i(step)))
            return self.cast(v, n.dtype)
        if op == "CAST":
            return self.cast(self.lower(n.srcs[0], idx), n.dtype)
        if op in ("CONTIG", "ASSIGN_SRC"):
            return self.lower(n.srcs[0], idx)
        if op in VIEW_OPS:
            sidx, valid = self.view_idx(n, idx)
            v = self.lower(n.srcs[0], sidx)
            if valid is not None:
                v = self.add(U_IWHERE, n.dtype.id, (valid, v, self.const(0, n.dtype)))
            return v
        if op == "ALU":
            return self.alu(n, idx)
        if op == "REDUCE":
            kind, axes = n.arg
            src = n.srcs[0]
            rs, sidx = [], list(idx)
            for a in axes:
                r = self.rng(src.shape[a], KAX_REDUCE)
                rs.append(r)
                sidx[a] = r
            if len(rs) > 3:
                raise NotImplementedError("reduce over more than 3 axes at once")
            body = self.lower(src, sidx)
            acc = n.dtype if dtypes.is_float(n.dtype) else dtypes.int32
            return self.add(U_REDUCE, acc.id, (self.cast(body, acc), *rs), (kind,))
        if op == "MATMUL":
            x, w = n.srcs[0], n.srcs[1]
            K = x.shape[-1]
            r = self.rng(K, KAX_REDUCE)
            bidx = idx[:-2]
            xi = _bcast_idx(self, x.shape[:-2], n.shape[:-2], bidx) + [idx[-2], r]
            wi = _bcast_idx(self, w.shape[:-2], n.shape[:-2], bidx) + [r, idx[-1]]
            acc = dtypes.float32 if dtypes.is_float(n.dtype) else dtypes.int32
            prod = self.add(U_MUL if acc.id == 13 else U_IMUL, acc.id,
                            (self.cast(self.lower(x, xi), acc), self.cast(self.lower(w, wi), acc)))
            v = self.add(U_REDUCE, acc.id, (prod, r), (REDUCE_SUM,))
            if len(n.srcs) > 2:
                b = n.srcs[2]
                v = self.add(U_ADD, acc.id, (v, self.cast(self.lower(b, [idx[-1]]), acc)))
            return self.cast(v, n.dtype)
        if op == "GATHER":
            w, ix = n.srcs
            tok = self.cast(self.lower(ix, idx[:-1]), dtypes.int32)
            if w.op != "BUF":
                raise AssertionError("gather table not realized")
            addr = self.iadd(self.i(w.offset), self.iadd(self.imul(tok, self.i(w.strides[0])),
                                                           self.imul(idx[-1], self.i(w.strides[1]))))
            b = self.buffer(w.rb, w.dtype)
            return self.add(U_LOAD, w.dtype.id, (self.add(U_INDEX_E, 5, (b, addr)),))
        raise NotImplementedError(f"lowering of {op}")

    def alu(self, n: LNode, idx) -> int:
        name = n.arg
        srcs = [self.lower(s, idx) for s in n.srcs]
        dt = n.dtype
        if name == "WHERE":
            return self.add(U_IWHERE, dt.id, (srcs[0], self.cast(srcs[1], dt), self.cast(srcs[2], dt)))
        if name in ("CMPLT", "CMPEQ"):
            t = _promote(n.srcs[0].dtype, n.srcs[1].dtype)
            a, b = self.cast(srcs[0], t), self.cast(srcs[1], t)
            code = U_CMPEQ if name == "CMPEQ" else (U_CMPLT if dtypes.is_float(t) else U_ILT)
            return self.add(code, 0, (a, b))
        srcs = [self.cast(s, dt) for s in srcs]
        fl = dtypes.is_float(dt)
        code = {"ADD": U_ADD if fl else U_IADD, "MUL": U_MUL if fl else U_IMUL, "NEG": U_NEG,
                "RECIP": U_RECIP, "EXP2": U_EXP2, "LOG2": U_LOG2, "SQRT": U_SQRT, "SIN": U_SIN,
                "IDIV": U_IDIV, "IMOD": U_IMOD, "XOR": U_IXOR, "AND": U_IAND, "OR": U_IOR,
                "SHL": U_ISHL, "SHR": U_ISHR}[name]
        return self.add(code, dt.id, tuple(srcs))


def _sym_cstrides(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc = _sym(acc * _sym(s)) if not isinstance(_sym(s), int) else acc * int(s)
    return list(reversed(st))


def _bcast_idx(kb: _KB, sshape, oshape, idx):
    pad = len(oshape) - len(sshape)
    out = []
    for i, s in enumerate(sshape):
        out.append(kb.i(0) if _eq(s, 1) and not _eq(oshape[pad + i], 1) else idx[pad + i])
    return out


# --------------------------------------------------------------------------- scheduling
def _deps(root: LNode) -> list:
    """Nodes to realize before root's kernel: reductions that cannot fuse,
    matmuls, contiguous points, gather tables."""
    out, seen = [], set()

    def walk(n: LNode, in_red: bool, expanded: bool, is_root: bool):
        key = (id(n), in_red, expanded)
        if key in seen:
            return
        seen.add(key)
        if n.op in ("BUF", "CONST", "ARANGE"):
            return
        if n.op == "MATMUL":
            if is_root:
                for s in n.srcs:
                    walk(s, True, False, False)
            else:
                out.append(n)
            return
        if n.op == "REDUCE":
            if is_root or (not in_red and not expanded):
                walk(n.srcs[0], True, False, False)
            else:
                out.append(n)
            return
        if n.op in ("CONTIG", "ASSIGN"):
            if is_root:
                walk(n.srcs[-1], in_red, expanded, False)
            else:
                out.append(n)
            return
        if n.op == "GATHER":
            if n.srcs[0].op != "BUF":
                out.append(n.srcs[0])
            walk(n.srcs[1], in_red, expanded, False)
            return
        exp = expanded or n.op == "EXPAND"
        for s in n.srcs:
            walk(s, in_red, exp, False)

    walk(root, False, False, True)
    return out


_RENDER_CACHE: dict = {}
_RNG_SEED = 0          # Tensor.manual_seed
_RNG_CTR = None        # the generator's device counter (a uint32 Tensor)
_IN_JIT = 0        # inside a TinyJit function's eager first call


def _beam_width() -> int:
    """Search width for a kernel rendered now: JITBEAM inside a TinyJit
    function (the kernels its graph will replay), else BEAM; 0 = no search
    (py/thvm tinygrad semantics, src/codegen/autotune.c:124-131)."""
    jb = int(os.environ.get("JITBEAM", "0") or 0)
    if _IN_JIT and jb > 0:
        return jb
    return int(os.environ.get("BEAM", "0") or 0)


GlobalCounters = type("GlobalCounters", (), {"kernel_count": 0, "gemv_count": 0})


def _dispatch_rendered(kb: _KB):
    key = tuple(kb.nodes)
    hit = _RENDER_CACHE.get(key)
    if hit is None:
        name = "r_%016x" % (hash(key) & 0xFFFFFFFFFFFFFFFF)
        src, info = _hip.render_kernel(kb.nodes, name)
        width = _beam_width()
        if width > 0 and _CAPTURE is None:
            # the reference's BEAM: search this kernel's geometry once, on its
            # own buffers (kernels that read their output are not searched)
            args = [b.id for b in kb.bufs]
            if info.kvar_slot:
                _KV.sync()
                args.append(_KV.get().id)
            try:
                opts = _hip.render_autotune(kb.nodes, args, beam=width)[0]
                src, info = _hip.render_kernel(kb.nodes, name, opts=opts)
            except _hip.ThvmHipError:
                pass
        hit = (name, src, int(info.grid_max), int(info.block), int(info.kvar_slot))
        _RENDER_CACHE[key] = hit
    name, src, grid, block, kvar_slot = hit
    ids = [b.id for b in kb.bufs]
    if kvar_slot:
        _KV.sync()
        ids.append(_KV.get().id)
    if _CAPTURE is not None:
        _CAPTURE.extend(kb.bufs)
    _hip.dispatch(name, src, ids, grid=(grid, 1, 1), block=(block, 1, 1), outs=(0,))
    GlobalCounters.kernel_count += 1


def _run_kernel(root: LNode, out: LNode, out_idx_fn=None):
    """One kernel computing `root` over its shape into `out` (a BUF node, or
    a view of one for ASSIGN)."""
    kb = _KB()
    ob = out if out.op == "BUF" else _view_base(out)
    kb.buffer(ob.rb, ob.dtype, slot=0)
    idx = [kb.i(0) if _eq(s, 1) else kb.rng(s, KAX_GLOBAL) for s in root.shape]
    val = kb.lower(root, idx)
    addr = _view_addr(kb, out, idx)
    b0 = kb.buffer(ob.rb, ob.dtype)
    kb.add(U_STORE, ob.dtype.id, (b0, addr, val))
    _dispatch_rendered(kb)


def _view_base(n: LNode) -> LNode:
    while n.op in VIEW_OPS or n.op == "CONTIG":
        n = n.srcs[0]
    if n.op != "BUF":
        raise RuntimeError("assign target is not a view of a realized buffer")
    return n


def _view_addr(kb: _KB, n: LNode, idx):
    while n.op != "BUF":
        if n.op in ("EXPAND", "PAD"):
            raise RuntimeError(f"cannot write through a {n.op} view")
        if n.op == "CONTIG":
            n = n.srcs[0]
            continue
        idx, _ = kb.view_idx(n, idx)
        n = n.srcs[0]
    addr = kb.i(n.offset)
    for ix, s, st in zip(idx, n.shape, n.strides):
        if not _eq(s, 1):
            addr = kb.iadd(addr, kb.imul(ix, kb.i(st)))
    return addr


def _is_contig_buf(n: LNode) -> bool:
    return n.op == "BUF" and n.offset == 0 and n.strides == _cstrides(n.shape) and \
        all(isinstance(_sym(s), int) for s in n.shape)


def _try_gemv(n: LNode) -> bool:
    """x @ W.T (+ b) on the gfx950 GEMV / MFMA builtin: W a contiguous
    realized [N, K] weight, x rows contiguous, M = rows <= 64."""
    x, w = n.srcs[0], n.srcs[1]
    if not (w.op == "PERMUTE" and w.arg == (1, 0) and _is_contig_buf(w.srcs[0])):
        return False
    W = w.srcs[0]
    if any(not isinstance(_sym(s), int) for s in n.shape):
        return False
    N, K = int(W.shape[0]), int(W.shape[1])
    M = int(_prod(n.shape[:-1]))
    wt, xt = W.dtype.id, x.dtype.id
    if xt not in (11, 12, 13) or wt not in (11, 12, 13) or n.dtype.id != xt:
        return False
    mfma = (wt == xt and wt in (11, 12) and K % 64 == 0)
    if M > 64 or (M > 4 and not mfma):
        return False
    bias = n.srcs[2] if len(n.srcs) > 2 else None
    if bias is not None and bias.dtype.id != xt:
        return False
    for s in ([x] + ([bias] if bias is not None else [])):
        if not _is_contig_buf(s):
            if s.op == "BUF":          # a strided / offset buffer: copy it
                c = LNode("CONTIG", (LNode("BUF", (), None, s.shape, s.dtype),), None, s.shape, s.dtype)
                c.srcs[0].make_buf(s.rb, s.strides, s.offset)
                _realize(c)
                s.make_buf(c.rb, c.strides, c.offset)
            else:
                _realize(s)
    x = n.srcs[0]
    out = RBuf(M * N * n.dtype.itemsize)
    args = [out.id, x.rb.id, W.rb.id] + ([bias.rb.id] if bias is not None else [])
    if _CAPTURE is not None:
        _CAPTURE.extend([out, x.rb, W.rb] + ([bias.rb] if bias is not None else []))
    _hip.builtin("gemv", args, m=M, n=N, k=K, wt=wt, xt=xt, yt=xt, epi=0,
                 bias=1 if bias is not None else 0)
    GlobalCounters.gemv_count += 1
    n.make_buf(out, _cstrides(n.shape))
    return True


def _host_gemv() -> bool:
    """THVM_HOST_GEMV=0 renders x @ W.T like every other kernel (a lifted
    reduce through the renderer target and its opts) instead of calling the
    GEMV builtin."""
    return os.environ.get("THVM_HOST_GEMV", "1") != "0"


def _realize(n: LNode):
    if n.op == "BUF":
        return
    if n.op == "MATMUL" and _host_gemv() and _try_gemv(n):
        return
    if n.op == "ASSIGN":
        target, value = n.srcs
        for d in _deps(value) + ([value] if value.op in ("MATMUL", "REDUCE") else []):
            _realize(d)
        _run_kernel(value, target)
        n.op, n.srcs, n.arg = target.op, target.srcs, target.arg
        n.rb, n.strides, n.offset = target.rb, target.strides, target.offset
        return
    for d in _deps(n):
        _realize(d)
    if n.op == "BUF":
        return
    shape_max = [smax(s) for s in n.shape]
    rb = RBuf(int(_prod(shape_max)) * n.dtype.itemsize)
    dst = LNode("BUF", (), None, n.shape, n.dtype)
    dst.make_buf(rb, _cstrides(n.shape))
    _run_kernel(n, dst)
    n.make_buf(rb, dst.strides)


# --------------------------------------------------------------------------- Tensor
Scalar = Union[int, float, bool]


class Tensor:
    """Lazy device tensor (reference py/thvm/tensor.py; tinygrad Tensor)."""
    __slots__ = ("node",)
    training = False
    no_grad = True

    def __init__(self, data, dtype: Optional[DType] = None, device: Optional[str] = None,
                 requires_grad: Optional[bool] = None):
        Device.canonicalize(device)
        if isinstance(data, LNode):
            self.node = data
            return
        if isinstance(data, Tensor):
            self.node = data.node
            return
        if isinstance(data, (int, float, bool)):
            dt = dtype or (dtypes.float32 if isinstance(data, float) else
                           dtypes.bool if isinstance(data, bool) else dtypes.int32)
            self.node = LNode("CONST", (), data, (), dt)
            return
        a = np.asarray(data)
        dt = dtype or dtypes.from_np(a.dtype)
        if dt.id == 12:
            a = _bf16_bits(np.asarray(a, np.float32))
        else:
            a = np.ascontiguousarray(a.astype(dt.np))
        rb = RBuf(a.nbytes)
        if a.nbytes:
            rb.b.write(a)
        n = LNode("BUF", (), None, a.shape, dt)
        n.make_buf(rb, _cstrides(a.shape))
        self.node = n

    # ---- properties ----
    @property
    def shape(self):
        return self.node.shape

    @property
    def dtype(self) -> DType:
        return self.node.dtype

    @property
    def device(self) -> str:
        return "HIP"

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def numel(self):
        return _prod(self.shape)

    def __repr__(self):
        return f"<Tensor {self.shape} {self.dtype} {self.node.op}>"

    # ---- creation ----
    @staticmethod
    def full(shape, fill_value, dtype: Optional[DType] = None, **kw) -> "Tensor":
        shape = tuple(shape) if isinstance(shape, (tuple, list)) else (shape,)
        dt = dtype or (dtypes.float32 if isinstance(fill_value, float) else
                       dtypes.bool if isinstance(fill_value, bool) else dtypes.int32)
        return Tensor(LNode("CONST", (), fill_value, (), dt)).reshape((1,) * len(shape)).expand(shape) \
            if shape else Tensor(LNode("CONST", (), fill_value, (), dt))

    @staticmethod
    def zeros(*shape, dtype: Optional[DType] = None, **kw) -> "Tensor":
        shape = shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        return Tensor.full(shape, 0.0 if dtype is None or dtypes.is_float(dtype) else 0,
                           dtype=dtype or dtypes.float32)

    @staticmethod
    def ones(*shape, dtype: Optional[DType] = None, **kw) -> "Tensor":
        shape = shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        return Tensor.full(shape, 1.0 if dtype is None or dtypes.is_float(dtype) else 1,
                           dtype=dtype or dtypes.float32)

    @staticmethod
    def arange(start, stop=None, step=1, dtype: Optional[DType] = None, **kw) -> "Tensor":
        if stop is None:
            start, stop = 0, start
        n = max(0, math.ceil((stop - start) / step))
        dt = dtype or (dtypes.float32 if any(isinstance(v, float) for v in (start, stop, step)) else dtypes.int32)
        return Tensor(LNode("ARANGE", (), (start, step), (n,), dt))

    @staticmethod
    def empty(*shape, dtype: Optional[DType] = None, **kw) -> "Tensor":
        return Tensor.zeros(*shape, dtype=dtype).contiguous()

    # ---- realization ----
    def realize(self) -> "Tensor":
        _realize(self.node)
        return self

    def contiguous(self) -> "Tensor":
        if _is_contig_buf(self.node):
            return self
        return Tensor(LNode("CONTIG", (self.node,), None, self.shape, self.dtype))

    def numpy(self) -> np.ndarray:
        if any(not isinstance(_sym(s), int) for s in self.shape):
            raise RuntimeError("numpy() of a symbolic shape")
        t = self if _is_contig_buf(self.node) else Tensor(LNode("CONTIG", (self.node,), None, self.shape, self.dtype))
        t.realize()
        n = t.node
        cnt = int(_prod(n.shape))
        if cnt == 0:
            return np.zeros(n.shape, n.dtype.np)
        a = n.rb.b.read(n.dtype.np if n.dtype.id != 0 else np.uint8, cnt)
        if n.dtype.id == 12:
            a = (a.astype(np.uint32) << 16).view(np.float32)
        if n.dtype.id == 0:
            a = a.astype(np.bool_)
        return a.reshape(n.shape)

    def tolist(self):
        return self.numpy().tolist()

    def item(self):
        return self.numpy().reshape(-1)[0].item()

    def replace(self, x) -> "Tensor":
        """This tensor now stands for x (same shape; x's dtype and data), as
        tinygrad's replace: the model's attribute keeps its identity."""
        x = x if isinstance(x, Tensor) else Tensor(x, dtype=self.dtype)
        if tuple(map(_key, x.shape)) != tuple(map(_key, self.shape)):
            raise ValueError(f"replace: shape {x.shape} for a tensor of shape {self.shape}")
        self.node = x.node
        return self

    def assign(self, x) -> "Tensor":
        x = x if isinstance(x, Tensor) else Tensor(x, dtype=self.dtype)
        if tuple(map(_key, x.shape)) != tuple(map(_key, self.shape)):
            x = x.expand(self.shape)
        if x.dtype.id != self.dtype.id:
            x = x.cast(self.dtype)
        src = LNode("ASSIGN_SRC", (x.node,), None, x.shape, x.dtype)
        return Tensor(LNode("ASSIGN", (self.node, src), None, self.shape, self.dtype))

    # ---- elementwise ----
    def _bin(self, o, op: str, rev=False, out_dtype=None) -> "Tensor":
        o = o if isinstance(o, Tensor) else Tensor(LNode("CONST", (), o, (), _scalar_dt(o, self.dtype)))
        a, b = (o, self) if rev else (self, o)
        a, b = _broadcast(a, b)
        dt = out_dtype or _promote(a.dtype, b.dtype)
        return Tensor(LNode("ALU", (a.node, b.node), op, a.shape, dt))

    def _un(self, op: str) -> "Tensor":
        dt = self.dtype if dtypes.is_float(self.dtype) or op == "NEG" else dtypes.float32
        return Tensor(LNode("ALU", (self.node,), op, self.shape, dt))

    def add(self, o): return self._bin(o, "ADD")
    def mul(self, o): return self._bin(o, "MUL")
    def sub(self, o): return self + (-(o if isinstance(o, Tensor) else Tensor(o, dtype=_scalar_dt(o, self.dtype))))

    def div(self, o):
        if not dtypes.is_float(self.dtype) and not (isinstance(o, float) or (isinstance(o, Tensor) and dtypes.is_float(o.dtype))):
            return self._bin(o, "IDIV")
        if not isinstance(o, Tensor):
            return self * (1.0 / o)
        return self * o.reciprocal()

    def __add__(self, o): return self.add(o)
    def __radd__(self, o): return self._bin(o, "ADD", rev=True)
    def __sub__(self, o): return self.sub(o)
    def __rsub__(self, o): return (-self).add(o)
    def __mul__(self, o): return self.mul(o)
    def __rmul__(self, o): return self._bin(o, "MUL", rev=True)
    def __truediv__(self, o): return self.div(o)
    def __rtruediv__(self, o): return self.reciprocal() * o
    def __neg__(self): return self._un("NEG")
    def __lt__(self, o): return self._bin(o, "CMPLT", out_dtype=dtypes.bool)
    def __gt__(self, o): return self._bin(o, "CMPLT", rev=True, out_dtype=dtypes.bool)
    def __ge__(self, o): return (self < o).logical_not()
    def __le__(self, o): return (self > o).logical_not()
    def __matmul__(self, o): return self.matmul(o)

    def __eq__(self, o):      # elementwise, as tinygrad
        return self._bin(o, "CMPEQ", out_dtype=dtypes.bool)

    def __ne__(self, o):
        return (self == o).logical_not()

    __hash__ = object.__hash__

    def __pow__(self, e):
        if isinstance(e, int) and e >= 1:
            r = self
            for _ in range(e - 1):
                r = r * self
            return r
        return (self.log2() * e).exp2()

    def logical_not(self) -> "Tensor":
        return self._bin(True, "XOR", out_dtype=dtypes.bool)

    def cast(self, dt: DType) -> "Tensor":
        return self if dt.id == self.dtype.id else Tensor(LNode("CAST", (self.node,), None, self.shape, dt))

    def float(self): return self.cast(dtypes.float32)
    def half(self): return self.cast(dtypes.float16)
    def int(self): return self.cast(dtypes.int32)
    def bool(self): return self.cast(dtypes.bool)

    def reciprocal(self): return self._un("RECIP")
    def exp2(self): return self._un("EXP2")
    def log2(self): return self._un("LOG2")
    def sqrt(self): return self._un("SQRT")
    def sin(self): return self._un("SIN")
    def cos(self): return ((math.pi / 2) - self).sin()
    def exp(self): return (self * (1.0 / math.log(2))).exp2()
    def log(self): return self.log2() * math.log(2)
    def rsqrt(self): return self.sqrt().reciprocal()
    def sigmoid(self): return (1 + (-self).exp()).reciprocal()
    def tanh(self): return 2.0 * (2.0 * self).sigmoid() - 1.0
    def relu(self): return (self > 0).where(self, 0.0)
    def square(self): return self * self
    def abs(self): return (self < 0).where(-self, self)

    def gelu(self):
        return 0.5 * self * (1 + (math.sqrt(2 / math.pi) * (self + 0.044715 * self ** 3)).tanh())

    def where(self, x, y) -> "Tensor":
        if not isinstance(x, Tensor) and not isinstance(y, Tensor):
            like = dtypes.float32 if isinstance(x, float) or isinstance(y, float) else dtypes.int32
        else:
            like = x.dtype if isinstance(x, Tensor) else y.dtype
        x = x if isinstance(x, Tensor) else Tensor(LNode("CONST", (), x, (), _scalar_dt(x, like)))
        y = y if isinstance(y, Tensor) else Tensor(LNode("CONST", (), y, (), _scalar_dt(y, like)))
        c, x, y = _broadcast(self, x, y)
        dt = _promote(x.dtype, y.dtype)
        return Tensor(LNode("ALU", (c.node, x.node, y.node), "WHERE", c.shape, dt))

    def maximum(self, o): return (self < o).where(o, self)
    def minimum(self, o): return (self < o).where(self, o)

    # ---- reductions ----
    def _reduce(self, kind: int, axis=None, keepdim=False) -> "Tensor":
        nd = self.ndim
        axes = tuple(range(nd)) if axis is None else tuple(a % nd for a in ((axis,) if isinstance(axis, int) else axis))
        shp = tuple(1 if i in axes else s for i, s in enumerate(self.shape))
        dt = self.dtype if dtypes.is_float(self.dtype) else dtypes.int32
        src = self if self.dtype.id == dt.id else self.cast(dt)
        r = Tensor(LNode("REDUCE", (src.node,), (kind, axes), shp, dt))
        return r if keepdim else r.reshape(tuple(s for i, s in enumerate(self.shape) if i not in axes))

    def sum(self, axis=None, keepdim=False): return self._reduce(REDUCE_SUM, axis, keepdim)
    def max(self, axis=None, keepdim=False): return self._reduce(REDUCE_MAX, axis, keepdim)
    def min(self, axis=None, keepdim=False): return -((-self).max(axis, keepdim))

    def mean(self, axis=None, keepdim=False):
        nd = self.ndim
        axes = tuple(range(nd)) if axis is None else tuple(a % nd for a in ((axis,) if isinstance(axis, int) else axis))
        cnt = _prod([self.shape[a] for a in axes])
        s = self.sum(axis, keepdim)
        if isinstance(_sym(cnt), int):
            return s * (1.0 / int(cnt))
        raise NotImplementedError("mean over a symbolic extent")

    def softmax(self, axis=-1):
        m = self - self.max(axis, keepdim=True)
        e = m.exp()
        return e / e.sum(axis, keepdim=True)

    def log_softmax(self, axis=-1):
        m = self - self.max(axis, keepdim=True)
        return m - m.exp().sum(axis, keepdim=True).log()

    def argmax(self, axis=None, keepdim=False) -> "Tensor":
        if axis is None:
            return self.flatten().argmax(0)
        axis = axis % self.ndim
        n = self.shape[axis]
        m = self == self.max(axis, keepdim=True)
        rev = Tensor.arange(int(n) - 1, -1, -1).reshape(tuple(n if i == axis else 1 for i in range(self.ndim)))
        idx = m.cast(dtypes.int32) * rev
        return (int(n) - 1) - idx.max(axis, keepdim)

    # ---- movement ----
    def reshape(self, shape, *args) -> "Tensor":
        shape = tuple(shape) if isinstance(shape, (tuple, list)) else (shape,) + args
        shape = tuple(self.shape[i] if s is None else s for i, s in enumerate(shape))
        if -1 in [s if isinstance(s, int) else 0 for s in shape]:
            known = _prod([s for s in shape if not (isinstance(s, int) and s == -1)])
            shape = tuple(int(_prod(self.shape)) // int(known) if isinstance(s, int) and s == -1 else s for s in shape)
        shape = tuple(_sym(s) if not isinstance(s, int) else s for s in shape)
        if tuple(map(_key, shape)) == tuple(map(_key, self.shape)):
            return self
        return Tensor(LNode("RESHAPE", (self.node,), None, shape, self.dtype))

    def view(self, *shape): return self.reshape(*shape)

    def permute(self, order, *args) -> "Tensor":
        order = tuple(order) if isinstance(order, (tuple, list)) else (order,) + args
        order = tuple(o % self.ndim for o in order)
        if order == tuple(range(self.ndim)):
            return self
        return Tensor(LNode("PERMUTE", (self.node,), order, tuple(self.shape[o] for o in order), self.dtype))

    def transpose(self, dim0=1, dim1=0) -> "Tensor":
        order = list(range(self.ndim))
        order[dim0 % self.ndim], order[dim1 % self.ndim] = order[dim1 % self.ndim], order[dim0 % self.ndim]
        return self.permute(order)

    @property
    def T(self): return self.transpose()

    def expand(self, shape, *args) -> "Tensor":
        shape = tuple(shape) if isinstance(shape, (tuple, list)) else (shape,) + args
        shape = tuple(self.shape[i] if s is None or (isinstance(s, int) and s == -1) else s for i, s in enumerate(shape))
        if tuple(map(_key, shape)) == tuple(map(_key, self.shape)):
            return self
        return Tensor(LNode("EXPAND", (self.node,), None, shape, self.dtype))

    def shrink(self, arg) -> "Tensor":
        arg = tuple((0, s) if a is None else (a[0], a[1]) for a, s in zip(arg, self.shape))
        if all(_eq(b, 0) and _eq(e, s) for (b, e), s in zip(arg, self.shape)):
            return self
        shape = tuple(_sym(e - b) if not (isinstance(e, int) and isinstance(b, int)) else e - b for b, e in arg)
        return Tensor(LNode("SHRINK", (self.node,), arg, shape, self.dtype))

    def pad(self, arg, value: float = 0.0) -> "Tensor":
        arg = tuple((0, 0) if a is None else a for a in arg)
        if value != 0.0:
            raise NotImplementedError("pad with a non-zero value")
        shape = tuple(s + b + e for s, (b, e) in zip(self.shape, arg))
        return Tensor(LNode("PAD", (self.node,), arg, shape, self.dtype))

    def flatten(self, start_dim=0) -> "Tensor":
        start_dim %= max(self.ndim, 1)
        return self.reshape(self.shape[:start_dim] + (_prod(self.shape[start_dim:]),))

    def unsqueeze(self, dim) -> "Tensor":
        dim = dim % (self.ndim + 1)
        return self.reshape(self.shape[:dim] + (1,) + self.shape[dim:])

    def squeeze(self, dim=None) -> "Tensor":
        if dim is None:
            return self.reshape(tuple(s for s in self.shape if not _eq(s, 1)))
        dim %= self.ndim
        return self.reshape(self.shape[:dim] + self.shape[dim + 1:]) if _eq(self.shape[dim], 1) else self

    def __getitem__(self, idx) -> "Tensor":
        if not isinstance(idx, tuple):
            idx = (idx,)
        if Ellipsis in idx:
            e = idx.index(Ellipsis)
            fill = self.ndim - (len(idx) - 1 - sum(1 for i in idx if i is None))
            idx = idx[:e] + (slice(None),) * fill + idx[e + 1:]
        dims = [i for i in idx if i is not None]
        idx = idx + (slice(None),) * (self.ndim - len(dims))
        shrink, out_shape, d = [], [], 0
        for i in idx:
            if i is None:
                out_shape.append(1)
                continue
            s = self.shape[d]
            if isinstance(i, (int, np.integer)):
                i = int(i)
                i = i + int(s) if i < 0 else i
                shrink.append((i, i + 1))
            elif isinstance(i, slice):
                if i.step not in (None, 1):
                    raise NotImplementedError("strided slices")
                b = 0 if i.start is None else i.start
                e = s if i.stop is None else i.stop
                if isinstance(b, int) and b < 0:
                    b += int(s)
                if isinstance(e, int) and e < 0:
                    e += int(s)
                if isinstance(e, int) and isinstance(s, int):
                    e = min(e, s)
                shrink.append((b, e))
                out_shape.append(_sym(e - b) if not (isinstance(e, int) and isinstance(b, int)) else e - b)
            else:
                raise NotImplementedError(f"index {i!r}")
            d += 1
        return self.shrink(tuple(shrink)).reshape(tuple(out_shape))

    def __setitem__(self, idx, v):
        self[idx].assign(v).realize()

    @staticmethod
    def stack(*tensors, dim=0) -> "Tensor":
        if len(tensors) == 1 and isinstance(tensors[0], (list, tuple)):
            tensors = tuple(tensors[0])
        ts = [t.unsqueeze(dim) for t in tensors]
        return ts[0].cat(*ts[1:], dim=dim)

    def cat(self, *others, dim=0) -> "Tensor":
        ts = [self, *others]
        dim %= self.ndim
        total = sum(int(t.shape[dim]) for t in ts)
        out, off = None, 0
        for t in ts:
            n = int(t.shape[dim])
            p = t.pad(tuple((off, total - off - n) if i == dim else (0, 0) for i in range(t.ndim)))
            out = p if out is None else out + p
            off += n
        return out

    def triu(self, diagonal: int = 0) -> "Tensor":
        r, c = self.shape[-2], self.shape[-1]
        rows = Tensor.arange(int(r)).reshape(int(r), 1)
        cols = Tensor.arange(int(c)).reshape(1, int(c))
        keep = (rows + diagonal - 1) < cols
        return keep.where(self, 0.0 if dtypes.is_float(self.dtype) else 0)

    def tril(self, diagonal: int = 0) -> "Tensor":
        r, c = self.shape[-2], self.shape[-1]
        rows = Tensor.arange(int(r)).reshape(int(r), 1)
        cols = Tensor.arange(int(c)).reshape(1, int(c))
        keep = cols < (rows + diagonal + 1)
        return keep.where(self, 0.0 if dtypes.is_float(self.dtype) else 0)

    @staticmethod
    def eye(n: int, m: Optional[int] = None, dtype: Optional[DType] = None, **kw) -> "Tensor":
        m = n if m is None else m
        dt = dtype or dtypes.float32
        eq = Tensor.arange(n).reshape(n, 1) == Tensor.arange(m).reshape(1, m)
        return eq.where(Tensor.full((), 1.0 if dtypes.is_float(dt) else 1, dtype=dt),
                        Tensor.full((), 0.0 if dtypes.is_float(dt) else 0, dtype=dt))

    def split(self, sizes, dim: int = 0) -> tuple:
        """Pieces along dim: equal pieces of `sizes` (the last one shorter), or
        the listed sizes."""
        dim = dim % self.ndim
        n = int(self.shape[dim])
        if isinstance(sizes, int):
            sizes = [min(sizes, n - i) for i in range(0, n, max(sizes, 1))]
        if sum(sizes) != n:
            raise ValueError(f"split: sizes {sizes} do not add up to {n}")
        out, o = [], 0
        for sz in sizes:
            out.append(self.shrink(tuple((o, o + sz) if i == dim else None for i in range(self.ndim))))
            o += sz
        return tuple(out)

    def chunk(self, chunks: int, dim: int = 0) -> tuple:
        n = int(self.shape[dim % self.ndim])
        return self.split(math.ceil(n / chunks) if n else 1, dim)

    # ---- more elementwise (tinygrad names) ----
    def eq(self, o): return self == o
    def ne(self, o): return self != o
    def neg(self): return -self
    def recip(self): return self.reciprocal()
    def pow(self, e): return self ** e
    def sign(self):
        one = 1.0 if dtypes.is_float(self.dtype) else 1
        return (self > 0).where(one, (self < 0).where(-one, 0.0 if dtypes.is_float(self.dtype) else 0))
    def trunc(self):
        """Toward zero (|x| < 2^31)."""
        return self.cast(dtypes.int32).cast(self.dtype) if dtypes.is_float(self.dtype) else self
    def erf(self):
        """erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7 before f32 rounding)."""
        x = self.abs()
        t = 1.0 / (1.0 + 0.3275911 * x)
        y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t
                   + 0.254829592) * t * (-(x * x)).exp()
        return self.sign() * y
    def elu(self, alpha: float = 1.0): return self.relu() - alpha * (1.0 - self.exp()).relu()
    def softmin(self, axis=-1): return (-self).softmax(axis)
    def bfloat16(self): return self.cast(dtypes.bfloat16)
    def bitwise_and(self, o): return self._bin(o, "AND")
    def bitwise_or(self, o): return self._bin(o, "OR")
    def bitwise_xor(self, o): return self._bin(o, "XOR")
    def bitwise_not(self):
        return self.logical_not() if self.dtype.id == 0 else self._bin(-1 if self.dtype.id == 5 else 0xFFFFFFFF, "XOR")
    def lshift(self, n: int): return self._bin(n, "SHL")
    def rshift(self, n: int): return self._bin(n, "SHR")

    # ---- statistics ----
    def var(self, axis=None, keepdim=False, correction=1):
        nd = self.ndim
        axes = tuple(range(nd)) if axis is None else tuple(a % nd for a in ((axis,) if isinstance(axis, int) else axis))
        n = int(_prod([self.shape[a] for a in axes]))
        d = self - self.mean(axes, keepdim=True)
        return (d * d).sum(axes, keepdim) * (1.0 / max(n - correction, 0) if n - correction > 0 else math.inf)
    def std(self, axis=None, keepdim=False, correction=1): return self.var(axis, keepdim, correction).sqrt()
    def var_mean(self, axis=None, keepdim=False, correction=1):
        return self.var(axis, keepdim, correction), self.mean(axis, keepdim)
    def std_mean(self, axis=None, keepdim=False, correction=1):
        return self.std(axis, keepdim, correction), self.mean(axis, keepdim)

    # ---- like-constructors and housekeeping ----
    def zeros_like(self, **kw): return Tensor.zeros(*self.shape, dtype=kw.get("dtype", self.dtype))
    def ones_like(self, **kw): return Tensor.ones(*self.shape, dtype=kw.get("dtype", self.dtype))
    def full_like(self, v, **kw): return Tensor.full(self.shape, v, dtype=kw.get("dtype", self.dtype))
    def empty_like(self, **kw): return Tensor.empty(*self.shape, dtype=kw.get("dtype", self.dtype))
    def clone(self): return Tensor(LNode("CONTIG", (self.node,), None, self.shape, self.dtype)).realize()
    def detach(self): return self
    def to(self, device) -> "Tensor":
        Device.canonicalize(device)
        return self
    def to_(self, device) -> "Tensor":
        Device.canonicalize(device)
        return self
    def size(self, dim: Optional[int] = None):
        return self.shape if dim is None else self.shape[dim]
    def element_size(self) -> int: return self.dtype.itemsize
    def is_floating_point(self) -> bool: return dtypes.is_float(self.dtype)

    # ---- random numbers (on the device) ----
    @staticmethod
    def manual_seed(seed: int = 0) -> None:
        """Seed the device generator and restart its stream."""
        global _RNG_SEED, _RNG_CTR
        _RNG_SEED, _RNG_CTR = int(seed) & 0xFFFFFFFF, None

    @staticmethod
    def _bits(n: int) -> "Tensor":
        """n uniform 32-bit words: a counter-based hash (Wellons' lowbias32
        finaliser over index, stream counter and seed), the counter a device
        word read by the kernel and advanced by n afterwards, so a TinyJit
        replay draws new words.  Its own generator: not the reference's
        threefry stream."""
        global _RNG_CTR
        if _RNG_CTR is None:
            _RNG_CTR = Tensor(np.zeros(1, np.uint32))
        u32 = dtypes.uint32
        c = _RNG_CTR.reshape(1).expand((n,))
        i = Tensor.arange(n).cast(u32)
        x = ((i + c) * 0x9E3779B1).bitwise_xor(_RNG_SEED * 0x85EBCA77 & 0xFFFFFFFF)
        x = x.bitwise_xor(x.rshift(16)) * 0x7FEB352D
        x = x.bitwise_xor(x.rshift(15)) * 0x846CA68B
        x = x.bitwise_xor(x.rshift(16)).contiguous().realize()
        _RNG_CTR.assign(_RNG_CTR + n).realize()
        return x

    @staticmethod
    def rand(*shape, dtype: Optional[DType] = None, **kw) -> "Tensor":
        """Uniform [0, 1): the top 24 bits of each word."""
        shape = shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        n = int(_prod(shape)) if shape else 1
        u = Tensor._bits(n).rshift(8).cast(dtypes.float32) * (1.0 / (1 << 24))
        u = u.reshape(shape) if shape else u.reshape(())
        return u.cast(dtype) if dtype is not None and dtype.id != 13 else u

    def rand_like(self, **kw): return Tensor.rand(*self.shape, dtype=kw.get("dtype", self.dtype))

    @staticmethod
    def randn(*shape, dtype: Optional[DType] = None, **kw) -> "Tensor":
        """Standard normal by Box-Muller over two uniform draws."""
        shape = shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        u = Tensor.rand(2, *shape)
        u1, u2 = u[0], u[1]
        z = ((1.0 - u1).log() * -2.0).sqrt() * (u2 * (2 * math.pi)).cos()
        return z.cast(dtype) if dtype is not None and dtype.id != 13 else z

    def randn_like(self, **kw): return Tensor.randn(*self.shape, dtype=kw.get("dtype", self.dtype))

    @staticmethod
    def uniform(*shape, low=0.0, high=1.0, dtype: Optional[DType] = None, **kw) -> "Tensor":
        return Tensor.rand(*shape, dtype=dtype) * (high - low) + low

    @staticmethod
    def normal(*shape, mean=0.0, std=1.0, dtype: Optional[DType] = None, **kw) -> "Tensor":
        return Tensor.randn(*shape, dtype=dtype) * std + mean

    @staticmethod
    def randint(*shape, low=0, high=10, dtype: Optional[DType] = None, **kw) -> "Tensor":
        shape = shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        r = (Tensor.rand(*shape) * (high - low)).cast(dtypes.int32) + low
        return r.cast(dtype) if dtype is not None else r

    def multinomial(self, num_samples: int = 1, replacement: bool = False) -> "Tensor":
        """num_samples indices per row, drawn with probability proportional to
        self's weights: each draw is argmax(log w + Gumbel noise) (the
        Gumbel-max form of a categorical draw); without replacement the drawn
        entries are masked before the next draw (sequential draws of the same
        distribution as the reference's Efraimidis-Spirakis keys)."""
        assert 1 <= self.ndim <= 2 and num_samples > 0
        w = self.unsqueeze(0) if self.ndim == 1 else self
        R, N = int(w.shape[0]), int(w.shape[1])
        assert replacement or num_samples <= N, "no replacement samples must not exceed population size"
        lw = w.float().log()
        if replacement or num_samples == 1:        # independent draws, all at once
            g = -(-(Tensor.rand(num_samples, R, N).maximum(1e-30)).log()).log()
            idx = (lw.unsqueeze(0) + g).argmax(2).permute(1, 0)
            return (idx.squeeze(0) if self.ndim == 1 else idx).cast(dtypes.int32)
        cols, mask = [], None
        for _ in range(num_samples):
            g = -(-(Tensor.rand(R, N).maximum(1e-30)).log()).log()
            key = lw + g
            if mask is not None:
                key = mask.where(-math.inf, key)
            pick = key.argmax(1, keepdim=True)
            cols.append(pick)
            if not replacement:
                hit = Tensor.arange(N).reshape(1, N) == pick
                mask = hit if mask is None else (mask.cast(dtypes.int32) + hit.cast(dtypes.int32)) > 0
        idx = cols[0] if num_samples == 1 else cols[0].cat(*cols[1:], dim=1)
        return (idx.squeeze(0) if self.ndim == 1 else idx).cast(dtypes.int32)

    # ---- linear algebra ----
    def matmul(self, w: "Tensor") -> "Tensor":
        x = self
        if x.ndim == 1:
            return x.unsqueeze(0).matmul(w).squeeze(-2)
        if w.ndim == 1:
            return x.matmul(w.unsqueeze(-1)).squeeze(-1)
        if not _eq(x.shape[-1], w.shape[-2]):
            raise ValueError(f"matmul {x.shape} @ {w.shape}")
        bx, bw = x.shape[:-2], w.shape[:-2]
        nb = max(len(bx), len(bw))
        bx, bw = (1,) * (nb - len(bx)) + tuple(bx), (1,) * (nb - len(bw)) + tuple(bw)
        batch = tuple(a if not _eq(a, 1) else b for a, b in zip(bx, bw))
        dt = _promote(x.dtype, w.dtype)     # operands keep their rank: lowering broadcasts
        return Tensor(LNode("MATMUL", (x.node, w.node), None, batch + (x.shape[-2], w.shape[-1]), dt))

    def dot(self, w): return self.matmul(w)

    def linear(self, weight: "Tensor", bias: Optional["Tensor"] = None) -> "Tensor":
        out = self.matmul(weight)
        if bias is None:
            return out
        if out.node.op == "MATMUL" and bias.ndim == 1:
            n = out.node
            return Tensor(LNode("MATMUL", (*n.srcs, bias.node), None, n.shape, n.dtype))
        return out + bias

    def scaled_dot_product_attention(self, key: "Tensor", value: "Tensor", attn_mask: Optional["Tensor"] = None,
                                     is_causal: bool = False) -> "Tensor":
        qk = self.matmul(key.transpose(-2, -1)) * (1.0 / math.sqrt(int(self.shape[-1])))
        if is_causal:
            raise NotImplementedError("is_causal: pass an explicit mask")
        if attn_mask is not None:
            qk = qk + attn_mask
        return qk.softmax(-1).matmul(value)

    def layernorm(self, axis=-1, eps: float = 1e-5) -> "Tensor":
        y = self - self.mean(axis, keepdim=True)
        return y * ((y * y).mean(axis, keepdim=True) + eps).rsqrt()

    def gather_rows(self, idx: "Tensor") -> "Tensor":
        """table[idx] for a 2-D table: one row per index (Embedding)."""
        return Tensor(LNode("GATHER", (self.node, idx.node), None, tuple(idx.shape) + (self.shape[1],), self.dtype))


def _bf16_bits(f: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def _key(s):
    s = _sym(s)
    return s.key() if isinstance(s, Sym) else int(s)


def _scalar_dt(v, like: DType) -> DType:
    if isinstance(v, bool):
        return dtypes.bool
    if isinstance(v, float):
        return like if dtypes.is_float(like) else dtypes.float32
    return like if like.id != 0 else dtypes.int32


def _broadcast(*ts):
    nd = max(t.ndim for t in ts)
    ts = [t.reshape((1,) * (nd - t.ndim) + tuple(t.shape)) if t.ndim < nd else t for t in ts]
    shape = []
    for dims in zip(*[t.shape for t in ts]):
        big = [d for d in dims if not _eq(d, 1)]
        shape.append(big[0] if big else 1)
    shape = tuple(shape)
    return [t.expand(shape) for t in ts]


# --------------------------------------------------------------------------- TinyJit
class TinyJit:
    """Capture on the second call, replay afterwards (reference
    py/thvm/_misc.py:172-245 over src/jit/capture.c:644-745, 2687-2884).

    Call 1 runs the function eagerly.  Call 2 records every kernel it fires
    into a library JIT slot (replayed as one hipGraph launch).  Later calls
    copy the new input tensors into the captured input buffers, refresh the
    bound variables in the device variable buffer, and replay; the returned
    tensors alias the captured outputs."""

    def __init__(self, fxn):
        self.fxn = fxn
        self.cnt = 0
        self.jit = None
        self.in_bufs: list = []
        self.keep: list = []
        self.ret = None

    def reset(self):
        if self.jit is not None:
            self.jit.drop()
        self.jit, self.cnt, self.keep, self.ret = None, 0, [], None

    @staticmethod
    def _inputs(args, kwargs):
        return [a for a in list(args) + list(kwargs.values()) if isinstance(a, Tensor)]

    def __call__(self, *args, **kwargs):
        global _CAPTURE
        ins = self._inputs(args, kwargs)
        for t in ins:
            if not _is_contig_buf(t.node):
                t.node = t.contiguous().realize().node
            t.realize()
        global _IN_JIT
        if self.cnt == 0:
            self.cnt = 1
            _IN_JIT += 1
            try:
                return _realize_ret(self.fxn(*args, **kwargs))
            finally:
                _IN_JIT -= 1
        if self.cnt == 1:
            _KV.sync()
            _CAPTURE = []
            try:
                with _hip.Jit() as j:
                    ret = _realize_ret(self.fxn(*args, **kwargs))
            finally:
                self.keep, _CAPTURE = _CAPTURE, None
            self.jit, self.ret, self.cnt = j, ret, 2
            self.in_bufs = [(t.node.rb, t.node.rb.nbytes) for t in ins]
            self.keep.extend(t.node.rb for t in ins)
            return ret
        if len(ins) != len(self.in_bufs):
            raise RuntimeError("TinyJit: input count changed")
        for t, (rb, nb) in zip(ins, self.in_bufs):
            if t.node.rb is not rb:
                if t.node.rb.nbytes != nb:
                    raise RuntimeError("TinyJit: input shape changed")
                _hip._check(_hip.lib().thvm_hip_buf_copy(rb.id, t.node.rb.id, nb), "jit input copy")
        _KV.sync()
        self.jit.replay()
        return self.ret


def _realize_ret(r):
    if isinstance(r, Tensor):
        return r.realize()
    if isinstance(r, (tuple, list)):
        return type(r)(_realize_ret(x) for x in r)
    return r
