"""Lifted-DAG builders for the renderer's MFMA matmul path and fp8 stores
(rows as the reference lowers them: reference op numbers, RANGE axis ids,
the reduce split over two axes the way its scheduler splits k, e.g.
tests/golden/ref_lifted_narrow.npz linear_f16/0)."""
CONST, ADD, MUL, NEG, REDUCE, LOAD, CAST, RANGE, INDEX, IADD, IMUL = 2, 9, 10, 11, 17, 21, 23, 25, 26, 27, 29
BUFFER, STORE = 36, 37
FP8, F16, BF16, F32, I32 = 9, 11, 12, 13, 5


class Dag:
    def __init__(self):
        self.rows = []

    def add(self, op, dt, srcs=(), args=()):
        self.rows.append((op, dt, tuple(srcs), tuple(args)))
        return len(self.rows) - 1

    def c(self, v):
        return self.add(CONST, I32, (), (int(v),))


def matmul(M, N, K, dt, out_dt, b_trans=False, split=4, bias=False, cast_to=None, widen=False):
    """out[m, n] = epilogue(sum_k A[m, k] * B[k, n]) with A [M, K] row-major
    and B [K, N] row-major (or [N, K] with b_trans).  The reduce runs over two
    axes k = ko * split + ki as the reference's scheduler splits it (split=0:
    one axis).  bias: + bias[n] (slot 3) after the sum; cast_to: a CAST of the
    sum to that dtype before the epilogue; widen: operands read through a
    CAST to f32 (the form a mixed-precision graph lowers to)."""
    d = Dag()
    out = d.add(BUFFER, out_dt, (), (0, M * N))
    m = d.add(RANGE, I32, (), (0, 0, M))
    n = d.add(RANGE, I32, (), (1, 0, N))
    addr_c = d.add(IADD, I32, (d.add(IMUL, I32, (m, d.c(N))), n))
    a = d.add(BUFFER, dt, (), (1, M * K))
    if split:
        ko = d.add(RANGE, I32, (), (2, 1, K // split))
        ki = d.add(RANGE, I32, (), (3, 3, split))
        k = d.add(IADD, I32, (d.add(IMUL, I32, (ko, d.c(split))), ki))
        axes = (ko, ki)
    else:
        k = d.add(RANGE, I32, (), (2, 1, K))
        axes = (k,)
    addr_a = d.add(IADD, I32, (d.add(IMUL, I32, (m, d.c(K))), k))
    b = d.add(BUFFER, dt, (), (2, K * N))
    if b_trans:
        addr_b = d.add(IADD, I32, (d.add(IMUL, I32, (n, d.c(K))), k))
    else:
        addr_b = d.add(IADD, I32, (d.add(IMUL, I32, (k, d.c(N))), n))
    xa = d.add(INDEX, dt, (a, addr_a))
    xb = d.add(INDEX, dt, (b, addr_b))
    if widen:
        xa = d.add(CAST, F32, (xa,))
        xb = d.add(CAST, F32, (xb,))
    prod = d.add(MUL, F32 if widen else dt, (xa, xb))
    red = d.add(REDUCE, F32 if widen else dt, (prod,) + axes, (0,))
    val = red
    if cast_to is not None:
        val = d.add(CAST, cast_to, (val,))
    if bias:
        bb = d.add(BUFFER, dt, (), (3, N))
        val = d.add(ADD, dt, (val, d.add(INDEX, dt, (bb, n))))
    d.add(STORE, out_dt, (out, addr_c, val))
    return d.rows


def scale_store(n, in_dt, out_dt, scale_bits):
    """out[i] = x[i] * scale, stored in out_dt (an fp8 store when out_dt = 9)."""
    d = Dag()
    out = d.add(BUFFER, out_dt, (), (0, n))
    x = d.add(BUFFER, in_dt, (), (1, n))
    i = d.add(RANGE, I32, (), (0, 0, n))
    v = d.add(MUL, in_dt, (d.add(INDEX, in_dt, (x, i)), d.add(CONST, in_dt, (), (scale_bits,))))
    d.add(STORE, out_dt, (out, i, v))
    return d.rows
