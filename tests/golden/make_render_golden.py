"""Write the renderer's reference fixtures: every kernel the compiled
reference schedules for a set of GPT-2 step operations, captured at its CPU
dispatch by oracle/ref_harness.c (ref_capture_*): the kernel's lifted DAG as
renderer rows (op, dtype, src0..3, arg0..3; the reference's UOP_* and DT_*
numbers), its input buffers, the reference CPU output, the OPT annotations
the reference's hand opts attached and, for a symbolic extent, the bound
values of its variables.  Data only: the rows are the reference's own DAGs,
the buffers its own inputs and outputs.

  ref_lifted_kernels.npz   f32: linear, softmax, layernorm, RMSNorm, GELU,
                           causal attention, one whole GPT-2 block
  ref_lifted_narrow.npz    fp16 and bf16 (the reference's uop walker path):
                           linear, softmax, layernorm and GELU over GPT-2 XL
                           rows (1600 wide), one GPT-2 block; decode
                           attention over a cache whose length is a bound
                           variable (symbolic extents), f32 and fp16

Run in the build container (the reference tree is not on the GPU box):
    make -C oracle && python tests/golden/make_render_golden.py
"""
import ctypes as C
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "tests"))
import _oracle as O  # noqa: E402

OUT = Path(__file__).with_name("ref_lifted_kernels.npz")
OUT_NARROW = Path(__file__).with_name("ref_lifted_narrow.npz")
MAXROWS = 4096


class RefUop(C.Structure):
    _fields_ = [("op", C.c_uint32), ("dtype", C.c_uint32), ("src", C.c_int32 * 4), ("arg", C.c_int64 * 4)]


def scenarios(rng):
    M, K, N = 4, 64, 32
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32)
    H, T, hd = 2, 8, 16
    q, k, v = (rng.standard_normal((H, T, hd)).astype(np.float32) for _ in range(3))
    ym, yk = np.empty((M, N), np.float32), np.empty((M, K), np.float32)
    o = np.empty((H, T, hd), np.float32)
    # one GPT-2 block over 8 tokens (causal prefill): D 64, 2 heads, F 256
    T2, D2, H2, F2 = 8, 64, 2, 256
    xb = rng.standard_normal((T2, D2)).astype(np.float32)
    shapes = [(D2,), (D2,), (D2, D2), (D2,), (D2, D2), (D2,), (D2, D2), (D2,), (D2, D2), (D2,),
              (D2,), (D2,), (D2, F2), (F2,), (F2, D2), (D2,)]
    params = [(rng.standard_normal(sh) * (0.1 if len(sh) == 2 else 0.5) + (1.0 if i in (0, 10) else 0.0))
              .astype(np.float32) for i, sh in enumerate(shapes)]
    pp = (C.c_void_p * 16)(*[a.ctypes.data for a in params])
    ob = np.empty((T2, D2), np.float32)
    keep = [x, w, q, k, v, ym, yk, o, xb, params, pp, ob]
    L = O.ref()
    return keep, [
        ("linear", lambda: L.ref_linear_f32(x.ctypes.data, w.ctypes.data, ym.ctypes.data, M, N, K)),
        ("softmax", lambda: L.ref_softmax_f32(x.ctypes.data, yk.ctypes.data, M, K)),
        ("layernorm", lambda: L.ref_layernorm_f32(x.ctypes.data, yk.ctypes.data, M, K, 1e-5)),
        ("rmsnorm", lambda: L.ref_rmsnorm_f32(x.ctypes.data, yk.ctypes.data, M, K, 1e-6)),
        ("gelu", lambda: L.ref_gelu_f32(x.ctypes.data, yk.ctypes.data, M, K)),
        ("attention", lambda: L.ref_sdpa_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, o.ctypes.data, H, T, hd)),
        ("gpt2_block", lambda: L.ref_gpt2_block_f32(xb.ctypes.data, C.cast(pp, C.c_void_p), ob.ctypes.data,
                                                     T2, D2, H2, F2)),
    ]


def narrow_scenarios(rng):
    """fp16 / bf16 operations and symbolic-length decode attention."""
    L = O.ref()
    u32, vp = C.c_uint32, C.c_void_p
    L.ref_linear_t.argtypes = [u32, vp, vp, vp, u32, u32, u32]
    L.ref_softmax_t.argtypes = [u32, vp, vp, u32, u32]
    L.ref_layernorm_t.argtypes = [u32, vp, vp, u32, u32, C.c_double]
    L.ref_gelu_t.argtypes = [u32, vp, vp, u32, u32]
    L.ref_gpt2_block_t.argtypes = [u32, vp, vp, vp, u32, u32, u32, u32]
    L.ref_sym_attn_t.argtypes = [u32, vp, vp, vp, vp, u32, u32, u32, u32, C.c_float]
    for f in ("ref_linear_t", "ref_softmax_t", "ref_layernorm_t", "ref_gelu_t", "ref_gpt2_block_t",
              "ref_sym_attn_t"):
        getattr(L, f).restype = C.c_int
    keep, scen = [], []
    M, K, N, W = 4, 64, 32, 1600
    T2, D2, H2, F2 = 4, 64, 2, 256
    shapes = [(D2,), (D2,), (D2, D2), (D2,), (D2, D2), (D2,), (D2, D2), (D2,), (D2, D2), (D2,),
              (D2,), (D2,), (D2, F2), (F2,), (F2, D2), (D2,)]
    for dt, tag in ((11, "f16"), (12, "bf16")):
        x = rng.standard_normal((M, K)).astype(np.float32)
        w = (rng.standard_normal((N, K)) * 0.2).astype(np.float32)
        xw = (rng.standard_normal((M, W)) * 2).astype(np.float32)
        y1, y2 = np.empty((M, N), np.uint16), np.empty((M, W), np.uint16)
        params = [(rng.standard_normal(sh) * (0.1 if len(sh) == 2 else 0.5) + (1.0 if i in (0, 10) else 0.0))
                  .astype(np.float32) for i, sh in enumerate(shapes)]
        pp = (C.c_void_p * 16)(*[a.ctypes.data for a in params])
        xb, ob = rng.standard_normal((T2, D2)).astype(np.float32), np.empty((T2, D2), np.uint16)
        keep += [x, w, xw, y1, y2, params, pp, xb, ob]
        scen += [
            (f"linear_{tag}", lambda dt=dt, x=x, w=w, y1=y1: L.ref_linear_t(dt, x.ctypes.data, w.ctypes.data,
                                                                             y1.ctypes.data, M, N, K)),
            (f"softmax_{tag}", lambda dt=dt, xw=xw, y2=y2: L.ref_softmax_t(dt, xw.ctypes.data, y2.ctypes.data, M, W)),
            (f"layernorm_{tag}", lambda dt=dt, xw=xw, y2=y2: L.ref_layernorm_t(dt, xw.ctypes.data, y2.ctypes.data,
                                                                               M, W, 1e-5)),
            (f"gelu_{tag}", lambda dt=dt, xw=xw, y2=y2: L.ref_gelu_t(dt, xw.ctypes.data, y2.ctypes.data, M, W)),
            (f"gpt2_block_{tag}", lambda dt=dt, xb=xb, pp=pp, ob=ob: L.ref_gpt2_block_t(
                dt, xb.ctypes.data, C.cast(pp, C.c_void_p), ob.ctypes.data, T2, D2, H2, F2)),
        ]
    for dt, tag, hd, Lr in ((13, "f32", 16, 37), (11, "f16", 64, 100)):
        H, Lmax = 2, 128
        q = rng.standard_normal((H, hd)).astype(np.float32)
        k = rng.standard_normal((H, Lmax, hd)).astype(np.float32)
        v = rng.standard_normal((H, Lmax, hd)).astype(np.float32)
        o = np.empty((H, hd), np.float32 if dt == 13 else np.uint16)
        keep += [q, k, v, o]
        scen.append((f"sym_attention_{tag}", lambda dt=dt, q=q, k=k, v=v, o=o, H=H, Lmax=Lmax, Lr=Lr, hd=hd:
                     L.ref_sym_attn_t(dt, q.ctypes.data, k.ctypes.data, v.ctypes.data, o.ctypes.data, H, Lmax,
                                      Lr, hd, float(hd) ** -0.5)))
    return keep, scen


def capture(scen, path):
    L = O.ref()
    L.ref_capture_vars.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32]
    out, names, skipped = {}, [], []
    kid = 0
    for name, fn in scen:
        L.ref_capture_begin()
        rc = fn()
        n = L.ref_capture_end()
        if rc != 0:
            raise SystemExit(f"{name}: the reference returned {rc}")
        for k in range(n):
            rows = (RefUop * MAXROWS)()
            nn, ns, no = C.c_uint32(), C.c_uint32(), C.c_uint32()
            opts = (C.c_uint32 * 16)()
            why = C.create_string_buffer(96)
            st = L.ref_capture_kernel(k, C.cast(rows, C.c_void_p), MAXROWS, C.byref(nn), C.byref(ns),
                                      C.cast(opts, C.c_void_p), C.byref(no), why, 96)
            if st != 1:
                skipped.append(f"{name} kernel {k}: {why.value.decode()}")
                continue
            r = np.array([[u.op, u.dtype, *u.src, *u.arg] for u in rows[:nn.value]], np.int64)
            dts, numels = [], []
            for s in range(ns.value):
                dt, ne = C.c_uint32(), C.c_uint64()
                L.ref_capture_slot(k, s, C.byref(dt), C.byref(ne), None, 0)
                nb = int(ne.value) * {13: 4, 12: 2, 11: 2, 5: 4, 6: 4, 0: 1, 7: 8}[dt.value]
                b = np.empty(nb, np.uint8)
                if L.ref_capture_slot(k, s, C.byref(dt), C.byref(ne), b.ctypes.data, nb) != 0:
                    raise SystemExit(f"{name} kernel {k}: slot {s} unreadable")
                out[f"k{kid}_slot{s}"] = b
                dts.append(dt.value)
                numels.append(ne.value)
            out[f"k{kid}_rows"] = r
            out[f"k{kid}_dt"] = np.array(dts, np.uint32)
            out[f"k{kid}_numel"] = np.array(numels, np.uint64)
            out[f"k{kid}_opts"] = np.array([[opts[2 * i], opts[2 * i + 1]] for i in range(no.value)],
                                           np.uint32).reshape(-1, 2)
            vals = (C.c_uint32 * 12)()
            nv = L.ref_capture_vars(k, C.cast(vals, C.c_void_p), 4)
            if nv:
                out[f"k{kid}_vars"] = np.array(vals[:3 * nv], np.uint32).reshape(nv, 3)   # value, lo, hi
            names.append(f"{name}/{k}")
            kid += 1
    out["names"] = np.array(names)
    out["skipped"] = np.array(skipped)
    np.savez_compressed(path, **out)
    print(f"{path}: {kid} kernels ({len(skipped)} skipped: {skipped})")


def main():
    L = O.ref()
    if L is None:
        raise SystemExit("oracle/_ref/libref.so is not built (make -C oracle)")
    rng = np.random.default_rng(20261202)
    keep, scen = scenarios(rng)
    capture(scen, OUT)
    keep2, scen2 = narrow_scenarios(np.random.default_rng(20261203))
    capture(scen2, OUT_NARROW)
    del keep, keep2


if __name__ == "__main__":
    main()
