"""Write the golden fixtures under tests/golden/ from the compiled reference
harness (oracle/_ref/libref.so, built from /root/reference by oracle/Makefile).

Fixtures hold inputs and the reference's outputs only:
  ref_codecs.npz   every fp8 e4m3 / e5m2 / fp16 pattern decoded by the
                   reference codecs (src/dtype/fp8.c, src/dtype/fp_convert.c),
                   and a seeded f32 sweep encoded by each reference encoder
  ref_ops_f32.npz  seeded f32 inputs and the reference CPU path's outputs for
                   linear (src/nn/dot.c), softmax (src/nn/softmax.c),
                   layernorm (src/nn/layernorm.c) and the RMSNorm norm
                   (py/thvm/nn.py:219), each realized through the reference's
                   own rangeify + clang CPU JIT.
Run: python tests/golden/make_golden.py   (needs the reference tree)."""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import _oracle as O  # noqa: E402


def sweep():
    rng = np.random.default_rng(20261201)
    bits = np.arange(0, 2**32, 131071, dtype=np.uint64).astype(np.uint32)
    g = (rng.standard_normal(8000) * 10.0 ** rng.uniform(-9, 5, 8000)).astype(np.float32)
    extra = np.array([0.0, -0.0, 448.0, 464.0, 465.0, -464.0, 2**-10, 2**-9, 1.5 * 2**-9, 2**-6,
                      57344.0, 61440.0, 65504.0, 65520.0, 3.0e38, np.inf, -np.inf, 1e-40,
                      2**-24, 2**-25, 1.5 * 2**-24], np.float32)
    return np.concatenate([bits.view(np.float32), extra, g])


def main():
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libref.so not built (make -C oracle ref)")
    f = sweep()
    dec8 = np.array([R.ref_fp8e4m3_to_f32(i) for i in range(256)], np.float32)
    dec5 = np.array([R.ref_fp8e5m2_to_f32(i) for i in range(256)], np.float32)
    dec16 = np.array([R.ref_fp16_to_f32_manual(i) for i in range(65536)], np.float32)
    enc = {}
    for name, fn, dt in [("bf16", R.ref_f32_to_bf16, np.uint16),
                         ("fp16", R.ref_f32_to_fp16_manual, np.uint16),
                         ("e4m3", R.ref_f32_to_fp8e4m3, np.uint8),
                         ("e4m3_sat", R.ref_f32_to_fp8e4m3_sat, np.uint8),
                         ("e5m2", R.ref_f32_to_fp8e5m2, np.uint8),
                         ("e5m2_sat", R.ref_f32_to_fp8e5m2_sat, np.uint8)]:
        enc[name] = np.array([fn(float(v)) for v in f], dt)
    xe = np.linspace(-160, 140, 3001).astype(np.float32)
    exp2 = np.array([R.ref_xexp2f(float(v)) for v in xe], np.float32)
    np.savez_compressed(HERE / "ref_codecs.npz", dec_e4m3=dec8, dec_e5m2=dec5, dec_fp16=dec16,
                        sweep=f, xexp2_x=xe, xexp2_y=exp2,
                        **{"enc_" + k: v for k, v in enc.items()})

    rng = np.random.default_rng(7)
    out = {}
    M, N, K = 2, 300, 64
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    y = np.empty((M, N), np.float32)
    assert R.ref_linear_f32(x.ctypes.data, w.ctypes.data, y.ctypes.data, M, N, K) == 0
    out.update(lin_x=x, lin_w=w, lin_y=y)
    M, N, K = 1, 128, 768
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    y = np.empty((M, N), np.float32)
    assert R.ref_linear_f32(x.ctypes.data, w.ctypes.data, y.ctypes.data, M, N, K) == 0
    out.update(lin2_x=x, lin2_w=w, lin2_y=y)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    y = np.empty_like(x)
    assert R.ref_softmax_f32(x.ctypes.data, y.ctypes.data, 4, 4096) == 0
    out.update(sm_x=x, sm_y=y)
    x = rng.standard_normal((3, 1600)).astype(np.float32)
    y = np.empty_like(x)
    assert R.ref_layernorm_f32(x.ctypes.data, y.ctypes.data, 3, 1600, 1e-5) == 0
    out.update(ln_x=x, ln_y=y)
    x = rng.standard_normal((3, 4096)).astype(np.float32)
    y = np.empty_like(x)
    assert R.ref_rmsnorm_f32(x.ctypes.data, y.ctypes.data, 3, 4096, 1e-6) == 0
    out.update(rms_x=x, rms_y=y)
    np.savez_compressed(HERE / "ref_ops_f32.npz", **out)
    print("wrote", HERE / "ref_codecs.npz", HERE / "ref_ops_f32.npz")


if __name__ == "__main__":
    main()
