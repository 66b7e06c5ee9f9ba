"""C2, the single-op sweep, at its stated shapes: y = x.W^T for W fp16
N(0, 0.02) of [N, K] in {(4096, 4096), (14336, 4096), (50257, 768)} and x
fp16 N(0, 1) of [M, K], M in {1, 8, 64}, f32 accumulation (M = 1 runs the
GEMV, M = 8 and 64 the MFMA GEMM); row softmax and RMSNorm (eps 1e-6) over
[M, 4096] fp16 N(0, 1) inputs.

Bars: f32 outputs within 1e-5 of sum_k |x_k w_k| (the row's rounding floor)
against a float64 product and against the oracle's serial f32 or_gemv;
fp16 outputs within one fp16 rounding (2^-10 relative) of the oracle."""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu

DT_F16, DT_F32 = 11, 13


def say(*a):
    print(*a, flush=True)


def up(hip, a):
    return hip.Buffer.from_numpy(np.ascontiguousarray(a))


def f16(rng, shape, std):
    return (rng.standard_normal(shape) * std).astype(np.float16)


@pytest.mark.parametrize("M", [1, 8, 64])
@pytest.mark.parametrize("NK", [(4096, 4096), (14336, 4096), (50257, 768)])
def test_c2_gemv_gemm_fp16(hip, NK, M):
    N, K = NK
    say(f"case: C2 gemv/gemm fp16 N={N} K={K} M={M}")
    rng = np.random.default_rng(N + K + M)
    w, x = f16(rng, (N, K), 0.02), f16(rng, (M, K), 1.0)
    y = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y, up(hip, x.view(np.uint16)), up(hip, w.view(np.uint16))], m=M, n=N, k=K,
                wt=DT_F16, xt=DT_F16, yt=DT_F32, epi=0)
    got = y.read(np.float32).reshape(M, N).astype(np.float64)
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    floor = np.abs(x64) @ np.abs(w64).T
    exact = x64 @ w64.T
    assert np.all(np.abs(got - exact) <= 1e-5 * floor), np.max(np.abs(got - exact) / floor)
    if M == 1:      # the oracle's serial f32 sum (the reference CPU order) at the same bar
        ref = O.gemv(x.view(np.uint16), DT_F16, w.view(np.uint16), DT_F16, None, M=M, N=N, K=K)
        assert np.all(np.abs(got - ref) <= 1e-5 * floor)


@pytest.mark.parametrize("M", [1, 8, 64])
@pytest.mark.parametrize("yt", [DT_F16, DT_F32])
def test_c2_softmax_fp16(hip, M, yt):
    K = 4096
    say(f"case: C2 softmax fp16 [{M},{K}] -> dt {yt}")
    x = f16(np.random.default_rng(M + yt), (M, K), 1.0)
    y = hip.Buffer(M * K * (2 if yt == DT_F16 else 4))
    hip.builtin("softmax", [y, up(hip, x.view(np.uint16))], m=M, k=K, xt=DT_F16, yt=yt)
    want = np.empty(M * K, np.uint16 if yt == DT_F16 else np.float32)
    xs = np.ascontiguousarray(x.view(np.uint16))
    O.oracle().or_softmax(want.ctypes.data, yt, xs.ctypes.data, DT_F16, M, K)
    if yt == DT_F16:
        got, want = y.read(np.uint16).view(np.float16).astype(np.float64), want.view(np.float16).astype(np.float64)
        assert np.all(np.abs(got - want) <= 2.0 ** -10 * np.abs(want) + 2.0 ** -24)
    else:
        got = y.read(np.float32).astype(np.float64)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-12)
    # the definition, in float64
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    assert np.allclose(got.reshape(M, K), e / e.sum(1, keepdims=True), rtol=2.0 ** -9, atol=1e-7)


@pytest.mark.parametrize("M", [1, 8, 64])
@pytest.mark.parametrize("gain", ["ones", "random"])
def test_c2_rmsnorm_fp16(hip, M, gain):
    K, eps = 4096, 1e-6
    say(f"case: C2 rmsnorm fp16 [{M},{K}] eps {eps} gain {gain}")
    rng = np.random.default_rng(M)
    x = f16(rng, (M, K), 1.0)
    g = (np.ones(K) if gain == "ones" else 1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    y = hip.Buffer(M * K * 2)
    xs = np.ascontiguousarray(x.view(np.uint16))
    hip.builtin("norm", [y, up(hip, xs), up(hip, g)], m=M, k=K, xt=DT_F16, yt=DT_F16, eps=eps, ln=0)
    want = np.empty(M * K, np.uint16)
    O.oracle().or_rmsnorm(want.ctypes.data, DT_F16, xs.ctypes.data, DT_F16, g.ctypes.data, M, K, eps)
    got = y.read(np.uint16).view(np.float16).astype(np.float64)
    w16 = want.view(np.float16).astype(np.float64)
    assert np.all(np.abs(got - w16) <= 2.0 ** -10 * np.abs(w16) + 2.0 ** -24)
    x64 = x.astype(np.float64)
    exact = x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + eps) * g
    assert np.allclose(got.reshape(M, K), exact, rtol=2.0 ** -10, atol=2.0 ** -24)
