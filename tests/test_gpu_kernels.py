"""GPU parity of the hand-written gfx950 kernels against the CPU oracle.

Each test prints its case before touching the GPU.  Tolerances follow the
bit-exact for codecs / integer / index outputs; f32 results
within 1e-5 relative to sum|x||w| (the per-row floor); values stored in a
16-bit float within one storage rounding (2^-7 relative) plus that floor."""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu

DT_FP8, DT_F16, DT_BF16, DT_F32, DT_I32 = 9, 11, 12, 13, 5
NP_STORE = {DT_F32: np.float32, DT_F16: np.uint16, DT_BF16: np.uint16, DT_FP8: np.uint8}
SZ = {DT_F32: 4, DT_F16: 2, DT_BF16: 2, DT_FP8: 1}


def say(*a):
    print(*a, flush=True)


def up(hip, a):
    return hip.Buffer.from_numpy(np.ascontiguousarray(a))


def rand_store(rng, shape, dt, std=1.0):
    """random values of dtype dt (as storage) and their f32 value"""
    f = (rng.standard_normal(shape) * std).astype(np.float32)
    if dt == DT_F32:
        return f, f
    s = O.encode(f, dt)
    return s, O.decode(s, dt)


# ---------------------------------------------------------------- codecs ----
def test_fp8_decode_all_patterns(hip):
    say("case: fp8 e4m3 decode, all 256 patterns")
    src = up(hip, np.arange(256, dtype=np.uint8))
    dst = hip.Buffer(256 * 4)
    hip.builtin("cast", [dst, src], n=256, xt=DT_FP8, yt=DT_F32)
    got = dst.read(np.float32)
    want = O.decode(np.arange(256, dtype=np.uint8), DT_FP8)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _sweep_f32(rng):
    bits = np.arange(0, 2**32, 65521, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    extra = np.array([0.0, -0.0, 448.0, 464.0, 465.0, -464.0, 2**-10, 2**-9, 1.5 * 2**-9,
                      2**-6, 3.0e38, np.inf, -np.inf, 1e-40], np.float32)
    g = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-8, 4, 20000)).astype(np.float32)
    f = np.concatenate([f, extra, g])
    return f[~np.isnan(f)]


@pytest.mark.parametrize("dt", [DT_FP8, DT_BF16, DT_F16])
def test_encode_sweep(hip, dt):
    say(f"case: f32 -> dt {dt} store encode sweep")
    f = _sweep_f32(np.random.default_rng(1))
    src = up(hip, f)
    dst = hip.Buffer(f.size * SZ[dt])
    hip.builtin("cast", [dst, src], n=f.size, xt=DT_F32, yt=dt)
    got = dst.read(NP_STORE[dt])
    want = O.encode(f, dt)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, e.g. x={f[bad[:4]]} got={got[bad[:4]]} want={want[bad[:4]]}"


# ------------------------------------------------------------------ gemv ----
def _gemv_case(hip, rng, wdt, M, N, K, xdt=DT_BF16, ydt=DT_F32, epi=0, extra=None):
    xs, xf = rand_store(rng, (M, K), xdt)
    if wdt == DT_FP8:
        wf32 = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        scale = (np.abs(wf32).max(1) / 448.0).astype(np.float32)
        ws = O.encode(wf32 / scale[:, None], DT_FP8)
        wdq = O.decode(ws, DT_FP8) * scale[:, None]
    else:
        ws, wdq = rand_store(rng, (N, K), wdt, 0.02)
        scale = None
    ref = O.gemv(xs, xdt, ws, wdt, scale, M=M, N=N, K=K)
    floor = np.abs(xf) @ np.abs(wdq).T
    return xs, ws, scale, ref, floor


@pytest.mark.parametrize("wdt", [DT_F32, DT_F16, DT_BF16, DT_FP8])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("NK", [(64, 256), (97, 768), (256, 4096), (130, 1600)])
def test_gemv_store_f32(hip, wdt, M, NK):
    N, K = NK
    if (K * SZ[wdt]) % 16:
        pytest.skip("row bytes not a multiple of 16")
    say(f"case: gemv wdt={wdt} M={M} N={N} K={K}")
    rng = np.random.default_rng(1000 * wdt + 10 * M + N)
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, wdt, M, N, K)
    y = hip.Buffer(M * N * 4)
    args = [y, up(hip, xs), up(hip, ws)] + ([up(hip, scale)] if scale is not None else [])
    hip.builtin("gemv", args, m=M, n=N, k=K, wt=wdt, xt=DT_BF16, yt=DT_F32, epi=0)
    got = y.read(np.float32).reshape(M, N)
    err = np.abs(got - ref)
    assert np.all(err <= 1e-5 * floor + 1e-30), f"max rel {np.max(err / (floor + 1e-30))}"


def test_gemv_fp32_matches_reference_linear(hip):
    """fp32 GEMV against the reference CPU JIT's own linear output (golden)."""
    g = np.load(O.ROOT / "tests" / "golden" / "ref_ops_f32.npz")
    x, w, want = g["lin_x"], g["lin_w"], g["lin_y"]
    M, K = x.shape
    N = w.shape[0]
    say(f"case: gemv f32 vs reference linear golden M={M} N={N} K={K}")
    y = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y, up(hip, x), up(hip, w)], m=M, n=N, k=K, wt=DT_F32, xt=DT_F32,
                yt=DT_F32, epi=0)
    got = y.read(np.float32).reshape(M, N)
    floor = np.abs(x) @ np.abs(w).T
    assert np.all(np.abs(got - want) <= 1e-5 * floor)


def _rb(v):      # round through bf16 storage
    return O.decode(O.encode(np.asarray(v, np.float32), DT_BF16), DT_BF16)


def _close16(got, want, floor):
    err = np.abs(got - want)
    ok = err <= 2.0 ** -7 * np.abs(want) + 2e-5 * floor + 1e-6
    return ok


@pytest.mark.parametrize("wdt", [DT_BF16, DT_FP8])
def test_gemv_residual_epilogue(hip, wdt):
    M, N, K = 2, 256, 512
    say(f"case: gemv residual wdt={wdt}")
    rng = np.random.default_rng(7)
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, wdt, M, N, K)
    rs, rf = rand_store(rng, (M, N), DT_BF16)
    y = up(hip, rs)   # in-place residual
    args = [y, up(hip, xs), up(hip, ws)] + ([up(hip, scale)] if scale is not None else []) + [y]
    hip.builtin("gemv", args, m=M, n=N, k=K, wt=wdt, xt=DT_BF16, yt=DT_BF16, epi=1)
    got = O.decode(y.read(np.uint16), DT_BF16).reshape(M, N)
    want = _rb(rf + _rb(ref))
    assert np.all(_close16(got, want, floor + np.abs(rf)))


@pytest.mark.parametrize("wdt", [DT_BF16, DT_FP8])
def test_gemv_swiglu_epilogue(hip, wdt):
    M, F, K = 1, 384, 512
    say(f"case: gemv swiglu wdt={wdt}")
    rng = np.random.default_rng(8)
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, wdt, M, 2 * F, K)
    y = hip.Buffer(M * F * 2)
    args = [y, up(hip, xs), up(hip, ws)] + ([up(hip, scale)] if scale is not None else [])
    hip.builtin("gemv", args, m=M, n=2 * F, k=K, wt=wdt, xt=DT_BF16, yt=DT_BF16, epi=2)
    got = O.decode(y.read(np.uint16), DT_BF16).reshape(M, F)
    g, u = _rb(ref[:, 0::2]), _rb(ref[:, 1::2])
    want = _rb(g / (1 + np.exp(-g)) * u)
    fl = floor[:, 0::2] + floor[:, 1::2]
    assert np.all(_close16(got, want, fl))


def test_gemv_qkv_rope_epilogue(hip):
    H, Hkv, hd, D, ms, pos = 4, 2, 64, 256, 32, 5
    N = (H + 2 * Hkv) * hd
    say("case: gemv qkv+rope epilogue")
    rng = np.random.default_rng(9)
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, DT_FP8, 1, N, D)
    half = hd // 2
    f = 1.0 / (500000.0 ** (np.arange(half) * 2.0 / hd))
    ang = np.arange(ms)[:, None] * f[None, :]
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    q = hip.Buffer(H * hd * 2)
    kc, vc = hip.Buffer(Hkv * ms * hd * 2), hip.Buffer(Hkv * ms * hd * 2)
    L = up(hip, np.array([pos + 1], np.int32))
    hip.builtin("gemv", [q, up(hip, xs), up(hip, ws), up(hip, scale), up(hip, cs), up(hip, sn), L,
                         kc, vc], m=1, n=N, k=D, wt=DT_FP8, xt=DT_BF16, yt=DT_BF16, epi=4, h=H,
                hkv=Hkv, hd=hd, maxseq=ms)
    v = _rb(ref[0]).astype(np.float32)
    c, s = cs[pos], sn[pos]
    ro = v.copy()
    for n in range(0, (H + Hkv) * hd, 2):
        j = (n % hd) // 2
        ro[n:n + 2] = _rb(np.array([v[n] * c[j] - v[n + 1] * s[j],
                                    v[n + 1] * c[j] + v[n] * s[j]], np.float32))
    gq = O.decode(q.read(np.uint16), DT_BF16)
    gk = O.decode(kc.read(np.uint16), DT_BF16).reshape(Hkv, ms, hd)[:, pos].ravel()
    gv = O.decode(vc.read(np.uint16), DT_BF16).reshape(Hkv, ms, hd)[:, pos].ravel()
    got = np.concatenate([gq, gk, gv])
    fl = floor[0] * 2 + 1e-3
    assert np.all(_close16(got, ro, fl)), np.max(np.abs(got - ro))
    # other cache rows untouched
    assert not np.any(kc.read(np.uint16).reshape(Hkv, ms, hd)[:, pos + 1:])


@pytest.mark.parametrize("kind", [1, 2])
@pytest.mark.parametrize("wdt,xdt", [(DT_FP8, DT_BF16), (DT_F16, DT_F16), (DT_F32, DT_F32)])
def test_gemv_fused_norm(hip, kind, wdt, xdt):
    """GEMV with the RMSNorm (1) / LayerNorm (2) prologue == norm kernel
    semantics (oracle or_rmsnorm / or_layernorm, output rounded to x's dtype)
    followed by the GEMV."""
    M, N, K = 2, 192, 1600
    say(f"case: gemv fused norm kind={kind} wdt={wdt} xdt={xdt}")
    rng = np.random.default_rng(40 + kind + wdt)
    xs, xf = rand_store(rng, (M, K), xdt)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(K)).astype(np.float32)
    xn = np.empty((M, K), NP_STORE[xdt])
    if kind == 1:
        O.oracle().or_rmsnorm(xn.ctypes.data, xdt, xs.ctypes.data, xdt, g.ctypes.data, M, K, 1e-5)
    else:
        O.oracle().or_layernorm(xn.ctypes.data, xdt, xs.ctypes.data, xdt, g.ctypes.data,
                                b.ctypes.data, M, K, 1e-5)
    xnf = O.decode(xn, xdt)
    if wdt == DT_FP8:
        wf32 = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        scale = (np.abs(wf32).max(1) / 448.0).astype(np.float32)
        ws = O.encode(wf32 / scale[:, None], DT_FP8)
        wdq = O.decode(ws, DT_FP8) * scale[:, None]
    else:
        ws, wdq = rand_store(rng, (N, K), wdt, 0.02)
        scale = None
    ref = O.gemv(xn, xdt, ws, wdt, scale, M=M, N=N, K=K)
    floor = np.abs(xnf) @ np.abs(wdq).T
    y = hip.Buffer(M * N * 4)
    args = [y, up(hip, xs), up(hip, ws)] + ([up(hip, scale)] if scale is not None else [])
    args += [up(hip, g)] + ([up(hip, b)] if kind == 2 else [])
    hip.builtin("gemv", args, m=M, n=N, k=K, wt=wdt, xt=xdt, yt=DT_F32, epi=0, norm=kind, eps=1e-5)
    got = y.read(np.float32).reshape(M, N)
    # the norm's own rounding may differ by one storage ulp per element
    ulp = 1e-5 if xdt == DT_F32 else 2.0 ** -7
    assert np.all(np.abs(got - ref) <= (1e-5 + ulp) * floor + 1e-6), np.max(np.abs(got - ref) / floor)


@pytest.mark.parametrize("waves,r,u", [(1, 1, 4), (2, 2, 8), (8, 1, 8), (16, 2, 4)])
def test_gemv_tuning_knobs_agree(hip, waves, r, u):
    M, N, K = 1, 512, 4096
    say(f"case: gemv tuning waves={waves} r={r} u={u}")
    rng = np.random.default_rng(77)
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, DT_FP8, M, N, K)
    y = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y, up(hip, xs), up(hip, ws), up(hip, scale)], m=M, n=N, k=K, wt=DT_FP8,
                xt=DT_BF16, yt=DT_F32, epi=0, waves=waves, r=r, u=u, blocks=7)
    got = y.read(np.float32).reshape(M, N)
    assert np.all(np.abs(got - ref) <= 1e-5 * floor)


# ------------------------------------------------------------- MFMA GEMM ----
MFMA_TYPES = [(DT_F16, DT_F16), (DT_BF16, DT_BF16), (DT_FP8, DT_BF16), (DT_FP8, DT_F16)]


@pytest.mark.parametrize("wx", MFMA_TYPES)
@pytest.mark.parametrize("M", [1, 5, 8, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("NK", [(64, 256), (97, 768), (256, 4096), (130, 1600)])
def test_gemm_mfma_store_f32(hip, wx, M, NK):
    """The MFMA small-M GEMM (forced with path=2, the default above M=4)
    against the oracle's f32 serial dot products; N not a multiple of the
    16-row tile and M not a multiple of 16 exercise the padded edges."""
    wdt, xdt = wx
    N, K = NK
    say(f"case: gemm mfma wdt={wdt} xdt={xdt} M={M} N={N} K={K}")
    rng = np.random.default_rng(5000 + 100 * wdt + 10 * xdt + M + N)
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, wdt, M, N, K, xdt=xdt)
    y = hip.Buffer(M * N * 4)
    args = [y, up(hip, xs), up(hip, ws)] + ([up(hip, scale)] if scale is not None else [])
    hip.builtin("gemv", args, m=M, n=N, k=K, wt=wdt, xt=xdt, yt=DT_F32, epi=0, path=2)
    got = y.read(np.float32).reshape(M, N)
    err = np.abs(got - ref)
    assert np.all(err <= 1e-5 * floor + 1e-30), f"max rel {np.max(err / (floor + 1e-30))}"


@pytest.mark.parametrize("xdt", [DT_BF16, DT_F16])
def test_gemm_mfma_fp8_operand_decode_all_patterns(hip, xdt):
    """Every finite e4m3 pattern through the MFMA GEMM's operand decode:
    x rows are one-hot (row m = 1.0 at k = m), so y[m][n] is the decoded
    W[n][m] alone (times a row scale of 1.0) and must equal the table value
    exactly.  W[n][k] = (n + k) mod 256 puts each pattern at every k; the two
    NaN patterns are replaced by 0."""
    N, K, M = 256, 64, 64
    say(f"case: gemm mfma fp8 operand decode, all patterns, xdt={xdt}")
    w = ((np.arange(N)[:, None] + np.arange(K)[None, :]) % 256).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] = 0
    x = O.encode(np.eye(M, K, dtype=np.float32), xdt)
    scale = np.ones(N, np.float32)
    y = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y, up(hip, x), up(hip, w), up(hip, scale)], m=M, n=N, k=K, wt=DT_FP8,
                xt=xdt, yt=DT_F32, epi=0, path=2)
    got = y.read(np.float32).reshape(M, N)
    want = O.decode(w, DT_FP8).T[:M]            # y[m][n] = decode(W[n][m])
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} values differ"


@pytest.mark.parametrize("nt", [1, 2, 4, 7, 8])
@pytest.mark.parametrize("M", [5, 16, 64])
def test_gemm_mfma_tile_counts_agree(hip, nt, M):
    """Every tile count per block (N = 200: 13 tiles, so the last block is
    partial at every count); 7 and 8 tiles take one x tile (M <= 16) and fp8
    weights, and are refused above 16 rows."""
    N, K = 200, 2048
    say(f"case: gemm mfma nt={nt} M={M}")
    rng = np.random.default_rng(91 + M)
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, DT_FP8, M, N, K)
    y = hip.Buffer(M * N * 4)
    args = [y, up(hip, xs), up(hip, ws), up(hip, scale)]
    kw = dict(m=M, n=N, k=K, wt=DT_FP8, xt=DT_BF16, yt=DT_F32, epi=0, path=2, r=nt)
    if nt >= 7 and M > 16:
        with pytest.raises(hip.ThvmHipError, match="tiles per block"):
            hip.builtin("gemv", args, **kw)
        return
    hip.builtin("gemv", args, **kw)
    got = y.read(np.float32).reshape(M, N)
    assert np.all(np.abs(got - ref) <= 1e-5 * floor)


@pytest.mark.parametrize("N", [20000, 40000])
def test_gemm_mfma_wide_default_tiles_fused_norm(hip, N):
    """Wide N at 16 rows picks 7 (N = 20000: 1250 tiles) or 8 (40000) tiles
    per block by default, so the grid is one round of blocks per CU (or
    whole rounds); with the fused RMSNorm, against the norm kernel's
    semantics and the oracle GEMV as in the fused-norm test."""
    M, K = 16, 512
    say(f"case: gemm mfma wide default tiles N={N}")
    rng = np.random.default_rng(8100 + N)
    xs, xf = rand_store(rng, (M, K), DT_BF16, 3.0)
    g = (1 + 0.2 * rng.standard_normal(K)).astype(np.float32)
    xn = np.empty((M, K), np.uint16)
    O.oracle().or_rmsnorm(xn.ctypes.data, DT_BF16, xs.ctypes.data, DT_BF16, g.ctypes.data, M, K, 1e-5)
    xnf = O.decode(xn, DT_BF16)
    wf32 = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    scale = (np.abs(wf32).max(1) / 448.0).astype(np.float32)
    ws = O.encode(wf32 / scale[:, None], DT_FP8)
    wdq = O.decode(ws, DT_FP8) * scale[:, None]
    ref = O.gemv(xn, DT_BF16, ws, DT_FP8, scale, M=M, N=N, K=K)
    floor = np.abs(xnf) @ np.abs(wdq).T
    y = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y, up(hip, xs), up(hip, ws), up(hip, scale), up(hip, g)], m=M, n=N, k=K,
                wt=DT_FP8, xt=DT_BF16, yt=DT_F32, epi=0, norm=1, eps=1e-5)
    got = y.read(np.float32).reshape(M, N)
    err = np.abs(got - ref)
    assert np.all(err <= (1e-5 + 2.0 ** -7) * floor + 1e-6), np.max(err / floor)
    # and the same bits as an explicit 4 tiles per block
    y4 = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y4, up(hip, xs), up(hip, ws), up(hip, scale), up(hip, g)], m=M, n=N, k=K,
                wt=DT_FP8, xt=DT_BF16, yt=DT_F32, epi=0, norm=1, eps=1e-5, r=4)
    assert np.array_equal(y4.read(np.uint32), y.read(np.uint32))


@pytest.mark.parametrize("M", [5, 16, 40])
def test_gemm_mfma_epilogues(hip, M):
    """Residual (in place), SwiGLU, GELU+bias and q/k RoPE + KV append through
    the MFMA path, each against the oracle GEMV output finished on the host
    with the same rounding points."""
    say(f"case: gemm mfma epilogues M={M}")
    rng = np.random.default_rng(300 + M)
    N, K = 256, 512
    # residual, bf16 weights
    xs, ws, _, ref, floor = _gemv_case(hip, rng, DT_BF16, M, N, K)
    rs, rf = rand_store(rng, (M, N), DT_BF16)
    y = up(hip, rs)
    hip.builtin("gemv", [y, up(hip, xs), up(hip, ws), y], m=M, n=N, k=K, wt=DT_BF16,
                xt=DT_BF16, yt=DT_BF16, epi=1)
    got = O.decode(y.read(np.uint16), DT_BF16).reshape(M, N)
    assert np.all(_close16(got, _rb(rf + _rb(ref)), floor + np.abs(rf)))
    # swiglu, fp8 weights
    F = 192
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, DT_FP8, M, 2 * F, K)
    y = hip.Buffer(M * F * 2)
    hip.builtin("gemv", [y, up(hip, xs), up(hip, ws), up(hip, scale)], m=M, n=2 * F, k=K,
                wt=DT_FP8, xt=DT_BF16, yt=DT_BF16, epi=2)
    got = O.decode(y.read(np.uint16), DT_BF16).reshape(M, F)
    g, u = _rb(ref[:, 0::2]), _rb(ref[:, 1::2])
    assert np.all(_close16(got, _rb(g / (1 + np.exp(-g)) * u), floor[:, 0::2] + floor[:, 1::2]))
    # gelu + bias, fp16
    xs, ws, _, ref, floor = _gemv_case(hip, rng, DT_F16, M, N, K, xdt=DT_F16)
    bs, bf = rand_store(rng, (N,), DT_F16, 0.1)
    y = hip.Buffer(M * N * 2)
    hip.builtin("gemv", [y, up(hip, xs), up(hip, ws), up(hip, bs)], m=M, n=N, k=K, wt=DT_F16,
                xt=DT_F16, yt=DT_F16, epi=3, bias=1)
    got = O.decode(y.read(np.uint16), DT_F16).reshape(M, N)
    v = O.decode(O.encode((ref + bf[None, :]).astype(np.float32), DT_F16), DT_F16)
    want = 0.5 * v * (1 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3)))
    assert np.all(np.abs(got - want) <= 2.0 ** -10 * np.abs(want) + 2e-5 * floor + 1e-4)
    # q/k rope + kv append, fp8
    H, Hkv, hd, ms, pos = 4, 2, 64, 32, 9
    Nq = (H + 2 * Hkv) * hd
    xs, ws, scale, ref, floor = _gemv_case(hip, rng, DT_FP8, M, Nq, K)
    half = hd // 2
    f = 1.0 / (500000.0 ** (np.arange(half) * 2.0 / hd))
    ang = np.arange(ms)[:, None] * f[None, :]
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    q = hip.Buffer(M * H * hd * 2)
    kc, vc = hip.Buffer(M * Hkv * ms * hd * 2), hip.Buffer(M * Hkv * ms * hd * 2)
    L = up(hip, np.array([pos + 1], np.int32))
    hip.builtin("gemv", [q, up(hip, xs), up(hip, ws), up(hip, scale), up(hip, cs), up(hip, sn), L,
                         kc, vc], m=M, n=Nq, k=K, wt=DT_FP8, xt=DT_BF16, yt=DT_BF16, epi=4, h=H,
                hkv=Hkv, hd=hd, maxseq=ms)
    v = _rb(ref)
    c, s = cs[pos], sn[pos]
    ro = v.copy()
    nr = (H + Hkv) * hd
    j = (np.arange(0, nr, 2) % hd) // 2
    ro[:, 0:nr:2] = _rb(v[:, 0:nr:2] * c[j] - v[:, 1:nr:2] * s[j])
    ro[:, 1:nr:2] = _rb(v[:, 1:nr:2] * c[j] + v[:, 0:nr:2] * s[j])
    gq = O.decode(q.read(np.uint16), DT_BF16).reshape(M, H * hd)
    gk = O.decode(kc.read(np.uint16), DT_BF16).reshape(M, Hkv, ms, hd)[:, :, pos].reshape(M, -1)
    gv = O.decode(vc.read(np.uint16), DT_BF16).reshape(M, Hkv, ms, hd)[:, :, pos].reshape(M, -1)
    got = np.concatenate([gq, gk, gv], 1)
    assert np.all(_close16(got, ro, floor * 2 + 1e-3)), np.max(np.abs(got - ro))
    assert not np.any(kc.read(np.uint16).reshape(M, Hkv, ms, hd)[:, :, pos + 1:])


@pytest.mark.parametrize("wdt", [DT_FP8, DT_BF16])
@pytest.mark.parametrize("M", [5, 16, 17, 33, 64])
@pytest.mark.parametrize("NK", [(97, 768), (130, 1600), (256, 4096)])
def test_gemm_mfma_fused_rmsnorm(hip, wdt, M, NK):
    """RMSNorm fused into the MFMA GEMM (bf16 x, the default above 4 rows)
    against the norm kernel's semantics (oracle or_rmsnorm, rounded to bf16)
    followed by the oracle GEMV.  The GEMM rounds x*g and scales the row sums
    by 1/rms, so each product's one bf16 rounding sits elsewhere: within two
    storage half-ulps per element, 2^-7 of the row's absolute sum.  K = 1600
    (25 steps of 64 over 8 waves) gives uneven k slices, whose staging runs
    past each slice's end."""
    N, K = NK
    say(f"case: gemm mfma fused rmsnorm wdt={wdt} M={M} N={N} K={K}")
    rng = np.random.default_rng(7000 + 10 * wdt + M + K)
    xs, xf = rand_store(rng, (M, K), DT_BF16, 3.0)
    g = (1 + 0.2 * rng.standard_normal(K)).astype(np.float32)
    xn = np.empty((M, K), np.uint16)
    O.oracle().or_rmsnorm(xn.ctypes.data, DT_BF16, xs.ctypes.data, DT_BF16, g.ctypes.data, M, K, 1e-5)
    xnf = O.decode(xn, DT_BF16)
    if wdt == DT_FP8:
        wf32 = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        scale = (np.abs(wf32).max(1) / 448.0).astype(np.float32)
        ws = O.encode(wf32 / scale[:, None], DT_FP8)
        wdq = O.decode(ws, DT_FP8) * scale[:, None]
    else:
        ws, wdq = rand_store(rng, (N, K), wdt, 0.02)
        scale = None
    ref = O.gemv(xn, DT_BF16, ws, wdt, scale, M=M, N=N, K=K)
    floor = np.abs(xnf) @ np.abs(wdq).T
    y = hip.Buffer(M * N * 4)
    args = [y, up(hip, xs), up(hip, ws)] + ([up(hip, scale)] if scale is not None else []) + [up(hip, g)]
    hip.builtin("gemv", args, m=M, n=N, k=K, wt=wdt, xt=DT_BF16, yt=DT_F32, epi=0, norm=1, eps=1e-5, path=2)
    got = y.read(np.float32).reshape(M, N)
    err = np.abs(got - ref)
    assert np.all(err <= (1e-5 + 2.0 ** -7) * floor + 1e-6), np.max(err / floor)
    # and well inside that on the whole: the roundings do not pile up one way
    assert np.sum(err) <= 2.0 ** -9 * np.sum(floor)


def test_gemm_mfma_fused_norm_limits(hip):
    """The MFMA path fuses RMSNorm over bf16 x only: LayerNorm, fp16 x or a
    missing gain are refused when path=2 forces it; by default such a batch
    runs the GEMV in chunks of 4 rows with its own fused norm."""
    M, N, K = 8, 64, 256
    say("case: gemm mfma fused norm limits")
    rng = np.random.default_rng(8)
    xs, _ = rand_store(rng, (M, K), DT_F16)
    ws, _ = rand_store(rng, (N, K), DT_F16, 0.02)
    g = np.ones(K, np.float32)
    y = hip.Buffer(M * N * 4)
    with pytest.raises(hip.ThvmHipError, match="RMSNorm"):
        hip.builtin("gemv", [y, up(hip, xs), up(hip, ws), up(hip, g)], m=M, n=N, k=K, wt=DT_F16,
                    xt=DT_F16, yt=DT_F32, epi=0, norm=1, eps=1e-5, path=2)
    hip.builtin("gemv", [y, up(hip, xs), up(hip, ws), up(hip, g)], m=M, n=N, k=K, wt=DT_F16,
                xt=DT_F16, yt=DT_F32, epi=0, norm=1, eps=1e-5)
    assert np.isfinite(y.read(np.float32)).all()


def _tile_ref(w: np.ndarray, lb: int) -> np.ndarray:
    """The MFMA tile layout written from its definition (kern_api.h,
    thvm_k_tile_w) for lanes reading lb bytes per step (a step is 4 lb bytes
    of a row): for 16-row group g and step s, lb/16 pieces jj of 64 lanes x
    16 bytes; lane l holds row 16 g + l % 16, bytes s*4lb + (l // 16)*lb +
    jj*16; rows past N are zero."""
    N, RB = w.shape
    npad = (N + 15) // 16 * 16
    wp = np.zeros((npad, RB), np.uint8)
    wp[:N] = w
    out = np.empty(npad * RB, np.uint8)
    o = 0
    for g in range(npad // 16):
        for s in range(RB // (4 * lb)):
            for jj in range(lb // 16):
                for l in range(64):
                    b0 = s * 4 * lb + (l // 16) * lb + jj * 16
                    out[o:o + 16] = wp[g * 16 + l % 16, b0:b0 + 16]
                    o += 16
    return out


@pytest.mark.parametrize("wdt", [DT_FP8, DT_BF16])
@pytest.mark.parametrize("lb", [0, 16, 32])
@pytest.mark.parametrize("N", [40, 97])
def test_tile_w_layout(hip, wdt, lb, N):
    """tile_w writes the layout's definition byte for byte (a padded last
    row group included); lb 0 is the GEMM's 16 bytes per element byte."""
    es = 1 if wdt == DT_FP8 else 2
    K = 256
    say(f"case: tile_w layout wdt={wdt} lb={lb} N={N}")
    rng = np.random.default_rng(17 + N + wdt + lb)
    w = rng.integers(0, 256, (N, K * es), dtype=np.uint8)
    npad = (N + 15) // 16 * 16
    t = hip.Buffer(npad * K * es)
    hip.builtin("tile_w", [t, up(hip, w)], n=N, k=K, wt=wdt, lb=lb)
    assert np.array_equal(t.read(np.uint8), _tile_ref(w, lb or 16 * es))


@pytest.mark.parametrize("wx", MFMA_TYPES)
@pytest.mark.parametrize("M", [8, 16, 40, 64])
@pytest.mark.parametrize("NK", [(97, 768), (1000, 512), (256, 4096)])
def test_gemm_mfma_tiled_weights_bit_equal(hip, wx, M, NK):
    """The MFMA GEMM over tiled weights (tiled=1) gives the row-major
    launch's bits: the same bytes reach the same lanes, only the addresses
    change.  Store and residual epilogues, every tile count."""
    wdt, xdt = wx
    N, K = NK
    es = 1 if wdt == DT_FP8 else 2
    say(f"case: gemm tiled wdt={wdt} xdt={xdt} M={M} N={N} K={K}")
    rng = np.random.default_rng(7000 + 100 * wdt + M + N)
    xs, ws, scale, _, _ = _gemv_case(hip, rng, wdt, M, N, K, xdt=xdt)
    wb = up(hip, ws)
    tw = hip.Buffer((N + 15) // 16 * 16 * K * es)
    hip.builtin("tile_w", [tw, wb], n=N, k=K, wt=wdt)
    xb = up(hip, xs)
    sc = [up(hip, scale)] if scale is not None else []
    for r in (1, 2, 4) + ((7, 8) if wdt == DT_FP8 and M <= 16 else ()):
        y0, y1 = hip.Buffer(M * N * 4), hip.Buffer(M * N * 4)
        hip.builtin("gemv", [y0, xb, wb] + sc, m=M, n=N, k=K, wt=wdt, xt=xdt, yt=DT_F32, epi=0, path=2, r=r)
        hip.builtin("gemv", [y1, xb, tw] + sc, m=M, n=N, k=K, wt=wdt, xt=xdt, yt=DT_F32, epi=0, path=2, r=r,
                    tiled=1)
        assert np.array_equal(y0.read(np.uint32), y1.read(np.uint32)), f"r={r}"
    rs, _ = rand_store(rng, (M, N), xdt)
    y0, y1 = up(hip, rs), up(hip, rs)
    hip.builtin("gemv", [y0, xb, wb] + sc + [y0], m=M, n=N, k=K, wt=wdt, xt=xdt, yt=xdt, epi=1)
    hip.builtin("gemv", [y1, xb, tw] + sc + [y1], m=M, n=N, k=K, wt=wdt, xt=xdt, yt=xdt, epi=1, tiled=1)
    assert np.array_equal(y0.read(np.uint16), y1.read(np.uint16))


def test_gemv_refuses_tiled_weights(hip):
    """Tiled weights exist for the MFMA path only: the GEMV (M <= 4) refuses
    them instead of reading the wrong bytes."""
    N, K = 64, 256
    w = np.zeros((N, K), np.uint16)
    with pytest.raises(hip.ThvmHipError):
        hip.builtin("gemv", [hip.Buffer(N * 4), up(hip, np.zeros(K, np.uint16)), up(hip, w)], m=1, n=N, k=K,
                    wt=DT_BF16, xt=DT_BF16, yt=DT_F32, epi=0, tiled=1)


@pytest.mark.parametrize("NK", [(4096, 4096), (14336, 4096), (50257, 768)])
@pytest.mark.parametrize("M", [8, 64])
def test_gemm_mfma_c2_shapes(hip, NK, M):
    """The single-op sweep's fp16 GEMM shapes at full size (W N(0,0.02), x
    N(0,1)), against a float64 product; the f32-accumulation bar is 1e-5 of
    sum|x||w| per output."""
    N, K = NK
    say(f"case: gemm c2 fp16 M={M} N={N} K={K}")
    rng = np.random.default_rng(N + M)
    xs = O.encode(rng.standard_normal((M, K)).astype(np.float32), DT_F16)
    ws = O.encode((rng.standard_normal((N, K)) * 0.02).astype(np.float32), DT_F16)
    xf, wf = O.decode(xs, DT_F16).astype(np.float64), O.decode(ws, DT_F16).astype(np.float64)
    want = xf @ wf.T
    floor = np.abs(xf) @ np.abs(wf).T
    y = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y, up(hip, xs), up(hip, ws)], m=M, n=N, k=K, wt=DT_F16, xt=DT_F16,
                yt=DT_F32, epi=0)
    got = y.read(np.float32).reshape(M, N).astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-5 * floor)


def test_gemv_rejects_bad_shapes(hip):
    say("case: gemv argument validation (host-side errors, no launch)")
    y, x, w = hip.Buffer(64), hip.Buffer(64), hip.Buffer(64)
    with pytest.raises(hip.ThvmHipError):
        hip.builtin("gemv", [y, x, w], m=1, n=64, k=256, wt=DT_F32, xt=DT_F32, yt=DT_F32)
    with pytest.raises(hip.ThvmHipError):
        hip.builtin("gemv", [y, x, w], m=9, n=1, k=4, wt=DT_F32, xt=DT_F32, yt=DT_F32)


# ------------------------------------------------------------- row ops ----
@pytest.mark.parametrize("ln", [0, 1])
@pytest.mark.parametrize("dt", [DT_F32, DT_BF16, DT_F16])
def test_norm(hip, ln, dt):
    M, K = 3, 1600
    say(f"case: norm ln={ln} dt={dt}")
    rng = np.random.default_rng(11)
    xs, xf = rand_store(rng, (M, K), dt)
    g = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(K)).astype(np.float32)
    y = hip.Buffer(M * K * SZ[dt])
    args = [y, up(hip, xs), up(hip, g)] + ([up(hip, b)] if ln else [])
    hip.builtin("norm", args, m=M, k=K, xt=dt, yt=dt, eps=1e-5, ln=ln, bias=ln)
    want = np.empty(M * K, NP_STORE[dt])
    if ln:
        O.oracle().or_layernorm(want.ctypes.data, dt, xs.ctypes.data, dt, g.ctypes.data,
                                b.ctypes.data, M, K, 1e-5)
    else:
        O.oracle().or_rmsnorm(want.ctypes.data, dt, xs.ctypes.data, dt, g.ctypes.data, M, K, 1e-5)
    gw = O.decode(y.read(NP_STORE[dt]), dt)
    ww = O.decode(want, dt)
    tol = 1e-5 if dt == DT_F32 else 2.0 ** -7
    assert np.all(np.abs(gw - ww) <= tol * np.abs(ww) + 1e-5), np.max(np.abs(gw - ww))


@pytest.mark.parametrize("K,xt", [(4096, DT_F16), (1000, DT_BF16), (257, DT_F32), (1, DT_F16),
                                  (5000, DT_F16)])
def test_softmax(hip, K, xt):
    """Rows up to 4096 run the register-resident typed kernel, longer rows
    the looping one (K = 5000); ragged K leaves the last threads' slots
    masked."""
    M = 4
    say(f"case: softmax dt {xt} [{M},{K}]")
    rng = np.random.default_rng(12 + K)
    xs, xf = rand_store(rng, (M, K), xt)
    y = hip.Buffer(M * K * 4)
    hip.builtin("softmax", [y, up(hip, xs)], m=M, k=K, xt=xt, yt=DT_F32)
    want = np.empty(M * K, np.float32)
    O.oracle().or_softmax(want.ctypes.data, DT_F32, np.ascontiguousarray(xs).ctypes.data, xt, M, K)
    got = y.read(np.float32)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-9)
    assert np.allclose(got.reshape(M, K).sum(1), 1.0, atol=1e-5)


def test_rope(hip):
    B, nh, hd, ms, pos = 2, 3, 128, 16, 9
    say("case: rope")
    rng = np.random.default_rng(13)
    xs, xf = rand_store(rng, (B, nh, hd), DT_BF16)
    half = hd // 2
    ang = np.arange(ms)[:, None] / (500000.0 ** (np.arange(half) * 2.0 / hd))[None]
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    xb = up(hip, xs)
    hip.builtin("rope", [xb, up(hip, cs), up(hip, sn), up(hip, np.array([pos + 1], np.int32))],
                b=B, nh=nh, hd=hd, dt=DT_BF16, maxseq=ms)
    want = xs.copy()
    O.oracle().or_rope(want.ctypes.data, DT_BF16, cs.ctypes.data, sn.ctypes.data, B, nh, hd, pos)
    assert np.array_equal(xb.read(np.uint16), want.ravel())


@pytest.mark.parametrize("cdt", [DT_BF16, DT_F32])
@pytest.mark.parametrize("H,Hkv,hd", [(8, 2, 128), (4, 4, 64), (32, 8, 128), (8, 1, 64)])
@pytest.mark.parametrize("L", [1, 63, 64, 65, 200])
def test_attention_decode(hip, H, Hkv, hd, L, cdt):
    B, ms = 2, 256
    say(f"case: attn H={H} Hkv={Hkv} hd={hd} L={L} cache dt={cdt}")
    rng = np.random.default_rng(H * 1000 + L)
    qs, qf = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    nsplit = (ms + 63) // 64
    out = hip.Buffer(B * H * hd * SZ[cdt])
    part = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    hip.builtin("attn", [out, up(hip, qs), up(hip, ks), up(hip, vs),
                         up(hip, np.array([L], np.int32)), part],
                b=B, h=H, hkv=Hkv, hd=hd, maxseq=ms, chunk=64, nsplit=nsplit, qt=cdt,
                ct=cdt, ot=cdt, scale=scale, mf=2)
    want = np.empty(B * H * hd, NP_STORE[cdt])
    O.oracle().or_attn_decode(want.ctypes.data, cdt, qs.ctypes.data, cdt, ks.ctypes.data,
                              vs.ctypes.data, cdt, B, H, Hkv, hd, ms, L, scale)
    got = O.decode(out.read(NP_STORE[cdt]), cdt)
    ww = O.decode(want, cdt)
    if cdt == DT_F32:   # f32: 1e-5 relative to the magnitude of the V rows mixed
        assert np.all(np.abs(got - ww) <= 1e-5 * (np.abs(ww) + 1.0)), np.max(np.abs(got - ww))
    else:
        assert np.all(np.abs(got - ww) <= 2.0 ** -7 * np.abs(ww) + 2e-3), np.max(np.abs(got - ww))
    # the one-launch form (split + last-unit merge) equals the two-kernel form
    # of one chunk per block bit for bit, and leaves its merge counters zero
    # for the next launch
    out = hip.Buffer(B * H * hd * SZ[cdt])
    hip.builtin("attn", [out, up(hip, qs), up(hip, ks), up(hip, vs),
                         up(hip, np.array([L], np.int32)), part],
                b=B, h=H, hkv=Hkv, hd=hd, maxseq=ms, chunk=64, nsplit=nsplit, qt=cdt,
                ct=cdt, ot=cdt, scale=scale, cpb=1, mf=2)
    assert attn_close(O.decode(out.read(NP_STORE[cdt]), cdt), ww, cdt)
    out2 = hip.Buffer(B * H * hd * SZ[cdt])
    part2 = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    hip.builtin("attn", [out2, up(hip, qs), up(hip, ks), up(hip, vs),
                         up(hip, np.array([L], np.int32)), part2],
                b=B, h=H, hkv=Hkv, hd=hd, maxseq=ms, chunk=64, nsplit=nsplit, qt=cdt,
                ct=cdt, ot=cdt, scale=scale, fused=1)
    assert np.array_equal(out.read(np.uint8), out2.read(np.uint8))
    ctr = part2.read(np.uint32)[B * H * nsplit * (hd + 2):]
    assert not ctr.any(), ctr


def run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, part=None, **kw):
    nsplit = (ms + 63) // 64
    out = hip.Buffer(B * H * hd * SZ[cdt])
    if part is None:
        part = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    hip.builtin("attn", [out, up(hip, qs), up(hip, ks), up(hip, vs),
                         up(hip, np.array([L], np.int32)), part],
                b=B, h=H, hkv=Hkv, hd=hd, maxseq=ms, chunk=64, nsplit=nsplit, qt=cdt,
                ct=cdt, ot=cdt, scale=scale, **kw)
    want = np.empty(B * H * hd, NP_STORE[cdt])
    O.oracle().or_attn_decode(want.ctypes.data, cdt, qs.ctypes.data, cdt, ks.ctypes.data,
                              vs.ctypes.data, cdt, B, H, Hkv, hd, ms, L, scale)
    return O.decode(out.read(NP_STORE[cdt]), cdt), O.decode(want, cdt)


def attn_close(got, ww, cdt):
    if cdt == DT_F32:   # f32: 1e-5 relative to the magnitude of the V rows mixed
        return np.all(np.abs(got - ww) <= 1e-5 * (np.abs(ww) + 1.0))
    return np.all(np.abs(got - ww) <= 2.0 ** -7 * np.abs(ww) + 2e-3)


@pytest.mark.parametrize("cdt", [DT_BF16, DT_F32])
@pytest.mark.parametrize("H,Hkv,hd", [(32, 8, 128), (4, 4, 64), (8, 2, 128)])
@pytest.mark.parametrize("L", [1, 63, 64, 65, 129, 200, 256])
@pytest.mark.parametrize("cpb", [2, 3, 4, 9])
def test_attention_multi_chunk(hip, H, Hkv, hd, L, cdt, cpb):
    """Blocks of several consecutive chunks (online softmax per row group, one
    partial per block; 9 is clamped to the 4 splits there are) against the
    oracle, at the one-chunk form's bars; lengths inside, at and past chunk
    and block edges."""
    B, ms = 3, 256
    say(f"case: attn multi-chunk cpb={cpb} H={H} Hkv={Hkv} hd={hd} L={L} dt={cdt}")
    rng = np.random.default_rng(H * 1000 + L + 7 * cpb)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    got, ww = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, cpb=cpb, mf=2)
    assert attn_close(got, ww, cdt), np.max(np.abs(got - ww))


@pytest.mark.parametrize("mf", [0, 2])
def test_attention_multi_chunk_auto_repeated(hip, mf):
    """The batched C4 head shape at 12 rows with the chunks per block picked
    by the kernel (mf=0: the MFMA split it picks; mf=2: the VALU split, 4
    chunks per block); one partial buffer across launches at changing
    lengths (stale partials of a longer launch are never read)."""
    B, H, Hkv, hd, ms, cdt = 12, 32, 8, 128, 2176, DT_BF16
    say(f"case: attn multi-chunk auto, 12 rows, 5 launches, mf={mf}")
    rng = np.random.default_rng(9)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    nsplit = (ms + 63) // 64
    part = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    for L in (2100, 700, 2176, 1, 257):
        got, ww = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, part=part, mf=mf)
        assert attn_close(got, ww, cdt), (L, np.max(np.abs(got - ww)))


@pytest.mark.parametrize("mf", [0, 2])
@pytest.mark.parametrize("L,ms", [(20000, 20480), (131000, 131072)])
def test_attention_long_context(hip, L, ms, mf):
    """Caches far past 8192 rows (up to the 131072-row limit): the automatic
    chunks per block and a merge of tens of partials per (row, kv head),
    against the oracle; the split picked by the kernel (MFMA) and the VALU
    split."""
    B, H, Hkv, hd, cdt = 1, 8, 2, 64, DT_BF16
    say(f"case: attn long context L={L} max_seq={ms} mf={mf}")
    rng = np.random.default_rng(L)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    got, ww = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, mf=mf)
    assert attn_close(got, ww, cdt), np.max(np.abs(got - ww))


@pytest.mark.parametrize("cdt", [DT_BF16, DT_F16])
@pytest.mark.parametrize("H,Hkv,hd", [(32, 8, 128), (8, 8, 64), (16, 2, 64), (8, 4, 128)])
@pytest.mark.parametrize("L", [1, 15, 16, 17, 63, 65, 200, 256])
@pytest.mark.parametrize("cpb", [0, 1, 3])
def test_attention_mfma_split(hip, H, Hkv, hd, L, cdt, cpb):
    """The split on MFMA (mf=1: scores and the weighted sum as 16x16 MFMA
    tiles, a wave per 16 cache rows) against the oracle at the 16-bit bars,
    and against the VALU split (mf=2) within one output ulp: lengths inside
    and at the edges of a 16-row tile, a 64-row chunk and a block of cpb
    chunks; G = 1, 2, 4, 8; head dims 64 and 128."""
    B, ms = 3, 256
    say(f"case: attn mfma H={H} Hkv={Hkv} hd={hd} L={L} dt={cdt} cpb={cpb}")
    rng = np.random.default_rng(H * 1000 + L + 13 * cpb + cdt)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    got, ww = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, cpb=cpb, mf=1)
    assert attn_close(got, ww, cdt), np.max(np.abs(got - ww))
    if H // Hkv == 8 and cpb > 1:
        return                                   # the VALU split runs 8 heads one chunk per block
    valu, _ = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, cpb=cpb, mf=2)
    # the two roundings of nearly equal sums to the output type: one ulp,
    # at most 2^-7 (bf16) or 2^-10 (fp16) of the value
    ulp = 2.0 ** (-7 if cdt == DT_BF16 else -10)
    assert np.all(np.abs(got - valu) <= ulp * np.abs(valu) + 1e-4), np.max(np.abs(got - valu))


@pytest.mark.parametrize("H,Hkv,hd", [(32, 8, 128), (16, 2, 64)])
@pytest.mark.parametrize("B,L", [(8, 17), (9, 200)])
def test_attention_mfma_split_batched(hip, H, Hkv, hd, B, L):
    """At 8 rows and more the MFMA path merges one block per (row, query
    head) instead of per kv-head group: the same bars against the oracle and
    the VALU split."""
    ms, cdt = 256, DT_BF16
    say(f"case: attn mfma batched B={B} H={H} Hkv={Hkv} hd={hd} L={L}")
    rng = np.random.default_rng(B * 7 + H + L)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    got, ww = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, mf=1)
    assert attn_close(got, ww, cdt), np.max(np.abs(got - ww))
    valu, _ = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, mf=2)
    assert np.all(np.abs(got - valu) <= 2.0 ** -7 * np.abs(valu) + 1e-4), np.max(np.abs(got - valu))


@pytest.mark.parametrize("mf", [1, 2])
def test_attention_stale_rows_are_never_mixed(hip, mf):
    """Cache rows at and past L hold NaN (a stale or never-written row):
    neither split reads them into a product (zero weight times NaN would
    still be NaN), at lengths inside a tile and a chunk."""
    B, H, Hkv, hd, ms, cdt = 2, 32, 8, 128, 256, DT_BF16
    rng = np.random.default_rng(77 + mf)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    for L in (5, 70, 130):
        say(f"case: attn stale NaN rows mf={mf} L={L}")
        k2, v2 = ks.copy(), vs.copy()
        k2[:, :, L:, :] = 0x7FC0
        v2[:, :, L:, :] = 0x7FC0
        got, ww = run_attn(hip, qs, k2, v2, B, H, Hkv, hd, ms, L, cdt, mf=mf)
        assert np.all(np.isfinite(got)) and attn_close(got, ww, cdt), L


def test_attention_mfma_errors(hip):
    """The MFMA split refuses f32 caches and more than 8 heads per kv head;
    mf out of range is an error."""
    B, Hkv, hd, ms = 1, 1, 64, 128
    for H, cdt, kw in ((4, DT_F32, dict(mf=1)), (16, DT_BF16, dict(mf=1)), (16, DT_BF16, dict(mf=1, fused=1)),
                       (4, DT_BF16, dict(mf=3))):
        z = np.zeros(B * H * hd, NP_STORE[cdt])
        kv = np.zeros(B * Hkv * ms * hd, NP_STORE[cdt])
        with pytest.raises(hip.ThvmHipError, match="mf|MFMA"):
            run_attn(hip, z, kv, kv, B, H, Hkv, hd, ms, 5, cdt, **kw)


def test_attention_cpb_errors(hip):
    B, H, Hkv, hd, ms, cdt = 1, 16, 2, 64, 128, DT_BF16
    z = np.zeros(B * H * hd, np.uint16)
    kv = np.zeros(B * Hkv * ms * hd, np.uint16)
    for kw in (dict(cpb=2, fused=1), dict(cpb=3, fused=1)):
        with pytest.raises(hip.ThvmHipError):
            run_attn(hip, z, kv, kv, B, H, Hkv, hd, ms, 5, cdt, **kw)
    with pytest.raises(hip.ThvmHipError):        # the VALU split, 8 heads per kv head: one chunk per block only
        run_attn(hip, z, kv, kv, B, H, Hkv, hd, ms, 5, cdt, cpb=2, mf=2)


@pytest.mark.parametrize("H,Hkv,hd", [(32, 8, 128), (8, 8, 64), (16, 2, 64)])
def test_attention_mfma_one_launch_repeated(hip, H, Hkv, hd):
    """The one-launch MFMA form (the last split block of a row and kv head
    merges) on one partial buffer over changing lengths and chunks per block:
    every merge finds its counter at zero, and the outputs are the two-launch
    MFMA form's bit for bit (the same fold) and within the bars of the
    oracle."""
    B, ms, cdt = 2, 640, DT_BF16
    rng = np.random.default_rng(H + hd)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    nsplit = (ms + 63) // 64
    part1 = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    part2 = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    for L, cpb in ((640, 0), (1, 0), (65, 2), (300, 0), (17, 3), (129, 1), (640, 4), (64, 0)):
        say(f"case: attn mfma one launch H={H} Hkv={Hkv} hd={hd} L={L} cpb={cpb}")
        one, ww = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, part=part1, mf=1, fused=1, cpb=cpb)
        two, _ = run_attn(hip, qs, ks, vs, B, H, Hkv, hd, ms, L, cdt, part=part2, mf=1, fused=0, cpb=cpb)
        assert np.array_equal(one, two), (L, cpb, np.max(np.abs(one - two)))
        assert attn_close(one, ww, cdt), (L, cpb, np.max(np.abs(one - ww)))


def test_attention_fused_repeated(hip):
    """Ten launches on one partial buffer at changing lengths: every merge
    finds its counter at zero and the outputs match the two-kernel form of
    one chunk per block."""
    B, H, Hkv, hd, ms, cdt = 1, 32, 8, 128, 2176, DT_BF16
    say("case: fused attention, 10 launches on one partial buffer")
    rng = np.random.default_rng(5)
    qs, _ = rand_store(rng, (B, H, hd), cdt)
    ks, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    vs, _ = rand_store(rng, (B, Hkv, ms, hd), cdt)
    nsplit = (ms + 63) // 64
    qb, kb, vb = up(hip, qs), up(hip, ks), up(hip, vs)
    part = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    part2 = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    for L in (2049, 2050, 1, 64, 65, 2176, 700, 129, 2048, 3):
        outs = []
        for fused, pb in ((1, part), (0, part2)):
            o = hip.Buffer(B * H * hd * 2)
            hip.builtin("attn", [o, qb, kb, vb, up(hip, np.array([L], np.int32)), pb], b=B, h=H,
                        hkv=Hkv, hd=hd, maxseq=ms, chunk=64, nsplit=nsplit, qt=cdt, ct=cdt, ot=cdt,
                        scale=scale, fused=fused, cpb=1, mf=2)
            outs.append(o.read(np.uint16))
        assert np.array_equal(outs[0], outs[1]), L


def test_argmax_ties_lowest_index(hip):
    B, V = 3, 50257
    say("case: argmax ties")
    rng = np.random.default_rng(14)
    lg = rng.standard_normal((B, V)).astype(np.float32)
    lg[0, [7, 30000, 50000]] = 100.0           # three-way tie -> 7
    lg[1, [40000, 40001]] = 50.0               # tie -> 40000
    lg[2, V - 1] = 60.0
    tok, pv, pi = hip.Buffer(B * 4), hip.Buffer(B * 256 * 4), hip.Buffer(B * 256 * 4)
    hip.builtin("argmax", [tok, up(hip, lg), pv, pi], b=B, v=V, nb=256)
    want = np.empty(B, np.int32)
    O.oracle().or_argmax(want.ctypes.data, lg.ctypes.data, B, V)
    assert list(tok.read(np.int32)) == list(want) == [7, 40000, V - 1]


def test_embed(hip):
    B, D, V = 2, 768, 1000
    say("case: embed")
    rng = np.random.default_rng(15)
    es, ef = rand_store(rng, (V, D), DT_BF16)
    tok = np.array([3, 999], np.int32)
    x = hip.Buffer(B * D * 2)
    hip.builtin("embed", [x, up(hip, es), up(hip, tok)], b=B, d=D, v=V, et=DT_BF16, xt=DT_BF16)
    assert np.array_equal(x.read(np.uint16).reshape(B, D), es[tok])


def test_len_bump(hip):
    say("case: len_bump")
    L = up(hip, np.array([41], np.int32))
    hip.builtin("len_bump", [L], delta=1)
    hip.builtin("len_bump", [L], delta=1)
    assert L.read(np.int32)[0] == 43


def test_touch_reads_and_leaves_data(hip):
    """The read-only pass (the bench's read ceiling, the autotuner's cache
    flush): the range is unchanged, the sink is written only on its 1-in-2^32
    xor value (zero here), and a range that is not whole 16-byte pieces is
    refused."""
    say("case: touch")
    a = np.zeros(1 << 20, np.uint32)            # 2^18 pieces: one per thread of 1024 x 256
    a[0] = 0x9E3779B9                           # piece 0 xors to the sink value, the rest to 0
    x = up(hip, a)
    sink = up(hip, np.zeros(1024, np.uint32))
    hip.builtin("touch", [x, sink], outs=(1,), n=a.nbytes, blocks=1024)
    assert np.array_equal(x.read(np.uint32), a)
    s = sink.read(np.uint32)
    assert s[0] == 0x9E3779B9 and not s[1:].any()     # thread 0 of block 0 read that piece
    with pytest.raises(hip.ThvmHipError):
        hip.builtin("touch", [x, sink], outs=(1,), n=a.nbytes - 8, blocks=1024)


def test_copy_and_kernel_timing(hip):
    """The plain copy kernel is byte-exact (odd 16-byte multiples, a partial
    grid-stride pass), rejects unaligned sizes, and the per-kernel timer binds
    its events to the kernel: an enabled timer records one positive duration
    per launch, a disabled one records nothing."""
    say("case: copy + kprof")
    rng = np.random.default_rng(16)
    for n in (16, 4096 + 48, (256 * 256 * 16 + 3) * 16):
        src = rng.integers(0, 256, n, dtype=np.uint8)
        x, y = up(hip, src), hip.Buffer(n)
        hip.kprof(True)
        hip.kprof_reset()
        hip.builtin("copy", [y, x], n=n)
        ms, cnt = hip.kprof_query("copy")
        hip.kprof(False)
        assert cnt == 1 and 0.0 < ms < 1000.0
        assert np.array_equal(y.read(np.uint8), src)
    hip.kprof_reset()
    hip.builtin("copy", [y, x], n=16)
    assert hip.kprof_query("copy")[1] == 0
    with pytest.raises(hip.ThvmHipError):
        hip.builtin("copy", [y, x], n=24)


# ------------------------------------------------ custom kernels + JIT ----
SRC_ADDONE = """extern "C" __global__ void addone(const float *x, float *y) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 8) y[i] = x[i] + 1.0f;
}"""
SRC_DBL = """extern "C" __global__ void dbl(const float *x, float *s) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 8) s[i] = x[i] * 2.0f;
}"""
SRC_ADD3 = """extern "C" __global__ void add3(const float *s, float *y) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 8) y[i] = s[i] + 3.0f;
}"""
SRC_TWO = """extern "C" __global__ void twoout(const float *x, float *y1, float *y2) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 8) { y1[i] = x[i] + 1.0f; y2[i] = x[i] * 10.0f; }
}"""


def test_custom_kernel_eager_and_jit_replay(hip):
    """The reference's custom-kernel CUDA test (tests/test_custom_kernel_cuda.c)
    on HIP: eager add-one, a 2-kernel chain, a JIT capture of the chain with 3
    replays over refreshed inputs (replay 1 captures the hipGraph, 2-3 hit it),
    and a two-output kernel."""
    say("case: custom hiprtc kernels + jit")
    g, b = (1, 1, 1), (8, 1, 1)
    xv = np.arange(8, dtype=np.float32)
    x, y = up(hip, xv), hip.Buffer(32)
    hip.dispatch("addone", SRC_ADDONE, [x, y], grid=g, block=b, outs=(1,))
    assert np.array_equal(y.read(np.float32), xv + 1)
    cx, s, cy = up(hip, xv), hip.Buffer(32), hip.Buffer(32)
    hip.dispatch("dbl", SRC_DBL, [cx, s], grid=g, block=b, outs=(1,))
    hip.dispatch("add3", SRC_ADD3, [s, cy], grid=g, block=b, outs=(1,))
    assert np.array_equal(cy.read(np.float32), xv * 2 + 3)
    with hip.Jit() as jit:
        hip.dispatch("dbl", SRC_DBL, [cx, s], grid=g, block=b, outs=(1,))
        hip.dispatch("add3", SRC_ADD3, [s, cy], grid=g, block=b, outs=(1,))
    assert jit.op_count() == 2
    for rep in (1, 2, 3):
        xr = (10 * rep + np.arange(8)).astype(np.float32)
        cx.write(xr)
        cy.write(np.full(8, -999, np.float32))
        jit.replay()
        assert np.array_equal(cy.read(np.float32), xr * 2 + 3), f"replay {rep}"
    jit.drop()
    y1, y2 = hip.Buffer(32), hip.Buffer(32)
    hip.dispatch("twoout", SRC_TWO, [x, y1, y2], grid=g, block=b, outs=(1, 2))
    assert np.array_equal(y1.read(np.float32), xv + 1)
    assert np.array_equal(y2.read(np.float32), xv * 10)


def test_custom_kernel_errors(hip):
    say("case: custom kernel error paths")
    x = hip.Buffer(32)
    with pytest.raises(hip.ThvmHipError):
        hip.dispatch("nosuch", "extern \"C\" __global__ void k(float *x) {}", [x])
    with pytest.raises(hip.ThvmHipError):
        hip.dispatch("bad", "this is not HIP", [x])
    with pytest.raises(hip.ThvmHipError):
        hip.builtin("nosuchkernel", [x])
    with pytest.raises(hip.ThvmHipError):   # too small a buffer for the shape
        hip.builtin("cast", [x, x], n=1000, xt=DT_F32, yt=DT_F32)
