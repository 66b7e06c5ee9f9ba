"""Pin the CPU oracle before trusting it (CPU only).

Checks, per oracle function:
  * golden vectors written by the compiled reference (tests/golden/*.npz,
    made by tests/golden/make_golden.py from oracle/_ref/libref.so);
  * the reference test suite's own known answers (tests/test_fp8_nonfinite.c
    values computed with tinygrad 365f87a8a; tests/test_matvec_blas.c all-ones
    -> K; tests/test_sym_decode_step.c uniform attention over rows 0..3 = 1.5);
  * what the mathematics fixes: IEEE binary16 decode (numpy float16),
    encode(decode(b)) == b on every finite pattern, float64 brute force;
  * the live reference harness, when it was built in this container."""
import sys

import numpy as np
import pytest

import _oracle as O

G = O.ROOT / "tests" / "golden"
DT_FP8, DT_E5M2, DT_F16, DT_BF16, DT_F32 = 9, 10, 11, 12, 13


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same_float(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(bits(a[~na]), bits(b[~nb]))


@pytest.fixture(scope="module")
def codecs():
    return np.load(G / "ref_codecs.npz")


# ---------------------------------------------------------------- codecs ----
def test_fp8_decode_tables_match_reference(codecs):
    b = np.arange(256, dtype=np.uint8)
    assert same_float(O.decode(b, DT_FP8), codecs["dec_e4m3"])
    assert same_float(O.decode(b, DT_E5M2), codecs["dec_e5m2"])


def test_fp16_decode_matches_reference_and_ieee(codecs):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    d = O.decode(h, DT_F16)
    assert same_float(d, codecs["dec_fp16"])
    ieee = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(ieee)
    assert np.array_equal(bits(d[fin]), bits(ieee[fin]))


def test_e4m3_decode_closed_form():
    for b in range(256):
        s, e, m = b >> 7, (b >> 3) & 15, b & 7
        v = O.oracle().or_fp8e4m3_to_f32(b)
        if (b & 0x7F) == 0x7F:
            assert np.isnan(v)
            continue
        want = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        assert v == (-want if s else want), b


def test_e5m2_decode_closed_form():
    for b in range(256):
        s, e, m = b >> 7, (b >> 2) & 31, b & 3
        v = O.oracle().or_fp8e5m2_to_f32(b)
        if e == 31:
            assert (np.isinf(v) and (v < 0) == bool(s)) if m == 0 else np.isnan(v), b
            continue
        want = (m / 4.0) * 2.0 ** -14 if e == 0 else (1 + m / 4.0) * 2.0 ** (e - 15)
        assert v == (-want if s else want), b


def _nearest_even_code(x, table, max_code):
    """Brute force: the finite code whose value is nearest to x (float64),
    ties to the even code, magnitudes past the largest finite saturated."""
    ax = abs(x)
    codes = np.arange(max_code + 1)
    d = np.abs(table[codes].astype(np.float64) - ax)
    best = np.flatnonzero(d == d.min())
    c = int(best[0]) if len(best) == 1 else int(best[best % 2 == 0][0])
    return c | (0x80 if np.signbit(x) else 0)


@pytest.mark.parametrize("dt,max_code", [(DT_FP8, 0x7E), (DT_E5M2, 0x7B)])
def test_fp8_encoders_brute_force_nearest_even(dt, max_code):
    """Every midpoint between adjacent codes (a tie), one f32 ulp either side
    of it, every code value itself, and random values over the whole range,
    against a nearest-value search over the decode table."""
    R = O.oracle()
    table = O.decode(np.arange(256, dtype=np.uint8), dt).astype(np.float64)
    vals = table[: max_code + 1]
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(0))
    rng = np.random.default_rng(5)
    rnd = (rng.standard_normal(4000) * 2.0 ** rng.uniform(-22, 18, 4000)).astype(np.float32)
    top = np.float32(vals[max_code] * 1.2)
    xs = np.concatenate([mids, up, dn, vals.astype(np.float32), rnd, [top, -top, 0.0, -0.0]])
    xs = np.concatenate([xs, -xs]).astype(np.float32)
    enc = {DT_FP8: (R.or_f32_to_fp8e4m3, R.or_f32_to_fp8e4m3_sat),
           DT_E5M2: (R.or_f32_to_fp8e5m2, R.or_f32_to_fp8e5m2_sat)}[dt]
    for x in xs:
        want = _nearest_even_code(float(x), table, max_code)
        assert enc[0](float(x)) == want and enc[1](float(x)) == want, (float(x), want)


@pytest.mark.parametrize("name,dt,sat", [("bf16", DT_BF16, None), ("fp16", DT_F16, None),
                                         ("e4m3", DT_FP8, 0), ("e4m3_sat", DT_FP8, 1),
                                         ("e5m2", DT_E5M2, 0), ("e5m2_sat", DT_E5M2, 1)])
def test_encoders_match_reference_sweep(codecs, name, dt, sat):
    f = codecs["sweep"]
    R = O.oracle()
    fn = {"bf16": R.or_f32_to_bf16, "fp16": R.or_f32_to_fp16, "e4m3": R.or_f32_to_fp8e4m3,
          "e4m3_sat": R.or_f32_to_fp8e4m3_sat, "e5m2": R.or_f32_to_fp8e5m2,
          "e5m2_sat": R.or_f32_to_fp8e5m2_sat}[name]
    got = np.array([fn(float(v)) for v in f])
    assert np.array_equal(got, codecs["enc_" + name].astype(got.dtype))


def test_encode_decode_roundtrip_all_finite():
    b8 = np.arange(256, dtype=np.uint8)
    d8 = O.decode(b8, DT_FP8)
    fin = ~np.isnan(d8)
    assert np.array_equal(O.encode(d8[fin], DT_FP8), b8[fin])
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dh = O.decode(h, DT_F16)
    fin = np.isfinite(dh)
    assert np.array_equal(O.encode(dh[fin], DT_F16), h[fin])


def test_bf16_encode_is_round_to_nearest_even():
    rng = np.random.default_rng(3)
    f = (rng.standard_normal(50000) * 10.0 ** rng.uniform(-30, 30, 50000)).astype(np.float32)
    got = O.encode(f, DT_BF16).astype(np.uint32) << 16
    got = got.view(np.float32).astype(np.float64)
    lo = (bits(f) & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi = ((bits(f) & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    x = f.astype(np.float64)
    dl, dh = np.abs(x - lo), np.abs(hi - x)
    nearest = np.where(dl < dh, lo, np.where(dh < dl, hi, np.nan))
    tie = np.isnan(nearest)
    assert np.array_equal(got[~tie], nearest[~tie])
    even = np.where((bits(f[tie]) >> 16) & 1 == 0, lo[tie], hi[tie])
    assert np.array_equal(got[tie], even)


def test_fp8_nonfinite_known_answers():
    """tests/test_fp8_nonfinite.c:110-192 (values computed with tinygrad)."""
    R = O.oracle()
    f32 = lambda u: float(np.array([u], np.uint32).view(np.float32)[0])  # noqa: E731
    nans = [0x7FC00000, 0x7F800001, 0x7FA00000, 0x7FFFFFFF]
    neg = [0xFFC00000, 0xFF800001, 0xFFA00000, 0xFFFFFFFF]
    assert R.or_f32_to_fp8e4m3(float("inf")) == 0x7F and R.or_f32_to_fp8e4m3(float("-inf")) == 0xFF
    assert R.or_f32_to_fp8e5m2(float("inf")) == 0x7C and R.or_f32_to_fp8e5m2(float("-inf")) == 0xFC
    for u, v in zip(nans, neg):
        assert R.or_f32_to_fp8e4m3(f32(u)) == 0x7F and R.or_f32_to_fp8e4m3(f32(v)) == 0xFF
        assert R.or_f32_to_fp8e5m2(f32(u)) == 0x7F and R.or_f32_to_fp8e5m2(f32(v)) == 0xFF
    assert R.or_f32_to_fp8e4m3_sat(float("inf")) == 0x7E and R.or_f32_to_fp8e4m3_sat(float("-inf")) == 0xFE
    assert R.or_f32_to_fp8e5m2_sat(float("inf")) == 0x7B and R.or_f32_to_fp8e5m2_sat(float("-inf")) == 0xFB
    # the NaN payloads go through memory (a Python float would quiet them)
    pats = np.array(nans + neg, np.uint32).view(np.float32)
    assert list(O.encode(pats, DT_FP8)) == [0x7F, 0x7F, 0x7F, 0x7F, 0xFF, 0xFF, 0xFF, 0xFF]
    assert list(O.encode(pats, DT_E5M2)) == [0x7E, 0x7C, 0x7D, 0x7F, 0xFE, 0xFC, 0xFD, 0xFF]
    assert R.or_f32_to_fp8e4m3_sat(464.0) == 0x7E
    assert R.or_f32_to_fp8e4m3_sat(f32(0xFF7FFFFF)) == 0xFE
    assert R.or_f32_to_fp8e5m2_sat(61440.0) == 0x7B
    assert R.or_f32_to_fp8e5m2_sat(f32(0x7F7FFFFF)) == 0x7B


# ------------------------------------------------------------------- ops ----
def test_gemv_matches_reference_linear_bit_exact():
    g = np.load(G / "ref_ops_f32.npz")
    for p in ("lin", "lin2"):
        x, w, want = g[p + "_x"], g[p + "_w"], g[p + "_y"]
        M, K = x.shape
        y = O.gemv(x, DT_F32, w, DT_F32, None, M=M, N=w.shape[0], K=K)
        assert np.array_equal(bits(y), bits(want)), p


def test_gemv_all_ones_is_k():
    """tests/test_matvec_blas.c:14-30: a ones matvec sums to K (LM-head shape)."""
    K, N = 768, 2048
    y = O.gemv(np.ones((1, K), np.float32), DT_F32, np.ones((N, K), np.float32), DT_F32, None,
               M=1, N=N, K=K)
    assert np.all(y == K)


@pytest.mark.parametrize("wdt", [DT_F32, DT_F16, DT_BF16, DT_FP8])
def test_gemv_brute_force(wdt):
    rng = np.random.default_rng(wdt)
    M, N, K = 3, 37, 96
    x = rng.standard_normal((M, K)).astype(np.float32)
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    scale = None
    if wdt == DT_FP8:
        scale = (np.abs(wf).max(1) / 448).astype(np.float32)
        ws = O.encode(wf / scale[:, None], DT_FP8)
        wd = O.decode(ws, DT_FP8).astype(np.float64) * scale[:, None]
    elif wdt == DT_F32:
        ws, wd = wf, wf.astype(np.float64)
    else:
        ws = O.encode(wf, wdt)
        wd = O.decode(ws, wdt).astype(np.float64)
    y = O.gemv(x, DT_F32, ws, wdt, scale, M=M, N=N, K=K)
    want = x.astype(np.float64) @ wd.T
    floor = np.abs(x) @ np.abs(wd).T
    assert np.all(np.abs(y - want) <= 1e-6 * floor * K ** 0.5)
    # a transposed operand is caught
    assert not np.allclose(y, (x.astype(np.float64) @ wd[::-1].T), atol=1e-3)


def test_softmax_layernorm_rmsnorm_match_reference():
    g = np.load(G / "ref_ops_f32.npz")
    x = g["sm_x"]
    y = np.empty_like(x)
    O.oracle().or_softmax(y.ctypes.data, DT_F32, x.ctypes.data, DT_F32, *x.shape)
    assert np.allclose(y, g["sm_y"], rtol=2e-6, atol=0)
    x = g["ln_x"]
    y = np.empty_like(x)
    O.oracle().or_layernorm(y.ctypes.data, DT_F32, x.ctypes.data, DT_F32, None, None, *x.shape, 1e-5)
    assert np.allclose(y, g["ln_y"], rtol=1e-5, atol=1e-6)
    x = g["rms_x"]
    y = np.empty_like(x)
    O.oracle().or_rmsnorm(y.ctypes.data, DT_F32, x.ctypes.data, DT_F32, None, *x.shape, 1e-6)
    assert np.allclose(y, g["rms_y"], rtol=1e-5, atol=1e-6)


def test_rope_brute_force():
    rng = np.random.default_rng(4)
    B, nh, hd, ms, pos = 2, 3, 8, 6, 4
    x = rng.standard_normal((B, nh, hd)).astype(np.float32)
    ang = np.arange(ms)[:, None] / (10000.0 ** (np.arange(hd // 2) * 2.0 / hd))[None]
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = x.copy()
    O.oracle().or_rope(y.ctypes.data, DT_F32, cs.ctypes.data, sn.ctypes.data, B, nh, hd, pos)
    z = x[..., 0::2] + 1j * x[..., 1::2]
    r = z * np.exp(1j * ang[pos])
    want = np.stack([r.real, r.imag], -1).reshape(B, nh, hd)
    assert np.allclose(y, want, atol=1e-5)
    # rotation preserves each pair's norm
    assert np.allclose(np.abs(y[..., 0::2] + 1j * y[..., 1::2]), np.abs(z), atol=1e-5)


def test_attention_closed_form_and_brute_force():
    """tests/test_sym_decode_step.c: with q=0 the scores tie, the softmax is
    uniform, and the output is the mean of V rows 0..3 = 1.5."""
    B, H, Hkv, hd, ms, L = 1, 2, 1, 4, 8, 4
    q = np.zeros((B, H, hd), np.float32)
    k = np.random.default_rng(0).standard_normal((B, Hkv, ms, hd)).astype(np.float32)
    v = np.zeros((B, Hkv, ms, hd), np.float32)
    v[0, 0, :L, :] = np.arange(L)[:, None]
    out = np.empty(B * H * hd, np.float32)
    O.oracle().or_attn_decode(out.ctypes.data, DT_F32, q.ctypes.data, DT_F32, k.ctypes.data,
                              v.ctypes.data, DT_F32, B, H, Hkv, hd, ms, L, 0.5)
    assert np.all(out == 1.5)
    rng = np.random.default_rng(1)
    B, H, Hkv, hd, ms, L = 2, 8, 2, 16, 40, 33
    q = rng.standard_normal((B, H, hd)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, ms, hd)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, ms, hd)).astype(np.float32)
    out = np.empty((B, H, hd), np.float32)
    O.oracle().or_attn_decode(out.ctypes.data, DT_F32, q.ctypes.data, DT_F32, k.ctypes.data,
                              v.ctypes.data, DT_F32, B, H, Hkv, hd, ms, L, 0.25)
    for b in range(B):
        for h in range(H):
            kk, vv = k[b, h // (H // Hkv), :L].astype(np.float64), v[b, h // (H // Hkv), :L]
            s = kk @ q[b, h] * 0.25
            p = np.exp(s - s.max())
            assert np.allclose(out[b, h], (p / p.sum()) @ vv, atol=1e-5)


def test_argmax_lowest_index():
    lg = np.array([[1, 5, 5, 2], [9, 9, 9, 9]], np.float32)
    t = np.empty(2, np.int32)
    O.oracle().or_argmax(t.ctypes.data, lg.ctypes.data, 2, 4)
    assert list(t) == [1, 0]


def test_live_reference_codecs_random():
    R = O.ref()
    if R is None:
        pytest.skip("reference harness not built in this checkout")
    rng = np.random.default_rng(11)
    f = (rng.standard_normal(4000) * 10.0 ** rng.uniform(-12, 6, 4000)).astype(np.float32)
    Or = O.oracle()
    for v in f:
        v = float(v)
        assert Or.or_f32_to_fp8e4m3_sat(v) == R.ref_f32_to_fp8e4m3_sat(v)
        assert Or.or_f32_to_bf16(v) == R.ref_f32_to_bf16(v)
        assert Or.or_f32_to_fp16(v) == R.ref_f32_to_fp16_manual(v)


# ------------------------------------------------------------ DeepSeek-V2 ----
class _Tensors:
    """A decoder-like view of numpy tensors for the oracle models."""

    def __init__(self, t):
        self.t = t

    def read_tensor(self, name):
        return self.t[name]


def _dsv2_run(t, cfg, prompt, count):
    om = O.OracleDsv2(_Tensors(t), dict(cfg, wdtype=12))
    ids, top = [], []
    tok = np.array([prompt[0]], np.int32)
    for pos in range(len(prompt) + count - 1):
        lg, nx = om.step(tok, pos)
        if pos >= len(prompt) - 1:
            ids.append(int(nx[0]))
            o = np.argsort(-lg[0], kind="stable")[:2]
            top.append((o[0], lg[0, o[0]], o[1], lg[0, o[1]]))
        tok = np.array([prompt[pos + 1] if pos + 1 < len(prompt) else nx[0]], np.int32)
    return ids, top


@pytest.mark.parametrize("fixture", ["dsv2_ref.npz", "dsv2_ref_dense.npz"])
def test_dsv2_oracle_reproduces_reference_trajectory(fixture):
    """The oracle's DeepSeek-V2 step (or_dsv2_step: MLA prep/attention, router,
    routed + shared experts, the dense first layer, split-K projections)
    against the compiled reference DSV2 decode bench on the same seeded model
    (fixtures written by tests/golden/make_dsv2_golden.py through a DSV2PK01
    weight pack; the second has a dense first layer): the greedy ids are
    identical and the top-2 logits agree to 1e-5."""
    import _dsv2_weights as W
    sys.path.insert(0, str(O.ROOT / "tests" / "golden"))
    import make_dsv2_golden as G
    cfg = G.FIXTURES[fixture]
    g = np.load(O.ROOT / "tests" / "golden" / fixture)
    t = W.make_dsv2(cfg, int(g["seed"]))
    assert G.weight_digest(t) == str(g["digest"]), "weight generator drifted from the fixture"
    ids, top = _dsv2_run(t, cfg, list(g["prompt"]), len(g["gen_ids"]))
    assert ids == list(g["gen_ids"])
    for (i1, v1, i2, v2), ref in zip(top[1:], g["top2"]):
        assert (i1, i2) == (int(ref[1]), int(ref[3]))
        assert abs(v1 - ref[2]) <= 1e-5 and abs(v2 - ref[4]) <= 1e-5


def test_dsv2_dense_activation_matches_reference_uops():
    """h = silu(g) * u of the dense first layer, bit for bit against the
    compiled reference realizing the same bf16 uop DAG
    (oracle/ref_harness.c ref_dense_silu_mul_bf16) on 60,000 pairs, including
    large |g| (exp2 overflow / underflow) and signed zeros."""
    R = O.ref()
    if R is None:
        pytest.skip("reference harness not built in this checkout")
    rng = np.random.default_rng(17)
    n = 60000
    gf = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 2.2, n)).astype(np.float32)
    gf[:4] = [0.0, -0.0, 200.0, -200.0]
    g, u = O.encode(gf, DT_BF16), O.encode(rng.standard_normal(n).astype(np.float32), DT_BF16)
    want, got = np.zeros(n, np.uint16), np.zeros(n, np.uint16)
    assert R.ref_dense_silu_mul_bf16(g.ctypes.data, u.ctypes.data, want.ctypes.data, n) == 0
    O.oracle().or_dsv2_dense_act(g.ctypes.data, u.ctypes.data, got.ctypes.data, n)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} differ, e.g. g={O.decode(g[bad[:3]], DT_BF16)}"


def test_route_brute_force_and_ties():
    rng = np.random.default_rng(3)
    for E, K in ((64, 6), (8, 3), (5, 5)):
        g = rng.standard_normal(E).astype(np.float32)
        g[[1, E - 1]] = g.max() + 1.0                    # a tie at the top -> lower id first
        sel, pr = np.empty(K, np.int32), np.empty(K, np.float32)
        O.oracle().or_route(sel.ctypes.data, pr.ctypes.data, g.ctypes.data, E, K)
        assert list(sel) == list(np.lexsort((np.arange(E), -g))[:K])
        p = np.exp(g.astype(np.float64) - g.max())
        p /= p.sum()
        assert np.allclose(pr, p[sel], rtol=1e-6)


def test_mla_attn_closed_forms():
    """One live row: softmax weight 1, olat = that latent row, o = W_uv . row;
    equal rows: the same for any scores."""
    rng = np.random.default_rng(4)
    H, kv, dr, dv = 4, 64, 16, 32
    bf = lambda a: O.encode(np.asarray(a, np.float32), 12)
    wuv = bf(rng.standard_normal((H * dv, kv)) * 0.1)
    qlat = rng.standard_normal((H, kv)).astype(np.float32)
    qpe = bf(rng.standard_normal((H, dr)))
    for L, same in ((1, False), (9, True)):
        row = bf(rng.standard_normal(kv))
        ckv = np.tile(row, (L, 1)) if same else row[None, :].copy()
        kpe = bf(rng.standard_normal((L, dr)))
        o = np.empty((H, dv), np.uint16)
        O.oracle().or_mla_attn(o.ctypes.data, qlat.ctypes.data, qpe.ctypes.data, ckv.ctypes.data,
                               kpe.ctypes.data, L, wuv.ctypes.data, 12, None, H, kv, dr, dv, 0.3)
        want = O.decode(wuv, 12).astype(np.float64) @ O.decode(row, 12).astype(np.float64)
        got = O.decode(o, 12).ravel()
        assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-6)


def test_moe_brute_force():
    """or_moe against a float64 restatement written from the expert-FFN
    definition (gate/up interleaved per expert, probs-weighted routed sum plus
    the shared expert)."""
    rng = np.random.default_rng(5)
    D, E, K, I, S = 64, 6, 2, 32, 64
    bf = lambda a: O.encode(np.asarray(a, np.float32), 12)
    wgu, wd = bf(rng.standard_normal((E, 2 * I, D)) * 0.1), bf(rng.standard_normal((E, D, I)) * 0.1)
    wgs, wds = bf(rng.standard_normal((2 * S, D)) * 0.1), bf(rng.standard_normal((D, S)) * 0.1)
    xb = bf(rng.standard_normal(D))
    sel, probs = np.array([4, 1], np.int32), np.array([0.6, 0.3], np.float32)
    out = np.empty(D, np.float32)
    O.oracle().or_moe(out.ctypes.data, xb.ctypes.data, sel.ctypes.data, probs.ctypes.data,
                      wgu.ctypes.data, None, wd.ctypes.data, None, wgs.ctypes.data, None,
                      wds.ctypes.data, None, 12, D, I, S, K)
    f = lambda a: O.decode(a, 12).astype(np.float64)
    x = f(xb)
    silu = lambda v: v / (1 + np.exp(-v))
    want = np.zeros(D)
    for e, p in zip(sel, probs):
        g, u = f(wgu[e, 0::2]) @ x, f(wgu[e, 1::2]) @ x
        want += p * (f(wd[e]) @ (silu(g) * u))
    g, u = f(wgs[0::2]) @ x, f(wgs[1::2]) @ x
    want += f(wds) @ (silu(g) * u)
    assert np.allclose(out, want, rtol=1e-4, atol=1e-6)


# ------------------------------------------------------------- sampling ----
def test_sexpf_is_exp_to_float_accuracy():
    """or_sexpf (Cody-Waite + degree-8 Taylor): within 2 ulp of exp over the
    range the sampler uses, exact at 0, zero below -80."""
    R = O.oracle()
    xs = np.concatenate([np.linspace(-80, 0, 200001), -np.logspace(-8, 1.9, 2000), [0.0, -1e-30]])
    got = np.array([R.or_sexpf(float(x)) for x in xs], np.float64)
    want = np.exp(xs.astype(np.float32).astype(np.float64))
    assert np.all(np.abs(got - want) <= 2.5e-7 * want)
    assert R.or_sexpf(0.0) == 1.0 and R.or_sexpf(-80.5) == 0.0 and R.or_sexpf(float("-inf")) == 0.0


def test_sample_u01_uniform_and_keyed():
    R = O.oracle()
    u = np.array([R.or_sample_u01(7, 0, L) for L in range(20000)])
    assert np.all((u >= 0) & (u < 1))
    from scipy import stats
    assert stats.kstest(u, "uniform").pvalue > 1e-3
    assert R.or_sample_u01(7, 0, 5) == R.or_sample_u01(7, 0, 5)
    assert R.or_sample_u01(7, 0, 5) != R.or_sample_u01(7, 1, 5) != R.or_sample_u01(8, 0, 5)


def _sample(lg, nb, temp, seed, L):
    B, V = lg.shape
    tok = np.full(B, -1, np.int32)
    lg = np.ascontiguousarray(lg, np.float32)
    O.oracle().or_sample(tok.ctypes.data, lg.ctypes.data, B, V, nb, 1.0 / temp, seed, L)
    return tok


@pytest.mark.parametrize("V,nb", [(50, 1), (1000, 16), (128256, 256)])
@pytest.mark.parametrize("temp", [0.7, 1.0, 3.0])
def test_sample_is_the_inverse_cdf_of_the_tempered_softmax(V, nb, temp):
    """Each sampled id is where the float64 CDF of softmax(z / T), in index
    order, crosses the same uniform draw u: cdf(i-1) <= u <= cdf(i) up to f32
    rounding.  A wrong chunk, offset or threshold misses this."""
    R = O.oracle()
    rng = np.random.default_rng(V + int(temp * 10))
    lg = (rng.standard_normal((1, V)) * 2).astype(np.float32)
    z = lg[0].astype(np.float32) * np.float32(1.0 / temp)
    p = np.exp(z.astype(np.float64) - z.max())
    cdf = np.cumsum(p / p.sum())
    n = 40 if V > 10000 else 300
    for L in range(n):
        u = R.or_sample_u01(11, 0, L)
        i = int(_sample(lg, nb, temp, 11, L)[0])
        lo_c = cdf[i - 1] if i > 0 else 0.0
        assert lo_c - 2e-5 <= u <= cdf[i] + 2e-5, (L, i, u, lo_c, cdf[i])


def test_sample_frequencies_match_softmax():
    from scipy import stats
    V = 12
    lg = np.array([[0.1, 2.0, -1.0, 0.5, 3.0, 0.0, -2.0, 1.5, 1.0, -0.5, 2.5, 0.2]], np.float32)
    p = np.exp(lg[0].astype(np.float64) / 1.3)
    p /= p.sum()
    ids = np.array([_sample(lg, 1, 1.3, 5, L)[0] for L in range(30000)])
    counts = np.bincount(ids, minlength=V)
    assert stats.chisquare(counts, p * len(ids)).pvalue > 1e-4


def test_sample_edge_cases():
    # one overwhelming logit; -inf logits never drawn; a tiny temperature is
    # the argmax; rows are independent draws
    lg = np.full((3, 500), -np.inf, np.float32)
    lg[0, 123] = 0.0
    lg[1, :] = 0.0
    lg[1, ::2] = -np.inf
    lg[2, :] = np.linspace(-1, 1, 500)
    for L in range(50):
        t = _sample(lg, 4, 1.0, 3, L)
        assert t[0] == 123 and t[1] % 2 == 1
    assert all(_sample(lg[2:3], 4, 1e-4, 3, L)[0] == 499 for L in range(20))


# ---- blind speculative draft / commit (or_spec_draft, or_spec_accept) ----
# Known answers worked by hand from the reference's statement of draft_prep
# and accept_commit (bench/dsv2_decode_bench.c:1116-1170), and the property
# that makes speculation exact: committing through draft / verify / accept
# reproduces plain greedy decoding for any deterministic next-token rule.

@pytest.mark.parametrize("hist,L,S,V,forced,want_ca,want_ce", [
    # bigram (5,6) recurs at j=0; j=4 is the current bigram itself (j+1 = P)
    ([5, 6, 7, 8, 5, 6], 6, 4, 100, False, [6, 7, 8, 5], [6, 7, 8, 5]),
    # the most recent earlier match wins (j=3 over j=0)
    ([1, 2, 3, 1, 2, 4, 1, 2], 8, 4, 100, False, [2, 4, 1, 2], [2, 4, 1, 2]),
    # the continuation stops at P: later drafts are holes, embedded as the pending id
    ([9, 9, 9], 3, 3, 100, False, [9, 9, -1], [9, 9, 9]),
    ([1, 2, 3, 4], 4, 3, 100, False, [4, -1, -1], [4, 4, 4]),            # no match
    ([5, 6, 70, 5, 6], 5, 3, 50, False, [6, -1, 5], [6, 6, 5]),           # id >= V: a hole
    ([7], 1, 2, 100, False, [7, -1], [7, 7]),                             # P = 0: no bigram
    ([1, 2, 3, 10, 11, 12, 0], 4, 3, 100, True, [10, 11, 12], [10, 11, 12]),   # forced drafts
])
def test_spec_draft_known_answers(hist, L, S, V, forced, want_ca, want_ce):
    ca, ce = O.spec_draft(hist, L, S, V, forced)
    assert ca.tolist() == want_ca and ce.tolist() == want_ce


def test_spec_accept_known_answers():
    h = [5, 6, 7, 8, 5, 6] + [0] * 6
    # two drafts verified, the third rejected: commit 7, 8 and the bonus am[2]
    h2, L2 = O.spec_accept(h, 6, [6, 7, 8, 5], [7, 8, 0, 3], 4)
    assert L2 == 9 and h2[6:9].tolist() == [7, 8, 0] and h2[:6].tolist() == h[:6]
    # every draft verified: S ids committed
    h3, L3 = O.spec_accept(h, 6, [6, 1, 2, 3], [1, 2, 3, 4], 4)
    assert L3 == 10 and h3[6:10].tolist() == [1, 2, 3, 4]
    # a hole never matches: only the bonus
    h4, L4 = O.spec_accept(h, 6, [6, -1, 2, 3], [-1, 2, 3, 4], 4)
    assert L4 == 7 and h4[6] == -1
    # no room for S rows: unchanged
    h5, L5 = O.spec_accept(h, 9, [6, 1, 2, 3], [1, 2, 3, 4], 4)
    assert L5 == 9 and h5.tolist() == h


@pytest.mark.parametrize("S", [2, 3, 4])
@pytest.mark.parametrize("rule", range(4))
def test_spec_reproduces_greedy(S, rule):
    rng = np.random.default_rng(rule)
    V = 12
    table = rng.integers(0, V, (V, V))
    def nxt(seq):            # a deterministic "model": a function of the last two ids
        return int(table[seq[-2] if len(seq) > 1 else 0, seq[-1]])
    prompt = rng.integers(0, V, 5).tolist()
    n = 60
    greedy = list(prompt)
    while len(greedy) < len(prompt) + n:
        greedy.append(nxt(greedy))
    cap = len(prompt) + n + S + 2
    hist = np.zeros(cap, np.int32)
    hist[:len(prompt)] = prompt
    L, steps, advanced = len(prompt), 0, []
    while L < len(prompt) + n:
        ca, ce = O.spec_draft(hist, L, S, V)
        # verify: row s continues the committed history with the embedded candidates 0..s
        base = hist[:L - 1].tolist()
        am = [nxt(base + ce[:s + 1].tolist()) for s in range(S)]
        hist, L2 = O.spec_accept(hist, L, ca, am, S)
        advanced.append(L2 - L)
        L = L2
        steps += 1
    got = hist[:len(prompt) + n].tolist()
    assert got == greedy[:len(prompt) + n]
    assert all(1 <= a <= S for a in advanced)
    assert steps < n     # a loop-prone rule accepts some drafts
