"""GPU parity of the DeepSeek-V2 decode path (MLA latent attention, MoE
routing and expert FFN, the whole DSV2 decoder) against the CPU oracle
(oracle/oracle.c or_mla_prep / or_mla_attn / or_route / or_moe /
or_dsv2_step).  Bars: routing ids bit-exact; f32 results within 1e-5 of the
magnitude sum; bf16 outputs within one storage rounding (2^-7 relative) plus
that floor; decoder logits within 2e-2 relative (fp8 weights) or 1e-2
absolute (bf16 weights)."""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13


def say(*a):
    print(*a, flush=True)


def up(hip, a):
    return hip.Buffer.from_numpy(np.ascontiguousarray(a))


def bf(a):
    return O.encode(np.asarray(a, np.float32), DT_BF16)


def unbf(a):
    return O.decode(a, DT_BF16)


def fp8_rows(rng, rows, cols, std=0.02):
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    s = (np.abs(w).max(1) / 448.0).astype(np.float32)
    q = O.encode(w / s[:, None], DT_FP8)
    return q, s, O.decode(q, DT_FP8) * s[:, None]


def weights(rng, rows, cols, wdt):
    if wdt == DT_FP8:
        return fp8_rows(rng, rows, cols)
    w = bf(rng.standard_normal((rows, cols)) * 0.02)
    return w, None, unbf(w)


def close_bf16(got, want, floor=0.0):
    return np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-5 * floor + 1e-6


MLA_SHAPES = [dict(H=16, dn=128, dr=64, kv=512, dv=128, B=2, ms=256, L=130),
              dict(H=8, dn=32, dr=16, kv=64, dv=32, B=1, ms=128, L=64),
              dict(H=8, dn=32, dr=16, kv=128, dv=32, B=3, ms=64, L=1),
              dict(H=16, dn=128, dr=64, kv=512, dv=128, B=8, ms=192, L=150),   # all heads per block
              dict(H=16, dn=128, dr=64, kv=512, dv=128, B=1, ms=320, L=257)]   # chunk groups + 1-row tail

# split kernels of mla_attn: (mode, cpb); the MFMA split exists for the
# DeepSeek-V2 shape (16 heads, kv 512, rope 64) only
MLA_SPLITS = [(0, 0), (1, 0), (2, 1), (2, 2), (2, 3), (2, 4)]


def mla_splits(H, kv, dr):
    mf = H == 16 and kv == 512 and dr == 64
    return [(m, c) for m, c in MLA_SPLITS if m != 2 or mf]


@pytest.mark.parametrize("wdt", [DT_FP8, DT_BF16])
@pytest.mark.parametrize("shape", MLA_SHAPES, ids=["c5", "smoke", "L1", "c5_b8", "c5_tail"])
def test_mla_prep_and_attn(hip, shape, wdt):
    H, dn, dr, kv, dv, B, ms, L = (shape[k] for k in ("H", "dn", "dr", "kv", "dv", "B", "ms", "L"))
    say(f"case: mla {shape} wdt={wdt}")
    rng = np.random.default_rng(H * 100 + kv + L + wdt)
    ldq = H * (dn + dr) + kv + dr
    qkv = bf(rng.standard_normal((B, ldq)))
    wuk, suk, wukf = weights(rng, H * kv, dn, wdt)
    wuv, suv, wuvf = weights(rng, H * dv, kv, wdt)
    wkvn = (1 + 0.1 * rng.standard_normal(kv)).astype(np.float32)
    ang = rng.uniform(0, 6.3, (ms, dr // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    ckv0 = bf(rng.standard_normal((B, ms, kv)))
    kpe0 = bf(rng.standard_normal((B, ms, dr)))
    pos = L - 1
    ckv, kpe = up(hip, ckv0), up(hip, kpe0)
    qlat, qpe = hip.Buffer(B * H * kv * 4), hip.Buffer(B * H * dr * 2)
    Lb = up(hip, np.array([L], np.int32))
    f8 = wdt == DT_FP8
    args = [up(hip, qkv), up(hip, wuk)] + ([up(hip, suk)] if f8 else []) + [
        up(hip, wkvn), up(hip, cs), up(hip, sn), Lb, ckv, kpe, qlat, qpe]
    hip.builtin("mla_prep", args, b=B, h=H, dn=dn, dr=dr, kv=kv, dv=dv, maxseq=ms, wt=wdt, eps=1e-6)
    g_qlat = qlat.read(np.float32).reshape(B, H, kv)
    g_qpe = qpe.read(np.uint16).reshape(B, H, dr)
    g_ckv = ckv.read(np.uint16).reshape(B, ms, kv)
    g_kpe = kpe.read(np.uint16).reshape(B, ms, dr)
    for b in range(B):
        w_qpe = np.empty((H, dr), np.uint16)
        w_qlat = np.empty((H, kv), np.float32)
        w_crow, w_prow = np.empty(kv, np.uint16), np.empty(dr, np.uint16)
        O.oracle().or_mla_prep(w_qpe.ctypes.data, w_qlat.ctypes.data, w_crow.ctypes.data,
                               w_prow.ctypes.data, np.ascontiguousarray(qkv[b]).ctypes.data,
                               wuk.ctypes.data, wdt, suk.ctypes.data if f8 else None,
                               wkvn.ctypes.data, np.ascontiguousarray(cs[pos]).ctypes.data,
                               np.ascontiguousarray(sn[pos]).ctypes.data, H, dn, dr, kv, 1e-6)
        assert np.all(close_bf16(unbf(g_qpe[b]), unbf(w_qpe)))
        qn = unbf(qkv[b, :H * (dn + dr)].reshape(H, dn + dr)[:, :dn])
        floor = (np.abs(wukf.reshape(H, kv, dn)) @ np.abs(qn)[:, :, None])[..., 0]
        assert np.all(np.abs(g_qlat[b] - w_qlat) <= 1e-5 * floor + 1e-30)
        assert np.all(close_bf16(unbf(g_ckv[b, pos]), unbf(w_crow)))
        assert np.all(close_bf16(unbf(g_kpe[b, pos]), unbf(w_prow)))
        # rows other than pos untouched
        keep = np.arange(ms) != pos
        assert np.array_equal(g_ckv[b, keep], ckv0[b, keep])
        assert np.array_equal(g_kpe[b, keep], kpe0[b, keep])

    scale = 0.1352
    nsplit = (ms + 63) // 64
    w_o = np.empty((B, H, dv), np.uint16)
    for b in range(B):
        O.oracle().or_mla_attn(w_o[b].ctypes.data, np.ascontiguousarray(g_qlat[b]).ctypes.data,
                               np.ascontiguousarray(g_qpe[b]).ctypes.data,
                               np.ascontiguousarray(g_ckv[b]).ctypes.data,
                               np.ascontiguousarray(g_kpe[b]).ctypes.data, L, wuv.ctypes.data, wdt,
                               suv.ctypes.data if f8 else None, H, kv, dr, dv, scale)
    for mode, cpb in mla_splits(H, kv, dr):
        say(f"case: mla_attn mode={mode} cpb={cpb}")
        o = hip.Buffer(B * H * dv * 2)
        part = hip.Buffer(B * nsplit * H * (kv + 4) * 4)
        args = [o, qlat, qpe, ckv, kpe, Lb, part, up(hip, wuv)] + ([up(hip, suv)] if f8 else [])
        hip.builtin("mla_attn", args, b=B, h=H, dn=dn, dr=dr, kv=kv, dv=dv, maxseq=ms, nsplit=nsplit,
                    wt=wdt, scale=scale, mode=mode, cpb=cpb)
        g_o = unbf(o.read(np.uint16).reshape(B, H, dv))
        outs = [("o", g_o)]
        if kv % 64 == 0:
            # the merge in latent quarters: four f32 quarter sums, which the
            # o projection adds, scales and rounds (quarter_x: its staging)
            o4 = hip.Buffer(4 * B * H * dv * 4)
            hip.builtin("mla_attn", [o4] + args[1:], b=B, h=H, dn=dn, dr=dr, kv=kv, dv=dv, maxseq=ms,
                        nsplit=nsplit, wt=wdt, scale=scale, mode=mode, cpb=cpb, oq=1)
            sc = np.tile(suv, B) if f8 else None
            outs.append(("oq", unbf(quarter_x(o4.read(np.float32), sc)).reshape(B, H, dv)))
        for name, got in outs:
            for b in range(B):
                # floor: |olat| <= max_j |ckv_j| per column
                cmax = np.abs(unbf(g_ckv[b, :L])).max(0)
                floor = np.abs(wuvf.reshape(H, dv, kv)) @ cmax
                assert np.all(close_bf16(got[b], unbf(w_o[b]), floor)), \
                    (name, mode, cpb, np.max(np.abs(got[b] - unbf(w_o[b]))))


def quarter_x(o4, scale):
    """bf16(scale * ((q0 + q1) + (q2 + q3))) in f32 over the four quarter sums
    (a GEMV with norm=3 stages exactly this)."""
    q = o4.reshape(4, -1)
    v = ((q[0] + q[1]) + (q[2] + q[3])).astype(np.float32)
    if scale is not None:
        v = (v * scale.astype(np.float32)).astype(np.float32)
    return O.encode(v, DT_BF16)


@pytest.mark.parametrize("wdt,N,K,waves", [(DT_FP8, 2048, 2048, 0), (DT_BF16, 640, 1024, 0),
                                           (DT_FP8, 256, 2048, 16), (DT_FP8, 96, 528, 0)])
def test_gemv_summed_x_equals_staged_bf16(hip, wdt, N, K, waves):
    """A GEMV with norm=3 stages x = bf16(g * ((x0 + x1) + (x2 + x3))) from four
    f32 vectors: bit for bit the plain GEMV over that bf16 row (residual
    epilogue, the o projection's), with and without gains; its limits are
    refused."""
    say(f"case: gemv summed x wdt={wdt} N={N} K={K} waves={waves}")
    rng = np.random.default_rng(N + K + wdt)
    xqs = K + 8
    o4 = np.zeros((4, xqs), np.float32)
    o4[:, :K] = rng.standard_normal((4, K)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    w, sw, _ = weights(rng, N, K, wdt)
    f8 = wdt == DT_FP8
    res = bf(rng.standard_normal((1, N)))
    for gain in (True, False):
        xb = quarter_x(o4[:, :K].copy(), g if gain else None)
        y1, y2 = up(hip, res), up(hip, res)
        tune = dict(waves=waves) if waves else {}
        hip.builtin("gemv", [y1, up(hip, o4), up(hip, w)] + ([up(hip, sw)] if f8 else []) +
                    ([up(hip, g)] if gain else []) + [y1], m=1, n=N, k=K, wt=wdt, xt=DT_BF16, yt=DT_BF16,
                    epi=1, norm=3, xqs=xqs, ngain=int(gain), **tune)
        hip.builtin("gemv", [y2, up(hip, xb), up(hip, w)] + ([up(hip, sw)] if f8 else []) + [y2],
                    m=1, n=N, k=K, wt=wdt, xt=DT_BF16, yt=DT_BF16, epi=1, **tune)
        assert np.array_equal(y1.read(np.uint16), y2.read(np.uint16)), gain
    # one x row only, bf16 staging, K within four elements per thread
    for bad in (dict(m=2), dict(xt=DT_F16), dict(k=K, waves=1)):
        kw = dict(m=1, n=N, k=K, wt=wdt, xt=DT_BF16, yt=DT_BF16, epi=1, norm=3, xqs=xqs, ngain=0)
        kw.update(bad)
        y = hip.Buffer(kw["m"] * N * 2)
        with pytest.raises(Exception):
            hip.builtin("gemv", [y, up(hip, np.zeros((4, xqs * kw["m"]), np.float32)), up(hip, w)] +
                        ([up(hip, sw)] if f8 else []) + [y], **kw)


def test_mla_closed_form_equal_rows(hip):
    """Every live latent row equal: the softmax weights sum to one, so olat is
    that row whatever the scores, and o = W_uv . row (independent of q)."""
    H, dn, dr, kv, dv, B, ms, L = 16, 128, 64, 512, 128, 1, 192, 150
    say("case: mla closed form (equal latent rows)")
    rng = np.random.default_rng(5)
    row = bf(rng.standard_normal(kv))
    ckv = np.tile(row, (B, ms, 1))
    kpe = bf(rng.standard_normal((B, ms, dr)))
    qlat = rng.standard_normal((B, H, kv)).astype(np.float32)
    qpe = bf(rng.standard_normal((B, H, dr)))
    wuv = bf(rng.standard_normal((H * dv, kv)) * 0.02)
    nsplit = 3
    want = (unbf(wuv).astype(np.float64) @ unbf(row).astype(np.float64)).reshape(H, dv)
    floor = (np.abs(unbf(wuv)) @ np.abs(unbf(row))).reshape(H, dv)
    for mode, cpb in mla_splits(H, kv, dr):
        o = hip.Buffer(B * H * dv * 2)
        hip.builtin("mla_attn", [o, up(hip, qlat), up(hip, qpe), up(hip, ckv), up(hip, kpe),
                                 up(hip, np.array([L], np.int32)), hip.Buffer(B * nsplit * H * (kv + 4) * 4),
                                 up(hip, wuv)],
                    b=B, h=H, dn=dn, dr=dr, kv=kv, dv=dv, maxseq=ms, nsplit=nsplit, wt=DT_BF16, scale=0.2,
                    mode=mode, cpb=cpb)
        got = unbf(o.read(np.uint16).reshape(H, dv))
        assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-5 * floor), (mode, cpb)


def test_route_topk_ties_bit_exact(hip):
    B, E, K = 4, 64, 6
    say("case: route top-k with ties")
    rng = np.random.default_rng(11)
    lg = rng.standard_normal((B, E)).astype(np.float32)
    lg[0, [5, 9, 40]] = 3.0          # three-way tie at the top
    lg[1, :] = 1.0                   # all equal: ids 0..K-1
    lg[2, [63, 0]] = 4.0             # tie across the ends
    sel, probs = hip.Buffer(B * K * 4), hip.Buffer(B * K * 4)
    hip.builtin("route", [sel, probs, up(hip, lg)], b=B, e=E, k=K)
    g_sel = sel.read(np.int32).reshape(B, K)
    g_p = probs.read(np.float32).reshape(B, K)
    for b in range(B):
        ws, wp = np.empty(K, np.int32), np.empty(K, np.float32)
        O.oracle().or_route(ws.ctypes.data, wp.ctypes.data, np.ascontiguousarray(lg[b]).ctypes.data, E, K)
        assert np.array_equal(g_sel[b], ws)
        order = np.lexsort((np.arange(E), -lg[b]))[:K]    # brute force: value desc, id asc
        assert np.array_equal(g_sel[b], order)
        assert np.all(np.abs(g_p[b] - wp) <= 1e-6 * np.abs(wp) + 1e-9)
    assert list(g_sel[0, :3]) == [5, 9, 40] and list(g_sel[1]) == list(range(K))
    assert list(g_sel[2, :2]) == [0, 63]
    # signed zeros tie (lowest id first), and fewer experts than lanes
    for E2, K2 in ((64, 6), (20, 4), (3, 3)):
        say(f"case: route zeros E={E2} K={K2}")
        lz = -np.abs(rng.standard_normal((2, E2))).astype(np.float32) - 0.5
        lz[0, [E2 - 1, 1, 0]] = np.array([0.0, -0.0, 0.0], np.float32)
        lz[1, :] = rng.standard_normal(E2).astype(np.float32)
        lz[1, E2 // 2] = lz[1].max()                     # a tie at the top across the middle
        sel2, probs2 = hip.Buffer(2 * K2 * 4), hip.Buffer(2 * K2 * 4)
        hip.builtin("route", [sel2, probs2, up(hip, lz)], b=2, e=E2, k=K2)
        gs = sel2.read(np.int32).reshape(2, K2)
        gp = probs2.read(np.float32).reshape(2, K2)
        for b in range(2):
            ws, wp = np.empty(K2, np.int32), np.empty(K2, np.float32)
            O.oracle().or_route(ws.ctypes.data, wp.ctypes.data, np.ascontiguousarray(lz[b]).ctypes.data, E2, K2)
            assert np.array_equal(gs[b], ws), (E2, b, gs[b], ws)
            assert np.array_equal(gs[b], np.lexsort((np.arange(E2), -lz[b]))[:K2])
            assert np.all(np.abs(gp[b] - wp) <= 1e-6 * np.abs(wp) + 1e-9)
        assert list(gs[0, :3]) == [0, 1, E2 - 1]


@pytest.mark.parametrize("wdt", [DT_FP8, DT_BF16])
@pytest.mark.parametrize("shape", [dict(D=256, E=8, K=3, I=128, S=256, B=2),
                                   dict(D=2048, E=8, K=6, I=1408, S=2816, B=1)], ids=["small", "c5"])
def test_moe_gateup_down(hip, shape, wdt):
    D, E, K, I, S, B = (shape[k] for k in ("D", "E", "K", "I", "S", "B"))
    say(f"case: moe {shape} wdt={wdt}")
    rng = np.random.default_rng(D + E + wdt)
    f8 = wdt == DT_FP8
    wgue, sgue, _ = weights(rng, E * 2 * I, D, wdt)
    wde, sde, _ = weights(rng, E * D, I, wdt)
    wgus, sgus, _ = weights(rng, 2 * S, D, wdt)
    wds, sds, _ = weights(rng, D, S, wdt)
    x = rng.standard_normal((B, D)).astype(np.float32)
    res0 = bf(rng.standard_normal((B, D)))
    sel = np.stack([rng.permutation(E)[:K] for _ in range(B)]).astype(np.int32)
    probs = rng.uniform(0.05, 0.3, (B, K)).astype(np.float32)
    h = hip.Buffer(B * (K * I + S) * 4)
    selb, pb = up(hip, sel), up(hip, probs)
    args = [h, up(hip, x), selb, up(hip, wgue)] + ([up(hip, sgue)] if f8 else []) + \
        [up(hip, wgus)] + ([up(hip, sgus)] if f8 else [])
    hip.builtin("moe_gateup", args, b=B, d=D, e=E, k=K, i=I, s=S, wt=wdt)
    res = up(hip, res0)
    args = [res, h, selb, pb, up(hip, wde)] + ([up(hip, sde)] if f8 else []) + \
        [up(hip, wds)] + ([up(hip, sds)] if f8 else [])
    hip.builtin("moe_down", args, b=B, d=D, e=E, k=K, i=I, s=S, wt=wdt)
    got = unbf(res.read(np.uint16).reshape(B, D))
    for b in range(B):
        out = np.empty(D, np.float32)
        xb = bf(x[b])
        O.oracle().or_moe(out.ctypes.data, xb.ctypes.data, np.ascontiguousarray(sel[b]).ctypes.data,
                          np.ascontiguousarray(probs[b]).ctypes.data, wgue.ctypes.data,
                          sgue.ctypes.data if f8 else None, wde.ctypes.data,
                          sde.ctypes.data if f8 else None, wgus.ctypes.data,
                          sgus.ctypes.data if f8 else None, wds.ctypes.data,
                          sds.ctypes.data if f8 else None, wdt, D, I, S, K)
        r = unbf(res0[b])
        want = unbf(bf(r + unbf(bf(out))))
        # each step of the chain within one bf16 rounding of the oracle's
        tol = 2.0 ** -7 * (np.abs(want) + np.abs(out)) + 1e-4 * np.abs(out).max() + 1e-6
        assert np.all(np.abs(got[b] - want) <= tol), np.max(np.abs(got[b] - want) - tol)


def run_moe(hip, grouped, B, D, E, K, I, S, wdt, x, sel, probs, res0, w):
    """One gate/up + down through the builtins; returns (h, res, live)."""
    f8 = wdt == DT_FP8
    wgue, sgue, wde, sde, wgus, sgus, wds, sds = w
    h = hip.Buffer(B * (K * I + S) * 4)
    selb, pb = up(hip, sel), up(hip, probs)
    extra_gu, extra_dn, live = [], [], None
    if grouped:                     # 1: VALU grouped kernels, 2: MFMA
        plan = hip.Buffer((E + E * B * K) * 4)
        live = up(hip, np.zeros(1, np.int32))
        part = hip.Buffer((B * K * D + B * D) * 4)
        extra_gu, extra_dn = [plan, live], [plan, part]
    args = [h, up(hip, x), selb, up(hip, wgue)] + ([up(hip, sgue)] if f8 else []) + \
        [up(hip, wgus)] + ([up(hip, sgus)] if f8 else []) + extra_gu
    hip.builtin("moe_gateup", args, b=B, d=D, e=E, k=K, i=I, s=S, wt=wdt, grouped=int(grouped))
    res = up(hip, res0)
    args = [res, h, selb, pb, up(hip, wde)] + ([up(hip, sde)] if f8 else []) + \
        [up(hip, wds)] + ([up(hip, sds)] if f8 else []) + extra_dn
    hip.builtin("moe_down", args, b=B, d=D, e=E, k=K, i=I, s=S, wt=wdt, grouped=int(grouped))
    return (h.read(np.float32), res.read(np.uint16),
            int(live.read(np.int32)[0]) if grouped else None)


@pytest.mark.parametrize("wdt", [DT_FP8, DT_BF16])
@pytest.mark.parametrize("shape", [dict(D=256, E=8, K=3, I=128, S=256, B=32),
                                   dict(D=2048, E=16, K=6, I=1408, S=2816, B=8)], ids=["small", "c5"])
def test_moe_grouped_equals_per_row(hip, shape, wdt):
    """The expert-grouped MoE (each live expert streamed once for all its rows)
    against the per-row kernels on the same routing: h and the residual
    output bit for bit.  The routing is skewed so that one expert takes more
    than one 8-row staging pass and some experts take none."""
    D, E, K, I, S, B = (shape[k] for k in ("D", "E", "K", "I", "S", "B"))
    say(f"case: grouped moe {shape} wdt={wdt}")
    rng = np.random.default_rng(7 * D + E + wdt)
    w = weights(rng, E * 2 * I, D, wdt)[:2] + weights(rng, E * D, I, wdt)[:2] + \
        weights(rng, 2 * S, D, wdt)[:2] + weights(rng, D, S, wdt)[:2]
    x = rng.standard_normal((B, D)).astype(np.float32)
    res0 = bf(rng.standard_normal((B, D)))
    pool = np.arange(E // 2)                      # experts E/2.. never chosen
    sel = np.stack([np.concatenate([[0], rng.permutation(pool[1:])[:K - 1]]) for _ in range(B)]).astype(np.int32)
    probs = rng.uniform(0.05, 0.3, (B, K)).astype(np.float32)
    h0, r0, _ = run_moe(hip, False, B, D, E, K, I, S, wdt, x, sel, probs, res0, w)
    h1, r1, live = run_moe(hip, True, B, D, E, K, I, S, wdt, x, sel, probs, res0, w)
    assert np.array_equal(h0.view(np.uint32), h1.view(np.uint32)), "gate/up outputs differ"
    assert np.array_equal(r0, r1), "residual outputs differ"
    assert live == len(np.unique(sel)), (live, len(np.unique(sel)))


@pytest.mark.parametrize("wdt", [DT_FP8, DT_BF16])
@pytest.mark.parametrize("shape", [dict(D=256, E=8, K=3, I=128, S=256, B=40),
                                   dict(D=2048, E=16, K=6, I=1408, S=2816, B=32),
                                   dict(D=2048, E=16, K=6, I=1408, S=2816, B=8)],
                         ids=["small_b40", "c5_b32", "c5_b8"])
def test_moe_mfma_close_to_per_row(hip, shape, wdt):
    """The expert-grouped MoE on MFMA (grouped=2) against the per-row kernels
    on the same routing.  Gate/up: the same bf16-rounded x against the same
    exactly decoded weights, only the f32 summation order differs, so h agrees
    to 1e-4 relative (of the row's largest |h|).  Down: h enters as bf16 hi +
    lo (about 16 significant bits).  The residual output is
    bf16(res + bf16(acc)): a near-tie of either rounding may flip one bf16
    ulp of acc or of the result, so it is bounded by 2^-6 (|res| + |out|)
    and almost all entries are equal.  Expert 0 takes every row (two column
    tiles at 32 rows, two column groups at 40), half the experts none."""
    D, E, K, I, S, B = (shape[k] for k in ("D", "E", "K", "I", "S", "B"))
    say(f"case: mfma moe {shape} wdt={wdt}")
    rng = np.random.default_rng(11 * D + E + wdt + B)
    w = weights(rng, E * 2 * I, D, wdt)[:2] + weights(rng, E * D, I, wdt)[:2] + \
        weights(rng, 2 * S, D, wdt)[:2] + weights(rng, D, S, wdt)[:2]
    x = rng.standard_normal((B, D)).astype(np.float32)
    res0 = bf(rng.standard_normal((B, D)))
    pool = np.arange(E // 2)
    sel = np.stack([np.concatenate([[0], rng.permutation(pool[1:])[:K - 1]]) for _ in range(B)]).astype(np.int32)
    probs = rng.uniform(0.05, 0.3, (B, K)).astype(np.float32)
    h0, r0, _ = run_moe(hip, 0, B, D, E, K, I, S, wdt, x, sel, probs, res0, w)
    h2, r2, live = run_moe(hip, 2, B, D, E, K, I, S, wdt, x, sel, probs, res0, w)
    P = K * I + S
    h0, h2 = h0.reshape(B, P), h2.reshape(B, P)
    scale = np.abs(h0).max(axis=1, keepdims=True)
    err = np.abs(h2 - h0) / scale
    assert err.max() <= 1e-4, f"h: max relative error {err.max():.3g}"
    f0, f2, fr = unbf(r0), unbf(r2), unbf(res0).reshape(-1)
    bound = 2.0 ** -6 * (np.abs(fr) + np.abs(f0)) + 1e-6
    assert (np.abs(f2 - f0) <= bound).all(), f"residual: max diff {np.abs(f2 - f0).max():.3g}"
    assert (r0 == r2).mean() >= 0.95, f"residual: only {(r0 == r2).mean():.3f} equal"
    assert live == len(np.unique(sel)), (live, len(np.unique(sel)))


@pytest.mark.parametrize("M", [8, 32])
def test_gemv_f32_row_chunks(hip, M):
    """M > 4 rows with f32 operands (the DSV2 router at batch 32) run the GEMV
    in chunks of 4 rows: every output equals an M=4 launch on that chunk."""
    N, K = 64, 2048
    say(f"case: f32 gemv row chunks M={M}")
    rng = np.random.default_rng(M)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wb, xb = up(hip, w), up(hip, x)
    y = hip.Buffer(M * N * 4)
    hip.builtin("gemv", [y, xb, wb], m=M, n=N, k=K, wt=DT_F32, xt=DT_F32, yt=DT_F32)
    got = y.read(np.float32).reshape(M, N)
    for m0 in range(0, M, 4):
        y4 = hip.Buffer(4 * N * 4)
        hip.builtin("gemv", [y4, up(hip, x[m0:m0 + 4]), wb], m=4, n=N, k=K, wt=DT_F32, xt=DT_F32, yt=DT_F32)
        assert np.array_equal(got[m0:m0 + 4].view(np.uint32), y4.read(np.float32).reshape(4, N).view(np.uint32))
    assert np.allclose(got, x.astype(np.float64) @ w.T.astype(np.float64), rtol=1e-4, atol=1e-4)


DSV2 = dict(arch=3, n_layers=3, dim=256, n_heads=8, n_kv_heads=8, head_dim=48, ffn=512,
            vocab=512, max_seq=128, eps=1e-6, rope_theta=10000.0, init_std=0.02, kv_lora=64,
            d_nope=32, d_rope=16, d_v=32, n_experts=8, n_shared=2, top_k=3, moe_inter=64,
            first_dense=1, adtype=DT_BF16)


@pytest.mark.parametrize("wdt,batch", [(DT_FP8, 1), (DT_FP8, 2), (DT_BF16, 1), (DT_FP8, 8), (DT_BF16, 8)])
def test_dsv2_decoder_parity(hip, wdt, batch):
    """The DSV2 decoder (1 dense + 2 MoE layers at the reference's CPU smoke
    shape) against or_dsv2_step, teacher-forced: every MoE layer's routing
    equal or a proven near tie, logits at the bar, ids equal or a near tie;
    then eager and captured runs bit-identical.  Batch 8 runs the batched
    path (MFMA projections, expert-grouped MoE, chunked f32 router)."""
    from test_gpu_decoder import run_parity
    run_parity(hip, dict(DSV2, wdtype=wdt, batch=batch), steps=5, ctx=20, seed=21)


def test_mla_split_mode_errors(hip):
    """mla_attn rejects the MFMA split outside the shape it is built for, and
    chunk counts it has no kernel for."""
    H, dn, dr, kv, dv, B, ms = 8, 32, 16, 64, 32, 1, 128
    args = [hip.Buffer(B * H * dv * 2), hip.Buffer(B * H * kv * 4), hip.Buffer(B * H * dr * 2),
            hip.Buffer(B * ms * kv * 2), hip.Buffer(B * ms * dr * 2), up(hip, np.array([5], np.int32)),
            hip.Buffer(B * 2 * H * (kv + 4) * 4), hip.Buffer(H * dv * kv * 2)]
    for bad in (dict(mode=2), dict(mode=3), dict(mode=1, cpb=2)):
        with pytest.raises(hip.ThvmHipError):
            hip.builtin("mla_attn", args, b=B, h=H, dn=dn, dr=dr, kv=kv, dv=dv, maxseq=ms, nsplit=2,
                        wt=DT_BF16, scale=0.2, **bad)


def test_moe_mfma_matches_oracle_at_c5_geometry(hip):
    """The default C5 batch-32 MoE -- expert-grouped, on MFMA -- against the
    oracle's per-row or_moe at the C5 geometry: 64 experts, top-6, I 1408,
    2 shared experts (S 2816), D 2048, fp8 weights, 32 rows routed at random
    (every row 6 distinct experts; about 50 experts live).  Bar: the north
    star's fp8 tolerance, 2e-2 of the row's largest |MoE output|, on the
    residual output bf16(res + bf16(moe)); and each element within 2^-6
    (|res| + |moe|) of the oracle chain, the bf16 roundings' reach."""
    D, E, K, I, S, B = 2048, 64, 6, 1408, 2816, 32
    say("case: mfma moe vs or_moe at E=64 K=6 I=1408 B=32")
    rng = np.random.default_rng(64)

    def f8w(rows, cols):                 # random e4m3 codes (no NaN), per-row scales
        q = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        q[(q & 0x7F) == 0x7F] = 0
        return q, rng.uniform(0.5, 1.5, rows).astype(np.float32) * 1e-4
    wgue, sgue = f8w(E * 2 * I, D)
    wde, sde = f8w(E * D, I)
    wgus, sgus = f8w(2 * S, D)
    wds, sds = f8w(D, S)
    w = (wgue, sgue, wde, sde, wgus, sgus, wds, sds)
    x = rng.standard_normal((B, D)).astype(np.float32)
    res0 = bf(rng.standard_normal((B, D)))
    sel = np.stack([rng.permutation(E)[:K] for _ in range(B)]).astype(np.int32)
    probs = rng.uniform(0.05, 0.3, (B, K)).astype(np.float32)
    _, r2, live = run_moe(hip, 2, B, D, E, K, I, S, DT_FP8, x, sel, probs, res0, w)
    assert live == len(np.unique(sel))
    got = unbf(r2).reshape(B, D)
    for b in range(B):
        out = np.empty(D, np.float32)
        xb, sb, pb = bf(x[b]), np.ascontiguousarray(sel[b]), np.ascontiguousarray(probs[b])   # kept alive
        O.oracle().or_moe(out.ctypes.data, xb.ctypes.data, sb.ctypes.data, pb.ctypes.data,
                          wgue.ctypes.data, sgue.ctypes.data,
                          wde.ctypes.data, sde.ctypes.data, wgus.ctypes.data, sgus.ctypes.data,
                          wds.ctypes.data, sds.ctypes.data, DT_FP8, D, I, S, K)
        r = unbf(res0[b])
        want = unbf(bf(r + unbf(bf(out))))
        err = np.abs(got[b] - want)
        assert err.max() <= 2e-2 * np.abs(out).max(), (b, err.max(), np.abs(out).max())
        assert (err <= 2.0 ** -6 * (np.abs(r) + np.abs(out)) + 1e-6).all(), b


@pytest.mark.parametrize("B,D,E,K", [(1, 2048, 64, 6), (32, 2048, 64, 6), (3, 4096, 64, 8),
                                     (2, 512, 8, 3), (1, 1008, 20, 4)])
def test_moe_gate_and_gateup_routing_equal_the_split_kernels(hip, B, D, E, K):
    """The one-launch gate (RMSNorm f32 out + f32 router GEMV) is bit for bit
    the norm and GEMV kernels (xn, logits); the top-K picked inside the
    per-row gate/up (route=1) is the route kernel's (ids, probabilities) and
    so is the gate/up output.  One row's logits tie at the top (two equal
    router rows) to hold the lowest-id rule."""
    say(f"case: moe_gate B={B} D={D} E={E} K={K}")
    rng = np.random.default_rng(B * D + E)
    x = bf(rng.standard_normal((B, D)))
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    gate = (rng.standard_normal((E, D)) * 0.05).astype(np.float32)
    gate[E - 1] = gate[1]                               # a tie between experts 1 and E-1
    xb, gb, wb = up(hip, x), up(hip, g), up(hip, gate)
    I, S = 64, 128
    wgue, sgue, _ = fp8_rows(rng, E * 2 * I, D)
    wgus, sgus, _ = fp8_rows(rng, 2 * S, D)
    wg = [up(hip, wgue), up(hip, sgue), up(hip, wgus), up(hip, sgus)]
    outs = []
    for fused in (True, False):
        xn, lg = hip.Buffer(B * D * 4), hip.Buffer(B * E * 4)
        sel, pr = hip.Buffer(B * K * 4), hip.Buffer(B * K * 4)
        h = hip.Buffer(B * (K * I + S) * 4)
        kw = dict(b=B, d=D, e=E, k=K, i=I, s=S, wt=DT_FP8)
        if fused:
            hip.builtin("moe_gate", [xn, lg, xb, gb, wb], outs=(0, 1), b=B, d=D, e=E, eps=1e-6)
            hip.builtin("moe_gateup", [h, xn, sel] + wg[:2] + wg[2:] + [lg, pr], outs=(0, 2, 6),
                        route=1, **kw)
        else:
            hip.builtin("norm", [xn, xb, gb], m=B, k=D, xt=DT_BF16, yt=DT_F32, eps=1e-6)
            hip.builtin("gemv", [lg, xn, wb], m=B, n=E, k=D, wt=DT_F32, xt=DT_F32, yt=DT_F32, epi=0)
            hip.builtin("route", [sel, pr, lg], outs=(0, 1), b=B, e=E, k=K)
            hip.builtin("moe_gateup", [h, xn, sel] + wg, **kw)
        outs.append([b.read(np.uint32) for b in (xn, lg, sel, pr, h)])
    for name, f, s in zip(("xn", "logits", "sel", "probs", "h"), outs[0], outs[1]):
        assert np.array_equal(f, s), name
    assert np.isfinite(outs[0][1].view(np.float32)).all()
