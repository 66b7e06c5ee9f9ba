"""Full-depth parity by per-sublayer teacher forcing, at the BASELINE configs'
real shapes and depths: C3 (48 layers fp16, batch 1 and 8), C4 (32 layers
fp8, batch 1 and 16, context 2048) and C5 (27 layers fp8 MLA + MoE, batch 1
and 32, context 4096).

One eager device step runs a sublayer at a time (Decoder.step_probed: the
same kernels the captured step replays); after every sublayer the device's
residual and that sublayer's intermediates are read back.  The oracle then
runs the same step with each sublayer restarted from the device's residual
at its input (OrModel / OrDsv2 tf_x) and, for DeepSeek-V2, with the device's
routing (tf_sel / tf_probs).  Every sublayer's outputs therefore come from
identical inputs on both sides and are held to the north-star bars, layer
by layer, with no accumulated drift:

  * fp8 weights (C4, C5): every residual, q, attention output, FFN hidden
    and the logits within 2e-2 relative (max |diff| / max |oracle|);
  * fp16 (C3): within 1e-2 absolute, or one fp16 rounding of the value
    where an fp16 ulp exceeds 1e-2 (|x| >= 16: the residual is stored in
    fp16, so a value one ulp away is the closest the storage allows);
  * embedding rows bit-exact;
  * DeepSeek-V2 routing: the device's router logits within the f32 GEMV
    bar (1e-5 of sum |x||w| per expert) of the oracle's on the same router
    input; the device's experts bit-exact with the oracle's top-K (or_route)
    applied to the device's router logits, and their f32 softmax weights
    within 1e-5 relative of or_route's.

End to end, the free-running oracle step (no forcing) gives the greedy ids:
the device's ids equal them, or differ only at a proven near tie (the
oracle's logit margin within twice the logit drift); at batch 1 two steps
run.  The free-running logit distance at full depth is printed, not held
(16-bit rounding points between 27-48 layers make two correct f32
summation orders drift apart; the per-sublayer checks above are the bar)."""
import numpy as np
import pytest

import _oracle as O
import _parity as P

pytestmark = pytest.mark.gpu

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13

C3 = dict(arch=2, n_layers=48, dim=1600, n_heads=25, n_kv_heads=25, head_dim=64, ffn=6400,
          vocab=50257, wdtype=DT_F16, adtype=DT_F16, eps=1e-5, init_std=0.02)
C4 = dict(arch=1, n_layers=32, dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
          vocab=128256, wdtype=DT_FP8, adtype=DT_BF16, eps=1e-5, rope_theta=500000.0,
          init_std=0.02)
C5 = dict(arch=3, n_layers=27, dim=2048, n_heads=16, n_kv_heads=16, head_dim=192, ffn=10944,
          vocab=102400, wdtype=DT_FP8, adtype=DT_BF16, eps=1e-6, rope_theta=10000.0,
          init_std=0.02, kv_lora=512, d_nope=128, d_rope=64, d_v=128, n_experts=64, n_shared=2,
          top_k=6, moe_inter=1408, first_dense=1)

say = P.say


def _f32(a, dt):
    if dt == DT_F32:
        return a.astype(np.float32)
    return O.decode(a, dt)


class Bars:
    """The north-star bar of the config, applied tensor by tensor."""

    def __init__(self, cfg):
        self.adt = cfg["adtype"]
        self.kind, self.tol = P.logit_bar(cfg)
        self.worst = {}

    def check(self, what, dev, ref, where):
        dev = np.asarray(dev, np.float64)
        ref = np.asarray(ref, np.float64)
        assert dev.shape == ref.shape, (what, dev.shape, ref.shape)
        assert np.all(np.isfinite(dev)), f"{where} {what}: non-finite device values"
        d = np.abs(dev - ref)
        if self.kind == "rel":
            e = float(d.max() / max(np.abs(ref).max(), 1e-30))
            ok = e <= self.tol
        else:                           # 16-bit absolute, or one storage rounding where larger
            ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) \
                if self.adt == DT_F16 else 0.0
            e = float(d.max())
            ok = bool(np.all(d <= np.maximum(self.tol, ulp)))
        w = self.worst.get(what)
        if w is None or e > w[0]:
            self.worst[what] = (e, where)
        assert ok, f"{where} {what}: {self.kind} err {e:.4g} > bar {self.tol}"

    def report(self, label):
        for k, (e, where) in sorted(self.worst.items()):
            say(f"  {label}: worst {k:10s} {self.kind} err {e:.3g} at {where} (bar {self.tol})")


def _reads(cfg):
    arch, first_dense = cfg["arch"], cfg.get("first_dense", 0)

    def reads(tag):
        if tag < 0:
            return ["x"]
        l, sub = divmod(tag, 2)
        if arch == 3:
            if sub == 0:
                # one row: the MLA merge in latent quarters leaves four f32
                # quarter sums (the o projection adds, scales and rounds them)
                if _quarters(cfg):
                    return ["x", "o4"] + ([f"l{l}.wuv.scale"] if cfg.get("wdtype", DT_FP8) == DT_FP8 else [])
                return ["x", "o"]
            return ["x"] if l < first_dense else ["x", "xnf", f"l{l}.gate_logits", f"l{l}.sel", f"l{l}.probs"]
        return ["x", "q", "att"] if sub == 0 else ["x", "h"]
    return reads


def _quarters(cfg):
    """Whether the DSV2 decoder runs the MLA merge in latent quarters."""
    return cfg["batch"] == 1 and cfg["kv_lora"] % 64 == 0


def _mla_o(r, cfg, l):
    """The attention output the o projection consumes: read as is, or, from
    the quarter sums, bf16(scale * ((q0 + q1) + (q2 + q3))) in f32 -- the
    GEMV's staging."""
    B = cfg["batch"]
    if "o4" not in r:
        return _f32(r["o"], DT_BF16).reshape(B, -1)
    q = r["o4"].view(np.float32).reshape(4, -1)
    v = ((q[0] + q[1]) + (q[2] + q[3])).astype(np.float32)
    sc = r.get(f"l{l}.wuv.scale")
    if sc is not None:
        v = (v * sc.view(np.float32)).astype(np.float32)
    return _f32(O.encode(v, DT_BF16), DT_BF16).reshape(B, -1)


def _device_step(dec, cfg, tok, pos):
    """One probed device step: {tag: {name: array}}, logits, next ids."""
    B = cfg["batch"]
    got = {}
    dec.set_state(tok, pos)
    dec.step_probed(_reads(cfg), lambda t, arrs: got.__setitem__(t, arrs))
    return got, dec.logits(), dec.tokens(pos + 2)[:, pos + 1].copy()


def _teacher(dec, om, cfg, tok, pos, bars, label):
    """Device step + teacher-forced oracle step; every sublayer to the bar."""
    B, D, L, adt = cfg["batch"], cfg["dim"], cfg["n_layers"], cfg["adtype"]
    got, glg, gnx = _device_step(dec, cfg, tok, pos)
    assert np.array_equal(gnx, np.argmax(glg, 1)), "device argmax != host argmax"
    xs = np.stack([_f32(got[t]["x"], adt).reshape(B, D) for t in [-1] + list(range(2 * L))])
    # the embedding row, bit for bit
    if cfg["arch"] == 2:
        emb = _f32(dec.read_tensor("wte"), adt).reshape(-1, D)[tok] + \
            _f32(dec.read_tensor("wpe"), adt).reshape(-1, D)[pos][None, :]
        emb = _f32(O.encode(emb.astype(np.float32), adt), adt) if adt != DT_F32 else emb
    else:
        emb = _f32(dec.read_tensor("emb"), adt).reshape(-1, D)[tok]
    assert np.array_equal(xs[0], emb.astype(np.float32)), f"{label}: embedding rows differ"

    kw = {}
    if cfg["arch"] == 3:
        K, E = cfg["top_k"], cfg["n_experts"]
        tsel = np.zeros((L, B, K), np.int32)
        tprob = np.zeros((L, B, K), np.float32)
        for l in range(cfg["first_dense"], L):
            r = got[2 * l + 1]
            tsel[l] = r[f"l{l}.sel"].reshape(B, K)
            tprob[l] = r[f"l{l}.probs"].reshape(B, K)
        kw = dict(tf_sel=tsel, tf_probs=tprob)
    olg, onx = om.step(tok, pos, tf_x=xs, **kw)
    tp = om.taps
    for t in range(2 * L):
        l, sub = divmod(t, 2)
        where = f"{label} pos {pos} layer {l} {'attn' if sub == 0 else 'ffn'}"
        bars.check("x." + ("attn" if sub == 0 else "ffn"), xs[t + 1], tp["x"][t], where)
        r = got[t]
        if cfg["arch"] == 3:
            if sub == 0:
                bars.check("o", _mla_o(r, cfg, l), tp["o"][l], where)
            elif l >= cfg["first_dense"]:
                _check_routing(dec, cfg, r, om, l, where)
        elif sub == 0:
            bars.check("q", _f32(r["q"], adt).reshape(B, -1), tp["q"][l], where)
            bars.check("att", _f32(r["att"], adt).reshape(B, -1), tp["att"][l], where)
        else:
            bars.check("h", _f32(r["h"], adt).reshape(B, -1), tp["h"][l], where)
    bars.check("logits", glg, olg, f"{label} pos {pos} LM head")
    return glg, gnx


def _check_routing(dec, cfg, r, om, l, where):
    """Router logits to the f32 GEMV bar on the same input; the device's
    routing equal to the oracle's top-K of the device's logits, bit for bit."""
    B, K, E, D = cfg["batch"], cfg["top_k"], cfg["n_experts"], cfg["dim"]
    gl = r[f"l{l}.gate_logits"].reshape(B, E)
    xnf = r["xnf"].reshape(B, D).astype(np.float64)
    gw = np.abs(dec.read_tensor(f"l{l}.gate").reshape(E, D).astype(np.float64))
    mag = np.abs(xnf) @ gw.T                                   # sum_k |x_k||w_ek|
    d = np.abs(gl.astype(np.float64) - om.gate[l].astype(np.float64))
    assert np.all(d <= 1e-5 * mag + 1e-30), f"{where}: router logits off by {float((d / mag).max()):.3g} of sum|x||w|"
    sel, probs = r[f"l{l}.sel"].reshape(B, K), r[f"l{l}.probs"].reshape(B, K)
    for b in range(B):
        s = np.empty(K, np.int32)
        p = np.empty(K, np.float32)
        g = np.ascontiguousarray(gl[b], np.float32)
        O.oracle().or_route(s.ctypes.data, p.ctypes.data, g.ctypes.data, E, K)
        assert np.array_equal(s, sel[b]), f"{where} row {b}: experts {sel[b]} vs or_route {s}"
        # the weights are f32 softmax values (the sum's order differs): the f32 bar
        assert np.all(np.abs(probs[b] - p) <= 1e-5 * np.abs(p)), f"{where} row {b}: weights {probs[b]} vs {p}"


def _ids_end_to_end(glg, gnx, olg, onx, cfg, label):
    drift_all = []
    for b in range(cfg["batch"]):
        drift = float(np.abs(glg[b].astype(np.float64) - olg[b]).max())
        drift_all.append(drift / float(np.abs(olg[b]).max()))
        if gnx[b] != onx[b]:
            margin = float(olg[b][onx[b]] - olg[b][gnx[b]])
            say(f"  {label} row {b}: id {gnx[b]} vs oracle {onx[b]}, margin {margin:.3g} drift {drift:.3g}")
            assert margin <= 2 * drift, f"{label} row {b}: id fork margin {margin} > 2 x drift {drift}"
    return int(np.sum(gnx != onx)), max(drift_all)


def _run(hip, cfg, seed, ctx, steps, label):
    say(f"case: {label}: layers={cfg['n_layers']} batch={cfg['batch']} ctx={ctx}")
    dec = hip.Decoder(seed=seed, **cfg)
    try:
        if ctx:
            dec.prefill_synthetic(ctx, seed=seed + 1)
        say(f"  {label}: reading the weights back for the oracle")
        om = O.OracleDsv2(dec, cfg) if cfg["arch"] == 3 else O.OracleModel(dec, cfg)
        bars = Bars(cfg)
        tok = np.random.default_rng(seed).integers(0, cfg["vocab"], cfg["batch"]).astype(np.int32)
        for s in range(steps):
            pos = ctx + s
            # free-running oracle first (end-to-end ids), then the teacher-forced
            # step, whose k/v rows at pos are the ones kept in the oracle's caches
            olg_free, onx_free = om.step(tok, pos)
            glg, gnx = _teacher(dec, om, cfg, tok, pos, bars, label)
            forks, drift = _ids_end_to_end(glg, gnx, olg_free, onx_free, cfg, f"{label} pos {pos}")
            say(f"  {label} pos {pos}: sublayers within the bar; end to end: {forks} id forks at "
                f"near ties, free-running logit drift {drift:.3g} of max|logit|")
            tok = onx_free.astype(np.int32)
        bars.report(label)
    finally:
        dec.close()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("batch", [1, 16])
def test_c4_full_depth_per_sublayer(hip, batch):
    cfg = dict(C4, batch=batch, max_seq=2056)
    _run(hip, cfg, 1234 + batch, 2048, 2 if batch == 1 else 1, f"C4 B={batch}")


@pytest.mark.timeout(900)
@pytest.mark.parametrize("batch", [1, 8])
def test_c3_full_depth_per_sublayer(hip, batch):
    cfg = dict(C3, batch=batch, max_seq=136)
    _run(hip, cfg, 1234 + batch, 128, 2 if batch == 1 else 1, f"C3 B={batch}")


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("batch", [1, 32])
def test_c5_full_depth_per_sublayer(hip, batch):
    cfg = dict(C5, batch=batch, max_seq=4104)
    _run(hip, cfg, 1234 + batch, 4096, 2 if batch == 1 else 1, f"C5 B={batch}")


SMALL = [
    ("llama fp8 B=1", dict(arch=1, n_layers=3, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512,
                           vocab=500, wdtype=DT_FP8, adtype=DT_BF16, eps=1e-5, rope_theta=500000.0,
                           init_std=0.02, batch=1, max_seq=96), 70),
    ("llama fp8 B=6", dict(arch=1, n_layers=3, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512,
                           vocab=500, wdtype=DT_FP8, adtype=DT_BF16, eps=1e-5, rope_theta=500000.0,
                           init_std=0.02, batch=6, max_seq=96), 70),
    ("gpt2 fp16 B=1", dict(arch=2, n_layers=3, dim=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn=1024,
                           vocab=500, wdtype=DT_F16, adtype=DT_F16, eps=1e-5, init_std=0.02, batch=1,
                           max_seq=48), 20),
    ("gpt2 f32 B=2", dict(arch=2, n_layers=3, dim=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn=1024,
                          vocab=500, wdtype=DT_F32, adtype=DT_F32, eps=1e-5, init_std=0.02, batch=2,
                          max_seq=48), 20),
    ("dsv2 fp8 B=1", dict(C5, n_layers=3, dim=512, vocab=700, n_experts=16, moe_inter=256, ffn=1024,
                          batch=1, max_seq=200), 150),
    ("dsv2 fp8 B=8", dict(C5, n_layers=3, dim=512, vocab=700, n_experts=16, moe_inter=256, ffn=1024,
                          batch=8, max_seq=200), 150),
]


@pytest.mark.parametrize("label,cfg,ctx", SMALL, ids=[s[0] for s in SMALL])
def test_small_models_per_sublayer(hip, label, cfg, ctx):
    """The same per-sublayer checks on small models of each architecture and
    path (GEMV at batch 1, MFMA GEMM / grouped MoE above 4 rows, f32)."""
    _run(hip, cfg, 99, ctx, 2, label)
