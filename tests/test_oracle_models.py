"""Pin the oracle's whole decode step (oracle/oracle.c or_decode_step, LLAMA
and GPT2) against the independent float64 restatement in _llama_ref.py
(CPU only).

The op-level pins in test_oracle.py cannot see a composition mistake (a
wrong GQA head map, RoPE pairing, residual placement or norm position).
Here the two step implementations run on the same seeded weights:

  * with the decode chain's storage rounding on both sides, the logits
    agree to the level of f32-vs-f64 summation differences;
  * a planted composition mistake in the float64 model (swapped RoPE
    pairing, a wrong head map, a missing residual, the norm after instead
    of before) moves the logits by far more than that, so the check would
    catch the same mistake in the oracle."""
import ctypes as C

import numpy as np
import pytest

import _llama_ref as LR
import _oracle as O

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13


class _Tensors:
    def __init__(self, t):
        self.t = t

    def read_tensor(self, name):
        return self.t[name]


def _enc(a, dt):
    if dt == DT_F32:
        return np.ascontiguousarray(a, np.float32)
    return O.encode(np.asarray(a, np.float32), dt)


def _dec(a, dt):
    if dt == DT_F32:
        return np.asarray(a, np.float64)
    return O.decode(a, dt).astype(np.float64)


def _weight(rng, rows, cols, wdt, std=0.02):
    """(stored, scale or None, dequantised float64)."""
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    if wdt == DT_FP8:
        s = (np.abs(w).max(1) / 448.0).astype(np.float32)
        q = O.encode(w / s[:, None], DT_FP8)
        return q, s, O.decode(q, DT_FP8).astype(np.float64) * s[:, None].astype(np.float64)
    q = _enc(w, wdt)
    return q, None, _dec(q, wdt)


def llama_model(cfg, seed, ctx):
    """Seeded Llama weights and a KV cache prefilled to ctx rows, as oracle
    tensors (device layouts) and as float64 LlamaRef weights."""
    rng = np.random.default_rng(seed)
    D, H, Hkv, hd, F, V = (cfg[k] for k in ("dim", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab"))
    ms, wdt, adt = cfg["max_seq"], cfg["wdtype"], cfg["adtype"]
    t, ref = {}, {"layers": []}
    emb = _enc(rng.standard_normal((V, D)) * 0.02, adt)
    t["emb"], ref["emb"] = emb, _dec(emb, adt)
    for l in range(cfg["n_layers"]):
        p = f"l{l}."
        wq, sq, fq = _weight(rng, H * hd, D, wdt)
        wk, sk, fk = _weight(rng, Hkv * hd, D, wdt)
        wv, sv, fv = _weight(rng, Hkv * hd, D, wdt)
        wo, so, fo = _weight(rng, D, H * hd, wdt)
        wg, sg, fg = _weight(rng, F, D, wdt)
        wu, su, fu = _weight(rng, F, D, wdt)
        wd, sd, fd = _weight(rng, D, F, wdt)
        t[p + "wqkv"] = np.concatenate([wq, wk, wv])
        gu = np.empty((2 * F, D), wg.dtype)
        gu[0::2], gu[1::2] = wg, wu
        t[p + "wgu"], t[p + "wo"], t[p + "wd"] = gu, wo, wd
        if wdt == DT_FP8:
            t[p + "wqkv.scale"] = np.concatenate([sq, sk, sv])
            sgu = np.empty(2 * F, np.float32)
            sgu[0::2], sgu[1::2] = sg, su
            t[p + "wgu.scale"], t[p + "wo.scale"], t[p + "wd.scale"] = sgu, so, sd
        g1 = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        g2 = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        t[p + "g_attn"], t[p + "g_ffn"] = g1, g2
        kc = _enc(rng.standard_normal((1, Hkv, ms, hd)), adt)
        vc = _enc(rng.standard_normal((1, Hkv, ms, hd)), adt)
        kc[:, :, ctx:] = 0
        vc[:, :, ctx:] = 0
        t[p + "kcache"], t[p + "vcache"] = kc, vc
        ref["layers"].append(dict(wq=fq, wk=fk, wv=fv, wo=fo, wg=fg, wu=fu, wd=fd,
                                  g1=g1.astype(np.float64), g2=g2.astype(np.float64),
                                  k=_dec(kc[0], adt), v=_dec(vc[0], adt)))
    gf = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    lm, slm, flm = _weight(rng, V, D, wdt)
    t["norm_f"], t["lm"] = gf, lm
    if wdt == DT_FP8:
        t["lm.scale"] = slm
    ref["gf"], ref["lm"] = gf.astype(np.float64), flm
    # the device's RoPE tables: f32 cos/sin of pos * theta^(-2j/hd)
    ang = np.arange(ms)[:, None] * cfg["rope_theta"] ** (-np.arange(0, hd, 2) / hd)
    t["rope.cos"] = np.cos(ang).astype(np.float32)
    t["rope.sin"] = np.sin(ang).astype(np.float32)
    return t, ref


def gpt2_model(cfg, seed):
    rng = np.random.default_rng(seed)
    D, H, hd, F, V = (cfg[k] for k in ("dim", "n_heads", "head_dim", "ffn", "vocab"))
    ms, wdt, adt = cfg["max_seq"], cfg["wdtype"], cfg["adtype"]
    t, ref = {}, {"layers": []}

    def vec(n, base=0.0, std=0.02):
        a = _enc(base + rng.standard_normal(n) * std, adt)
        return a, _dec(a, adt)

    wte = _enc(rng.standard_normal((V, D)) * 0.02, adt)
    wpe = _enc(rng.standard_normal((ms, D)) * 0.01, adt)
    t["wte"], t["wpe"], ref["wte"], ref["wpe"] = wte, wpe, _dec(wte, adt), _dec(wpe, adt)
    for l in range(cfg["n_layers"]):
        p, r = f"l{l}.", {}
        for n, rows, cols in (("c_attn", 3 * D, D), ("c_proj", D, D), ("c_fc", F, D),
                              ("mlp_proj", D, F)):
            w, _, fw = _weight(rng, rows, cols, wdt)
            b, fb = vec(rows)
            t[p + n], t[p + n + ".b"], r[n], r[n + "_b"] = w, b, fw, fb
        for n in ("ln1", "ln2"):
            g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
            b = (0.1 * rng.standard_normal(D)).astype(np.float32)
            t[p + n + ".g"], t[p + n + ".b"] = g, b
            r[n + "_g"], r[n + "_b"] = g.astype(np.float64), b.astype(np.float64)
        kc = np.zeros((1, H, ms, hd), np.float32 if adt == DT_F32 else np.uint16)
        vc = kc.copy()
        t[p + "kcache"], t[p + "vcache"] = kc, vc
        r["k"], r["v"] = np.zeros((H, ms, hd)), np.zeros((H, ms, hd))
        ref["layers"].append(r)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    t["lnf.g"], t["lnf.b"], ref["lnf_g"], ref["lnf_b"] = g, b, g.astype(np.float64), b.astype(np.float64)
    return t, ref


def oracle_run(t, cfg, toks, pos0):
    om = O.OracleModel(_Tensors(t), cfg)
    out = []
    for i, tok in enumerate(toks):
        lg, nx = om.step(np.array([tok], np.int32), pos0 + i)
        out.append((lg[0].astype(np.float64), int(nx[0])))
    return out


def ref_run(model, toks, pos0):
    return [model.step(tok, pos0 + i) for i, tok in enumerate(toks)]


LLAMA = dict(arch=1, n_layers=2, dim=128, n_heads=8, n_kv_heads=2, head_dim=32, ffn=256,
             vocab=300, max_seq=48, batch=1, eps=1e-5, rope_theta=500000.0)


def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("wdt,adt", [(DT_F32, DT_F32), (DT_BF16, DT_BF16), (DT_FP8, DT_BF16)])
def test_llama_step_matches_float64_definition(wdt, adt):
    cfg = dict(LLAMA, wdtype=wdt, adtype=adt)
    ctx, toks = 20, [5, 77, 123, 9]
    t, w = llama_model(cfg, seed=11, ctx=ctx)
    got = oracle_run(t, cfg, toks, ctx)
    want = ref_run(LR.LlamaRef(w, cfg), toks, ctx)
    for (lg, nx), rl in zip(got, want):
        # f32 weights and activations: the difference is f32 summation only
        tol = 1e-5 if adt == DT_F32 else 2e-3
        assert _rel(lg, rl) <= tol, _rel(lg, rl)
        assert nx == int(np.argmax(rl)) or np.sort(rl)[-1] - np.sort(rl)[-2] < tol * np.abs(rl).max()


class _RopeHalves(LR.LlamaRef):      # pairs (j, j + hd/2) instead of (2j, 2j+1)
    def rope(self, x, pos):
        hd = self.c["head_dim"]
        ww = self.c["rope_theta"] ** (-np.arange(0, hd, 2, dtype=np.float64) / hd)
        z = (x[..., : hd // 2] + 1j * x[..., hd // 2:]) * np.exp(1j * pos * ww)
        return np.concatenate([z.real, z.imag], -1)


class _RopeSign(LR.LlamaRef):        # rotation by -pos * w
    def rope(self, x, pos):
        return LR.rope_complex(x, -pos, self.c["rope_theta"], self.c["head_dim"])


class _HeadMap(LR.LlamaRef):         # query head h reads kv head h % Hkv
    def expand_kv(self, kv, G):
        return np.tile(kv, (G, 1, 1))


class _NoResidual(LR.LlamaRef):      # sublayer output replaces the stream
    def residual(self, x, d):
        return d


class _NoGain(LR.LlamaRef):          # norm gain dropped
    def prenorm(self, x, g):
        return LR.rmsnorm(x, 1.0, self.c["eps"])


@pytest.mark.parametrize("mutant", [_RopeHalves, _RopeSign, _HeadMap, _NoResidual, _NoGain],
                         ids=lambda m: m.__name__)
def test_llama_step_check_catches_composition_mistakes(mutant):
    """The pin's sensitivity: each planted mistake moves the logits by more
    than 100x the f32 tolerance the oracle is held to above."""
    cfg = dict(LLAMA, wdtype=DT_F32, adtype=DT_F32)
    ctx, toks = 20, [5, 77]
    t, w = llama_model(cfg, seed=11, ctx=ctx)
    got = oracle_run(t, cfg, toks, ctx)
    want = ref_run(mutant(w, cfg), toks, ctx)
    worst = max(_rel(lg, rl) for (lg, _), rl in zip(got, want))
    assert worst > 1e-3, f"planted mistake {mutant.__name__} went unseen ({worst})"


GPT2 = dict(arch=2, n_layers=2, dim=96, n_heads=3, n_kv_heads=3, head_dim=32, ffn=384,
            vocab=257, max_seq=32, batch=1, eps=1e-5)


@pytest.mark.parametrize("wdt,adt", [(DT_F32, DT_F32), (DT_F16, DT_F16)])
def test_gpt2_step_matches_float64_definition(wdt, adt):
    cfg = dict(GPT2, wdtype=wdt, adtype=adt)
    toks = [3, 100, 250, 7, 7]
    t, w = gpt2_model(cfg, seed=4)
    got = oracle_run(t, cfg, toks, 0)
    want = ref_run(LR.Gpt2Ref(w, cfg), toks, 0)
    for (lg, nx), rl in zip(got, want):
        tol = 1e-5 if adt == DT_F32 else 2e-3
        assert _rel(lg, rl) <= tol, _rel(lg, rl)
        assert nx == int(np.argmax(rl))
