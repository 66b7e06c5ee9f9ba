"""Independent numpy restatement of one Llama-style and one GPT-2-style
decode step, written from the model definitions (test infrastructure).

It exists to pin the C oracle's whole-step composition (or_decode_step):
the op-level pins cannot see a wrong GQA head map, RoPE pairing, residual
placement or norm position.  Everything here is formulated differently
from the oracle on purpose:

  * sums are float64 matrix products (numpy), not serial f32 loops;
  * RoPE is a complex multiplication of (x[2j] + i x[2j+1]) by
    exp(i pos theta^(-2j/hd)), with the angles computed in float64 here,
    not read from the device's cos/sin tables;
  * grouped-query attention repeats each KV head over its G query heads
    (np.repeat) and runs a batched softmax over all heads at once;
  * the storage rounding of 16-bit activations is one vectorised RNE
    bit operation (bf16) or numpy float16 (fp16).

Rounding points are those of the decode chain the oracle and the device
follow (bench/dsv2_decode_bench.c:20-34): every projection output, the
norm outputs, the attention output, the SwiGLU/GELU product and each
residual sum are stored in the activation dtype.  `round_points=False`
keeps everything in float64 (the exact-arithmetic model).

With `ft=np.float32` (and float32 weights) the same model computes in
float32 through numpy's BLAS: a second valid f32 implementation whose
summation order differs from the oracle's serial loops.  The distance
between the two measures how far any two correct f32 implementations of
this decode chain drift apart (the noise floor of the computation)."""
from __future__ import annotations

import numpy as np

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13


def bf16_round(x):
    """Round float values to bfloat16 (nearest, ties to even) and return them
    as float64; NaN stays NaN."""
    f = np.asarray(x, np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).astype(np.float64)
    return np.where(np.isnan(f), np.nan, out)


def store(x, adt, round_points=True, ft=np.float64):
    """x stored in the activation dtype adt, returned in the compute type ft."""
    if not round_points or adt == DT_F32:
        return np.asarray(x, ft)
    if adt == DT_BF16:
        return bf16_round(x).astype(ft)
    if adt == DT_F16:
        return np.asarray(x, np.float64).astype(np.float16).astype(ft)
    raise ValueError(adt)


def rope_complex(x, pos, theta, hd):
    """x: [..., hd] with adjacent pairs (2j, 2j+1) rotated by pos * w_j."""
    w = theta ** (-np.arange(0, hd, 2, dtype=np.float64) / hd)
    z = x[..., 0::2] + 1j * x[..., 1::2]
    z = z * np.exp(1j * pos * w)
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = z.real, z.imag
    return out


def rmsnorm(x, g, eps):
    return x / np.sqrt(np.mean(x * x, -1, keepdims=True) + eps) * g


def layernorm(x, g, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def gelu_tanh(x):
    c = x.dtype.type(np.sqrt(2.0 / np.pi))
    return x.dtype.type(0.5) * x * (1 + np.tanh(c * (x + x.dtype.type(0.044715) * x ** 3)))


class LlamaRef:
    """Weights as float64 arrays (already dequantised):
    emb [V,D]; per layer wq [H*hd,D], wk/wv [Hkv*hd,D], wo [D,H*hd],
    wg/wu [F,D], wd [D,F], g1/g2 [D]; gf [D]; lm [V,D]; caches
    k/v [Hkv, max_seq, hd] float64 (one batch row).

    The model's parts are methods (rope, expand_kv, residual, prenorm) so a
    test can plant a composition mistake by overriding one of them."""

    def __init__(self, w, cfg, round_points=True, ft=np.float64):
        self.w, self.c, self.rp, self.ft = w, cfg, round_points, ft

    def rope(self, x, pos):
        return rope_complex(x, pos, self.c["rope_theta"], self.c["head_dim"])

    def expand_kv(self, kv, G):
        """[Hkv, L, hd] -> [H, L, hd]: query head h reads kv head h // G."""
        return np.repeat(kv, G, axis=0)

    def residual(self, x, d):
        return x + d

    def prenorm(self, x, g):
        return rmsnorm(x, g, self.c["eps"])

    def step(self, tok, pos):
        c, w, rp = self.c, self.w, self.rp
        adt, H, Hkv, hd = c["adtype"], c["n_heads"], c["n_kv_heads"], c["head_dim"]
        G = H // Hkv
        S = lambda v: store(v, adt, rp, self.ft)  # noqa: E731
        x = S(w["emb"][tok])
        for ly in w["layers"]:
            a = S(self.prenorm(x, ly["g1"]))
            q = S(ly["wq"] @ a).reshape(H, hd)
            k = S(ly["wk"] @ a).reshape(Hkv, hd)
            v = S(ly["wv"] @ a).reshape(Hkv, hd)
            q, k = S(self.rope(q, pos)), S(self.rope(k, pos))
            ly["k"][:, pos], ly["v"][:, pos] = k, v
            K = self.expand_kv(ly["k"][:, : pos + 1], G)          # [H, L, hd]
            Vv = self.expand_kv(ly["v"][:, : pos + 1], G)
            s = np.matmul(K, q[:, :, None])[..., 0] / self.ft(np.sqrt(hd))
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            att = S(np.matmul(p[:, None, :], Vv)[:, 0].reshape(H * hd))
            x = S(self.residual(x, S(ly["wo"] @ att)))
            a = S(self.prenorm(x, ly["g2"]))
            g, u = S(ly["wg"] @ a), S(ly["wu"] @ a)
            m = S(g / (self.ft(1) + np.exp(-g)) * u)
            x = S(self.residual(x, S(ly["wd"] @ m)))
        a = S(rmsnorm(x, w["gf"], c["eps"]))
        return w["lm"] @ a


class Gpt2Ref:
    """GPT-2 (pre-LayerNorm, fused c_attn, tanh GELU, tied LM head).
    Weights float64: wte [V,D], wpe [P,D]; per layer c_attn [3D,D] + b,
    c_proj [D,D] + b, c_fc [F,D] + b, mlp_proj [D,F] + b, ln1/ln2 (g, b);
    lnf (g, b); caches k/v [H, max_seq, hd]."""

    def __init__(self, w, cfg, round_points=True, ft=np.float64):
        self.w, self.c, self.rp, self.ft = w, cfg, round_points, ft

    def step(self, tok, pos):
        c, w, rp = self.c, self.w, self.rp
        adt, H, hd, D = c["adtype"], c["n_heads"], c["head_dim"], c["dim"]
        S = lambda v: store(v, adt, rp, self.ft)  # noqa: E731
        x = S(w["wte"][tok] + w["wpe"][pos])
        for ly in w["layers"]:
            a = S(layernorm(x, ly["ln1_g"], ly["ln1_b"], c["eps"]))
            qkv = S(ly["c_attn"] @ a + ly["c_attn_b"])
            q, k, v = (qkv[i * D:(i + 1) * D].reshape(H, hd) for i in range(3))
            ly["k"][:, pos], ly["v"][:, pos] = k, v
            s = np.matmul(ly["k"][:, : pos + 1], q[:, :, None])[..., 0] / self.ft(np.sqrt(hd))
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            att = S(np.matmul(p[:, None, :], ly["v"][:, : pos + 1])[:, 0].reshape(D))
            x = S(x + S(ly["c_proj"] @ att + ly["c_proj_b"]))
            a = S(layernorm(x, ly["ln2_g"], ly["ln2_b"], c["eps"]))
            h = S(gelu_tanh(S(ly["c_fc"] @ a + ly["c_fc_b"])))
            x = S(x + S(ly["mlp_proj"] @ h + ly["mlp_proj_b"]))
        a = S(layernorm(x, w["lnf_g"], w["lnf_b"], c["eps"]))
        return w["wte"] @ a
