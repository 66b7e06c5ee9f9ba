"""thvm_amd.gpt2 -- GPT-2 decode on the thvm_amd Tensor host.

GPT-2 (Radford et al., 2019) is a pre-LayerNorm decoder: per block,
``x += c_proj(attn(ln_1(x)))`` with a fused q/k/v projection ``c_attn``,
then ``x += mlp_proj(gelu_tanh(c_fc(ln_2(x))))``; learned absolute
positions ``wpe`` are added to the token embedding ``wte``; a final
LayerNorm ``ln_f`` precedes the LM head, whose weight is ``wte`` (tied).

This driver decodes one token per call, which is all a decode benchmark
needs (the prompt is fed one position at a time):

* each layer owns a K and a V cache tensor ``[B, H, max_context, hd]``,
  head-major so one head's rows are contiguous; the new row is written with
  ``assign`` into ``cache[:, :, pos:pos+1]`` and attention reads
  ``cache[:, :, :pos+1]`` with ``pos`` a bound ``Variable`` (a symbolic
  length, so one captured graph serves every position);
* the one-token forward runs under ``TinyJit`` (captured on its second call,
  replayed after that with the position rebound);
* the next id is the greedy ``argmax`` of the last logits, or a sample from
  ``softmax(logits / temperature)`` (``sample_from``).

Weights are synthetic (there is no network here): ``GPT2.synthetic_weights``
draws them from a seeded generator in ``[out_features, in_features]``
layouts that the C oracle (arch GPT2) reads too.  The reference's driver
for the same model is bench/gpt2/thvm_gpt2.py."""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import numpy as np

from thvm_amd.tensor import Tensor, TinyJit, Variable, dtypes

# published GPT-2 shapes (layers, heads, d_model); vocab 50257, 1024 positions
SHAPES = {
    "gpt2": (12, 12, 768),
    "gpt2-medium": (24, 16, 1024),
    "gpt2-large": (36, 20, 1280),
    "gpt2-xl": (48, 25, 1600),
}


def sample_from(logits: np.ndarray, temperature: float, rng: np.random.Generator) -> np.ndarray:
    """One id per row from softmax(logits / temperature) by inverse-CDF
    sampling with a uniform draw per row (the reference samples with
    ``Tensor.multinomial``, bench/gpt2/thvm_gpt2.py:120-124)."""
    z = np.asarray(logits, np.float64) / temperature
    p = np.exp(z - z.max(-1, keepdims=True))
    cdf = np.cumsum(p, -1)
    u = rng.random(z.shape[0]) * cdf[:, -1]
    return np.minimum((cdf < u[:, None]).sum(-1), z.shape[-1] - 1).astype(np.int32)


class _Block:
    """Parameters of one transformer block and its KV cache."""

    def __init__(self, w: Dict[str, Tensor], batch: int, n_heads: int, dim: int,
                 max_context: int, dtype):
        self.w = w
        hd = dim // n_heads
        self.k = Tensor.zeros(batch, n_heads, max_context, hd, dtype=dtype).contiguous().realize()
        self.v = Tensor.zeros(batch, n_heads, max_context, hd, dtype=dtype).contiguous().realize()


class GPT2:
    """A GPT-2 decoder bound to its weights, one token per ``step``."""

    def __init__(self, weights: Dict[str, np.ndarray], n_layers: int, n_heads: int, dim: int,
                 vocab_size: int, max_context: int, batch: int = 1, norm_eps: float = 1e-5):
        self.n_layers, self.n_heads, self.dim = n_layers, n_heads, dim
        self.head_dim = dim // n_heads
        self.vocab_size, self.max_context, self.batch, self.eps = vocab_size, max_context, batch, norm_eps
        up = {k: Tensor(np.ascontiguousarray(v)) for k, v in weights.items()}
        self.wte, self.wpe = up["wte"], up["wpe"]
        self.lnf = (up["lnf.g"], up["lnf.b"])
        dt = self.wte.dtype
        names = ("c_attn", "c_attn.b", "c_proj", "c_proj.b", "c_fc", "c_fc.b", "mlp_proj",
                 "mlp_proj.b", "ln1.g", "ln1.b", "ln2.g", "ln2.b")
        self.blocks: List[_Block] = [
            _Block({n: up[f"l{l}.{n}"] for n in names}, batch, n_heads, dim, max_context, dt)
            for l in range(n_layers)]
        self.pos = Variable("pos", 0, max_context - 1)
        self.jit = TinyJit(self._forward)
        self.logits: Optional[Tensor] = None

    # ---- the model ----
    def _ln(self, x: Tensor, g: Tensor, b: Tensor) -> Tensor:
        return x.layernorm(-1, self.eps) * g + b

    @staticmethod
    def _proj(x: Tensor, w: Tensor, b: Tensor) -> Tensor:
        return x.linear(w.transpose(), b)

    def _attention(self, blk: _Block, x: Tensor, pos) -> Tensor:
        B, H, hd, D = self.batch, self.n_heads, self.head_dim, self.dim
        qkv = self._proj(x, blk.w["c_attn"], blk.w["c_attn.b"]).reshape(B, 3, H, 1, hd)
        q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]                 # [B, H, 1, hd]
        blk.k[:, :, pos:pos + 1, :].assign(k).realize()
        blk.v[:, :, pos:pos + 1, :].assign(v).realize()
        keys, vals = blk.k[:, :, :pos + 1, :], blk.v[:, :, :pos + 1, :]
        s = q.matmul(keys.transpose(-2, -1)) * (1.0 / math.sqrt(hd))   # [B, H, 1, pos+1]
        o = s.softmax(-1).matmul(vals)                                    # [B, H, 1, hd]
        return self._proj(o.reshape(B, 1, D), blk.w["c_proj"], blk.w["c_proj.b"])

    def _mlp(self, blk: _Block, x: Tensor) -> Tensor:
        h = self._proj(x, blk.w["c_fc"], blk.w["c_fc.b"]).gelu()
        return self._proj(h, blk.w["mlp_proj"], blk.w["mlp_proj.b"])

    def _forward(self, tokens: Tensor, pos) -> Tensor:
        """tokens [B, 1] int32 at position pos -> greedy ids [B]."""
        x = self.wte.gather_rows(tokens.reshape(self.batch)).reshape(self.batch, 1, self.dim)
        x = x + self.wpe[pos:pos + 1].reshape(1, 1, self.dim)
        for blk in self.blocks:
            x = x + self._attention(blk, self._ln(x, blk.w["ln1.g"], blk.w["ln1.b"]), pos)
            x = (x + self._mlp(blk, self._ln(x, blk.w["ln2.g"], blk.w["ln2.b"]))).contiguous()
        x = self._ln(x, *self.lnf).reshape(self.batch, self.dim)
        self.logits = x.matmul(self.wte.transpose()).realize()         # tied head
        return self.logits.argmax(-1).realize()

    # ---- driving ----
    def step(self, tokens, pos: int, jit: bool = True, temperature: float = 0.0,
             rng: Optional[np.random.Generator] = None) -> np.ndarray:
        """Ids [B] at position pos -> next ids [B]: greedy at temperature 0,
        else sampled from the tempered softmax of the logits."""
        toks = Tensor(np.asarray(tokens, np.int32).reshape(self.batch, 1), dtype=dtypes.int32)
        bound = self.pos.bind(int(pos))
        nxt = (self.jit if jit else self._forward)(toks, bound).numpy().reshape(self.batch)
        if temperature > 0.0:
            return sample_from(self.logits.numpy(), temperature, rng or np.random.default_rng())
        return nxt

    def generate(self, prompt: List[int], n_new: int, jit: bool = True, temperature: float = 0.0,
                 seed: int = 0) -> np.ndarray:
        """Consume the prompt one position at a time, then produce n_new ids
        per batch row; returns [B, n_new]."""
        rng = np.random.default_rng(seed)
        cur = np.full(self.batch, prompt[0], np.int32)
        out = []
        for pos in range(len(prompt) + n_new - 1):
            nxt = self.step(cur, pos, jit, temperature, rng)
            if pos + 1 < len(prompt):
                cur = np.full(self.batch, prompt[pos + 1], np.int32)
            else:
                cur = nxt.astype(np.int32)
                out.append(cur.copy())
        return np.stack(out, axis=1)

    # ---- weights ----
    @staticmethod
    def synthetic_weights(n_layers: int, dim: int, vocab_size: int, n_positions: int,
                          seed: int = 0, std: float = 0.02) -> Dict[str, np.ndarray]:
        """Seeded weights: matrices and biases N(0, std), LayerNorm gains 1
        and biases N(0, std); matrices are [out_features, in_features]."""
        rng = np.random.default_rng(seed)

        def n(*s):
            return (rng.standard_normal(s) * std).astype(np.float32)

        w = {"wte": n(vocab_size, dim), "wpe": n(n_positions, dim),
             "lnf.g": np.ones(dim, np.float32), "lnf.b": n(dim)}
        for l in range(n_layers):
            p = f"l{l}."
            w.update({p + "c_attn": n(3 * dim, dim), p + "c_attn.b": n(3 * dim),
                      p + "c_proj": n(dim, dim), p + "c_proj.b": n(dim),
                      p + "c_fc": n(4 * dim, dim), p + "c_fc.b": n(4 * dim),
                      p + "mlp_proj": n(dim, 4 * dim), p + "mlp_proj.b": n(dim),
                      p + "ln1.g": np.ones(dim, np.float32), p + "ln1.b": n(dim),
                      p + "ln2.g": np.ones(dim, np.float32), p + "ln2.b": n(dim)})
        return w
