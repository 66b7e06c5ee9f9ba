"""thvm_amd.gpt2 -- the GPT-2 decode driver on the thvm_amd Tensor host.

The model follows the reference's driver (bench/gpt2/thvm_gpt2.py:25-118,
tinygrad's examples/gpt2.py): pre-LayerNorm blocks, fused c_attn, a
[2, B, MAX_CONTEXT, H, hd] KV cache updated with ``assign`` at
``start_pos``, symbolic ``start_pos`` reads of the cache, GELU MLP, tied LM
head, greedy ``argmax``, and ``TinyJit`` around the one-token forward.
Weights are synthetic (no network): ``GPT2.synthetic`` draws them from a
seeded generator in the oracle's layouts so the C oracle can run the same
model."""
from __future__ import annotations

from typing import Optional

import numpy as np

from thvm_amd.nn import Embedding, LayerNorm, Linear
from thvm_amd.tensor import Tensor, TinyJit, Variable, dtypes


class Attention:
    def __init__(self, dim: int, n_heads: int, max_context: int):
        self.c_attn = Linear(dim, 3 * dim, bias=True)
        self.c_proj = Linear(dim, dim, bias=True)
        self.n_heads, self.dim, self.head_dim = n_heads, dim, dim // n_heads
        self.max_context = max_context

    def __call__(self, x: Tensor, start_pos, mask: Optional[Tensor]) -> Tensor:
        sp_val = start_pos if isinstance(start_pos, int) else start_pos.val
        if mask is not None or sp_val == 0:
            start_pos = sp_val               # no symbolic shapes while consuming a prompt
        xqkv = self.c_attn(x).reshape(None, None, 3, self.n_heads, self.head_dim)
        xq, xk, xv = [xqkv[:, :, i, :, :] for i in range(3)]
        bsz, seqlen = int(xq.shape[0]), int(xq.shape[1])
        if not hasattr(self, "cache_kv"):
            self.cache_kv = Tensor.zeros(2, bsz, self.max_context, self.n_heads, self.head_dim,
                                         dtype=x.dtype).contiguous().realize()
        self.cache_kv[:, :, start_pos:start_pos + seqlen, :, :].assign(Tensor.stack([xk, xv])).realize()
        if sp_val > 0:
            keys = self.cache_kv[0][:, :start_pos + seqlen, :, :]
            values = self.cache_kv[1][:, :start_pos + seqlen, :, :]
        else:
            keys, values = xk, xv
        xq, keys, values = xq.transpose(1, 2), keys.transpose(1, 2), values.transpose(1, 2)
        o = xq.scaled_dot_product_attention(keys, values, mask).transpose(1, 2).reshape(bsz, seqlen, self.dim)
        return self.c_proj(o)


class FeedForward:
    def __init__(self, dim: int, hidden_dim: int):
        self.c_fc = Linear(dim, hidden_dim, bias=True)
        self.c_proj = Linear(hidden_dim, dim, bias=True)

    def __call__(self, x: Tensor) -> Tensor:
        return self.c_proj(self.c_fc(x).gelu())


class TransformerBlock:
    def __init__(self, dim: int, n_heads: int, norm_eps: float, max_context: int):
        self.attn = Attention(dim, n_heads, max_context)
        self.mlp = FeedForward(dim, 4 * dim)
        self.ln_1 = LayerNorm(dim, norm_eps)
        self.ln_2 = LayerNorm(dim, norm_eps)

    def __call__(self, x: Tensor, start_pos, mask: Optional[Tensor]) -> Tensor:
        h = x + self.attn(self.ln_1(x), start_pos, mask).float()
        return (h + self.mlp(self.ln_2(h))).contiguous()


class Transformer:
    def __init__(self, dim: int, n_heads: int, n_layers: int, norm_eps: float, vocab_size: int,
                 max_seq_len: int = 1024, max_context: int = 128):
        self.vocab_size, self.max_context = vocab_size, max_context
        self.wte = Embedding(vocab_size, dim)
        self.wpe = Embedding(max_seq_len, dim)
        self.h = [TransformerBlock(dim, n_heads, norm_eps, max_context) for _ in range(n_layers)]
        self.ln_f = LayerNorm(dim, norm_eps)
        self.lm_head = Linear(dim, vocab_size, bias=False)
        self.forward_jit = TinyJit(self.forward)
        self.logits: Optional[Tensor] = None

    def forward(self, tokens: Tensor, start_pos, temperature: float = 0.0) -> Tensor:
        if not hasattr(self, "allpos"):
            self.allpos = Tensor.arange(0, self.max_context).reshape(1, -1).realize()
        seqlen = int(tokens.shape[1])
        sp_val = start_pos if isinstance(start_pos, int) else start_pos.val
        tok_emb = self.wte(tokens)
        selected = (0, seqlen) if sp_val == 0 else (start_pos, start_pos + 1)
        pos_emb = self.wpe(self.allpos.shrink((None, selected)))
        h = tok_emb + pos_emb
        mask = Tensor.full((1, 1, seqlen, sp_val + seqlen), float("-inf")).triu(sp_val + 1) \
            if seqlen > 1 else None
        for hi in self.h:
            h = hi(h, start_pos, mask)
        logits = self.lm_head(self.ln_f(h))[:, -1, :]
        self.logits = logits.realize()
        if temperature >= 1e-6:
            raise NotImplementedError("sampling: greedy decode only")
        return logits.argmax(-1).flatten().realize()

    def __call__(self, tokens: Tensor, start_pos, temperature: float = 0.0, jit: bool = True) -> Tensor:
        fwd = self.forward_jit if jit and int(tokens.shape[1]) == 1 else self.forward
        return fwd(tokens, start_pos, temperature)


MODEL_PARAMS = {
    "gpt2": dict(n_layers=12, n_heads=12, dim=768, norm_eps=1e-5, vocab_size=50257),
    "gpt2-medium": dict(n_layers=24, n_heads=16, dim=1024, norm_eps=1e-5, vocab_size=50257),
    "gpt2-large": dict(n_layers=36, n_heads=20, dim=1280, norm_eps=1e-5, vocab_size=50257),
    "gpt2-xl": dict(n_layers=48, n_heads=25, dim=1600, norm_eps=1e-5, vocab_size=50257),
}


class GPT2:
    """Builds a Transformer and runs greedy decode, one token per step."""

    def __init__(self, model: Transformer):
        self.model = model

    @staticmethod
    def synthetic_weights(n_layers, dim, vocab_size, max_seq_len, seed=0, std=0.02):
        """Seeded N(0, std) weights (gains 1, biases N(0, std)) in the layouts
        the model and the C oracle share: Linear weights [out, in]."""
        rng = np.random.default_rng(seed)

        def n(*s):
            return (rng.standard_normal(s) * std).astype(np.float32)

        w = {"wte": n(vocab_size, dim), "wpe": n(max_seq_len, dim),
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

    @staticmethod
    def build(n_layers, n_heads, dim, vocab_size, max_seq_len, max_context, weights, norm_eps=1e-5):
        m = Transformer(dim, n_heads, n_layers, norm_eps, vocab_size, max_seq_len, max_context)
        T = Tensor
        m.wte.weight, m.wpe.weight = T(weights["wte"]), T(weights["wpe"])
        m.ln_f.weight, m.ln_f.bias = T(weights["lnf.g"]), T(weights["lnf.b"])
        m.lm_head.weight = m.wte.weight                  # tied, as the GPT-2 checkpoint
        for l, b in enumerate(m.h):
            p = f"l{l}."
            b.attn.c_attn.weight, b.attn.c_attn.bias = T(weights[p + "c_attn"]), T(weights[p + "c_attn.b"])
            b.attn.c_proj.weight, b.attn.c_proj.bias = T(weights[p + "c_proj"]), T(weights[p + "c_proj.b"])
            b.mlp.c_fc.weight, b.mlp.c_fc.bias = T(weights[p + "c_fc"]), T(weights[p + "c_fc.b"])
            b.mlp.c_proj.weight, b.mlp.c_proj.bias = T(weights[p + "mlp_proj"]), T(weights[p + "mlp_proj.b"])
            b.ln_1.weight, b.ln_1.bias = T(weights[p + "ln1.g"]), T(weights[p + "ln1.b"])
            b.ln_2.weight, b.ln_2.bias = T(weights[p + "ln2.g"]), T(weights[p + "ln2.b"])
        return GPT2(m)

    def step(self, tokens: np.ndarray, pos: int, jit: bool = True) -> np.ndarray:
        """One greedy step for every batch row: token ids [B] at position pos."""
        toks = Tensor(np.asarray(tokens, np.int32).reshape(-1, 1), dtype=dtypes.int32)
        start_pos = Variable("start_pos", 0, self.model.max_context - 1).bind(pos)
        return self.model(toks, start_pos, jit=jit).numpy()

    def generate(self, prompt: list, n_new: int, batch: int = 1, jit: bool = True):
        """Feed the prompt one token at a time, then n_new greedy tokens;
        returns the generated ids [batch, n_new]."""
        cur = np.full(batch, prompt[0], np.int32)
        out = []
        for pos in range(len(prompt) + n_new - 1):
            nxt = self.step(cur, pos, jit)
            if pos + 1 < len(prompt):
                cur = np.full(batch, prompt[pos + 1], np.int32)
            else:
                cur = nxt.astype(np.int32)
                out.append(cur.copy())
        return np.stack(out, axis=1)
