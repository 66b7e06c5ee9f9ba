"""The decoder shapes of the benchmark configurations:
ThvmDecodeConfig fields for the synthetic random-init models.  C2 is a
single-op sweep and has no decoder."""
from __future__ import annotations

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13

DECODERS = {
    # GPT-2 small fp32: 12 layers, d 768, 12 heads, MLP 3072, vocab 50257
    "C1": dict(arch=2, n_layers=12, dim=768, n_heads=12, n_kv_heads=12, head_dim=64, ffn=3072,
               vocab=50257, wdtype=DT_F32, adtype=DT_F32, eps=1e-5, init_std=0.02),
    # GPT-2 XL shape fp16: 48 layers, d 1600, 25 heads, MLP 6400, vocab 50257
    "C3": dict(arch=2, n_layers=48, dim=1600, n_heads=25, n_kv_heads=25, head_dim=64, ffn=6400,
               vocab=50257, wdtype=DT_F16, adtype=DT_F16, eps=1e-5, init_std=0.02),
    # Llama-8B shape, fp8 e4m3 weights (per-row absmax/448), bf16 activations
    "C4": dict(arch=1, n_layers=32, dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
               vocab=128256, wdtype=DT_FP8, adtype=DT_BF16, eps=1e-5, rope_theta=500000.0,
               init_std=0.02),
    # DeepSeek-V2-Lite shape: MLA kv_lora 512, dense layer 0 (10944), 64 experts
    # x 1408 top-6 + 2 shared, vocab 102400, fp8 weights
    "C5": dict(arch=3, n_layers=27, dim=2048, n_heads=16, n_kv_heads=16, head_dim=192, ffn=10944,
               vocab=102400, wdtype=DT_FP8, adtype=DT_BF16, eps=1e-6, rope_theta=10000.0,
               init_std=0.02, kv_lora=512, d_nope=128, d_rope=64, d_v=128, n_experts=64,
               n_shared=2, top_k=6, moe_inter=1408, first_dense=1),
}
