"""Parity at the real widths of the BASELINE configs (C1, C3, C4, C5 decoders;
C2's single ops are in test_gpu_c2.py), against the CPU oracle on the same
weights (generated on the device, read back), teacher-forced step by step
(tests/_parity.py): C1 at its full depth (12 layers fp32, 80 steps), the
others at 1-4 layers over several steps.

Bars are the north star's (fp32 1e-5 relative with identical ids; fp8
2e-2 relative; fp16/bf16 1e-2 absolute; ids may fork only at a proven near
tie).  The full depths of C3, C4 and C5 are held to the same bars sublayer
by sublayer in test_gpu_depth.py."""
import numpy as np
import pytest

import _oracle as O
import _parity as P

pytestmark = pytest.mark.gpu

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13

C1 = dict(arch=2, n_layers=12, dim=768, n_heads=12, n_kv_heads=12, head_dim=64, ffn=3072,
          vocab=50257, wdtype=DT_F32, adtype=DT_F32, eps=1e-5, init_std=0.02)
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


def _decoder(hip, cfg, seed, ctx):
    say(f"case: {cfg['arch']=} layers={cfg['n_layers']} batch={cfg['batch']} ctx={ctx} "
        f"dim={cfg['dim']} vocab={cfg['vocab']}")
    dec = hip.Decoder(seed=seed, **cfg)
    if ctx:
        dec.prefill_synthetic(ctx, seed=seed + 1)
    return dec


def _oracle(dec, cfg):
    return O.OracleDsv2(dec, cfg) if cfg["arch"] == 3 else O.OracleModel(dec, cfg)


def _first_ids(cfg, seed):
    return np.random.default_rng(seed).integers(0, cfg["vocab"], cfg["batch"]).astype(np.int32)


# ------------------------------------------------------------- C1 ----------
def test_c1_gpt2_small_fp32_full(hip):
    """C1 at its full shape: 12 layers fp32, a 16-id prompt drawn from
    [0, 50257), then 64 greedy tokens; ids identical on every step, logits
    within 1e-5 relative."""
    cfg = dict(C1, batch=1, max_seq=96)
    prompt = np.random.default_rng(16).integers(0, cfg["vocab"], 16).tolist()
    dec = _decoder(hip, cfg, seed=1234, ctx=0)
    try:
        om = _oracle(dec, cfg)
        r = P.lockstep(dec, om, cfg, None, 0, 64, "C1", prompt=prompt)
        assert r["forks"] == 0
        ids = dec.tokens(16 + 64)[0, 16:]
        assert len(ids) == 64 and np.all((ids >= 0) & (ids < cfg["vocab"]))
    finally:
        dec.close()


# ------------------------------------------------------------- C3 ----------
@pytest.mark.parametrize("batch", [1, 8])
def test_c3_gpt2_xl_fp16_full_width(hip, batch):
    """C3 widths (d 1600, 25 heads, MLP 6400, vocab 50257) at 2 layers, a
    16-id prompt then greedy steps; batch 8 runs the MFMA GEMM path."""
    cfg = dict(C3, n_layers=2, batch=batch, max_seq=64)
    prompt = np.random.default_rng(3).integers(0, cfg["vocab"], 16).tolist()
    dec = _decoder(hip, cfg, seed=33, ctx=0)
    try:
        P.lockstep(dec, _oracle(dec, cfg), cfg, None, 0, 4, f"C3 B={batch}", prompt=prompt)
    finally:
        dec.close()


# ------------------------------------------------------------- C4 ----------
@pytest.mark.parametrize("layers,batch", [(1, 1), (2, 1), (2, 16)])
def test_c4_llama8b_fp8_full_width(hip, layers, batch):
    """C4 widths (d 4096, GQA 32/8 x 128, FFN 14336, vocab 128256, fp8
    weights, bf16 KV prefilled to 2048) at 1-2 layers; batch 16 runs the
    MFMA GEMM path with separate norms."""
    cfg = dict(C4, n_layers=layers, batch=batch, max_seq=2056)
    dec = _decoder(hip, cfg, seed=41, ctx=2048)
    try:
        P.lockstep(dec, _oracle(dec, cfg), cfg, _first_ids(cfg, 4), 2048, 3 if batch == 1 else 2,
                   f"C4 L={layers} B={batch}")
    finally:
        dec.close()


# ------------------------------------------------------------- C5 ----------
@pytest.mark.parametrize("layers,batch", [(2, 1), (4, 1), (2, 32)])
def test_c5_dsv2_lite_fp8_full_width(hip, layers, batch):
    """C5 widths (d 2048, 16 heads, MLA kv 512 / nope 128 / rope 64 / v 128,
    dense layer 0 of 10944, 64 routed experts x 1408 top-6 + 2 shared, vocab
    102400, fp8, latent cache prefilled to 4096); every MoE layer's routing
    checked each step; batch 32 runs the expert-grouped MFMA MoE."""
    cfg = dict(C5, n_layers=layers, batch=batch, max_seq=4104)
    dec = _decoder(hip, cfg, seed=51, ctx=4096)
    try:
        r = P.lockstep(dec, _oracle(dec, cfg), cfg, _first_ids(cfg, 5), 4096,
                       3 if batch == 1 else 2, f"C5 L={layers} B={batch}")
        assert r["routing_forks"] <= max(1, batch // 8)
    finally:
        dec.close()
