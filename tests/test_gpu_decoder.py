"""Whole-model decode parity: the captured/replayed gfx950 decode step against
the oracle's decode step (oracle/oracle.c or_decode_step) on the same weights
(read back from the device), at scaled shapes of configs C1/C3/C4.

Bars (north star): fp32 greedy ids identical and logits within 1e-5
relative (to max|logit|, per step); bf16/fp16 logits within 1e-2 absolute;
fp8 logits within 2e-2 relative; teacher-forced, with ids equal or a proven near
tie on every step (tests/_parity.py)."""
import numpy as np
import pytest

import _oracle as O
import _parity as P

pytestmark = pytest.mark.gpu

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13


def say(*a):
    print(*a, flush=True)


def run_parity(hip, cfg, steps, ctx, seed=3):
    """Teacher-forced lockstep against the oracle (every step held to the
    bar, ids equal or a proven near tie), then the captured step replayed
    must reproduce an eager run's trajectory and logits bit for bit."""
    say(f"case: decoder {cfg} steps={steps} ctx={ctx}")
    B = cfg["batch"]
    tok = np.random.default_rng(seed).integers(0, cfg["vocab"], B).astype(np.int32)
    dec = hip.Decoder(seed=seed, **cfg)
    try:
        if ctx:
            dec.prefill_synthetic(ctx, seed=5)
        om = O.OracleDsv2(dec, cfg) if cfg["arch"] == 3 else O.OracleModel(dec, cfg)
        P.lockstep(dec, om, cfg, tok, ctx, steps, "small")
    finally:
        dec.close()
    runs = []
    for captured in (False, True):
        dec = hip.Decoder(seed=seed, **cfg)
        try:
            if ctx:
                dec.prefill_synthetic(ctx, seed=5)
            dec.set_state(tok, ctx)
            if captured:
                dec.capture()                  # runs step 1
                dec.replay(steps - 1)          # graph capture on replay 1, then hits
            else:
                for _ in range(steps):
                    dec.step()
            assert dec.position == ctx + steps
            runs.append((dec.tokens(ctx + steps + 1), dec.logits()))
        finally:
            dec.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))


LLAMA = dict(arch=1, n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512,
             vocab=512, max_seq=96, batch=1, eps=1e-5, rope_theta=500000.0, init_std=0.02)


@pytest.mark.parametrize("wdt", [DT_BF16, DT_FP8])
def test_llama_decode_parity(hip, wdt):
    run_parity(hip, dict(LLAMA, wdtype=wdt, adtype=DT_BF16), steps=6, ctx=20)


def test_llama_gqa4_hd128_batch2(hip):
    cfg = dict(LLAMA, dim=512, n_heads=4, n_kv_heads=1, head_dim=128, ffn=768, batch=2,
               wdtype=DT_FP8, adtype=DT_BF16)
    run_parity(hip, cfg, steps=4, ctx=70)


GPT2 = dict(arch=2, n_layers=2, dim=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn=1024,
            vocab=500, max_seq=64, batch=1, eps=1e-5, init_std=0.02)


def test_gpt2_fp32_greedy_ids_identical(hip):
    run_parity(hip, dict(GPT2, wdtype=DT_F32, adtype=DT_F32), steps=8, ctx=0)


def test_gpt2_fp16_decode_parity(hip):
    run_parity(hip, dict(GPT2, wdtype=DT_F16, adtype=DT_F16, batch=2), steps=5, ctx=0)


@pytest.mark.parametrize("batch", [8, 16])
def test_llama_fp8_batched_mfma(hip, batch):
    """Batches above 4 rows: separate norm kernels and MFMA GEMM projections
    (the C4 B=16 path at a small shape)."""
    cfg = dict(LLAMA, batch=batch, wdtype=DT_FP8, adtype=DT_BF16)
    run_parity(hip, cfg, steps=4, ctx=30)


def test_gpt2_fp16_batch8_mfma(hip):
    """The GPT-2 XL B=8 path (LayerNorm kernels, fp16 MFMA GEMM with bias and
    GELU epilogues) at a small shape."""
    run_parity(hip, dict(GPT2, wdtype=DT_F16, adtype=DT_F16, batch=8), steps=4, ctx=0)


@pytest.mark.parametrize("arch", ["llama-fp8", "llama-bf16", "gpt2-fp16", "dsv2-fp8"])
def test_batched_decoder_tiled_weights_bit_equal(hip, monkeypatch, arch):
    """Decoders above 4 rows read their projection weights from tiled copies
    (the MFMA GEMM's layout); with THVM_HIP_WTILE=0 they read the row-major
    tensors.  Both give the same bits: 3 steps' logits and ids, and a weight
    rewritten through write_tensor reaches the tiled copy (sync_weights)."""
    from test_gpu_dsv2 import DSV2
    cfg = {"llama-fp8": dict(LLAMA, batch=8, wdtype=DT_FP8, adtype=DT_BF16),
           "llama-bf16": dict(LLAMA, batch=8, wdtype=DT_BF16, adtype=DT_BF16),
           "gpt2-fp16": dict(GPT2, wdtype=DT_F16, adtype=DT_F16, batch=8),
           "dsv2-fp8": dict(DSV2, batch=8, wdtype=DT_FP8)}[arch]
    say(f"case: tiled vs row-major weights, {arch}")
    tok = np.random.default_rng(4).integers(0, cfg["vocab"], 8).astype(np.int32)
    runs = []
    for tile in ("1", "0"):
        monkeypatch.setenv("THVM_HIP_WTILE", tile)
        dec = hip.Decoder(seed=9, **cfg)
        try:
            tiled_names = ["lm.tiled" if arch != "gpt2-fp16" else "wte.tiled"]
            if arch == "dsv2-fp8":
                tiled_names += ["l1.wgu_e.tiled", "l1.wd_e.tiled"]
            for tn in tiled_names:
                try:
                    dec.tensor(tn)
                    has_tiled = True
                except hip.ThvmHipError:
                    has_tiled = False
                assert has_tiled == (tile == "1"), tn
            wn = {"gpt2-fp16": "l0.c_proj", "dsv2-fp8": "l1.wd_e"}.get(arch, "l0.wo")
            w = dec.read_tensor(wn)
            dec.write_tensor(wn, w[::-1].copy())
            dec.set_state(tok, 0)
            for _ in range(3):
                dec.step()
            runs.append((dec.tokens(4), dec.logits()))
        finally:
            dec.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))
