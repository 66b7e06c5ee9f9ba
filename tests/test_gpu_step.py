"""The persistent decode step (step_mode=1: the whole LLAMA step in one
launch, stages separated by grid barriers) against the multi-kernel step on
the same seeded model: logits, greedy ids, KV-cache rows and positions must be
identical bit for bit, step after step -- every row, split and merge runs the
same device code in the same order.  And against the CPU oracle, at the bars
of the multi-kernel decoder (test_gpu_decoder.run_parity)."""
import numpy as np
import pytest

from test_gpu_decoder import run_parity, say

pytestmark = pytest.mark.gpu

DT_FP8, DT_BF16 = 9, 12

BASE = dict(arch=1, n_layers=2, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024,
            vocab=1000, max_seq=200, batch=1, eps=1e-5, rope_theta=500000.0, init_std=0.02,
            wdtype=DT_FP8, adtype=DT_BF16)

CASES = {
    "fp8_b1_g4_hd64": dict(BASE),
    "bf16_b2_g1_hd128": dict(BASE, n_heads=4, n_kv_heads=4, head_dim=128, ffn=512, vocab=700,
                             batch=2, wdtype=DT_BF16),
    "fp8_b4_g2_hd128": dict(BASE, dim=1024, n_heads=8, n_kv_heads=4, head_dim=128, ffn=1536,
                            vocab=3000, max_seq=320, batch=4, n_layers=3),
}


def make(hip, cfg, mode, ctx, seed=11):
    # the op list with one-chunk attention blocks: the persistent step's form
    extra = dict(attn_cpb=1) if mode == 0 else {}
    dec = hip.Decoder(seed=seed, **dict(cfg, step_mode=mode, **extra))
    dec.prefill_synthetic(ctx, seed=4)
    rng = np.random.default_rng(seed)
    dec.set_state(rng.integers(0, cfg["vocab"], cfg["batch"]).astype(np.int32), ctx)
    return dec


def same_state(a, b, cfg, upto):
    la, lb = a.logits(), b.logits()
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), \
        f"logits differ: max abs {np.abs(la - lb).max()}"
    assert np.array_equal(a.tokens(upto), b.tokens(upto)), "greedy ids differ"
    assert a.position == b.position
    for l in range(cfg["n_layers"]):
        for c in ("kcache", "vcache"):
            ka, kb = a.read_tensor(f"l{l}.{c}"), b.read_tensor(f"l{l}.{c}")
            assert np.array_equal(ka, kb), f"layer {l} {c} differs"


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("ctx", [63, 130])
def test_step_equals_op_list(hip, case, ctx):
    cfg = CASES[case]
    say(f"case: persistent step {case} ctx={ctx}")
    ref = make(hip, cfg, 0, ctx)
    per = make(hip, cfg, 1, ctx)
    try:
        assert per.step_kernels() == 1 and ref.step_kernels() > 1
        ref.step()
        per.step()                         # eager launch
        same_state(ref, per, cfg, ctx + 2)
        ref.capture()
        per.capture()                      # graph of the one launch
        same_state(ref, per, cfg, ctx + 3)
        ref.replay(5)
        per.replay(5)
        same_state(ref, per, cfg, ctx + 8)
        assert per.position == ctx + 7
    finally:
        ref.close()
        per.close()


def test_step_many_launches(hip):
    """Barrier targets grow with an epoch word across launches: 60 replays."""
    cfg = dict(BASE, n_layers=1, max_seq=128)
    say("case: persistent step, 60 replays")
    ref = make(hip, cfg, 0, 10)
    per = make(hip, cfg, 1, 10)
    try:
        ref.capture(); per.capture()
        ref.replay(59); per.replay(59)
        same_state(ref, per, cfg, 71)
    finally:
        ref.close()
        per.close()


@pytest.mark.parametrize("wdt", [DT_FP8, DT_BF16])
def test_step_oracle_parity(hip, wdt):
    run_parity(hip, dict(BASE, wdtype=wdt, step_mode=1), steps=5, ctx=40)


@pytest.mark.parametrize("bad", [dict(batch=3), dict(n_heads=16, n_kv_heads=2), dict(arch=2),
                                 dict(dim=640), dict(adtype=11, wdtype=11)])
def test_step_config_errors(hip, bad):
    with pytest.raises(hip.ThvmHipError):
        hip.Decoder(seed=1, **dict(BASE, step_mode=1, **bad))


@pytest.mark.parametrize("cpb", [65, 1000])
def test_attn_cpb_config_errors(hip, cpb):
    with pytest.raises(hip.ThvmHipError):
        hip.Decoder(seed=1, **dict(BASE, attn_cpb=cpb))
