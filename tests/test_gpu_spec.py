"""Blind speculative decode (ThvmDecodeConfig.spec_rows; reference DSV2_SPEC,
bench/dsv2_decode_bench.c:56-68, 1110-1170, 2255-2745).

* The draft and commit kernels against the oracle (or_spec_draft,
  or_spec_accept), bit-exact: histories with planted repeats, ids outside
  the vocabulary, the forced form, and the capacity edge.
* The reference's startup gate, extended to every row: each verify row s is
  bit-equal to the one-row step run at position P+s on the same embedded
  candidate (row 0 is the reference's memcmp of the two logit rows), at a
  scaled shape and at the C4 widths (D 4096, F 14336, V 128256, H 32/8, fp8).
* Exactness: the speculative stream commits the greedy ids, through
  generate() and through captured replays, which equal eager steps bit for
  bit; the forced-acceptance gate: drafts seeded with the greedy ids advance
  the position by exactly S on every step."""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu

DT_FP8, DT_BF16 = 9, 12


def say(*a):
    print(*a, flush=True)


def up(hip, a):
    return hip.Buffer.from_numpy(np.ascontiguousarray(a))


@pytest.mark.parametrize("S", [2, 3, 4, 8])
def test_spec_draft_accept_match_oracle(hip, S):
    say(f"case: spec draft/accept kernels S={S}")
    rng = np.random.default_rng(S)
    V, cap = 50, 300
    for trial in range(48):
        alpha = 4 if trial % 2 else V            # small alphabets repeat bigrams often
        hist = rng.integers(0, alpha, cap).astype(np.int32)
        if trial % 5 == 0:
            hist[rng.integers(0, cap, 6)] = V + 3   # ids outside the vocabulary
        L = {0: 1, 1: 2, 2: cap - S, 3: cap - S + 1}.get(trial, int(rng.integers(1, cap - S)))
        forced = trial % 7 == 3
        ca_w, ce_w = O.spec_draft(hist, L, S, V, forced)
        ca, ce, hb, Lb = hip.Buffer(S * 4), hip.Buffer(S * 4), up(hip, hist), up(hip, np.array([L], np.int32))
        hip.builtin("spec_draft", [ca, ce, hb, Lb], outs=(0, 1), s=S, v=V, hcap=cap, forced=int(forced))
        got_ca, got_ce = ca.read(np.int32), ce.read(np.int32)
        assert np.array_equal(got_ca, ca_w) and np.array_equal(got_ce, ce_w), (trial, L)
        # verify ids: each draft confirmed with probability 0.7
        am = rng.integers(0, V, S).astype(np.int32)
        keep = rng.random(S - 1) < 0.7
        am[:-1] = np.where(keep & (ca_w[1:] >= 0), ca_w[1:], am[:-1])
        h_w, L_w = O.spec_accept(hist, L, ca_w, am, S)
        tok = up(hip, np.array([-7], np.int32))
        hip.builtin("spec_accept", [hb, Lb, ca, up(hip, am), tok], outs=(0, 1, 4), s=S, hcap=cap)
        assert Lb.read(np.int32)[0] == L_w, (trial, L)
        assert np.array_equal(hb.read(np.int32), h_w), (trial, L)
        assert tok.read(np.int32)[0] == (h_w[L_w - 1] if L_w != L else -7)
        for b in (ca, ce, hb, Lb, tok):
            b.free()


LLAMA = dict(arch=1, n_layers=2, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024,
             vocab=1024, max_seq=320, batch=1, eps=1e-5, rope_theta=500000.0, init_std=0.02,
             wdtype=DT_FP8, adtype=DT_BF16)
C4_1L = dict(arch=1, n_layers=1, dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
             vocab=128256, max_seq=4096, batch=1, eps=1e-5, rope_theta=500000.0, init_std=0.02,
             wdtype=DT_FP8, adtype=DT_BF16)


def _seed_history(dec, cfg, ctx, rng):
    """A token history over [0, ctx] with a repeated stretch, so the drafts
    at P = ctx are real ids; returns it."""
    h = np.zeros(cfg["max_seq"] + 1, np.int32)
    h[:ctx + 1] = rng.integers(0, cfg["vocab"], ctx + 1)
    n = min(12, ctx // 2)
    h[ctx + 1 - n:ctx + 1] = h[ctx // 4:ctx // 4 + n]      # (h[P-1], h[P]) recurs earlier
    dec.write_tensor("hist", h)
    return h


@pytest.mark.parametrize("cfg,ctx,S", [(LLAMA, 40, 4), (LLAMA, 200, 3), (C4_1L, 2048, 4)],
                         ids=["scaled-S4", "scaled-S3", "c4-width-S4"])
def test_spec_verify_rows_bit_equal_one_row_step(hip, cfg, ctx, S):
    say(f"case: spec verify rows vs one-row step, ctx={ctx} S={S} dim={cfg['dim']}")
    rng = np.random.default_rng(ctx)
    dec = hip.Decoder(seed=11, **dict(cfg, spec_rows=S))
    try:
        dec.prefill_synthetic(ctx, seed=5)
        h = _seed_history(dec, cfg, ctx, rng)
        dec.set_state([int(h[ctx])], ctx)
        dec.spec_step()
        slog = dec.read_tensor("s.logits").reshape(S, cfg["vocab"])
        ce = dec.read_tensor("s.ce")
        ca = dec.read_tensor("s.ca")
        w_ca, w_ce = O.spec_draft(h, ctx + 1, S, cfg["vocab"])
        assert np.array_equal(ca, w_ca) and np.array_equal(ce, w_ce)
        assert (ca[1:] >= 0).any(), "the planted repeat should give real drafts"
        # the one-row step on each embedded candidate at its position
        for s in range(S):
            dec.set_state([int(ce[s])], ctx + s)
            dec.step()
            base = dec.logits()[0]
            assert np.isfinite(base).all()
            assert np.array_equal(base.view(np.uint32), slog[s].view(np.uint32)), f"row {s}"
    finally:
        dec.close()


def _greedy(hip, cfg, prompt, n, seed):
    dec = hip.Decoder(seed=seed, **cfg)
    try:
        ids, cnt = dec.generate(np.array([prompt], np.int32), n)
        assert cnt[0] == n
        return ids[0]
    finally:
        dec.close()


@pytest.mark.parametrize("S", [2, 4])
def test_spec_generate_commits_the_greedy_ids(hip, S):
    say(f"case: spec generate == greedy S={S}")
    cfg = dict(LLAMA, vocab=64)                 # a small vocabulary loops soon: drafts get accepted
    prompt = [3, 9, 3, 9, 3, 9, 5, 7]
    n = 120
    want = _greedy(hip, cfg, prompt, n, seed=4)
    dec = hip.Decoder(seed=4, **dict(cfg, spec_rows=S))
    try:
        ids, cnt = dec.generate(np.array([prompt], np.int32), n)
        assert cnt[0] == n and np.array_equal(ids[0], want)
        end = dec.position + 1
        assert end >= len(prompt) + n
        say(f"  committed {end - len(prompt)} ids")
    finally:
        dec.close()


def test_spec_replay_equals_eager_and_counts_acceptance(hip):
    say("case: spec captured replay == eager")
    S, cfg = 4, dict(LLAMA, vocab=64)
    prompt = [3, 9, 3, 9, 3, 9, 5, 7]
    runs = []
    for captured in (False, True):
        dec = hip.Decoder(seed=4, **dict(cfg, spec_rows=S))
        try:
            for i, t in enumerate(prompt[:-1]):
                dec.set_state([t], i)
                dec.step()
            dec.set_state([prompt[-1]], len(prompt) - 1)
            adv = []
            for k in range(30):
                p0 = dec.position
                if captured:
                    dec.spec_capture() if k == 0 else dec.spec_replay(1)
                else:
                    dec.spec_step()
                adv.append(dec.position - p0)
            runs.append((dec.tokens(dec.position + 1)[0], dec.read_tensor("s.logits"), adv))
        finally:
            dec.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))
    assert runs[0][2] == runs[1][2] and all(1 <= a <= S for a in runs[0][2])
    n_new = len(runs[0][0]) - len(prompt)
    want = _greedy(hip, cfg, prompt, n_new, seed=4)
    assert np.array_equal(runs[0][0][len(prompt):], want)
    say(f"  30 spec steps committed {n_new} ids ({n_new / 30:.2f} per step)")


def test_spec_forced_drafts_advance_by_S(hip):
    say("case: spec forced-acceptance gate")
    S, cfg = 4, LLAMA
    prompt = [11, 200, 37, 5, 900]
    n = 40
    want = _greedy(hip, cfg, prompt, n + S, seed=6)
    dec = hip.Decoder(seed=6, **dict(cfg, spec_rows=S, spec_forced=1))
    try:
        for i, t in enumerate(prompt[:-1]):
            dec.set_state([t], i)
            dec.step()
        P = len(prompt) - 1
        dec.set_state([prompt[-1]], P)
        h = dec.read_tensor("hist")
        h[P + 1:P + 1 + len(want)] = want            # the drafts the gate seeds
        dec.write_tensor("hist", h)
        dec.spec_capture()
        steps = 1
        while dec.position - P < n:
            dec.spec_replay(1)
            steps += 1
        assert dec.position - P == S * steps
        got = dec.tokens(dec.position + 1)[0][P + 1:]
        assert np.array_equal(got, want[:len(got)])
    finally:
        dec.close()
