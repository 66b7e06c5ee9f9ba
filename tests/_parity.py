"""Teacher-forced lockstep between a device decoder and the CPU oracle
(test infrastructure).

Both sides are fed the same token ids at every position: after each step
the device's next token is overwritten with the oracle's greedy id
(``set_state``), so a near-tie fork in the ids does not end the comparison;
every step's logits are held to the bar.

Bars:
  * fp32 activations: logits within 1e-5 of max|logit| (relative) and greedy
    ids identical on every step;
  * fp8 weights: logits within 2e-2 relative;
  * fp16 / bf16 weights with 16-bit activations: logits within 1e-2 absolute;
  * 16-bit activations: a greedy id may differ from the oracle's only at a
    near tie -- the oracle's logit of the device's pick lies within twice the
    step's measured logit drift of the oracle's maximum (asserted, with the
    margin printed);
  * the device's argmax equals the host argmax of the device logits (lowest
    index on ties), bit for bit.

DeepSeek-V2: every MoE layer's routing is compared each step (``l<i>.sel``
against the oracle's per-layer record).  The same expert set in another slot
order is accepted at a proven near tie (the swapped experts' router logits
within twice the drift); a different set likewise (the oracle's K-th /
(K+1)-th gap within twice the drift), after which that row runs a
legitimately different computation and is not compared further."""
from __future__ import annotations

import numpy as np

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13


def say(*a):
    print(*a, flush=True)


def logit_bar(cfg):
    """(kind, tolerance) for this config."""
    if cfg["adtype"] == DT_F32:
        return "rel", 1e-5
    if cfg["wdtype"] == DT_FP8:
        return "rel", 2e-2
    return "abs", 1e-2


def _err(glg, olg, kind):
    d = np.abs(glg.astype(np.float64) - olg.astype(np.float64)).max()
    return d / np.abs(olg).max() if kind == "rel" else d


def check_routing(dec, om, cfg, s, forked):
    """Per-layer routing of one step; returns rows that forked (sets differ)."""
    B, K = cfg["batch"], cfg["top_k"]
    new = set()
    for l in range(cfg.get("first_dense", 0), cfg["n_layers"]):
        gsel = dec.read_tensor(f"l{l}.sel").reshape(B, K)
        ggl = dec.read_tensor(f"l{l}.gate_logits").reshape(B, -1)
        osel, ogl = om.sel[l], om.gate[l]
        for b in range(B):
            if b in forked or b in new:
                continue
            if np.array_equal(gsel[b], osel[b]):
                continue
            drift = float(np.abs(ggl[b] - ogl[b]).max())
            if np.array_equal(np.sort(gsel[b]), np.sort(osel[b])):
                ex = np.union1d(gsel[b][gsel[b] != osel[b]], osel[b][gsel[b] != osel[b]])
                gap = float(ogl[b][ex].max() - ogl[b][ex].min())
                say(f"  step {s} layer {l} row {b}: slot order {gsel[b]} vs {osel[b]}, "
                    f"gap {gap:.3g} drift {drift:.3g}")
                assert gap <= 2 * drift, f"step {s} layer {l} row {b}: slot swap gap {gap} > 2 x drift {drift}"
                continue
            srt = np.sort(ogl[b])[::-1]
            gap = float(srt[K - 1] - srt[K])
            say(f"  step {s} layer {l} row {b}: routing fork {np.sort(gsel[b])} vs {np.sort(osel[b])}, "
                f"K-th gap {gap:.3g} drift {drift:.3g}")
            assert gap <= 2 * drift, f"step {s} layer {l} row {b}: routing gap {gap} > 2 x drift {drift}"
            new.add(b)
    return new


def lockstep(dec, om, cfg, tok, pos0, steps, label="", prompt=None):
    """Run `steps` teacher-forced steps from position pos0 with ids `tok`.
    `prompt` (optional, [n] ids) is consumed first, one position at a time,
    with the same checks.  Returns a summary dict."""
    B = cfg["batch"]
    kind, tol = logit_bar(cfg)
    dsv2 = cfg["arch"] == 3
    if prompt is not None:
        tok = np.full(B, prompt[0], np.int32)
    tok = np.asarray(tok, np.int32).reshape(B)
    n_prompt = 0 if prompt is None else len(prompt) - 1
    dec.set_state(tok, pos0)
    worst, forks, ties, forked = 0.0, 0, [], set()
    total = n_prompt + steps
    for s in range(total):
        pos = pos0 + s
        dec.step()
        glg = dec.logits()
        gnx = dec.tokens(pos + 2)[:, pos + 1]
        olg, onx = om.step(tok, pos)
        assert np.array_equal(gnx, np.argmax(glg, 1)), f"step {s}: device argmax != host argmax"
        assert np.all(np.isfinite(glg)), f"step {s}: non-finite device logits"
        if dsv2:
            forked |= check_routing(dec, om, cfg, s, forked)
        for b in range(B):
            if b in forked:
                continue
            e = _err(glg[b], olg[b], kind)
            worst = max(worst, e)
            assert e <= tol, f"{label} step {s} row {b}: logits {kind} err {e:.4g} > {tol}"
            if gnx[b] != onx[b]:
                drift = float(np.abs(glg[b].astype(np.float64) - olg[b]).max())
                margin = float(olg[b][onx[b]] - olg[b][gnx[b]])
                ties.append((s, b, margin, drift))
                say(f"  {label} step {s} row {b}: id {gnx[b]} vs oracle {onx[b]}, oracle margin "
                    f"{margin:.3g}, drift {drift:.3g}")
                assert cfg["adtype"] != DT_F32, f"step {s}: fp32 greedy ids must be identical"
                assert margin <= 2 * drift, f"step {s} row {b}: id fork with margin {margin} > 2 x drift {drift}"
                forks += 1
        tok = np.full(B, prompt[s + 1], np.int32) if s < n_prompt else onx.astype(np.int32)
        dec.set_state(tok, pos + 1)
    say(f"  {label}: {total} steps x {B} rows, worst logits {kind} err {worst:.3g} (bar {tol}), "
        f"id forks at near ties {forks}, routing forks {len(forked)}")
    return dict(worst=worst, forks=forks, ties=ties, routing_forks=len(forked))
