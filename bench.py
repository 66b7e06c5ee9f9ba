"""Decode throughput of the MI355X DEV=hip device on the BASELINE.json metric.

Default (the headline line): batch-1 greedy decode of the Llama-8B-shape fp8
model (config C4) in tokens/s, with the achieved HBM bandwidth of its dominant
kernel (the fp8 GEMV) against 8 TB/s.  `--config` selects another workload:

  C1  GPT-2 small fp32 (12L, D768, V50257), context 16, batch 1
  C2  single-op sweep: fp16 GEMV/GEMM (M 1/8/64) at the three weight shapes,
      fp16 softmax and RMSNorm over [M, 4096]
  C3  GPT-2 XL fp16 (48L, D1600, H25, F6400, V50257), context 128, batch 1 or 8
  C4  Llama-8B shape fp8 weight-only, bf16 activations, context 2048, batch 1 or 16
  C5  DeepSeek-V2-Lite shape (27L, D2048, MLA kv_lora 512, 64 experts top-6 + 2
      shared, V102400) fp8 weights, bf16 latent cache at context 4096, batch 1
      or 32 (above 4 rows: expert-grouped MoE, MFMA projections)

One "step" is one greedy decode token for every batch row: one hipGraph
replay of the captured decode step (embedding, per-layer norm + projections +
RoPE/KV append + split-sequence attention + residuals + FFN, final norm, LM
head, argmax, position bump).  Weights are synthetic N(0, 0.02) (fp8: per-row
absmax/448 e4m3), the KV cache is prefilled with N(0, 1) rows up to the
context, all generated on the device from fixed seeds.

Prints ONE JSON line per run.  The cpu_baseline leg times the CPU oracle
(oracle/oracle.c, the restatement of the reference CPU path) on one core on a
bounded sample of steps of the same model at the same context, on weights
read back from the device, in lockstep with the device (its greedy ids are
checked equal)."""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tokens/s at batch 1 and achieved HBM GB/s vs 8 TB/s peak (8B fp8)"
PEAK_GBS = 8000.0
DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13
DT_NAME = {DT_FP8: "fp8e4m3", DT_F16: "fp16", DT_BF16: "bf16", DT_F32: "fp32"}

from thvm_amd.configs import DECODERS as _DEC  # noqa: E402

MODELS = {
    "C1": dict(cfg=_DEC["C1"], ctx=16, cpu_steps=4,
               name="C1 GPT-2 small fp32 greedy decode, context 16 (prompt length)"),
    "C3": dict(cfg=_DEC["C3"], ctx=128, cpu_steps=2,
               name="C3 GPT-2 XL-shape fp16 greedy decode, KV prefilled to context 128 (prompt length)"),
    "C5": dict(cfg=_DEC["C5"], ctx=4096, cpu_steps=2,
               name="C5 DeepSeek-V2-Lite-shape MLA + MoE fp8 decode, latent cache prefilled to "
                    "context 4096"),
    "C4": dict(cfg=_DEC["C4"], ctx=2048, cpu_steps=2,
               name="C4 Llama-8B-shape fp8 weight-only decode, KV prefilled to context 2048"),
}


def _attn_on_mfma(cfg, batch) -> bool:
    """Whether the attention builtin runs its MFMA split for this decode:
    16-bit caches, head dim 64 or 128, at most 8 heads per kv head (a power of
    two), where the attention runs as two launches (more than 8 chunks of 64
    rows), unless the config forces a split."""
    G = cfg["n_heads"] // cfg["n_kv_heads"]
    n_split = (cfg["max_seq"] + 63) // 64
    one_launch = cfg.get("attn_fused", 0) == 1 or (cfg.get("attn_fused", 0) == 0 and n_split <= 8)
    if cfg.get("attn_mf", 0):
        return cfg["attn_mf"] == 1
    return (cfg.get("adtype") != 13 and cfg.get("head_dim") in (64, 128) and G <= 8 and (G & (G - 1)) == 0
            and not one_launch)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def attn_bytes_per_step(cfg, L) -> int:
    """K and V rows [0, L) of every layer and batch row, plus q read and the
    attention output written.  MLA (arch 3): the latent and k-pe rows [0, L),
    the absorbed W_uv (fp8 + row scales), qlat/q-pe read and o written."""
    B, H = cfg["batch"], cfg["n_heads"]
    if cfg["arch"] == 3:
        kv, dr, dv = cfg["kv_lora"], cfg["d_rope"], cfg["d_v"]
        per = B * (L * (kv + dr) * 2 + H * (kv * 4 + dr * 2 + dv * 2)) + H * dv * (kv + 4)
        return cfg["n_layers"] * per
    Hkv, hd = cfg["n_kv_heads"], cfg["head_dim"]
    es = 4 if cfg["adtype"] == DT_F32 else 2
    return cfg["n_layers"] * B * (2 * Hkv * L * hd * es + 2 * H * hd * es)


CPU_BUILD = None


def cpu_baseline(dec, cfg, n_steps: int):
    """Oracle decode on 1 core from the device's current state; returns
    (tokens/s, ids_match, seconds, max logit error relative to max|logit|)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np
    import _oracle as O
    pos = dec.position
    tok = dec.tokens(pos + 1)[:, pos].astype(np.int32)
    global CPU_BUILD
    try:                                       # the reference CPU JIT's flags, for this host
        CPU_BUILD = O.use_native_build(ROOT / "gpurun_out" / "oracle_native")
    except Exception as e:                     # no compiler: the shipped build, said so
        CPU_BUILD = f"shipped build (cc -std=c11 -O3 -fno-math-errno -ffp-contract=off; native build failed: {e})"
    log(f"[bench] cpu baseline oracle: {CPU_BUILD}")
    t_read = time.time()
    om = O.OracleDsv2(dec, dict(cfg)) if cfg["arch"] == 3 else O.OracleModel(dec, dict(cfg))
    log(f"[bench] cpu baseline: read back {sum(a.nbytes for a in om.keep) / 1e9:.2f} GB of "
        f"weights + {sum(a.nbytes for a in om.caches) / 1e9:.2f} GB KV in {time.time() - t_read:.1f}s")
    t_cpu, errs, match = 0.0, [], True
    cur = tok
    for s in range(n_steps):
        t0 = time.perf_counter()
        olg, onx = om.step(cur, pos + s, threads=1)      # one core, rows one after another
        t_cpu += time.perf_counter() - t0
        dec.replay(1)                              # the same step on the device
        glg = dec.logits()
        gnx = dec.tokens(pos + s + 2)[:, pos + s + 1]
        errs.append(float(np.abs(glg - olg).max() / np.abs(olg).max()))
        match = match and bool(np.array_equal(gnx, onx))
        log(f"[bench] cpu oracle step {s}: {t_cpu:.1f}s cumulative, logits rel err {errs[-1]:.2e}, "
            f"ids equal {bool(np.array_equal(gnx, onx))}")
        cur = gnx.astype(np.int32)                 # lockstep on the device's token
    return cfg["batch"] * n_steps / t_cpu, match, t_cpu, max(errs)


def run_decode(thvm, key: str, batch: int, args) -> dict:
    spec = MODELS[key]
    cfg = dict(spec["cfg"], batch=batch)
    if args.layers:
        cfg["n_layers"] = args.layers
    # --step-mode 1: the persistent step (one launch per token; LLAMA, batch
    # 1/2/4, fp8 or bf16 weights).  The default is one launch per op, which
    # measures faster at these shapes.
    persist = args.step_mode == "1"
    if persist:
        cfg["step_mode"] = 1
    if args.moe_mode and spec["cfg"].get("arch") == 3:
        cfg["moe_mode"] = args.moe_mode
    if args.attn_fused and spec["cfg"].get("arch") != 3:
        cfg["attn_fused"] = args.attn_fused
    if args.attn_mf and spec["cfg"].get("arch") != 3:
        cfg["attn_mf"] = args.attn_mf
    if args.attn_cpb and spec["cfg"].get("arch") != 3:
        cfg["attn_cpb"] = args.attn_cpb
    ctx = spec["ctx"]
    # the oracle decodes batch rows one after another on one core, so its rate
    # is the batch-1 rate; batches above 16 rows would take minutes and are
    # not run (cpu_baseline null with that note)
    cpu_steps = 0 if (args.no_cpu or batch > 16) else \
        (args.cpu_steps or (spec["cpu_steps"] if batch <= 4 else 1))
    cfg["max_seq"] = ((ctx + args.warmup + args.steps + cpu_steps + 8 + 63) // 64) * 64
    t0 = time.time()
    dec = thvm.Decoder(seed=1234, **cfg)
    dec.prefill_synthetic(ctx, seed=99)
    dec.set_state(list(range(1, batch + 1)), ctx)
    thvm.synchronize()
    log(f"[bench] {key} B={batch}: model built in {time.time() - t0:.1f}s, {dec.step_kernels()} "
        f"kernels/step, {thvm.lib().thvm_hip_mem_live_bytes() / 1e9:.2f} GB on device")

    dec.capture()                                  # step 1 (eager, recorded)
    dec.replay(max(args.warmup, 1))                # graph capture + warmup
    thvm.synchronize()
    L_mid = dec.position + args.steps // 2 + 1
    t = thvm.lib().thvm_hip_timer_start()
    t_wall = time.perf_counter()
    dec.replay(args.steps)
    ms = thvm.lib().thvm_hip_timer_stop(t)
    wall = time.perf_counter() - t_wall
    ms_per_step = ms / args.steps
    tps = batch * args.steps / (ms / 1000.0)
    log(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/step (wall {wall * 1000 / args.steps:.3f})")

    stages = None
    if persist:
        # block 0's stage clock over 4 replays: per stage type, the time between
        # barrier openings, and within a stage the wait for its barrier, the
        # block's own work and the drain of its stores
        import numpy as np
        NL = cfg["n_layers"]
        nb, ns = 5 * NL + 2, 5 * NL + 1
        names = ["qkv", "attn", "o", "gate_up", "down"]
        acc = {}
        for _ in range(4):
            dec.replay(1)
            c = dec.stage_clock()
            bar, det = c[:nb], c[nb:].reshape(ns, 4)
            span = np.diff(bar)
            for st in range(ns):
                nm = "lm_head+tail" if st == ns - 1 else names[st % 5]
                acc.setdefault(nm, []).append((span[st], det[st, 1] - det[st, 0],
                                               det[st, 2] - det[st, 1], det[st, 3] - det[st, 2]))
        stages = {nm: dict(zip(("span_us", "wait_us", "work_us", "drain_us"),
                               [round(float(x), 2) for x in np.mean(v, 0)]))
                  for nm, v in acc.items()}
        for nm, v in stages.items():
            log(f"[bench] stage {nm}: {v}")

    # live per-kernel timing: a bounded sleep kernel (~10 ms) goes first so the
    # host enqueues whole eager steps behind it and they run back to back; each
    # builtin launch carries a hipEvent pair bound to its kernels' own start and
    # end (hipExtLaunchKernel)
    dummy = thvm.Buffer(64)
    prof_steps = 2
    grouped = cfg["arch"] == 3 and batch > 4
    if grouped:   # experts the grouped MoE streams: counted on the device
        import numpy as np
        dec.write_tensor("moe.live", np.zeros(1, np.int32))
    thvm.kprof(True)
    thvm.kprof_reset()
    for _ in range(prof_steps):
        thvm.builtin("delay", [dummy], n=3000)
        dec.step()
    mla = cfg["arch"] == 3
    atag = "mla_attn" if mla else "attn"
    kern = {}
    for tag in ("gemv", "moe_gateup", "moe_down", "mla_prep", "moe_gate", "route", "norm", atag, "llama_step"):
        ms_t, n_t = thvm.kprof_query(tag)
        if n_t:
            kern[tag] = (ms_t, n_t, thvm.kprof_bytes(tag))
    thvm.kprof(False)
    dummy.free()
    L_prof = dec.position - 1
    live_per_step = None
    if grouped:
        # each live expert's gate/up and down rows (+ fp8 row scales) once per
        # layer, the shared experts once per layer, h / x / out traffic
        live = int(dec.read_tensor("moe.live")[0])
        live_per_step = live / prof_steps
        D, I, S, K, E = cfg["dim"], cfg["moe_inter"], cfg["n_shared"] * cfg["moe_inter"], cfg["top_k"], cfg["n_experts"]
        ws = 1 if cfg["wdtype"] == DT_FP8 else 2
        f8 = cfg["wdtype"] == DT_FP8
        nmoe = cfg["n_layers"] - cfg["first_dense"]
        gu_e, dn_e = 2 * I * D * ws + (8 * I if f8 else 0), D * I * ws + (4 * D if f8 else 0)
        gu_s, dn_s = 2 * S * D * ws + (8 * S if f8 else 0), D * S * ws + (4 * D if f8 else 0)
        act = batch * (K * I + S) * 4
        for tag, per_e, per_s, extra in (("moe_gateup", gu_e, gu_s, act + batch * D * 4),
                                         ("moe_down", dn_e, dn_s, act + batch * D * 4 + batch * D * 2)):
            ms_t, n_t, _ = kern[tag]
            kern[tag] = (ms_t, n_t, live * per_e + prof_steps * nmoe * (per_s + extra))
    if persist:
        # one launch holds every stage: its bytes are the weights (counted by
        # the dispatcher) plus the live KV rows of the two profiled steps
        s_ms, s_n, s_b = kern["llama_step"]
        kern["llama_step"] = (s_ms, s_n, s_b + sum(attn_bytes_per_step(cfg, L_prof - i)
                                                   for i in range(prof_steps)))
        kern[atag] = (0.0, 0, 0)
    a_ms, a_n, _ = kern[atag]
    if not persist:
        kern[atag] = (a_ms, a_n, attn_bytes_per_step(cfg, L_prof) * prof_steps)
    for tag, (ms_t, n_t, b_t) in kern.items():
        if n_t:
            log(f"[bench] {tag}: {n_t // prof_steps} launches/step, {ms_t / n_t * 1000:.1f} us avg"
                + (f", {b_t / (ms_t / 1000.0) / 1e9:.0f} GB/s" if b_t else ""))
    # the dominant kernel: the one moving the most algorithmic bytes per step
    dom = max((t for t in kern if t != atag), key=lambda t: kern[t][2])
    g_ms, g_n, g_bytes = kern[dom]
    gemv_gbs = g_bytes / (g_ms / 1000.0) / 1e9
    attn_gbs = kern[atag][2] / (a_ms / 1000.0) / 1e9 if a_ms else None
    if persist:
        step_bytes = (kern["llama_step"][2] - sum(attn_bytes_per_step(cfg, L_prof - i)
                                                  for i in range(prof_steps))) // prof_steps + \
            attn_bytes_per_step(cfg, L_mid)
    else:
        step_bytes = sum(b for t, (_, _, b) in kern.items() if t != atag) // prof_steps + \
            attn_bytes_per_step(cfg, L_mid)

    ceil = None
    if dom == "gemv" and batch <= 4 and cfg["arch"] == 1 and not persist:
        ceil = read_ceiling(thvm, dec, cfg)
        log(f"[bench] read ceiling (k_touch over the same weights, step order): {ceil:.0f} GB/s; "
            f"the GEMV reaches {gemv_gbs / ceil:.3f} of it")

    cpu = None
    if cpu_steps:
        tps_cpu, match, secs, lerr = cpu_baseline(dec, cfg, cpu_steps)
        cpu = {"value": round(tps_cpu, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"{cpu_steps} greedy decode steps x batch {batch} of the same model at "
                         f"context ~{dec.position - cpu_steps}, oracle/oracle.c or_decode_step on "
                         f"one core of {cpu_model_name()} ({os.cpu_count()} visible), in lockstep "
                         f"with the device on the same inputs",
               "seconds": round(secs, 2), "ids_match": match, "logits_max_rel_err": lerr,
               "build": CPU_BUILD}
    mfma = batch > 4
    if dom == "llama_step":
        gkern = ("k_llama_step (the whole decode step in one persistent launch: %s weight GEMVs, "
                 "split-sequence attention, LM head and argmax)" % DT_NAME[cfg["wdtype"]])
    elif dom == "gemv":
        gkern = ("k_gemm (MFMA v_mfma_f32_16x16x32, %s weights)" if mfma else
                 "k_gemv (%s weight GEMV)") % DT_NAME[cfg["wdtype"]]
    else:
        gkern = f"k_{dom} ({DT_NAME[cfg['wdtype']]} expert weights gathered by the router)"
    out = {
        "metric": METRIC, "value": round(tps, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": f"{DT_NAME[cfg['wdtype']]} weights x {DT_NAME[cfg['adtype']]} activations, "
                 "f32 accumulate",
        "data": "synthetic",
        "config": {"workload": f"{spec['name']}, batch {batch}, greedy, hipGraph replay per token",
                   "layers": cfg["n_layers"], "d_model": cfg["dim"], "heads": cfg["n_heads"],
                   "kv_heads": cfg["n_kv_heads"], "head_dim": cfg["head_dim"], "ffn": cfg["ffn"],
                   "vocab": cfg["vocab"], "batch": batch, "context": ctx,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(gemv_gbs / PEAK_GBS, 4),
                     "traffic": (measured_traffic() if key == "C4" and batch == 1 and not args.layers and not persist
                                 else None),
                     "kernel": gkern,
                     "algorithmic_bytes_per_launch": g_bytes // max(g_n, 1),
                     "launches_per_step": g_n // prof_steps,
                     "avg_launch_us": round(g_ms / g_n * 1000, 2),
                     "read_ceiling": (None if ceil is None else
                                      {"kernel": "k_touch: plain 16-byte loads over the same weight "
                                                 "matrices, one launch each, step order",
                                       "achieved": round(ceil, 1), "frac": round(ceil / PEAK_GBS, 4),
                                       "gemv_of_ceiling": round(gemv_gbs / ceil, 4)})},
        "attention": ({"kernel": "a stage of k_llama_step (its bytes are in the roofline line)"}
                      if persist else
                      {"kernel": (("k_mla_split_mf (MFMA)" if (cfg["n_heads"], cfg["kv_lora"], cfg["d_rope"]) == (16, 512, 64)
                                   else "k_mla_split") +
                                  (" + k_mla_out_q (latent quarters)" if batch == 1 and cfg["kv_lora"] % 64 == 0
                                   else " + k_mla_out") if mla else
                                  "k_attn_mf (MFMA) + k_attn_merge" if _attn_on_mfma(cfg, batch) else
                                  "k_attn_multi + k_attn_merge" if cfg["n_heads"] // cfg["n_kv_heads"] <= 4
                                  else "k_attn + k_attn_merge"),
                       "achieved_gbs": round(attn_gbs, 1), "frac": round(attn_gbs / PEAK_GBS, 4),
                       "avg_launch_us": round(a_ms / max(a_n, 1) * 1000, 2)}),
        "kernels": {t: {"launches_per_step": n_t // prof_steps,
                        "avg_launch_us": round(ms_t / n_t * 1000, 2),
                        "gbs": round(b_t / (ms_t / 1000.0) / 1e9, 1) if b_t else None}
                    for t, (ms_t, n_t, b_t) in kern.items() if n_t},
        "step_mode": "persistent (one launch per step)" if persist else "one launch per op (hipGraph)",
        **({"stage_clock": stages} if stages else {}),
        "step_hbm_gbs": round(step_bytes / (ms_per_step / 1000.0) / 1e9, 1),
        "step_bytes": step_bytes,
        "kernels_per_step": dec.step_kernels(),
        **({"moe_live_experts_per_layer": round(live_per_step / (cfg["n_layers"] - cfg["first_dense"]), 2)}
           if live_per_step is not None else {}),
        "cpu_baseline": cpu if cpu or batch <= 16 else
        {"value": None, "note": "not run above 16 rows: the oracle decodes rows serially on one core, "
                                "so its tokens/s is the batch-1 configuration's"},
    }
    if args.layers:
        out["config"]["note"] = "DEBUG: reduced layer count, not the configured model"
    dec.close()
    return out


def run_c2(thvm, args) -> dict:
    """Single-op sweep: each op launched `reps` times behind a sleep kernel,
    with a cache-evicting copy before every launch; kernel time from the event
    pairs bound to each launch."""
    import numpy as np
    rng = np.random.default_rng(7)
    reps = 20
    ops = []
    # a 256 MiB copy between launches evicts the 256 MB Infinity Cache, so each
    # timed launch reads its operands from HBM as a decode step would
    flush = thvm.Buffer(512 << 20)
    half = thvm.lib().thvm_hip_buf_view(flush.id, 256 << 20, 256 << 20)

    def timed(tag, fn):
        dummy = thvm.Buffer(64)
        fn()                                       # warm (code object load)
        thvm.synchronize()
        thvm.kprof(True)
        thvm.kprof_reset()
        thvm.builtin("delay", [dummy], n=1000)
        for _ in range(reps):
            thvm.dispatch("flush", "thvm-builtin:copy n=%d" % (256 << 20), [flush.id, half])
            fn()
        ms, n = thvm.kprof_query(tag)
        nb = thvm.kprof_bytes(tag)
        thvm.kprof(False)
        dummy.free()
        return ms / n * 1000.0, nb / n

    def f16(a):
        return a.astype(np.float16).view(np.uint16)

    for N, K in ((4096, 4096), (14336, 4096), (50257, 768)):
        w = thvm.Buffer.from_numpy(f16(rng.standard_normal((N, K), np.float32) * 0.02))
        for M in (1, 8, 64):
            x = thvm.Buffer.from_numpy(f16(rng.standard_normal((M, K), np.float32)))
            y = thvm.Buffer(M * N * 4)
            us, nb = timed("gemv", lambda: thvm.builtin("gemv", [y, x, w], m=M, n=N, k=K, wt=DT_F16,
                                                        xt=DT_F16, yt=DT_F32, epi=0))
            gbs = nb / (us * 1e-6) / 1e9
            ops.append({"op": "gemv" if M <= 4 else "gemm_mfma", "N": N, "K": K, "M": M,
                        "us": round(us, 2), "bytes": int(nb), "gbs": round(gbs, 1),
                        "frac": round(gbs / PEAK_GBS, 4),
                        "tflops": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 2)})
            x.free()
            y.free()
        w.free()
    K = 4096
    g = thvm.Buffer.from_numpy(np.ones(K, np.float32))
    for M in (1, 8, 64):
        x = thvm.Buffer.from_numpy(f16(rng.standard_normal((M, K), np.float32)))
        y = thvm.Buffer(M * K * 2)
        us, nb = timed("softmax", lambda: thvm.builtin("softmax", [y, x], m=M, k=K, xt=DT_F16,
                                                       yt=DT_F16))
        ops.append({"op": "softmax", "M": M, "K": K, "us": round(us, 2), "bytes": int(nb),
                    "gbs": round(nb / (us * 1e-6) / 1e9, 1)})
        us, nb = timed("norm", lambda: thvm.builtin("norm", [y, x, g], m=M, k=K, xt=DT_F16,
                                                    yt=DT_F16, eps=1e-6))
        ops.append({"op": "rmsnorm", "M": M, "K": K, "us": round(us, 2), "bytes": int(nb),
                    "gbs": round(nb / (us * 1e-6) / 1e9, 1)})
        x.free()
        y.free()
    g.free()
    thvm.lib().thvm_hip_buf_free(half)
    flush.free()
    mats = [o for o in ops if o["op"] in ("gemv", "gemm_mfma")]
    best = max(mats, key=lambda o: o["gbs"])
    return {"metric": "C2 single-op sweep: kernel time and achieved HBM GB/s vs 8 TB/s",
            "value": best["gbs"], "unit": "GB/s (best GEMV/GEMM)", "n_gpus": 1, "steps": reps,
            "warmup": 1, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp16 in, f32 accumulate", "data": "synthetic",
            "config": {"workload": "C2 fp16 GEMV/GEMM y=x.W^T (N,K) in {(4096,4096),(14336,4096),"
                                   "(50257,768)}, M in {1,8,64}; softmax and RMSNorm eps 1e-6 over "
                                   "[M,4096] fp16"},
            "roofline": {"bound": "hbm", "achieved": best["gbs"], "peak": PEAK_GBS, "unit": "GB/s",
                         "frac": best["frac"], "traffic": None,
                         "kernel": f"{best['op']} N={best['N']} K={best['K']} M={best['M']}"},
            "ops": ops, "cpu_baseline": None}


COPY_BYTES = 1 << 30


def copy_calibration(thvm) -> int:
    """A plain copy of COPY_BYTES, 4 launches: each reads and writes exactly
    COPY_BYTES, so a counter's reading per dispatch over COPY_BYTES/1024 is
    its KiB scale."""
    src, dst = thvm.Buffer(COPY_BYTES), thvm.Buffer(COPY_BYTES)
    thvm.kprof(True)
    thvm.kprof_reset()
    for _ in range(4):
        thvm.builtin("copy", [dst, src], n=COPY_BYTES)
    ms, n = thvm.kprof_query("copy")
    thvm.kprof(False)
    src.free()
    dst.free()
    us = ms / n * 1000
    print(json.dumps({"calibration": "copy", "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES,
                      "launches": n, "avg_launch_us": round(us, 2),
                      "gbs": round(2 * COPY_BYTES / (us * 1e-6) / 1e9, 1)}), flush=True)
    return 0


def read_ceiling(thvm, dec, cfg, passes=2):
    """What one plain-read launch reaches over the same bytes: k_touch (16-byte
    loads over the whole range, 2048 blocks of 256 threads -- the best of a
    512..8192 sweep at every C4 shape -- nothing computed)
    over each weight matrix of the LLAMA step's GEMV launches, in step order
    (qkv, o, gate/up, down per layer, then the LM head), timed like the GEMV
    (event pairs on the kernels, queued behind a sleep kernel so they run back
    to back).  The whole pass reads every weight once, more than the 256 MB
    last-level cache holds, so each launch reads cold.  Returns GB/s."""
    names = [f"l{i}.{w}" for i in range(cfg["n_layers"]) for w in ("wqkv", "wo", "wgu", "wd")] + ["lm"]
    bufs = [dec.tensor(n) for n in names]
    sink, dummy = thvm.Buffer(2048 * 4), thvm.Buffer(64)
    thvm.kprof(True)
    thvm.kprof_reset()
    for _ in range(passes):
        thvm.builtin("delay", [dummy], n=3000)
        for bid, _, nb in bufs:
            thvm.builtin("touch", [bid, sink], outs=(1,), n=nb, blocks=2048)
    ms, _ = thvm.kprof_query("touch")
    nbytes = thvm.kprof_bytes("touch")
    thvm.kprof(False)
    sink.free()
    dummy.free()
    return nbytes / (ms / 1000.0) / 1e9


def measured_traffic():
    """HBM bytes per k_gemv launch of the C4 batch-1 step from the committed
    counter passes (FETCH_SIZE, WRITE_SIZE, each scaled by the plain-copy
    calibration), or None when that summary is absent."""
    p = ROOT / "profiles" / "gemv_fp8_c4_traffic.json"
    try:
        return int(json.loads(p.read_text())["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def run_host_gpt2(thvm, key: str, args) -> dict:
    """C1 / C3 through the Python Tensor host (thvm_amd.tensor + TinyJit):
    the reference's GPT-2 driver path (bench/gpt2/thvm_gpt2.py) rather than
    the C decoder.  A step is one greedy token end to end: token upload,
    TinyJit replay of the captured graph, token read-back."""
    import numpy as np
    from thvm_amd import tensor as T
    from thvm_amd.gpt2 import GPT2
    spec = MODELS[key]
    c = spec["cfg"]
    L = args.layers or c["n_layers"]
    ctx = spec["ctx"]
    max_ctx = ((ctx + args.warmup + args.steps + 8 + 63) // 64) * 64
    w = GPT2.synthetic_weights(L, c["dim"], c["vocab"], max_ctx, seed=1234, std=c["init_std"])
    if c["wdtype"] == DT_F16:
        w = {k: v.astype(np.float16) for k, v in w.items()}
    g = GPT2(w, L, c["n_heads"], c["dim"], c["vocab"], max_ctx)
    prompt = [(7 * i + 3) % c["vocab"] for i in range(ctx)]
    t0 = time.time()
    cur = np.array([prompt[0]], np.int32)
    for pos in range(ctx - 1):                      # prompt, one token at a time (captures the JIT)
        g.step(cur, pos)
        cur = np.array([prompt[pos + 1]], np.int32)
    pos = ctx - 1
    for _ in range(args.warmup):
        cur = g.step(cur, pos).astype(np.int32)
        pos += 1
    log(f"[bench] host {key}: prompt + warmup {time.time() - t0:.1f}s, "
        f"{T.GlobalCounters.kernel_count} rendered + {T.GlobalCounters.gemv_count} GEMV dispatches so far")
    thvm.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        cur = g.step(cur, pos).astype(np.int32)
        pos += 1
    thvm.synchronize()
    dt = time.perf_counter() - t1
    jit = g.jit
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, str(ROOT / "tests"))
        import _oracle as O

        class _W:
            def __init__(s):
                s.t = {k: np.ascontiguousarray(v, np.float32) for k, v in w.items()}
                hd = c["dim"] // c["n_heads"]
                for l in range(L):
                    s.t[f"l{l}.kcache"] = np.zeros((1, c["n_heads"], max_ctx, hd), np.float32)
                    s.t[f"l{l}.vcache"] = np.zeros((1, c["n_heads"], max_ctx, hd), np.float32)

            def read_tensor(s, name):
                return s.t[name]
        ocfg = dict(c, n_layers=L, batch=1, max_seq=max_ctx, wdtype=DT_F32, adtype=DT_F32)
        try:
            build = O.use_native_build(ROOT / "gpurun_out" / "oracle_native")
        except Exception as e:
            build = f"shipped build (native build failed: {e})"
        om = O.OracleModel(_W(), ocfg)
        n_cpu = args.cpu_steps or 2
        tc = time.perf_counter()
        for s in range(n_cpu):
            om.step(np.array([prompt[s]], np.int32), s)
        tcpu = time.perf_counter() - tc
        cpu = {"value": round(n_cpu / tcpu, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"{n_cpu} decode steps of the same model (fp32) from position 0 on the C oracle",
               "build": build}
    return {"metric": METRIC, "value": round(args.steps / dt, 2), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": f"{DT_NAME[c['wdtype']]} weights and activations, f32 accumulate",
            "data": "synthetic",
            "config": {"workload": spec["name"] + ", through the Python Tensor host (TinyJit replay)",
                       "layers": L, "d_model": c["dim"], "heads": c["n_heads"], "vocab": c["vocab"],
                       "batch": 1, "context": ctx, "parallelism": "single GPU", "path": "tensor-host",
                       "matmul": "rendered" if args.host_rendered else "gemv builtin",
                       "beam": args.beam},
            "jit_kernels_per_step": int(jit.jit.op_count()) if jit.jit is not None else None,
            "cpu_baseline": cpu}


def run_spec(thvm, args) -> dict:
    """Speculative decode at C4 batch 1 (decoder spec_rows S): one captured
    spec step = a bigram draft of S-1 ids, S verify rows of the sequence,
    argmax and the commit.  Two measurements on the same model and context:
    forced acceptance (spec_forced: the drafts are the greedy ids a base run
    recorded, so every step commits S ids -- the throughput at full
    acceptance), and the bigram draft on the model's own output (how many
    ids it commits per step here).  The base one-row step is timed beside."""
    import numpy as np
    S = args.spec
    spec = MODELS["C4"]
    ctx, n = spec["ctx"], args.steps
    res = {}
    for forced in (1, 0):
        cfg = dict(spec["cfg"], batch=1, spec_rows=S, spec_forced=forced)
        cfg["max_seq"] = ((ctx + (n + 2) * S + args.warmup * S + 72 + 63) // 64) * 64
        dec = thvm.Decoder(seed=1234, **cfg)
        try:
            dec.prefill_synthetic(ctx, seed=99)
            dec.set_state([1], ctx)
            dec.capture()
            m = (n + args.warmup + 4) * S
            dec.replay(m - 1)                        # the greedy continuation (base step)
            thvm.synchronize()
            greedy = dec.tokens(ctx + m + 1)[0][ctx + 1:].copy()
            dec.set_state([1], ctx)
            t = thvm.lib().thvm_hip_timer_start()
            dec.replay(n)
            base_ms = thvm.lib().thvm_hip_timer_stop(t) / n
            dec.set_state([1], ctx)
            if forced:
                h = dec.read_tensor("hist")
                h[ctx + 1:ctx + 1 + len(greedy)] = greedy
                dec.write_tensor("hist", h)
            dec.spec_capture()
            dec.spec_replay(max(args.warmup, 1))
            thvm.synchronize()
            p0 = dec.position
            t = thvm.lib().thvm_hip_timer_start()
            dec.spec_replay(n)
            ms = thvm.lib().thvm_hip_timer_stop(t)
            adv = dec.position - p0
            got = dec.tokens(dec.position + 1)[0][ctx + 1:]
            ok = bool(np.array_equal(got, greedy[:len(got)]))
            res[forced] = dict(ms_per_step=ms / n, ids_per_step=adv / n, tokens_per_s=adv / (ms / 1000.0),
                               base_ms=base_ms, greedy_equal=ok)
            log(f"[bench] spec S={S} forced={forced}: {ms / n:.3f} ms per spec step, {adv / n:.2f} ids per step, "
                f"{adv / (ms / 1000.0):.1f} tok/s (base step {base_ms:.3f} ms); committed ids == greedy: {ok}")
        finally:
            dec.close()
    f, b = res[1], res[0]
    return {"metric": METRIC, "value": round(f["tokens_per_s"], 2), "unit": "tokens/s", "n_gpus": 1,
            "steps": n, "warmup": args.warmup, "ms_per_step": round(f["ms_per_step"], 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp8e4m3 weights x bf16 activations, f32 accumulate", "data": "synthetic",
            "config": {"workload": f"C4 Llama-8B-shape fp8 speculative decode, S={S} verify rows, forced "
                                   "acceptance (drafts = the recorded greedy ids), KV prefilled to context 2048",
                       "batch": 1, "context": ctx, "spec_rows": S, "parallelism": "single GPU"},
            "base_step_ms": round(f["base_ms"], 4),
            "speedup_vs_base_at_full_acceptance": round(f["tokens_per_s"] * f["base_ms"] / 1000.0, 3),
            "bigram_draft": {"ids_per_step": round(b["ids_per_step"], 3), "tokens_per_s": round(b["tokens_per_s"], 2),
                             "ms_per_step": round(b["ms_per_step"], 4)},
            "committed_ids_equal_greedy": f["greedy_equal"] and b["greedy_equal"]}


PHASES = {
    "gemv": ["entry", "loads issued", "x staged", "first batch consumed", "rows done", "partials summed",
             "t0 x arrived", "end (drained)"],
    "attn": ["entry", "loads issued + q", "first chunk consumed", "chunks done", "row groups combined",
             "waves in LDS", "", "end (drained)"],
    "merge": ["entry", "partials folded", "partitions combined", "", "", "", "", "end (drained)"],
    "mla_prep": ["entry", "q nope staged / latent row read", "", "", "", "", "", "end (drained)"],
    "mla_split": ["entry", "q staged", "first chunk scored", "first chunk softmax", "chunks done",
                  "rows issued", "t0 rows arrived", "end (drained)"],
    "mla_out": ["entry", "split weights", "partials summed", "olat in LDS", "loads issued",
                "t0 m,l arrived", "t0 W_uv arrived", "end (drained)"],
    "moe_gate": ["entry", "loads issued", "x normalised", "", "", "", "", "end (drained)"],
    "moe_gateup": ["entry", "top-K picked", "rows issued", "x staged", "t0 logits arrived", "t0 rows arrived",
                   "wave 0 routed", "end (drained)"],
    "moe_down": ["entry", "rows issued", "h staged", "half sums", "t0 ids arrived", "t0 rows arrived", "",
                 "end (drained)"],
}
# ops with phase-clock marks: kernel name -> (first launch's kind, second launch's kind or None)
CLOCKED = {"gemv": ("gemv", None), "attn": ("attn", "merge"), "mla_prep": ("mla_prep", None),
           "mla_attn": ("mla_split", "mla_out"), "moe_gate": ("moe_gate", None),
           "moe_gateup": ("moe_gateup", None), "moe_down": ("moe_down", None)}


def _clock_record(rec, name, kern, c):
    """Fold one launch's clock slots ([2][blocks][10]) into rec: per mark, the
    median and the maximum over blocks in us after the earliest block's entry,
    and per XCD the earliest entry (launch stagger across the 8 XCDs).
    Returns the op's earliest entry and latest end (clock ticks) for the
    layer timeline."""
    import numpy as np
    k0, k1 = CLOCKED[kern]
    parts = [(k0, c[0])]
    if k1 and c[1, :, 0].any():
        parts.append((k1, c[1]))
    if not (c[0, :, 0] > 0).any():
        raise RuntimeError(f"{name}: no phase-clock marks recorded (the kernels come from the "
                           "measurement build libthvm_hip_pclk.so: python -m thvm_amd.build --variant pclk)")
    t0 = min(int(p[p[:, 0] > 0, 0].min()) for _, p in parts)
    for pname, p in parts:
        live = p[p[:, 0] > 0]
        key = f"{name}/{pname}" if pname == k1 else name
        r = rec.setdefault(key, {"kind": pname, "blocks": len(live), "marks": [], "xcd_entry": []})
        row = []
        for m in range(8):
            v = live[:, m]
            v = v[v > 0]
            row.append((float(np.median(v - t0)) / 100.0, float((v - t0).max()) / 100.0)
                       if len(v) else (None, None))
        r["marks"].append(row)
        xe = [float((live[live[:, 8] == x, 0] - t0).min()) / 100.0 if (live[:, 8] == x).any() else None
              for x in range(8)]
        r["xcd_entry"].append(xe)
    ends = [int(p[p[:, 7] > 0, 7].max()) for _, p in parts if (p[:, 7] > 0).any()]
    return t0, (max(ends) if ends else t0)


def run_phase_clock(thvm, args) -> dict:
    """Per-phase clock of one layer's kernels inside an eager step: the
    step runs op by op; the ops of layer `--clock-layer` are re-dispatched
    with the builtin's clk= option (thread 0 of every block records the 100
    MHz wall clock at marks; see the kernels' pclk calls).  Per op and mark:
    the median and the maximum over blocks, in us after the earliest block's
    entry; over `--steps` steps, the median of those."""
    import numpy as np
    spec = MODELS[args.config if args.config != "all" else "C4"]
    cfg = dict(spec["cfg"], batch=args.batch)
    ctx = spec["ctx"]
    cfg["max_seq"] = ((ctx + args.steps + args.warmup + 8 + 63) // 64) * 64
    dec = thvm.Decoder(seed=1234, **cfg)
    dec.prefill_synthetic(ctx, seed=99)
    dec.set_state(list(range(1, args.batch + 1)), ctx)
    dec.capture()
    dec.replay(max(args.warmup, 1))
    thvm.synchronize()
    layer = args.clock_layer
    tags = dec.op_tags()
    ops = [i for i in range(len(tags)) if tags[i] in (2 * layer, 2 * layer + 1)]
    CAP, NS = 2048, 10
    clk = thvm.Buffer(CAP * 2 * NS * 8)
    zero = np.zeros(CAP * 2 * NS, np.uint64)
    rec, raw, timeline = {}, {}, {}
    if args.clock_graph:
        # the whole step captured as one graph (as the decoder replays it), the
        # layer's GEMV / attention ops with clocks of their own
        bufs, info = {}, []
        with thvm.Jit() as j:
            for i in range(len(tags)):
                name, prog, ids = dec.op_info(i)
                kern = prog.split()[0].split(":")[1]
                if i in ops and kern in CLOCKED:
                    bufs[i] = thvm.Buffer(CAP * 2 * NS * 8)
                    bufs[i].write(zero)
                    thvm.dispatch(name, prog + f" clk={CAP}", ids + [bufs[i].id])
                    info.append((i, name, kern))
                else:
                    thvm.dispatch(name, prog, ids)
        for s in range(args.steps):
            for b in bufs.values():
                b.write(zero)
            j.replay()
            thvm.synchronize()
            spans = {}
            for i, name, kern in info:
                c = bufs[i].read(np.uint64).reshape(2, CAP, NS).astype(np.int64)
                raw.setdefault(name, []).append(c.copy())
                spans[name] = _clock_record(rec, name, kern, c)
            # the layer timeline: each op's first entry and last end after
            # the layer's first op entered (launch gaps between the ops)
            base = min(v[0] for v in spans.values())
            for name, (t0, t1) in spans.items():
                timeline.setdefault(name, []).append(((t0 - base) / 100.0, (t1 - base) / 100.0))
        j.drop()
    for s in range(0 if args.clock_graph else args.steps):
        i = 0
        while i < len(tags):
            if i not in ops:
                j = i
                while j < len(tags) and j not in ops:
                    j += 1
                dec.run_ops(i, j - i)
                i = j
                continue
            name, prog, ids = dec.op_info(i)
            kern = prog.split()[0].split(":")[1]
            if kern not in CLOCKED:
                dec.run_ops(i, 1)
                i += 1
                continue
            clk.write(zero)
            thvm.dispatch(name, prog + f" clk={CAP}", ids + [clk.id])
            c = clk.read(np.uint64).reshape(2, CAP, NS).astype(np.int64)
            raw.setdefault(name, []).append(c.copy())
            _clock_record(rec, name, kern, c)
            i += 1
    rdir = ROOT / "gpurun_out"
    rdir.mkdir(exist_ok=True)
    np.savez_compressed(rdir / ("phase_clock_graph_raw.npz" if args.clock_graph else "phase_clock_raw.npz"),
                        **{k: np.stack(v) for k, v in raw.items()})
    out = {}
    for key, r in rec.items():
        names = PHASES[r["kind"]]
        marks = {}
        for m in range(8):
            vals = [row[m] for row in r["marks"] if row[m][0] is not None]
            if not vals or not names[m]:
                continue
            marks[names[m]] = {"median_us": round(float(np.median([v[0] for v in vals])), 2),
                               "max_us": round(float(np.median([v[1] for v in vals])), 2)}
        xe = np.array([[v if v is not None else np.nan for v in row] for row in r["xcd_entry"]])
        stagger = [round(float(v), 2) for v in np.nanmedian(xe, 0)]
        out[key] = {"blocks": r["blocks"], "marks": marks, "xcd_first_entry_us": stagger}
        if key in timeline:
            tl = np.array(timeline[key])
            out[key]["layer_span_us"] = [round(float(np.median(tl[:, 0])), 2), round(float(np.median(tl[:, 1])), 2)]
        log(f"[clock] {key} ({r['blocks']} blocks): " +
            ", ".join(f"{k} {v['median_us']}/{v['max_us']}" for k, v in marks.items()) +
            f"; first entry per XCD {stagger}" +
            (f"; in layer {out[key]['layer_span_us']}" if "layer_span_us" in out[key] else ""))
    dec.close()
    return {"metric": "phase clock (us after the earliest block's entry: median/max over blocks)",
            "config": {"workload": spec["name"], "layer": layer, "batch": args.batch, "steps": args.steps,
                       "context": ctx, "mode": "graph replay" if args.clock_graph else "eager"},
            "ops": out}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--config", default="C4", choices=["C1", "C2", "C3", "C4", "C5", "all"])
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--cpu-steps", type=int, default=0, help="oracle steps (0: the config's default)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--step-mode", default="0", choices=["0", "1"],
                    help="0: one launch per op (hipGraph); 1: the persistent one-launch step (LLAMA)")
    ap.add_argument("--attn-fused", type=int, default=0, choices=[0, 1, 2],
                    help="attention form: 0 auto, 1 one launch, 2 split + merge launches")
    ap.add_argument("--attn-mf", type=int, default=0, choices=[0, 1, 2],
                    help="attention split: 0 picked by the kernel, 1 MFMA, 2 VALU")
    ap.add_argument("--attn-cpb", type=int, default=0,
                    help="attention split: 64-row chunks per block (0: picked by the kernel)")
    ap.add_argument("--moe-mode", type=int, default=0, choices=[0, 1, 2],
                    help="DSV2 above 4 rows: expert-grouped MoE on MFMA (0/2) or on the VALU (1)")
    ap.add_argument("--layers", type=int, default=None, help="debug only: fewer layers (invalid metric)")
    ap.add_argument("--host-rendered", action="store_true",
                    help="with --host: matmuls rendered like every other kernel (THVM_HOST_GEMV=0), "
                         "no GEMV builtin")
    ap.add_argument("--beam", type=int, default=0,
                    help="with --host: BEAM width for the rendered kernels' geometry search (0: hand-coded)")
    ap.add_argument("--spec", type=int, default=0,
                    help="C4 batch 1 speculative decode with S verify rows (2..4): forced-acceptance "
                         "throughput and the bigram draft's ids per step")
    ap.add_argument("--phase-clock", action="store_true",
                    help="per-phase wall clock of one layer's GEMV and attention kernels inside an "
                         "eager step (measurement, not the metric)")
    ap.add_argument("--clock-layer", type=int, default=16)
    ap.add_argument("--clock-graph", action="store_true",
                    help="with --phase-clock: the step captured and replayed as one graph")
    ap.add_argument("--host", action="store_true",
                    help="C1/C3: run the GPT-2 driver on the Python Tensor host (TinyJit) "
                         "instead of the C decoder")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only the plain 1 GiB copy kernel that calibrates the HBM traffic "
                         "counters (FETCH_SIZE/WRITE_SIZE) and print its timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        return 2

    if args.phase_clock:           # the measurement build: kernels with phase-clock marks
        os.environ["THVM_HIP_LIB_VARIANT"] = "pclk"
    if args.host_rendered:
        os.environ["THVM_HOST_GEMV"] = "0"
    if args.beam:
        os.environ["BEAM"] = str(args.beam)
    import thvm_amd as thvm
    thvm.init()
    try:
        if args.copy_calibration:
            return copy_calibration(thvm)
        if args.spec:
            print(json.dumps(run_spec(thvm, args)), flush=True)
            return 0
        if args.phase_clock:
            print(json.dumps(run_phase_clock(thvm, args)), flush=True)
            return 0
        if args.config == "all":
            runs = [("C4", 1), ("C4", 16), ("C5", 1), ("C5", 32), ("C3", 1), ("C3", 8), ("C1", 1), ("C2", 0)]
        else:
            runs = [(args.config, args.batch)]
        for key, batch in runs:
            if args.host and key in ("C1", "C3"):
                out = run_host_gpt2(thvm, key, args)
            else:
                out = run_c2(thvm, args) if key == "C2" else run_decode(thvm, key, batch, args)
            print(json.dumps(out), flush=True)
    finally:
        thvm.shutdown()
    return 0


if __name__ == "__main__":
    sys.exit(main())
