"""ctypes access to the CPU oracle (oracle/build/liboracle.so) and, when it was
built here, the reference harness (oracle/_ref/libref.so).  Test
infrastructure: the checker, never the thing measured."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "build" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libref.so"

_f, _u8, _u16, _u32, _u64, _vp, _i = (C.c_float, C.c_uint8, C.c_uint16, C.c_uint32, C.c_uint64,
                                      C.c_void_p, C.c_int)


class OrLayer(C.Structure):
    _fields_ = [(n, _vp) for n in ("wqkv", "sqkv", "wo", "so", "wgu", "sgu", "wd", "sd",
                                   "g1", "b1", "g2", "b2", "bqkv", "bo", "bfc", "bpr",
                                   "kcache", "vcache")]


class OrModel(C.Structure):
    _fields_ = [(n, _u32) for n in ("arch", "n_layers", "dim", "n_heads", "n_kv_heads",
                                    "head_dim", "ffn", "vocab", "max_seq", "batch", "wdt",
                                    "adt")] + [("eps", _f)] + [
        (n, _vp) for n in ("emb", "pos_emb", "gf", "bf", "lm", "lm_s", "rope_cos", "rope_sin")] + [
        ("layers", C.POINTER(OrLayer))] + [
        (n, _vp) for n in ("tf_x", "tp_x", "tp_q", "tp_att", "tp_h")] + [("b0", _u32), ("b1", _u32)]


class OrDsv2Layer(C.Structure):
    _fields_ = [(n, _vp) for n in (
        "win", "wkvn", "wpost", "wqkv", "sqkv", "wuk", "suk", "wuv", "suv", "wo", "so",
        "wgu", "sgu", "wd", "sd", "gate", "wgu_e", "sgu_e", "wd_e", "sd_e",
        "wgu_s", "sgu_s", "wd_s", "sd_s", "ckv", "kpe")]


class OrDsv2(C.Structure):
    _fields_ = [(n, _u32) for n in (
        "n_layers", "dim", "n_heads", "kv_lora", "d_nope", "d_rope", "d_v", "n_experts",
        "n_shared", "top_k", "moe_inter", "dense_inter", "first_dense", "vocab", "max_seq",
        "batch", "wdt")] + [("eps", _f), ("scale", _f)] + [
        (n, _vp) for n in ("emb", "gf", "lm", "lm_s", "rope_cos", "rope_sin")] + [
        ("layers", C.POINTER(OrDsv2Layer)), ("sel_out", _vp), ("probs_out", _vp),
        ("gate_out", _vp)] + [
        (n, _vp) for n in ("tf_x", "tp_x", "tp_o", "tf_sel", "tf_probs")] + [("b0", _u32), ("b1", _u32)]


_OR = None
_REF = None


# the reference CPU JIT's compile flags (src/backend/cpu/jit.c:318-345)
REF_JIT_FLAGS = ["-O3", "-fno-math-errno", "-ffp-contract=off", "-march=native", "-mno-avx512f"]


def oracle() -> C.CDLL:
    global _OR
    if _OR is None:
        if not ORACLE_SO.exists():
            subprocess.run(["make", "-C", str(ROOT / "oracle"), "build/liboracle.so"], check=True,
                           capture_output=True)
        _OR = _bind(C.CDLL(str(ORACLE_SO)))
    return _OR


def use_native_build(outdir) -> str:
    """Compile oracle/oracle.c on this machine with the reference CPU JIT's
    flags (-march=native for this host) into `outdir` and use that build from
    here on; returns the compile command.  The flags allow no reassociation
    (-ffp-contract=off, no -ffast-math), so the results are the shipped
    build's bit for bit; only the instructions chosen differ."""
    global _OR
    from pathlib import Path as _P
    so = _P(outdir) / "liboracle_native.so"
    so.parent.mkdir(parents=True, exist_ok=True)
    cmd = ["cc", "-std=c11", *REF_JIT_FLAGS, "-fPIC", "-shared", "-o", str(so),
           str(ROOT / "oracle" / "oracle.c"), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)
    _OR = _bind(C.CDLL(str(so)))
    return " ".join(cmd[:-4] + ["oracle/oracle.c", "-lm"])


def _bind(L: C.CDLL) -> C.CDLL:
    """Set the oracle's function signatures on a loaded build."""
    sig = {
        "or_bf16_to_f32": (_f, [_u16]), "or_f32_to_bf16": (_u16, [_f]),
        "or_fp16_to_f32": (_f, [_u16]), "or_f32_to_fp16": (_u16, [_f]),
        "or_fp8e4m3_to_f32": (_f, [_u8]), "or_fp8e5m2_to_f32": (_f, [_u8]),
        "or_f32_to_fp8e4m3": (_u8, [_f]), "or_f32_to_fp8e4m3_sat": (_u8, [_f]),
        "or_f32_to_fp8e5m2": (_u8, [_f]), "or_f32_to_fp8e5m2_sat": (_u8, [_f]),
        "or_decode": (None, [_vp, _u32, _vp, _u64]),
        "or_encode": (None, [_vp, _u32, _vp, _u64]),
        "or_gemv": (None, [_vp, _vp, _u32, _u32, _vp, _u32, _vp, _u32, _u32, _u32]),
        "or_rmsnorm": (None, [_vp, _u32, _vp, _u32, _vp, _u32, _u32, _f]),
        "or_layernorm": (None, [_vp, _u32, _vp, _u32, _vp, _vp, _u32, _u32, _f]),
        "or_softmax": (None, [_vp, _u32, _vp, _u32, _u32, _u32]),
        "or_rope": (None, [_vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32]),
        "or_attn_decode": (None, [_vp, _u32, _vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32,
                                  _u32, _u32, _u32, _f]),
        "or_argmax": (None, [_vp, _vp, _u32, _u32]),
        "or_sexpf": (_f, [_f]), "or_sample_u01": (_f, [_u64, _u32, C.c_int32]),
        "or_sample": (None, [_vp, _vp, _u32, _u32, _u32, _f, _u64, C.c_int32]),
        "or_spec_draft": (None, [_vp, _vp, _vp, C.c_int32, _u32, _u32, _u32, _i]),
        "or_spec_accept": (C.c_int32, [_vp, C.c_int32, _vp, _vp, _u32, _u32]),
        "or_decode_step": (_i, [C.POINTER(OrModel), _vp, _u32, _vp, _vp]),
        "or_mla_prep": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp,
                               _u32, _u32, _u32, _u32, _f]),
        "or_mla_attn": (None, [_vp, _vp, _vp, _vp, _vp, _u32, _vp, _u32, _vp, _u32, _u32,
                               _u32, _u32, _f]),
        "or_route": (None, [_vp, _vp, _vp, _u32, _u32]),
        "or_moe": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                          _u32, _u32, _u32, _u32, _u32]),
        "or_dsv2_step": (_i, [C.POINTER(OrDsv2), _vp, _u32, _vp, _vp]),
        "or_dsv2_dense_act": (None, [_vp, _vp, _vp, _u64]),
    }
    for k, (r, a) in sig.items():
        fn = getattr(L, k)
        fn.restype, fn.argtypes = r, a
    return L


def ref():
    """The compiled reference harness, or None where it was not built."""
    global _REF
    if _REF is None and REF_SO.exists():
        L = C.CDLL(str(REF_SO))
        sig = {
            "ref_f32_to_fp8e4m3": (_u8, [_f]), "ref_f32_to_fp8e4m3_sat": (_u8, [_f]),
            "ref_f32_to_fp8e5m2": (_u8, [_f]), "ref_f32_to_fp8e5m2_sat": (_u8, [_f]),
            "ref_fp8e4m3_to_f32": (_f, [_u8]), "ref_fp8e5m2_to_f32": (_f, [_u8]),
            "ref_f32_to_bf16": (_u16, [_f]), "ref_bf16_to_f32": (_f, [_u16]),
            "ref_f32_to_fp16": (_u16, [_f]), "ref_fp16_to_f32": (_f, [_u16]),
            "ref_f32_to_fp16_manual": (_u16, [_f]), "ref_fp16_to_f32_manual": (_f, [_u16]),
            "ref_xexp2f": (_f, [_f]),
            "ref_linear_f32": (_i, [_vp, _vp, _vp, _u32, _u32, _u32]),
            "ref_softmax_f32": (_i, [_vp, _vp, _u32, _u32]),
            "ref_layernorm_f32": (_i, [_vp, _vp, _u32, _u32, C.c_double]),
            "ref_rmsnorm_f32": (_i, [_vp, _vp, _u32, _u32, C.c_double]),
            "ref_dense_silu_mul_bf16": (_i, [_vp, _vp, _vp, _u32]),
            "ref_gelu_f32": (_i, [_vp, _vp, _u32, _u32]),
            "ref_sdpa_f32": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32]),
            "ref_gpt2_block_f32": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _u32]),
            "ref_capture_begin": (_i, []), "ref_capture_end": (_i, []),
            "ref_capture_kernel": (_i, [_u32, _vp, _u32, C.POINTER(_u32), C.POINTER(_u32), _vp,
                                        C.POINTER(_u32), C.c_char_p, _u32]),
            "ref_capture_slot": (_i, [_u32, _u32, C.POINTER(_u32), C.POINTER(_u64), _vp, _u64]),
        }
        for k, (r, a) in sig.items():
            fn = getattr(L, k)
            fn.restype, fn.argtypes = r, a
        _REF = L
    return _REF


def ptr(a: np.ndarray):
    return a.ctypes.data if a is not None else None


# ---- numpy conveniences over the oracle codecs ----
DT_FP8E4M3, DT_FP8E5M2, DT_FP16, DT_BF16, DT_FP32 = 9, 10, 11, 12, 13
_STORE_NP = {DT_FP32: np.float32, DT_FP16: np.uint16, DT_BF16: np.uint16, DT_FP8E4M3: np.uint8,
             DT_FP8E5M2: np.uint8}


def decode(a: np.ndarray, dt: int) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty(a.size, np.float32)
    oracle().or_decode(a.ctypes.data, dt, out.ctypes.data, a.size)
    return out.reshape(a.shape)


def encode(f: np.ndarray, dt: int) -> np.ndarray:
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.size, _STORE_NP[dt])
    oracle().or_encode(f.ctypes.data, dt, out.ctypes.data, f.size)
    return out.reshape(f.shape)


def gemv(x: np.ndarray, xdt: int, w: np.ndarray, wdt: int, scale=None, M=None, N=None, K=None):
    """y[M,N] f32 = x @ dequant(w)^T (oracle or_gemv)."""
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w)
    y = np.empty((M, N), np.float32)
    sc = None if scale is None else np.ascontiguousarray(scale, np.float32)
    oracle().or_gemv(y.ctypes.data, x.ctypes.data, xdt, K, w.ctypes.data, wdt,
                     sc.ctypes.data if sc is not None else None, M, N, K)
    return y


def spec_draft(hist, L, S, V, forced=False):
    """(cand_acc, cand_emb) of or_spec_draft over one token history."""
    h = np.ascontiguousarray(hist, np.int32)
    ca, ce = np.empty(S, np.int32), np.empty(S, np.int32)
    oracle().or_spec_draft(ca.ctypes.data, ce.ctypes.data, h.ctypes.data, int(L), S, V, h.size,
                           int(forced))
    return ca, ce


def spec_accept(hist, L, ca, am, S):
    """(new history, new L) of or_spec_accept."""
    h = np.array(hist, np.int32)
    ca = np.ascontiguousarray(ca, np.int32)
    am = np.ascontiguousarray(am, np.int32)
    Ln = oracle().or_spec_accept(h.ctypes.data, int(L), ca.ctypes.data, am.ctypes.data, S, h.size)
    return h, Ln


DT_FP8_W = 9


def _threads(B):
    import os
    return max(1, min(B, 16, os.cpu_count() or 1))


def _run_rows(fn, m, B, *args, threads=None):
    """Run `fn(m_rows, *args)` over row ranges on threads (the oracle keeps
    every row's state apart: caches, logits and taps are indexed by row; ctypes
    releases the GIL during the call).  `threads` 1 runs every row on the
    calling thread."""
    from concurrent.futures import ThreadPoolExecutor
    nt = _threads(B) if threads is None else max(1, min(int(threads), B))
    if nt == 1:
        return [fn(C.byref(m), *args)]
    cuts = np.linspace(0, B, nt + 1).astype(int)
    ms = []
    for i in range(nt):
        mi = type(m).from_buffer_copy(m)
        mi.b0, mi.b1 = int(cuts[i]), int(cuts[i + 1])
        ms.append(mi)
    with ThreadPoolExecutor(nt) as ex:
        return list(ex.map(lambda mi: fn(C.byref(mi), *args), ms))


class OracleModel:
    """OrModel over numpy copies of the decoder's device tensors."""

    def __init__(self, dec, cfg):
        self.keep = []
        self.cfg = cfg
        m = OrModel()
        arch = cfg["arch"]
        m.arch = arch
        for k in ("n_layers", "dim", "n_heads", "head_dim", "ffn", "vocab", "max_seq", "batch"):
            setattr(m, k, cfg[k])
        m.n_kv_heads = cfg.get("n_kv_heads", cfg["n_heads"])
        m.wdt, m.adt, m.eps = cfg["wdtype"], cfg["adtype"], cfg["eps"]

        def t(name):
            a = dec.read_tensor(name)
            self.keep.append(a)
            return a.ctypes.data

        L = cfg["n_layers"]
        self.layers = (OrLayer * L)()
        self.caches = []
        f8 = cfg["wdtype"] == DT_FP8_W
        for l in range(L):
            ly = self.layers[l]
            p = f"l{l}."
            if arch == 1:
                ly.wqkv, ly.wo, ly.wgu, ly.wd = (t(p + n) for n in ("wqkv", "wo", "wgu", "wd"))
                if f8:
                    ly.sqkv, ly.so, ly.sgu, ly.sd = (t(p + n + ".scale") for n in ("wqkv", "wo", "wgu", "wd"))
                ly.g1, ly.g2 = t(p + "g_attn"), t(p + "g_ffn")
            else:
                ly.wqkv, ly.wo, ly.wgu, ly.wd = (t(p + n) for n in ("c_attn", "c_proj", "c_fc", "mlp_proj"))
                ly.bqkv, ly.bo, ly.bfc, ly.bpr = (t(p + n + ".b") for n in ("c_attn", "c_proj", "c_fc", "mlp_proj"))
                ly.g1, ly.b1, ly.g2, ly.b2 = (t(p + n) for n in ("ln1.g", "ln1.b", "ln2.g", "ln2.b"))
            kc, vc = dec.read_tensor(p + "kcache"), dec.read_tensor(p + "vcache")
            self.caches += [kc, vc]
            ly.kcache, ly.vcache = kc.ctypes.data, vc.ctypes.data
        if arch == 1:
            m.emb, m.gf, m.lm = t("emb"), t("norm_f"), t("lm")
            if f8:
                m.lm_s = t("lm.scale")
            m.rope_cos, m.rope_sin = t("rope.cos"), t("rope.sin")
        else:
            m.emb, m.pos_emb, m.gf, m.bf = t("wte"), t("wpe"), t("lnf.g"), t("lnf.b")
        m.layers = self.layers
        self.m = m

    def step(self, tok, pos, tf_x=None, taps=False, threads=None):
        """One step from ids `tok` at `pos`: (logits [B,V], next ids [B]).
        With `tf_x` ([2L+1, B, D] f32, the residual entering each sublayer
        taken from another implementation) every sublayer restarts from it.
        With `tf_x` or `taps`, `self.taps` holds this step's x/q/att/h outputs
        per sublayer."""
        cfg = self.cfg
        B, V, D, L = cfg["batch"], cfg["vocab"], cfg["dim"], cfg["n_layers"]
        tok = np.ascontiguousarray(tok, np.int32)
        lg = np.empty((B, V), np.float32)
        nx = np.empty(B, np.int32)
        m = self.m
        if tf_x is not None or taps:
            hq = cfg["n_heads"] * cfg["head_dim"]
            self.taps = dict(x=np.zeros((2 * L, B, D), np.float32), q=np.zeros((L, B, hq), np.float32),
                             att=np.zeros((L, B, hq), np.float32),
                             h=np.zeros((L, B, cfg["ffn"]), np.float32))
            m = OrModel.from_buffer_copy(self.m)
            m.tp_x, m.tp_q, m.tp_att, m.tp_h = (self.taps[k].ctypes.data for k in ("x", "q", "att", "h"))
        if tf_x is not None:
            tf = np.ascontiguousarray(tf_x, np.float32).reshape(2 * L + 1, B, D)
            m.tf_x = tf.ctypes.data
        rcs = _run_rows(oracle().or_decode_step, m, B, tok.ctypes.data, pos, lg.ctypes.data,
                        nx.ctypes.data, threads=threads)
        assert all(r == 0 for r in rcs)
        return lg, nx


def dsv2_scale(cfg) -> float:
    """(dn+dr)^-1/2 * mscale^2 with mscale = 0.1*0.707*ln(40) + 1 (YaRN)."""
    ms = 0.1 * 0.707 * np.log(40.0) + 1.0
    return float((cfg["d_nope"] + cfg["d_rope"]) ** -0.5 * ms * ms)


class OracleDsv2:
    """OrDsv2 over numpy copies of a DSV2 decoder's device tensors."""

    def __init__(self, dec, cfg):
        self.keep, self.caches, self.cfg = [], [], cfg
        m = OrDsv2()
        for k in ("n_layers", "dim", "n_heads", "kv_lora", "d_nope", "d_rope", "d_v", "n_experts",
                  "n_shared", "top_k", "moe_inter", "first_dense", "vocab", "max_seq", "batch"):
            setattr(m, k, cfg.get(k, 0))
        m.dense_inter, m.wdt, m.eps = cfg.get("ffn", 0), cfg["wdtype"], cfg["eps"]
        m.scale = dsv2_scale(cfg)
        f8 = cfg["wdtype"] == DT_FP8_W

        def t(name):
            a = dec.read_tensor(name)
            self.keep.append(a)
            return a.ctypes.data

        def w(ly, field, name):
            setattr(ly, field, t(name))
            if f8:
                setattr(ly, "s" + field[1:], t(name + ".scale"))

        L = cfg["n_layers"]
        self.layers = (OrDsv2Layer * L)()
        for l in range(L):
            ly, p = self.layers[l], f"l{l}."
            ly.win, ly.wkvn, ly.wpost = t(p + "win"), t(p + "wkvn"), t(p + "wpost")
            for f in ("wqkv", "wuk", "wuv", "wo"):
                w(ly, f, p + f)
            if l < cfg.get("first_dense", 0):
                w(ly, "wgu", p + "wgu")
                w(ly, "wd", p + "wd")
            else:
                ly.gate = t(p + "gate")
                w(ly, "wgu_e", p + "wgu_e")
                w(ly, "wd_e", p + "wd_e")
                if cfg.get("n_shared", 0):
                    w(ly, "wgu_s", p + "wgu_s")
                    w(ly, "wd_s", p + "wd_s")
            ck, kp = dec.read_tensor(p + "ckv"), dec.read_tensor(p + "kpe")
            self.caches += [ck, kp]
            ly.ckv, ly.kpe = ck.ctypes.data, kp.ctypes.data
        m.emb, m.gf, m.lm = t("emb"), t("norm_f"), t("lm")
        if f8:
            m.lm_s = t("lm.scale")
        m.rope_cos, m.rope_sin = t("rope.cos"), t("rope.sin")
        m.layers = self.layers
        B, K = cfg["batch"], cfg["top_k"]
        # per layer and row (dense layers keep zeros)
        self.sel = np.zeros((L, B, K), np.int32)
        self.probs = np.zeros((L, B, K), np.float32)
        self.gate = np.zeros((L, B, cfg["n_experts"]), np.float32)
        m.sel_out, m.probs_out = self.sel.ctypes.data, self.probs.ctypes.data
        m.gate_out = self.gate.ctypes.data
        self.m = m

    def step(self, tok, pos, tf_x=None, tf_sel=None, tf_probs=None, taps=False, threads=None):
        """One step: (logits [B,V], next ids [B]); per-layer routing in
        self.sel / self.probs / self.gate.  With `tf_x` ([2L+1, B, D]) every
        sublayer restarts from the given residual; with it or `taps`,
        `self.taps` holds the x / o outputs; with `tf_sel`, `tf_probs`
        ([L, B, K]) the MoE layers combine those experts instead of their own
        picks."""
        cfg = self.cfg
        B, V, D, L = cfg["batch"], cfg["vocab"], cfg["dim"], cfg["n_layers"]
        tok = np.ascontiguousarray(tok, np.int32)
        lg = np.empty((B, V), np.float32)
        nx = np.empty(B, np.int32)
        m, keep = self.m, []
        if tf_x is not None or tf_sel is not None or taps:
            m = OrDsv2.from_buffer_copy(self.m)
        if tf_x is not None or taps:
            self.taps = dict(x=np.zeros((2 * L, B, D), np.float32),
                             o=np.zeros((L, B, cfg["n_heads"] * cfg["d_v"]), np.float32))
            m.tp_x, m.tp_o = self.taps["x"].ctypes.data, self.taps["o"].ctypes.data
        if tf_x is not None:
            tf = np.ascontiguousarray(tf_x, np.float32).reshape(2 * L + 1, B, D)
            keep.append(tf)
            m.tf_x = tf.ctypes.data
        if tf_sel is not None:
            ts = np.ascontiguousarray(tf_sel, np.int32).reshape(L, B, cfg["top_k"])
            tp = np.ascontiguousarray(tf_probs, np.float32).reshape(L, B, cfg["top_k"])
            keep += [ts, tp]
            m.tf_sel, m.tf_probs = ts.ctypes.data, tp.ctypes.data
        rcs = _run_rows(oracle().or_dsv2_step, m, B, tok.ctypes.data, pos, lg.ctypes.data,
                        nx.ctypes.data, threads=threads)
        assert all(r == 0 for r in rcs)
        return lg, nx
