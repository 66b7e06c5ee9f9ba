"""TEST INFRASTRUCTURE.  Seeded synthetic DeepSeek-V2 weights in this
build's decoder layouts (the tensor names the DSV2 decoder uses), the YaRN
RoPE tables, and a writer for the reference's DSV2PK01 weight pack
(bench/dsv2_decode_bench.c pack format :229-310, tensor layouts of
model_init :2130-2210) so the compiled reference can run the same model."""
from __future__ import annotations

import struct

import numpy as np

import _oracle as O

DT_BF16, DT_F32 = 12, 13


def bf16(a):
    return O.encode(np.asarray(a, np.float32), DT_BF16)


def yarn_tables(max_seq, dr, theta=10000.0, factor=40.0, orig=4096.0, beta_fast=32.0, beta_slow=1.0):
    """[max_seq, dr/2] cos/sin of the DeepSeek-V2 YaRN-scaled RoPE."""
    half = dr // 2
    lo = np.floor(dr * np.log(orig / (beta_fast * 2 * np.pi)) / (2 * np.log(theta)))
    hi = np.ceil(dr * np.log(orig / (beta_slow * 2 * np.pi)) / (2 * np.log(theta)))
    lo, hi = max(lo, 0.0), min(hi, dr - 1.0)
    j = np.arange(half, dtype=np.float64)
    inv = 1.0 / theta ** (2 * j / dr)
    ramp = np.clip((j - lo) / max(hi - lo, 1e-3), 0.0, 1.0)
    f = inv / factor * ramp + inv * (1 - ramp)
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * f[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def make_dsv2(cfg, seed):
    """bf16 weights N(0, std) (gains 1, router f32) in the decoder's layouts."""
    rng = np.random.default_rng(seed)
    D, H, kv, dn, dr, dv = (cfg[k] for k in ("dim", "n_heads", "kv_lora", "d_nope", "d_rope", "d_v"))
    E, I, S, V, F = cfg["n_experts"], cfg["moe_inter"], cfg["n_shared"] * cfg["moe_inter"], cfg["vocab"], cfg["ffn"]
    std = cfg.get("init_std", 0.02)
    nqkv = H * (dn + dr) + kv + dr

    def w(*shape):
        return bf16(rng.standard_normal(shape) * std)

    t = {"emb": w(V, D), "norm_f": np.ones(D, np.float32), "lm": w(V, D)}
    for l in range(cfg["n_layers"]):
        p = f"l{l}."
        t[p + "win"], t[p + "wkvn"], t[p + "wpost"] = (np.ones(n, np.float32) for n in (D, kv, D))
        t[p + "wqkv"], t[p + "wuk"], t[p + "wuv"], t[p + "wo"] = w(nqkv, D), w(H * kv, dn), w(H * dv, kv), w(D, H * dv)
        if l < cfg["first_dense"]:
            t[p + "wgu"], t[p + "wd"] = w(2 * F, D), w(D, F)
        else:
            t[p + "gate"] = (rng.standard_normal((E, D)) * std).astype(np.float32)
            t[p + "wgu_e"], t[p + "wd_e"] = w(E * 2 * I, D), w(E * D, I)
            t[p + "wgu_s"], t[p + "wd_s"] = w(2 * S, D), w(D, S)
        t[p + "ckv"] = np.zeros((cfg["batch"], cfg["max_seq"], kv), np.uint16)
        t[p + "kpe"] = np.zeros((cfg["batch"], cfg["max_seq"], dr), np.uint16)
    t["rope.cos"], t["rope.sin"] = yarn_tables(cfg["max_seq"], dr)
    return t


def write_pack(t, cfg, path):
    """The DSV2PK01 pack of the same model in the reference's layouts:
    {in, out} projections, absorbed w_uk [(h*dn + d)*kv + k], w_uv
    [(h*dv + m)*kv + k], stacked experts, f32 norm gains and router."""
    D, H, kv, dn, dr, dv = (cfg[k] for k in ("dim", "n_heads", "kv_lora", "d_nope", "d_rope", "d_v"))
    E, I, S = cfg["n_experts"], cfg["moe_inter"], cfg["n_shared"] * cfg["moe_inter"]
    nq = H * (dn + dr)
    ents = [("embed", t["emb"]), ("norm", t["norm_f"]), ("lm_head", t["lm"].T)]
    for l in range(cfg["n_layers"]):
        p = f"l{l}."
        wqkv = t[p + "wqkv"]
        ents += [(p + "win", t[p + "win"]), (p + "wq", wqkv[:nq].T), (p + "wkv", wqkv[nq:].T),
                 (p + "wkvn", t[p + "wkvn"]),
                 (p + "wuk", t[p + "wuk"].reshape(H, kv, dn).transpose(0, 2, 1)),
                 (p + "wuv", t[p + "wuv"]), (p + "wo", t[p + "wo"].T), (p + "wpost", t[p + "wpost"])]
        if l < cfg["first_dense"]:
            ents += [(p + "wg1", t[p + "wgu"][0::2].T), (p + "wu1", t[p + "wgu"][1::2].T),
                     (p + "wd1", t[p + "wd"].T)]
        else:
            gu = t[p + "wgu_e"].reshape(E, 2 * I, D)
            gs = t[p + "wgu_s"]
            ents += [(p + "gate", t[p + "gate"].T), (p + "wg", gu[:, 0::2]), (p + "wu", gu[:, 1::2]),
                     (p + "wd", t[p + "wd_e"]), (p + "swg", gs[0::2]), (p + "swu", gs[1::2]),
                     (p + "swd", t[p + "wd_s"])]
    hdr = 16 + len(ents) * 72
    off = (hdr + 63) // 64 * 64
    table, blobs = [], []
    for name, a in ents:
        a = np.ascontiguousarray(a)
        dt = 0 if a.dtype == np.uint16 else 1
        assert a.dtype in (np.uint16, np.float32)
        blob = a.tobytes()
        table.append(struct.pack("<48sIIQQ", name.encode(), dt, 0, off, len(blob)))
        blobs.append((off, blob))
        off = (off + len(blob) + 63) // 64 * 64
    with open(path, "wb") as f:
        f.write(b"DSV2PK01" + struct.pack("<Q", len(ents)) + b"".join(table))
        for o, blob in blobs:
            f.seek(o)
            f.write(blob)
