"""The oracle's per-sublayer teacher forcing (oracle/oracle.c: OrModel /
OrDsv2 tf_x, tp_*, tf_sel, and the row range b0/b1), CPU only.

The full-depth GPU parity tests feed the device's residual at every sublayer
boundary into the oracle and compare each sublayer's outputs.  That is only
meaningful if the plumbing itself is right, which these checks pin:

  * identity: teacher inputs equal to the oracle's own trajectory (recorded
    by its taps) reproduce the free-running step bit for bit -- logits, ids
    and every tap;
  * locality: perturbing the input of sublayer t changes no tap before t and
    changes sublayer t's output (a wrong sublayer index, a swapped x/tap
    buffer or a forced input applied at the wrong boundary fails one of the
    two);
  * the final-norm input (t = 2L) drives the logits alone;
  * forced routing: the DSV2 MoE combines the given experts (its own picks
    reproduce the free run; another expert set changes that layer's FFN
    output and nothing before it);
  * rows split across threads (b0/b1) give the single-thread bits."""
import numpy as np
import pytest

import _dsv2_weights as DW
import _oracle as O
import test_oracle_models as M

DT_FP8, DT_F16, DT_BF16, DT_F32 = 9, 11, 12, 13

LLAMA = dict(M.LLAMA, n_layers=3, max_seq=40)
GPT2 = dict(arch=2, n_layers=3, dim=96, n_heads=4, n_kv_heads=4, head_dim=24, ffn=192, vocab=250,
            max_seq=32, batch=1, eps=1e-5)


def _batched(t, B):
    """Tile the single-row caches of a model to B rows."""
    out = dict(t)
    for k, v in t.items():
        if k.endswith(("kcache", "vcache")):
            out[k] = np.ascontiguousarray(np.repeat(v, B, axis=0))
    return out


def _copy(t):
    return {k: np.array(v, copy=True) for k, v in t.items()}


def _embed(t, cfg, tok, pos):
    adt = cfg["adtype"]
    if cfg["arch"] == 1:
        return O.decode(t["emb"].reshape(-1, cfg["dim"])[tok], adt) if adt != DT_F32 else \
            t["emb"].reshape(-1, cfg["dim"])[tok].astype(np.float32)
    wte = t["wte"].reshape(-1, cfg["dim"])[tok]
    wpe = t["wpe"].reshape(-1, cfg["dim"])[pos][None, :]
    if adt == DT_F32:
        return (wte + wpe).astype(np.float32)
    s = O.decode(wte, adt) + O.decode(wpe, adt)
    return O.decode(O.encode(s, adt), adt)


def _model(arch, wdt, adt, B):
    if arch == 1:
        cfg = dict(LLAMA, wdtype=wdt, adtype=adt, batch=B)
        t, _ = M.llama_model(dict(cfg, batch=1), 5, 12)
        pos = 12
    else:
        cfg = dict(GPT2, wdtype=wdt, adtype=adt, batch=B)
        t, _ = M.gpt2_model(dict(cfg, batch=1), 6)
        pos = 0
    return cfg, _batched(t, B), pos


@pytest.mark.parametrize("arch,wdt,adt", [(1, DT_FP8, DT_BF16), (1, DT_F32, DT_F32), (2, DT_F16, DT_F16)])
def test_teacher_identity_and_locality(arch, wdt, adt):
    B = 2
    cfg, t, pos = _model(arch, wdt, adt, B)
    L = cfg["n_layers"]
    tok = np.array([7, 123], np.int32)
    free = O.OracleModel(M._Tensors(_copy(t)), cfg)
    lg0, nx0 = free.step(tok, pos, taps=True)
    taps0 = {k: v.copy() for k, v in free.taps.items()}
    x0 = _embed(t, cfg, tok, pos)
    tf = np.concatenate([x0[None], taps0["x"]], axis=0)          # [2L+1, B, D]

    forced = O.OracleModel(M._Tensors(_copy(t)), cfg)
    lg1, nx1 = forced.step(tok, pos, tf_x=tf)
    assert np.array_equal(lg1, lg0) and np.array_equal(nx1, nx0)
    for k in taps0:
        assert np.array_equal(forced.taps[k], taps0[k]), k

    for tsub in range(2 * L):
        bad = tf.copy()
        bad[tsub, 1, 3] += 0.5
        pm = O.OracleModel(M._Tensors(_copy(t)), cfg)
        lg2, _ = pm.step(tok, pos, tf_x=bad)
        assert np.array_equal(pm.taps["x"][:tsub], taps0["x"][:tsub]), tsub
        assert not np.array_equal(pm.taps["x"][tsub, 1], taps0["x"][tsub, 1]), tsub
        assert np.array_equal(pm.taps["x"][tsub, 0], taps0["x"][tsub, 0]), tsub   # other row untouched
        assert np.array_equal(lg2, lg0)      # the logits follow the forced final input only

    bad = tf.copy()
    bad[2 * L, 0, :] *= 1.5
    bad[2 * L, 0, 0] += 1.0
    pm = O.OracleModel(M._Tensors(_copy(t)), cfg)
    lg3, _ = pm.step(tok, pos, tf_x=bad)
    assert np.array_equal(pm.taps["x"], taps0["x"])
    assert not np.array_equal(lg3[0], lg0[0]) and np.array_equal(lg3[1], lg0[1])


def test_rows_on_threads_match_one_thread(monkeypatch):
    cfg, t, pos = _model(1, DT_FP8, DT_BF16, 5)
    tok = np.array([1, 2, 3, 4, 5], np.int32)
    a = O.OracleModel(M._Tensors(_copy(t)), cfg)
    lga, nxa = a.step(tok, pos, taps=True)
    monkeypatch.setattr(O, "_threads", lambda B: 1)
    b = O.OracleModel(M._Tensors(_copy(t)), cfg)
    lgb, nxb = b.step(tok, pos, taps=True)
    assert np.array_equal(lga, lgb) and np.array_equal(nxa, nxb)
    for k in a.taps:
        assert np.array_equal(a.taps[k], b.taps[k]), k


DSV2 = dict(n_layers=3, dim=64, n_heads=4, kv_lora=32, d_nope=16, d_rope=8, d_v=16, n_experts=8,
            n_shared=1, top_k=2, moe_inter=32, ffn=96, first_dense=1, vocab=120, max_seq=16, batch=2,
            eps=1e-6, init_std=0.05, wdtype=DT_BF16)


def test_dsv2_teacher_identity_locality_and_forced_routing():
    cfg = DSV2
    L, B, K = cfg["n_layers"], cfg["batch"], cfg["top_k"]
    t = DW.make_dsv2(cfg, 11)
    tok = np.array([5, 77], np.int32)
    free = O.OracleDsv2(M._Tensors(_copy(t)), cfg)
    lg0, nx0 = free.step(tok, 0, taps=True)
    taps0 = {k: v.copy() for k, v in free.taps.items()}
    sel0, probs0 = free.sel.copy(), free.probs.copy()
    x0 = O.decode(t["emb"].reshape(-1, cfg["dim"])[tok], DT_BF16)
    tf = np.concatenate([x0[None], taps0["x"]], axis=0)

    forced = O.OracleDsv2(M._Tensors(_copy(t)), cfg)
    lg1, _ = forced.step(tok, 0, tf_x=tf, tf_sel=sel0, tf_probs=probs0)
    assert np.array_equal(lg1, lg0)
    for k in taps0:
        assert np.array_equal(forced.taps[k], taps0[k]), k
    assert np.array_equal(forced.sel, sel0) and np.array_equal(forced.probs, probs0)

    for tsub in range(2 * L):
        bad = tf.copy()
        bad[tsub, 0, 1] += 0.25
        pm = O.OracleDsv2(M._Tensors(_copy(t)), cfg)
        pm.step(tok, 0, tf_x=bad, tf_sel=sel0, tf_probs=probs0)
        assert np.array_equal(pm.taps["x"][:tsub], taps0["x"][:tsub]), tsub
        assert not np.array_equal(pm.taps["x"][tsub, 0], taps0["x"][tsub, 0]), tsub
        assert np.array_equal(pm.taps["x"][:, 1], taps0["x"][:, 1]), tsub

    # another expert set at layer 2 changes that layer's FFN output only
    sel2 = sel0.copy()
    sel2[2, 1] = [(s + 1) % cfg["n_experts"] for s in sel0[2, 1]]
    if len(set(sel2[2, 1])) < K:
        sel2[2, 1] = np.arange(K)
    pm = O.OracleDsv2(M._Tensors(_copy(t)), cfg)
    pm.step(tok, 0, tf_x=tf, tf_sel=sel2, tf_probs=probs0)
    assert np.array_equal(pm.taps["x"][:5], taps0["x"][:5])
    assert not np.array_equal(pm.taps["x"][5, 1], taps0["x"][5, 1])
    assert np.array_equal(pm.taps["x"][5, 0], taps0["x"][5, 0])
    assert np.array_equal(pm.sel, sel0)          # its own routing is still recorded
