"""GPU tests of the Tensor / TinyJit host (thvm_amd.tensor) and the renderer
target it drives.

Every op runs on the device: generic kernels are lifted uop DAGs rendered
to HIP by libthvm_hip.so and compiled by hiprtc; x @ W.T runs the gfx950
GEMV builtin.  Checks are against numpy in float64 with f32 tolerances
(the renderer computes f32 with exp2f / sqrtf / division, so results sit
within a few ulp of the f64 value), and integer / index results bit-exact.
The GPT-2 driver is checked against the C oracle's GPT-2 decode step
(oracle/oracle.c or_decode_step, arch GPT2) on the same seeded weights:
greedy ids identical, logits within 1e-5 relative."""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def T(hip):
    import thvm_amd.tensor as tensor
    return tensor


def close(got, want, rtol=2e-5, atol=2e-6):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    lim = atol + rtol * np.abs(want)
    assert np.all(err <= lim), f"max err {err.max():.3g} at {np.unravel_index(np.argmax(err - lim), err.shape)}"


def test_elementwise_and_broadcast(T):
    say("case: elementwise")
    rng = np.random.default_rng(1)
    a = rng.standard_normal((3, 5, 7)).astype(np.float32)
    b = rng.standard_normal((5, 1)).astype(np.float32)
    A, B = T.Tensor(a), T.Tensor(b)
    ad, bd = a.astype(np.float64), b.astype(np.float64)
    close((A + B).numpy(), ad + bd)
    close((A * B - 2.0).numpy(), ad * bd - 2.0)
    close((A / (B * B + 1.0)).numpy(), ad / (bd * bd + 1.0))
    close(A.exp().numpy(), np.exp(ad), rtol=1e-5)
    close((A * A + 1.0).log().numpy(), np.log(ad * ad + 1.0), rtol=1e-5, atol=1e-6)
    close((A * A).sqrt().numpy(), np.abs(ad), rtol=1e-6)
    close(A.tanh().numpy(), np.tanh(ad), rtol=1e-5, atol=1e-6)
    close(A.sigmoid().numpy(), 1 / (1 + np.exp(-ad)), rtol=1e-5)
    g = 0.5 * ad * (1 + np.tanh(np.sqrt(2 / np.pi) * (ad + 0.044715 * ad ** 3)))
    close(A.gelu().numpy(), g, rtol=1e-5, atol=1e-6)
    close(A.relu().numpy(), np.maximum(ad, 0))
    close(A.maximum(B).numpy(), np.maximum(ad, bd))
    close((A < B).where(A, -1.5).numpy(), np.where(ad < bd, ad, -1.5))
    assert np.array_equal((A < B).numpy(), a < b)
    assert np.array_equal((A == A).numpy(), np.ones_like(a, bool))
    ia = rng.integers(-50, 50, (4, 6)).astype(np.int32)
    IA = T.Tensor(ia)
    assert np.array_equal((IA * 3 + 7).numpy(), ia * 3 + 7)
    assert np.array_equal((IA + 100).div(7).numpy(), (ia + 100) // 7)


def test_reductions_softmax_argmax(T):
    say("case: reductions")
    rng = np.random.default_rng(2)
    a = rng.standard_normal((4, 3, 600)).astype(np.float32)     # 600: group-reduce kernels
    A = T.Tensor(a)
    ad = a.astype(np.float64)
    close(A.sum(-1).numpy(), ad.sum(-1), rtol=1e-5, atol=2e-5)
    close(A.max(1).numpy(), ad.max(1))
    close(A.mean((0, 2), keepdim=True).numpy(), ad.mean((0, 2), keepdims=True), atol=2e-6)
    e = np.exp(ad - ad.max(-1, keepdims=True))
    close(A.softmax(-1).numpy(), e / e.sum(-1, keepdims=True), rtol=1e-5, atol=1e-8)
    small = rng.standard_normal((5, 9)).astype(np.float32)     # thread-mode kernels
    close(T.Tensor(small).sum(0).numpy(), small.astype(np.float64).sum(0), atol=1e-6)
    # argmax: lowest index among ties
    t = np.array([[1, 5, 5, 2], [7, 7, 7, 7], [-1, -3, -1, -9]], np.float32)
    assert T.Tensor(t).argmax(-1).numpy().tolist() == [1, 0, 0]
    assert int(T.Tensor(a.reshape(-1)).argmax().item()) == int(np.argmax(a.reshape(-1)))
    x = rng.standard_normal((2, 700)).astype(np.float32)
    y = T.Tensor(x).layernorm(eps=1e-5).numpy()
    xd = x.astype(np.float64)
    mu, var = xd.mean(-1, keepdims=True), xd.var(-1, keepdims=True)
    close(y, (xd - mu) / np.sqrt(var + 1e-5), rtol=1e-4, atol=1e-5)


def test_movement(T):
    say("case: movement")
    rng = np.random.default_rng(3)
    a = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    A = T.Tensor(a)
    close(A.permute(2, 0, 3, 1).numpy(), a.transpose(2, 0, 3, 1))
    close(A.reshape(6, 20).numpy(), a.reshape(6, 20))
    close(A.permute(0, 2, 1, 3).reshape(8, 15).numpy(), a.transpose(0, 2, 1, 3).reshape(8, 15))
    close(A[1, :, 2:4, -1].numpy(), a[1, :, 2:4, -1])
    close(A[:, None, 1].numpy(), a[:, None, 1])
    close(A.shrink(((0, 2), (1, 3), None, (2, 5))).numpy(), a[0:2, 1:3, :, 2:5])
    close(A.pad(((0, 0), (1, 2), (0, 0), (3, 0))).numpy(), np.pad(a, ((0, 0), (1, 2), (0, 0), (3, 0))))
    close(A[:, :1].expand(2, 4, 4, 5).numpy(), np.broadcast_to(a[:, :1], (2, 4, 4, 5)))
    b = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    close(T.Tensor.stack(A, T.Tensor(b)).numpy(), np.stack([a, b]))
    close(A.cat(T.Tensor(b), dim=2).numpy(), np.concatenate([a, b], 2))
    m = T.Tensor.full((1, 1, 4, 6), float("-inf")).triu(3).numpy()
    want = np.triu(np.full((4, 6), -np.inf, np.float32), 3)[None, None]
    assert np.array_equal(m, want)
    assert T.Tensor.arange(3, 15, 4).numpy().tolist() == [3, 7, 11]


@pytest.mark.parametrize("M", [1, 3])
def test_linear_gemv_builtin_and_generic_matmul(T, M):
    say(f"case: linear M={M}")
    rng = np.random.default_rng(4 + M)
    K, N = 320, 200
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    X, W, Bv = T.Tensor(x), T.Tensor(w), T.Tensor(b)
    g0 = T.GlobalCounters.gemv_count
    y = X.linear(W.transpose(), Bv).numpy()
    assert T.GlobalCounters.gemv_count == g0 + 1, "x @ W.T + b did not run the GEMV builtin"
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    close(y, want, rtol=1e-4, atol=1e-4)
    # generic batched matmul (rendered reduce)
    p = rng.standard_normal((2, 3, 4, 33)).astype(np.float32)
    q = rng.standard_normal((2, 1, 33, 7)).astype(np.float32)
    close((T.Tensor(p) @ T.Tensor(q)).numpy(), p.astype(np.float64) @ q.astype(np.float64), rtol=1e-4, atol=1e-5)


def test_assign_and_symbolic_reads(T):
    say("case: assign + variable")
    rng = np.random.default_rng(5)
    cache = T.Tensor.zeros(2, 1, 16, 3, 4).contiguous().realize()
    rows = []
    for pos in range(5):
        sp = T.Variable("pos_t", 0, 15).bind(pos)
        k = rng.standard_normal((1, 1, 3, 4)).astype(np.float32)
        v = rng.standard_normal((1, 1, 3, 4)).astype(np.float32)
        rows.append((k, v))
        cache[:, :, sp:sp + 1, :, :].assign(T.Tensor.stack(T.Tensor(k), T.Tensor(v))).realize()
        keys = cache[0][:, :sp + 1, :, :]
        got = keys.sum(1).numpy()             # reduce over the symbolic length
        want = np.sum([r[0] for r in rows], axis=0)[:, 0]
        close(got, want, rtol=1e-5, atol=1e-6)
    full = cache.numpy()
    for pos, (k, v) in enumerate(rows):
        close(full[0, :, pos], k[:, 0])
        close(full[1, :, pos], v[:, 0])
    assert np.all(full[:, :, 5:] == 0)


def test_tinyjit_capture_and_replay(T):
    say("case: tinyjit")
    rng = np.random.default_rng(6)
    W = T.Tensor((rng.standard_normal((64, 96)) * 0.1).astype(np.float32))
    hist = T.Tensor.zeros(1, 32, 64).contiguous().realize()

    def f(x, sp):
        y = x.linear(W.transpose()).gelu()                       # [1, 64]
        hist[:, sp:sp + 1, :].assign(y.reshape(1, 1, 64)).realize()
        h = hist[:, :sp + 1, :]
        return (h.softmax(1) * h).sum(1).realize()                # softmax over the live length

    jf = T.TinyJit(f)
    hnp = np.zeros((32, 64))
    for step in range(6):
        x = rng.standard_normal((1, 96)).astype(np.float32)
        sp = T.Variable("sp_t", 0, 31).bind(step)
        got = jf(T.Tensor(x), sp).numpy()
        y = x.astype(np.float64) @ W.numpy().astype(np.float64).T
        y = 0.5 * y * (1 + np.tanh(np.sqrt(2 / np.pi) * (y + 0.044715 * y ** 3)))
        hnp[step] = y[0]
        h = hnp[:step + 1]
        e = np.exp(h - h.max(0))
        want = ((e / e.sum(0)) * h).sum(0)[None]
        close(got, want, rtol=1e-4, atol=1e-5)
    assert jf.cnt == 2 and jf.jit is not None and jf.jit.op_count() > 0


def _oracle_gpt2(weights, cfg):
    class Dec:
        def __init__(self):
            self.t = dict(weights)
            B, H, ms, hd = cfg["batch"], cfg["n_heads"], cfg["max_seq"], cfg["head_dim"]
            for l in range(cfg["n_layers"]):
                self.t[f"l{l}.kcache"] = np.zeros((B, H, ms, hd), np.float32)
                self.t[f"l{l}.vcache"] = np.zeros((B, H, ms, hd), np.float32)

        def read_tensor(self, name):
            return np.ascontiguousarray(self.t[name])

    return O.OracleModel(Dec(), cfg)


@pytest.mark.parametrize("host_gemv", ["1", "0"], ids=["gemv-builtin", "rendered-matmul"])
def test_gpt2_driver_matches_oracle(T, monkeypatch, host_gemv):
    """The GPT-2 driver against the oracle, with x @ W.T on the GEMV builtin
    and, THVM_HOST_GEMV=0, rendered through the renderer target like every
    other kernel (no builtin at all)."""
    say(f"case: gpt2 host vs oracle, THVM_HOST_GEMV={host_gemv}")
    monkeypatch.setenv("THVM_HOST_GEMV", host_gemv)
    n_gemv = T.GlobalCounters.gemv_count
    from thvm_amd.gpt2 import GPT2
    L, D, H, V, MS = 2, 128, 4, 1000, 32
    w = GPT2.synthetic_weights(L, D, V, MS, seed=7)
    g = GPT2(w, L, H, D, V, MS)
    cfg = dict(arch=2, n_layers=L, dim=D, n_heads=H, n_kv_heads=H, head_dim=D // H, ffn=4 * D, vocab=V,
               max_seq=MS, batch=1, wdtype=13, adtype=13, eps=1e-5)
    orc = _oracle_gpt2(w, cfg)
    prompt = [11, 503, 42, 7, 999]
    cur, n_new = prompt[0], 6
    for pos in range(len(prompt) + n_new - 1):
        nxt = int(g.step(np.array([cur], np.int32), pos)[0])
        lg_dev = g.logits.numpy().reshape(-1)
        lg_ref, nx_ref = orc.step(np.array([cur], np.int32), pos)
        err = np.abs(lg_dev - lg_ref[0]).max() / np.abs(lg_ref[0]).max()
        say(f"pos {pos}: id {nxt} ref {int(nx_ref[0])} logits rel err {err:.2e}")
        assert err <= 1e-5, err                  # fp32: 1e-5 relative (north star)
        assert nxt == int(nx_ref[0])
        cur = prompt[pos + 1] if pos + 1 < len(prompt) else nxt
    assert g.jit.cnt == 2, "the one-token forward was not captured"
    if host_gemv == "0":
        assert T.GlobalCounters.gemv_count == n_gemv, "a matmul reached the GEMV builtin"


def test_state_dict_save_load_roundtrip(T, tmp_path):
    """get_state_dict -> safe_save -> safe_load -> load_state_dict into a
    fresh model: every tensor bit-equal (f32 and a bf16 one), and the loaded
    model's forward equals the saved model's; a shape mismatch raises."""
    say("case: state dict roundtrip")
    from thvm_amd import nn, state as S

    class Net:
        def __init__(self):
            self.l1 = nn.Linear(32, 48)
            self.ln = nn.LayerNorm(48)
            self.l2 = nn.Linear(48, 16, bias=False)
            self.emb = T.Tensor(np.arange(12, dtype=np.float32).reshape(3, 4) / 7, dtype=T.dtypes.bfloat16)

        def __call__(self, x):
            return self.l2(self.ln(self.l1(x).relu()))

    nn.manual_seed(1)
    a = Net()
    nn.manual_seed(2)
    b = Net()
    x = T.Tensor(np.random.default_rng(3).standard_normal((5, 32)).astype(np.float32))
    fn = tmp_path / "net.safetensors"
    S.safe_save(S.get_state_dict(a), fn)
    loaded = S.safe_load(fn)
    assert loaded["emb"].dtype.id == T.dtypes.bfloat16.id
    got = S.load_state_dict(b, loaded)
    assert len(got) == len(S.get_parameters(a)) == 6
    for k, v in S.get_state_dict(a).items():
        assert np.array_equal(S.get_state_dict(b)[k].numpy(), v.numpy()), k
    assert np.array_equal(b(x).numpy(), a(x).numpy())
    bad = dict(loaded)
    bad["l1.weight"] = np.zeros((32, 48), np.float32)
    with pytest.raises(ValueError):
        S.load_state_dict(b, bad)


def test_more_elementwise_and_statistics(T):
    """The tinygrad-named ops a reference script reaches for: eq/ne, sign,
    trunc, erf, elu, softmin, bitwise and shifts, var/std, tril/eye,
    split/chunk, *_like, against numpy."""
    say("case: more ops")
    import math
    rng = np.random.default_rng(21)
    a = (rng.standard_normal((4, 33)) * 2).astype(np.float32)
    A, ad = T.Tensor(a), a.astype(np.float64)
    close(A.sign().numpy(), np.sign(ad))
    close(A.trunc().numpy(), np.trunc(ad))
    close(A.erf().numpy(), np.vectorize(math.erf)(ad), rtol=0, atol=1e-6)   # 1.5e-7 method + f32 rounding
    close(A.elu().numpy(), np.where(ad > 0, ad, np.exp(ad) - 1), rtol=1e-5, atol=1e-6)
    e = np.exp(-ad - (-ad).max(-1, keepdims=True))
    close(A.softmin(-1).numpy(), e / e.sum(-1, keepdims=True), rtol=1e-5, atol=1e-8)
    close(A.var(-1).numpy(), ad.var(-1, ddof=1), rtol=1e-5, atol=1e-6)
    close(A.std(1, correction=0).numpy(), ad.std(1), rtol=1e-5, atol=1e-6)
    v, m = A.var_mean(0)
    close(v.numpy(), ad.var(0, ddof=1), rtol=1e-5, atol=1e-6)
    close(m.numpy(), ad.mean(0), rtol=1e-5, atol=1e-6)
    assert np.array_equal(A.eq(A).numpy(), np.ones_like(a, bool)) and not A.ne(A).numpy().any()
    i = rng.integers(-1000, 1000, (3, 17)).astype(np.int32)
    I = T.Tensor(i)
    assert np.array_equal(I.bitwise_and(0x5A).numpy(), i & 0x5A)
    assert np.array_equal(I.bitwise_or(0x21).numpy(), i | 0x21)
    assert np.array_equal(I.bitwise_xor(77).numpy(), i ^ 77)
    assert np.array_equal(I.bitwise_not().numpy(), ~i)
    assert np.array_equal(I.lshift(3).numpy(), i << 3)
    assert np.array_equal(I.rshift(2).numpy(), i >> 2)
    sq = rng.standard_normal((5, 5)).astype(np.float32)
    assert np.array_equal(T.Tensor(sq).tril(-1).numpy(), np.tril(sq, -1))
    assert np.array_equal(T.Tensor(sq).tril(1).numpy(), np.tril(sq, 1))
    assert np.array_equal(T.Tensor.eye(3, 4).numpy(), np.eye(3, 4, dtype=np.float32))
    parts = A.split([10, 23], dim=1)
    assert np.array_equal(parts[1].numpy(), a[:, 10:])
    ch = A.chunk(4, dim=1)
    assert [c.shape[1] for c in ch] == [9, 9, 9, 6] and np.array_equal(ch[2].numpy(), a[:, 18:27])
    assert np.array_equal(A.zeros_like().numpy(), np.zeros_like(a))
    assert np.array_equal(A.full_like(2.5).numpy(), np.full_like(a, 2.5))
    assert np.array_equal(A.clone().numpy(), a) and A.size(1) == 33 and A.element_size() == 4


def test_device_random_and_multinomial(T):
    """rand / randn / randint / multinomial on the device generator: ranges
    and moments, reproducible after manual_seed, fresh draws on every call
    and on every TinyJit replay; multinomial frequencies against the weights
    (chi-square), without replacement never repeating an index.  Random
    streams are this generator's own, not the reference's."""
    say("case: device random")
    T.Tensor.manual_seed(7)
    u = T.Tensor.rand(200000).numpy()
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.005 and abs(u.var() - 1 / 12) < 0.002
    u2 = T.Tensor.rand(200000).numpy()
    assert not np.array_equal(u, u2)
    T.Tensor.manual_seed(7)
    assert np.array_equal(T.Tensor.rand(200000).numpy(), u)
    z = T.Tensor.randn(100000).numpy()
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1) < 0.02
    r = T.Tensor.randint(50000, low=3, high=9).numpy()
    assert r.min() == 3 and r.max() == 8
    p = np.array([0.1, 0.2, 0.3, 0.4], np.float32)
    draws = T.Tensor(p).multinomial(20000, replacement=True).numpy()
    cnt = np.bincount(draws, minlength=4)
    chi2 = (((cnt - 20000 * p) ** 2) / (20000 * p)).sum()
    assert chi2 < 16.3, (cnt, chi2)          # 3 dof, p = 0.001
    w = T.Tensor(np.ones((3, 6), np.float32))
    nr = w.multinomial(6).numpy()
    assert all(sorted(row) == list(range(6)) for row in nr)

    @T.TinyJit
    def draw(x):
        return (x + T.Tensor.rand(64)).realize()

    x = T.Tensor(np.zeros(64, np.float32))
    outs = [draw(x).numpy().copy() for _ in range(4)]
    assert all(not np.array_equal(outs[i], outs[i + 1]) for i in range(3))
