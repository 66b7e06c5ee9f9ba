"""The no-allocation attention entry point (thvm_hip_attn_decode_noalloc)
against the attention builtin with a caller-provided partials workspace
(thvm_hip_dispatch_custom "thvm-builtin:attn ..."): both run the same split
and merge kernels over the same partial layout, so the outputs agree bit for
bit.  Two calls in a row, the second with a smaller input, in the two-launch
and the one-launch (merge counters) forms; and a spec whose partials exceed
the static array is refused with an error."""
import ctypes as C

import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu

DT_BF16 = 12


def say(*a):
    print(*a, flush=True)


def up(hip, a):
    return hip.Buffer.from_numpy(np.ascontiguousarray(a))


def _case(hip, rng, B, H, Hkv, hd, ms, L):
    q = O.encode(rng.standard_normal((B, H, hd)).astype(np.float32), DT_BF16)
    kc = O.encode(rng.standard_normal((B, Hkv, ms, hd)).astype(np.float32), DT_BF16)
    vc = O.encode(rng.standard_normal((B, Hkv, ms, hd)).astype(np.float32), DT_BF16)
    return dict(q=up(hip, q), k=up(hip, kc), v=up(hip, vc), len=up(hip, np.array([L], np.int32)))


def _spec(B, H, Hkv, hd, ms, fused):
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    return (f"thvm-builtin:attn b={B} h={H} hkv={Hkv} hd={hd} maxseq={ms} qt=12 ct=12 ot=12 "
            f"scale={scale.hex()} fused={fused}")


@pytest.mark.parametrize("fused", [0, 1])
def test_attn_noalloc_matches_workspace_entry(hip, fused):
    L_ = hip.lib()
    rng = np.random.default_rng(40 + fused)
    for B, H, Hkv, hd, ms, L in ((4, 32, 8, 128, 2176, 2049), (1, 8, 2, 64, 256, 130)):
        say(f"case: attn noalloc fused={fused} B={B} H={H} Hkv={Hkv} hd={hd} maxseq={ms} L={L}")
        t = _case(hip, rng, B, H, Hkv, hd, ms, L)
        spec = _spec(B, H, Hkv, hd, ms, fused)
        nsplit = (ms + 63) // 64
        part = hip.Buffer(B * H * nsplit * (hd + 2) * 4 + B * Hkv * 4)
        out_ref, out_na = hip.Buffer(B * H * hd * 2), hip.Buffer(B * H * hd * 2)
        hip.dispatch("attn", spec, [out_ref, t["q"], t["k"], t["v"], t["len"], part])
        ids = (C.c_uint32 * 5)(out_na.id, t["q"].id, t["k"].id, t["v"].id, t["len"].id)
        assert L_.thvm_hip_attn_decode_noalloc(spec.encode(), ids, 5) == 0, hip.last_error()
        a, b = out_ref.read(np.uint16), out_na.read(np.uint16)
        assert np.array_equal(a, b), f"{np.sum(a != b)} of {a.size} outputs differ"
        assert np.all(np.isfinite(O.decode(b, DT_BF16)))


def test_attn_noalloc_rejects_oversize_and_bad_calls(hip):
    say("case: attn noalloc errors (host-side, no launch)")
    L_ = hip.lib()
    B, H, Hkv, hd, ms = 8, 64, 1, 64, 8192            # 17.3 MB of partials > 16 MiB
    bufs = [hip.Buffer(B * H * hd * 2), hip.Buffer(B * H * hd * 2),
            hip.Buffer(B * Hkv * ms * hd * 2), hip.Buffer(B * Hkv * ms * hd * 2),
            up(hip, np.array([5], np.int32))]
    ids = (C.c_uint32 * 5)(*[b.id for b in bufs])
    assert L_.thvm_hip_attn_decode_noalloc(_spec(B, H, Hkv, hd, ms, 0).encode(), ids, 5) == -1
    assert "static scratch" in hip.last_error()
    assert L_.thvm_hip_attn_decode_noalloc(b"thvm-builtin:softmax m=1 k=4", ids, 5) == -1
    assert L_.thvm_hip_attn_decode_noalloc(_spec(1, 8, 2, 64, 64, 0).encode(), ids, 4) == -1
