"""Checkpoint formats (thvm_amd/weights.py), CPU only.

* safetensors: our files read by the `safetensors` package and its files
  read by us, bf16 / fp8 / f16 / i64 tensors, metadata, zero-size tensors;
  the header layout of the reference's safe_save (compact JSON padded with
  spaces to 8 bytes).
* torch_load against torch.save in the zip and the legacy formats: f32,
  f16, bf16 (widened to f32), int64, a transposed (non-contiguous) tensor, a
  storage shared by two views; a pickle naming any other global is refused.
* DSV2PK01: the pack tests/_dsv2_weights.py writes reads back entry by entry.
* GGUF: files written here by the format's definition (header, metadata,
  tensor infos, aligned data) read back; Q8_0 and Q4_0 dequantise as the
  block definitions say; an unsupported type raises NotImplementedError.
* The Hugging Face rotate-half q/k row order converted to interleaved pairs
  gives the same attention scores (the RoPE definitions are equal)."""
import io
import os
import pickle
import struct

import numpy as np
import pytest

from thvm_amd import weights as W


def test_safetensors_roundtrip_and_interop(tmp_path):
    from safetensors.numpy import load_file, save_file
    rng = np.random.default_rng(0)
    t = {"a": rng.standard_normal((3, 5)).astype(np.float32),
         "b": rng.standard_normal(7).astype(np.float16),
         "c": np.arange(12, dtype=np.int64).reshape(3, 4),
         "z": np.zeros((0, 4), np.float32)}
    bf = W.f32_to_bf16(rng.standard_normal((4, 8)).astype(np.float32))
    fn = tmp_path / "ours.safetensors"
    W.safe_save(t, tmp_path / "plain.safetensors")
    theirs = load_file(str(tmp_path / "plain.safetensors"))   # their reader on our file
    assert set(theirs) == set(t) and all(np.array_equal(theirs[k], v) for k, v in t.items())
    W.safe_save(dict(t, bf=(bf, W.DT_BF16), f8=(np.arange(16, dtype=np.uint8), W.DT_FP8E4M3)),
                fn, metadata={"format": "pt"})
    n = int.from_bytes(open(fn, "rb").read(8), "little")
    assert n % 8 == 0
    torch = pytest.importorskip("torch")
    from safetensors.torch import load_file as tload
    tt = tload(str(fn))                    # bf16 / fp8 through their torch reader
    assert tt["bf"].dtype == torch.bfloat16 and np.array_equal(tt["bf"].view(torch.int16).numpy().view(np.uint16), bf)
    assert tt["f8"].dtype == torch.float8_e4m3fn
    ours = W.safe_load(fn)
    for k, v in t.items():
        assert ours[k].shape == v.shape and np.array_equal(np.asarray(ours[k].numpy()), v)
    assert ours["bf"].dtype == W.DT_BF16 and np.array_equal(ours["bf"].numpy(), bf)
    assert np.array_equal(ours["bf"].float32(), W.bf16_to_f32(bf))
    assert ours["f8"].dtype == W.DT_FP8E4M3
    fn2 = tmp_path / "theirs.safetensors"
    save_file(t, str(fn2))                 # our reader on their file
    back = W.safe_load(fn2)
    for k, v in t.items():
        assert np.array_equal(np.asarray(back[k].numpy()), v)


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, -2.5, np.inf, np.nan], np.float32)
    b = W.f32_to_bf16(x)
    assert list(b[:5]) == [0x3F80, 0x3F80, 0x3F81, 0xC020, 0x7F80]
    assert np.isnan(W.bf16_to_f32(b)[5])


def _torch():
    return pytest.importorskip("torch")


@pytest.mark.parametrize("zipped", [True, False])
def test_torch_load_matches_torch_save(tmp_path, zipped):
    torch = _torch()
    g = torch.Generator().manual_seed(1)
    base = torch.randn(6, 4, generator=g)
    sd = {"w": torch.randn(3, 5, generator=g), "h": torch.randn(4, generator=g).half(),
          "bf": torch.randn(2, 3, generator=g).to(torch.bfloat16),
          "i": torch.arange(10, dtype=torch.int64), "t": base.t(), "part": base[2:4]}
    fn = tmp_path / "ckpt.pt"
    torch.save(sd, fn, _use_new_zipfile_serialization=zipped)
    got = W.torch_load(fn)
    for k, v in sd.items():
        want = v.float().numpy() if v.dtype == torch.bfloat16 else v.numpy()
        assert got[k].shape == tuple(v.shape) and np.array_equal(got[k], want), k


def test_torch_load_refuses_foreign_globals(tmp_path):
    class Boom:
        def __reduce__(self):
            return (os.system, ("true",))
    fn = tmp_path / "evil.pt"
    with open(fn, "wb") as f:
        pickle.dump({"x": Boom()}, f)
    with pytest.raises(pickle.UnpicklingError):
        W.torch_load(fn)


def _crafted_ckpt(fn, numel, payload_elems, offset, size, stride):
    """A zip checkpoint whose pickle claims a view (offset, size, stride) of
    a float32 storage of `numel` elements holding `payload_elems` floats."""
    import collections
    import zipfile
    torch = _torch()

    class StorageRef:
        pass

    class View:
        def __reduce__(self):
            return (torch._utils._rebuild_tensor_v2,
                    (StorageRef(), offset, size, stride, False, collections.OrderedDict()))

    class P(pickle.Pickler):
        def persistent_id(self, obj):
            if isinstance(obj, StorageRef):
                return ("storage", torch.FloatStorage, "0", "cpu", numel)
            return None

    buf = io.BytesIO()
    P(buf, protocol=2).dump({"w": View()})
    with zipfile.ZipFile(fn, "w") as zf:
        zf.writestr("ckpt/data.pkl", buf.getvalue())
        zf.writestr("ckpt/data/0", np.arange(payload_elems, dtype=np.float32).tobytes())


@pytest.mark.parametrize("case", [
    dict(numel=4, payload_elems=4, offset=0, size=(1 << 20,), stride=(1,)),   # view past the end
    dict(numel=4, payload_elems=4, offset=3, size=(2,), stride=(1,)),         # off by one
    dict(numel=4, payload_elems=4, offset=-1, size=(2,), stride=(1,)),        # negative offset
    dict(numel=4, payload_elems=4, offset=0, size=(2,), stride=(-1,)),        # negative stride
    dict(numel=8, payload_elems=4, offset=0, size=(8,), stride=(1,)),         # short payload
])
def test_torch_load_refuses_views_outside_their_storage(tmp_path, case):
    fn = tmp_path / "crafted.pt"
    _crafted_ckpt(fn, **case)
    with pytest.raises(ValueError):
        W.torch_load(fn)


def test_torch_load_crafted_view_inside_storage_loads(tmp_path):
    fn = tmp_path / "ok.pt"
    _crafted_ckpt(fn, numel=6, payload_elems=6, offset=1, size=(2, 2), stride=(3, 1))
    got = W.torch_load(fn)["w"]
    assert np.array_equal(got, np.array([[1, 2], [4, 5]], np.float32))


def test_dsv2pk_reads_the_pack_writer(tmp_path):
    import _dsv2_weights as DW
    cfg = dict(n_layers=2, dim=64, n_heads=4, kv_lora=32, d_nope=16, d_rope=8, d_v=16, n_experts=4,
               n_shared=1, top_k=2, moe_inter=32, ffn=96, first_dense=1, vocab=100, max_seq=16,
               batch=1, eps=1e-6, init_std=0.02)
    t = DW.make_dsv2(cfg, 3)
    fn = tmp_path / "m.pack"
    DW.write_pack(t, cfg, str(fn))
    p = W.dsv2pk_load(fn)
    assert np.array_equal(p["embed"].numpy(), t["emb"].reshape(-1))
    assert np.array_equal(p["lm_head"].numpy(), np.ascontiguousarray(t["lm"].T).reshape(-1))
    assert np.array_equal(p["l1.gate"].float32(), np.ascontiguousarray(t["l1.gate"].T).reshape(-1))
    nq = cfg["n_heads"] * (cfg["d_nope"] + cfg["d_rope"])
    assert np.array_equal(p["l0.wkv"].numpy(), np.ascontiguousarray(t["l0.wqkv"][nq:].T).reshape(-1))
    assert p["l0.wg1"].dtype == W.DT_BF16 and p["norm"].dtype == W.DT_FP32
    with open(tmp_path / "bad.pack", "wb") as f:
        f.write(b"NOTAPACK" + bytes(8))
    with pytest.raises(ValueError):
        W.dsv2pk_load(tmp_path / "bad.pack")


def _gguf_str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _write_gguf(fn, tensors, align=32, extra_meta=()):
    """GGUF v3 by its definition: magic, version, tensor count, kv count,
    kv pairs, tensor infos (name, n_dims, dims fastest first, type, offset),
    padding to the alignment, then the aligned tensor data."""
    kv = [(_gguf_str("general.architecture"), 8, _gguf_str("test")),
          (_gguf_str("general.alignment"), 4, struct.pack("<I", align))] + list(extra_meta)
    out = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for k, t, v in kv:
        out += k + struct.pack("<I", t) + v
    off, blobs = 0, []
    for name, shape, typ, raw in tensors:
        out += _gguf_str(name) + struct.pack("<I", len(shape))
        out += struct.pack(f"<{len(shape)}Q", *reversed(shape)) + struct.pack("<IQ", typ, off)
        blobs.append((off, raw))
        off = (off + len(raw) + align - 1) // align * align
    pad = (len(out) + align - 1) // align * align
    data = bytearray(off)
    for o, raw in blobs:
        data[o:o + len(raw)] = raw
    with open(fn, "wb") as f:
        f.write(out + bytes(pad - len(out)) + bytes(data))


def test_gguf_reader(tmp_path):
    rng = np.random.default_rng(2)
    f32 = rng.standard_normal((3, 8)).astype(np.float32)
    f16 = rng.standard_normal((2, 32)).astype(np.float16)
    # Q8_0: 2 blocks of 32; Q4_0: 2 blocks of 32
    d8 = np.array([0.5, 0.25], np.float16)
    q8 = rng.integers(-127, 128, (2, 32)).astype(np.int8)
    raw8 = b"".join(d8[i:i + 1].tobytes() + q8[i].tobytes() for i in range(2))
    d4 = np.array([0.125, 2.0], np.float16)
    q4 = rng.integers(0, 16, (2, 32)).astype(np.uint8)
    raw4 = b"".join(d4[i:i + 1].tobytes() + (q4[i, :16] | (q4[i, 16:] << 4)).astype(np.uint8).tobytes()
                    for i in range(2))
    meta = [(_gguf_str("test.list"), 9, struct.pack("<IQ", 5, 3) + struct.pack("<3i", 1, -2, 3))]
    fn = tmp_path / "m.gguf"
    _write_gguf(fn, [("a", (3, 8), W.GGUF_F32, f32.tobytes()), ("b", (2, 32), W.GGUF_F16, f16.tobytes()),
                     ("c", (64,), W.GGUF_Q8_0, raw8), ("d", (2, 32), W.GGUF_Q4_0, raw4)], extra_meta=meta)
    m, t = W.gguf_load(fn)
    assert m["general.architecture"] == "test" and m["test.list"] == [1, -2, 3]
    assert np.array_equal(np.asarray(t["a"].numpy()), f32)
    assert np.array_equal(np.asarray(t["b"].numpy()), f16)
    assert np.array_equal(t["c"], (d8.astype(np.float32)[:, None] * q8.astype(np.float32)).reshape(64))
    assert np.array_equal(t["d"], d4.astype(np.float32)[:, None] * (q4.astype(np.float32) - 8))
    _write_gguf(tmp_path / "q6k.gguf", [("e", (256,), 14, bytes(210))])
    with pytest.raises(NotImplementedError):
        W.gguf_load(tmp_path / "q6k.gguf")


def test_hf_rotate_half_rows_become_interleaved_pairs():
    """HF Llama computes RoPE as q * cos + rotate_half(q) * sin over rows
    ordered for it; the decoder rotates adjacent pairs.  After the row
    permutation the two give the same rotated vectors (up to that
    permutation), hence the same attention scores q . k."""
    rng = np.random.default_rng(4)
    H, hd, D, pos, theta = 3, 16, 24, 37, 10000.0
    w = rng.standard_normal((H * hd, D))
    x = rng.standard_normal(D)
    inv = theta ** (-np.arange(0, hd, 2) / hd)
    ang = pos * inv
    q_hf = (w @ x).reshape(H, hd)
    cos = np.concatenate([np.cos(ang)] * 2)
    sin = np.concatenate([np.sin(ang)] * 2)
    rot = np.concatenate([-q_hf[:, hd // 2:], q_hf[:, :hd // 2]], 1)
    hf = q_hf * cos + rot * sin                                   # HF apply_rotary_pos_emb
    q_il = (W.hf_rope_rows_to_interleaved(w, H) @ x).reshape(H, hd)
    z = (q_il[:, 0::2] + 1j * q_il[:, 1::2]) * np.exp(1j * ang)   # adjacent-pair RoPE
    il = np.empty_like(q_il)
    il[:, 0::2], il[:, 1::2] = z.real, z.imag
    assert np.allclose(il[:, 0::2], hf[:, :hd // 2]) and np.allclose(il[:, 1::2], hf[:, hd // 2:])


@pytest.mark.parametrize("dt", [W.DT_FP8E4M3, W.DT_FP8E5M2])
def test_fp8_disk_tensors_decode_like_the_oracle(tmp_path, dt):
    """fp8 tensors in a safetensors file read back as the OCP values of their
    codes: every one of the 256 patterns against the oracle's decoder (pinned
    to the reference's tables), NaNs as NaN."""
    import _oracle as O
    codes = np.arange(256, dtype=np.uint8).reshape(16, 16)
    fn = tmp_path / "f8.safetensors"
    W.safe_save({"w": (codes, dt)}, fn)
    got = W.safe_load(fn)["w"].float32()
    want = O.decode(codes, dt)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])


def test_state_dict_names_follow_the_attribute_paths():
    """get_state_dict keys are dotted attribute paths, list indices and dict
    keys (py/thvm/nn_state.py:233-241), built without touching the device."""
    from thvm_amd import state as S
    from thvm_amd.tensor import LNode, Tensor, dtypes

    def t():
        return Tensor(LNode("CONST", (), 0.0, (), dtypes.float32))

    class Block:
        def __init__(self):
            self.ln = {"weight": t(), "bias": t()}
            self.mlp = [t(), t()]
            self.eps = 1e-5

    class Model:
        def __init__(self):
            self.wte = t()
            self.h = [Block(), Block()]

    m = Model()
    sd = S.get_state_dict(m)
    assert list(sd) == ["wte", "h.0.ln.weight", "h.0.ln.bias", "h.0.mlp.0", "h.0.mlp.1",
                        "h.1.ln.weight", "h.1.ln.bias", "h.1.mlp.0", "h.1.mlp.1"]
    assert sd["h.1.mlp.0"] is m.h[1].mlp[0]
    assert list(S.get_state_dict(m, prefix="model."))[0] == "model.wte"
    assert len(S.get_parameters(m)) == 9
    with pytest.raises(KeyError):
        S.load_state_dict(m, {"h.0.ln.weight": np.zeros(())})     # "wte" missing: strict
