"""thvm_amd.weights -- checkpoint formats and loading them into a decoder.

Reference counterparts: ``py/thvm/nn_state.py:51-123`` (safetensors load /
save, torch_load), ``bench/dsv2_decode_bench.c:229-310`` (the DSV2PK01 weight
pack), ``src/tensor/mmap.c`` (mmap-backed disk tensors) and
``py/thvm/gguf.py`` (which raises for every GGUF file; here the unquantised
and the 8-bit / 4-bit block types are read).

A ``DiskTensor`` is a byte range of a file: ``numpy()`` maps it
(``np.memmap``, zero copy) and ``upload(buffer)`` streams it to a device
buffer through the library's pinned staging ring
(``thvm_hip_buf_load_file``) without a host copy of the whole tensor.

``load_llama`` / ``load_gpt2`` / ``load_dsv2`` write a state dict into a
``thvm_amd.Decoder`` of the same shape, converting layouts on the host
(row concatenation, gate/up interleave, Hugging Face's rotate-half q/k row
order to the decoder's interleaved RoPE pairs) and quantising to fp8 on the
device (per-row absmax/448 e4m3, the builtin ``quant_fp8``) when the decoder
holds fp8 weights."""
from __future__ import annotations

import io
import json
import os
import pickle
import struct
import zipfile
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

DT_BOOL, DT_INT8, DT_UINT8, DT_INT16, DT_UINT16, DT_INT32, DT_UINT32, DT_INT64, DT_UINT64 = \
    0, 1, 2, 3, 4, 5, 6, 7, 8
DT_FP8E4M3, DT_FP8E5M2, DT_FP16, DT_BF16, DT_FP32, DT_FP64 = 9, 10, 11, 12, 13, 14

# dtype id -> (numpy storage type, itemsize); bf16 / fp8 are kept as raw bits
_STORE = {DT_BOOL: (np.bool_, 1), DT_INT8: (np.int8, 1), DT_UINT8: (np.uint8, 1),
          DT_INT16: (np.int16, 2), DT_UINT16: (np.uint16, 2), DT_INT32: (np.int32, 4),
          DT_UINT32: (np.uint32, 4), DT_INT64: (np.int64, 8), DT_UINT64: (np.uint64, 8),
          DT_FP8E4M3: (np.uint8, 1), DT_FP8E5M2: (np.uint8, 1), DT_FP16: (np.float16, 2),
          DT_BF16: (np.uint16, 2), DT_FP32: (np.float32, 4), DT_FP64: (np.float64, 8)}

# safetensors dtype tags (the format's own names)
SAFE_DTYPES = {"BOOL": DT_BOOL, "I8": DT_INT8, "U8": DT_UINT8, "I16": DT_INT16, "U16": DT_UINT16,
               "I32": DT_INT32, "U32": DT_UINT32, "I64": DT_INT64, "U64": DT_UINT64,
               "F16": DT_FP16, "BF16": DT_BF16, "F32": DT_FP32, "F64": DT_FP64,
               "F8_E4M3": DT_FP8E4M3, "F8_E5M2": DT_FP8E5M2}
_SAFE_TAGS = {v: k for k, v in SAFE_DTYPES.items()}


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def fp8_table(dt: int) -> np.ndarray:
    """The 256 values of an OCP OFP8 format as f32, from its definition:
    e4m3 (bias 7, 3 mantissa bits, S.1111.111 NaN, no infinities) or e5m2
    (bias 15, 2 mantissa bits, IEEE-style infinities and NaNs); subnormals
    at the smallest exponent."""
    mb, bias = (3, 7) if dt == DT_FP8E4M3 else (2, 15)
    b = np.arange(256)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> mb) & ((1 << (7 - mb)) - 1)
    m = b & ((1 << mb) - 1)
    v = np.where(e == 0, m / (1 << mb) * 2.0 ** (1 - bias), (1 + m / (1 << mb)) * 2.0 ** (e - bias))
    if dt == DT_FP8E4M3:
        v = np.where((b & 0x7F) == 0x7F, np.nan, v)
    else:
        top = e == 31
        v = np.where(top & (m == 0), np.inf, np.where(top, np.nan, v))
    return (s * v).astype(np.float32)


@dataclass
class DiskTensor:
    """A tensor stored in a file: `nbytes` bytes at `offset`."""
    path: str
    offset: int
    nbytes: int
    dtype: int
    shape: tuple

    def numpy(self) -> np.ndarray:
        """The bytes as a read-only memory map (bf16 / fp8 as raw bits)."""
        npdt, isz = _STORE[self.dtype]
        n = int(np.prod(self.shape)) if self.shape else 1
        if n * isz != self.nbytes:
            raise ValueError(f"{self.path}@{self.offset}: {self.nbytes} bytes for shape {self.shape}")
        if n == 0:
            return np.zeros(self.shape, npdt)
        return np.memmap(self.path, dtype=npdt, mode="r", offset=self.offset,
                         shape=tuple(self.shape) if self.shape else (1,))

    def float32(self) -> np.ndarray:
        a = self.numpy()
        if self.dtype == DT_BF16:
            return bf16_to_f32(a)
        if self.dtype in (DT_FP8E4M3, DT_FP8E5M2):
            return fp8_table(self.dtype)[np.asarray(a)]
        return np.asarray(a, np.float32)

    def upload(self, buf, dst_off: int = 0) -> None:
        """Stream the bytes into a device buffer (id or thvm_amd.Buffer)."""
        from thvm_amd import _check, lib
        bid = buf if isinstance(buf, int) else buf.id
        _check(lib().thvm_hip_buf_load_file(bid, dst_off, os.fsencode(self.path), self.offset,
                                            self.nbytes), f"load {self.path}")


# ------------------------------------------------------------ safetensors --
def safe_load_metadata(fn):
    """(8-byte header length + 8 = data start, the JSON header)."""
    with open(fn, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(n))
    return n + 8, header


def safe_load(fn) -> Dict[str, DiskTensor]:
    """A .safetensors file as disk tensors, each in its own dtype
    (py/thvm/nn_state.py:51-62)."""
    start, header = safe_load_metadata(fn)
    out = {}
    for k, v in header.items():
        if k == "__metadata__":
            continue
        lo, hi = v["data_offsets"]
        out[k] = DiskTensor(str(fn), start + lo, hi - lo, SAFE_DTYPES[v["dtype"]], tuple(v["shape"]))
    return out


def safe_save(tensors: Dict[str, "np.ndarray | tuple"], fn, metadata: Optional[dict] = None) -> None:
    """Write a .safetensors file: compact JSON header padded with spaces to 8
    bytes, tensors in insertion order (py/thvm/nn_state.py:64-85).  Values
    are numpy arrays, or (raw bits, dtype id) for bf16 / fp8."""
    headers, off, blobs = {}, 0, []
    if metadata:
        headers["__metadata__"] = metadata
    for k, v in tensors.items():
        if isinstance(v, tuple):
            arr, dt = np.ascontiguousarray(v[0]), v[1]
        else:
            arr = np.ascontiguousarray(v)
            dt = {np.dtype(t): d for d, (t, _) in _STORE.items()
                  if d not in (DT_BF16, DT_FP8E4M3, DT_FP8E5M2)}[arr.dtype]
        raw = arr.tobytes()
        headers[k] = {"dtype": _SAFE_TAGS[dt], "shape": list(arr.shape),
                      "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    j = json.dumps(headers, separators=(",", ":"))
    j += " " * ((len(j) + 7) // 8 * 8 - len(j))
    with open(fn, "wb") as f:
        f.write(len(j).to_bytes(8, "little"))
        f.write(j.encode("utf-8"))
        for b in blobs:
            f.write(b)


# ------------------------------------------------------------- torch_load --
_TORCH_STORAGE = {"FloatStorage": (np.float32, 4, False), "DoubleStorage": (np.float64, 8, False),
                  "HalfStorage": (np.float16, 2, False), "BFloat16Storage": (np.uint16, 2, True),
                  "LongStorage": (np.int64, 8, False), "IntStorage": (np.int32, 4, False),
                  "ShortStorage": (np.int16, 2, False), "CharStorage": (np.int8, 1, False),
                  "ByteStorage": (np.uint8, 1, False), "BoolStorage": (np.bool_, 1, False)}


class _Storage:
    """A placeholder for a torch storage class named in the pickle."""

    def __init__(self, name):
        self.name = name


def torch_load(path) -> Dict[str, np.ndarray]:
    """The tensors of a PyTorch checkpoint (zip or legacy format) as numpy
    arrays, bf16 widened to f32 (py/thvm/nn_state.py:112-220).  The pickle is
    read by a restricted unpickler: only the tensor-rebuild functions,
    OrderedDict and the storage type names resolve; any other global raises
    pickle.UnpicklingError, so a checkpoint cannot run code."""
    raw = open(path, "rb").read()
    data: Dict[str, bytes] = {}
    sizes: Dict[str, int] = {}

    def rebuild(storage, storage_offset, size, stride, *_):
        st, key, numel = storage[1], storage[2], storage[4]   # ('storage', type, key, location, numel, ...)
        npdt, isz, bf = _TORCH_STORAGE[st.name]
        sizes[key] = numel * isz
        if key not in data:
            return None
        size, stride = tuple(int(s) for s in size), tuple(int(s) for s in stride)
        storage_offset, numel = int(storage_offset), int(numel)
        if len(size) != len(stride) or any(s < 0 for s in size) or numel < 0:
            raise ValueError(f"torch_load: tensor view of storage {key!r} has a bad shape "
                             f"{size} / stride {stride}")
        n = int(np.prod(size)) if len(size) else 1
        if len(data[key]) < numel * isz:
            raise ValueError(f"torch_load: storage {key!r} holds {len(data[key])} bytes, "
                             f"the pickle says {numel} x {isz}")
        if n > 0:
            last = storage_offset + sum((s - 1) * st for s, st in zip(size, stride))
            if storage_offset < 0 or any(st < 0 for st in stride) or last >= numel:
                raise ValueError(f"torch_load: tensor view (offset {storage_offset}, size {size}, "
                                 f"stride {stride}) lies outside its storage of {numel} elements")
        flat = np.frombuffer(data[key], dtype=npdt, count=numel)
        if bf:
            flat = bf16_to_f32(flat)
        if n == 0:
            return np.zeros(size, flat.dtype)
        st_b = flat.itemsize
        view = np.lib.stride_tricks.as_strided(flat[storage_offset:], shape=tuple(size),
                                               strides=tuple(s * st_b for s in stride))
        return np.array(view)

    class Param:
        def __setstate__(self, state):
            self.tensor = state[0]

    allowed = {("torch._utils", "_rebuild_tensor_v2"): rebuild,
               ("torch._utils", "_rebuild_tensor"): rebuild,
               ("torch._utils", "_rebuild_parameter"): (lambda t, *_: t),
               ("torch.nn.parameter", "Parameter"): Param,
               ("collections", "OrderedDict"): __import__("collections").OrderedDict}

    class Restricted(pickle.Unpickler):
        def find_class(self, module, name):
            if (module, name) in allowed:
                return allowed[(module, name)]
            if module == "torch" and name in _TORCH_STORAGE:
                return _Storage(name)
            raise pickle.UnpicklingError(f"torch_load: refusing global {module}.{name}")

        def persistent_load(self, pid):
            return pid

    def tensors(d):
        out = {}
        for k, v in d.items():
            if isinstance(v, Param):
                v = v.tensor
            if isinstance(v, np.ndarray):
                out[k] = v
        return out

    if zipfile.is_zipfile(io.BytesIO(raw)):
        with zipfile.ZipFile(io.BytesIO(raw)) as zf:
            names = zf.namelist()
            pkl = next(n for n in names if n.endswith("data.pkl"))
            root = pkl.rsplit("/", 1)[0]
            for n in names:
                if n.startswith(root + "/data/"):
                    data[n.rsplit("/", 1)[1]] = zf.read(n)
            return tensors(Restricted(io.BytesIO(zf.read(pkl))).load())
    # legacy: magic, protocol, sys info, the state pickle, the storage keys,
    # then each storage as an 8-byte element count and its bytes
    f = io.BytesIO(raw)
    up = Restricted(f)
    for _ in range(3):
        up.load()
    rewind = f.tell()
    up.load()                       # records the storage sizes
    keys = up.load()
    pos = f.tell()
    for k in keys:
        pos += 8
        data[k] = raw[pos:pos + sizes[k]]
        pos += sizes[k]
    f.seek(rewind)
    return tensors(Restricted(f).load())


# ------------------------------------------------------------- DSV2PK01 ----
_PACK_ENT = struct.Struct("<48sIIQQ")


def dsv2pk_load(fn) -> Dict[str, DiskTensor]:
    """The DSV2PK01 weight pack (bench/dsv2_decode_bench.c:229-310): "DSV2PK01",
    u64 count, count x {name[48], u32 dtype (0 bf16, 1 f32), u32 pad, u64
    offset, u64 nbytes}, payloads in the reference kernels' layouts.  Shapes
    are not stored: each entry is a flat disk tensor."""
    with open(fn, "rb") as f:
        if f.read(8) != b"DSV2PK01":
            raise ValueError(f"{fn}: not a DSV2PK01 pack")
        n = int.from_bytes(f.read(8), "little")
        tab = f.read(n * _PACK_ENT.size)
    size = os.path.getsize(fn)
    out = {}
    for i in range(n):
        name, dt, _, off, nb = _PACK_ENT.unpack_from(tab, i * _PACK_ENT.size)
        name = name.split(b"\0", 1)[0].decode()
        if dt not in (0, 1) or off + nb > size:
            raise ValueError(f"{fn}: bad entry {name}")
        d = DT_BF16 if dt == 0 else DT_FP32
        out[name] = DiskTensor(str(fn), off, nb, d, (nb // (2 if dt == 0 else 4),))
    return out


# ------------------------------------------------------------------ GGUF ---
GGUF_F32, GGUF_F16, GGUF_Q4_0, GGUF_Q8_0, GGUF_BF16 = 0, 1, 2, 8, 30
# (block elements, block bytes) of the block-quantised types read here
_GGUF_BLOCK = {GGUF_Q4_0: (32, 18), GGUF_Q8_0: (32, 34)}
_GGUF_PLAIN = {GGUF_F32: DT_FP32, GGUF_F16: DT_FP16, GGUF_BF16: DT_BF16}


def _gguf_value(f, t):
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
           11: "<q", 12: "<d"}
    if t in fmt:
        s = struct.Struct(fmt[t])
        return s.unpack(f.read(s.size))[0]
    if t == 8:
        n = struct.unpack("<Q", f.read(8))[0]
        return f.read(n).decode("utf-8", "replace")
    if t == 9:
        et, n = struct.unpack("<IQ", f.read(12))
        return [_gguf_value(f, et) for _ in range(n)]
    raise ValueError(f"gguf: value type {t}")


def gguf_load(fn):
    """(metadata, {name: array}) of a GGUF v2/v3 file.  F32 / F16 / BF16
    tensors come back as disk tensors; Q8_0 (blocks of 32: f16 scale d, 32
    int8 q, x = d q) and Q4_0 (f16 d, 16 bytes of nibbles, low nibbles first:
    x = d (q - 8)) are dequantised to f32 arrays.  Other types raise
    NotImplementedError, as the reference's gguf_load does for all."""
    with open(fn, "rb") as f:
        if f.read(4) != b"GGUF":
            raise ValueError(f"{fn}: not a GGUF file")
        ver, nt, nkv = struct.unpack("<IQQ", f.read(20))
        if ver not in (2, 3):
            raise ValueError(f"{fn}: GGUF version {ver}")
        meta = {}
        for _ in range(nkv):
            kl = struct.unpack("<Q", f.read(8))[0]
            k = f.read(kl).decode()
            meta[k] = _gguf_value(f, struct.unpack("<I", f.read(4))[0])
        infos = []
        for _ in range(nt):
            nl = struct.unpack("<Q", f.read(8))[0]
            name = f.read(nl).decode()
            nd = struct.unpack("<I", f.read(4))[0]
            dims = struct.unpack(f"<{nd}Q", f.read(8 * nd))
            t, off = struct.unpack("<IQ", f.read(12))
            infos.append((name, tuple(reversed(dims)), t, off))   # ne[0] is the fastest dim
        align = int(meta.get("general.alignment", 32))
        base = (f.tell() + align - 1) // align * align
    out = {}
    for name, shape, t, off in infos:
        n = int(np.prod(shape)) if shape else 1
        if t in _GGUF_PLAIN:
            dt = _GGUF_PLAIN[t]
            out[name] = DiskTensor(str(fn), base + off, n * _STORE[dt][1], dt, shape)
        elif t in _GGUF_BLOCK:
            be, bb = _GGUF_BLOCK[t]
            if n % be:
                raise ValueError(f"{fn}: {name} has {n} elements, not whole blocks of {be}")
            blk = np.memmap(fn, np.uint8, "r", offset=base + off, shape=(n // be, bb))
            d = blk[:, :2].copy().view(np.float16).astype(np.float32)
            if t == GGUF_Q8_0:
                q = blk[:, 2:].view(np.int8).astype(np.float32)
            else:
                nib = blk[:, 2:]
                q = np.concatenate([nib & 15, nib >> 4], 1).astype(np.float32) - 8.0
            out[name] = (d * q).reshape(shape)
        else:
            raise NotImplementedError(f"gguf: tensor {name} has ggml type {t} (F32, F16, BF16, "
                                      f"Q8_0 and Q4_0 are read)")
    return meta, out


# ------------------------------------------------- decoder loading ---------
def _f32(t) -> np.ndarray:
    if isinstance(t, DiskTensor):
        return t.float32()
    a = np.asarray(t)
    return a.astype(np.float32) if a.dtype != np.float32 else a


def write_weight(dec, name: str, w: np.ndarray) -> None:
    """Write a [rows, cols] float matrix into decoder tensor `name` in the
    decoder's weight dtype; fp8 decoders quantise on the device (per-row
    absmax/448 e4m3 and the `name.scale` vector)."""
    import thvm_amd as T
    w = np.ascontiguousarray(w, np.float32)
    _, dt, nb = dec.tensor(name)
    if dt == DT_FP8E4M3:
        rows, cols = w.shape
        if rows * cols != nb:
            raise ValueError(f"{name}: {rows}x{cols} weights, the tensor holds {nb}")
        src = T.Buffer.from_numpy(w)          # f32: the checkpoint's values, exactly
        try:
            sid, _, _ = dec.tensor(name + ".scale")
            T.builtin("quant_fp8", [dec.tensor(name)[0], sid, src], outs=(0, 1), rows=rows,
                      cols=cols, xt=DT_FP32)
        finally:
            src.free()
        dec.sync_weights(name)
        return
    if dt == DT_FP32:
        dec.write_tensor(name, w)
    elif dt == DT_BF16:
        dec.write_tensor(name, f32_to_bf16(w))
    elif dt == DT_FP16:
        dec.write_tensor(name, w.astype(np.float16).view(np.uint16))
    else:
        raise ValueError(f"{name}: decoder dtype {dt}")


def write_vector(dec, name: str, v: np.ndarray) -> None:
    """A norm gain / bias / table in the decoder tensor's own dtype."""
    v = np.ascontiguousarray(v, np.float32)
    _, dt, _ = dec.tensor(name)
    if dt == DT_FP32:
        dec.write_tensor(name, v)
    elif dt == DT_BF16:
        dec.write_tensor(name, f32_to_bf16(v))
    elif dt == DT_FP16:
        dec.write_tensor(name, v.astype(np.float16).view(np.uint16))
    else:
        raise ValueError(f"{name}: dtype {dt}")


def hf_rope_rows_to_interleaved(w: np.ndarray, n_heads: int) -> np.ndarray:
    """Hugging Face Llama checkpoints order each head's q/k rows for the
    rotate-half RoPE (pair j = rows j and j + hd/2); the decoder rotates
    adjacent rows (2j, 2j + 1).  Row 2j takes HF row j, row 2j+1 HF row
    j + hd/2."""
    rows, cols = w.shape
    hd = rows // n_heads
    return np.ascontiguousarray(
        w.reshape(n_heads, 2, hd // 2, cols).transpose(0, 2, 1, 3).reshape(rows, cols))


def load_llama(dec, sd: Dict[str, object], hf_rope_order: bool = True) -> None:
    """A Llama state dict with Hugging Face names (model.embed_tokens.weight,
    model.layers.<i>.self_attn.{q,k,v,o}_proj.weight, mlp.{gate,up,down}_proj.
    weight, input_layernorm.weight, post_attention_layernorm.weight,
    model.norm.weight, lm_head.weight) into an arch-LLAMA decoder."""
    c = dec.cfg
    H, Hkv = c.n_heads, c.n_kv_heads
    g = lambda k: _f32(sd[k])  # noqa: E731
    write_vector(dec, "emb", g("model.embed_tokens.weight").reshape(-1))
    for l in range(c.n_layers):
        p = f"model.layers.{l}."
        q, k, v = g(p + "self_attn.q_proj.weight"), g(p + "self_attn.k_proj.weight"), g(p + "self_attn.v_proj.weight")
        if hf_rope_order:
            q, k = hf_rope_rows_to_interleaved(q, H), hf_rope_rows_to_interleaved(k, Hkv)
        write_weight(dec, f"l{l}.wqkv", np.concatenate([q, k, v]))
        write_weight(dec, f"l{l}.wo", g(p + "self_attn.o_proj.weight"))
        gate, upw = g(p + "mlp.gate_proj.weight"), g(p + "mlp.up_proj.weight")
        gu = np.empty((2 * gate.shape[0], gate.shape[1]), np.float32)
        gu[0::2], gu[1::2] = gate, upw
        write_weight(dec, f"l{l}.wgu", gu)
        write_weight(dec, f"l{l}.wd", g(p + "mlp.down_proj.weight"))
        write_vector(dec, f"l{l}.g_attn", g(p + "input_layernorm.weight"))
        write_vector(dec, f"l{l}.g_ffn", g(p + "post_attention_layernorm.weight"))
    write_vector(dec, "norm_f", g("model.norm.weight"))
    lm = sd.get("lm_head.weight", sd["model.embed_tokens.weight"])
    write_weight(dec, "lm", _f32(lm))


def load_gpt2(dec, sd: Dict[str, object]) -> None:
    """A GPT-2 state dict with Hugging Face names (transformer.wte/wpe.weight,
    transformer.h.<i>.{ln_1,ln_2}.{weight,bias}, attn.c_attn, attn.c_proj,
    mlp.c_fc, mlp.c_proj .{weight,bias} stored [in, out] (Conv1D),
    transformer.ln_f) into an arch-GPT2 decoder (tied LM head)."""
    c = dec.cfg
    g = lambda k: _f32(sd[k if k in sd else "transformer." + k])  # noqa: E731
    write_weight(dec, "wte", g("wte.weight"))
    wpe = g("wpe.weight")
    _, dt, nb = dec.tensor("wpe")
    rows = nb // (wpe.shape[1] * _STORE[dt][1])
    if rows > wpe.shape[0]:
        raise ValueError(f"wpe: the decoder holds {rows} positions, the checkpoint {wpe.shape[0]}")
    write_weight(dec, "wpe", wpe[:rows])
    for l in range(c.n_layers):
        p = f"h.{l}."
        for src, dst in (("attn.c_attn", "c_attn"), ("attn.c_proj", "c_proj"), ("mlp.c_fc", "c_fc"),
                         ("mlp.c_proj", "mlp_proj")):
            write_weight(dec, f"l{l}.{dst}", g(p + src + ".weight").T)
            write_vector(dec, f"l{l}.{dst}.b", g(p + src + ".bias"))
        for n in ("ln_1", "ln_2"):
            d = "ln1" if n == "ln_1" else "ln2"
            write_vector(dec, f"l{l}.{d}.g", g(p + n + ".weight"))
            write_vector(dec, f"l{l}.{d}.b", g(p + n + ".bias"))
    write_vector(dec, "lnf.g", g("ln_f.weight"))
    write_vector(dec, "lnf.b", g("ln_f.bias"))


def load_dsv2(dec, pack: Dict[str, DiskTensor]) -> None:
    """A DSV2PK01 pack (reference layouts: {in, out} projections, absorbed
    w_uk [h][dn][kv], stacked experts) into an arch-DSV2 decoder."""
    c = dec.cfg
    D, H, kv, dn, dr, dv = c.dim, c.n_heads, c.kv_lora, c.d_nope, c.d_rope, c.d_v
    E, I, S, F, V = c.n_experts, c.moe_inter, c.n_shared * c.moe_inter, c.ffn, c.vocab
    g = lambda k, *shape: _f32(pack[k]).reshape(shape)  # noqa: E731
    write_vector(dec, "emb", g("embed", V * D))
    write_vector(dec, "norm_f", g("norm", D))
    write_weight(dec, "lm", g("lm_head", D, V).T)
    nq = H * (dn + dr)
    for l in range(c.n_layers):
        p = f"l{l}."
        write_vector(dec, p + "win", g(p + "win", D))
        write_vector(dec, p + "wkvn", g(p + "wkvn", kv))
        write_vector(dec, p + "wpost", g(p + "wpost", D))
        write_weight(dec, p + "wqkv", np.concatenate([g(p + "wq", D, nq).T, g(p + "wkv", D, kv + dr).T]))
        write_weight(dec, p + "wuk", g(p + "wuk", H, dn, kv).transpose(0, 2, 1).reshape(H * kv, dn))
        write_weight(dec, p + "wuv", g(p + "wuv", H * dv, kv))
        write_weight(dec, p + "wo", g(p + "wo", H * dv, D).T)
        if l < c.first_dense:
            gu = np.empty((2 * F, D), np.float32)
            gu[0::2], gu[1::2] = g(p + "wg1", D, F).T, g(p + "wu1", D, F).T
            write_weight(dec, p + "wgu", gu)
            write_weight(dec, p + "wd", g(p + "wd1", F, D).T)
            continue
        write_vector(dec, p + "gate", g(p + "gate", D, E).T.reshape(-1))
        gu = np.empty((E, 2 * I, D), np.float32)
        gu[:, 0::2], gu[:, 1::2] = g(p + "wg", E, I, D), g(p + "wu", E, I, D)
        write_weight(dec, p + "wgu_e", gu.reshape(E * 2 * I, D))
        write_weight(dec, p + "wd_e", g(p + "wd", E * D, I))
        if S:
            gs = np.empty((2 * S, D), np.float32)
            gs[0::2], gs[1::2] = g(p + "swg", S, D), g(p + "swu", S, D)
            write_weight(dec, p + "wgu_s", gs)
            write_weight(dec, p + "wd_s", g(p + "swd", D, S))
