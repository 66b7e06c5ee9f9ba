"""thvm_amd -- Python host for the MI355X (gfx950) ``DEV=hip`` device.

A thin ctypes layer over ``libthvm_hip.so`` (C-ABI declared in
``include/thvm_hip.h``).  It mirrors the reference's Python host surface for
the decode path (reference ``py/thvm/device.py:28-41`` ``Device`` from
``DEV``, ``py/csource/thvm_py.c:95-130`` tensor create/read/write, ``:407-420``
the JIT entry points): device buffers from and to numpy, custom-kernel
dispatch, JIT capture/replay, and the synthetic decode drivers.

There is no CPU fallback: every call goes to the HIP library, and importing
the library fails loudly when it has not been built
(``python -m thvm_amd.build``)."""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Optional

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "lib" / "libthvm_hip.so"


def _lib_path() -> Path:
    """The library lib() loads: the product build, or with
    THVM_HIP_LIB_VARIANT=pclk (read at the first load) the measurement build
    whose kernels carry phase-clock marks."""
    v = os.environ.get("THVM_HIP_LIB_VARIANT")
    return LIB_PATH.with_name(f"libthvm_hip_{v}.so") if v else LIB_PATH

# dtype ids (reference src/thvm.h:254-271)
DT = dict(bool=0, int8=1, uint8=2, int16=3, uint16=4, int32=5, uint32=6, int64=7, uint64=8,
          fp8e4m3=9, fp8e5m2=10, fp16=11, bf16=12, fp32=13, fp64=14)
DT_FP8E4M3, DT_FP16, DT_BF16, DT_FP32, DT_INT32 = 9, 11, 12, 13, 5
ARCH = dict(llama=1, gpt2=2, dsv2=3)
EPI = dict(store=0, resid=1, swiglu=2, gelu=3, qkv_rope=4, qkv=5)

_NP_OF_DT = {DT_FP32: np.float32, DT_FP16: np.uint16, DT_BF16: np.uint16,
             DT_FP8E4M3: np.uint8, DT_INT32: np.int32, 2: np.uint8}


class ThvmHipError(RuntimeError):
    pass


class DecodeConfig(C.Structure):
    """ThvmDecodeConfig (include/thvm_hip.h)."""
    _fields_ = [(n, C.c_uint32) for n in (
        "arch", "n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
        "max_seq", "batch", "wdtype", "adtype")] + [
        ("eps", C.c_float), ("rope_theta", C.c_float), ("init_std", C.c_float)] + [
        (n, C.c_uint32) for n in ("kv_lora", "d_nope", "d_rope", "d_v", "n_experts",
                                  "n_shared", "top_k", "moe_inter", "first_dense", "step_mode",
                                  "moe_mode", "attn_cpb")] + [
        ("temperature", C.c_float), ("sample_seed_lo", C.c_uint32), ("sample_seed_hi", C.c_uint32),
        ("spec_rows", C.c_uint32), ("spec_forced", C.c_uint32), ("attn_fused", C.c_uint32),
        ("attn_mf", C.c_uint32)]


class Uop(C.Structure):
    """ThvmUop (include/thvm_hip.h): one node of a kernel's lifted DAG."""
    _fields_ = [("op", C.c_uint32), ("dtype", C.c_uint32), ("src", C.c_int32 * 4),
                ("arg", C.c_int64 * 4)]


class RenderInfo(C.Structure):
    """ThvmRenderInfo (include/thvm_hip.h)."""
    _fields_ = [("n_slots", C.c_uint32), ("kvar_slot", C.c_uint32), ("group", C.c_uint32),
                ("block", C.c_uint32), ("grid_max", C.c_uint64), ("upcast", C.c_uint32),
                ("reserved", C.c_uint32)]


class RenderOpts(C.Structure):
    """ThvmRenderOpts (include/thvm_hip.h): block, group, upcast."""
    _fields_ = [("block", C.c_uint32), ("group", C.c_uint32), ("upcast", C.c_uint32),
                ("reserved", C.c_uint32)]


_u32, _u64, _i32, _vp, _cp, _d = C.c_uint32, C.c_uint64, C.c_int, C.c_void_p, C.c_char_p, C.c_double
_SIGS = {
    "thvm_hip_init": (_i32, []), "thvm_hip_shutdown": (None, []),
    "thvm_hip_available": (_i32, []), "thvm_hip_last_error": (_cp, []),
    "thvm_hip_version": (_cp, []),
    "thvm_hip_buf_alloc": (_u32, [_u64]), "thvm_hip_buf_free": (None, [_u32]),
    "thvm_hip_buf_incref": (None, [_u32]), "thvm_hip_buf_decref": (None, [_u32]),
    "thvm_hip_buf_jit_pin": (None, [_u32]), "thvm_hip_buf_jit_unpin": (None, [_u32]),
    "thvm_hip_buf_read": (_i32, [_u32, _vp, _u64]), "thvm_hip_buf_write": (_i32, [_u32, _vp, _u64]),
    "thvm_hip_buf_copy": (_i32, [_u32, _u32, _u64]),
    "thvm_hip_buf_write_at": (_i32, [_u32, _u64, _vp, _u64]),
    "thvm_hip_buf_copy_at": (_i32, [_u32, _u64, _u32, _u64]),
    "thvm_hip_buf_copy_row": (_i32, [_u32, _u64, _u64, _u32, _u64, _u32, _u64]),
    "thvm_hip_buf_load_file": (_i32, [_u32, _u64, _cp, _u64, _u64]),
    "thvm_hip_buf_refcount": (_u32, [_u32]), "thvm_hip_buf_freelist_push": (None, [_u32]),
    "thvm_hip_buf_freelist_remove": (None, [_u32]), "thvm_hip_buf_storage_root": (_u32, [_u32]),
    "thvm_hip_buf_nbytes": (_u64, [_u32]), "thvm_hip_buf_zero": (None, [_u32]),
    "thvm_hip_buf_view": (_u32, [_u32, _u64, _u64]), "thvm_hip_buf_device_ptr": (_u64, [_u32]),
    "thvm_hip_mem_live_bytes": (_u64, []), "thvm_hip_mem_peak_bytes": (_u64, []),
    "thvm_hip_buf_pool_begin": (_u32, []),
    "thvm_hip_buf_pool_rollback_with_preserve": (None, [_u32]),
    "thvm_hip_buf_pool_free_unpreserved": (None, [_u32]),
    "thvm_hip_buf_mark_preserved": (None, [_u32]), "thvm_hip_buf_clear_preserved": (None, [_u32]),
    "thvm_hip_buf_clear_preserved_arena_views": (None, [_u32]),
    "thvm_hip_buf_free_unpreserved_all": (_u64, []), "thvm_hip_buf_arena_alloc": (_u32, [_u64]),
    "thvm_hip_buf_slots_used": (_u32, []), "thvm_hip_buf_slot_highwater": (_u32, []),
    "thvm_hip_dispatch_begin": (None, []), "thvm_hip_dispatch_flush": (None, []),
    "thvm_hip_dispatch_end": (None, []),
    "thvm_hip_dispatch_custom": (_i32, [_cp, _cp, _vp, _vp, _u32, _vp, _u32, _u64]),
    "thvm_hip_program_check": (_i32, [_cp, _cp]),
    "thvm_hip_attn_decode_noalloc": (_i32, [_cp, _vp, _u32]),
    "thvm_hip_render_kernel": (_i32, [C.POINTER(Uop), _u32, _cp, _vp, _u64, C.POINTER(RenderInfo)]),
    "thvm_hip_render_kernel_opts": (_i32, [C.POINTER(Uop), _u32, _cp, C.POINTER(RenderOpts), _vp, _u64,
                                           C.POINTER(RenderInfo)]),
    "thvm_hip_render_autotune": (_i32, [C.POINTER(Uop), _u32, _vp, _u32, _u32, C.POINTER(RenderOpts),
                                        C.POINTER(_d), C.POINTER(_d)]),
    "thvm_hip_jit_capture_begin": (_u32, []), "thvm_hip_jit_capture_end": (None, []),
    "thvm_hip_jit_capture_op_count": (_u32, [_u32]), "thvm_hip_jit_replay": (_i32, [_u32]),
    "thvm_hip_jit_rebind": (_i32, [_u32, _vp, _vp, _u32]),
    "thvm_hip_jit_capture_drop": (None, [_u32]), "thvm_hip_jit_is_capturing": (_i32, []),
    "thvm_hip_graph_replay": (_i32, [_u32]), "thvm_hip_graph_capture_begin": (_i32, []),
    "thvm_hip_graph_capture_end_and_launch": (_i32, [_u32]),
    "thvm_hip_graph_invalidate": (None, [_u32]),
    "thvm_hip_timer_start": (_u32, []), "thvm_hip_timer_stop": (_d, [_u32]),
    "thvm_hip_kprof_enable": (None, [_i32]), "thvm_hip_kprof_reset": (None, []),
    "thvm_hip_kprof_query": (_d, [_cp, C.POINTER(_u64)]),
    "thvm_hip_kprof_bytes": (_u64, [_cp]),
    "thvm_hip_decoder_create": (_u32, [C.POINTER(DecodeConfig), _u64]),
    "thvm_hip_decoder_destroy": (None, [_u32]),
    "thvm_hip_decoder_generate": (_i32, [_u32, _vp, _u32, _u32, C.c_int32, _vp, _vp]),
    "thvm_hip_decoder_serve": (_i32, [_u32, _i32, _i32, C.c_int32, _u32]),
    "thvm_hip_decoder_prefill_synthetic": (_i32, [_u32, _u32, _u64]),
    "thvm_hip_decoder_set_state": (_i32, [_u32, _vp, _u32]),
    "thvm_hip_decoder_step": (_i32, [_u32]), "thvm_hip_decoder_capture": (_u32, [_u32]),
    "thvm_hip_decoder_replay": (_i32, [_u32, _u32]),
    "thvm_hip_decoder_spec_step": (_i32, [_u32]), "thvm_hip_decoder_spec_capture": (_u32, [_u32]),
    "thvm_hip_decoder_spec_replay": (_i32, [_u32, _u32]),
    "thvm_hip_decoder_read_tokens": (_i32, [_u32, _vp, _u32]),
    "thvm_hip_decoder_read_logits": (_i32, [_u32, _vp, _u64]),
    "thvm_hip_decoder_position": (_u32, [_u32]),
    "thvm_hip_decoder_tensor": (_u32, [_u32, _cp, C.POINTER(_u32), C.POINTER(_u64)]),
    "thvm_hip_decoder_sync_weights": (_i32, [_u32, _cp]),
    "thvm_hip_decoder_step_bytes": (_u64, [_u32]),
    "thvm_hip_decoder_step_kernels": (_u32, [_u32]),
    "thvm_hip_decoder_stage_clock": (C.c_int, [_u32, C.c_void_p, _u32]),
    "thvm_hip_decoder_op_tags": (C.c_int, [_u32, C.c_void_p, _u32]),
    "thvm_hip_decoder_run_ops": (_i32, [_u32, _u32, _u32]),
    "thvm_hip_decoder_op_info": (_i32, [_u32, _u32, _cp, _u32, _cp, _u32, _vp, _u32]),
}

_LIB = None


def lib() -> C.CDLL:
    """The loaded libthvm_hip.so with argument types bound.  Raises when the
    library has not been built: there is no fallback path."""
    global _LIB
    if _LIB is None:
        path = _lib_path()
        if not path.exists():
            raise ThvmHipError(f"{path} not built: run `python -m thvm_amd.build`")
        L = C.CDLL(str(path))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


def exported_symbols() -> list[str]:
    return list(_SIGS)


def last_error() -> str:
    return lib().thvm_hip_last_error().decode(errors="replace")


def _check(rc, what: str):
    if rc != 0:
        raise ThvmHipError(f"{what}: {last_error()}")


def init() -> None:
    """Start the HIP device (reference Device canonicalisation: one device,
    index 0 only, py/thvm/device.py:29-35)."""
    _check(lib().thvm_hip_init(), "thvm_hip_init")


def shutdown() -> None:
    lib().thvm_hip_shutdown()


def synchronize() -> None:
    lib().thvm_hip_dispatch_end()


class Buffer:
    """A device buffer id with numpy upload/download (py_ten_create /
    py_ten_read / py_ten_write, reference py/csource/thvm_py.c:95-130)."""

    def __init__(self, nbytes: int):
        self.id = lib().thvm_hip_buf_alloc(int(nbytes))
        if self.id == 0:
            raise ThvmHipError(f"buf_alloc({nbytes}): {last_error()}")
        self.nbytes = int(nbytes)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.write(a)
        return b

    def write(self, a: np.ndarray, byte_off: int = 0) -> None:
        a = np.ascontiguousarray(a)
        _check(lib().thvm_hip_buf_write_at(self.id, byte_off, a.ctypes.data, a.nbytes), "buf_write")

    def read(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(n, dtype)
        _check(lib().thvm_hip_buf_read(self.id, out.ctypes.data, out.nbytes), "buf_read")
        return out

    def free(self) -> None:
        if self.id:
            lib().thvm_hip_buf_free(self.id)
            self.id = 0


def _u32arr(vals):
    return (C.c_uint32 * len(vals))(*[int(v) for v in vals])


def dispatch(name: str, program: str, args, grid=(1, 1, 1), block=(1, 1, 1), shared: int = 0,
             outs=(0,)) -> None:
    """Fire a custom program (kernel_emit_custom_program + kernel_custom_fire,
    reference src/schedule/kernel_custom.c:47-218).  `args` are Buffers or ids."""
    ids = [a.id if isinstance(a, Buffer) else int(a) for a in args]
    mask = 0
    for s in outs:
        mask |= 1 << int(s)
    _check(lib().thvm_hip_dispatch_custom(name.encode(), program.encode(), _u32arr(grid),
                                          _u32arr(block), shared, _u32arr(ids), len(ids), mask),
           f"dispatch {name}")


def builtin(kernel: str, args, outs=(0,), **params) -> None:
    """Fire a built-in gfx950 kernel: program "thvm-builtin:<kernel> k=v ..."."""
    toks = [f"{k}={float(v).hex() if isinstance(v, float) else int(v)}" for k, v in params.items()]
    dispatch(kernel, "thvm-builtin:" + kernel + (" " + " ".join(toks) if toks else ""), args,
             outs=outs)


class Jit:
    """The capture/replay API (reference src/jit/capture.c:644-745, 2687-2884)."""

    def __init__(self):
        self.slot = 0

    def __enter__(self):
        self.slot = lib().thvm_hip_jit_capture_begin()
        if self.slot == 0:
            raise ThvmHipError(f"jit_capture_begin: {last_error()}")
        return self

    def __exit__(self, exc_type, exc, tb):
        lib().thvm_hip_jit_capture_end()
        if exc_type is not None:      # a failed capture leaves no slot behind
            self.drop()
        return False

    def op_count(self) -> int:
        return lib().thvm_hip_jit_capture_op_count(self.slot)

    def replay(self) -> None:
        _check(lib().thvm_hip_jit_replay(self.slot), "jit_replay")

    def drop(self) -> None:
        if self.slot:
            lib().thvm_hip_jit_capture_drop(self.slot)
            self.slot = 0


class Decoder:
    """Synthetic random-init decoder driven by one captured decode step."""

    def __init__(self, seed: int = 0, **cfg):
        c = DecodeConfig()
        for k, v in cfg.items():
            setattr(c, k, v)
        self.cfg = c
        self.h = lib().thvm_hip_decoder_create(C.byref(c), seed)
        if self.h == 0:
            raise ThvmHipError(f"decoder_create: {last_error()}")

    def tensor(self, name: str) -> tuple[int, int, int]:
        dt, nb = C.c_uint32(), C.c_uint64()
        bid = lib().thvm_hip_decoder_tensor(self.h, name.encode(), C.byref(dt), C.byref(nb))
        if bid == 0:
            raise ThvmHipError(last_error())
        return bid, dt.value, nb.value

    def read_tensor(self, name: str) -> np.ndarray:
        bid, dt, nb = self.tensor(name)
        npdt = np.dtype(_NP_OF_DT.get(dt, np.uint8))
        out = np.empty(nb // npdt.itemsize, npdt)
        _check(lib().thvm_hip_buf_read(bid, out.ctypes.data, out.nbytes), "buf_read")
        return out

    def write_tensor(self, name: str, a: np.ndarray) -> None:
        bid, _, nb = self.tensor(name)
        a = np.ascontiguousarray(a)
        if a.nbytes != nb:
            raise ThvmHipError(f"write_tensor {name}: {a.nbytes} bytes, tensor holds {nb}")
        _check(lib().thvm_hip_buf_write(bid, a.ctypes.data, a.nbytes), "buf_write")
        self.sync_weights(name)

    def sync_weights(self, name: Optional[str] = None) -> None:
        """Refresh the MFMA GEMM's tiled copy of a weight written through its
        buffer (decoders above 4 rows; every weight when name is None)."""
        _check(lib().thvm_hip_decoder_sync_weights(self.h, name.encode() if name else None),
               "decoder_sync_weights")

    def set_state(self, tokens, pos: int) -> None:
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        _check(lib().thvm_hip_decoder_set_state(self.h, t.ctypes.data, pos), "set_state")

    def prefill_synthetic(self, ctx: int, seed: int = 1) -> None:
        _check(lib().thvm_hip_decoder_prefill_synthetic(self.h, ctx, seed), "prefill")

    def step(self) -> None:
        _check(lib().thvm_hip_decoder_step(self.h), "decoder_step")

    def capture(self) -> int:
        s = lib().thvm_hip_decoder_capture(self.h)
        if s == 0:
            raise ThvmHipError(f"decoder_capture: {last_error()}")
        return s

    def replay(self, n: int = 1) -> None:
        _check(lib().thvm_hip_decoder_replay(self.h, n), "decoder_replay")

    def spec_step(self) -> None:
        """One eager speculative step (draft, verify, commit)."""
        _check(lib().thvm_hip_decoder_spec_step(self.h), "decoder_spec_step")

    def spec_capture(self) -> int:
        s = lib().thvm_hip_decoder_spec_capture(self.h)
        if s == 0:
            raise ThvmHipError(f"decoder_spec_capture: {last_error()}")
        return s

    def spec_replay(self, n: int = 1) -> None:
        _check(lib().thvm_hip_decoder_spec_replay(self.h, n), "decoder_spec_replay")

    def generate(self, prompts, max_new: int, eos: int = -1):
        """prompts [batch][n] (or [n] for every row) -> (ids [batch][max_new]
        with -1 after a row stops, counts [batch])."""
        B = self.cfg.batch
        p = np.asarray(prompts, np.int32)
        if p.ndim == 1:
            p = np.tile(p, (B, 1))
        p = np.ascontiguousarray(p)
        out = np.empty((B, max_new), np.int32)
        n = np.empty(B, np.uint32)
        _check(lib().thvm_hip_decoder_generate(self.h, p.ctypes.data, p.shape[1], max_new, eos,
                                               out.ctypes.data, n.ctypes.data), "generate")
        return out, n.astype(np.int64)

    def serve(self, in_fd: int, out_fd: int, eos: int = -1, default_max_new: int = 256) -> None:
        _check(lib().thvm_hip_decoder_serve(self.h, in_fd, out_fd, eos, default_max_new), "serve")

    def tokens(self, n: int) -> np.ndarray:
        out = np.empty((self.cfg.batch, n), np.int32)
        _check(lib().thvm_hip_decoder_read_tokens(self.h, out.ctypes.data, n), "read_tokens")
        return out

    def logits(self) -> np.ndarray:
        out = np.empty((self.cfg.batch, self.cfg.vocab), np.float32)
        _check(lib().thvm_hip_decoder_read_logits(self.h, out.ctypes.data, out.size), "read_logits")
        return out

    @property
    def position(self) -> int:
        return lib().thvm_hip_decoder_position(self.h)

    def step_bytes(self) -> int:
        return lib().thvm_hip_decoder_step_bytes(self.h)

    def step_kernels(self) -> int:
        return lib().thvm_hip_decoder_step_kernels(self.h)

    def stage_clock(self) -> np.ndarray:
        """Persistent step only: microseconds after the last step's start at
        which each grid barrier opened and the step's end (5 L + 2 values),
        then per stage (5 L + 1) its entry, barrier open, work done and stores
        drained -- block 0's clock."""
        n = self.cfg.n_layers * 5 + 2 + 4 * (self.cfg.n_layers * 5 + 1)
        out = np.zeros(n, np.float64)
        got = lib().thvm_hip_decoder_stage_clock(self.h, out.ctypes.data, n)
        if got < 0:
            raise ThvmHipError(f"stage_clock: {last_error()}")
        return out[:got]

    def op_tags(self) -> np.ndarray:
        """The sublayer of each dispatch of the step: 2l (layer l's
        attention), 2l+1 (its FFN), -1 before the layers, -2 after."""
        n = lib().thvm_hip_decoder_op_tags(self.h, None, 0)
        if n < 0:
            raise ThvmHipError(f"op_tags: {last_error()}")
        out = np.empty(n, np.int32)
        if lib().thvm_hip_decoder_op_tags(self.h, out.ctypes.data, n) < 0:
            raise ThvmHipError(f"op_tags: {last_error()}")
        return out

    def op_info(self, i: int):
        """(name, program, buffer ids) of dispatch i of the step."""
        name, prog = C.create_string_buffer(64), C.create_string_buffer(1024)
        ids = np.zeros(32, np.uint32)
        n = lib().thvm_hip_decoder_op_info(self.h, i, name, 64, prog, 1024, ids.ctypes.data, 32)
        if n < 0:
            raise ThvmHipError(f"op_info: {last_error()}")
        return name.value.decode(), prog.value.decode(), [int(v) for v in ids[:n]]

    def run_ops(self, first: int, count: int) -> None:
        """Dispatch ops [first, first + count) of the step eagerly."""
        _check(lib().thvm_hip_decoder_run_ops(self.h, first, count), "run_ops")

    def step_probed(self, reads, on_boundary):
        """One eager step run a sublayer at a time.  After the embedding
        (tag -1) and after each sublayer t, `on_boundary(t, {name: array})`
        receives the tensors named in `reads(t)` as read from the device;
        the tail then runs (logits, argmax, length bump)."""
        tags = self.op_tags()
        i, n = 0, len(tags)
        while i < n and tags[i] != -2:
            j = i
            while j < n and tags[j] == tags[i]:
                j += 1
            self.run_ops(i, j - i)
            on_boundary(int(tags[i]), {k: self.read_tensor(k) for k in reads(int(tags[i]))})
            i = j
        self.run_ops(i, n - i)

    def close(self) -> None:
        if self.h:
            lib().thvm_hip_decoder_destroy(self.h)
            self.h = 0


def kprof(on: bool = True) -> None:
    lib().thvm_hip_kprof_enable(1 if on else 0)


def kprof_reset() -> None:
    lib().thvm_hip_kprof_reset()


def kprof_query(tag: str) -> tuple[float, int]:
    n = C.c_uint64()
    ms = lib().thvm_hip_kprof_query(tag.encode(), C.byref(n))
    return ms, n.value


def _uops(nodes):
    arr = (Uop * len(nodes))()
    for i, (op, dt, srcs, args) in enumerate(nodes):
        u = arr[i]
        u.op, u.dtype = op, dt
        for k in range(4):
            u.src[k] = srcs[k] if k < len(srcs) else -1
            u.arg[k] = args[k] if k < len(args) else 0
    return arr


def render_kernel(nodes, name: str, cap: int = 1 << 20, opts=None) -> tuple[str, RenderInfo]:
    """HIP source + launch geometry of one lifted-DAG kernel (the renderer
    target, reference src/codegen/render_uop.c:4964-5113).  `nodes` is a
    sequence of (op, dtype, (src..), (arg..)) in topological order; `opts`
    (block, group, upcast) overrides the hand-coded geometry."""
    arr = _uops(nodes)
    buf = C.create_string_buffer(cap)
    info = RenderInfo()
    if opts is None:
        rc = lib().thvm_hip_render_kernel(arr, len(nodes), name.encode(), buf, cap, C.byref(info))
    else:
        o = RenderOpts(*[int(v) for v in opts], 0)
        rc = lib().thvm_hip_render_kernel_opts(arr, len(nodes), name.encode(), C.byref(o), buf, cap,
                                               C.byref(info))
    _check(rc, "render_kernel")
    return buf.value.decode(), info


def render_autotune(nodes, args, reps: int = 20, beam: Optional[int] = None):
    """Device search of a kernel's (block, group, upcast) over its argument
    buffers (reference src/codegen/autotune.c): returns (opts, best_us,
    hand_coded_us); the output buffer holds the winner's result.  `beam`
    overrides the library's $BEAM width for this call."""
    arr = _uops(nodes)
    ids = _u32arr([a.id if isinstance(a, Buffer) else int(a) for a in args])
    best, bu, hu = RenderOpts(), C.c_double(), C.c_double()
    old = os.environ.get("BEAM")
    if beam is not None:
        os.environ["BEAM"] = str(int(beam))
    try:
        rc = lib().thvm_hip_render_autotune(arr, len(nodes), ids, len(args), reps, C.byref(best),
                                            C.byref(bu), C.byref(hu))
    finally:
        if beam is not None:
            if old is None:
                del os.environ["BEAM"]
            else:
                os.environ["BEAM"] = old
    _check(rc, "render_autotune")
    return (best.block, best.group, best.upcast), bu.value, hu.value


def kprof_bytes(tag: str) -> int:
    return int(lib().thvm_hip_kprof_bytes(tag.encode()))


def device_from_env() -> str:
    """`DEV` selection (reference src/thvm.c:638-645): this package serves hip."""
    dev = os.environ.get("DEV", "hip").split(":")[0].lower()
    if dev not in ("hip", "gpu", "amd"):
        raise ThvmHipError(f"DEV={dev}: this package is the hip device only")
    return "hip"
