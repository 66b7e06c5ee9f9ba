"""CPU tests of the renderer target (thvm_hip_render_kernel) and of the Tensor
host's kernel lowering.  Nothing here touches a device: the renderer is pure
host code, and the lowering tests give the host placeholder buffers and
capture the rendered kernels instead of dispatching them.  One rendered
source per case is compiled for gfx950 with hipcc to prove it is valid HIP."""
import shutil
import subprocess

import numpy as np
import pytest

import thvm_amd as hip

HIPCC = "/opt/rocm/bin/hipcc"

# reference op numbers (src/thvm.h)
CONST, ADD, MUL, EXP2, REDUCE, DEFINE_VAR, LOAD, CAST, RANGE, INDEX, IADD, IMUL = 2, 9, 10, 13, 17, 18, 21, 23, 25, 26, 27, 29
BUFFER, STORE = 36, 37
F32, I32 = 13, 5


def compile_ok(src: str, tmp_path) -> None:
    if not shutil.which(HIPCC):
        pytest.skip("hipcc not present")
    p = tmp_path / "k.hip"
    p.write_text("#include <hip/hip_runtime.h>\n" + src)
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "--cuda-device-only", "-c", str(p),
                        "-o", str(tmp_path / "k.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[:2000]


def row_sum_dag(n_rows, n_cols, symbolic=False):
    """out[r] = sum_c exp2(x[r, c]) * 2  (x row-major [rows, cols])."""
    nodes = []

    def add(op, dt, srcs=(), args=()):
        nodes.append((op, dt, tuple(srcs), tuple(args)))
        return len(nodes) - 1

    out = add(BUFFER, F32, (), (0, n_rows))
    x = add(BUFFER, F32, (), (1, n_rows * n_cols))
    r = add(RANGE, I32, (), (0, 5, n_rows))
    if symbolic:
        v = add(DEFINE_VAR, I32, (), (3, 1, n_cols))
        c = add(RANGE, I32, (v,), (1, 1, 0))
    else:
        c = add(RANGE, I32, (), (1, 1, n_cols))
    k = add(CONST, I32, (), (n_cols,))
    addr = add(IADD, I32, (add(IMUL, I32, (r, k)), c))
    ld = add(LOAD, F32, (add(INDEX, I32, (x, addr)),))
    e = add(EXP2, F32, (ld,))
    red = add(REDUCE, F32, (e, c), (0,))
    two = add(CONST, F32, (), (0x40000000,))
    val = add(MUL, F32, (red, two))
    add(STORE, F32, (out, r, val))
    return nodes


def test_render_group_and_thread_geometry(tmp_path):
    src, info = hip.render_kernel(row_sum_dag(8, 1024), "k_rowsum")
    assert info.group == 256 and info.grid_max == 8 and info.block == 256 and info.kvar_slot == 0
    assert "wsum(" in src and "__syncthreads" in src and "extern \"C\" __global__" in src
    # the row offset does not read the reduce axis: hoisted out of the loop
    loop = src.index("for (int rr")
    assert src.index("((int)v") < loop
    compile_ok(src, tmp_path)
    src2, info2 = hip.render_kernel(row_sum_dag(1000, 16), "k_rowsum_small")
    assert info2.group == 1 and info2.grid_max == (1000 + 255) // 256
    assert "for (int a1 = 0; a1 < 16; a1++)" in src2


@pytest.mark.parametrize("opts,group,grid", [((128, 8, 1), 8, (1000 + 15) // 16), ((64, 64, 1), 64, 1000),
                                             ((512, 256, 1), 256, 500), ((256, 1, 4), 1, 1),
                                             ((1024, 1024, 1), 1024, 1000)])
def test_render_opts_geometry(tmp_path, opts, group, grid):
    """The LOCAL / GROUP_REDUCE / UPCAST opts: block threads, group threads per
    output (xor shuffles inside a wave, LDS across waves), upcast outputs per
    thread; each variant compiles for gfx950."""
    src, info = hip.render_kernel(row_sum_dag(1000, 1024), "k_opts", opts=opts)
    assert (info.block, info.group, info.upcast, info.grid_max) == (opts[0], group, opts[2], grid)
    if group > 64:
        assert "__syncthreads" in src and "act_" in src
    elif group > 1:
        assert "__shfl_xor" in src and "__syncthreads" not in src
    if opts[2] > 1:
        assert "for (int uj_ = 0; uj_ < 4; uj_++)" in src
    compile_ok(src, tmp_path)


def test_render_opts_refused():
    for opts in ((96, 1, 1), (64, 128, 1), (256, 4, 2), (256, 1, 16)):
        with pytest.raises(hip.ThvmHipError):
            hip.render_kernel(row_sum_dag(8, 1024), "k_bad", opts=opts)
    # a group needs a reduction: out[i] = x[i] * x[i]
    F, I = 13, 5
    ew = [(BUFFER, F, (), (0, 64)), (BUFFER, F, (), (1, 64)), (RANGE, I, (), (0, 5, 64)),
          (INDEX, I, (1, 2), ()), (LOAD, F, (3,), ()), (MUL, F, (4, 4), ()), (STORE, F, (0, 2, 5), ())]
    hip.render_kernel(ew, "k_ew")
    with pytest.raises(hip.ThvmHipError):
        hip.render_kernel(ew, "k_bad2", opts=(256, 8, 1))


def test_render_symbolic_extent_reads_variable_buffer(tmp_path):
    src, info = hip.render_kernel(row_sum_dag(4, 300, symbolic=True), "k_sym")
    assert info.kvar_slot == 2 and info.n_slots == 3
    assert "kv_[3]" in src
    compile_ok(src, tmp_path)


def test_render_guards_and_errors():
    src, _ = hip.render_kernel(row_sum_dag(3, 300), "k_guard")
    assert "< 900ull" in src and "< 3ull" in src          # capacity-guarded load and store
    bad = row_sum_dag(3, 300)[:-1]                          # no STORE root
    with pytest.raises(hip.ThvmHipError, match="STORE"):
        hip.render_kernel(bad, "k_bad")
    fwd = list(row_sum_dag(3, 300))
    op, dt, srcs, args = fwd[5]
    fwd[5] = (op, dt, (len(fwd) - 1,) + srcs[1:], args)       # a source after its user
    with pytest.raises(hip.ThvmHipError):
        hip.render_kernel(fwd, "k_bad2")
    unk = list(row_sum_dag(3, 300))
    op, dt, srcs, args = unk[-2]
    unk[-2] = (52, dt, srcs, args)                           # COPY: not rendered here
    with pytest.raises(hip.ThvmHipError, match="not rendered"):
        hip.render_kernel(unk, "k_bad3")


# ---------------------------------------------------------------- host lowering
@pytest.fixture
def fake_host(monkeypatch):
    import thvm_amd.tensor as T

    class FakeBuffer:
        n = 100

        def __init__(self, nbytes):
            FakeBuffer.n += 1
            self.id, self.nbytes = FakeBuffer.n, nbytes

        def write(self, a, byte_off=0):
            pass

        def free(self):
            self.id = 0

    rendered = []

    def dispatch(kb):
        rendered.append(hip.render_kernel(kb.nodes, "k%d" % len(rendered)))

    monkeypatch.setattr(T._hip, "Buffer", FakeBuffer)
    monkeypatch.setattr(T, "_ensure_init", lambda: None)
    monkeypatch.setattr(T, "_dispatch_rendered", dispatch)
    monkeypatch.setattr(T._KV, "buf", None)
    return T, rendered


def test_lowering_softmax_is_three_kernels(fake_host):
    T, rendered = fake_host
    x = T.Tensor(np.zeros((4, 1000), np.float32))
    x.softmax(-1).realize()
    # max and sum(exp) share each row among threads (hand-coded: 1000 / 4 -> 128), normalise is elementwise
    assert [r[1].group for r in rendered] == [128, 128, 1]


def test_lowering_fuses_elementwise_and_mean(fake_host):
    T, rendered = fake_host
    a = T.Tensor(np.zeros((2, 512), np.float32))
    b = T.Tensor(np.zeros((512,), np.float32))
    ((a * 2.0 + b).exp() - 1.0).realize()
    assert len(rendered) == 1 and rendered[0][1].group == 1
    rendered.clear()
    a.mean(-1).realize()                                     # sum and scale in one kernel
    assert len(rendered) == 1 and rendered[0][1].group == 128


def test_lowering_symbolic_shrink(fake_host):
    T, rendered = fake_host
    cache = T.Tensor(np.zeros((1, 64, 8), np.float32))
    sp = T.Variable("lower_pos", 0, 63).bind(10)
    cache[:, :sp + 1, :].sum(1).realize()
    src, info = rendered[-1]
    assert info.kvar_slot > 0 and "kv_[" in src


def test_symbolic_ints():
    from thvm_amd.tensor import Sym, Variable, smax, sval
    v = Variable("sym_test", 1, 100).bind(7)
    s = v + 3
    assert isinstance(s, Sym) and smax(s) == 103 and sval(s) == 10
    assert (s - v) == 3 and (2 * s).vmax == 206
    assert Variable("sym_test", 1, 100).slot == v.slot
    with pytest.raises(ValueError):
        Variable("sym_test", 1, 100).bind(0)


def test_beam_width_env(monkeypatch):
    """BEAM sets the search width; JITBEAM overrides it inside a TinyJit
    function's first call (the kernels its graph replays), as the
    reference's autotune reads them."""
    import thvm_amd.tensor as T
    monkeypatch.delenv("BEAM", raising=False)
    monkeypatch.delenv("JITBEAM", raising=False)
    assert T._beam_width() == 0
    monkeypatch.setenv("BEAM", "4")
    assert T._beam_width() == 4
    monkeypatch.setenv("JITBEAM", "2")
    assert T._beam_width() == 4
    monkeypatch.setattr(T, "_IN_JIT", 1)
    assert T._beam_width() == 2
    monkeypatch.delenv("BEAM")
    assert T._beam_width() == 2
    monkeypatch.setattr(T, "_IN_JIT", 0)
    assert T._beam_width() == 0


def test_autotune_refuses_output_buffer_bound_as_input():
    """An input slot carrying the output's buffer id is an in-place update:
    each timed repetition would read what the previous one wrote, so the
    search refuses it (before touching the device)."""
    import thvm_amd as H
    nodes = [(36, 13, (), (0,)), (36, 13, (), (1,)), (37, 13, (1,), ())]
    with pytest.raises(H.ThvmHipError, match="reads its output buffer"):
        H.render_autotune(nodes, [7, 7])


# ---------------------------------------------------- matmuls on MFMA, fp8 stores
import _matmul_dag as MD  # noqa: E402


@pytest.mark.parametrize("dt", [MD.F16, MD.BF16])
@pytest.mark.parametrize("shape", [(32, 48, 64, 4, False), (16, 16, 48, 0, True), (64, 32, 32, 8, False)])
def test_render_matmul_takes_mfma(tmp_path, dt, shape):
    """A lifted fp16 / bf16 matmul with M, N, K multiples of 16 renders as
    the MFMA tile kernel (16x16x32 where 32 divides K, else 16x16x16), one
    wave per 16x16 tile; the source compiles for gfx950."""
    M, N, K, split, bt = shape
    src, info = hip.render_kernel(MD.matmul(M, N, K, dt, MD.F32, b_trans=bt, split=split), "k_mm")
    assert "__builtin_amdgcn_mfma_f32_16x16x" in src
    assert ("16x16x32" in src) == (K % 32 == 0)
    assert info.block == 256 and info.grid_max == (M // 16) * (N // 16) // 4 + ((M // 16) * (N // 16) % 4 > 0)
    compile_ok(src, tmp_path)


def test_render_matmul_epilogue_and_fallbacks(tmp_path):
    """The epilogue (a CAST and + bias[n]) runs on the tile's results; shapes
    and forms outside the tile path (M = 4 as the reference's decode
    schedules, f32 operands, explicit opts) keep the generic kernel."""
    src, _ = hip.render_kernel(MD.matmul(32, 32, 64, MD.BF16, MD.BF16, bias=True, cast_to=MD.BF16), "k_mm_epi")
    assert "mfma" in src and "rt_bf16" in src
    compile_ok(src, tmp_path)
    src, _ = hip.render_kernel(MD.matmul(32, 32, 64, MD.F16, MD.F32, widen=True), "k_mm_wide")
    assert "mfma" in src
    for rows, opts in ((MD.matmul(4, 32, 64, MD.F16, MD.F16), None),
                       (MD.matmul(32, 32, 64, MD.F32, MD.F32), None),
                       (MD.matmul(32, 32, 64, MD.F16, MD.F16), (256, 1, 1)),
                       (MD.matmul(32, 32, 40, MD.F16, MD.F16, split=0), None)):
        src, _ = hip.render_kernel(rows, "k_mm_generic", opts=opts)
        assert "mfma" not in src


def test_render_fp8_store(tmp_path):
    """An fp8 e4m3 output renders with the store narrowing (saturating RNE)
    and compiles."""
    src, _ = hip.render_kernel(MD.scale_store(1000, MD.F32, MD.FP8, 0x3F800000), "k_fp8")
    assert "f2fp8e4m3" in src
    compile_ok(src, tmp_path)
