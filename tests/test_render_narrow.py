"""The renderer target's fp16 / bf16 and symbolic-extent test vectors: every
kernel the compiled reference schedules for linear, softmax, layernorm and
GELU over 16-bit tensors (GPT-2 XL-width rows), a whole fp16 / bf16 GPT-2
block, and decode attention over a cache whose length is a bound variable
(f32 and fp16), captured at its CPU dispatch with its lifted DAG, inputs,
output and bound variable values (tests/golden/ref_lifted_narrow.npz,
written by tests/golden/make_render_golden.py).

The reference realizes 16-bit kernels through its uop walker: each op's
value rounds to f32 (or stays double where the C render would hold a
double), and values narrow to fp16 / bf16 only at a CAST into the type and
at the STORE (src/backend/cpu/uop_walk.c:272-293).  On the CPU: a numpy
evaluation of the rows with those semantics reproduces the reference's
output to within one storage rounding (it rounds every op to f32, so where
the reference held a double the two can straddle a rounding boundary), and
every kernel renders, symbolic extents included.  The GPU test
(test_gpu_render_ref.py) runs them."""
import numpy as np
import pytest

import _dag_eval as E
import _oracle as O

GN = np.load(O.ROOT / "tests" / "golden" / "ref_lifted_narrow.npz")
NAMES_N = [str(x) for x in GN["names"]]


def storage_ulp(v, dt):
    """Spacing of the storage type at |v| (f32 for dt 13)."""
    a = np.abs(np.asarray(v, np.float64))
    if dt == 11:
        return np.spacing(a.astype(np.float16)).astype(np.float64)
    if dt == 12:
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
        return 2.0 ** (e - 7)
    return np.spacing(a.astype(np.float32)).astype(np.float64)


def close_storage(got, want, dt, ulps=1.0):
    """Within `ulps` roundings of the output's storage type plus 2^-20 of
    its largest magnitude (sums whose f32 terms cancel); equal values,
    infinities and NaNs match."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    fin = np.isfinite(want)
    scale = np.abs(want[fin]).max() if fin.any() else 0.0
    with np.errstate(invalid="ignore"):
        ok = same | (np.abs(got - want) <= ulps * storage_ulp(want, dt) + 2.0 ** -20 * scale)
    return bool(np.all(ok)), float(np.mean(same))


def kernel_n(k):
    rows = GN[f"k{k}_rows"]
    dts = [int(d) for d in GN[f"k{k}_dt"]]
    slots = {s: E.decode_slot(GN[f"k{k}_slot{s}"], dts[s]) for s in range(len(dts))}
    vars_ = [int(v[0]) for v in GN[f"k{k}_vars"]] if f"k{k}_vars" in GN.files else []
    return rows, dts, slots, vars_


def test_captured_set():
    ops = {n.split("/")[0] for n in NAMES_N}
    assert ops == {f"{o}_{t}" for o in ("linear", "softmax", "layernorm", "gelu", "gpt2_block")
                   for t in ("f16", "bf16")} | {"sym_attention_f32", "sym_attention_f16"}
    assert len(GN["skipped"]) == 0
    dts = {int(GN[f"k{k}_dt"][0]) for k in range(len(NAMES_N))}
    assert {11, 12, 13} <= dts
    sym = [k for k in range(len(NAMES_N)) if f"k{k}_vars" in GN.files]
    assert len(sym) >= 8 and all(NAMES_N[k].startswith("sym_attention") for k in sym)
    for k in sym:          # every symbolic kernel reads its extent from a DEFINE_VAR row
        rows = GN[f"k{k}_rows"]
        assert any(r[0] == E.RANGE and r[2] >= 0 and rows[r[2]][0] == E.DEFINE_VAR for r in rows)


@pytest.mark.parametrize("k", range(len(NAMES_N)), ids=NAMES_N)
def test_rows_evaluate_to_the_reference_output(k):
    rows, dts, slots, vars_ = kernel_n(k)
    got, mask = E.evaluate(rows, {s: v for s, v in slots.items() if s > 0}, vars_, written=True)
    if dts[0] == 13:
        from test_render_ref import close
        assert close(got[mask], slots[0][mask]), NAMES_N[k]
    else:
        ok, exact = close_storage(got[mask], slots[0][mask], dts[0])
        assert ok, f"{NAMES_N[k]}: exact fraction {exact}"
    if vars_:      # a symbolic kernel writes only the live rows of its padded output
        assert 0 < mask.sum() < len(mask) or mask.all()


def test_narrowing_points_matter():
    """Rounding every 16-bit intermediate to its storage type, instead of at
    CAST / STORE, moves outputs of these kernels beyond one storage rounding:
    the fixtures tell the two semantics apart (and the renderer follows the
    reference's)."""
    worst = {}
    for k in range(len(NAMES_N)):
        rows, dts, slots, vars_ = kernel_n(k)
        if dts[0] == 13:
            continue
        got = E.evaluate(rows, {s: v for s, v in slots.items() if s > 0}, vars_, narrow_every_op=True)
        with np.errstate(invalid="ignore"):
            err = np.abs(got - slots[0]) / storage_ulp(slots[0], dts[0])
        op = NAMES_N[k].split("/")[0]
        worst[op] = max(worst.get(op, 0.0), float(np.nanmax(err)))
    assert max(worst.values()) > 2.0, worst


@pytest.mark.parametrize("k", range(len(NAMES_N)), ids=NAMES_N)
def test_rows_render(k):
    import thvm_amd as T
    rows = GN[f"k{k}_rows"]
    nodes = [(int(r[0]), int(r[1]), tuple(int(x) for x in r[2:6]), tuple(int(x) for x in r[6:10])) for r in rows]
    src, info = T.render_kernel(nodes, f"rn{k}")
    assert "extern \"C\" __global__" in src and info.grid_max >= 1 and info.block >= 64
    has_var = f"k{k}_vars" in GN.files
    assert info.n_slots == len(GN[f"k{k}_dt"]) + (1 if has_var else 0)
    if has_var:
        assert "kv_" in src and info.kvar_slot == len(GN[f"k{k}_dt"])
