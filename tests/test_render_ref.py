"""The renderer target's test vectors: every kernel the compiled reference
schedules for GPT-2 step operations (linear, softmax, layernorm, RMSNorm,
GELU, causal attention, a whole GPT-2 block), captured at its CPU dispatch with its lifted DAG,
inputs and output (tests/golden/ref_lifted_kernels.npz, written by
tests/golden/make_render_golden.py).  On the CPU: a plain numpy evaluation
of the rows reproduces the reference's own output (pinning what the rows
mean), and every kernel renders.  The GPU test (test_gpu_render_ref.py)
runs the rendered kernels."""
import numpy as np
import pytest

import _dag_eval as E
import _oracle as O

G = np.load(O.ROOT / "tests" / "golden" / "ref_lifted_kernels.npz")
NAMES = [str(x) for x in G["names"]]


def close(got, want):
    """f32 1e-5 relative per element, plus 1e-6 of the output's largest
    finite magnitude (sums whose terms cancel); equal infinities match."""
    fin = np.isfinite(want)
    scale = np.abs(want[fin]).max() if fin.any() else 0.0
    with np.errstate(invalid="ignore"):
        ok = (got == want) | (np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-6 * scale)
    return bool(np.all(ok))


def kernel(k):
    rows = G[f"k{k}_rows"]
    dts = [int(d) for d in G[f"k{k}_dt"]]
    slots = {s: E.decode_slot(G[f"k{k}_slot{s}"], dts[s]) for s in range(len(dts))}
    return rows, dts, slots


def test_captured_set():
    assert len(NAMES) >= 30
    ops = {n.split("/")[0] for n in NAMES}
    assert ops == {"linear", "softmax", "layernorm", "rmsnorm", "gelu", "attention", "gpt2_block"}


@pytest.mark.parametrize("k", range(len(NAMES)), ids=NAMES)
def test_rows_evaluate_to_the_reference_output(k):
    rows, dts, slots = kernel(k)
    want = slots[0]
    got = E.evaluate(rows, {s: v for s, v in slots.items() if s > 0})
    assert close(got, want), NAMES[k]


@pytest.mark.parametrize("k", range(len(NAMES)), ids=NAMES)
def test_rows_render(k):
    import thvm_amd as T
    rows = G[f"k{k}_rows"]
    nodes = [(int(r[0]), int(r[1]), tuple(int(x) for x in r[2:6]), tuple(int(x) for x in r[6:10])) for r in rows]
    src, info = T.render_kernel(nodes, f"rk{k}")
    assert "extern \"C\" __global__" in src and info.grid_max >= 1 and info.block >= 64
    assert info.n_slots == len(G[f"k{k}_dt"])
