"""GPU parity of the dequant-GEMV path against the CPU oracle (MI355X).

Bar: dequantized values bit-exact with value_at (src/quant.rs:349-456);
GEMV outputs within 1e-3 relative error of dot_row_scalar
(src/quant.rs:458-648), measured as
    max_i |y_i - ref_i| <= 1e-3 * max_i |ref_i|               (norm-wise)
    |y_i - ref_i| <= 1e-3 * |ref_i| + 1e-4 * max_i |ref_i|     (element-wise)
The tuned kernels multiply the weight codes with the activation held as two
int8 digit planes per 16-element block (|error| <= 3.1e-5 of the block's
largest |x|), so outputs that cancel to near zero carry an absolute error of
a few 1e-5 of the output scale: the element-wise floor is 1e-4 of it.  The
generic kernels accumulate in f32 in another order than the scalar loop.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ALL_TYPES = [0, 1, 30, 2, 3, 6, 7, 8, 12, 13, 14]
NAMES = {0: "F32", 1: "F16", 30: "BF16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0",
         12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}


def assert_gemv_close(y, ref, what=""):
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    rel = float(err.max() / scale) if ref.size and scale > 0 else 0.0
    print(f"[gemv] {what} max rel err {rel:.2e}", flush=True)
    assert rel <= 1e-3, (what, rel)
    bad = err > 1e-3 * np.abs(ref) + 1e-4 * scale
    assert not bad.any(), (what, int(np.argmax(bad)), y[bad][:4], ref[bad][:4])


def run_case(llrs, backend, oracle, ty, rows, cols, seed):
    print(f"[case] {NAMES[ty]} {rows}x{cols} seed={seed}", flush=True)
    data = llrs.blocks.random_tensor_bytes(ty, rows, cols, seed=seed)
    x = llrs.blocks.random_activation(cols, seed=seed + 1)
    t = llrs.QuantTensor.from_owned(data, (rows, cols), ty)
    dt = backend.upload(t)
    y = np.empty(rows, np.float32)
    backend.matvec(dt, x, y)
    ref = oracle.matvec(data, ty, rows, cols, x)
    assert_gemv_close(y, ref, f"{NAMES[ty]} {rows}x{cols}")
    return dt, data


@pytest.mark.parametrize("ty", ALL_TYPES, ids=[NAMES[t] for t in ALL_TYPES])
def test_dequant_row_bit_exact(llrs, backend, oracle, ty):
    rows, cols = 37, 768 if ty in (12, 13, 14) else 416
    data = llrs.blocks.random_tensor_bytes(ty, rows, cols, seed=11 + ty)
    dt = backend.upload(llrs.QuantTensor.from_owned(data, (rows, cols), ty))
    assert dt.download() == data
    out = np.empty(cols, np.float32)
    for r in (0, 1, 17, rows - 1):
        dt.row_into(r, out)
        want = oracle.dequant_row(data, ty, r, cols)
        np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("ty", ALL_TYPES, ids=[NAMES[t] for t in ALL_TYPES])
def test_gemv_small_shapes(llrs, backend, oracle, ty):
    for rows, cols in ((1, 256), (3, 512), (130, 1024), (257, 2304)):
        run_case(llrs, backend, oracle, ty, rows, cols, seed=1000 + rows + ty)


def test_config1_q4k_8960x1536(llrs, backend, oracle):
    """Benchmark config 1: the Qwen2.5-1.5B ffn_gate shape, seed 1."""
    run_case(llrs, backend, oracle, 12, 8960, 1536, seed=1)


@pytest.mark.parametrize("ty", [2, 3, 6, 7, 8, 13, 14, 1, 30],
                         ids=[NAMES[t] for t in [2, 3, 6, 7, 8, 13, 14, 1, 30]])
@pytest.mark.parametrize("shape", [(18944, 3584), (3584, 18944)], ids=["up", "down"])
def test_config2_type_sweep(llrs, backend, oracle, ty, shape):
    """Benchmark config 2: every KernelBackend dot path at the 7B FFN shapes."""
    run_case(llrs, backend, oracle, ty, shape[0], shape[1], seed=2)


def test_ragged_and_empty_shapes(llrs, backend, oracle):
    QT = llrs.QuantType
    for ty, rows, cols in ((0, 5, 7), (1, 3, 33), (30, 2, 1), (0, 1, 1), (8, 1, 32), (14, 1, 256)):
        run_case(llrs, backend, oracle, ty, rows, cols, seed=77)
    empty = backend.upload(llrs.QuantTensor.from_owned(b"", (0, 256), QT.Q4K))
    y = np.empty(0, np.float32)
    backend.matvec(empty, np.zeros(256, np.float32), y)


def test_validate_matvec_errors(llrs, backend):
    QT = llrs.QuantType
    data = llrs.blocks.random_tensor_bytes(12, 4, 256, seed=3)
    dt = backend.upload(llrs.QuantTensor.from_owned(data, (4, 256), QT.Q4K))
    with pytest.raises(llrs.LlrsError, match="input mismatch"):
        backend.matvec(dt, np.zeros(255, np.float32), np.empty(4, np.float32))
    with pytest.raises(llrs.LlrsError, match="output mismatch"):
        backend.matvec(dt, np.zeros(256, np.float32), np.empty(5, np.float32))
    with pytest.raises(llrs.LlrsError, match="byte length"):
        backend.upload(llrs.QuantTensor(data[:-1], (4, 256), QT.Q4K))
    with pytest.raises(llrs.LlrsError, match="not divisible"):
        backend.upload(llrs.QuantTensor(b"\0" * 144, (1, 200), QT.Q4K))
    out = np.empty(256, np.float32)
    with pytest.raises(llrs.LlrsError, match="out of bounds"):
        dt.row_into(4, out)


def test_backend_identity(backend):
    assert backend.name() == "hip-gfx950"
    assert backend.threads() >= 200  # compute units of an MI355X


def outlier_activation(n: int, seed: int, kind: str) -> np.ndarray:
    """Activations whose 16-element blocks mix scales: "spike" puts one element
    10^3 times the others' scale in every block (the tuned kernels' int8 digits
    are scaled per block by its largest |x|, so the small elements keep only
    ~15 - 10 = 5 bits); "student_t" draws from a Student-t with 2 degrees of
    freedom (heavy tails, infinite variance)."""
    rng = np.random.default_rng(seed)
    if kind == "spike":
        x = rng.standard_normal(n, dtype=np.float32)
        at = np.arange(0, n, 16) + rng.integers(0, 16, n // 16)
        x[at] = np.float32(1e3) * np.sign(rng.standard_normal(at.size)).astype(np.float32)
        return x
    return rng.standard_t(2, n).astype(np.float32)


@pytest.mark.parametrize("kind", ["spike", "student_t"])
@pytest.mark.parametrize("ty", [12, 14, 8, 6, 2, 13, 30],
                         ids=[NAMES[t] for t in [12, 14, 8, 6, 2, 13, 30]])
@pytest.mark.parametrize("shape", [(18944, 3584), (3584, 18944)], ids=["up", "down"])
def test_gemv_outlier_activations(llrs, backend, oracle, ty, shape, kind):
    """The 1e-3 GEMV bar (src/quant.rs:458-648) holds for activations with
    outliers, at the config 2 shapes."""
    rows, cols = shape
    print(f"[case] {NAMES[ty]} {rows}x{cols} {kind}", flush=True)
    data = llrs.blocks.random_tensor_bytes(ty, rows, cols, seed=5)
    x = outlier_activation(cols, seed=6, kind=kind)
    dt = backend.upload(llrs.QuantTensor.from_owned(data, (rows, cols), ty))
    y = np.empty(rows, np.float32)
    backend.matvec(dt, x, y)
    ref = oracle.matvec(data, ty, rows, cols, x)
    assert_gemv_close(y, ref, f"{NAMES[ty]} {rows}x{cols} {kind}")
