"""Decode GEMV on the GPU against the fp64 oracle (model.rs:1050-1064 semantics:
y = x . W^T), tolerance from tests/parity.py (1e-3 normwise and elementwise)."""
import ctypes

import numpy as np
import pytest

from openmini_qmm import synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7


def run_gemv(qmm, w, x):
    B, K = x.shape
    dx = qmm.DeviceBuffer.from_numpy(x)
    dy = qmm.DeviceBuffer(B * w.n_rows * 4)
    w.gemv(dx, dy, B)
    return dy.download(np.float32, (B, w.n_rows))


def case(qmm, orc, qtype, N, K, B, seed, sigma=0.02):
    print(f"gemv type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = synth.weight_blocks(qtype, N, K, seed=seed, sigma=sigma)
    x = synth.normal(seed + 1, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = run_gemv(qmm, w, x)
    ref = orc.linear_f64(qtype, blocks, N, K, x)
    return assert_parity(y, ref, TOL, f"type={qtype} N={N} K={K} B={B}"), w, blocks, x, y


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("N,K", [(1, 32), (5, 64), (37, 96), (130, 2080), (257, 4128), (64, 8192)])
@pytest.mark.parametrize("B", [1, 2, 3, 4, 5, 8])
def test_gemv_small_shapes(qmm, orc, qtype, N, K, B):
    case(qmm, orc, qtype, N, K, B, seed=1000 + N + K + B)


@pytest.mark.parametrize("qtype,N,K,B", [
    (Q4_0, 4096, 4096, 1),      # config 0
    (Q4_0, 11008, 4096, 1),     # headline, gate/up orientation
    (Q4_0, 4096, 11008, 1),     # headline, down orientation
    (Q8_0, 11008, 4096, 1),     # config 1
    (Q8_0, 4096, 11008, 1),
    (Q8_0, 11008, 4096, 8),
    (Q8_0, 4096, 11008, 8),
])
def test_gemv_baseline_configs(qmm, orc, qtype, N, K, B):
    p, *_ = case(qmm, orc, qtype, N, K, B, seed=0x5EED0000 + N + B)
    print(p)


@pytest.mark.parametrize("B", [1, 4, 16])
def test_gemv_70b_q_proj(qmm, orc, B):
    case(qmm, orc, Q4_0, 8192, 8192, B, seed=0x7000 + B, sigma=0.015)


def test_gemv_batch_over_8_is_sliced(qmm, orc):
    p, *_ = case(qmm, orc, Q4_0, 300, 512, 19, seed=5)


def test_gemv_linearity_full_size(qmm):
    """Size-independent property at the largest 70B shape: y(a x1 + x2) = a y(x1) + y(x2)
    within fp32 reassociation, and y(0) = 0 exactly."""
    N, K = 28672, 8192
    print(f"gemv linearity N={N} K={K}", flush=True)
    blocks = synth.weight_blocks(Q4_0, N, K, seed=77, sigma=0.015)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    x1 = synth.normal(78, (1, K), 1.0)
    x2 = synth.normal(79, (1, K), 1.0)
    y1, y2 = run_gemv(qmm, w, x1), run_gemv(qmm, w, x2)
    y12 = run_gemv(qmm, w, (np.float32(2.0) * x1 + x2).astype(np.float32))
    # fp32 reassociation only: tight normwise, contract tolerance elementwise
    p = assert_parity(y12, 2.0 * y1.astype(np.float64) + y2, TOL, "linearity")
    assert p["normwise"] <= 2e-6, p
    assert np.all(run_gemv(qmm, w, np.zeros((1, K), np.float32)) == 0.0)


def test_gemv_repeatable(qmm):
    N, K = 4096, 4096
    blocks = synth.weight_blocks(Q4_0, N, K, seed=3)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    x = synth.normal(4, (1, K), 1.0)
    a, b = run_gemv(qmm, w, x), run_gemv(qmm, w, x)
    assert np.array_equal(a, b)  # fixed reduction order: bitwise deterministic


def test_gemv_error_paths(qmm):
    from openmini_qmm import _native
    blocks = synth.weight_blocks(Q4_0, 8, 64, seed=1)
    w = qmm.QuantizedWeight(Q4_0, blocks, 8, 64)
    dx = qmm.DeviceBuffer(1024)
    dy = qmm.DeviceBuffer(1024)
    L = _native.lib()
    assert L.openmini_qmm_gemv(w.handle, dx.ptr, dy.ptr, 0, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemv(w.handle, ctypes.c_void_p(dx.ptr.value + 4), dy.ptr, 1, None) \
        == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemv(None, dx.ptr, dy.ptr, 1, None) == _native.ERR_INVALID_PARAM


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_engine_matmul_and_linear(qmm, orc, qtype):
    """GemmEngine-shaped host API (linear / linear_gemm, model.rs:1050-1064)."""
    N, K, M = 200, 1024, 21
    blocks = synth.weight_blocks(qtype, N, K, seed=31)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(32, (M, K), 1.0)
    ref = orc.linear_f64(qtype, blocks, N, K, x)
    eng = qmm.get_gemm_engine()
    assert eng.is_available() and eng.name() == "hip_quant"
    assert_parity(eng.matmul(x, w), ref, TOL, "matmul")
    assert_parity(qmm.linear(x, w), ref, TOL, "linear")
    assert_parity(qmm.linear_gemm(x[:1], w), ref[:1], TOL, "linear_gemm")
    with pytest.raises(qmm.InvalidInput):
        eng.matmul(x[:, :512], w)


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_gemv_activation_dynamic_range(qmm, orc, qtype):
    """Per-block block-floating activations: outliers (x1e4), tiny blocks (x1e-6),
    all-zero blocks and subnormals must all stay within the contract."""
    N, K = 512, 4096
    blocks = synth.weight_blocks(qtype, N, K, seed=61)
    x = synth.normal(62, (2, K), 1.0)
    x[0, 5] *= 1e4
    x[0, 1000:1032] *= 1e-6
    x[0, 2048:2080] = 0.0
    x[1, :] *= 1e-30
    x[1, 100:110] = np.float32(1e-41)  # subnormal
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = run_gemv(qmm, w, x)
    ref = orc.linear_f64(qtype, blocks, N, K, x)
    assert_parity(y[:1], ref[:1], TOL, "outliers")
    assert_parity(y[1:], ref[1:], TOL, "tiny")


def test_gemv_nonfinite_activation(qmm, orc):
    """An inf / NaN activation makes every output non-finite, as in the reference's
    f32 path (inf * w + ... is +-inf or NaN)."""
    N, K = 64, 256
    blocks = synth.weight_blocks(Q4_0, N, K, seed=63)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    for bad in (np.inf, np.nan):
        x = synth.normal(64, (1, K), 1.0)
        x[0, 77] = bad
        y = run_gemv(qmm, w, x)
        with np.errstate(invalid="ignore"):
            ref = orc.linear_f64(Q4_0, blocks, N, K, x)
        assert not np.any(np.isfinite(ref)) and not np.any(np.isfinite(y))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_gemv_nonfinite_row_stays_in_its_row(qmm, orc, qtype):
    """In a batch, a non-finite activation row makes only that row's outputs
    non-finite; the other rows match the oracle (row-wise f32 dots in the reference)."""
    N, K = 96, 512
    blocks = synth.weight_blocks(qtype, N, K, seed=65)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(66, (4, K), 1.0)
    x[1, 300] = np.nan
    x[3, 0] = -np.inf
    y = run_gemv(qmm, w, x)
    assert not np.any(np.isfinite(y[1])) and not np.any(np.isfinite(y[3]))
    for r in (0, 2):
        assert_parity(y[r:r + 1], orc.linear_f64(qtype, blocks, N, K, x[r:r + 1]), TOL, f"row {r}")


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_gemv_ragged_tiles(qmm, orc, qtype):
    """Rows not a multiple of 16 and blocks not a multiple of 4 (tile padding)."""
    for N, K in ((17, 32), (33, 160), (1000, 4000), (255, 4064)):
        case(qmm, orc, qtype, N, K, 1, seed=N + K)
        case(qmm, orc, qtype, N, K, 3, seed=N + K + 1)


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_gemv_ragged_k_reads_stop_at_k(qmm, orc, qtype):
    """K = 160 leaves the last 4-block group one block long: the kernel must read no
    activation past a row's K elements.  Row 1 starts with a NaN right after row 0's
    last element, and row 0 must still match the oracle."""
    N, K = 48, 160
    blocks = synth.weight_blocks(qtype, N, K, seed=67)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(68, (2, K), 1.0)
    x[1, 0] = np.nan
    y = run_gemv(qmm, w, x)
    assert_parity(y[:1], orc.linear_f64(qtype, blocks, N, K, x[:1]), TOL, "row 0")
    assert not np.any(np.isfinite(y[1]))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("B", [1, 3, 5])
def test_gemv_x_in_nan_tailed_buffer(qmm, orc, qtype, B):
    """x at the start of a larger allocation whose tail is NaN (K = 4000: the last
    group holds one block): nothing past x[B, K] is read, by the single-row kernel
    (B = 1, 3) or the batched one (B = 5)."""
    N, K = 40, 4000
    blocks = synth.weight_blocks(qtype, N, K, seed=69 + B)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(70 + B, (B, K), 1.0)
    buf = np.full(B * K + 1024, np.nan, np.float32)
    buf[:B * K] = x.ravel()
    dx = qmm.DeviceBuffer.from_numpy(buf)
    dy = qmm.DeviceBuffer(B * N * 4)
    w.gemv(dx, dy, B)
    assert_parity(dy.download(np.float32, (B, N)), orc.linear_f64(qtype, blocks, N, K, x), TOL, "tail")


def _zero_column(qtype, blocks, N, K, c):
    """The GGUF blocks with element c of every row set to the code of 0.0."""
    bpb = 18 if qtype == Q4_0 else 34
    b = blocks.copy().reshape(N, K // 32, bpb)
    j = c % 32
    if qtype == Q4_0:  # code 8; element 2i in the high nibble of byte i
        byte = 2 + j // 2
        b[:, c // 32, byte] = ((b[:, c // 32, byte] & 0x0F) | 0x80) if j % 2 == 0 \
            else ((b[:, c // 32, byte] & 0xF0) | 0x08)
    else:
        b[:, c // 32, 2 + j] = 0
    return b.ravel()


def _adversarial_rows(w_f32, K, seed):
    """Activation rows that stress a per-block representation of x:
    0  a x3e4 outlier on a feature every weight row ignores (its weights are 0), so
       the block's other 31 elements carry the output at 1e-4 of the block maximum;
    1  mixed exponents: N(0, 1) * 2^u, u uniform in [-20, 20], per element;
    2  near-cancelling: projected so outputs 0..7 are ~0 (error is all absolute);
    3  a x3e4 outlier on a feature the weights use."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((4, K)).astype(np.float32)
    x[0, 5] = np.float32(3e4)
    x[1] = (x[1] * np.exp2(rng.integers(-20, 21, K))).astype(np.float32)
    xx = x[2].astype(np.float64)
    for r in range(8):
        wr = w_f32[r].astype(np.float64)
        xx = xx - (xx @ wr) / (wr @ wr) * wr
    x[2] = xx.astype(np.float32)
    x[3, 100] = np.float32(3e4)
    return x


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("B", [3, 4, 8, 16])
def test_gemv_error_within_fp32_path(qmm, orc, qtype, B):
    """The activation arithmetic is not narrower than the reference's f32 path: on
    adversarial rows, the largest error of each output row against the fp64 oracle is
    at most 4x that of the f32 GEMV over the dequantized weights (the reference's
    per-token path, oracle.cpu_asrun_linear).  B = 3 runs the single-row kernel
    (30-bit block-floating activations); B = 4, 8 and 16 the batched one (fp16 hi / lo
    split) with 4, 2 and 1 lanes per activation row."""
    N, K = 512, 4096
    blocks = _zero_column(qtype, synth.weight_blocks(qtype, N, K, seed=0xAD0 + qtype), N, K, 5)
    w_f32 = orc.dequantize(qtype, blocks, N * K).reshape(N, K)
    assert np.all(w_f32[:, 5] == 0.0)
    x = _adversarial_rows(w_f32, K, 0xAD1)[:B]
    if B > 4:
        x = np.concatenate([x, synth.normal(0xAD2, (B - 4, K), 1.0)])
    wq = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = run_gemv(qmm, wq, x)
    ref = orc.linear_f64(qtype, blocks, N, K, x)
    y32 = orc.cpu_asrun_linear(w_f32, x, None, False)
    for r in range(B):
        e_gpu = float(np.max(np.abs(y[r] - ref[r])))
        e_f32 = float(np.max(np.abs(y32[r] - ref[r])))
        print(f"row {r}: gpu {e_gpu:.3e} f32 path {e_f32:.3e}")
        if r < 4:  # the adversarial rows; the N(0, 1) filler rows only fill the batch
            assert e_gpu <= 4.0 * e_f32, (r, e_gpu, e_f32)
        assert_parity(y[r:r + 1], ref[r:r + 1], TOL, f"row {r}")


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_engine_full_surface(qmm, orc, qtype):
    """The rest of the GemmEngine surface (gemm_engine.rs:37-56): batched_matmul over one
    weight per batch slice (and the reference's batch-mismatch error), fused_gemm_relu
    with a bias, and fused_gemm_silu as FFNWeights::forward's silu(gate) * up."""
    N, K, M = 160, 512, 6
    bs = [synth.weight_blocks(qtype, N, K, seed=0xE00 + i) for i in range(3)]
    ws = [qmm.QuantizedWeight(qtype, b, N, K) for b in bs]
    eng = qmm.get_gemm_engine()
    x3 = synth.normal(0xE10, (3, M, K), 1.0)
    y3 = eng.batched_matmul(x3, ws)
    for i in range(3):
        assert_parity(y3[i], orc.linear_f64(qtype, bs[i], N, K, x3[i]), TOL, f"batched {i}")
    with pytest.raises(qmm.InvalidInput, match="Batch dimension mismatch"):
        eng.batched_matmul(x3, ws[:2])
    x = x3[0]
    bias = synth.normal(0xE11, (N,), 1.0)
    ref = np.maximum(orc.linear_f64(qtype, bs[0], N, K, x) + bias, 0.0)
    got = eng.fused_gemm_relu(x, ws[0], bias)
    assert np.all(got >= 0.0)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-3 * float(np.max(np.abs(ref))))
    h = eng.fused_gemm_silu(x, ws[1], ws[2])
    assert_parity(h, orc.ffn_hidden_f64(qtype, bs[1], bs[2], N, K, x), TOL, "silu(gate) * up")
    hb = eng.fused_gemm_silu(x, ws[1], ws[2], bias)
    np.testing.assert_allclose(hb, h + bias, rtol=0, atol=0)
