"""Prefill GEMM (bf16 activations, MFMA) against the fp64 oracle on the same
bf16-rounded activations, tolerance from tests/parity.py."""
import numpy as np
import pytest

from openmini_qmm import synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7


def run_gemm(qmm, w, xb16):
    """y = x . W^T on the GPU, y NaN-filled first so an output the kernel never
    writes cannot pass."""
    M = xb16.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(xb16)
    dy = qmm.DeviceBuffer(M * w.n_rows * 4)
    dy.fill(0xFF)
    w.gemm_bf16(dx, dy, M)
    return dy.download(np.float32, (M, w.n_rows))


def make(qmm, qtype, N, K, M, seed, sigma=0.02):
    blocks = synth.weight_blocks(qtype, N, K, seed=seed, sigma=sigma)
    xb = synth.to_bf16_bits(synth.normal(seed + 1, (M, K), 1.0))
    return blocks, xb, qmm.QuantizedWeight(qtype, blocks, N, K)


@pytest.mark.parametrize("qtype", [Q8_0, Q4_0])
@pytest.mark.parametrize("N,K,M", [(16, 32, 1), (100, 96, 5), (128, 64, 128), (130, 4096, 130),
                                   (257, 2080, 200), (640, 512, 384)])
def test_gemm_small_shapes(qmm, orc, qtype, N, K, M):
    print(f"gemm type={qtype} N={N} K={K} M={M}", flush=True)
    blocks, xb, w = make(qmm, qtype, N, K, M, seed=N + K + M)
    y = run_gemm(qmm, w, xb)
    assert_parity(y, orc.linear_bf16x_f64(qtype, blocks, N, K, xb), TOL, f"{qtype} {N}x{K} M={M}")


@pytest.mark.parametrize("M", [128, 512, 2048])
def test_gemm_configs3_full_output(qmm, orc, M):
    """BASELINE configs[3] (Q8_0 W[11008, 4096], bf16 x, M = 128 / 512 / 2048), every
    output checked: the reference is the fp64 product of the oracle's dequantized
    weights (bit-exact with quant.rs, pinned by the oracle tests) and the bf16-rounded
    activations, y = x . W^T (model.rs:1060-1064)."""
    N, K = 11008, 4096
    print(f"gemm full output type=Q8_0 N={N} K={K} M={M}", flush=True)
    blocks, xb, w = make(qmm, Q8_0, N, K, M, seed=0x5EED0000 + M + N)
    y = run_gemm(qmm, w, xb)
    assert np.all(np.isfinite(y)), "unwritten (NaN) outputs"
    w64 = orc.dequantize(Q8_0, blocks, N * K).reshape(N, K).astype(np.float64)
    x64 = synth.bf16_bits_to_f32(xb).reshape(M, K).astype(np.float64)
    print(assert_parity(y, x64 @ w64.T, TOL, f"Q8_0 {N}x{K} M={M}"))


@pytest.mark.parametrize("N,K", [(8192, 8192), (28672, 8192), (8192, 28672)])
def test_gemm_configs4_full_output(qmm, orc, N, K):
    """BASELINE configs[4] prefill (Q4_0 70B-style projections, M = 1024): every output
    against the decode GEMV kernel on the same bf16-valued activations read as fp32
    (an independent kernel, oracle-pinned at these shapes by the configs tests), which
    differs only by fp32 reassociation; plus a row sample against the fp64 oracle."""
    M = 1024
    print(f"gemm full output type=Q4_0 N={N} K={K} M={M}", flush=True)
    blocks, xb, w = make(qmm, Q4_0, N, K, M, seed=0x5EED0000 + M + N, sigma=0.015)
    y = run_gemm(qmm, w, xb)
    assert np.all(np.isfinite(y)), "unwritten (NaN) outputs"
    dx = qmm.DeviceBuffer.from_numpy(synth.bf16_bits_to_f32(xb).reshape(M, K))
    dy = qmm.DeviceBuffer(M * N * 4)
    dy.fill(0xFF)
    w.gemv(dx, dy, M)
    y_mv = dy.download(np.float32, (M, N))
    p = assert_parity(y, y_mv.astype(np.float64), TOL, f"gemm vs gemv Q4_0 {N}x{K}")
    assert p["normwise"] <= 2e-6, p
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(N + K).integers(0, M, 6)]))
    print(assert_parity(y[rows], orc.linear_bf16x_f64(Q4_0, blocks, N, K, xb[rows]), TOL, f"Q4_0 {N}x{K} rows"))


def test_gemm_matches_gemv_on_bf16_inputs(qmm):
    """Two independent kernels on the same bf16-representable inputs agree to fp32
    reassociation (the GEMV reads them as fp32)."""
    N, K, M = 1000, 4096, 8
    blocks, xb, w = make(qmm, Q8_0, N, K, M, seed=42)
    y_mm = run_gemm(qmm, w, xb)
    x32 = synth.bf16_bits_to_f32(xb).reshape(M, K)
    dx = qmm.DeviceBuffer.from_numpy(x32)
    dy = qmm.DeviceBuffer(M * N * 4)
    w.gemv(dx, dy, M)
    y_mv = dy.download(np.float32, (M, N))
    # fp32 reassociation only: tight normwise, contract tolerance elementwise
    p = assert_parity(y_mm, y_mv.astype(np.float64), TOL, "gemm vs gemv")
    assert p["normwise"] <= 2e-6, p


def test_gemm_repeatable(qmm):
    blocks, xb, w = make(qmm, Q8_0, 512, 1024, 256, seed=8)
    assert np.array_equal(run_gemm(qmm, w, xb), run_gemm(qmm, w, xb))
