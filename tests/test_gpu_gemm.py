"""Prefill GEMM (bf16 activations, MFMA) against the fp64 oracle on the same
bf16-rounded activations, tolerance from tests/parity.py."""
import numpy as np
import pytest

from openmini_qmm import synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7


def run_gemm(qmm, w, xb16):
    M = xb16.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(xb16)
    dy = qmm.DeviceBuffer(M * w.n_rows * 4)
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


@pytest.mark.parametrize("qtype,N,K,M", [
    (Q8_0, 11008, 4096, 128),
    (Q8_0, 11008, 4096, 512),
    (Q8_0, 11008, 4096, 2048),
    (Q4_0, 8192, 8192, 1024),
    (Q4_0, 28672, 8192, 1024),
    (Q4_0, 8192, 28672, 1024),
])
def test_gemm_baseline_configs_row_sample(qmm, orc, qtype, N, K, M):
    """Full-size configs.  y[m, :] depends only on x[m, :], so the oracle runs on a
    sample of rows (first, last and random ones) and those rows must match."""
    print(f"gemm full type={qtype} N={N} K={K} M={M}", flush=True)
    sigma = 0.015 if K == 8192 or N == 8192 else 0.02
    blocks, xb, w = make(qmm, qtype, N, K, M, seed=0x5EED0000 + M + N, sigma=sigma)
    y = run_gemm(qmm, w, xb)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).integers(0, M, 6)]))
    ref = orc.linear_bf16x_f64(qtype, blocks, N, K, xb[rows])
    print(assert_parity(y[rows], ref, TOL, f"{qtype} {N}x{K} M={M}"))


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
