"""BASELINE configs at full size against the fp64 oracle on every output.

configs[4] (Llama-70B-style Q4_0 layer, weights N(0, 0.015), activations N(0, 1)):
the gate W[28672, 8192] and down W[8192, 28672] projections at decode batch 1, 4 and
16, which exercise every launch shape of the single-row GEMV (batch 1-4) and of the
batched GEMV (8 row tiles per workgroup for the gate, 1 for the down projection);
plus the Llama-7B Q4_0 up projection at batch 16 (4 row tiles per workgroup).

Every output buffer is filled with NaN before the launch, so a row tile the kernel
skipped or wrote to the wrong place fails the parity check instead of passing as a
stale value.  Semantics: y = x . W^T (model.rs:1050-1064); tolerance from
tests/parity.py (1e-3 normwise and elementwise).
"""
import numpy as np
import pytest

from openmini_qmm import synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0 = 2


def gemv_nan_filled(qmm, w, x):
    B, K = x.shape
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x))
    dy = qmm.DeviceBuffer(B * w.n_rows * 4)
    dy.fill(0xFF)  # every float 0xFFFFFFFF: a NaN
    w.gemv(dx, dy, B)
    return dy.download(np.float32, (B, w.n_rows))


def _weight(qmm, N, K, seed, sigma):
    print(f"config weight Q4_0 N={N} K={K} sigma={sigma}", flush=True)
    blocks = synth.weight_blocks(Q4_0, N, K, seed=seed, sigma=sigma)
    return blocks, qmm.QuantizedWeight(Q4_0, blocks, N, K)


@pytest.fixture(scope="module")
def gate_70b(qmm):
    return (28672, 8192) + _weight(qmm, 28672, 8192, 0x70C4, 0.015)


@pytest.fixture(scope="module")
def down_70b(qmm):
    return (8192, 28672) + _weight(qmm, 8192, 28672, 0x70C5, 0.015)


@pytest.mark.parametrize("B", [1, 4, 16])
def test_70b_gate_full(qmm, orc, gate_70b, B):
    N, K, blocks, w = gate_70b
    print(f"gemv 70B gate N={N} K={K} B={B}", flush=True)
    x = synth.normal(0x70D0 + B, (B, K), 1.0)
    y = gemv_nan_filled(qmm, w, x)
    print(assert_parity(y, orc.linear_f64(Q4_0, blocks, N, K, x), TOL, f"gate B={B}"))


@pytest.mark.parametrize("B", [1, 4, 16])
def test_70b_down_full(qmm, orc, down_70b, B):
    N, K, blocks, w = down_70b
    print(f"gemv 70B down N={N} K={K} B={B}", flush=True)
    x = synth.normal(0x70E0 + B, (B, K), 1.0)
    y = gemv_nan_filled(qmm, w, x)
    print(assert_parity(y, orc.linear_f64(Q4_0, blocks, N, K, x), TOL, f"down B={B}"))


def test_7b_up_batch16_full(qmm, orc):
    N, K, B = 11008, 4096, 16
    blocks, w = _weight(qmm, N, K, 0x7B16, 0.02)
    x = synth.normal(0x7B17, (B, K), 1.0)
    y = gemv_nan_filled(qmm, w, x)
    print(assert_parity(y, orc.linear_f64(Q4_0, blocks, N, K, x), TOL, "7B up B=16"))
