"""Prefill GEMM on fp32 activations (openmini_qmm_gemm_f32, the input type of
linear_gemm, model.rs:1060-1064) and the host operator's route to it
(openmini_qmm_linear_host from 128 rows on), against the fp64 oracle.

The activations reach the fp16 MFMA as a per-row power-of-two scale and fp16 hi + lo
parts (22 significant bits); the products with the exact fp16 codes are exact, sums are
fp32.  Besides the 1e-3 parity gate, adversarial rows must stay within 4x the error of
the reference's own f32 path (oracle.cpu_asrun_linear)."""
import ctypes

import numpy as np
import pytest

from openmini_qmm import _native, synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0, Q8_0, Q4_K, Q6_K = 2, 7, 12, 14


def blocks_for(qtype, N, K, seed, sigma=0.02):
    if qtype in (Q4_K, Q6_K):
        return synth.kquant_blocks(qtype, N, K, seed=seed)
    return synth.weight_blocks(qtype, N, K, seed=seed, sigma=sigma)


def run_gemm_f32(qmm, w, x):
    """y = x . W^T through openmini_qmm_gemm_f32, y NaN-filled first."""
    M = x.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    dy = qmm.DeviceBuffer(M * w.n_rows * 4)
    dy.fill(0xFF)
    w.gemm_f32(dx, dy, M)
    return dy.download(np.float32, (M, w.n_rows))


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def linear_host(w, x):
    y = np.full((x.shape[0], w.n_rows), np.nan, np.float32)
    _native.check(_native.lib().openmini_qmm_linear_host(w.handle, _ptr(x), _ptr(y), x.shape[0]))
    return y


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("N,K,M", [(16, 256, 1), (100, 512, 5), (130, 1024, 64), (257, 2304, 200),
                                   (640, 512, 384), (64, 6144, 130), (48, 11008, 129)])
def test_gemm_f32_shapes(qmm, orc, qtype, N, K, M):
    """Ragged N and M, both tile shapes (M <= 128 and above), every weight type, K from
    256 to 11008."""
    print(f"gemm_f32 type={qtype} N={N} K={K} M={M}", flush=True)
    blocks = blocks_for(qtype, N, K, seed=0xF00 + N + K + M)
    x = synth.normal(0xF01 + M, (M, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = run_gemm_f32(qmm, w, x)
    assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"{qtype} {N}x{K} M={M}")


@pytest.mark.parametrize("M", [128, 512, 2048])
def test_gemm_f32_configs3_full_output(qmm, orc, M):
    """configs[3]'s weight and sizes (Q8_0 W[11008, 4096], M = 128 / 512 / 2048) with the
    fp32 activations the reference's linear_gemm takes: every output against the fp64
    product of the oracle's dequantized weights."""
    N, K = 11008, 4096
    print(f"gemm_f32 full output type=Q8_0 N={N} K={K} M={M}", flush=True)
    blocks = synth.weight_blocks(Q8_0, N, K, seed=0x5EED0F00 + M)
    x = synth.normal(0x5EED0F01 + M, (M, K), 1.0)
    w = qmm.QuantizedWeight(Q8_0, blocks, N, K)
    y = run_gemm_f32(qmm, w, x)
    assert np.all(np.isfinite(y)), "unwritten (NaN) outputs"
    w64 = orc.dequantize(Q8_0, blocks, N * K).reshape(N, K).astype(np.float64)
    print(assert_parity(y, x.astype(np.float64) @ w64.T, TOL, f"Q8_0 {N}x{K} M={M}"))


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


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_gemm_f32_error_within_fp32_path(qmm, orc, qtype):
    """Adversarial activation rows at M = 128, each row's largest error against the fp64
    oracle at most 4x that of the f32 GEMV over the dequantized weights (the reference's
    per-token path):
    0  a x3e4 outlier on a feature every weight row ignores (weights 0 there);
    1  mixed exponents, N(0, 1) * 2^u, u uniform in [-20, 20] per element;
    2  near-cancelling outputs (x projected off W's first 8 rows);
    3  a x3e4 outlier on a used feature;
    4  rows scaled by 1e-30 (fp32 subnormal products) and 5 by 1e30;
    the other rows N(0, 1)."""
    N, K, M = 512, 4096, 128
    blocks = _zero_column(qtype, synth.weight_blocks(qtype, N, K, seed=0xF10 + qtype), N, K, 5)
    w_f32 = orc.dequantize(qtype, blocks, N * K).reshape(N, K)
    rng = np.random.default_rng(0xF11)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, 5] = np.float32(3e4)
    x[1] = (x[1] * np.exp2(rng.integers(-20, 21, K))).astype(np.float32)
    xx = x[2].astype(np.float64)
    for r in range(8):
        wr = w_f32[r].astype(np.float64)
        xx = xx - (xx @ wr) / (wr @ wr) * wr
    x[2] = xx.astype(np.float32)
    x[3, 100] = np.float32(3e4)
    x[4] *= np.float32(1e-30)
    x[5] *= np.float32(1e30)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = run_gemm_f32(qmm, w, x)
    ref = orc.linear_f64(qtype, blocks, N, K, x)
    y32 = orc.cpu_asrun_linear(w_f32, x, None, False)
    for r in range(M):
        e_gpu = float(np.max(np.abs(y[r] - ref[r])))
        e_f32 = float(np.max(np.abs(y32[r] - ref[r])))
        if r < 6:
            print(f"row {r}: gpu {e_gpu:.3e} f32 path {e_f32:.3e}")
            assert e_gpu <= 4.0 * e_f32, (r, e_gpu, e_f32)
        assert_parity(y[r:r + 1], ref[r:r + 1], TOL, f"row {r}")


def test_gemm_f32_non_finite_rows(qmm, orc):
    """A row holding inf or NaN gives NaN outputs in that row only; an all-zero row gives
    zeros."""
    N, K, M = 200, 1024, 70
    blocks = synth.weight_blocks(Q8_0, N, K, seed=0xF20)
    x = synth.normal(0xF21, (M, K), 1.0)
    x[3, 17] = np.inf
    x[40, 1000] = np.nan
    x[41] = 0.0
    w = qmm.QuantizedWeight(Q8_0, blocks, N, K)
    y = run_gemm_f32(qmm, w, x)
    assert np.all(np.isnan(y[3])) and np.all(np.isnan(y[40]))
    assert np.all(y[41] == 0.0)
    ok = [r for r in range(M) if r not in (3, 40)]
    assert_parity(y[ok], orc.linear_f64(Q8_0, blocks, N, K, x[ok]), TOL, "finite rows")


def test_gemm_f32_repeatable_and_row_independent(qmm):
    """Fixed reduction order: repeated calls are bitwise equal, and a row's bits do not
    depend on the other rows of the call (the split scale is per row)."""
    N, K = 700, 2048
    blocks = synth.weight_blocks(Q4_0, N, K, seed=0xF30)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    x = synth.normal(0xF31, (300, K), 1.0)
    y = run_gemm_f32(qmm, w, x)
    assert np.array_equal(y.view(np.uint32), run_gemm_f32(qmm, w, x).view(np.uint32))
    x2 = x.copy()
    x2[150:] *= np.float32(1e6)
    y2 = run_gemm_f32(qmm, w, x2)
    assert np.array_equal(y[:150].view(np.uint32), y2[:150].view(np.uint32))


@pytest.mark.parametrize("N,K", [(1100, 4096), (10240, 1024), (1024, 8192)])
@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_linear_host_routes_prefill_to_gemm(qmm, orc, qtype, N, K):
    """openmini_qmm_linear_host (GemmEngine::matmul's binding) runs the decode GEMVs below
    the weight's openmini_qmm_gemm_min_rows (64-128 by the weight's shape) and the fp32
    GEMM from there on: one row below the threshold it equals openmini_qmm_gemv, at the
    threshold and at 300 rows openmini_qmm_gemm_f32, bit for bit, and both meet the
    oracle.  A short-K weight of many rows switches at the lowest count, a long-K
    weight of few rows (whose GEMM grid stays small) at the highest."""
    blocks = synth.weight_blocks(qtype, N, K, seed=0xF40 + qtype)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    t = w.gemm_min_rows()
    assert qmm.GEMM_MIN_ROWS_LOW <= t <= qmm.GEMM_MIN_ROWS
    if (N, K) == (10240, 1024):
        assert t == qmm.GEMM_MIN_ROWS_LOW
    if (N, K) == (1024, 8192):
        assert t == qmm.GEMM_MIN_ROWS
    assert not w.prefill_gemm(t - 1) and w.prefill_gemm(t)
    for M in (t - 1, t, 300):
        print(f"linear_host route type={qtype} N={N} K={K} M={M}", flush=True)
        x = synth.normal(0xF41 + M, (M, K), 1.0)
        y = linear_host(w, x)
        if M < t:
            dx, dy = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(M * N * 4)
            w.gemv(dx, dy, M)
            other = dy.download(np.float32, (M, N))
        else:
            other = run_gemm_f32(qmm, w, x)
        assert np.array_equal(y.view(np.uint32), other.view(np.uint32)), M
        assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"N={N} M={M}")


def test_ffn_gate_up_f32(qmm, orc):
    """FFNWeights::forward's hidden state silu(x . Wg^T) * (x . Wu^T) (model.rs:728-731)
    on fp32 prefill activations: one split of x, the gate GEMM, then the up GEMM with the
    SwiGLU epilogue; and the host engine's fused_gemm_silu, which takes this path from
    GEMM_MIN_ROWS rows on."""
    N, K, M = 1408, 1024, 160
    assert M >= qmm.GEMM_MIN_ROWS
    bg = synth.weight_blocks(Q4_0, N, K, seed=0xF50)
    bu = synth.weight_blocks(Q4_0, N, K, seed=0xF51)
    wg, wu = qmm.QuantizedWeight(Q4_0, bg, N, K), qmm.QuantizedWeight(Q4_0, bu, N, K)
    x = synth.normal(0xF52, (M, K), 1.0)
    dx, dh = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(M * N * 4)
    dh.fill(0xFF)
    work = qmm.gemm_f32_workspace(M, K)
    _native.check(_native.lib().openmini_qmm_ffn_gate_up_f32(wg.handle, wu.handle, dx.ptr, dh.ptr, M, work.ptr,
                                                             work.nbytes, None))
    h = dh.download(np.float32, (M, N))
    assert_parity(h, orc.ffn_hidden_f64(Q4_0, bg, bu, N, K, x), TOL, "ffn_gate_up_f32")
    g, u = run_gemm_f32(qmm, wg, x), run_gemm_f32(qmm, wu, x)
    h_ref = (g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))) * u
    np.testing.assert_allclose(h, h_ref, rtol=1e-5, atol=1e-6 * float(np.max(np.abs(h_ref))))
    h_eng = qmm.get_gemm_engine().fused_gemm_silu(x, wg, wu)
    assert np.array_equal(h_eng.view(np.uint32), h.view(np.uint32))


def test_gemm_f32_workspace_checks(qmm):
    """A workspace that is too small or misaligned is refused before any launch."""
    L = _native.lib()
    N, K, M = 64, 512, 8
    w = qmm.QuantizedWeight(Q8_0, synth.weight_blocks(Q8_0, N, K, seed=0xF60), N, K)
    need = L.openmini_qmm_gemm_f32_workspace_bytes(M, K)
    assert need >= M * K * 4 + M * 4
    dx, dy = qmm.DeviceBuffer(M * K * 4), qmm.DeviceBuffer(M * N * 4)
    work = qmm.DeviceBuffer(need + 512)
    assert L.openmini_qmm_gemm_f32(w.handle, dx.ptr, dy.ptr, M, work.ptr, need - 1, None) == _native.ERR_INVALID_PARAM
    assert b"workspace" in L.openmini_qmm_last_error()
    misaligned = ctypes.c_void_p(work.ptr.value + 16)
    assert L.openmini_qmm_gemm_f32(w.handle, dx.ptr, dy.ptr, M, misaligned, need, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemm_f32(w.handle, dx.ptr, dy.ptr, M, None, need, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemm_f32_workspace_bytes(0, K) == 0


@pytest.mark.parametrize("split_x", [False, True])
@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_gemm_every_launch_shape(qmm, orc, qtype, split_x):
    """The prefill GEMM picks one of four launch shapes (128 or 64 rows x 3 or 2 weight
    tiles per wave) from the problem size.  Over these sizes every shape must be picked
    at least once, for every weight type, with bf16 and with split fp32 activations,
    and every call meets the oracle (sampled rows, y NaN-filled).  Q6_K on bf16
    activations has no 128 x 96 shape (its per-super-block sums would not fit the
    registers), and split activations no 64 x 96 shape (64 x 64 runs faster or within
    0.6% there)."""
    L = _native.lib()
    K = 512
    seen = {}
    for N, M in ((100, 5), (4096, 512), (8192, 1024), (11008, 512), (11008, 128)):
        blocks = blocks_for(qtype, N, K, seed=0xF70 + N + M)
        w = qmm.QuantizedWeight(qtype, blocks, N, K)
        shape = L.openmini_qmm_gemm_launch_shape(w.handle, M, int(split_x))
        assert 0 <= shape <= 3, shape
        print(f"gemm shape {shape}: type={qtype} split_x={split_x} N={N} M={M}", flush=True)
        x = synth.normal(0xF71 + M, (M, K), 1.0)
        rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(N).integers(0, M, 6)]))
        if split_x:
            y = run_gemm_f32(qmm, w, x)
            ref = orc.linear_f64(qtype, blocks, N, K, x[rows])
        else:
            xb = synth.to_bf16_bits(x)
            dx, dy = qmm.DeviceBuffer.from_numpy(xb), qmm.DeviceBuffer(M * N * 4)
            dy.fill(0xFF)
            w.gemm_bf16(dx, dy, M)
            y = dy.download(np.float32, (M, N))
            ref = orc.linear_bf16x_f64(qtype, blocks, N, K, xb[rows])
        assert np.all(np.isfinite(y)), "unwritten (NaN) outputs"
        assert_parity(y[rows], ref, TOL, f"shape {shape} N={N} M={M}")
        seen.setdefault(shape, (N, M))
    expect = [0, 1, 3] if split_x else [1, 2, 3] if qtype == 14 else [0, 1, 2, 3]
    assert sorted(seen) == expect, seen
