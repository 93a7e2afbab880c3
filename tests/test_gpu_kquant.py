"""Decode GEMV on Q4_K / Q6_K weights, read the way the reference reads those blocks
(openmini-server/src/model/inference/quant.rs:338-410 and :515-600; the Q4_K minimum
is always 0 there), against the fp64 oracle over orc_dequantize_q4_k / _q6_k
(model.rs:1050-1064 semantics, y = x . W^T; tolerance from tests/parity.py).

The weights stay in their K-quant form on the GPU (repacked codes, per-sub-block
scales, one d per row and super-block); the element values are exact products of an
integer code and an fp32 factor, which the one-hot test checks bit for bit."""
import ctypes

import numpy as np
import pytest

import gguf_fixtures as fx
from openmini_qmm import _native, synth
from openmini_qmm import gguf as G
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
BPB = {Q4_K: 144, Q6_K: 210}


def gemv_nan_filled(qmm, w, x):
    B = x.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x))
    dy = qmm.DeviceBuffer(B * w.n_rows * 4)
    dy.fill(0xFF)  # NaN: a row the kernel does not write fails the check
    w.gemv(dx, dy, B)
    return dy.download(np.float32, (B, w.n_rows))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("N,K", [(1, 256), (37, 512), (130, 2304), (300, 4096)])
@pytest.mark.parametrize("B", [1, 2, 4, 5])
def test_kquant_gemv_parity(qmm, orc, qtype, N, K, B):
    print(f"kquant gemv type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xC000 + N + K + B)
    x = synth.normal(0xC001 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    assert_parity(gemv_nan_filled(qmm, w, x), orc.linear_f64(qtype, blocks, N, K, x), TOL, f"N={N} K={K} B={B}")


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("N,K", [(4096, 11008), (11008, 4096)])
@pytest.mark.parametrize("B", [1, 4])
def test_kquant_gemv_llama_shapes(qmm, orc, qtype, N, K, B):
    """The Llama-7B down (4096 x 11008) and up (11008 x 4096) projections."""
    print(f"kquant gemv type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xC100 + N + B)
    x = synth.normal(0xC101 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    print(assert_parity(gemv_nan_filled(qmm, w, x), orc.linear_f64(qtype, blocks, N, K, x), TOL, "llama"))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_kquant_one_hot_columns_exact(qmm, orc, qtype):
    """x = e_k makes y = W[:, k] exactly: the activation's block is 2^29 e_k in one digit,
    the code's integer dot product is exact, and code * (d * scale) equals the
    reference's (code * d) * scale (both exact).  Columns at sub-block, half and
    super-block edges of the first, a middle and the last super-block."""
    N, K = 77, 1024
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xC200 + qtype)
    W = orc.dequantize(qtype, blocks, N * K).reshape(N, K)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    cols = [0, 15, 16, 31, 32, 255, 256, 511, 700, 1023]
    x = np.zeros((len(cols), K), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    y = np.concatenate([gemv_nan_filled(qmm, w, x[i:i + 4]) for i in range(0, len(cols), 4)])
    for i, c in enumerate(cols):
        assert np.array_equal(y[i], W[:, c]), (c, np.nonzero(y[i] != W[:, c]))
    # all ten rows in one call: the batched kernel (fp16 codes and hi / lo activations)
    yb = gemv_nan_filled(qmm, w, x)
    for i, c in enumerate(cols):
        assert np.array_equal(yb[i], W[:, c]), (c, np.nonzero(yb[i] != W[:, c]))


def test_q4_k_nonfinite_dmin_poisons_its_rows(qmm, orc):
    """An inf / NaN dmin makes every value of its super-block NaN in the reference
    (dmin * 0.0, quant.rs:376-385), so exactly the outputs of that row are NaN."""
    N, K = 48, 768
    blocks = synth.kquant_blocks(Q4_K, N, K, seed=0xC300).reshape(N, K // 256, 144)
    blocks[5, 1, 2:4] = np.frombuffer(np.float16(np.inf).tobytes(), np.uint8)
    blocks[20, 2, 2:4] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
    blocks = blocks.ravel()
    w = qmm.QuantizedWeight(Q4_K, blocks, N, K)
    x = synth.normal(0xC301, (2, K), 1.0)
    y = gemv_nan_filled(qmm, w, x)
    with np.errstate(invalid="ignore"):
        ref = orc.linear_f64(Q4_K, blocks, N, K, x)
    bad = [5, 20]
    assert not np.any(np.isfinite(ref[:, bad])) and not np.any(np.isfinite(y[:, bad]))
    good = [n for n in range(N) if n not in bad]
    assert_parity(y[:, good], ref[:, good], TOL, "finite rows")
    # the batched kernel (8 rows) and the prefill GEMM poison exactly the same rows
    x8 = synth.normal(0xC302, (8, K), 1.0)
    y8 = gemv_nan_filled(qmm, w, x8)
    with np.errstate(invalid="ignore"):
        ref8 = orc.linear_f64(Q4_K, blocks, N, K, x8)
    assert not np.any(np.isfinite(y8[:, bad]))
    assert_parity(y8[:, good], ref8[:, good], TOL, "finite rows, batched")
    xb = synth.to_bf16_bits(synth.normal(0xC303, (130, K), 1.0))
    ym = run_gemm(qmm, w, xb)
    with np.errstate(invalid="ignore"):
        refm = orc.linear_bf16x_f64(Q4_K, blocks, N, K, xb)
    assert not np.any(np.isfinite(ym[:, bad]))
    assert_parity(ym[:, good], refm[:, good], TOL, "finite rows, gemm")


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_kquant_layer_calls(qmm, orc, qtype):
    """gemv_multi (q / k / v sharing x) and the FFN hidden state silu(gate) * up on
    K-quant weights, at batch 1 (single-row kernel) and at batch 6 (batched kernel)."""
    H, F = 512, 1280
    bq, bk = synth.kquant_blocks(qtype, H, H, 0xC400), synth.kquant_blocks(qtype, 256, H, 0xC401)
    bg, bu = synth.kquant_blocks(qtype, F, H, 0xC402), synth.kquant_blocks(qtype, F, H, 0xC403)
    wq, wk = qmm.QuantizedWeight(qtype, bq, H, H), qmm.QuantizedWeight(qtype, bk, 256, H)
    wg, wu = qmm.QuantizedWeight(qtype, bg, F, H), qmm.QuantizedWeight(qtype, bu, F, H)
    for B in (1, 6):
        x = synth.normal(0xC410 + B, (B, H), 1.0)
        dx = qmm.DeviceBuffer.from_numpy(x)
        dq, dk = qmm.DeviceBuffer(B * H * 4), qmm.DeviceBuffer(B * 256 * 4)
        qmm.gemv_multi((wq, wk), dx, (dq, dk), B)
        assert_parity(dq.download(np.float32, (B, H)), orc.linear_f64(qtype, bq, H, H, x), TOL, "q")
        assert_parity(dk.download(np.float32, (B, 256)), orc.linear_f64(qtype, bk, 256, H, x), TOL, "k")
        dh = qmm.DeviceBuffer(B * F * 4)
        qmm.ffn_gate_up(wg, wu, dx, dh, B)
        assert_parity(dh.download(np.float32, (B, F)), orc.ffn_hidden_f64(qtype, bg, bu, F, H, x), TOL, "hidden")


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_kquant_from_gguf_file(qmm, tmp_path, qtype):
    """A K-quant projection read from a GGUF file uploads as its raw super-blocks and
    gives exactly what the same bytes give through openmini_qmm_upload."""
    N, K = 96, 1536
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xC500 + qtype)
    path = tmp_path / "kq.gguf"
    path.write_bytes(fx.build([("general.architecture", fx.STRING, "llama")],
                              [("model.layers.0.ffn.up_proj", [K, N], qtype, blocks.tobytes())], "standard"))
    w_file = G.GgufFile(str(path)).upload_weight("model.layers.0.ffn.up_proj")
    w_direct = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(0xC501, (3, K), 1.0)
    assert np.array_equal(gemv_nan_filled(qmm, w_file, x), gemv_nan_filled(qmm, w_direct, x))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("offset", [0, 1, 2, 3, 6])
def test_kquant_upload_from_device_any_alignment(qmm, orc, qtype, offset):
    """Repack from super-blocks already in HBM at any byte offset.  The repack copies
    each row's span to LDS in 4-byte words read from the source rounded down to 4
    bytes, and the source's last word may be partial; the bytes around the source are
    0xA5 here, so any byte read from outside it would change the result.  An odd
    super-block count and a ragged last row tile; the GEMV equals the host-uploaded
    weight's bit for bit and the oracle within tolerance."""
    N, K = 37, 256 * 9
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xC700 + offset)
    staged = np.full(blocks.size + 16, 0xA5, dtype=np.uint8)
    staged[offset: offset + blocks.size] = blocks
    dbuf = qmm.DeviceBuffer.from_numpy(staged)
    view = qmm.DeviceBuffer.__new__(qmm.DeviceBuffer)
    view.nbytes, view.ptr = blocks.size, ctypes.c_void_p(dbuf.ptr.value + offset)
    w_dev = qmm.QuantizedWeight.from_device(qtype, view, blocks.size, N, K)
    view.ptr = ctypes.c_void_p()  # not owned
    w_host = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(0xC701, (2, K), 1.0)
    y = gemv_nan_filled(qmm, w_dev, x)
    assert np.array_equal(y.view(np.uint32), gemv_nan_filled(qmm, w_host, x).view(np.uint32))
    assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"offset {offset}")


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("N,K", [(1, 256), (37, 512), (130, 2304), (1000, 4096)])
@pytest.mark.parametrize("B", [5, 8, 16, 21])
def test_kquant_batch_parity(qmm, orc, qtype, N, K, B):
    """Five and more rows go through the batched kernel (one pass over W for up to 16
    rows): ragged tiles, an odd super-block count, a batch split into 16 + 5."""
    print(f"kquant gemv batch type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xCD00 + N + K + B)
    x = synth.normal(0xCD01 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    assert_parity(gemv_nan_filled(qmm, w, x), orc.linear_f64(qtype, blocks, N, K, x), TOL, f"N={N} K={K} B={B}")


@pytest.mark.parametrize("qtype,N,K,B", [(Q4_K, 11008, 4096, 8), (Q6_K, 11008, 4096, 8),
                                         (Q4_K, 4096, 11008, 16), (Q6_K, 4096, 11008, 16)])
def test_kquant_batch_llama_shapes(qmm, orc, qtype, N, K, B):
    print(f"kquant gemv batch type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xCE00 + N + B)
    x = synth.normal(0xCE01 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    print(assert_parity(gemv_nan_filled(qmm, w, x), orc.linear_f64(qtype, blocks, N, K, x), TOL, "llama"))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_kquant_batch_rows_independent(qmm, qtype):
    """A row's output in the batched kernel depends only on its own activations: the
    first 8 rows of a 16-row call equal an 8-row call bit for bit."""
    N, K = 640, 2048
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xCF00 + qtype)
    x = synth.normal(0xCF01, (16, K), 1.0)
    x[8:] *= 1e3
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y16, y8 = gemv_nan_filled(qmm, w, x), gemv_nan_filled(qmm, w, x[:8])
    assert np.array_equal(y16[:8].view(np.uint32), y8.view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_kquant_batch_ffn_gate_up(qmm, orc, qtype):
    """silu(x . Wg^T) * (x . Wu^T) for 8 rows through the batched kernel's pair kind."""
    N, K, B = 1280, 1024, 8
    bg, bu = synth.kquant_blocks(qtype, N, K, 0xD000), synth.kquant_blocks(qtype, N, K, 0xD001)
    wg, wu = qmm.QuantizedWeight(qtype, bg, N, K), qmm.QuantizedWeight(qtype, bu, N, K)
    x = synth.normal(0xD002, (B, K), 1.0)
    dx, dh = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(B * N * 4)
    qmm.ffn_gate_up(wg, wu, dx, dh, B)
    assert_parity(dh.download(np.float32, (B, N)), orc.ffn_hidden_f64(qtype, bg, bu, N, K, x), TOL, "hidden")


def test_kquant_error_paths(qmm):
    L = _native.lib()
    blocks = synth.kquant_blocks(Q4_K, 16, 512, seed=0xC600)
    h = ctypes.c_void_p()
    ptr = blocks.ctypes.data_as(ctypes.c_void_p)
    # K must be a multiple of the 256-element super-block
    assert L.openmini_qmm_upload(Q4_K, ptr, blocks.size, 32, 256 + 32, ctypes.byref(h)) == _native.ERR_INVALID_PARAM
    # 16 rows of K = 512 need 16 * 2 * 144 bytes
    assert L.openmini_qmm_upload(Q4_K, ptr, blocks.size - 1, 16, 512, ctypes.byref(h)) \
        == _native.ERR_INSUFFICIENT_DATA
    w = qmm.QuantizedWeight(Q4_K, blocks, 16, 512)
    assert w.info().gguf_bytes == 16 * 2 * 144
    dy = qmm.DeviceBuffer(16 * 512 * 4)
    assert L.openmini_qmm_dequant_weight(w.handle, dy.ptr, None) == _native.ERR_UNSUPPORTED


def run_gemm(qmm, w, xb16):
    M = xb16.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(xb16))
    dy = qmm.DeviceBuffer(M * w.n_rows * 4)
    dy.fill(0xFF)  # NaN: an output the kernel does not write fails the check
    w.gemm_bf16(dx, dy, M)
    return dy.download(np.float32, (M, w.n_rows))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("N,K,M", [(16, 256, 1), (37, 512, 5), (130, 2304, 130), (300, 4096, 200),
                                   (257, 1024, 384)])
def test_kquant_gemm_parity(qmm, orc, qtype, N, K, M):
    """Prefill GEMM on K-quant weights (bf16 x): both tile shapes (M <= 128 and
    above), ragged row tiles, an odd super-block count, against the fp64 oracle over
    the reference's element values."""
    print(f"kquant gemm type={qtype} N={N} K={K} M={M}", flush=True)
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xC800 + N + K + M)
    xb = synth.to_bf16_bits(synth.normal(0xC801 + M, (M, K), 1.0))
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    assert_parity(run_gemm(qmm, w, xb), orc.linear_bf16x_f64(qtype, blocks, N, K, xb), TOL, f"{N}x{K} M={M}")


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("N,K,M", [(11008, 4096, 512), (4096, 11008, 128)])
def test_kquant_gemm_llama_shapes_row_sample(qmm, orc, qtype, N, K, M):
    """Llama-7B up / down projections at prefill sizes.  A row of y depends only on
    its own x row, so the oracle runs on a sample of rows."""
    print(f"kquant gemm full type={qtype} N={N} K={K} M={M}", flush=True)
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xC900 + N + M)
    xb = synth.to_bf16_bits(synth.normal(0xC901 + M, (M, K), 1.0))
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = run_gemm(qmm, w, xb)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M + N).integers(0, M, 6)]))
    print(assert_parity(y[rows], orc.linear_bf16x_f64(qtype, blocks, N, K, xb[rows]), TOL, "llama"))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("M", [4, 200])
def test_kquant_gemm_one_hot_columns_exact(qmm, orc, qtype, M):
    """x rows = e_k (bf16 1.0) make y[m] = W[:, k] exactly.  Q4_K: the code
    (q - 8) / 16 times 16 d * scale is one exact product.  Q6_K: q * scale goes in as
    bf16 hi + lo, whose MFMA sum is exact, and one rounding of (q * scale) * d equals
    the reference's ((q * d) * scale) (q * d exact).  Columns at sub-block, half and
    super-block edges."""
    N, K = 77, 1024
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xCA00 + qtype)
    W = orc.dequantize(qtype, blocks, N * K).reshape(N, K)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    cols = np.array([0, 15, 16, 31, 32, 255, 256, 511, 700, 1023])
    cols = np.resize(cols, M)
    x = np.zeros((M, K), np.float32)
    x[np.arange(M), cols] = 1.0
    y = run_gemm(qmm, w, synth.to_bf16_bits(x))
    for i, c in enumerate(cols):  # value equality: a zero weight may be -0.0 in the reference
        assert np.array_equal(y[i], W[:, c]), (i, c, np.nonzero(y[i] != W[:, c]))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_kquant_gemm_matches_gemv(qmm, qtype):
    """The GEMM and the decode GEMV are independent kernels; on the same
    bf16-representable activations they agree to fp32 reassociation."""
    N, K, M = 1000, 4096, 8
    blocks = synth.kquant_blocks(qtype, N, K, seed=0xCB00 + qtype)
    xb = synth.to_bf16_bits(synth.normal(0xCB01, (M, K), 1.0))
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y_mm = run_gemm(qmm, w, xb)
    x32 = synth.bf16_bits_to_f32(xb).reshape(M, K)
    y_mv = np.concatenate([gemv_nan_filled(qmm, w, x32[i:i + 4]) for i in range(0, M, 4)])
    p = assert_parity(y_mm, y_mv.astype(np.float64), TOL, "gemm vs gemv")
    assert p["normwise"] <= 2e-6, p


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("N,K,M", [(1280, 512, 96), (11008, 4096, 256)])
def test_kquant_ffn_gate_up_bf16(qmm, orc, qtype, N, K, M):
    """Prefill FFN hidden state silu(x . Wg^T) * (x . Wu^T) through the GEMM's
    SwiGLU epilogue on K-quant weights (oracle on a sample of rows at full size)."""
    print(f"kquant ffn_gate_up_bf16 type={qtype} N={N} K={K} M={M}", flush=True)
    bg, bu = synth.kquant_blocks(qtype, N, K, 0xCC00 + N), synth.kquant_blocks(qtype, N, K, 0xCC01 + N)
    wg, wu = qmm.QuantizedWeight(qtype, bg, N, K), qmm.QuantizedWeight(qtype, bu, N, K)
    xb = synth.to_bf16_bits(synth.normal(0xCC02 + M, (M, K), 1.0))
    dx, dh = qmm.DeviceBuffer.from_numpy(xb), qmm.DeviceBuffer(M * N * 4)
    qmm.ffn_gate_up_bf16(wg, wu, dx, dh, M)
    h = dh.download(np.float32, (M, N))
    rows = np.arange(M)
    if M * N * K > (1 << 31):
        rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M + N).integers(0, M, 6)]))
    assert_parity(h[rows], orc.ffn_hidden_bf16x_f64(qtype, bg, bu, N, K, xb[rows]), TOL, "hidden bf16")
