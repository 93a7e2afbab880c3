"""Q8_K weights, read the way the reference reads the 258-byte super-block: fp16 d,
then 256 int8 codes, element i = q_i * d (openmini-server/src/model/inference/
quant.rs:768-800).  That is eight Q8_0 blocks sharing one d, so the upload writes
Q8_0 chunks and every Q8_0 kernel serves the weight.

Pinned three ways: the uploaded weight dequantizes bit for bit to the oracle's
orc_dequantize_q8_k; each product equals, bit for bit, the same product on the Q8_0
blocks holding the same codes and d; and the products match the fp64 oracle over
the dequantized weight (model.rs:1050-1064 semantics, y = x . W^T; tolerance from
tests/parity.py)."""
import ctypes

import numpy as np
import pytest

import gguf_fixtures as fx
from openmini_qmm import gguf as G
from openmini_qmm import synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q8_0, Q8_K = 7, 15


def as_q8_0(blocks, N, K):
    """The Q8_0 blocks (34 B: d, 32 codes) of the same values: each super-block's d
    in front of each of its eight 32-code runs, rows in the same order."""
    sb = blocks.reshape(N * (K // 256), 258)
    out = np.empty((N * (K // 256), 8, 34), dtype=np.uint8)
    out[:, :, 0:2] = sb[:, None, 0:2]
    out[:, :, 2:] = sb[:, 2:].reshape(-1, 8, 32)
    return out.ravel()


def gemv_nan_filled(qmm, w, x):
    B = x.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x))
    dy = qmm.DeviceBuffer(B * w.n_rows * 4)
    dy.fill(0xFF)  # NaN: an output the kernel does not write fails the check
    w.gemv(dx, dy, B)
    return dy.download(np.float32, (B, w.n_rows))


def gemm_bf16(qmm, w, xb16):
    M = xb16.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(xb16))
    dy = qmm.DeviceBuffer(M * w.n_rows * 4)
    dy.fill(0xFF)
    w.gemm_bf16(dx, dy, M)
    return dy.download(np.float32, (M, w.n_rows))


@pytest.mark.parametrize("N,K", [(1, 256), (37, 512), (130, 2304)])
def test_q8k_upload_dequantizes_bit_exact(qmm, orc, N, K):
    print(f"q8k dequant N={N} K={K}", flush=True)
    blocks = synth.kquant_blocks(Q8_K, N, K, seed=0xE100 + N)
    w = qmm.QuantizedWeight(Q8_K, blocks, N, K)
    info = w.info()
    assert info.type == Q8_K and info.gguf_bytes == N * (K // 256) * 258
    ref = orc.dequantize(Q8_K, blocks, N * K).reshape(N, K)
    assert np.array_equal(w.dequantize().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("N,K", [(37, 512), (300, 2304), (11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("B", [1, 3, 8, 16])
def test_q8k_gemv_equals_q8_0_and_oracle(qmm, orc, N, K, B):
    """Both decode kernels (1-3 rows single-row, 4+ batched, with the K split of the
    4096-row weights), every output checked with y NaN-filled first."""
    print(f"q8k gemv N={N} K={K} B={B}", flush=True)
    blocks = synth.kquant_blocks(Q8_K, N, K, seed=0xE200 + N + K)
    x = synth.normal(0xE201 + B, (B, K), 1.0)
    y = gemv_nan_filled(qmm, qmm.QuantizedWeight(Q8_K, blocks, N, K), x)
    y0 = gemv_nan_filled(qmm, qmm.QuantizedWeight(Q8_0, as_q8_0(blocks, N, K), N, K), x)
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32))
    assert_parity(y, orc.linear_f64(Q8_K, blocks, N, K, x), TOL, f"N={N} K={K} B={B}")


@pytest.mark.parametrize("N,K,M", [(37, 512, 5), (300, 4096, 200), (11008, 4096, 512)])
def test_q8k_prefill_gemm(qmm, orc, N, K, M):
    """The bf16 prefill GEMM equals the Q8_0 weight's bit for bit and the fp64 oracle on
    the same bf16 activations; linear() on fp32 rows (128+ rows: the fp32 GEMM) matches
    the oracle."""
    print(f"q8k gemm N={N} K={K} M={M}", flush=True)
    blocks = synth.kquant_blocks(Q8_K, N, K, seed=0xE300 + N + M)
    w = qmm.QuantizedWeight(Q8_K, blocks, N, K)
    w0 = qmm.QuantizedWeight(Q8_0, as_q8_0(blocks, N, K), N, K)
    x = synth.normal(0xE301 + M, (M, K), 1.0)
    xb = synth.to_bf16_bits(x)
    y = gemm_bf16(qmm, w, xb)
    assert np.array_equal(y.view(np.uint32), gemm_bf16(qmm, w0, xb).view(np.uint32))
    assert_parity(y, orc.linear_bf16x_f64(Q8_K, blocks, N, K, xb), TOL, f"bf16 N={N} K={K} M={M}")
    assert_parity(qmm.linear(x, w), orc.linear_f64(Q8_K, blocks, N, K, x), TOL, f"f32 N={N} K={K} M={M}")


@pytest.mark.parametrize("offset", [0, 1, 2, 3, 6])
def test_q8k_upload_from_device_any_alignment(qmm, orc, offset):
    """Repack from super-blocks already in HBM at any byte offset, with 0xA5 around the
    source (a byte read from outside it would change the result): an odd super-block
    count and a ragged last row tile; the GEMV equals the host-uploaded weight's bit
    for bit."""
    N, K = 37, 256 * 9
    blocks = synth.kquant_blocks(Q8_K, N, K, seed=0xE400 + offset)
    staged = np.full(blocks.size + 16, 0xA5, dtype=np.uint8)
    staged[offset: offset + blocks.size] = blocks
    dbuf = qmm.DeviceBuffer.from_numpy(staged)
    view = qmm.DeviceBuffer.__new__(qmm.DeviceBuffer)
    view.nbytes, view.ptr = blocks.size, ctypes.c_void_p(dbuf.ptr.value + offset)
    w_dev = qmm.QuantizedWeight.from_device(Q8_K, view, blocks.size, N, K)
    view.ptr = ctypes.c_void_p()  # not owned
    w_host = qmm.QuantizedWeight(Q8_K, blocks, N, K)
    x = synth.normal(0xE401, (5, K), 1.0)
    y = gemv_nan_filled(qmm, w_dev, x)
    assert np.array_equal(y.view(np.uint32), gemv_nan_filled(qmm, w_host, x).view(np.uint32))
    assert_parity(y, orc.linear_f64(Q8_K, blocks, N, K, x), TOL, f"offset {offset}")


def test_q8k_from_gguf_file(qmm, tmp_path):
    """A Q8_K projection read from a GGUF file uploads as its raw super-blocks and gives
    exactly what the same bytes give through openmini_qmm_upload."""
    N, K = 96, 1536
    blocks = synth.kquant_blocks(Q8_K, N, K, seed=0xE500)
    path = tmp_path / "q8k.gguf"
    path.write_bytes(fx.build([("general.architecture", fx.STRING, "llama")],
                              [("model.layers.0.ffn.up_proj", [K, N], Q8_K, blocks.tobytes())], "standard"))
    w_file = G.GgufFile(str(path)).upload_weight("model.layers.0.ffn.up_proj")
    w_direct = qmm.QuantizedWeight(Q8_K, blocks, N, K)
    x = synth.normal(0xE501, (3, K), 1.0)
    assert np.array_equal(gemv_nan_filled(qmm, w_file, x), gemv_nan_filled(qmm, w_direct, x))
