"""Decode GEMV on the block-minimum weight types, read the way the reference reads them:
Q4_1 q * d + m (openmini-server/src/model/inference/quant.rs:216-262) and Q5_K
(q - 16) * d * scale + dmin * minimum (quant.rs:433-505, the reference's own reading
of the 176-byte super-block), against the fp64 oracle over orc_dequantize_q4_1 /
_q5_k (model.rs:1050-1064 semantics, y = x . W^T; tolerance from tests/parity.py).

Each block's product gains min * (sum of the block's activations); the prefill GEMM
does not take these types, so linear() runs the GEMVs at any row count and the GEMM
entry points refuse them."""
import ctypes

import numpy as np
import pytest

from openmini_qmm import _native, synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_1, Q5_K, Q6_K = 3, 13, 14
BPB = {Q4_1: 20, Q5_K: 176}


def blocks_of(qtype, N, K, seed):
    if qtype == Q4_1:
        return synth.quantize_q4_1(synth.normal(seed, (N, K), 0.02))
    return synth.kquant_blocks(qtype, N, K, seed=seed)


def gemv_nan_filled(qmm, w, x):
    B = x.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x))
    dy = qmm.DeviceBuffer(B * w.n_rows * 4)
    dy.fill(0xFF)  # NaN: an output the kernel does not write fails the check
    w.gemv(dx, dy, B)
    return dy.download(np.float32, (B, w.n_rows))


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
@pytest.mark.parametrize("N,K", [(1, 256), (37, 512), (300, 2304), (777, 4096)])
@pytest.mark.parametrize("B", [1, 2, 3, 4, 7, 16])
def test_minfmt_gemv_parity(qmm, orc, qtype, N, K, B):
    """Both decode kernels (1-3 rows: the single-row kernel; 4+: the batched one), ragged
    N, every output checked with y NaN-filled first."""
    print(f"minfmt gemv type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = blocks_of(qtype, N, K, 0xD100 + N + K)
    x = synth.normal(0xD101 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = gemv_nan_filled(qmm, w, x)
    assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"type={qtype} N={N} K={K} B={B}")


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
@pytest.mark.parametrize("N,K,B", [(11008, 4096, 1), (4096, 11008, 1), (11008, 4096, 8), (4096, 11008, 8),
                                   (8192, 8192, 4), (8192, 8192, 16), (1024, 8192, 16)])
def test_minfmt_gemv_llama_shapes(qmm, orc, qtype, N, K, B):
    """The launch shapes of the Llama projections: several tiles per workgroup, the
    single-row kernel's 16-wave phases (4096 x 11008 Q4_1), the batched K split (4096-
    and 8192-row weights) and its four-way split (1024 rows)."""
    print(f"minfmt llama type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = blocks_of(qtype, N, K, 0xD200 + N)
    x = synth.normal(0xD201 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = gemv_nan_filled(qmm, w, x)
    assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"type={qtype} N={N} K={K} B={B}")


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
def test_minfmt_batch_rows_independent(qmm, qtype):
    """A row's result in the batched kernel depends neither on the other rows nor on
    the batch size (each row's activation-block sums are its own): rows of a 16-row call
    equal 4- and 8-row calls of the same rows bit for bit, with a loud neighbour."""
    N, K = 777, 2048
    w = qmm.QuantizedWeight(qtype, blocks_of(qtype, N, K, 0xD300), N, K)
    x = synth.normal(0xD301, (16, K), 1.0)
    x[3] *= 1e5
    y16 = gemv_nan_filled(qmm, w, x)
    for lo, hi in ((0, 4), (8, 16), (4, 12)):
        print(f"minfmt rows {lo}..{hi - 1} of 16", flush=True)
        assert np.array_equal(y16[lo:hi].view(np.uint32), gemv_nan_filled(qmm, w, x[lo:hi]).view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
@pytest.mark.parametrize("B", [2, 6])
def test_minfmt_nonfinite_row_stays_in_its_row(qmm, orc, qtype, B):
    """An inf in one activation row makes that row's outputs non-finite and leaves the
    others at parity (the block sum of that row is inf; no other row reads it)."""
    N, K = 300, 1024
    blocks = blocks_of(qtype, N, K, 0xD400)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(0xD401, (B, K), 1.0)
    x[1, 77] = np.inf
    y = gemv_nan_filled(qmm, w, x)
    assert not np.any(np.isfinite(y[1]))
    keep = [b for b in range(B) if b != 1]
    assert_parity(y[keep], orc.linear_f64(qtype, blocks, N, K, x[keep]), TOL, f"type={qtype} B={B}")


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_minfmt_upload_from_device_any_alignment(qmm, orc, qtype, offset):
    """Repack from blocks already in HBM at any byte offset (the staged copies need an
    aligned source and rows of whole 16-byte pieces; the others read byte by byte)."""
    N, K = 130, 4096
    blocks = blocks_of(qtype, N, K, 0xD500 + offset)
    staged = np.full(blocks.size + 16, 0xA5, dtype=np.uint8)
    staged[offset: offset + blocks.size] = blocks
    dbuf = qmm.DeviceBuffer.from_numpy(staged)
    view = qmm.DeviceBuffer.__new__(qmm.DeviceBuffer)
    view.nbytes, view.ptr = blocks.size, ctypes.c_void_p(dbuf.ptr.value + offset)
    w = qmm.QuantizedWeight.from_device(qtype, view, blocks.size, N, K)
    view.ptr = ctypes.c_void_p()  # not owned
    x = synth.normal(0xD501, (3, K), 1.0)
    assert_parity(gemv_nan_filled(qmm, w, x), orc.linear_f64(qtype, blocks, N, K, x), TOL, f"offset={offset}")


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
def test_minfmt_prefill_rows_run_the_gemv(qmm, orc, qtype):
    """linear_host at 150 rows (the fp32 GEMM's range for other types) runs the batched
    GEMV in passes of 16 rows for these types and matches the oracle; the GEMM entry
    points and the launch-shape query refuse them with UNSUPPORTED."""
    L = _native.lib()
    N, K, m = 1000, 2048, 150
    blocks = blocks_of(qtype, N, K, 0xD600)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(0xD601, (m, K), 1.0)
    y = np.full((m, N), np.nan, np.float32)
    _native.check(L.openmini_qmm_linear_host(w.handle, x.ctypes.data_as(ctypes.c_void_p),
                                             y.ctypes.data_as(ctypes.c_void_p), m))
    assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"type={qtype} m={m}")
    assert w.prefill_gemm(m) is False and w.gemm_min_rows() == 0
    dx = qmm.DeviceBuffer.from_numpy(x)
    dy = qmm.DeviceBuffer(m * N * 4)
    work = qmm.gemm_f32_workspace(m, K)
    assert L.openmini_qmm_gemm_f32(w.handle, dx.ptr, dy.ptr, m, work.ptr, work.nbytes, None) == _native.ERR_UNSUPPORTED
    assert b"no prefill GEMM" in L.openmini_qmm_last_error()
    xb = qmm.DeviceBuffer.from_numpy(synth.to_bf16_bits(x))
    assert L.openmini_qmm_gemm_bf16(w.handle, xb.ptr, dy.ptr, m, None) == _native.ERR_UNSUPPORTED
    assert L.openmini_qmm_gemm_launch_shape(w.handle, m, 0) == _native.ERR_UNSUPPORTED


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
@pytest.mark.parametrize("B", [1, 8])
def test_minfmt_ffn_gate_up_and_grouped_qkv(qmm, orc, qtype, B):
    """The layer's fused launches on these types: the (gate, up) pair writing
    silu(gate) * up (model.rs:713-735) and the grouped q / k / v GEMV."""
    from openmini_qmm import layer
    H, I = 512, 1024
    gb, ub = blocks_of(qtype, I, H, 0xD700), blocks_of(qtype, I, H, 0xD701)
    gate, up = qmm.QuantizedWeight(qtype, gb, I, H), qmm.QuantizedWeight(qtype, ub, I, H)
    x = synth.normal(0xD702 + B, (B, H), 1.0)
    dx = qmm.DeviceBuffer.from_numpy(x)
    dh = qmm.DeviceBuffer(B * I * 4)
    dh.fill(0xFF)
    layer.ffn_gate_up(gate, up, dx, dh, B)
    g, u = orc.linear_f64(qtype, gb, I, H, x), orc.linear_f64(qtype, ub, I, H, x)
    assert_parity(dh.download(np.float32, (B, I)), g / (1.0 + np.exp(-g)) * u, TOL, f"pair type={qtype} B={B}")
    qkv = [blocks_of(qtype, n, H, 0xD710 + n) for n in (512, 256, 256)]
    ws = [qmm.QuantizedWeight(qtype, b, n, H) for b, n in zip(qkv, (512, 256, 256))]
    outs = [qmm.DeviceBuffer(B * n * 4) for n in (512, 256, 256)]
    for o in outs:
        o.fill(0xFF)
    layer.gemv_multi(ws, dx, outs, B)
    for b, n, o in zip(qkv, (512, 256, 256), outs):
        assert_parity(o.download(np.float32, (B, n)), orc.linear_f64(qtype, b, n, H, x), TOL, f"qkv N={n} B={B}")


def test_minfmt_ffn_forward_mixed_types(qmm, orc):
    """A Q5_K_M-style block: gate / up in Q5_K, down in Q6_K.  At 150 rows the pair runs
    the GEMV and the down projection the fp32 GEMM, each as its own type allows."""
    from openmini_qmm import layer
    H, I, m = 512, 1024, 150
    gb, ub = blocks_of(Q5_K, I, H, 0xD800), blocks_of(Q5_K, I, H, 0xD801)
    db = synth.kquant_blocks(Q6_K, H, I, seed=0xD802)
    ffn = layer.FFNWeights(qmm.QuantizedWeight(Q5_K, gb, I, H), qmm.QuantizedWeight(Q5_K, ub, I, H),
                           qmm.QuantizedWeight(Q6_K, db, H, I))
    x = synth.normal(0xD803, (m, H), 1.0)
    y = ffn.forward(x)
    g, u = orc.linear_f64(Q5_K, gb, I, H, x), orc.linear_f64(Q5_K, ub, I, H, x)
    h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
    assert_parity(y, orc.linear_f64(Q6_K, db, H, I, h), 2 * TOL, "mixed ffn")


@pytest.mark.parametrize("qtype", [Q4_1, Q5_K])
@pytest.mark.parametrize("dialect", ["reference", "standard"])
def test_minfmt_from_gguf_file(qmm, tmp_path, qtype, dialect):
    """A Q4_1 / Q5_K projection read from a GGUF file uploads as its raw blocks and gives
    exactly what the same bytes give through openmini_qmm_upload."""
    import gguf_fixtures as fx
    from openmini_qmm import gguf as G
    N, K = 96, 1536
    blocks = blocks_of(qtype, N, K, 0xD900 + qtype)
    path = tmp_path / "mf.gguf"
    path.write_bytes(fx.build([("general.architecture", fx.STRING, "llama")],
                              [("model.layers.0.ffn.up_proj", [K, N], qtype, blocks.tobytes())], dialect))
    print(f"minfmt gguf type={qtype} dialect={dialect}", flush=True)
    w_file = G.GgufFile(str(path)).upload_weight("model.layers.0.ffn.up_proj")
    w_direct = qmm.QuantizedWeight(qtype, blocks, N, K)
    assert w_file.info().gguf_bytes == blocks.size
    x = synth.normal(0xD901, (5, K), 1.0)
    assert np.array_equal(gemv_nan_filled(qmm, w_file, x), gemv_nan_filled(qmm, w_direct, x))
