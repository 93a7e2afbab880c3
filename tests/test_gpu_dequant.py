"""GPU dequantization and upload/repack: bit-exact against the oracle.

Reference semantics: quant::dequantize_q4_0 / _q8_0 (src/model/inference/quant.rs:152-195,
282-316) and quant_simd::safe_dequantize (quant_simd.rs:150-241, 284-302).
"""
import json
import os

import numpy as np
import pytest

from openmini_qmm import synth

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7
BPB = {Q4_0: 18, Q8_0: 34}
KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def random_blocks(qtype, nblocks, seed, finite=True):
    raw = np.random.default_rng(seed).integers(0, 256, nblocks * BPB[qtype], dtype=np.uint8)
    if finite:
        raw[1::BPB[qtype]] &= 0x7B  # fp16 exponent never all-ones
    return raw


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("shape", [(1, 32), (3, 96), (37, 4160), (256, 4096), (4096, 4096),
                                   (11008, 4096), (4096, 11008)])
def test_upload_then_dequant_is_bit_exact(qmm, orc, qtype, shape):
    N, K = shape
    print(f"dequant_weight type={qtype} N={N} K={K}", flush=True)
    blocks = synth.weight_blocks(qtype, N, K, seed=N * 7 + K + qtype)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    info = w.info()
    assert (info.n_rows, info.k_cols, info.blocks_per_row) == (N, K, K // 32)
    assert info.gguf_bytes == blocks.size
    got = w.dequantize()
    ref = orc.dequantize(qtype, blocks, N * K).reshape(N, K)
    assert np.array_equal(bits(got), bits(ref))
    w.close()


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_random_bytes_bit_exact_including_signed_zero(qmm, orc, qtype):
    # every code value and many scales, including zero scales (-0.0 from (q-8) * +0)
    nblk = 5000
    raw = random_blocks(qtype, nblk, seed=qtype)
    raw[:BPB[qtype] * 10:BPB[qtype]] = 0
    raw[1:BPB[qtype] * 10:BPB[qtype]] = 0
    w = qmm.QuantizedWeight(qtype, raw, 50, nblk * 32 // 50)
    got = w.dequantize().ravel()
    ref = orc.dequantize(qtype, raw, nblk * 32)
    assert np.array_equal(bits(got), bits(ref))
    # the same bytes through the raw-GGUF (GpuQuantOps) path
    assert np.array_equal(bits(qmm.safe_dequantize(raw, qtype, nblk * 32)), bits(ref))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_non_finite_scales_propagate(qmm, orc, qtype):
    raw = random_blocks(qtype, 64, seed=99, finite=False)
    raw[1::BPB[qtype]] |= 0x7C  # exponent all ones: inf / nan scales
    got = qmm.safe_dequantize(raw, qtype, 64 * 32)
    ref = orc.dequantize(qtype, raw, 64 * 32)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin], ref[fin])


@pytest.mark.parametrize("case", KATS["dequantize"], ids=lambda c: c["src"].split()[-1])
def test_reference_kats_on_gpu(qmm, orc, case):
    data = bytes.fromhex(case["hex"])
    need = (case["n"] + 31) // 32 * BPB[case["type"]]
    if len(data) < need:
        # quant::dequantize zero-fills; the safe GPU API reports InsufficientData
        with pytest.raises(qmm.InsufficientData) as ei:
            qmm.safe_dequantize(data, case["type"], case["n"])
        assert ei.value.expected == need and ei.value.actual == len(data)
        return
    got = qmm.safe_dequantize(data, case["type"], case["n"])
    assert got.size == case["expect_len"]
    assert np.array_equal(bits(got), bits(orc.dequantize(case["type"], data, case["n"])))
    if "expect_prefix" in case:
        exp = np.array(case["expect_prefix"], dtype=np.float32)
        assert np.all(np.abs(got[: exp.size] - exp) <= case["tol"])


@pytest.mark.parametrize("case", KATS["safe_dequantize"], ids=lambda c: c["src"].split()[1])
def test_reference_safe_kats_on_gpu(qmm, case):
    data = bytes.fromhex(case["hex"])
    if case["ok"]:
        out = qmm.safe_dequantize(data, case["type"], case["n"])
        assert out.size == case["expect_len"]
        if "abs_below" in case:
            assert np.all(np.isfinite(out)) and np.all(np.abs(out) < case["abs_below"])
    else:
        with pytest.raises(qmm.InsufficientData) as ei:
            qmm.safe_dequantize(data, case["type"], case["n"])
        assert (ei.value.expected, ei.value.actual) == (case["expected"], case["actual"])


def test_reference_generators_non_aligned_and_truncated(qmm, orc):
    for n in KATS["non_aligned_sizes"]["sizes"] + [1_000_000]:
        for qt, gen in ((Q4_0, orc.create_test_q4_0_data), (Q8_0, orc.create_test_q8_0_data)):
            data = gen(n) if n < 10_000 else np.tile(gen(32 * 64), (n + 2047) // 2048)
            got = qmm.safe_dequantize(data, qt, n)
            assert got.size == n
            assert np.array_equal(bits(got), bits(orc.dequantize(qt, data, n)))
    spec = KATS["truncated"]
    full = orc.create_test_q4_0_data(spec["n"])
    for ln in spec["lengths"]:
        if ln >= spec["ok_from"]:
            assert qmm.safe_dequantize(full[:ln], Q4_0, spec["n"]).size == spec["n"]
        else:
            with pytest.raises(qmm.InsufficientData):
                qmm.safe_dequantize(full[:ln], Q4_0, spec["n"])


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("offset", [0, 2, 6])
def test_upload_from_device_any_alignment(qmm, orc, qtype, offset):
    """Repack from blocks already in HBM, including sources that are not 16-byte
    aligned (GGUF data offsets are only guaranteed 32-aligned in the file)."""
    N, K = 300, 4096 + 32 * 3
    blocks = synth.weight_blocks(qtype, N, K, seed=offset + qtype)
    staged = np.zeros(blocks.size + 16, dtype=np.uint8)
    staged[offset: offset + blocks.size] = blocks
    dbuf = qmm.DeviceBuffer.from_numpy(staged)
    import ctypes
    view = qmm.DeviceBuffer.__new__(qmm.DeviceBuffer)
    view.nbytes, view.ptr = blocks.size, ctypes.c_void_p(dbuf.ptr.value + offset)
    w = qmm.QuantizedWeight.from_device(qtype, view, blocks.size, N, K)
    view.ptr = ctypes.c_void_p()  # not owned
    got = w.dequantize()
    ref = orc.dequantize(qtype, blocks, N * K).reshape(N, K)
    assert np.array_equal(bits(got), bits(ref))


def test_gpu_quant_ops_mirror(qmm, orc):
    ops = qmm.HipQuantOps()
    assert ops.is_available()
    assert "gfx950" in ops.device_info()
    data = orc.create_test_q4_0_data(256)
    assert np.array_equal(bits(ops.dequantize_q4_0_gpu(data, 256)), bits(orc.dequantize(Q4_0, data, 256)))
    data8 = orc.create_test_q8_0_data(256)
    outs = ops.batch_dequantize_gpu([(Q4_0, data, 256), (Q8_0, data8, 256)])
    assert np.array_equal(bits(outs[1]), bits(orc.dequantize(Q8_0, data8, 256)))
    with pytest.raises(ops.GpuQuantOpsError):
        ops.dequantize_q8_0_gpu(bytes(10), 32)
    with pytest.raises(ops.GpuQuantOpsError):
        ops.dequantize_q4_1_gpu(bytes(20), 32)
