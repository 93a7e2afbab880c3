"""GPU dequantization and upload/repack: bit-exact against the oracle.

Reference semantics: quant::dequantize and its per-layout arms (src/model/inference/
quant.rs:56-800) and quant_simd::safe_dequantize (quant_simd.rs:150-302).
"""
import json
import os

import numpy as np
import pytest

from openmini_qmm import synth

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7
BPB = {Q4_0: 18, Q8_0: 34}
# every layout of the any-type entry point: type -> (block size, bytes per block)
LAYOUTS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 7: (32, 34), 10: (256, 68),
           11: (256, 162), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 258)}
SAFE = (2, 3, 7)
# byte offsets of the fp16 fields (scales, minimums) inside each block
F16_FIELDS = {2: (0,), 3: (0, 2), 7: (0,), 10: (0, 2), 11: (0,), 12: (0, 2), 13: (0, 2), 14: (0,),
              15: (0,)}
KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def random_blocks(qtype, nblocks, seed, finite=True):
    raw = np.random.default_rng(seed).integers(0, 256, nblocks * BPB[qtype], dtype=np.uint8)
    if finite:
        raw[1::BPB[qtype]] &= 0x7B  # fp16 exponent never all-ones
    return raw


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("shape", [(1, 32), (3, 96), (37, 4160), (37, 4096), (256, 4096), (4096, 4096),
                                   (11008, 4096), (4096, 11008), (1000, 11008)])
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
    t = case["type"]
    bs, bpb = LAYOUTS[t]
    need = (case["n"] + bs - 1) // bs * bpb
    ref = orc.dequantize(t, data, case["n"])
    # quant::dequantize semantics (zero tail on short input) for every layout
    got = qmm.dequantize(data, t, case["n"])
    assert got.size == case["expect_len"]
    assert np.array_equal(bits(got), bits(ref))
    if "expect_prefix" in case:
        exp = np.array(case["expect_prefix"], dtype=np.float32)
        assert np.all(np.abs(got[: exp.size] - exp) <= case["tol"])
    if "all_value" in case:
        assert np.all(got == np.float32(case["all_value"]))
    if t not in SAFE:
        return
    if len(data) < need:
        # the safe GPU API reports InsufficientData
        with pytest.raises(qmm.InsufficientData) as ei:
            qmm.safe_dequantize(data, t, case["n"])
        assert ei.value.expected == need and ei.value.actual == len(data)
        return
    assert np.array_equal(bits(qmm.safe_dequantize(data, t, case["n"])), bits(ref))


def layout_bytes(qtype, nblocks, seed, finite=True):
    bs, bpb = LAYOUTS[qtype]
    raw = np.random.default_rng(seed).integers(0, 256, nblocks * bpb, dtype=np.uint8)
    if finite:
        for f in F16_FIELDS.get(qtype, ()):
            raw[f + 1::bpb] &= 0x7B  # fp16 exponent never all-ones
        if qtype == 1:
            raw[1::2] &= 0x7B
        if qtype == 0:
            raw[3::4] &= 0x7E  # no inf / nan floats
    return raw


@pytest.mark.parametrize("qtype", sorted(LAYOUTS))
def test_every_layout_random_bytes_bit_exact(qmm, orc, qtype):
    """Random bytes in every field (scales, minimums, codes, high bits), zero scales on
    some blocks (signed zeros), a ragged n, and a short buffer (zero tail)."""
    bs, bpb = LAYOUTS[qtype]
    nblk = 3000 if bs == 256 else 20000
    raw = layout_bytes(qtype, nblk, seed=qtype + 1)
    for f in F16_FIELDS.get(qtype, ()):  # zero d / m / dmin on the first blocks
        for k in range(20):
            raw[k * bpb + f: k * bpb + f + 2] = 0
    print(f"dequantize_any type={qtype} blocks={nblk}", flush=True)
    for n in (nblk * bs, nblk * bs - bs // 2 - 3):
        got = qmm.dequantize(raw, qtype, n)
        assert np.array_equal(bits(got), bits(orc.dequantize(qtype, raw, n))), n
    short = raw[: (nblk // 2) * bpb + bpb // 3]
    got = qmm.dequantize(short, qtype, nblk * bs)
    ref = orc.dequantize(qtype, short, nblk * bs)
    assert np.array_equal(bits(got), bits(ref))
    assert np.all(got[(nblk // 2) * bs:] == 0.0)


@pytest.mark.parametrize("qtype", [3, 10, 11, 12, 13, 14, 15])
def test_every_layout_non_finite_scales(qmm, orc, qtype):
    raw = layout_bytes(qtype, 64, seed=77, finite=False)
    bpb = LAYOUTS[qtype][1]
    for f in F16_FIELDS[qtype]:
        raw[f + 1::bpb] |= 0x7C  # inf / nan scales and minimums
    n = 64 * LAYOUTS[qtype][0]
    got, ref = qmm.dequantize(raw, qtype, n), orc.dequantize(qtype, raw, n)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(bits(got[fin]), bits(ref[fin]))


@pytest.mark.parametrize("qtype", [12, 14])
def test_k_quant_llama_projection_size(qmm, orc, qtype):
    """A full 11008 x 4096 projection in the layouts real deployments use (Q4_K, Q6_K)."""
    n = 11008 * 4096
    raw = layout_bytes(qtype, n // 256, seed=qtype * 3)
    got = qmm.dequantize(raw, qtype, n)
    assert np.array_equal(bits(got), bits(orc.dequantize(qtype, raw, n)))


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
@pytest.mark.parametrize("offset", [0, 1, 2, 3, 6])
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


def test_upload_device_into_one_arena(qmm, orc):
    """openmini_qmm_upload_device_into: four weights (Q4_0, a Q8_0 with a K-split
    workspace, a Q4_K, a Q8_K with a K-split workspace) placed back to back in one
    caller allocation at 256-byte boundaries.  Each dequantizes bit-exactly (the Q4_K
    aside), and its GEMV at 1 and 8 rows equals the same weight uploaded with its own
    allocation, bit for bit.  Closing the handles
    leaves the arena to the caller, which then reuses it for another weight."""
    specs = [(Q4_0, 1000, 4096, 0xD00), (Q8_0, 4096, 11008, 0xD01), (12, 777, 2048, 0xD02),
             (15, 4096, 11008, 0xD03)]
    sizes = [qmm.weight_device_bytes(t, n, k) for t, n, k, _ in specs]
    offsets = np.cumsum([0] + [(b + 255) // 256 * 256 for b in sizes])
    arena = qmm.DeviceBuffer(int(offsets[-1]))
    arena.fill(0xA5)  # stale bytes: the repack and the split-counter clear must cover them
    own, placed = [], []
    for (t, n, k, seed), off, size in zip(specs, offsets, sizes):
        blocks = synth.kquant_blocks(t, n, k, seed=seed) if t >= 12 else synth.weight_blocks(t, n, k, seed=seed)
        d = qmm.DeviceBuffer.from_numpy(blocks)
        w = qmm.QuantizedWeight.from_device_into(t, d, blocks.size, n, k, arena, int(off))
        ref = qmm.QuantizedWeight(t, blocks, n, k)
        assert w.info().device_bytes == ref.info().device_bytes == size
        if t != 12:
            assert np.array_equal(bits(w.dequantize()), bits(orc.dequantize(t, blocks, n * k).reshape(n, k)))
        own.append(ref)
        placed.append(w)
    for (t, n, k, seed), w, ref in zip(specs, placed, own):
        for b in (1, 8):
            print(f"upload_into type={t} N={n} K={k} b={b}", flush=True)
            x = qmm.DeviceBuffer.from_numpy(synth.normal(seed + b, (b, k), 1.0))
            ya, yb = qmm.DeviceBuffer(b * n * 4), qmm.DeviceBuffer(b * n * 4)
            w.gemv(x, ya, b)
            ref.gemv(x, yb, b)
            assert np.array_equal(ya.download(np.float32, (b, n)).view(np.uint32),
                                  yb.download(np.float32, (b, n)).view(np.uint32))
    for w in placed:
        w.close()
    t, n, k, seed = specs[0]
    blocks = synth.weight_blocks(t, n, k, seed=seed + 7)
    w = qmm.QuantizedWeight.from_device_into(t, qmm.DeviceBuffer.from_numpy(blocks), blocks.size, n, k, arena,
                                             int(offsets[1]))
    assert np.array_equal(bits(w.dequantize()), bits(orc.dequantize(t, blocks, n * k).reshape(n, k)))
    w.close()
    arena.free()


def test_upload_device_into_rejects_bad_memory(qmm):
    """Memory that is unaligned, too small, or host memory is rejected with
    INVALID_PARAM and no handle."""
    import ctypes
    from openmini_qmm import _native
    L = _native.lib()
    N, K = 64, 1024
    blocks = synth.weight_blocks(Q4_0, N, K, seed=0xD10)
    d = qmm.DeviceBuffer.from_numpy(blocks)
    need = qmm.weight_device_bytes(Q4_0, N, K)
    arena = qmm.DeviceBuffer(need + 512)
    h = ctypes.c_void_p()
    host = np.zeros(need + 256, np.uint8)
    host_ptr = ctypes.c_void_p((host.ctypes.data + 255) // 256 * 256)
    for mem, size, what in ((ctypes.c_void_p(arena.ptr.value + 128), need, b"aligned"),
                            (arena.ptr, need - 1, b"needed"), (host_ptr, need, b"device memory"),
                            (ctypes.c_void_p(), need, b"aligned")):
        rc = L.openmini_qmm_upload_device_into(Q4_0, d.ptr, blocks.size, N, K, mem, size, None, ctypes.byref(h))
        assert rc == _native.ERR_INVALID_PARAM and not h.value, (rc, what)
        assert what in L.openmini_qmm_last_error(), L.openmini_qmm_last_error()
    out = ctypes.c_size_t()
    assert L.openmini_qmm_weight_device_bytes(Q4_0, N, K + 1, ctypes.byref(out)) == _native.ERR_INVALID_PARAM
    assert out.value == 0
    arena.free()


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
    data1 = orc.create_test_q4_1_data(256)
    assert np.array_equal(bits(ops.dequantize_q4_1_gpu(data1, 256)), bits(orc.dequantize(3, data1, 256)))
    with pytest.raises(ops.GpuQuantOpsError):
        ops.dequantize_q4_1_gpu(bytes(19), 32)
    # batch: any implemented layout, dequantize_simd semantics (short input: zero tail)
    kq = layout_bytes(12, 4, seed=5)
    outs = ops.batch_dequantize_gpu([(12, kq, 1024), (12, kq[:300], 1024), (14, bytes(210), 256)])
    assert np.array_equal(bits(outs[0]), bits(orc.dequantize(12, kq, 1024)))
    assert np.array_equal(bits(outs[1]), bits(orc.dequantize(12, kq[:300], 1024)))
    assert np.all(outs[1][512:] == 0.0) and np.all(np.signbit(outs[2]))
    with pytest.raises(ops.GpuQuantOpsError):
        ops.batch_dequantize_gpu([(16, bytes(64), 256)])


@pytest.mark.parametrize("qtype", [2, 12, 1])
def test_dequant_beyond_one_launch_slice(qmm, orc, qtype):
    """Tensors above 2^30 elements are dequantized in slices of 2^30 (a launch stays below
    2^32 work-items).  Around the slice boundary and at the tail the output matches the
    oracle bit for bit; with a buffer that ends inside the second slice, everything
    after the last whole block is 0.0 and everything before it is unchanged."""
    import ctypes
    from openmini_qmm import _native
    L = _native.lib()
    bs, bpb = LAYOUTS[qtype]
    S = 1 << 30
    nblk = S // bs + 4096
    n = nblk * bs
    print(f"dequantize_any_device type={qtype} n={n}", flush=True)
    raw = np.zeros(nblk * bpb, dtype=np.uint8)
    b0 = S // bs - 64  # 128 random blocks straddling the boundary, 64 at the end
    raw[b0 * bpb:(b0 + 128) * bpb] = layout_bytes(qtype, 128, seed=qtype + 900)
    raw[(nblk - 64) * bpb:] = layout_bytes(qtype, 64, seed=qtype + 901)
    d_in = qmm.DeviceBuffer.from_numpy(raw)
    d_out = qmm.DeviceBuffer(n * 4)

    def window(e0, count):
        host = np.empty(count, dtype=np.float32)
        src = ctypes.c_void_p(d_out.ptr.value + 4 * e0)
        assert L.openmini_qmm_memcpy_d2h(host.ctypes.data_as(ctypes.c_void_p), src, host.nbytes, None) == 0
        return host

    for nbytes in (raw.size, (S // bs + 10) * bpb + bpb // 2):
        d_out.fill(0xFF)  # NaN pattern: every output must be written
        assert L.openmini_qmm_dequantize_any_device(qtype, d_in.ptr, nbytes, n, d_out.ptr, None) == 0
        ref = orc.dequantize(qtype, raw[b0 * bpb:(b0 + 128) * bpb][: max(0, nbytes - b0 * bpb)], 128 * bs)
        assert np.array_equal(bits(window(b0 * bs, 128 * bs)), bits(ref)), nbytes
        tail = window(n - 64 * bs, 64 * bs)
        if nbytes == raw.size:
            assert np.array_equal(bits(tail), bits(orc.dequantize(qtype, raw[(nblk - 64) * bpb:], 64 * bs)))
        else:
            assert np.all(tail == 0.0) and not np.any(np.signbit(tail))
    d_in.free()
    d_out.free()


@pytest.mark.parametrize("qtype", [0, 1, 2, 3, 7, 12, 24])
def test_convert_to_soa_layout_matches_oracle(qmm, orc, qtype):
    """convert_to_soa_layout on the GPU (quant_simd.rs:3245-3397) byte for byte against
    the oracle: whole blocks, a ragged n, inputs cut inside a block and inside an fp16
    field, n larger than the input, and empty input."""
    bpb = {0: 4, 1: 2, 2: 18, 3: 20, 7: 34, 12: 144, 24: 1}[qtype]
    nblk = 4099
    raw = np.random.default_rng(qtype + 40).integers(0, 256, nblk * bpb, dtype=np.uint8)
    print(f"convert_to_soa type={qtype} bytes={raw.size}", flush=True)
    for data, n in ((raw, nblk * 32), (raw, nblk * 32 - 7), (raw[: 17 * bpb + 1], 17 * 32),
                    (raw[: 17 * bpb + 3], 40 * 32), (raw, nblk * 64), (raw[:0], 64), (raw, 0)):
        got = qmm.convert_to_soa_layout(data, qtype, n)
        assert np.array_equal(got, orc.convert_to_soa(qtype, data, n)), (qtype, data.size, n)


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("offset", [1, 3])
def test_device_dequantize_odd_source_address(qmm, orc, qtype, offset):
    """Raw GGUF bytes at an odd device address (a tensor of the reference's dialect can
    start at any file offset, and a device copy of the file keeps that offset): the
    any-type and the safe device entry points read the scale and codes byte by byte."""
    import ctypes
    from openmini_qmm import _native
    L = _native.lib()
    n = 32 * 777 + 5
    raw = random_blocks(qtype, (n + 31) // 32, seed=90 + offset)
    staged = np.zeros(raw.size + 16, np.uint8)
    staged[offset:offset + raw.size] = raw
    dbuf = qmm.DeviceBuffer.from_numpy(staged)
    src = ctypes.c_void_p(dbuf.ptr.value + offset)
    ref = orc.dequantize(qtype, raw, n)
    out = qmm.DeviceBuffer(n * 4)
    _native.check(L.openmini_qmm_dequantize_any_device(qtype, src, raw.size, n, out.ptr, None))
    assert np.array_equal(bits(out.download(np.float32, (n,))), bits(ref))
    out2 = qmm.DeviceBuffer(n * 4)
    _native.check(L.openmini_qmm_dequantize_device(qtype, src, raw.size, n, out2.ptr, None, None))
    assert np.array_equal(bits(out2.download(np.float32, (n,))), bits(ref))


def test_f32_f16_short_input_zero_tail(qmm, orc):
    """F32 / F16 input holding fewer than n whole elements gives those elements, then
    0.0: dequantize_simd's fixed-length result (quant_simd.rs:332-340).  The reference's
    quant::dequantize_f32 / _f16 (quant.rs:95-133) return the same leading values
    without the tail.  Stray bytes of an incomplete element are ignored."""
    f32 = np.array([1.0, -2.5, 3.25], np.float32).tobytes() + bytes([0x00, 0x00, 0x80])
    want32 = np.array([1.0, -2.5, 3.25, 0.0, 0.0, 0.0], np.float32)
    assert np.array_equal(bits(qmm.dequantize(f32, 0, 6)), bits(want32))
    assert np.array_equal(bits(orc.dequantize(0, np.frombuffer(f32, np.uint8), 6)), bits(want32))
    f16 = np.array([1.0, -0.5], np.float16).tobytes() + bytes([0x3C])
    want16 = np.array([1.0, -0.5, 0.0, 0.0], np.float32)
    assert np.array_equal(bits(qmm.dequantize(f16, 1, 4)), bits(want16))
    assert np.array_equal(bits(orc.dequantize(1, np.frombuffer(f16, np.uint8), 4)), bits(want16))
