"""Pins the CPU oracle (oracle/qmm_oracle.c) before any GPU result is compared to it.

Each check is chosen so a plausible mistake fails it: the reference's own known
answers (tests/golden/reference_kats.json, transcribed with file:line), exhaustive
or library comparisons for the float conversions (numpy float16), an asymmetric
nibble KAT for the element order the reference source fixes, hand-computed
quantizer blocks, and numpy float64 matmul for the contraction.
"""
import json
import os

import numpy as np
import pytest

from openmini_qmm import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
KATS = json.load(open(os.path.join(GOLDEN, "reference_kats.json")))
Q4_0, Q8_0 = 2, 7


# ---- float conversions ----------------------------------------------------------------

def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(orc):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25,
                  1.5 * 2.0 ** -25, 2.0 ** -14, 0.1, 0.2, 100.0, np.inf, -np.inf], dtype=np.float32),
        # exact halfway cases between fp16 neighbours
        (np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_rne(orc):
    # hand-checked: ties to even on both sides, carry into the exponent
    cases = {0x3F800000: 0x3F80, 0x3F808000: 0x3F80, 0x3F818000: 0x3F82, 0x3F808001: 0x3F81,
             0x3F7FFFFF: 0x3F80, 0x7F7FFFFF: 0x7F80, 0x80000000: 0x8000, 0xBF808000: 0xBF80}
    for f_bits, b in cases.items():
        f = np.array([f_bits], dtype=np.uint32).view(np.float32)[0]
        assert orc.f32_to_bf16(float(f)) == b
        assert int(synth.to_bf16_bits(np.array([f]))[0]) == b
    rng = np.random.default_rng(3)
    v = rng.standard_normal(5000).astype(np.float32)
    assert np.array_equal(orc.f32_to_bf16_array(v), synth.to_bf16_bits(v))


# ---- reference known answers ------------------------------------------------------------

@pytest.mark.parametrize("case", KATS["dequantize"], ids=lambda c: c["src"].split()[-1])
def test_reference_dequantize_kats(orc, case):
    data = bytes.fromhex(case["hex"])
    out = orc.dequantize(case["type"], data, case["n"])
    assert out.size == case["expect_len"]
    if "expect_prefix" in case:
        exp = np.array(case["expect_prefix"], dtype=np.float32)
        assert np.all(np.abs(out[: exp.size] - exp) <= case["tol"])
    if case.get("all_zero"):
        assert np.all(out == 0.0)
    if "all_value" in case:
        assert np.all(out == np.float32(case["all_value"]))


@pytest.mark.parametrize("case", KATS["safe_dequantize"], ids=lambda c: c["src"].split()[1])
def test_reference_safe_dequantize_kats(orc, case):
    data = bytes.fromhex(case["hex"])
    st, out, expected = orc.safe_dequantize(case["type"], data, case["n"])
    if case["ok"]:
        assert st == 0 and out.size == case["expect_len"]
        if "abs_below" in case:
            assert np.all(np.isfinite(out)) and np.all(np.abs(out) < case["abs_below"])
    else:
        assert st == 1 and expected == case["expected"] and len(data) == case["actual"]


def test_reference_truncated_inputs(orc):
    spec = KATS["truncated"]
    full = orc.create_test_q4_0_data(spec["n"])
    assert full.size == 36
    for ln in spec["lengths"]:
        st, _, expected = orc.safe_dequantize(Q4_0, full[:ln], spec["n"])
        if ln >= spec["ok_from"]:
            assert st == 0
        else:
            assert st == 1 and expected == 36


def test_reference_non_aligned_sizes(orc):
    for n in KATS["non_aligned_sizes"]["sizes"]:
        for qt, gen in ((Q4_0, orc.create_test_q4_0_data), (Q8_0, orc.create_test_q8_0_data)):
            st, out, _ = orc.safe_dequantize(qt, gen(n), n)
            assert st == 0 and out.size == n and np.all(np.isfinite(out))


def test_unsupported_type(orc):
    # tests/quant_simd_regression_test.rs:271-273: safe_dequantize(&[], Q2K, 32) is an error
    st, _, _ = orc.safe_dequantize(10, b"", 32)
    assert st == 2


@pytest.mark.parametrize("case", KATS["geometry"], ids=lambda c: str(c["type"]))
def test_reference_geometry(orc, case):
    L = orc.lib()
    assert L.orc_bytes_per_block(case["type"]) == case["bytes_per_block"]
    assert L.orc_block_size(case["type"]) == case["block_size"]


def test_data_size_closed_form(orc):
    for qt, bpb in ((Q4_0, 18), (Q8_0, 34)):
        for n in (0, 1, 31, 32, 33, 4096 * 4096, 4096 * 11008):
            assert orc.data_size(qt, n) == (n + 31) // 32 * bpb
    assert orc.data_size(Q4_0, 4096 * 11008) == 25_362_432
    assert orc.data_size(Q8_0, 4096 * 11008) == 47_906_816


@pytest.mark.parametrize("case", KATS["f16"], ids=lambda c: c["src"].split()[-1])
def test_reference_f16_kats(orc, case):
    for b, v in zip(case["bits"], case["values"]):
        assert orc.f16_to_f32(b) == v


def test_q4_0_nibble_order_asymmetric(orc):
    # quant.rs:179-188: element 2j = (qs[j] >> 4) - 8, element 2j+1 = (qs[j] & 0xF) - 8.
    blk = bytes([0x00, 0x3C, 0x1F, 0xA0]) + bytes(14)  # d = 1.0
    out = orc.dequantize(Q4_0, blk, 32)
    assert out[:4].tolist() == [1 - 8, 15 - 8, 10 - 8, 0 - 8]
    assert np.all(out[4:] == -8.0)
    # a scale of 0.5 (0x3800) multiplies once: (q - 8) * 0.5
    blk = bytes([0x00, 0x38, 0x9E]) + bytes(15)
    out = orc.dequantize(Q4_0, blk, 2)
    assert out.tolist() == [0.5, 3.0]


def test_q8_0_sign_and_scale(orc):
    blk = bytes([0x00, 0xC0]) + bytes([0x80, 0x7F, 0xFF, 0x01]) + bytes(28)  # d = -2.0
    out = orc.dequantize(Q8_0, blk, 4)
    assert out.tolist() == [256.0, -254.0, 2.0, -2.0]


def _numpy_dequant(qtype, data, n):
    """Vectorised restatement (independent of the C loop structure)."""
    bpb = 18 if qtype == Q4_0 else 34
    nblk = len(data) // bpb
    a = np.frombuffer(bytes(data[: nblk * bpb]), dtype=np.uint8).reshape(nblk, bpb)
    d = a[:, :2].copy().view(np.float16).astype(np.float32)
    if qtype == Q4_0:
        q = np.empty((nblk, 32), dtype=np.int32)
        q[:, 0::2] = (a[:, 2:] >> 4).astype(np.int32) - 8
        q[:, 1::2] = (a[:, 2:] & 15).astype(np.int32) - 8
    else:
        q = a[:, 2:].view(np.int8).astype(np.int32)
    out = np.zeros(n, dtype=np.float32)
    v = (q.astype(np.float32) * d).ravel()
    m = min(n, v.size)
    out[:m] = v[:m]
    return out


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_dequant_vs_vectorised_restatement(orc, qtype):
    rng = np.random.default_rng(11)
    gen = orc.create_test_q4_0_data if qtype == Q4_0 else orc.create_test_q8_0_data
    for n in (1, 33, 1000, 4096):
        data = gen(n)
        assert np.array_equal(orc.dequantize(qtype, data, n).view(np.uint32),
                              _numpy_dequant(qtype, data, n).view(np.uint32))
    bpb = 18 if qtype == Q4_0 else 34
    raw = rng.integers(0, 256, 64 * bpb, dtype=np.uint8)
    raw[1::bpb] &= 0x7B  # keep scales finite
    for n in (64 * 32, 64 * 32 - 5):
        assert np.array_equal(orc.dequantize(qtype, raw, n).view(np.uint32),
                              _numpy_dequant(qtype, raw, n).view(np.uint32))


# ---- SoA repack (the reference's only layout conversion) ---------------------------------

@pytest.mark.parametrize("case", KATS["soa"], ids=lambda c: str(c["type"]))
def test_reference_soa_kats(orc, case):
    data = bytes.fromhex(case["block_hex"]) * case["blocks"]
    soa = orc.convert_to_soa(case["type"], data, case["n"])
    assert soa.size == case["expect_len"]
    if "expect_prefix_hex" in case:
        p = bytes.fromhex(case["expect_prefix_hex"])
        assert bytes(soa[: len(p)]) == p


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, 3])
def test_soa_is_the_position_major_permutation(orc, qtype):
    """numpy restatement: the fp16 fields of every block (scale; Q4_1 also min) field by
    field, then the code bytes position-major; a short input reads as zeros."""
    bpb = {Q4_0: 18, Q8_0: 34, 3: 20}[qtype]
    hdr = 4 if qtype == 3 else 2
    nblk = 7
    raw = np.random.default_rng(5).integers(0, 256, nblk * bpb, dtype=np.uint8)
    soa = orc.convert_to_soa(qtype, raw, nblk * 32)
    blocks = raw.reshape(nblk, bpb)
    fields = np.concatenate([blocks[:, f:f + 2].reshape(-1) for f in range(0, hdr, 2)])
    assert np.array_equal(soa[: hdr * nblk], fields)
    assert np.array_equal(soa[hdr * nblk:].reshape(bpb - hdr, nblk), blocks[:, hdr:].T)
    # ragged n: ceil(n / 32) blocks; code bytes past the input are zeros, and an fp16
    # field is copied only when both of its bytes are there (quant_simd.rs:3339-3343)
    for cut in (bpb + 1, bpb + 3):
        short = orc.convert_to_soa(qtype, raw[:cut], 2 * 32 - 5)
        padded = np.concatenate([raw[:cut], np.zeros(2 * bpb - cut, np.uint8)]).reshape(2, bpb)
        fld = [padded[:, f:f + 2].copy() for f in range(0, hdr, 2)]
        for i, f in enumerate(range(0, hdr, 2)):
            if bpb + f + 2 > cut:
                fld[i][1] = 0
        want = np.concatenate([x.reshape(-1) for x in fld] + [padded[:, hdr:].T.reshape(-1)])
        assert np.array_equal(short, want), cut
    assert orc.convert_to_soa(qtype, b"", 32).size == 0
    assert orc.convert_to_soa(qtype, raw, 0).size == 0


def test_soa_copy_arms(orc):
    """F32 / F16: the first min(n * element size, len) bytes; other types: the input
    as it is (quant_simd.rs:3257-3292)."""
    raw = np.random.default_rng(6).integers(0, 256, 103, dtype=np.uint8)
    assert np.array_equal(orc.convert_to_soa(0, raw, 10), raw[:40])
    assert np.array_equal(orc.convert_to_soa(0, raw, 1000), raw)
    assert np.array_equal(orc.convert_to_soa(1, raw, 7), raw[:14])
    for t in (10, 12, 14, 8, 24):
        assert np.array_equal(orc.convert_to_soa(t, raw, 5), raw)


# ---- synthetic-weight quantizers ---------------------------------------------------------

def test_q4_0_quantizer_hand_block(orc):
    x = np.zeros(32, dtype=np.float32)
    x[0], x[1], x[2], x[3] = -0.8, 0.7, 0.05, -0.05
    blk = orc.quantize(Q4_0, x)
    d = blk[:2].copy().view(np.float16)[0]
    assert d == np.float16(0.1)                   # d = max / -8 with max = -0.8
    # codes: -0.8*10+8.5=0.5->0, 0.7*10+8.5=15.5->15, 0.05*10+8.5=9.0->9, -0.5+8.5=8.0->8
    assert blk[2] == (0 << 4) | 15 and blk[3] == (9 << 4) | 8
    assert np.all(blk[4:] == 0x88)
    assert np.array_equal(blk, synth.quantize_q4_0(x))


def test_q8_0_quantizer_hand_block(orc):
    x = np.zeros(32, dtype=np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 2.5, -2.5, -0.4999
    blk = orc.quantize(Q8_0, x)
    assert blk[0] == 0x00 and blk[1] == 0x3C      # d = 1.0
    assert blk[2:6].view(np.int8).tolist() == [127, 3, -3, 0]  # round half away from zero
    assert np.array_equal(blk, synth.quantize_q8_0(x))
    assert np.all(orc.quantize(Q8_0, np.zeros(32, np.float32))[2:] == 0)


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_quantizer_round_trip_bounds(orc, qtype):
    x = synth.normal(123, (64, 256), 0.02)
    blocks = orc.quantize(qtype, x)
    assert np.array_equal(blocks, synth.quantize(qtype, x))
    w = orc.dequantize(qtype, blocks, x.size).reshape(-1, 32)
    d = np.abs(blocks.reshape(-1, 18 if qtype == Q4_0 else 34)[:, :2].copy().view(np.float16)
               .astype(np.float32))
    err = np.abs(w - x.reshape(-1, 32))
    # rounding to the nearest code (Q4_0: a value at -max clamps from code 16 to 15,
    # a full step), plus the fp16 rounding of the scale (<= 2^-11 relative)
    steps = 8.0 if qtype == Q4_0 else 127.0
    half = 1.0 if qtype == Q4_0 else 0.5
    assert np.all(err <= d * (half + steps * 2.0 ** -10))
    if qtype == Q4_0:
        assert np.mean(err <= d * (0.5 + steps * 2.0 ** -10)) > 0.99


# ---- the contraction -----------------------------------------------------------------------

@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_linear_f64_matches_numpy_float64(orc, qtype):
    N, K, B = 40, 256, 3
    blocks = synth.weight_blocks(qtype, N, K, seed=9)
    x = synth.normal(10, (B, K), 1.0)
    w = orc.dequantize(qtype, blocks, N * K).reshape(N, K).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    got = orc.linear_f64(qtype, blocks, N, K, x)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    xb = synth.to_bf16_bits(x)
    got_b = orc.linear_bf16x_f64(qtype, blocks, N, K, xb)
    ref_b = synth.bf16_bits_to_f32(xb).astype(np.float64) @ w.T
    assert np.allclose(got_b, ref_b, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("qtype", [12, 14])
def test_linear_f64_kquant_rows(orc, qtype):
    """K-quant weights: row n of W[N, K] is its own K / 256 super-blocks (GGUF ne0 = K
    contiguous).  Each output must equal the fp64 dot of x with that row dequantized on
    its own, so a row stride of K / 32 blocks (the Q4_0 geometry) fails."""
    N, K, B = 6, 768, 2
    bpb = 144 if qtype == 12 else 210
    blocks = synth.kquant_blocks(qtype, N, K, seed=21 + qtype)
    x = synth.normal(22, (B, K), 1.0)
    got = orc.linear_f64(qtype, blocks, N, K, x)
    row_bytes = K // 256 * bpb
    for n in range(N):
        wr = orc.dequantize(qtype, blocks[n * row_bytes:(n + 1) * row_bytes], K).astype(np.float64)
        assert np.allclose(got[:, n], x.astype(np.float64) @ wr, rtol=1e-12, atol=1e-12), n


def test_linear_closed_form(orc):
    # every code 0x99 -> q = 9 - 8 = 1, d = 0.5: w = 0.5 everywhere; x = 1 -> y = 0.5 K
    K, N = 96, 3
    blocks = (bytes([0x00, 0x38]) + bytes([0x99]) * 16) * (N * K // 32)
    y = orc.linear_f64(Q4_0, np.frombuffer(blocks, np.uint8), N, K, np.ones((1, K), np.float32))
    assert np.all(y == 0.5 * K)


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_cpu_baselines_agree_with_oracle(orc, qtype):
    N, K = 64, 512
    blocks = synth.weight_blocks(qtype, N, K, seed=21)
    x = synth.normal(22, (2, K), 1.0)
    ref = orc.linear_f64(qtype, blocks, N, K, x)
    w = orc.dequantize(qtype, blocks, N * K).reshape(N, K)
    scratch = np.empty(N * K, dtype=np.float32)
    for tc in (False, True):
        y = orc.cpu_asrun_linear(w, x, scratch, tc)
        assert np.max(np.abs(y - ref)) <= 1e-4 * np.max(np.abs(ref))
    y = np.empty((2, N), dtype=np.float32)
    orc.cpu_fused_linear(qtype, blocks, N, K, x, y, 0, N)
    assert np.max(np.abs(y - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_golden_regression(orc):
    """Committed oracle outputs (tests/golden/make_golden.py) still reproduce."""
    g = np.load(os.path.join(GOLDEN, "oracle_small.npz"))
    for qtype, tag in ((Q4_0, "q4"), (Q8_0, "q8")):
        blocks, x = g[f"{tag}_blocks"], g[f"{tag}_x"]
        N, K = g[f"{tag}_shape"]
        assert np.array_equal(orc.linear_f64(qtype, blocks, int(N), int(K), x), g[f"{tag}_y"])
        assert np.array_equal(orc.dequantize(qtype, blocks, int(N * K)), g[f"{tag}_w"])


# ---- Q4_1 and the K-quant layouts (quant.rs:216-262, 338-800) --------------------------
# Each block below sets every field of its layout to a distinct value and the expected
# outputs are worked out by hand from the reference source, so a swapped nibble, a
# wrong field offset, a dropped term or a wrong sign changes at least one of them.
Q4_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 3, 10, 11, 12, 13, 14, 15


def _f16(v):
    return list(np.array([v], dtype=np.float16).view(np.uint8))


def test_q4_1_hand_block(orc):
    blk = bytearray(_f16(2.0) + _f16(-1.5) + [0] * 16)
    blk[4] = 0x3A    # elements 0, 1: q = 3, 10
    blk[19] = 0xF0   # elements 30, 31: q = 15, 0
    out = orc.dequantize(Q4_1, bytes(blk), 32)
    assert out[0] == 4.5 and out[1] == 18.5 and out[30] == 28.5 and out[31] == -1.5
    assert np.all(out[2:30] == -1.5)   # q = 0: the offset alone


def test_q4_k_hand_block_and_missing_minimum(orc):
    blk = bytearray(144)
    blk[0:2] = bytes(_f16(0.5))
    blk[2:4] = bytes(_f16(3.0))        # dmin: its term vanishes (min read past scales)
    blk[4] = 0xC5                      # sub-block 0 scale = 0xC5 & 0x3F = 5
    blk[5] = 0x02                      # sub-block 1 scale = 2
    blk[12] = 0x9F                     # elements 0, 1: q = 9, 15
    blk[12 + 16] = 0x70                # elements 32, 33: q = 7, 0
    out = orc.dequantize(Q4_K, bytes(blk), 256)
    assert out[0] == 2.5 and out[1] == 17.5 and out[32] == -1.0 and out[33] == -8.0
    assert out[2] == -20.0             # q = 0 in sub-block 0: (0 - 8) * 0.5 * 5
    assert np.all(out[64:] == 0.0)     # scales 0: (q - 8) * d * 0 + 0


def test_q5_k_hand_block(orc):
    blk = bytearray(176)
    blk[0:2] = bytes(_f16(1.0))
    blk[2:4] = bytes(_f16(0.5))
    blk[4], blk[5] = 3, 4              # scales of sub-blocks 0, 1
    blk[4 + 8] = 0x21                  # minimums: sub-block 0 low nibble 1, 1 high nibble 2
    blk[20] = 0b00000010               # qh of sub-block 0: bit 1 -> element 1 gets +16
    blk[36] = 0x5A                     # elements 0, 1: nibbles 5, 10
    blk[36 + 16] = 0x01                # elements 32, 33: nibbles 0, 1
    out = orc.dequantize(Q5_K, bytes(blk), 256)
    assert out[0] == (5 - 16) * 3 + 0.5 * 1          # -32.5
    assert out[1] == (26 - 16) * 3 + 0.5 * 1         # 30.5
    assert out[32] == (0 - 16) * 4 + 0.5 * 2         # -63
    assert out[33] == (1 - 16) * 4 + 0.5 * 2         # -59


def test_q6_k_hand_block(orc):
    blk = bytearray(210)
    blk[0:2] = bytes(_f16(0.25))
    blk[2] = 0x2F                      # elements 0, 1: low nibbles 15 (even), 2 (odd)
    blk[66] = 0b00011011               # high 2-bit fields of elements 0..3: 3, 2, 1, 0
    blk[130] = 0xFE                    # scale of elements 0..15: -2
    blk[131] = 0x03                    # scale of elements 16..31: 3
    out = orc.dequantize(Q6_K, bytes(blk), 256)
    assert out[0] == 31 * 0.25 * -2    # q = 15 | (48 - 32)
    assert out[1] == 2 * 0.25 * -2     # q = 2 | (32 - 32)
    assert out[2] == -16 * 0.25 * -2   # q = 0 | (16 - 32)
    assert out[3] == -32 * 0.25 * -2   # q = 0 | (0 - 32)
    assert out[16] == -32 * 0.25 * 3


def test_q2_k_hand_block_and_short_code_array(orc):
    blk = bytearray(68)
    blk[0:2] = bytes(_f16(1.0))
    blk[2:4] = bytes(_f16(0.5))
    blk[4], blk[20] = 3, 2             # sub-block 0: scale 3, minimum 2
    blk[4 + 4], blk[20 + 4] = 1, 0     # sub-block 4: scale 1, minimum 0
    blk[36] = 0b11100100               # elements 0..3: q = 0, 1, 2, 3
    out = orc.dequantize(Q2_K, bytes(blk), 256)
    assert list(out[:4]) == [-5.0, -2.0, 1.0, 4.0]
    # sub-block 4 starts past the 32 code bytes: q = 1 (quant.rs:645-649)
    assert np.all(out[64:80] == -1.0)


def test_q3_k_hand_block(orc):
    blk = bytearray(162)
    blk[0:2] = bytes(_f16(2.0))
    blk[2] = 0x75                      # elements 0, 1: 3-bit fields 5 and 7
    blk[66] = 0b00000100               # element 1 (bit 2) gets bit 3 set
    blk[130] = 3                       # scale of elements 0..7
    out = orc.dequantize(Q3_K, bytes(blk), 256)
    assert out[0] == (5 - 16) * 2 * 3 and out[1] == ((7 | 8) - 16) * 2 * 3
    assert out[2] == -16 * 2 * 3


def test_q8_k_hand_block(orc):
    blk = bytearray(258)
    blk[0:2] = bytes(_f16(0.5))
    blk[2], blk[3], blk[257] = 0x80, 0x7F, 0x01
    out = orc.dequantize(Q8_K, bytes(blk), 256)
    assert out[0] == -64.0 and out[1] == 63.5 and out[255] == 0.5


def test_k_quant_signed_zeros(orc):
    """All-zero blocks: the reference's operation order leaves -0.0 where no addition
    follows (Q3_K, Q6_K: (q < 0) * 0 * 0) and +0.0 where one does (Q2_K, Q4_K, Q5_K)."""
    for qt, neg in ((Q3_K, True), (Q6_K, True), (Q2_K, False), (Q4_K, False), (Q5_K, False)):
        out = orc.dequantize(qt, bytes(orc.BYTES_PER_BLOCK[qt]), 256)
        assert np.all(out == 0.0) and np.all(np.signbit(out) == neg), qt


@pytest.mark.parametrize("qt", [Q4_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K])
def test_short_input_stops_at_first_incomplete_block(orc, qt):
    bpb, bs = orc.BYTES_PER_BLOCK[qt], orc.BLOCK_SIZE[qt]
    rng = np.random.default_rng(qt)
    data = rng.integers(0, 256, 3 * bpb, dtype=np.uint8)
    data[1::max(bpb // 2, 1)] &= 0x3B  # keep fp16 scales finite-ish
    full = orc.dequantize(qt, data, 3 * bs)
    part = orc.dequantize(qt, data[: 2 * bpb + bpb // 2], 3 * bs)
    assert np.array_equal(part[: 2 * bs].view(np.uint32), full[: 2 * bs].view(np.uint32))
    assert np.all(part[2 * bs:] == 0.0)


def test_safe_dequantize_q4_1_regression_generator(orc):
    # tests/quant_simd_regression_test.rs:257-275: sizes 32..256 are Ok and finite
    for n in (32, 64, 128, 256):
        st, out, _ = orc.safe_dequantize(Q4_1, orc.create_test_q4_1_data(n), n)
        assert st == 0 and out.size == n and np.all(np.isfinite(out))
    # block 1 of the generator: d = f16(0.165), m = f16(-0.9), byte j = (16 + j) % 16 twice
    data = orc.create_test_q4_1_data(64)
    d = np.float32(np.float16(np.float32(0.15) + np.float32(0.015)))
    m = np.float32(np.float16(np.float32(-1.0) + np.float32(0.1)))
    out = orc.dequantize(Q4_1, data, 64)
    assert out[32 + 2 * 5] == np.float32(np.float32(5) * d) + m


def test_silu_pins(orc):
    """silu(v) = v / (1 + exp(-v)) (model.rs:1187-1189): fixed points, the odd-part
    identity silu(v) - silu(-v) = v, and v * expit(v) from scipy."""
    from scipy.special import expit
    assert orc.silu_f64(0.0) == 0.0
    assert orc.silu_f64(1.0) == 1.0 / (1.0 + np.exp(-1.0))
    assert orc.silu_f64(-1000.0) == 0.0 and np.signbit(orc.silu_f64(-1000.0))
    assert orc.silu_f64(1000.0) == 1000.0
    v = np.random.default_rng(5).normal(0.0, 4.0, 10_000)
    np.testing.assert_allclose(orc.silu_f64(v) - orc.silu_f64(-v), v, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(orc.silu_f64(v), v * expit(v), rtol=1e-13, atol=1e-300)


def test_ffn_hidden_composition(orc):
    """silu(g) * u over the oracle's own linear layers: a swapped gate / up (the
    gate * silu(up) mistake) fails it."""
    from scipy.special import expit
    from openmini_qmm import synth
    N, K = 48, 256
    wg = synth.weight_blocks(Q4_0, N, K, seed=1)
    wu = synth.weight_blocks(Q4_0, N, K, seed=2)
    x = synth.normal(3, (2, K), 1.0)
    g = orc.linear_f64(Q4_0, wg, N, K, x)
    u = orc.linear_f64(Q4_0, wu, N, K, x)
    h = orc.ffn_hidden_f64(Q4_0, wg, wu, N, K, x)
    np.testing.assert_allclose(h, g * expit(g) * u, rtol=1e-12)
    assert not np.allclose(h, u * expit(u) * g, rtol=1e-3)


def test_f32_f16_short_input_kat(orc):
    """KAT: F32 / F16 bytes holding fewer than n whole elements -> those elements, then
    0.0 (dequantize_simd's fixed-length result, quant_simd.rs:332-340; quant.rs:95-133
    returns the same leading values without the tail)."""
    f32 = np.array([1.0, -2.5, 3.25], np.float32).tobytes() + bytes([0x00, 0x00, 0x80])
    got = orc.dequantize(0, np.frombuffer(f32, np.uint8), 6)
    assert np.array_equal(got.view(np.uint32),
                          np.array([1.0, -2.5, 3.25, 0, 0, 0], np.float32).view(np.uint32))
    f16 = np.array([1.0, -0.5], np.float16).tobytes() + bytes([0x3C])
    got = orc.dequantize(1, np.frombuffer(f16, np.uint8), 4)
    assert np.array_equal(got.view(np.uint32), np.array([1.0, -0.5, 0, 0], np.float32).view(np.uint32))
