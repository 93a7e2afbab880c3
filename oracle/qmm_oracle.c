/*
 * qmm_oracle.c -- CPU restatement of OpenMini-V1's quantized linear-layer
 * semantics.  TEST INFRASTRUCTURE ONLY: this file is the checker for the
 * HIP path.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it; the product library never links or calls it.
 *
 * Reference paths below are relative to /root/reference/openmini-server/.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   orc_f16_to_f32          exhaustive over all 65536 encodings vs numpy float16
 *   orc_f32_to_f16 / bf16   vs numpy float16 casts / an independent numpy bf16 RNE,
 *                           plus hand-checked special values
 *   orc_dequantize_*        reference KATs (quant.rs tests, quant_simd tests,
 *                           tests/quant_simd_regression_test.rs), asymmetric-nibble
 *                           KAT from quant.rs:179-190, and an independent numpy
 *                           vectorised restatement on the regression generators
 *   orc_dequantize_q4_1/_k  reference KATs where they exist (quant.rs:1499-1610,
 *                           2093-2130, quant_simd.rs:4270-4290), hand-computed blocks
 *                           for every field of each layout, and a numpy restatement
 *   orc_safe_dequantize     InsufficientData payloads of the regression tests
 *   orc_convert_to_soa      quant_simd.rs KATs (lengths 72/68/60, first scale bytes,
 *                           empty input)
 *                           plus a brute-force permutation check
 *   orc_quantize_*          not in the reference (synthetic-weight generator fixed by
 *                           BASELINE configs = ggml's textbook quantizers): pinned by
 *                           hand-computed blocks and round-trip error bounds
 *   orc_linear_f64 / bf16   numpy float64 matmul of the dequantized matrix
 *   orc_cpu_* baselines     agree with orc_linear_f64 within fp32 tolerance
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define QK 32

/* ---- scalar conversions ---------------------------------------------- */

/* IEEE binary16 -> binary32, exact.  Mirrors half 2.7.1 f16::to_f32 as used at
 * src/model/inference/quant.rs:166-167 and :296-297. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even (half 2.7.1 f16::from_f32, used by the
 * reference test generators, tests/quant_simd_regression_test.rs:36). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) { /* result subnormal or zero (|f| < 2^-14) */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;                        /* biased exponent */
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;    /* 24-bit significand */
        uint32_t shift = 126u - e;                    /* m * 2^(e-150) / 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* binary32 -> bfloat16 bits, round to nearest even; NaN stays NaN. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7FFFu + lsb;
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ---- GGUF block geometry (src/model/inference/gguf.rs:327-379, 424-438) ---- */

enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q8_0 = 7,
    ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15
};

size_t orc_block_size(int type) {
    switch (type) {
    case ORC_F32: case ORC_F16: return 1;
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q8_0: return 32;
    case ORC_Q2_K: case ORC_Q3_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K: return 256;
    default: return 0;
    }
}

size_t orc_bytes_per_block(int type) {
    switch (type) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q8_0: return 34;
    case ORC_Q2_K: return 68;
    case ORC_Q3_K: return 162;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_Q8_K: return 258;
    default: return 0;
    }
}

/* GgufTensor::data_size: ceil(n / block_size) * bytes_per_block (gguf.rs:431-438). */
size_t orc_data_size(int type, size_t n) {
    size_t bs = orc_block_size(type);
    if (bs == 0) return 0;
    return ((n + bs - 1) / bs) * orc_bytes_per_block(type);
}

/* ---- dequantization (src/model/inference/quant.rs) -------------------- */

/* quant::dequantize_q4_0, quant.rs:152-195.  Output is pre-zeroed; the loop stops at
 * the first block that does not fit in `len` bytes (:161-163) and clips at n
 * (:175-177).  Element 2j takes the HIGH nibble of byte j, element 2j+1 the LOW
 * nibble (:179-188); value = (q - 8) * f32(d) (:190). */
void orc_dequantize_q4_0(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + QK - 1) / QK;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 18;
        if (off + 18 > len) break;
        uint16_t dh = (uint16_t)(data[off] | (data[off + 1] << 8));
        float d = orc_f16_to_f32(dh);
        const uint8_t *qs = data + off + 2;
        for (size_t i = 0; i < QK; ++i) {
            size_t idx = b * QK + i;
            if (idx >= n) break;
            uint8_t byte = qs[i / 2];
            int q = (i % 2 == 0) ? (int)(byte >> 4) - 8 : (int)(byte & 0x0F) - 8;
            out[idx] = (float)q * d;
        }
    }
}

/* quant::dequantize_q8_0, quant.rs:282-316: value = f32(i8 qs[i]) * f32(d) (:310-311). */
void orc_dequantize_q8_0(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + QK - 1) / QK;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 34;
        if (off + 34 > len) break;
        uint16_t dh = (uint16_t)(data[off] | (data[off + 1] << 8));
        float d = orc_f16_to_f32(dh);
        const uint8_t *qs = data + off + 2;
        for (size_t i = 0; i < QK; ++i) {
            size_t idx = b * QK + i;
            if (idx >= n) break;
            out[idx] = (float)(int8_t)qs[i] * d;
        }
    }
}

static float f16_at(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* Every formula below is evaluated in the reference's order with one IEEE operation per
 * Rust operator (Rust does not contract a * b + c).  All its products are exact in
 * binary32, so only the final additions round. */

/* quant::dequantize_q4_1, quant.rs:216-262: 20-byte blocks [d f16][m f16][16 B codes];
 * element 2j = high nibble of byte j, 2j+1 = low nibble; value = q * d + m. */
void orc_dequantize_q4_1(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + QK - 1) / QK;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 20;
        if (off + 20 > len) break;
        float d = f16_at(data + off), m = f16_at(data + off + 2);
        const uint8_t *qs = data + off + 4;
        for (size_t i = 0; i < QK; ++i) {
            size_t idx = b * QK + i;
            if (idx >= n) break;
            float q = (float)((i % 2 == 0) ? (qs[i / 2] >> 4) : (qs[i / 2] & 0x0F));
            float prod = q * d;
            out[idx] = prod + m;
        }
    }
}

/* quant::dequantize_q4_k, quant.rs:338-410: 144-byte blocks [d][dmin][scales 8 B]
 * [codes from byte 12]; 8 sub-blocks of 32; scale = scales[sb] & 0x3F; the minimum is
 * read from scales[8 + sb / 2], past the 8-byte slice, so it is 0.0 (:360-378);
 * value = (q - 8) * d * scale + dmin * min. */
void orc_dequantize_q4_k(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 144;
        if (off + 144 > len) break;
        const uint8_t *blk = data + off;
        float d = f16_at(blk), dmin = f16_at(blk + 2);
        const uint8_t *scales = blk + 4, *qs = blk + 12;
        for (int sb = 0; sb < 8; ++sb) {
            float scale = (float)(scales[sb] & 0x3F);
            float min_val = 0.0f;
            for (int i = 0; i < 32; ++i) {
                size_t idx = b * 256 + (size_t)sb * 32 + (size_t)i;
                if (idx >= n) break;
                uint8_t byte = qs[sb * 16 + i / 2];
                float q = (float)((i % 2 == 0) ? (byte >> 4) : (byte & 0x0F));
                float t = (q - 8.0f) * d;
                t = t * scale;
                float u = dmin * min_val;
                out[idx] = t + u;
            }
        }
    }
}

/* quant::dequantize_q5_k, quant.rs:433-505: 176-byte blocks [d][dmin][scales 16 B]
 * [qh 16 B][codes from byte 36]; scale = scales[sb] & 0x3F, min = nibble (sb even: low,
 * odd: high) of scales[8 + sb / 2]; q = nibble + 16 * bit (i % 8) of qh[sb];
 * value = (q - 16) * d * scale + dmin * min. */
void orc_dequantize_q5_k(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 176;
        if (off + 176 > len) break;
        const uint8_t *blk = data + off;
        float d = f16_at(blk), dmin = f16_at(blk + 2);
        const uint8_t *scales = blk + 4, *qh = blk + 20, *qs = blk + 36;
        for (int sb = 0; sb < 8; ++sb) {
            float scale = (float)(scales[sb] & 0x3F);
            uint8_t mb = scales[8 + sb / 2];
            float min_val = (float)((sb % 2 == 0) ? (mb & 0x0F) : (mb >> 4));
            for (int i = 0; i < 32; ++i) {
                size_t idx = b * 256 + (size_t)sb * 32 + (size_t)i;
                if (idx >= n) break;
                float qh_bit = (float)((qh[sb] >> (i % 8)) & 1);
                uint8_t byte = qs[sb * 16 + i / 2];
                float q4 = (float)((i % 2 == 0) ? (byte >> 4) : (byte & 0x0F));
                float hi = qh_bit * 16.0f;
                float q = q4 + hi;
                float t = (q - 16.0f) * d;
                t = t * scale;
                float u = dmin * min_val;
                out[idx] = t + u;
            }
        }
    }
}

/* quant::dequantize_q6_k, quant.rs:515-600: 210-byte blocks [d][ql 64 B][qh 64 B]
 * [scales 32 x i8]; element i: low = nibble of ql[i / 2] (even i: low, odd: high),
 * high = 2 bits (i % 4) of qh[i / 4]; q = low | ((high << 4) - 32);
 * value = q * d * scales[i / 16]. */
void orc_dequantize_q6_k(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 210;
        if (off + 210 > len) break;
        const uint8_t *blk = data + off;
        float d = f16_at(blk);
        const uint8_t *ql = blk + 2, *qh = blk + 66, *scales = blk + 130;
        for (int i = 0; i < 256; ++i) {
            size_t idx = b * 256 + (size_t)i;
            if (idx >= n) break;
            float scale = (float)(int8_t)scales[i / 16];
            int low = (i % 2 == 0) ? (ql[i / 2] & 0x0F) : (ql[i / 2] >> 4);
            int high = (qh[i / 4] >> ((i % 4) * 2)) & 0x03;
            int q = low | ((high << 4) - 32);
            float t = (float)q * d;
            out[idx] = t * scale;
        }
    }
}

/* quant::dequantize_q2_k, quant.rs:605-660: 68-byte blocks [d][dmin][scales 16 x u8]
 * [mins 16 x u8][codes 32 B]; 16 sub-blocks of 16; code byte sb * 8 + i / 4 (past the
 * 32 code bytes from sub-block 4 on: q = 1, :645-649), 2 bits (i % 4);
 * value = (q - 2) * d * scale + dmin * min. */
void orc_dequantize_q2_k(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 68;
        if (off + 68 > len) break;
        const uint8_t *blk = data + off;
        float d = f16_at(blk), dmin = f16_at(blk + 2);
        const uint8_t *scales = blk + 4, *mins = blk + 20, *qs = blk + 36;
        for (int sb = 0; sb < 16; ++sb) {
            float scale = (float)scales[sb], min_val = (float)mins[sb];
            for (int i = 0; i < 16; ++i) {
                size_t idx = b * 256 + (size_t)sb * 16 + (size_t)i;
                if (idx >= n) break;
                int byte_idx = sb * 8 + i / 4;
                float q = byte_idx < 32 ? (float)((qs[byte_idx] >> ((i % 4) * 2)) & 0x03) : 1.0f;
                float t = (q - 2.0f) * d;
                t = t * scale;
                float u = dmin * min_val;
                out[idx] = t + u;
            }
        }
    }
}

/* quant::dequantize_q3_k, quant.rs:682-760: 162-byte blocks [d][ql 64 B][qh 64 B]
 * [scales 32 x i8]; element i: 3 bits (even i: bits 0-2, odd: bits 4-6) of ql[i / 2],
 * bit 2 (i % 4) of qh[i / 4] as bit 3; q = that - 16; value = q * d * scales[i / 8]. */
void orc_dequantize_q3_k(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 162;
        if (off + 162 > len) break;
        const uint8_t *blk = data + off;
        float d = f16_at(blk);
        const uint8_t *ql = blk + 2, *qh = blk + 66, *scales = blk + 130;
        for (int i = 0; i < 256; ++i) {
            size_t idx = b * 256 + (size_t)i;
            if (idx >= n) break;
            float scale = (float)(int8_t)scales[i / 8];
            int lb = (i % 2 == 0) ? (ql[i / 2] & 0x07) : ((ql[i / 2] >> 4) & 0x07);
            int hb = (qh[i / 4] >> ((i % 4) * 2)) & 0x01;
            int q = (lb | (hb << 3)) - 16;
            float t = (float)q * d;
            out[idx] = t * scale;
        }
    }
}

/* quant::dequantize_q8_k, quant.rs:768-800: 258-byte blocks [d][256 x i8];
 * value = q * d. */
void orc_dequantize_q8_k(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        size_t off = b * 258;
        if (off + 258 > len) break;
        float d = f16_at(data + off);
        const uint8_t *qs = data + off + 2;
        for (int i = 0; i < 256; ++i) {
            size_t idx = b * 256 + (size_t)i;
            if (idx >= n) break;
            out[idx] = (float)(int8_t)qs[i] * d;
        }
    }
}

/* quant::dequantize dispatcher, quant.rs:56-79 (the IQ types are not restated here;
 * other types -> zeros :78).  Returns 1 for a type restated here, 0 otherwise (output
 * zeroed).  F32 / F16 with fewer than n whole elements in `len`: the whole ones, then
 * 0.0 up to n -- the fixed-length result of dequantize_simd's F32 / F16 arms
 * (quant_simd.rs:304-313, dequantize_f32_impl :332-340 `vec![0.0f32; n]`).
 * quant::dequantize_f32 / _f16 (quant.rs:95-133) return the same leading values but
 * a shorter Vec (no tail). */
int orc_dequantize(int type, const uint8_t *data, size_t len, size_t n, float *out) {
    switch (type) {
    case ORC_Q4_0: orc_dequantize_q4_0(data, len, n, out); return 1;
    case ORC_Q4_1: orc_dequantize_q4_1(data, len, n, out); return 1;
    case ORC_Q8_0: orc_dequantize_q8_0(data, len, n, out); return 1;
    case ORC_Q2_K: orc_dequantize_q2_k(data, len, n, out); return 1;
    case ORC_Q3_K: orc_dequantize_q3_k(data, len, n, out); return 1;
    case ORC_Q4_K: orc_dequantize_q4_k(data, len, n, out); return 1;
    case ORC_Q5_K: orc_dequantize_q5_k(data, len, n, out); return 1;
    case ORC_Q6_K: orc_dequantize_q6_k(data, len, n, out); return 1;
    case ORC_Q8_K: orc_dequantize_q8_k(data, len, n, out); return 1;
    case ORC_F32:
        for (size_t i = 0; i < n; ++i) {
            if (4 * i + 4 <= len) memcpy(&out[i], data + 4 * i, 4); else out[i] = 0.0f;
        }
        return 1;
    case ORC_F16:
        for (size_t i = 0; i < n; ++i) {
            out[i] = (2 * i + 2 <= len)
                ? orc_f16_to_f32((uint16_t)(data[2 * i] | (data[2 * i + 1] << 8))) : 0.0f;
        }
        return 1;
    default:
        for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
        return 0;
    }
}

/* quant_simd::safe_dequantize{,_q4_0,_q8_0,_q4_1}, quant_simd.rs:150-302.
 * Returns 0 = Ok, 1 = InsufficientData{expected=*expected, actual=len},
 * 2 = UnsupportedType.  n == 0 -> Ok with empty output. */
int orc_safe_dequantize(int type, const uint8_t *data, size_t len, size_t n, float *out,
                        size_t *expected) {
    if (expected) *expected = 0;
    if (type != ORC_Q4_0 && type != ORC_Q8_0 && type != ORC_Q4_1) return 2;
    if (n == 0) return 0;
    size_t need = orc_data_size(type, n);
    if (len < need) {
        if (expected) *expected = need;
        return 1;
    }
    orc_dequantize(type, data, len, n, out);
    return 0;
}

/* quant_simd::convert_to_soa_layout (quant_simd.rs:3245-3293) and its arms
 * convert_q4_0_to_soa (:3300-3327), convert_q4_1_to_soa (:3330-3367),
 * convert_q8_0_to_soa (:3370-3397):
 *   - empty data or n == 0: nothing;
 *   - F32 / F16: the first min(n * 4 | 2, len) bytes, copied;
 *   - Q4_0 / Q8_0: [fp16 scale of every block][byte position 0 of every block] ...
 *     [last position of every block]; Q4_1: [scales][mins][16 positions]; for
 *     ceil(n / 32) blocks, bytes missing from `data` read as 0;
 *   - any other type: all of `data`, copied.
 * Returns the output length. */
size_t orc_soa_bytes(int type, size_t len, size_t n) {
    if (len == 0 || n == 0) return 0;
    if (type == ORC_F32) return n * 4 < len ? n * 4 : len;
    if (type == ORC_F16) return n * 2 < len ? n * 2 : len;
    if (type == ORC_Q4_0 || type == ORC_Q4_1 || type == ORC_Q8_0)
        return (n + QK - 1) / QK * orc_bytes_per_block(type);
    return len;
}

size_t orc_convert_to_soa(int type, const uint8_t *data, size_t len, size_t n, uint8_t *out) {
    size_t total = orc_soa_bytes(type, len, n);
    if (type != ORC_Q4_0 && type != ORC_Q4_1 && type != ORC_Q8_0) {
        memcpy(out, data, total);
        return total;
    }
    if (total == 0) return 0;
    size_t bpb = orc_bytes_per_block(type);
    size_t fields = type == ORC_Q4_1 ? 2 : 1; /* fp16 scale (and min) per block */
    size_t nq = bpb - 2 * fields;
    size_t blocks = (n + QK - 1) / QK;
    size_t o = 0;
    for (size_t f = 0; f < fields; ++f)
        for (size_t b = 0; b < blocks; ++b) {
            size_t off = b * bpb + 2 * f;
            if (off + 2 <= len) { out[o] = data[off]; out[o + 1] = data[off + 1]; }
            else { out[o] = 0; out[o + 1] = 0; }
            o += 2;
        }
    for (size_t pos = 0; pos < nq; ++pos)
        for (size_t b = 0; b < blocks; ++b) {
            size_t off = b * bpb + 2 * fields + pos;
            out[o++] = off < len ? data[off] : 0;
        }
    return o;
}

/* ---- synthetic-weight quantizers (ggml textbook; not part of the reference) ----
 * Q4_0: max = signed value of largest |x| (first on ties); d = max / -8;
 * id = d ? 1/d : 0; code = min(15, (int8)(x*id + 8.5)); fp16(d) stored.  Codes are
 * packed in the REFERENCE nibble order: element 2j -> high nibble of byte j. */
void orc_quantize_q4_0(const float *x, size_t n, uint8_t *out) {
    size_t blocks = n / QK;
    for (size_t b = 0; b < blocks; ++b) {
        const float *v = x + b * QK;
        float amax = 0.0f, max = 0.0f;
        for (int i = 0; i < QK; ++i) {
            float a = fabsf(v[i]);
            if (amax < a) { amax = a; max = v[i]; }
        }
        float d = max / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = orc_f32_to_f16(d);
        uint8_t *blk = out + b * 18;
        blk[0] = (uint8_t)(dh & 0xFF);
        blk[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < QK / 2; ++j) {
            int q0 = (int)(int8_t)(v[2 * j] * id + 8.5f);
            int q1 = (int)(int8_t)(v[2 * j + 1] * id + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            blk[2 + j] = (uint8_t)((q0 << 4) | q1);
        }
    }
}

/* Q8_0: d = amax / 127; id = d ? 1/d : 0; code = roundf(x * id) (half away from 0). */
void orc_quantize_q8_0(const float *x, size_t n, uint8_t *out) {
    size_t blocks = n / QK;
    for (size_t b = 0; b < blocks; ++b) {
        const float *v = x + b * QK;
        float amax = 0.0f;
        for (int i = 0; i < QK; ++i) {
            float a = fabsf(v[i]);
            if (amax < a) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = orc_f32_to_f16(d);
        uint8_t *blk = out + b * 34;
        blk[0] = (uint8_t)(dh & 0xFF);
        blk[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < QK; ++i) blk[2 + i] = (uint8_t)(int8_t)roundf(v[i] * id);
    }
}

/* ---- the contraction (src/model/inference/model.rs:1050-1064) -------------
 * linear(x, W) = x . W^T with W[N,K] stored as GGUF blocks, row n = K/32
 * consecutive blocks (K/256 super-blocks for the K-quants).  Dequantized with quant::dequantize, accumulated in fp64:
 *   y[b, n] = sum_k x[b, k] * w[n, k]. */
static void dequant_row(int type, const uint8_t *w, size_t K, size_t n, float *row) {
    size_t bpb = orc_bytes_per_block(type);
    size_t row_bytes = (K / orc_block_size(type)) * bpb; /* 32 or 256 (K-quant super-blocks) */
    orc_dequantize(type, w + n * row_bytes, row_bytes, K, row);
}

void orc_linear_f64(int type, const uint8_t *w, size_t N, size_t K, const float *x, size_t B,
                    double *y) {
    float row[1 << 16];
    for (size_t n = 0; n < N; ++n) {
        dequant_row(type, w, K, n, row);
        for (size_t b = 0; b < B; ++b) {
            const float *xb = x + b * K;
            double acc = 0.0;
            for (size_t k = 0; k < K; ++k) acc += (double)xb[k] * (double)row[k];
            y[b * N + n] = acc;
        }
    }
}

/* Same contraction with bf16 activations X[M,K] (bits), widened exactly to fp32. */
void orc_linear_bf16x_f64(int type, const uint8_t *w, size_t N, size_t K, const uint16_t *xb16,
                          size_t M, double *y) {
    float row[1 << 16];
    for (size_t n = 0; n < N; ++n) {
        dequant_row(type, w, K, n, row);
        for (size_t m = 0; m < M; ++m) {
            const uint16_t *xm = xb16 + m * K;
            double acc = 0.0;
            for (size_t k = 0; k < K; ++k) acc += (double)orc_bf16_to_f32(xm[k]) * (double)row[k];
            y[m * N + n] = acc;
        }
    }
}

/* ---- CPU baselines (what the reference executes per token) ------------------
 * As run: weights were dequantized to f32 once at load (quant_loader.rs:76-92); each
 * call of linear() copies W^T (model.rs:1052 `weight.t().to_owned()`) and runs an
 * f32 matmul (gemm_engine.rs:69-71, ndarray -> matrixmultiply sgemm, one thread).
 * wt_scratch must hold N*K floats. */
void orc_cpu_asrun_linear(const float *w_f32, size_t N, size_t K, const float *x, size_t B,
                          float *y, float *wt_scratch, int do_transpose_copy) {
    if (do_transpose_copy) {
        /* W^T materialised as a [K, N] row-major array */
        for (size_t n = 0; n < N; ++n)
            for (size_t k = 0; k < K; ++k) wt_scratch[k * N + n] = w_f32[n * K + k];
        for (size_t b = 0; b < B; ++b) {
            float *yb = y + b * N;
            for (size_t n = 0; n < N; ++n) yb[n] = 0.0f;
            for (size_t k = 0; k < K; ++k) {
                float xv = x[b * K + k];
                const float *wr = wt_scratch + k * N;
                for (size_t n = 0; n < N; ++n) yb[n] += xv * wr[n];
            }
        }
        return;
    }
    for (size_t b = 0; b < B; ++b)
        for (size_t n = 0; n < N; ++n) {
            const float *wr = w_f32 + n * K;
            const float *xb = x + b * K;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            size_t k = 0;
            for (; k + 8 <= K; k += 8)
                for (int l = 0; l < 8; ++l) acc[l] += xb[k + l] * wr[k + l];
            float s = 0.0f;
            for (int l = 0; l < 8; ++l) s += acc[l];
            for (; k < K; ++k) s += xb[k] * wr[k];
            y[b * N + n] = s;
        }
}

/* quant_simd-style fused path: dequantize one block (reference formula) into 32 floats
 * and dot it with x, straight from the GGUF bytes.  Rows n0..n1-1. */
void orc_cpu_fused_linear(int type, const uint8_t *w, size_t N, size_t K, const float *x,
                          size_t B, float *y, size_t n0, size_t n1) {
    size_t bpb = orc_bytes_per_block(type);
    size_t nb = K / QK;
    (void)N;
    for (size_t n = n0; n < n1; ++n) {
        const uint8_t *row = w + n * nb * bpb;
        for (size_t b = 0; b < B; ++b) {
            const float *xb = x + b * K;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (size_t blk = 0; blk < nb; ++blk) {
                const uint8_t *p = row + blk * bpb;
                float d = orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
                float v[QK];
                if (type == ORC_Q4_0) {
                    for (int j = 0; j < 16; ++j) {
                        v[2 * j] = (float)((int)(p[2 + j] >> 4) - 8) * d;
                        v[2 * j + 1] = (float)((int)(p[2 + j] & 0x0F) - 8) * d;
                    }
                } else {
                    for (int i = 0; i < QK; ++i) v[i] = (float)(int8_t)p[2 + i] * d;
                }
                const float *xk = xb + blk * QK;
                for (int i = 0; i < QK; i += 8)
                    for (int l = 0; l < 8; ++l) acc[l] += xk[i + l] * v[i + l];
            }
            float s = 0.0f;
            for (int l = 0; l < 8; ++l) s += acc[l];
            y[b * N + n] = s;
        }
    }
}
