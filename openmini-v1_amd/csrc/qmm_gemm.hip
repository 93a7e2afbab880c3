// Prefill GEMM: y[m, n] = sum_k x[m, k] * w[n, k], x bf16, y fp32, on bf16 MFMA.
//
// Replaces, per prefill call of linear_gemm() (openmini-server/src/model/inference/
// model.rs:1060-1064), the f32 GEMM over weights dequantized at load
// (gemm_engine.rs:69-71).  Numerics: each code is exact in bf16 (Q4_0 as
// (q-8)/16, Q8_0 as q), bf16 x bf16 products are exact in fp32, and one
// v_mfma_f32_16x16x32_bf16 covers exactly one 32-element block, so every block's
// partial sum is scaled by its fp32 scale and added to an fp32 accumulator:
//   y[m, n] = sum_b d[n, b] * (sum_{k in b} x[m, k] * q[n, k]).
// Weights are never rounded (no bf16 q*d), activations are not requantized.  The
// per-block rescale costs 4 VALU FMAs per MFMA, about as many VALU cycles as the
// MFMA takes, so the kernel keeps both busy: two waves per SIMD, MFMA results in
// VGPRs, and each MFMA issued before the FMAs of the previous one.
// K-quant weights (the reference's reading, quant.rs:338-410 and :515-600) use their
// 32-element sub-blocks as the blocks.  Q4_K: codes as Q4_0, block factor
// 16 * d * scale (exact).  Q6_K: its scale changes every 16 elements, inside one
// MFMA's 32, so q * scale (an exact integer of at most 13 bits) enters as bf16
// hi + lo (two chained MFMAs, both exact), and the row's d is the block factor.
//
// Tiling: a workgroup computes a kBM x (16 kWT kNW) tile of y with kNW column slices
// x kKS K parts of waves (choose_shape picks 128 or 64 rows and 3 or 2 weight tiles per
// wave by problem size).  A wave owns kBM rows x 16 kWT columns (kBM/16 x kWT MFMA
// subtiles of fp32 accumulators) over one K part, and the parts are added through
// LDS at the end (fixed order).  A K step is two blocks (64 elements):
//   * x: each K part's kBM x 64 bf16 slab is copied HBM -> LDS by buffer loads with
//     an LDS destination (no registers), double-buffered, rows XOR-swizzled in
//     16-byte segments so the A-fragment reads are bank-conflict free;
//   * weights: each wave loads its kWT tiles' codes and scales straight into
//     registers two K steps ahead (three register sets: first-touch weights come
//     from HBM, whose latency under load exceeds one step) and converts its own B
//     fragments (its columns are its own, so nothing is converted twice).
#include "qmm_device.hpp"

namespace qmm {
namespace {

constexpr int kBMMax = 128;  // most x rows per workgroup
constexpr int kCeilWT = 3;   // weight tiles per wave of the launch shapes the ceiling yardstick mirrors

__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    // bf16 of exactly-representable values = high halves of their fp32 bits.
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 8 Q4_0 nibbles (one code word of two's-complement q - 8, elements in order) ->
// 8 bf16 (q-8)/16.
__device__ __forceinline__ bf16x8 cvt_q4(uint32_t w) {
    uint32_t h = w >> 4;
    asm("" : "+v"(h));  // keep the shift: 1 shift + 4 SDWA converts, not 4 bit-field extracts
    const float a0 = __builtin_amdgcn_cvt_off_f32_i4(w & 0xFFu);
    const float a1 = __builtin_amdgcn_cvt_off_f32_i4((w >> 8) & 0xFFu);
    const float a2 = __builtin_amdgcn_cvt_off_f32_i4((w >> 16) & 0xFFu);
    const float a3 = __builtin_amdgcn_cvt_off_f32_i4(w >> 24);
    const float b0 = __builtin_amdgcn_cvt_off_f32_i4(h & 0xFFu);
    const float b1 = __builtin_amdgcn_cvt_off_f32_i4((h >> 8) & 0xFFu);
    const float b2 = __builtin_amdgcn_cvt_off_f32_i4((h >> 16) & 0xFFu);
    const float b3 = __builtin_amdgcn_cvt_off_f32_i4(h >> 24);
    uint32_t p[4] = {pack_hi16(a0, a1), pack_hi16(a2, a3), pack_hi16(b0, b1), pack_hi16(b2, b3)};
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<uint4*>(p));
}

// 8 Q8_0 codes (two words) -> 8 bf16 q in k order.
__device__ __forceinline__ bf16x8 cvt_q8(uint32_t w0, uint32_t w1) {
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = (float)(int8_t)((w0 >> (8 * i)) & 0xFFu);
        f[4 + i] = (float)(int8_t)((w1 >> (8 * i)) & 0xFFu);
    }
    uint32_t p[4] = {pack_hi16(f[0], f[1]), pack_hi16(f[2], f[3]), pack_hi16(f[4], f[5]),
                     pack_hi16(f[6], f[7])};
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<uint4*>(p));
}

// Chunk geometry the GEMM reads, by weight format (layouts in qmm_internal.hpp).
template <int kFmt>
struct GFmt {
    static constexpr bool kQ8 = kFmt == OPENMINI_QMM_Q8_0;
    static constexpr bool kQ4K = kFmt == OPENMINI_QMM_Q4_K;
    static constexpr bool kQ6K = kFmt == OPENMINI_QMM_Q6_K;
    static constexpr bool kKQ = kQ4K || kQ6K;
    static constexpr bool kNib = !kQ8 && !kQ6K;            // Q4_0 / Q4_K: 16 B of nibbles per slot
    static constexpr int kCB = kQ8 ? 32 : 16;               // bytes of a slot's (low) codes
    static constexpr int kWords = kNib ? 1 : 2;             // code words per lane and block
    static constexpr int kScaleOff = kTileEntries * (kQ6K ? 24 : kCB);
    static constexpr int kDOff = kScaleOff + (kQ6K ? 2 : 1) * kTileEntries;  // K-quant: fp16 d per row
    static constexpr int kChunk = kQ4K ? kQ4KChunk : kQ6K ? kQ6KChunk : chunk_bytes_for(!kQ8);
    // buffer loads one load_b issues per (tile, block), plus the K-quant d per tile
    static constexpr int kLoadsPerBlock = kQ6K ? 3 : 2;
    static constexpr int kLoadsPerTile = kKQ ? 1 : 0;
};

// A wave's weight operands for one K step: per weight tile j and block tt of the
// step, the lane's 8 codes (Q4_0 / Q4_K one word of nibbles, Q8_0 two words of
// bytes, Q6_K the low-nibble word and the top-bit word), its column's scale, and for
// K-quants the column's d (one per step: a step stays inside one group).
template <int kFmt, int kSB, int kWT>
struct BRegs {
    uint32_t c[kWT][kSB][GFmt<kFmt>::kWords];
    uint32_t s[kWT][kSB];
    uint32_t d[kWT];
};

// 8 Q6_K codes of lane quarter kq -> bf16 hi / lo parts of q * sc, q * sc exact (at
// most 13 significant bits): hi keeps the top 8 bits, lo = q * sc - hi has at most 5.
// w: the slot's low-nibble word kq; hm: its top-bit word kq / 2 (qmm_internal.hpp).
__device__ __forceinline__ void split_q6(uint32_t w, uint32_t hm, int kq, float sc4, bf16x8& hi, bf16x8& lo) {
    // 4 q per int8 byte: low 4 bits at 2..5, the top 2 bits (fields 2 (kq & 1) and
    // 2 (kq & 1) + 1 of each byte of hm) at 6..7; elements 8 kq + 0..3, then + 4..7
    const int sh = (kq & 1) * 4;
    const uint32_t b0 = ((w << 2) & 0x3C3C3C3Cu) | ((hm << (6 - sh)) & 0xC0C0C0C0u);
    const uint32_t b1 = ((w >> 2) & 0x3C3C3C3Cu) | ((hm << (4 - sh)) & 0xC0C0C0C0u);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // (4 q) * (sc / 4): exact
        f[i] = (float)(int8_t)((b0 >> (8 * i)) & 0xFFu) * sc4;
        f[4 + i] = (float)(int8_t)((b1 >> (8 * i)) & 0xFFu) * sc4;
    }
    uint32_t h[4], l[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t u0 = __float_as_uint(f[2 * p]), u1 = __float_as_uint(f[2 * p + 1]);
        const float r0 = f[2 * p] - __uint_as_float(u0 & 0xFFFF0000u);
        const float r1 = f[2 * p + 1] - __uint_as_float(u1 & 0xFFFF0000u);
        h[p] = __builtin_amdgcn_perm(u1, u0, 0x07060302u);
        l[p] = pack_hi16(r0, r1);
    }
    hi = __builtin_bit_cast(bf16x8, *reinterpret_cast<uint4*>(h));
    lo = __builtin_bit_cast(bf16x8, *reinterpret_cast<uint4*>(l));
}

// The same q * sc as fp16 hi (rounded toward zero: 11 significant bits) + lo (the
// remaining at most 2 bits), both exact.
__device__ __forceinline__ void split_q6_f16(uint32_t w, uint32_t hm, int kq, float sc4, f16x8& hi, f16x8& lo) {
    const int sh = (kq & 1) * 4;
    const uint32_t b0 = ((w << 2) & 0x3C3C3C3Cu) | ((hm << (6 - sh)) & 0xC0C0C0C0u);
    const uint32_t b1 = ((w >> 2) & 0x3C3C3C3Cu) | ((hm << (4 - sh)) & 0xC0C0C0C0u);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = (float)(int8_t)((b0 >> (8 * i)) & 0xFFu) * sc4;
        f[4 + i] = (float)(int8_t)((b1 >> (8 * i)) & 0xFFu) * sc4;
    }
    uint32_t h[4], l[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const auto hp = __builtin_amdgcn_cvt_pkrtz(f[2 * p], f[2 * p + 1]);
        h[p] = __builtin_bit_cast(uint32_t, hp);
        l[p] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f[2 * p] - (float)hp[0], f[2 * p + 1] - (float)hp[1]));
    }
    hi = __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(h));
    lo = __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(l));
}

// Workgroup shape: kBM x rows, kNW column slices x kKS K parts of waves; a K step is
// kSB blocks.
template <int kBM, int kNW, int kKS, int kSB, int kWT_>
struct Shape {
    static constexpr int kWT = kWT_;                       // weight tiles (16 columns each) per wave
    static constexpr int kMI = kBM / 16;                   // MFMA row subtiles per wave
    static constexpr int kThreads = 64 * kNW * kKS;
    static constexpr int kBT = kNW * kWT;                 // weight tiles per workgroup
    static constexpr int kRowB = kSB * kQK * 2;            // bytes of one x row per step
    static constexpr int kSegs = kRowB / 16;               // 16-byte segments per row
    static constexpr int kSlabB = kBM * kRowB;             // one K part's x slab per step
    static constexpr int kStageB = kKS * kSlabB;
    static constexpr int kRowsPerCopy = 1024 / kRowB;      // one 1 KB copy instruction
    static constexpr int kCopies = kSlabB / kNW / 1024;     // copies per wave per step
    static constexpr int kRedB = (kKS - 1) * kNW * kMI * kWT * 4 * 64 * 4;  // K-part partials
    static constexpr int kLdsB = 2 * kStageB > kRedB ? 2 * kStageB : kRedB;
    static_assert(kTileBlocks % kSB == 0, "a step covers whole blocks of one group");
};

// kGate: y holds the gate projection on entry and each element is replaced by
// silu(gate) * (x . W^T), silu(v) = v / (1 + exp(-v)) (model.rs:713-735, :1187-1189).
// kX2: x holds split fp32 activations (split_rows_kernel): per 32-element block 32 fp16
// hi parts, then 32 fp16 lo parts, of x scaled by 2^e per row (x_exp[m] = e); k is
// then the length of such a row in fp16 elements (twice K).  Each block runs two
// chained fp16 MFMAs per subtile (hi, then lo, into one fp32 sum) with fp16 codes,
// then the same rescale; outputs are scaled back by 2^-e.
// Two waves per SIMD (512 / threads workgroups per CU): the register budget is 256.
template <int kFmt, int kBM, int kNW, int kKS, int kSB, int kWT, bool kGate, bool kX2>
__global__ __launch_bounds__(64 * kNW * kKS, 512 / (64 * kNW * kKS)) void gemm_kernel(
    const uint16_t* __restrict__ x, const int* __restrict__ x_exp, const uint8_t* __restrict__ chunks,
    float* __restrict__ y, int m_rows, int n_rows, int n_tiles, int groups, int k) {
    using S = Shape<kBM, kNW, kKS, kSB, kWT>;
    using F = GFmt<kFmt>;
    constexpr int kMI = S::kMI;
    constexpr int kCB = F::kCB;
    constexpr int kChunk = F::kChunk;
    constexpr int kWB = kX2 ? kSB / 2 : kSB;  // weight blocks per step
    static_assert(kWB >= 1, "a step holds at least one weight block");
    constexpr int kStepsPerGroup = kTileBlocks / kWB;
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kLdsB];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kh = wave / kNW, wn = wave % kNW;
    const int li = lane & 15;  // A row / B column inside a 16 x 16 subtile
    const int kq = lane >> 4;  // which 8-element quarter of the 32-element block
    const int bx = blockIdx.x, by = blockIdx.y;
    const int m0 = by * kBM;
    const int tile0 = bx * S::kBT + wn * kWT;

    // this K part's steps; all parts step together (barriers), a shorter one idles
    const int units = groups * kStepsPerGroup;
    const int u0 = (int)((int64_t)units * kh / kKS);
    const int u1 = (int)((int64_t)units * (kh + 1) / kKS);
    const int steps = (units + kKS - 1) / kKS;

    // x is < 2 GiB (the launcher splits m); the chunks < 4 GiB (checked at upload)
    const __amdgpu_buffer_rsrc_t x_rs = make_rsrc(x, (uint32_t)m_rows * (uint32_t)k * 2u);
    const __amdgpu_buffer_rsrc_t w_rs = make_rsrc(chunks, (uint32_t)n_tiles * groups * kChunk);

    // ---- x slab copies: kCopies x 1 KB per wave per step, kRowsPerCopy rows each.
    // LDS position p of row r holds the row's 16-byte segment s = p ^ (r % kSegs).
    // Offsets are recomputed per copy (registers are the scarce resource here).
    const int r_lane = wn * (kBM / kNW) + lane / S::kSegs;
    const int p_lane = lane % S::kSegs;
    auto issue_x = [&](int u, int stage) {
        uint8_t* base = lds + stage * S::kStageB + kh * S::kSlabB + wn * S::kCopies * 1024;
        const uint32_t kk0 = (uint32_t)u * (kSB * kQK);
#pragma unroll
        for (int j = 0; j < S::kCopies; ++j) {
            const int r = r_lane + j * S::kRowsPerCopy;
            const uint32_t seg = (uint32_t)((p_lane ^ (r % S::kSegs)) * 8) + kk0;
            const uint32_t gm = (uint32_t)min(m0 + r, m_rows - 1);  // rows past m repeat the last one
            // segments past K read zero (an out-of-range buffer offset)
            const uint32_t voff = seg < (uint32_t)k ? (gm * (uint32_t)k + seg) * 2u : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                x_rs, (__attribute__((address_space(3))) void*)(base + j * 1024), 16, voff, 0, 0, 0);
        }
    };

    // ---- weight operands: chunk (tile j, group g), slot (t, li), quarter kq
    uint32_t tile_off[kWT];
#pragma unroll
    for (int j = 0; j < kWT; ++j) tile_off[j] = (uint32_t)min(tile0 + j, n_tiles - 1) * groups * kChunk;
    auto load_b = [&](BRegs<kFmt, kWB, kWT>& B, int u) {
        const int g = u / kStepsPerGroup, t0 = (u % kStepsPerGroup) * kWB;
#pragma unroll
        for (int j = 0; j < kWT; ++j) {
            const uint32_t soff = tile_off[j] + (uint32_t)g * kChunk;
            if constexpr (F::kKQ) B.d[j] = __builtin_amdgcn_raw_buffer_load_b16(w_rs, F::kDOff + li * 2, soff, 0);
#pragma unroll
            for (int tt = 0; tt < kWB; ++tt) {
                const uint32_t slot = (uint32_t)((t0 + tt) * kTileRows + li);
                if constexpr (F::kQ4K)
                    B.s[j][tt] = __builtin_amdgcn_raw_buffer_load_b8(w_rs, F::kScaleOff + slot, soff, 0);
                else if constexpr (F::kQ6K)  // the scale of the lane's 16-element half
                    B.s[j][tt] = __builtin_amdgcn_raw_buffer_load_b8(w_rs, F::kScaleOff + slot * 2 + (kq >> 1), soff, 0);
                else
                    B.s[j][tt] = __builtin_amdgcn_raw_buffer_load_b16(w_rs, F::kScaleOff + slot * 2, soff, 0);
                if constexpr (F::kNib) {
                    B.c[j][tt][0] = __builtin_amdgcn_raw_buffer_load_b32(w_rs, slot * kCB + kq * 4, soff, 0);
                } else if constexpr (F::kQ6K) {
                    B.c[j][tt][0] = __builtin_amdgcn_raw_buffer_load_b32(w_rs, slot * kCB + kq * 4, soff, 0);
                    B.c[j][tt][1] = __builtin_amdgcn_raw_buffer_load_b32(
                        w_rs, kTileEntries * 16 + slot * 8 + (kq >> 1) * 4, soff, 0);
                } else {
                    const uint2 v = __builtin_bit_cast(
                        uint2, __builtin_amdgcn_raw_buffer_load_b64(w_rs, slot * kCB + kq * 8, soff, 0));
                    B.c[j][tt][0] = v.x;
                    B.c[j][tt][1] = v.y;
                }
            }
        }
    };

    f32x4 acc[kMI][kWT];
    // Q6_K on bf16 x: the sums of the current super-block, before its d (one per tile
    // row and super-block); the other instances leave them unused.
    constexpr bool kChain = F::kQ6K && !kX2;
    f32x4 sacc[kMI][kWT];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int j = 0; j < kWT; ++j) acc[i][j] = sacc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // A fragments of 32-element segment tt of the step in LDS stage `stage`: rows
    // i * 16 + li, elements 8 kq .. 8 kq + 7 of the segment (swizzled); bf16 x, or the
    // fp16 hi (tt even) / lo (tt odd) parts of one block of split x.
    typedef uint4 AFrags[kMI];
    auto read_a = [&](AFrags& a, int stage, int tt) {
        const uint8_t* slab = lds + stage * S::kStageB + kh * S::kSlabB;
#pragma unroll
        for (int i = 0; i < kMI; ++i) {
            const int r = i * 16 + li;
            a[i] = *reinterpret_cast<const uint4*>(slab + r * S::kRowB + (((tt * 4 + kq) ^ (r % S::kSegs)) * 16));
        }
    };
    auto bf = [](const uint4& v) { return __builtin_bit_cast(bf16x8, v); };
    auto hf = [](const uint4& v) { return __builtin_bit_cast(f16x8, v); };
    // Q6_K block tt: the scale changes every 16 elements, inside an MFMA's 32, so it is
    // folded into the codes: q * sc (exact integers) as bf16 hi + lo.  The d is one per
    // tile row and super-block, so the blocks of a super-block chain into one sum per
    // output (sacc; all hi MFMAs, then all lo ones, so no MFMA waits on the one before),
    // and flush_q6 applies d once per super-block: one FMA per output per 8 blocks
    // instead of one per block.
    auto compute_q6 = [&](const BRegs<kFmt, kWB, kWT>& B, const AFrags& a, int tt) {
        if constexpr (F::kQ6K && !kX2) {
            bf16x8 bh[kWT], bl[kWT];
#pragma unroll
            for (int j = 0; j < kWT; ++j)
                split_q6(B.c[j][tt][0], B.c[j][tt][1], kq, (float)(int8_t)(B.s[j][tt] & 0xFFu) * 0.25f, bh[j], bl[j]);
#pragma unroll
            for (int q = 0; q < kMI * kWT; ++q)
                sacc[q / kWT][q % kWT] =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf(a[q / kWT]), bh[q % kWT], sacc[q / kWT][q % kWT], 0, 0, 0);
#pragma unroll
            for (int q = 0; q < kMI * kWT; ++q)
                sacc[q / kWT][q % kWT] =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf(a[q / kWT]), bl[q % kWT], sacc[q / kWT][q % kWT], 0, 0, 0);
        }
    };
    // Q6_K: after the last block of a super-block, or of this K part, acc += sacc * d.
    auto flush_q6 = [&](const BRegs<kFmt, kWB, kWT>& B) {
        if constexpr (kChain) {
#pragma unroll
            for (int j = 0; j < kWT; ++j) {
                const float d = f16_bits_to_f32((uint16_t)B.d[j]);
#pragma unroll
                for (int i = 0; i < kMI; ++i) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(sacc[i][j][r], d, acc[i][j][r]);
                    sacc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    };
    // Block tt of one step: 8 x 3 MFMAs on A fragments `a` and the weight registers.
    auto compute = [&](const BRegs<kFmt, kWB, kWT>& B, const AFrags& a, int tt) {
        if constexpr (F::kQ6K) {
            compute_q6(B, a, tt);
            return;
        }
        bf16x8 b[kWT];
        float d[kWT];
#pragma unroll
        for (int j = 0; j < kWT; ++j) {
            const uint16_t dh = (uint16_t)B.s[j][tt];
            if constexpr (F::kQ4K) {  // (q - 8) / 16 codes; block factor 16 d * scale (exact)
                b[j] = cvt_q4(B.c[j][tt][0]);
                d[j] = f16_bits_to_f32((uint16_t)B.d[j]) * (float)(B.s[j][tt] & 0xFFu) * 16.0f;
            } else if constexpr (F::kNib) {
                b[j] = cvt_q4(B.c[j][tt][0]);
                d[j] = f16_bits_to_f32(dh) * 16.0f;
            } else {
                b[j] = cvt_q8(B.c[j][tt][0], B.c[j][tt][1]);
                d[j] = f16_bits_to_f32(dh);
            }
        }
        // MFMA q + 1 is issued before the FMAs of q (two result registers)
        f32x4 pp[2];
        pp[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf(a[0]), b[0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < kMI * kWT; ++q) {
            if (q + 1 < kMI * kWT)
                pp[(q + 1) & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    bf(a[(q + 1) / kWT]), b[(q + 1) % kWT], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[q / kWT][q % kWT][r] = fmaf(pp[q & 1][r], d[q % kWT], acc[q / kWT][q % kWT][r]);
        }
    };
    // Split x, the step's one block: per subtile the hi and the lo fragments times the
    // same fp16 codes, chained into one fp32 sum (exact products), then the rescale.
    // Q6_K: q * scale as fp16 hi + lo codes, four chained MFMAs per subtile.  (Chaining
    // a super-block's blocks as on bf16 x was slower here: 194 -> 225 us at M = 512;
    // these four MFMAs per block outweigh the rescale, and the chained sums' registers
    // rule out the 128 x 96 tiles.)
    auto compute_x2 = [&](const BRegs<kFmt, kWB, kWT>& B, const AFrags& ah, const AFrags& al) {
        if constexpr (kX2) {
            constexpr int kCodes = F::kQ6K ? 2 : 1;
            f16x8 b[kWT][kCodes];
            float d[kWT];
#pragma unroll
            for (int j = 0; j < kWT; ++j) {
                if constexpr (F::kQ6K) {
                    split_q6_f16(B.c[j][0][0], B.c[j][0][1], kq, (float)(int8_t)(B.s[j][0] & 0xFFu) * 0.25f, b[j][0],
                                 b[j][1]);
                    d[j] = f16_bits_to_f32((uint16_t)B.d[j]);
                } else if constexpr (F::kQ4K) {  // q - 8 codes; block factor d * scale (exact)
                    b[j][0] = codes_q4(B.c[j][0][0]);
                    d[j] = f16_bits_to_f32((uint16_t)B.d[j]) * (float)(B.s[j][0] & 0xFFu);
                } else if constexpr (F::kNib) {
                    b[j][0] = codes_q4(B.c[j][0][0]);
                    d[j] = f16_bits_to_f32((uint16_t)B.s[j][0]);
                } else {
                    b[j][0] = codes_q8(B.c[j][0][0], B.c[j][0][1]);
                    d[j] = f16_bits_to_f32((uint16_t)B.s[j][0]);
                }
            }
            auto block = [&](int q) {
                const int i = q / kWT, j = q % kWT;
                f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(hf(ah[i]), b[j][0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(hf(al[i]), b[j][0], t, 0, 0, 0);
#pragma unroll
                for (int c = 1; c < kCodes; ++c) {
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(hf(ah[i]), b[j][c], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(hf(al[i]), b[j][c], t, 0, 0, 0);
                }
                return t;
            };
            // the MFMAs of subtile q + 1 are issued before the FMAs of q
            f32x4 pp[2];
            pp[0] = block(0);
#pragma unroll
            for (int q = 0; q < kMI * kWT; ++q) {
                if (q + 1 < kMI * kWT) pp[(q + 1) & 1] = block(q + 1);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[q / kWT][q % kWT][r] = fmaf(pp[q & 1][r], d[q % kWT], acc[q / kWT][q % kWT][r]);
            }
        }
    };

    // Step `it` (unit u = u0 + it): the x copies for u were issued one step earlier,
    // the weights for u two steps earlier.  Per step the wave issues x(u + 1), then
    // the weights of u + 2 (kBLoads loads), so waiting until at most kBLoads loads
    // are outstanding completes x(u) and everything older; one barrier then makes
    // every wave's copies visible and frees the other x stage.  The loads are
    // unconditional (units past this part's end re-load its last unit, a cache hit)
    // so the count of outstanding loads is the same on every path; the compiler's
    // own waits before the barrier then cover only the x copies.
    constexpr int kBLoads = kWT * (kWB * F::kLoadsPerBlock + F::kLoadsPerTile);
    static_assert(kBLoads <= 63, "vmcnt counts up to 63");
    const int u_last = max(u1 - 1, 0);
    // Q6_K: unit u holds blocks u kWB .. u kWB + kWB - 1 of the row; a super-block is 8
    // blocks, and a K part may start or end inside one
    auto q6_ends = [&](int u) { return kChain && (((u + 1) * kWB) % 8 == 0 || u == u1 - 1); };
    auto step = [&](int it, const BRegs<kFmt, kWB, kWT>& cur, BRegs<kFmt, kWB, kWT>& far) {
        const int u = u0 + it;
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kBLoads));
        __syncthreads();
        issue_x(min(u + 1, u_last), (it + 1) & 1);
        // The weight loads go between the step's blocks: issued right after the copies,
        // every wave of the CU would queue its vector-memory instructions at once and
        // stall its MFMAs behind them.  The memory clobbers keep the issue order (the
        // copies before the weights) that the vmcnt count above relies on.
        asm volatile("" ::: "memory");
        const bool live = u < u1;  // uniform per wave
        if constexpr (kX2) {  // one block per step: its hi and lo fragments, then the weights
            AFrags ah, al;
            if (live) {
                read_a(ah, it & 1, 0);
                read_a(al, it & 1, 1);
                __builtin_amdgcn_s_setprio(3);
                compute_x2(cur, ah, al);
                __builtin_amdgcn_s_setprio(0);
            }
            asm volatile("" ::: "memory");
            load_b(far, min(u + 2, u_last));
            asm volatile("" ::: "memory");
            if (live && q6_ends(u)) flush_q6(cur);
            return;
        }
        AFrags a;
        // A block's MFMAs and rescale run at raised wave priority, so the SIMD's other
        // wave (copies, weight loads, a barrier) yields issue slots to them: Q8_0
        // M=512 83.5-83.7 -> 81.9-82.1 us, Q4_0 28672x8192 M=1024 598-601 -> 588-591 us
        // (three interleaved passes, one box; priority 1 gained about half of that).
        if (live) {
            read_a(a, it & 1, 0);
            __builtin_amdgcn_s_setprio(3);
            compute(cur, a, 0);
            __builtin_amdgcn_s_setprio(0);
        }
        asm volatile("" ::: "memory");
        load_b(far, min(u + 2, u_last));
        asm volatile("" ::: "memory");
#pragma unroll
        for (int tt = 1; tt < kSB; ++tt)
            if (live) {
                read_a(a, it & 1, tt);
                __builtin_amdgcn_s_setprio(3);
                compute(cur, a, tt);
                __builtin_amdgcn_s_setprio(0);
            }
        if (live && q6_ends(u)) flush_q6(cur);
    };

    BRegs<kFmt, kWB, kWT> b0, b1, b2;
    issue_x(min(u0, u_last), 0);
    asm volatile("" ::: "memory");
    load_b(b0, min(u0, u_last));
    load_b(b1, min(u0 + 1, u_last));
    int it = 0;
    for (; it + 2 < steps; it += 3) {  // three register sets rotate: no copies
        step(it, b0, b2);
        step(it + 1, b1, b0);
        step(it + 2, b2, b1);
    }
    if (it < steps) step(it, b0, b2);
    if (it + 1 < steps) step(it + 1, b1, b0);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // no copy may land after the stages are reused

    // ---- K parts meet in LDS (the stages are free after this barrier), then store.
    // Parts 1.. hand their sums over as one 16-byte LDS write per subtile and lane;
    // part 0 issues all its LDS reads together, adds the parts in order (fixed, so the
    // bits do not depend on timing) and stores.
    __syncthreads();
    f32x4* red = reinterpret_cast<f32x4*>(lds);
    auto slot = [&](int h, int i, int j) { return ((((h - 1) * kNW + wn) * kMI + i) * kWT + j) * 64 + lane; };
    if (kh > 0) {
#pragma unroll
        for (int i = 0; i < kMI; ++i)
#pragma unroll
            for (int j = 0; j < kWT; ++j) red[slot(kh, i, j)] = acc[i][j];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
        for (int h = 1; h < kKS; ++h) {
            f32x4 part[kMI][kWT];  // all of a part's reads in flight before the first add
#pragma unroll
            for (int i = 0; i < kMI; ++i)
#pragma unroll
                for (int j = 0; j < kWT; ++j) part[i][j] = red[slot(h, i, j)];
#pragma unroll
            for (int i = 0; i < kMI; ++i)
#pragma unroll
                for (int j = 0; j < kWT; ++j) acc[i][j] += part[i][j];
        }
        // split x: the row scale 2^-e of each of the lane's output rows
        int rexp[kX2 ? kMI : 1][4];
        if constexpr (kX2) {
#pragma unroll
            for (int i = 0; i < kMI; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) rexp[i][r] = -x_exp[min(m0 + i * 16 + kq * 4 + r, m_rows - 1)];
        }
        // lane holds D[4 kq + r][li] of each 16 x 16 subtile
        auto store = [&](int i, int j, int r) {
            float* yp = y + (size_t)(m0 + i * 16 + kq * 4 + r) * n_rows + (tile0 + j) * kTileRows + li;
            float v = acc[i][j][r];
            if constexpr (kX2) v = __builtin_amdgcn_ldexpf(v, rexp[i][r]);
            if constexpr (kGate) {
                const float g = *yp;
                v = g / (1.0f + expf(-g)) * v;
            }
            *yp = v;
        };
        if (m0 + kBM <= m_rows && (tile0 + kWT) * kTileRows <= n_rows) {  // whole tile inside y
#pragma unroll
            for (int j = 0; j < kWT; ++j)
#pragma unroll
                for (int i = 0; i < kMI; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) store(i, j, r);
        } else {
#pragma unroll
            for (int j = 0; j < kWT; ++j)
#pragma unroll
                for (int i = 0; i < kMI; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (m0 + i * 16 + kq * 4 + r < m_rows && (tile0 + j) * kTileRows + li < n_rows) store(i, j, r);
        }
    }
}

// x rows of kx 2-byte elements (K for bf16 x, 2 K for split x).
template <int kFmt, int kBM, int kNW, int kKS, int kSB, int kWT, bool kGate, bool kX2>
hipError_t launch_shape(const Weight& w, const uint16_t* x, const int* x_exp, float* y, int64_t m, int64_t kx,
                        hipStream_t s) {
    using S = Shape<kBM, kNW, kKS, kSB, kWT>;
    const dim3 grid((unsigned)((w.n_tiles + S::kBT - 1) / S::kBT), (unsigned)((m + kBM - 1) / kBM));
    hipLaunchKernelGGL((gemm_kernel<kFmt, kBM, kNW, kKS, kSB, kWT, kGate, kX2>), grid, dim3(S::kThreads), 0, s, x,
                       x_exp, w.chunks, y, (int)m, (int)w.n, (int)w.n_tiles, (int)w.groups, (int)kx);
    return hipGetLastError();
}

// Tile families: 128-row tiles with 2 column slices x 2 K halves of waves (64 KB of LDS,
// two workgroups per CU so one's barriers overlap the other's work), and 64-row tiles
// with 2 column slices x 4 K parts (72 KB of LDS) for more, smaller workgroups.  Split
// x uses the same shapes with one block per step (its hi and lo parts fill the step's
// 64-element slab).
// Launch shape by problem size.
//   0: 128-row tiles, 3 weight tiles per wave (128 x 96, 4 waves)
//   1: 128-row tiles, 2 weight tiles per wave (128 x 64, 4 waves)
//   2:  64-row tiles, 3 weight tiles per wave ( 64 x 96, 8 waves)
//   3:  64-row tiles, 2 weight tiles per wave ( 64 x 64, 8 waves)
// Few and large workgroups leave CUs idle or a last round part-filled; small ones
// cost more per flop (each B fragment serves fewer MFMAs, each A fragment fewer
// tiles).  The model: workgroups run in rounds of (CUs x workgroups per CU, from the
// kernel's occupancy); a round costs (workgroups per CU) x (tile work) x (the shape's
// relative cost per flop), a last round of at most one workgroup per CU 0.67 of that
// where a CU holds two (a workgroup alone on its CU runs faster than two sharing it);
// at one workgroup per CU a last round costs a full one (each workgroup already has
// its CU alone).
// The relative costs are fitted to shape-by-shape timings on MI355X (Q4_0 / Q8_0,
// M = 128..2048, 1024..28672 rows): on bf16 x the model picks the fastest shape in
// 66 of 70 cases (worst +12%); split x, whose steps run twice the MFMAs, has costs of
// its own and picks the fastest in 39 of 40 (worst +0.6%).  Fixed per shape, so a
// row's bits depend only on m and the weight.  A shape with per_cu < 0 is not built
// for the instance: Q6_K on bf16 x has no 128 x 96 tiles (its super-block sums take
// 96 more registers and would spill), and split x no 64 x 96 tiles (64 x 64 ran
// faster or within 0.6% at every measured size).
int choose_shape(const Weight& w, int64_t m, const int (&per_cu)[4], bool split_x) {
    static const int bm[4] = {128, 128, 64, 64}, wt[4] = {3, 2, 3, 2};
    static const double cost_per_flop[2][4] = {{1.00, 1.10, 1.25, 1.35},   // bf16 x
                                               {1.00, 1.10, 1.40, 1.20}};  // split x
    const int64_t cus = 256;
    int best = -1;
    double best_cost = 0.0;
    for (int i = 0; i < 4; ++i) {
        if (per_cu[i] < 0) continue;
        const int spc = per_cu[i] > 0 ? per_cu[i] : 1;
        const int64_t wgs = (w.n_tiles + 2 * wt[i] - 1) / (2 * wt[i]) * ((m + bm[i] - 1) / bm[i]);
        const int64_t slots = cus * spc;
        const double round = (double)spc * bm[i] * wt[i] * cost_per_flop[split_x][i] * (spc == 1 ? 1.2 : 1.0);
        double cost = (double)(wgs / slots) * round;
        if (wgs % slots) cost += round * (spc > 1 && wgs % slots <= cus ? 0.67 : 1.0);
        if (best < 0 || cost < best_cost) best = i, best_cost = cost;
    }
    return best;
}

// Workgroups of `kernel` (at `threads` per workgroup) one CU holds at once.
int blocks_per_cu(const void* kernel, int threads) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess) return 1;
    return n;
}

// Shape 0 is built for every instance but Q6_K on bf16 x.
template <int kFmt, bool kX2>
constexpr bool kWideTiles = kFmt != OPENMINI_QMM_Q6_K || kX2;

template <int kFmt, bool kGate, bool kX2>
int shape0_per_cu() {
    if constexpr (kWideTiles<kFmt, kX2>)
        return blocks_per_cu((const void*)gemm_kernel<kFmt, 128, 2, 2, 2, 3, kGate, kX2>, 256);
    else
        return -1;
}

// Shape 2 is built for bf16 x only.
template <int kFmt, bool kGate, bool kX2>
int shape2_per_cu() {
    if constexpr (!kX2)
        return blocks_per_cu((const void*)gemm_kernel<kFmt, 64, 2, 4, 2, 3, kGate, kX2>, 512);
    else
        return -1;
}

// Workgroups per CU of the four shapes' kernels (queried once per instantiation).
template <int kFmt, bool kGate, bool kX2>
const int (&shape_occupancy())[4] {
    static const int per_cu[4] = {
        shape0_per_cu<kFmt, kGate, kX2>(),
        blocks_per_cu((const void*)gemm_kernel<kFmt, 128, 2, 2, 2, 2, kGate, kX2>, 256),
        shape2_per_cu<kFmt, kGate, kX2>(),
        blocks_per_cu((const void*)gemm_kernel<kFmt, 64, 2, 4, 2, 2, kGate, kX2>, 512)};
    return per_cu;
}

template <int kFmt, bool kGate, bool kX2>
hipError_t launch_kind(const Weight& w, const uint16_t* x, const int* x_exp, float* y, int64_t m, int64_t kx,
                       hipStream_t s) {
    switch (choose_shape(w, m, shape_occupancy<kFmt, kGate, kX2>(), kX2)) {
    case 0:
        if constexpr (kWideTiles<kFmt, kX2>) return launch_shape<kFmt, 128, 2, 2, 2, 3, kGate, kX2>(w, x, x_exp, y, m, kx, s);
        return hipErrorInvalidValue;
    case 1: return launch_shape<kFmt, 128, 2, 2, 2, 2, kGate, kX2>(w, x, x_exp, y, m, kx, s);
    case 2:
        if constexpr (!kX2) return launch_shape<kFmt, 64, 2, 4, 2, 3, kGate, kX2>(w, x, x_exp, y, m, kx, s);
        return hipErrorInvalidValue;
    default: return launch_shape<kFmt, 64, 2, 4, 2, 2, kGate, kX2>(w, x, x_exp, y, m, kx, s);
    }
}

template <bool kGate, bool kX2>
hipError_t launch_type(const Weight& w, const uint16_t* x, const int* x_exp, float* y, int64_t m, int64_t kx,
                       hipStream_t s) {
    switch (w.type) {
    case OPENMINI_QMM_Q4_0: return launch_kind<OPENMINI_QMM_Q4_0, kGate, kX2>(w, x, x_exp, y, m, kx, s);
    case OPENMINI_QMM_Q8_0: return launch_kind<OPENMINI_QMM_Q8_0, kGate, kX2>(w, x, x_exp, y, m, kx, s);
    case OPENMINI_QMM_Q4_K: return launch_kind<OPENMINI_QMM_Q4_K, kGate, kX2>(w, x, x_exp, y, m, kx, s);
    case OPENMINI_QMM_Q6_K: return launch_kind<OPENMINI_QMM_Q6_K, kGate, kX2>(w, x, x_exp, y, m, kx, s);
    default: return hipErrorInvalidValue;
    }
}

// fp32 activations for the fp16 MFMA: row m of x [m, k] is scaled by 2^e, e chosen so
// the row's largest |x| lands in [2^14, 2^15), and each element x' = x 2^e is split
// into hi = x' rounded toward zero to fp16 (11 significant bits) and lo = x' - hi
// (exact in fp32, at most 13 bits, |lo| < 2^-10 |x'|) rounded to nearest fp16: the
// pair carries x' to within 2^-22 |x'|, and to within 2^-25 absolute (2^-39 of the
// row maximum) for elements more than 2^17 below it, where lo is an fp16 subnormal.
// Written per 32-element block as 32 hi then 32 lo (x2 row = 2 k fp16), e in
// x_exp[m].  A row holding inf or NaN is written as NaN (hi) and 0 (lo) with e = 0,
// so every output of that row is NaN (the decode GEMVs do the same).  One workgroup
// per row; x rows 16-byte aligned (k % 32 == 0).
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ x, uint16_t* __restrict__ x2,
                                                         int* __restrict__ x_exp, int k) {
    __shared__ uint32_t wave_max[4];
    const size_t row = blockIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + row * (size_t)k);
    const int quads = k / 4;
    uint32_t mx = 0;  // largest |x| as bits (inf / NaN above every finite value)
    for (int i = (int)threadIdx.x; i < quads; i += 256) {
        const float4 v = xr[i];
        mx = max(max(mx, __float_as_uint(v.x) & 0x7FFFFFFFu), __float_as_uint(v.y) & 0x7FFFFFFFu);
        mx = max(max(mx, __float_as_uint(v.z) & 0x7FFFFFFFu), __float_as_uint(v.w) & 0x7FFFFFFFu);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
    if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = max(max(wave_max[0], wave_max[1]), max(wave_max[2], wave_max[3]));
    const bool bad = mx >= 0x7F800000u;
    // max |x| in [2^(f - 1), 2^f): e = 15 - f puts it in [2^14, 2^15)
    const int e = (bad || mx == 0) ? 0 : 15 - __builtin_amdgcn_frexp_expf(__uint_as_float(mx));
    uint16_t* out = x2 + row * (size_t)(2 * k);
    for (int i = (int)threadIdx.x; i < quads; i += 256) {
        const float4 v = xr[i];
        uint2 hi, lo;
        if (bad) {
            hi = make_uint2(0x7E007E00u, 0x7E007E00u);  // fp16 NaN
            lo = make_uint2(0u, 0u);
        } else {
            const float a0 = __builtin_amdgcn_ldexpf(v.x, e), a1 = __builtin_amdgcn_ldexpf(v.y, e);
            const float a2 = __builtin_amdgcn_ldexpf(v.z, e), a3 = __builtin_amdgcn_ldexpf(v.w, e);
            const auto h01 = __builtin_amdgcn_cvt_pkrtz(a0, a1), h23 = __builtin_amdgcn_cvt_pkrtz(a2, a3);
            hi = make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
            const f16x2 l01 = {(_Float16)(a0 - (float)h01[0]), (_Float16)(a1 - (float)h01[1])};
            const f16x2 l23 = {(_Float16)(a2 - (float)h23[0]), (_Float16)(a3 - (float)h23[1])};
            lo = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
        }
        const int b = i >> 3, e0 = (i & 7) * 4;  // 32-element block, element within it
        *reinterpret_cast<uint2*>(out + b * 64 + e0) = hi;
        *reinterpret_cast<uint2*>(out + b * 64 + 32 + e0) = lo;
    }
    if (threadIdx.x == 0) x_exp[row] = e;
}

// Compute-only ceiling of the prefill GEMM (Q4_0 / Q8_0): gemm_kernel's grid and
// waves, each running only its per-block register work -- kCeilWT code conversions,
// kMI x kCeilWT MFMAs and their rescale FMAs, in the same order -- for as many blocks as
// its K part holds, on operands that stay in registers.  No loads, LDS, barriers or
// stores (a sentinel store keeps the work live), so its time is what the GEMM's
// instruction mix alone costs under the same clock and power conditions.
template <int kFmt, int kMI>
__global__ __launch_bounds__(512) void gemm_ceiling_kernel(int blocks, float* __restrict__ sink) {
    constexpr bool kNib = kFmt == OPENMINI_QMM_Q4_0;
    const int lane = threadIdx.x & 63;
    bf16x8 a[kMI];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) a[i][e] = (__bf16)((float)((lane + 7 * i + e) & 15) * 0.125f);
    uint32_t c0[kCeilWT], c1[kCeilWT], sc[kCeilWT];
#pragma unroll
    for (int j = 0; j < kCeilWT; ++j) {
        c0[j] = 0x01030507u * (uint32_t)(lane + j + 1);
        c1[j] = 0x02040608u * (uint32_t)(lane + j + 1);
        sc[j] = 0x3C00u;  // fp16 1.0
    }
    f32x4 acc[kMI][kCeilWT];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int j = 0; j < kCeilWT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < blocks; ++b) {
        // new operands every block, as the A-fragment reads and weight loads give
#pragma unroll
        for (int i = 0; i < kMI; ++i) asm volatile("" : "+v"(a[i]));
#pragma unroll
        for (int j = 0; j < kCeilWT; ++j) asm volatile("" : "+v"(c0[j]), "+v"(c1[j]), "+v"(sc[j]));
        bf16x8 bq[kCeilWT];
        float d[kCeilWT];
#pragma unroll
        for (int j = 0; j < kCeilWT; ++j) {
            if constexpr (kNib) {
                bq[j] = cvt_q4(c0[j]);
                d[j] = f16_bits_to_f32((uint16_t)sc[j]) * 16.0f;
            } else {
                bq[j] = cvt_q8(c0[j], c1[j]);
                d[j] = f16_bits_to_f32((uint16_t)sc[j]);
            }
        }
        f32x4 pp[2];
        pp[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], bq[0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < kMI * kCeilWT; ++q) {
            if (q + 1 < kMI * kCeilWT)
                pp[(q + 1) & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    a[(q + 1) / kCeilWT], bq[(q + 1) % kCeilWT], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[q / kCeilWT][q % kCeilWT][r] = fmaf(pp[q & 1][r], d[q % kCeilWT], acc[q / kCeilWT][q % kCeilWT][r]);
        }
    }
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int j = 0; j < kCeilWT; ++j) t += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
    if (t == 1234.5f) sink[0] = t;
}

template <int kFmt>
hipError_t launch_ceiling(int64_t m, int64_t n_tiles, int64_t k, float* sink, hipStream_t s) {
    // the grid, workgroup and K split of launch_kind's two shapes
    const bool small = m <= kBMMax;
    const int bm = small ? 64 : 128, threads = small ? 512 : 256, parts = small ? 4 : 2;
    const int64_t bt = 2 * kCeilWT;  // weight tiles per workgroup (2 column slices)
    const dim3 grid((unsigned)((n_tiles + bt - 1) / bt), (unsigned)((m + bm - 1) / bm));
    const int blocks = (int)((k / kQK + parts - 1) / parts);
    if (small)
        hipLaunchKernelGGL((gemm_ceiling_kernel<kFmt, 4>), grid, dim3(threads), 0, s, blocks, sink);
    else
        hipLaunchKernelGGL((gemm_ceiling_kernel<kFmt, 8>), grid, dim3(threads), 0, s, blocks, sink);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_ceiling(int type, int64_t m, int64_t n, int64_t k, float* sink, hipStream_t s) {
    const int64_t n_tiles = (n + kTileRows - 1) / kTileRows;
    if (m <= 0 || n <= 0 || k <= 0 || (m + 127) / 128 > 65535 || n_tiles > INT32_MAX) return hipErrorInvalidValue;
    if (type == OPENMINI_QMM_Q4_0) return launch_ceiling<OPENMINI_QMM_Q4_0>(m, n_tiles, k, sink, s);
    if (type == OPENMINI_QMM_Q8_0) return launch_ceiling<OPENMINI_QMM_Q8_0>(m, n_tiles, k, sink, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_bf16(const Weight& w, const uint16_t* x, float* y, int64_t m, hipStream_t s,
                            bool gate_in_y) {
    // x offsets are 32-bit: launches cover row ranges whose x is below 2 GiB.
    const int64_t rows_per_launch = ((((int64_t)1 << 31) - 1) / (w.k * 2)) / kBMMax * kBMMax;
    if (rows_per_launch <= 0) return hipErrorInvalidValue;  // one row tile of x exceeds 2 GiB
    for (int64_t m_off = 0; m_off < m; m_off += rows_per_launch) {
        const int64_t mm = m - m_off < rows_per_launch ? m - m_off : rows_per_launch;
        const uint16_t* xs = x + m_off * w.k;
        float* ys = y + m_off * w.n;
        const hipError_t e = gate_in_y ? launch_type<true, false>(w, xs, nullptr, ys, mm, w.k, s)
                                       : launch_type<false, false>(w, xs, nullptr, ys, mm, w.k, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int gemm_shape(const Weight& w, int64_t m, bool split_x) {
    switch (w.type) {
    case OPENMINI_QMM_Q4_0:
        return split_x ? choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q4_0, false, true>(), split_x)
                       : choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q4_0, false, false>(), split_x);
    case OPENMINI_QMM_Q8_0:
        return split_x ? choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q8_0, false, true>(), split_x)
                       : choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q8_0, false, false>(), split_x);
    case OPENMINI_QMM_Q4_K:
        return split_x ? choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q4_K, false, true>(), split_x)
                       : choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q4_K, false, false>(), split_x);
    case OPENMINI_QMM_Q6_K:
        return split_x ? choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q6_K, false, true>(), split_x)
                       : choose_shape(w, m, shape_occupancy<OPENMINI_QMM_Q6_K, false, false>(), split_x);
    default: return -1;
    }
}

size_t gemm_f32_workspace_bytes(int64_t m, int64_t k) {
    return (((size_t)m * (size_t)k * 4 + 255) & ~(size_t)255) + (size_t)m * 4;
}

hipError_t split_rows(const float* x, int64_t m, int64_t k, void* work, hipStream_t s) {
    if (m <= 0 || m > INT32_MAX || k <= 0 || k % kQK != 0 || k > INT32_MAX / 2) return hipErrorInvalidValue;
    uint16_t* x2 = static_cast<uint16_t*>(work);
    int* x_exp = reinterpret_cast<int*>(static_cast<uint8_t*>(work) + (gemm_f32_workspace_bytes(m, k) - (size_t)m * 4));
    hipLaunchKernelGGL(split_rows_kernel, dim3((unsigned)m), dim3(256), 0, s, x, x2, x_exp, (int)k);
    return hipGetLastError();
}

hipError_t launch_gemm_split(const Weight& w, const void* work, int64_t m, float* y, hipStream_t s, bool gate_in_y) {
    const uint16_t* x2 = static_cast<const uint16_t*>(work);
    const int* x_exp =
        reinterpret_cast<const int*>(static_cast<const uint8_t*>(work) + (gemm_f32_workspace_bytes(m, w.k) - (size_t)m * 4));
    const int64_t kx = 2 * w.k;  // fp16 elements per split row
    const int64_t rows_per_launch = ((((int64_t)1 << 31) - 1) / (kx * 2)) / kBMMax * kBMMax;
    if (rows_per_launch <= 0) return hipErrorInvalidValue;
    for (int64_t m_off = 0; m_off < m; m_off += rows_per_launch) {
        const int64_t mm = m - m_off < rows_per_launch ? m - m_off : rows_per_launch;
        const uint16_t* xs = x2 + m_off * kx;
        const int* es = x_exp + m_off;
        float* ys = y + m_off * w.n;
        const hipError_t e = gate_in_y ? launch_type<true, true>(w, xs, es, ys, mm, kx, s)
                                       : launch_type<false, true>(w, xs, es, ys, mm, kx, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace qmm
