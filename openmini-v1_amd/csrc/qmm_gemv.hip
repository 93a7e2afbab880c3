// Decode GEMV: y[b, n] = sum_k x[b, k] * w[n, k] for 1..4 fp32 activation rows.
//
// Replaces, per call of linear()/linear_gemm() (openmini-server/src/model/inference/
// model.rs:1050-1064), the W^T copy plus f32 sgemm over weights dequantized at load.
// Here W stays quantized in HBM (0.5625 B/weight Q4_0, 1.0625 B/weight Q8_0), is read
// exactly once and streams from HBM; the kernel is HBM-bound.
//
// Arithmetic: exact integer dot products on the matrix cores.
//   * Per 32-element block, x is made block-floating: with M the block's max |x| and
//     2^(e-1) <= M < 2^e, X_k = round-to-nearest-even(x_k * 2^s), s = 30 - e, so
//     |X_k| < 2^30 and the error is <= 2^(e-31).  Elements within 2^6 of the block
//     maximum are exact (24 significant bits); smaller ones are rounded 2^-31 below
//     the maximum, which keeps the error of an outlier's block (an outlier on a
//     feature the weight row ignores) below the fp32 accumulation error of the
//     reference's f32 path.
//   * X_k = sum_h digit_h * 2^(8h), h = 0..3, with balanced int8 digits: the bytes of
//     (X + 0x80808080) ^ 0x80808080.
//   * v_mfma_i32_16x16x64_i8 forms sum_k c_k * digit_k exactly in int32, with c_k the
//     Q8_0 code or 16 (q_k - 8) for Q4_0 (the stored two's-complement nibble moved to
//     the top of its byte: 1.5 VALU ops per 4 weights).
//   * Per block: sum_k c_k x_k = 2^-s * ((D_0 + 2^8 D_1) + 2^16 (D_2 + 2^8 D_3)) (the
//     two halves exact in int32, their combination rounded once in fp32), times the
//     block's fp16 scale (and 1/16 for Q4_0), accumulated in fp32.
// Versus unpack + convert + FMA on the VALU (about 2.3 instructions per weight, most
// of the VALU budget at HBM speed), this is well under 1 per weight.
//
// MFMA mapping (A 16x64 activation digits, B 64x16 codes, D 16x16): the 64 k
// positions are four 16-element parts; part t is block slot t of a 4-block group.
// Lane l = 16t + n feeds row n's block-t codes -- exactly slot l of the (row tile,
// group) chunk, so a wave-wide load of a chunk's codes is one contiguous 1 KB (Q4_0)
// / 2 KB (Q8_0), followed by the 128 B of its scales.  A row 4t + h holds digit h of
// block t (other parts zero), so D[4t + h][n] is digit h's block-t dot product for
// row n, in lane (n, t), register h: the 16 rows are exactly 4 blocks x 4 digits.
// Two MFMAs cover a block's 32 elements.
//
// One launch can serve several weights that share x and K:
//   * kGroup: up to kMaxGroup weights (q / k / v projections); workgroup i takes
//     tile i - tile_begin[g] of weight g, where tile_begin partitions the grid;
//   * kPair: one (gate, up) pair of equal shape; every workgroup runs the same tile
//     of both weights on the same activation digits and writes silu(gate) * up, the
//     hidden state of the FFN (model.rs:713-735 with silu at :1187-1189:
//     v / (1 + exp(-v))).
//
// Work split: a workgroup owns one 16-row tile; its W waves split the K groups into
// contiguous slices (contiguous runs of the weight).  A wave walks its slice in
// phases of up to P groups: it first issues the phase's activation loads (L2 hits,
// ready long before the weights), then the chunk loads, turns the activations into
// digits (block max by DPP butterflies within the 16-lane row that holds a block,
// A fragments through LDS) while the chunks are still in flight, and finally runs
// the MFMAs as the chunks arrive.  The W partial sums of a row meet in LDS and are
// added in wave order (deterministic).
#include "qmm_device.hpp"

namespace qmm {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// DPP lane patterns inside a 16-lane row.
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each 16 lanes

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, true);
}

// Butterfly max over the 16 lanes of a row (every lane ends with the row result);
// each step compiles to one DPP-modified integer op.  It runs on the bit patterns of
// non-negative floats, which order like unsigned integers.
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
    v = max(v, dpp<kDppXor1>(v));
    v = max(v, dpp<kDppXor2>(v));
    v = max(v, dpp<kDppHalfMirror>(v));
    v = max(v, dpp<kDppMirror>(v));
    return v;
}

// Sum over the 16 lanes of a row, the same butterfly with adds (every lane ends with
// the same value: each step adds the same two operands in both lanes of a pair).
__device__ __forceinline__ float row16_sum(float v) {
    v += __uint_as_float(dpp<kDppXor1>(__float_as_uint(v)));
    v += __uint_as_float(dpp<kDppXor2>(__float_as_uint(v)));
    v += __uint_as_float(dpp<kDppHalfMirror>(__float_as_uint(v)));
    v += __uint_as_float(dpp<kDppMirror>(__float_as_uint(v)));
    return v;
}

// Sum over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48), in every
// lane, with the gfx950 row swaps (registers only, no LDS round trip).  Each step adds
// the same two values in every lane of a row pair, so the result is the one of
// v + v[l ^ 16], then + [l ^ 32].
__device__ __forceinline__ float sum_rows(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);  // rows (0, 0, 2, 2), (1, 1, 3, 3)
    const float w = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const uint32_t x = __float_as_uint(w);
    const auto q = __builtin_amdgcn_permlane32_swap(x, x, false, false);  // rows (0, 1, 0, 1), (2, 3, 2, 3)
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// v_cvt_i32_f32: float -> int32, toward zero, saturating (NaN -> 0).  Written out
// because a C++ conversion of a non-finite or out-of-range float is undefined.
__device__ __forceinline__ int cvt_i32(float v) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// One block's digit dot products (D_h: register h) -> their weighted sum
// D_0 + 2^8 D_1 + 2^16 (D_2 + 2^8 D_3): |D_h| <= 2^19, so each half is exact in int32
// and the combination rounds once in fp32.
__device__ __forceinline__ float digit_sum(const i32x4& D) {
    const int lo = D[0] + (int)((uint32_t)D[1] << 8), hi = D[2] + (int)((uint32_t)D[3] << 8);
    return fmaf((float)hi, 65536.0f, (float)lo);
}


// The weights of one launch (kernel argument, uniform).
struct GemvGroup {
    int tile_begin[kMaxGroup + 1];     // grid partition: weight g owns [tile_begin[g], tile_begin[g+1]);
                                       // entries past the last weight hold the grid size
    const uint8_t* chunks[kMaxGroup];  // a pair: [0] gate, [1] up
    float* y[kMaxGroup];
    int n_rows[kMaxGroup];
};

// LDS A-fragment slots of one wave for one phase: [p][b][u = block half][t = block
// slot][h = digit], 16 bytes each, then one zero slot read by lanes whose A fragment
// is zero.
constexpr int kDigits = 4;
template <int B, int P>
constexpr int kSlots = P * B * 2 * 4 * kDigits + 1;

// The leading arguments describe weight 0 (and the up weight of a pair) and fit the
// SGPRs the kernel arguments are preloaded into; `grp` is read only by workgroups of
// the later weights of a group.
// Launch kinds: one weight, a group of weights sharing x (tiles partitioned), or a
// (gate, up) pair run on the same tiles.
constexpr int kOne = 0, kGroup = 1, kPair = 2;

// Chunk geometry of a weight format (kFmt = its GGUF type id; qmm_internal.hpp):
// bytes of a slot's codes, where the per-slot scale and the per-row d live, and the
// power of two the int8 code bytes carry (Q4_0 / Q4_K codes are 16 (q - 8), Q6_K 4 q).
template <int kFmt>
struct Fmt {
    static constexpr bool kQ41 = kFmt == OPENMINI_QMM_Q4_1;
    static constexpr bool kQ5 = kFmt == OPENMINI_QMM_Q5_K;
    static constexpr bool kNib = kFmt == OPENMINI_QMM_Q4_0 || kFmt == OPENMINI_QMM_Q4_K || kQ41;  // 16 B of nibbles
    static constexpr bool kQ6 = kFmt == OPENMINI_QMM_Q6_K || kQ5;                        // Q6_K chunk layout
    static constexpr bool kKQ = kFmt == OPENMINI_QMM_Q4_K || kQ6;                        // K-quant
    static constexpr bool kMin = kQ41 || kQ5;                                            // block minimum
    static constexpr int kCB = kNib ? 16 : kQ6 ? 24 : 32;
    static constexpr int kCodeBytes = kTileEntries * kCB;
    static constexpr int kChunk = kFmt == OPENMINI_QMM_Q4_K ? kQ4KChunk
                                  : kQ5                     ? kQ5KChunk
                                  : kQ6                     ? kQ6KChunk
                                  : kQ41                    ? kQ41Chunk
                                                            : chunk_bytes_for(kFmt == OPENMINI_QMM_Q4_0);
    static constexpr int kDOff = kQ5 ? kQ5KDOff : kCodeBytes + (kQ6 ? 2 : 1) * kTileEntries;  // K-quant: fp16 d per row
    static constexpr int kCodeShift = kNib ? 4 : kQ6 ? 2 : 0;
};

template <int kFmt, int B, int W, int P, int kKind>
__global__ __launch_bounds__(64 * W) void gemv_kernel(const uint8_t* __restrict__ w0,
                                                      const uint8_t* __restrict__ w1,
                                                      const float* __restrict__ x, float* __restrict__ y0,
                                                      int n_rows0, int tiles0, int groups, int k,
                                                      const GemvGroup grp) {
    using F = Fmt<kFmt>;
    constexpr int kNW = kKind == kPair ? 2 : 1;  // weights per tile
    constexpr int kCodeBytes = F::kCodeBytes;
    constexpr int kChunk = F::kChunk;
    constexpr int kS = kSlots<B, P>;
    constexpr int kZero = kS - 1;
    // Q5_K with eight waves holds 56 KB of LDS so that at most two workgroups share a
    // CU.  Its 72 registers would let three in, and on 256-workgroup grids (4096-row
    // weights) the room was filled unevenly: interleaved A/B on one box, 4096 x 11008
    // b = 1 11.4 -> 9.4 us, b = 2 14.2 -> 11.7 us; 11008 x 4096 b = 1 8.3 -> 8.5-8.8 us.
    constexpr int kSAlloc = F::kQ5 && W == 8 && kS < 56 * 1024 / 16 / W ? 56 * 1024 / 16 / W : kS;
    __shared__ uint4 a_lds[W][kSAlloc];
    __shared__ float red[W][kNW][B][16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform per wave
    const int ln = lane & 15, lt = lane >> 4;
    // This workgroup's weight (uniform): weight 0 below tiles0, else the last g with
    // tile_begin[g] <= blockIdx.x (entries past the group's count hold the grid size).
    int tile_lo = 0, tile_hi = tiles0, n_rows = n_rows0;
    float* __restrict__ y = y0;
    const uint8_t* wp[kNW];
    wp[0] = w0;
    if constexpr (kNW == 2) wp[1] = w1;
    if constexpr (kKind == kGroup) {
        if ((int)blockIdx.x >= tiles0) {
#pragma unroll
            for (int i = 1; i < kMaxGroup; ++i) {
                const bool mine = (int)blockIdx.x >= grp.tile_begin[i];
                tile_lo = mine ? grp.tile_begin[i] : tile_lo;
                tile_hi = mine ? grp.tile_begin[i + 1] : tile_hi;
                n_rows = mine ? grp.n_rows[i] : n_rows;
                y = mine ? grp.y[i] : y;
                wp[0] = mine ? grp.chunks[i] : wp[0];
            }
        }
    }
    const int tile = (int)blockIdx.x - tile_lo;
    const int n_tiles = tile_hi - tile_lo;
    const int g0 = (int)((int64_t)groups * wave / W);
    const int g1 = (int)((int64_t)groups * (wave + 1) / W);

    // The chunks are < 4 GiB (checked at upload), so 32-bit buffer offsets suffice.
    __amdgpu_buffer_rsrc_t w_rs[kNW];
#pragma unroll
    for (int nw = 0; nw < kNW; ++nw)
        w_rs[nw] = make_rsrc(wp[nw], (uint32_t)n_tiles * groups * kChunk);
    __amdgpu_buffer_rsrc_t x_rs[B];
#pragma unroll
    for (int b = 0; b < B; ++b) x_rs[b] = make_rsrc(x + (size_t)b * k, (uint32_t)k * 4);
    const uint32_t tile_off = (uint32_t)tile * groups * kChunk;

    uint4* my_lds = a_lds[wave];
    if (lane == 0) my_lds[kZero] = make_uint4(0, 0, 0, 0);
    // This lane's A fragment: row m = ln = 4*at + ah of part lt, live iff at == lt; its
    // slot (t = at, h = ah) is then slot ln of the block half.
    const bool a_live = (ln >> 2) == lt;
    constexpr int kHalfSlots = 4 * kDigits;  // slots of one block half: (t, h)
    // Where this lane writes its two elements' digits: slot (u = ln / 8, t = lt, h),
    // halfword ln % 8 (a slot is 8 halfwords).
    uint16_t* wr16 =
        reinterpret_cast<uint16_t*>(my_lds) + ((ln >> 3) * kHalfSlots + lt * kDigits) * 8 + (ln & 7);

    float acc[kNW][B];
#pragma unroll
    for (int nw = 0; nw < kNW; ++nw)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[nw][b] = 0.0f;
    // Max of the bit patterns of |x| (they order like unsigned integers): finite x stays
    // below 0x7F800000, an inf or NaN reaches it.  Tracked per batch row: a non-finite
    // row poisons only its own outputs.
    uint32_t seen[B];
#pragma unroll
    for (int b = 0; b < B; ++b) seen[b] = 0;

    for (int g = g0; g < g1; g += P) {
        // A phase is straight-line code (branches would make the compiler wait for
        // every load at their joins): groups past the slice end re-read the slice's
        // last group (a cache hit) and get scale 0.
        int gp[P];
#pragma unroll
        for (int p = 0; p < P; ++p) gp[p] = min(g + p, g1 - 1);
        float2 xv[P][B];
        uint4 c[kNW][P][F::kNib ? 1 : 2];
        uint2 hb[kNW][P];      // Q6_K: the slot's 8 bytes of top code bits
        uint32_t sc[kNW][P];   // the slot's scale: fp16 bits (Q4_0 / Q8_0), u8 (Q4_K), 2 x int8 (Q6_K)
        uint32_t dk[kNW][P];   // K-quant: the row's fp16 d
        uint32_t mn[kNW][P];   // block minimum: Q4_1 the slot's fp16 m, Q5_K its minimum nibble
        uint32_t dm[kNW][P];   // Q5_K: the row's fp16 dmin
        // activations first: L2 hits that land before the weights do.  The whole offset
        // goes in the VGPR operand: the raw-buffer range check covers the VGPR offset
        // but not the SGPR one, so elements past k (a last group of fewer than 4
        // blocks) get an offset past the range and read zero without touching memory.
        uint32_t xoff[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t e = (uint32_t)gp[p] * 512u + (uint32_t)lane * 8u;
            xoff[p] = e < (uint32_t)k * 4u ? e : 0x80000000u;
        }
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int b = 0; b < B; ++b)
                xv[p][b] = __builtin_bit_cast(float2,
                                              __builtin_amdgcn_raw_buffer_load_b64(x_rs[b], xoff[p], 0, 0));
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t soff = tile_off + (uint32_t)gp[p] * kChunk;
#pragma unroll
            for (int nw = 0; nw < kNW; ++nw) {
                c[nw][p][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                            w_rs[nw], lane * (F::kQ6 ? 16 : F::kCB), soff, 0));
                if constexpr (kFmt == OPENMINI_QMM_Q8_0)
                    c[nw][p][1] = __builtin_bit_cast(
                        uint4, __builtin_amdgcn_raw_buffer_load_b128(w_rs[nw], lane * 32 + 16, soff, 0));
                if constexpr (F::kQ5)  // the slot's high-bit byte
                    hb[nw][p].x = __builtin_amdgcn_raw_buffer_load_b8(w_rs[nw], kQ5KQhOff + lane, soff, 0);
                else if constexpr (F::kQ6)
                    hb[nw][p] = __builtin_bit_cast(
                        uint2, __builtin_amdgcn_raw_buffer_load_b64(w_rs[nw], kTileEntries * 16 + lane * 8, soff, 0));
                if constexpr (kFmt == OPENMINI_QMM_Q4_K)
                    sc[nw][p] = __builtin_amdgcn_raw_buffer_load_b8(w_rs[nw], kCodeBytes + lane, soff, 0);
                else if constexpr (F::kQ5)
                    sc[nw][p] = __builtin_amdgcn_raw_buffer_load_b8(w_rs[nw], kQ5KScaleOff + lane, soff, 0);
                else
                    sc[nw][p] = __builtin_amdgcn_raw_buffer_load_b16(w_rs[nw], kCodeBytes + lane * 2, soff, 0);
                if constexpr (F::kKQ)
                    dk[nw][p] = __builtin_amdgcn_raw_buffer_load_b16(w_rs[nw], F::kDOff + ln * 2, soff, 0);
                if constexpr (F::kQ41)
                    mn[nw][p] = __builtin_amdgcn_raw_buffer_load_b16(w_rs[nw], kQ41MinOff + lane * 2, soff, 0);
                if constexpr (F::kQ5) {
                    mn[nw][p] = __builtin_amdgcn_raw_buffer_load_b8(w_rs[nw], kQ5KMinOff + lane, soff, 0);
                    dm[nw][p] = __builtin_amdgcn_raw_buffer_load_b16(w_rs[nw], kQ5KDminOff + ln * 2, soff, 0);
                }
            }
        }

        // digits of the phase's activation blocks -> LDS, while the chunks are in flight
        int shift[P][B];
        float bsum[P][B];  // block minimum: the sum of the lane's block of activations
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float x0 = xv[p][b].x, x1 = xv[p][b].y;
                const uint32_t mb = row16_max(max(__float_as_uint(x0) & 0x7FFFFFFFu,
                                                  __float_as_uint(x1) & 0x7FFFFFFFu));
                seen[b] = max(seen[b], mb);
                if constexpr (F::kMin) bsum[p][b] = row16_sum(x0 + x1);
                // 2^(e-1) <= max < 2^e with e = biased exponent - 126; s = 30 - e
                shift[p][b] = 156 - (int)(mb >> 23);
                // X = round(x * 2^s), |X| < 2^30 (x * 2^s is an integer from 2^23 up);
                // cvt_i32 also takes the inf / NaN of a non-finite block (its row's
                // outputs become NaN below)
                const int X0 = cvt_i32(__builtin_rintf(__builtin_amdgcn_ldexpf(x0, shift[p][b])));
                const int X1 = cvt_i32(__builtin_rintf(__builtin_amdgcn_ldexpf(x1, shift[p][b])));
                // bytes of (X + 0x80808080) ^ 0x80808080: the balanced digits, low first
                const uint32_t z0 = ((uint32_t)X0 + 0x80808080u) ^ 0x80808080u;
                const uint32_t z1 = ((uint32_t)X1 + 0x80808080u) ^ 0x80808080u;
                uint16_t* w16 = wr16 + (p * B + b) * 2 * kHalfSlots * 8;
#pragma unroll
                for (int h = 0; h < kDigits; ++h)
                    w16[h * 8] = (uint16_t)__builtin_amdgcn_perm(z1, z0, (uint32_t)(h | ((4 + h) << 8) | 0x0C0C0000u));
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int nw = 0; nw < kNW; ++nw) {
                i32x4 b0, b1;
                if constexpr (F::kNib) {
                    // 16 * (q - 8) as int8 bytes, elements in order
                    const uint4 w = c[nw][p][0];
                    b0 = i32x4{(int)((w.x << 4) & 0xF0F0F0F0u), (int)(w.x & 0xF0F0F0F0u),
                               (int)((w.y << 4) & 0xF0F0F0F0u), (int)(w.y & 0xF0F0F0F0u)};
                    b1 = i32x4{(int)((w.z << 4) & 0xF0F0F0F0u), (int)(w.z & 0xF0F0F0F0u),
                               (int)((w.w << 4) & 0xF0F0F0F0u), (int)(w.w & 0xF0F0F0F0u)};
                } else if constexpr (F::kQ6) {
                    // 4 q as int8 bytes: low 4 bits of the 6-bit code at bits 2..5, its top
                    // 2 bits at 6..7 (field f of top-bit word m: element 16 m + 4 f + i)
                    const uint4 w = c[nw][p][0];
                    uint2 h = hb[nw][p];
                    if constexpr (F::kQ5) {
                        // Q5_K: the top 2 bits of the code q - 16 are 3 where the element's
                        // high bit is 0, else 0; element e's high bit is bit e % 8 of the
                        // slot's byte, so both top-bit words are one word: byte i =
                        // 0x33 (1 - bit i) + 0xCC (1 - bit 4 + i)
                        const uint32_t nb = ~h.x & 0xFFu;
                        const uint32_t x2 = spread4(nb & 0xFu) | (spread4(nb >> 4) << 2);
                        const uint32_t y2 = x2 | (x2 << 1);
                        h.x = h.y = y2 | (y2 << 4);
                    }
                    auto lo = [](uint32_t wj, uint32_t hm, int sh) {
                        return (int)(((wj << 2) & 0x3C3C3C3Cu) | ((hm << sh) & 0xC0C0C0C0u));
                    };
                    auto hi = [](uint32_t wj, uint32_t hm, int sh) {
                        return (int)(((wj >> 2) & 0x3C3C3C3Cu) | ((hm << sh) & 0xC0C0C0C0u));
                    };
                    b0 = i32x4{lo(w.x, h.x, 6), hi(w.x, h.x, 4), lo(w.y, h.x, 2), hi(w.y, h.x, 0)};
                    b1 = i32x4{lo(w.z, h.y, 6), hi(w.z, h.y, 4), lo(w.w, h.y, 2), hi(w.w, h.y, 0)};
                } else {
                    const uint4 w0 = c[nw][p][0], w1 = c[nw][p][1];
                    b0 = i32x4{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w};
                    b1 = i32x4{(int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                }
                // the slot's fp32 factor(s), exact: fp16 scale; Q4_K d * scale; Q6_K d * scale
                // of each 16-element half; Q5_K d * scale (its two scale bytes are equal).
                // Groups past the slice end get 0.
                const bool live = g + p < g1;
                float d0, d1 = 0.0f;
                if constexpr (kFmt == OPENMINI_QMM_Q4_K) {
                    d0 = f16_bits_to_f32((uint16_t)dk[nw][p]) * (float)sc[nw][p];
                } else if constexpr (F::kQ6) {
                    const float dd = f16_bits_to_f32((uint16_t)dk[nw][p]);
                    d0 = dd * (float)(int8_t)(sc[nw][p] & 0xFFu);
                    d1 = dd * (float)(int8_t)((sc[nw][p] >> 8) & 0xFFu);
                    d1 = live ? d1 : 0.0f;
                } else {
                    d0 = f16_bits_to_f32((uint16_t)sc[nw][p]);
                }
                d0 = live ? d0 : 0.0f;
                // block minimum offset: Q4_1 (q - 8) d + (8 d + m); Q5_K dmin * minimum
                float mo = 0.0f;
                if constexpr (F::kQ41) mo = fmaf(8.0f, d0, f16_bits_to_f32((uint16_t)mn[nw][p]));
                if constexpr (F::kQ5) mo = f16_bits_to_f32((uint16_t)dm[nw][p]) * (float)mn[nw][p];
                mo = live ? mo : 0.0f;
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    const int base = (p * B + b) * 2 * kHalfSlots;
                    const uint4 v0 = my_lds[a_live ? base + ln : kZero];
                    const uint4 v1 = my_lds[a_live ? base + kHalfSlots + ln : kZero];
                    const i32x4 A0 = i32x4{(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w};
                    const i32x4 A1 = i32x4{(int)v1.x, (int)v1.y, (int)v1.z, (int)v1.w};
                    const int sh = -shift[p][b] - F::kCodeShift;
                    if constexpr (F::kQ6 && !F::kQ5) {
                        // the halves carry different scales: one MFMA each, not chained
                        const i32x4 D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, b0, i32x4{0, 0, 0, 0}, 0, 0, 0);
                        const i32x4 D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, b1, i32x4{0, 0, 0, 0}, 0, 0, 0);
                        acc[nw][b] = fmaf(d0, __builtin_amdgcn_ldexpf(digit_sum(D0), sh), acc[nw][b]);
                        acc[nw][b] = fmaf(d1, __builtin_amdgcn_ldexpf(digit_sum(D1), sh), acc[nw][b]);
                        if constexpr (F::kMin) acc[nw][b] = fmaf(mo, bsum[p][b], acc[nw][b]);
                    } else {
                        i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, b0, i32x4{0, 0, 0, 0}, 0, 0, 0);
                        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, b1, D, 0, 0, 0);
                        acc[nw][b] = fmaf(d0, __builtin_amdgcn_ldexpf(digit_sum(D), sh), acc[nw][b]);
                        if constexpr (F::kMin) acc[nw][b] = fmaf(mo, bsum[p][b], acc[nw][b]);
                    }
                }
            }
        // The next phase rewrites this wave's slots; a wave's LDS operations complete
        // in order, so its reads above are done before those writes.
    }

    // Sum the four block slots (lanes n, n+16, n+32, n+48), then the W K slices.
    // Any inf / NaN activation turns the outputs into NaN.
    bool bad[B];
#pragma unroll
    for (int b = 0; b < B; ++b) bad[b] = __ballot(seen[b] >= 0x7F800000u) != 0;
#pragma unroll
    for (int nw = 0; nw < kNW; ++nw)
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float v = sum_rows(acc[nw][b]);
            if (bad[b]) v = __builtin_nanf("");
            if (lane < 16) red[wave][nw][b][lane] = v;
        }
    __syncthreads();
    if (wave == 0 && lane < 16) {
        const int row = tile * kTileRows + lane;
        if (row < n_rows) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float v[kNW];
#pragma unroll
                for (int nw = 0; nw < kNW; ++nw) {
                    v[nw] = red[0][nw][b][lane];
#pragma unroll
                    for (int w = 1; w < W; ++w) v[nw] += red[w][nw][b][lane];
                }
                if constexpr (kNW == 2)
                    y[(size_t)b * n_rows + row] = v[0] / (1.0f + expf(-v[0])) * v[1];
                else
                    y[(size_t)b * n_rows + row] = v[0];
            }
        }
    }
}

template <int kFmt, int B, int W, int P, int kKind>
hipError_t run(const GemvGroup& grp, int64_t groups, int64_t k, const float* x, hipStream_t s) {
    // gfx950 gives a workgroup up to 160 KB of LDS; 4 batch rows x 8 waves take 66 KB
    static_assert(sizeof(uint4) * W * kSlots<B, P> <= 80 * 1024, "A-fragment LDS over budget");
    const unsigned wgs = (unsigned)grp.tile_begin[kMaxGroup];
    hipLaunchKernelGGL((gemv_kernel<kFmt, B, W, P, kKind>), dim3(wgs), dim3(64 * W), 0, s, grp.chunks[0],
                       grp.chunks[1], x, grp.y[0], grp.n_rows[0], grp.tile_begin[1], (int)groups, (int)k, grp);
    return hipGetLastError();
}

// K slices per row tile (phases of 4 groups).  One batch row: W = 8 or 16, whichever
// pads the last phases with fewer groups; ties (K a multiple of 8192): 8, two phases
// per wave and twice the resident workgroups per CU (three interleaved passes, one
// box, 28672 x 8192: Q8_0 44.1-44.3 -> 41.9 us, also over 500 launches 43.8 -> 41.6;
// Q4_0 25.4-25.5 -> 24.4-24.6 us, over 500 launches even at 22.5-22.8; Q4_K 25.2-25.4
// -> 24.4-24.5 us).  E.g. K = 4096 -> 8, 11008 -> 8.  Nibble codes on at most 512 row tiles
// (two workgroups per CU or fewer) with K of 64+ groups: 16 waves of 2-group phases,
// twice the waves in flight (two interleaved passes, Q4_0: 4096 x 11008 7.25-7.58 ->
// 7.03-7.14 us, 8192 x 28672 26.7-27.3 -> 25.5-25.6, 8192 x 8192 8.40-8.51 ->
// 8.31-8.36; Q8_0 4096 x 11008 lost 10% and 4096 x 4096 (32 groups) gained nothing;
// Q6_K 4096 x 11008 9.0-9.1 -> 9.4-9.5, 8192 x 8192 11.5 -> 13.7-13.9, Q5_K 4096 x 11008
// 9.4 -> 10.4-10.5).
// Fewer, longer waves lose at the headline shape: 11008 x 4096 Q4_0 W = 8 6.29-6.33
// us, W = 4 (8-group phases) 6.64-6.67, W = 2 8.02-8.10.
// More batch rows: at most 8 (LDS and registers per wave grow with the batch).  Short
// K: the most slices that keep 4 groups per wave.
template <int kFmt, int B, int kKind>
hipError_t run_w(const GemvGroup& grp, int64_t g, int64_t k, const float* x, hipStream_t s) {
    if (g >= 32) {
        if constexpr (B == 1 && Fmt<kFmt>::kNib)
            if (g >= 64 && grp.tile_begin[kMaxGroup] <= 512) return run<kFmt, B, 16, 2, kKind>(grp, g, k, x, s);
        if constexpr (B == 1) {
            const int64_t pad16 = (g + 63) / 64 * 64 - g, pad8 = (g + 31) / 32 * 32 - g;
            if (pad16 < pad8) return run<kFmt, B, 16, 4, kKind>(grp, g, k, x, s);
        }
        return run<kFmt, B, 8, 4, kKind>(grp, g, k, x, s);
    }
    if (g >= 16) return run<kFmt, B, 4, 4, kKind>(grp, g, k, x, s);
    if (g >= 8) return run<kFmt, B, 2, 4, kKind>(grp, g, k, x, s);
    return run<kFmt, B, 1, 4, kKind>(grp, g, k, x, s);
}

template <int kFmt, int kKind>
hipError_t dispatch(const GemvGroup& grp, int64_t g, int64_t k, const float* x, int batch, hipStream_t s) {
    switch (batch) {
    case 1: return run_w<kFmt, 1, kKind>(grp, g, k, x, s);
    case 2: return run_w<kFmt, 2, kKind>(grp, g, k, x, s);
    case 3: return run_w<kFmt, 3, kKind>(grp, g, k, x, s);
    case 4: return run_w<kFmt, 4, kKind>(grp, g, k, x, s);
    default: return hipErrorInvalidValue;
    }
}

template <int kFmt>
hipError_t dispatch_kind(const GemvGroup& grp, const Weight& w0, const float* x, int batch, int count, bool swiglu,
                         hipStream_t s) {
    if (swiglu) return dispatch<kFmt, kPair>(grp, w0.groups, w0.k, x, batch, s);
    if (count > 1) return dispatch<kFmt, kGroup>(grp, w0.groups, w0.k, x, batch, s);
    return dispatch<kFmt, kOne>(grp, w0.groups, w0.k, x, batch, s);
}

}  // namespace

hipError_t launch_gemv_group(const Weight* const* ws, float* const* ys, int count, const float* x, int batch,
                             bool swiglu, hipStream_t s) {
    if (count < 1 || count > kMaxGroup || (swiglu && count != 2)) return hipErrorInvalidValue;
    GemvGroup grp{};
    const int owners = swiglu ? 1 : count;  // weights that own tiles of the grid
    int64_t tiles = 0;
    for (int i = 0; i < count; ++i) {
        grp.chunks[i] = ws[i]->chunks;
        grp.n_rows[i] = (int)ws[i]->n;
        grp.y[i] = ys[swiglu ? 0 : i];
        if (!swiglu || i == 0) {
            grp.tile_begin[i] = (int)tiles;
            tiles += ws[i]->n_tiles;
        }
    }
    for (int i = owners; i <= kMaxGroup; ++i) grp.tile_begin[i] = (int)tiles;
    if (tiles > INT32_MAX) return hipErrorInvalidValue;
    const Weight& w0 = *ws[0];
    switch (w0.type) {
    case OPENMINI_QMM_Q4_0: return dispatch_kind<OPENMINI_QMM_Q4_0>(grp, w0, x, batch, count, swiglu, s);
    case OPENMINI_QMM_Q8_0: return dispatch_kind<OPENMINI_QMM_Q8_0>(grp, w0, x, batch, count, swiglu, s);
    case OPENMINI_QMM_Q4_K: return dispatch_kind<OPENMINI_QMM_Q4_K>(grp, w0, x, batch, count, swiglu, s);
    case OPENMINI_QMM_Q6_K: return dispatch_kind<OPENMINI_QMM_Q6_K>(grp, w0, x, batch, count, swiglu, s);
    case OPENMINI_QMM_Q4_1: return dispatch_kind<OPENMINI_QMM_Q4_1>(grp, w0, x, batch, count, swiglu, s);
    case OPENMINI_QMM_Q5_K: return dispatch_kind<OPENMINI_QMM_Q5_K>(grp, w0, x, batch, count, swiglu, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const Weight& w, const float* x, float* y, int batch, hipStream_t s) {
    const Weight* ws[1] = {&w};
    float* ys[1] = {y};
    return launch_gemv_group(ws, ys, 1, x, batch, false, s);
}

}  // namespace qmm
