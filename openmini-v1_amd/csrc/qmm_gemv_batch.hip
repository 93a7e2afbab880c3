// Batched decode GEMV: y[b, n] = sum_k x[b, k] * w[n, k] for up to 16 fp32 activation
// rows in one pass over W, on fp16 MFMA with the batch rows as the MFMA rows.
//
// Replaces, per call of linear()/linear_gemm() with several rows
// (openmini-server/src/model/inference/model.rs:1050-1064), the W^T copy plus f32
// sgemm over weights dequantized at load.
//
// Arithmetic (every product exact, fp32 accumulation):
//   * Codes are exact in fp16: Q4_0 / Q4_K as q - 8, Q8_0 as q, Q6_K as q in
//     [-32, 31].  They are built from the code bytes with the 1024 + u pattern
//     (0x64XX is the fp16 1024 + XX, spacing 1) and one packed fp16 subtraction;
//     nibbles by bit-field selects in the element order (0, 2, 1, 3, 4, 6, 5, 7),
//     in which the activations are then loaded (9 VALU per 8 codes against 12 in
//     order: 8192 x 8192 b = 16 18.8-19.6 -> 17.2-18.0 us, 11008 x 4096 b = 8
//     12.0-12.2 -> 11.4 us, Q4_K b = 8 12.4-12.5 -> 11.7-12.1 us).
//   * K-quant weights (the reference's reading, quant.rs:338-410 and :515-600) use
//     their 32-element sub-blocks as the blocks, with block factor d * scale (exact).
//     Q6_K's scale changes every 16 elements, inside one MFMA's 32: q * scale (at most
//     12 significant bits) goes in as fp16 hi + lo codes, four MFMAs per block, and
//     with no per-block factor left the group's blocks chain into one D, times d.
//     Q5_K shares Q6_K's chunk layout but has one scale per 32 elements: one MFMA
//     pair per block, like Q4_K.
//   * Per (batch row, 4-block group) the activations are scaled by 2^s, s chosen so
//     the group's largest |x| lands in [2^14, 2^15), and split into hi = x' rounded
//     toward zero to fp16 (11 significant bits: x' with its low 13 mantissa bits
//     cleared) and lo = x' - hi, exact in fp32, rounded toward zero to fp16 (at most
//     13 bits: a relative error below 2^-20 of the element; elements below 2^-14 of
//     the group maximum lose bits only below 2^-38 of it).  The scale is a range
//     guard: fp16 cannot hold the full fp32 exponent range.
//   * v_mfma_f32_16x16x32_f16 covers one 32-element block: D = (hi + lo) . q in fp32
//     for 16 batch rows x 16 weight rows.  Each block's D is scaled by its fp16 scale
//     into a group sum; each group sum by 2^-s into the row's accumulator.
//   * Non-finite activations propagate through the products (inf - inf and 0 * inf
//     are NaN), so a row holding inf / NaN gets non-finite outputs in its own row only.
//
// MFMA operands (16 x 16 x 32): lane l = 16 kq + i holds A row i (batch row), k
// elements 8 kq .. 8 kq + 7 of the block; B column i (weight row), the same k.  For a
// (row tile, group) chunk that is slot (t, i) of block t, word kq (Q4_0: 8 nibbles)
// or bytes 8 kq .. 8 kq + 7 (Q8_0).  A chunk arrives as in the single-row kernel --
// lane l reads slot l whole, one 1 KB (Q4_0) / 2 KB (Q8_0) wave load plus its 128 B
// of scales -- and a 4 x 4 register transpose across the wave's four 16-lane rows
// (row swaps, no LDS) hands every lane its words of all four blocks: one wide load per
// chunk costs the address unit what one narrow load would.  Batches of at most 8 or 4
// rows leave A rows free; there 2 or 4 lanes share an activation row (kRep, below).
// D: lane l holds column l % 16, rows 4 (l / 16) .. + 3.  VALU issue (code
// conversion, scale FMAs, the activation split) is what bounds the kernel.
//
// Work split: a workgroup owns T consecutive row tiles (of kNW weights: a (gate, up)
// pair runs both on the same tiles and writes silu(gate) * up, model.rs:713-735 with
// silu at :1187-1189); its W waves split the K groups into contiguous slices and walk
// them one group at a time, with the next group's loads (activations, then the chunks)
// in flight while the current group is split (once for the T tiles) and multiplied.
// The W partial sums of an output meet in LDS and are added in wave order
// (deterministic).  A weight of few row tiles also splits K over 2 or 4 workgroups per
// tile group (batch_split): each stores its sums in the weight's workspace and counts
// itself in; the last to arrive adds the splits' sums in split order, so the result
// does not depend on which one finishes last.
#include "qmm_device.hpp"

namespace qmm {
namespace {

// x - hi for the fp16 hi in the low (kHalf = 0) or high half of h, exact in fp32: one
// mixed-precision FMA reading hi's half directly.
template <int kHalf>
__device__ __forceinline__ float minus_half(uint32_t h, float x) {
    float r;
    if constexpr (kHalf == 0)
        asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    else
        asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}

// 8 scaled activations -> fp16 hi and lo parts: hi = x' rounded toward zero to fp16
// (11 significant bits for x' >= 2^-14), lo = x' - hi, exact in fp32, rounded toward
// zero to fp16.
__device__ __forceinline__ void split8(const float* v, int s, f16x8& hi, f16x8& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = __builtin_amdgcn_ldexpf(v[2 * j], s), b = __builtin_amdgcn_ldexpf(v[2 * j + 1], s);
        h[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
        l[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(minus_half<0>(h[j], a), minus_half<1>(h[j], b)));
    }
    hi = __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(h));
    lo = __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(l));
}

// Max over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four k quarters of A row l % 16),
// with the gfx950 row-swap permutes (no LDS round trip).
__device__ __forceinline__ float quarter_max(float m) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}


// Sum over the same four lanes (every lane ends with the same value).
__device__ __forceinline__ float quarter_sum(float m) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Register transposes across the four 16-lane rows of a wave (gfx950 row swaps:
// permlane32_swap exchanges rows 2, 3 of its first operand with rows 0, 1 of its
// second; permlane16_swap rows 1, 3 of the first with rows 0, 2 of the second).
// transpose4: register j of row r becomes register r of row j.
__device__ __forceinline__ void transpose4(uint32_t& a0, uint32_t& a1, uint32_t& a2, uint32_t& a3) {
    const auto p = __builtin_amdgcn_permlane32_swap(a0, a2, false, false);
    const auto q = __builtin_amdgcn_permlane32_swap(a1, a3, false, false);
    const auto u = __builtin_amdgcn_permlane16_swap(p[0], q[0], false, false);
    const auto v = __builtin_amdgcn_permlane16_swap(p[1], q[1], false, false);
    a0 = u[0];
    a1 = u[1];
    a2 = v[0];
    a3 = v[1];
}

// broadcast4: out[t] holds row t of v in every row.
__device__ __forceinline__ void broadcast4(float v, float* out) {
    const auto h = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const auto a = __builtin_amdgcn_permlane32_swap(h[0], h[0], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(h[1], h[1], false, false);
    out[0] = __uint_as_float(a[0]);
    out[1] = __uint_as_float(b[0]);
    out[2] = __uint_as_float(a[1]);
    out[3] = __uint_as_float(b[1]);
}

// v from the lane kRot places further round its 16-lane row (DPP row_ror).
template <int kRot>
__device__ __forceinline__ float row_ror(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + kRot, 0xF, 0xF, false));
}

// 8 fp16 values from lane li + kD (mod 16) of the lane's 16-lane row.
template <int kD>
__device__ __forceinline__ f16x8 from_lane(f16x8 v) {
    // row_ror:n gives lane i the value of lane i - n
    const uint4 u = __builtin_bit_cast(uint4, v);
    constexpr int kCtl = 0x120 + (16 - kD);
    return __builtin_bit_cast(
        f16x8, uint4{(uint32_t)__builtin_amdgcn_mov_dpp((int)u.x, kCtl, 0xF, 0xF, false),
                     (uint32_t)__builtin_amdgcn_mov_dpp((int)u.y, kCtl, 0xF, 0xF, false),
                     (uint32_t)__builtin_amdgcn_mov_dpp((int)u.z, kCtl, 0xF, 0xF, false),
                     (uint32_t)__builtin_amdgcn_mov_dpp((int)u.w, kCtl, 0xF, 0xF, false)});
}

// One group's operands in registers: the lane's activations of the 4 blocks and, per
// (weight, tile) pair, chunk slot `lane` (block lane / 16, row lane % 16) -- its codes
// and scale, one wide load each -- later transposed to the MFMA lanes.
// Chunk geometry by weight format (layouts in qmm_internal.hpp).
template <int kFmt>
struct BFmt {
    static constexpr bool kQ8 = kFmt == OPENMINI_QMM_Q8_0;
    static constexpr bool kQ4K = kFmt == OPENMINI_QMM_Q4_K;
    static constexpr bool kQ41 = kFmt == OPENMINI_QMM_Q4_1;
    static constexpr bool kQ5 = kFmt == OPENMINI_QMM_Q5_K;
    static constexpr bool kQ6K = kFmt == OPENMINI_QMM_Q6_K || kQ5;  // Q6_K chunk layout
    static constexpr bool kKQ = kQ4K || kQ6K;
    static constexpr bool kMin = kQ41 || kQ5;    // block minimum
    static constexpr bool kNib = !kQ8 && !kQ6K;  // Q4_0 / Q4_1 / Q4_K: the codes are nibbles q ^ 8
    static constexpr int kCB = kQ8 ? 32 : 16;      // bytes of a slot's (low) codes
    static constexpr int kScaleOff = kQ5 ? kQ5KScaleOff : kTileEntries * (kQ6K ? 24 : kCB);
    static constexpr int kDOff = kQ5 ? kQ5KDOff : kScaleOff + (kQ6K ? 2 : 1) * kTileEntries;  // K-quant: fp16 d per row
    static constexpr int kChunk = kQ4K ? kQ4KChunk : kQ5 ? kQ5KChunk : kQ6K ? kQ6KChunk : kQ41 ? kQ41Chunk
                                                                                          : chunk_bytes_for(!kQ8);
};

template <int kFmt, int kNT, int kXB>
struct Stage {
    float x[kXB][8];
    uint4 c[kNT][BFmt<kFmt>::kQ8 ? 2 : 1];
    uint2 hb[BFmt<kFmt>::kQ6K ? kNT : 1];  // Q6_K: the slot's top code bits; Q5_K: its high-bit byte
    uint32_t sc[kNT];
    uint32_t dk[BFmt<kFmt>::kKQ ? kNT : 1];  // K-quant: the fp16 d of the slot's row
    uint32_t mn[BFmt<kFmt>::kMin ? kNT : 1];  // Q4_1: the slot's fp16 m; Q5_K: its minimum nibble
    uint32_t dm[BFmt<kFmt>::kQ5 ? kNT : 1];   // Q5_K: the fp16 dmin of the slot's row
};

// Q6_K low-nibble word kq and top-bit word kq / 2 of a slot -> 8 fp16 q, elements
// 8 kq .. 8 kq + 7 in order: bytes u = (q & 63) ^ 32 = q + 32 through the 1024 + u
// pattern, minus 1056.
__device__ __forceinline__ f16x8 codes_q6(uint32_t w, uint32_t hm, int kq) {
    const int f = (kq & 1) * 4;  // bit of field 2 (kq & 1); field + 1 for elements + 4..7
    const uint32_t lo = ((w & 0x0F0F0F0Fu) | (((hm >> f) & 0x03030303u) << 4)) ^ 0x20202020u;
    const uint32_t hi = (((w >> 4) & 0x0F0F0F0Fu) | (((hm >> (f + 2)) & 0x03030303u) << 4)) ^ 0x20202020u;
    uint32_t p[4] = {pk_sub(magic_pair(lo, kSel01), (_Float16)1056.0f), pk_sub(magic_pair(lo, kSel23), (_Float16)1056.0f),
                     pk_sub(magic_pair(hi, kSel01), (_Float16)1056.0f), pk_sub(magic_pair(hi, kSel23), (_Float16)1056.0f)};
    return __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(p));
}

// Q5_K low-nibble word kq of a slot and its high-bit byte -> 8 fp16 q - 16, elements
// 8 kq .. 8 kq + 7 (element e's high bit is bit e % 8: bits 0..3 for the low nibbles,
// 4..7 for the high ones): bytes u = q4 + 16 + 16 bit through the 1024 + u pattern,
// minus 1056.
__device__ __forceinline__ f16x8 codes_q5(uint32_t w, uint32_t qh) {
    const uint32_t lo = (w & 0x0F0F0F0Fu) | ((spread4(qh & 0xFu) << 4) + 0x10101010u);
    const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | ((spread4((qh >> 4) & 0xFu) << 4) + 0x10101010u);
    uint32_t p[4] = {pk_sub(magic_pair(lo, kSel01), (_Float16)1056.0f), pk_sub(magic_pair(lo, kSel23), (_Float16)1056.0f),
                     pk_sub(magic_pair(hi, kSel01), (_Float16)1056.0f), pk_sub(magic_pair(hi, kSel23), (_Float16)1056.0f)};
    return __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(p));
}

// Workgroup: T row tiles of kNW weights, W waves splitting K.  A wave walks its slice
// one group at a time with the next group's loads in flight (two register stages).
// kRep lanes share each activation row (batches of at most 16 / kRep rows): lane
// (kq, i) loads and splits blocks kXB p .. kXB p + kXB - 1 of batch row i % (16 / kRep),
// p = i / (16 / kRep), so the group's split costs 1 / kRep of the 16-row one; the
// other parts' hi / lo values then come from lanes i + 16 p / kRep of the same 16-lane
// row (DPP).  A rows past the batch hold other rows' values (their D rows are never
// stored), and every stored result follows the same arithmetic whatever kRep (bitwise
// identical for any batch size).
template <int kFmt, int T, int W, int kNW, int kRep>
__global__ __launch_bounds__(64 * W) void gemv_batch_kernel(const uint8_t* __restrict__ w0,
                                                            const uint8_t* __restrict__ w1,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int n_rows, int n_tiles, int groups, int k, int batch,
                                                            float* __restrict__ sums, uint32_t* __restrict__ cnt,
                                                            int splits) {
    static_assert(kRep == 1 || kRep == 2 || kRep == 4, "lanes per activation row");
    constexpr int kNT = kNW * T;  // (weight, tile) pairs of the workgroup
    constexpr int kXB = 4 / kRep;  // blocks of a group a lane loads and splits
    constexpr int kPartRows = 16 / kRep;  // A rows per part: the batch rows
    using F = BFmt<kFmt>;
    using St = Stage<kFmt, kNT, kXB>;
    constexpr int kCB = F::kCB;
    constexpr int kCodeBytes = kTileEntries * kCB;
    constexpr int kChunk = F::kChunk;
    // per wave: the 16 A rows' 2^-s of the current group while running, then the
    // partial sums [W][kNT][64 lanes][4] for the reduction
    constexpr int kRed = W * kNT * 256;
    // per wave: 16 range scales, then (block minimum) 4 blocks x 16 activation-block sums
    constexpr int kScale = W * 16 + (F::kMin ? W * 64 : 0);
    __shared__ __attribute__((aligned(16))) float lds[kRed > kScale ? kRed : kScale];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15, kq = lane >> 4;
    // workgroup = (tile group, K split): the split's contiguous K groups [gs0, gs1)
    const int split = (int)blockIdx.x % splits;
    const int tgroup = (int)blockIdx.x / splits;
    const int tile0 = tgroup * T;
    const int gs0 = (int)((int64_t)groups * split / splits);
    const int gsn = (int)((int64_t)groups * (split + 1) / splits) - gs0;
    // Eight waves walk the split's K range as two halves of four waves, each half cut
    // as a two-way split cuts K for four waves: an eight-wave workgroup then computes
    // bitwise what two four-wave splits compute (choose_batch_shape relies on it).
    constexpr int kWH = W == 8 ? 4 : W;  // waves per half
    const int hs0 = gs0 + (int)((int64_t)gsn * (wave / kWH) / (W / kWH));
    const int hsn = gs0 + (int)((int64_t)gsn * (wave / kWH + 1) / (W / kWH)) - hs0;
    const int g0 = hs0 + (int)((int64_t)hsn * (wave % kWH) / kWH);
    const int g1 = hs0 + (int)((int64_t)hsn * (wave % kWH + 1) / kWH);

    const __amdgpu_buffer_rsrc_t w_rs0 = make_rsrc(w0, (uint32_t)n_tiles * groups * kChunk);
    const __amdgpu_buffer_rsrc_t w_rs1 = make_rsrc(kNW == 2 ? w1 : w0, (uint32_t)n_tiles * groups * kChunk);
    // Tiles past the last one re-read it (cache hits) and are not stored.
    uint32_t tile_off[T];
#pragma unroll
    for (int i = 0; i < T; ++i) tile_off[i] = (uint32_t)min(tile0 + i, n_tiles - 1) * groups * kChunk;
    // x: one buffer of batch * k floats.  A row li carries batch row
    // min(li % kPartRows, batch - 1) (rows past the batch are computed and not stored);
    // the lane's blocks of a group start kXB * 32 * part elements in.  Elements past k
    // read zero: k is a multiple of 32, so a block is in range iff its first element is.
    const int part = li / kPartRows;
    const __amdgpu_buffer_rsrc_t x_rs = make_rsrc(x, (uint32_t)batch * (uint32_t)k * 4u);
    const uint32_t x_lane =
        ((uint32_t)min(li % kPartRows, batch - 1) * (uint32_t)k + (uint32_t)(part * kXB * 32 + kq * 8)) * 4u;
    const int x_lim = k - part * kXB * 32;  // slot element offset g * 128 + 32 tt must be below
    float* my_scale = lds + wave * 16;
    float* my_sums = lds + W * 16 + wave * 64;  // [block][batch row]; block-minimum formats

    f32x4 acc[kNT];
#pragma unroll
    for (int i = 0; i < kNT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Issue group g's loads: activations first (L2 hits), then the chunks.
    auto load = [&](St& st, int g) {
#pragma unroll
        for (int tt = 0; tt < kXB; ++tt) {
            const int ge = g * 128 + tt * 32;
            const uint32_t off = x_lane + (ge < x_lim ? (uint32_t)ge * 4u : 0x80000000u);
            const float4 a = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(x_rs, off, 0, 0));
            const float4 b = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(x_rs, off + 16u, 0, 0));
            if constexpr (F::kNib) {  // codes_q4_perm's element order
                st.x[tt][0] = a.x; st.x[tt][1] = a.z; st.x[tt][2] = a.y; st.x[tt][3] = a.w;
                st.x[tt][4] = b.x; st.x[tt][5] = b.z; st.x[tt][6] = b.y; st.x[tt][7] = b.w;
            } else {
                st.x[tt][0] = a.x; st.x[tt][1] = a.y; st.x[tt][2] = a.z; st.x[tt][3] = a.w;
                st.x[tt][4] = b.x; st.x[tt][5] = b.y; st.x[tt][6] = b.z; st.x[tt][7] = b.w;
            }
        }
#pragma unroll
        for (int i = 0; i < kNT; ++i) {
            const __amdgpu_buffer_rsrc_t rs = i / T == 0 ? w_rs0 : w_rs1;
            const uint32_t soff = tile_off[i % T] + (uint32_t)g * kChunk;
            st.c[i][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * kCB, soff, 0));
            if constexpr (F::kQ8)
                st.c[i][1] =
                    __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * kCB + 16, soff, 0));
            if constexpr (F::kQ5)
                st.hb[i].x = __builtin_amdgcn_raw_buffer_load_b8(rs, kQ5KQhOff + lane, soff, 0);
            else if constexpr (F::kQ6K)
                st.hb[i] = __builtin_bit_cast(
                    uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, kCodeBytes + lane * 8, soff, 0));
            if constexpr (F::kQ4K || F::kQ5)
                st.sc[i] = __builtin_amdgcn_raw_buffer_load_b8(rs, F::kScaleOff + lane, soff, 0);
            else
                st.sc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, F::kScaleOff + lane * 2, soff, 0);
            if constexpr (F::kKQ)  // the d of slot lane's row, lane % 16
                st.dk[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, F::kDOff + li * 2, soff, 0);
            if constexpr (F::kQ41) st.mn[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, kQ41MinOff + lane * 2, soff, 0);
            if constexpr (F::kQ5) {
                st.mn[i] = __builtin_amdgcn_raw_buffer_load_b8(rs, kQ5KMinOff + lane, soff, 0);
                st.dm[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, kQ5KDminOff + li * 2, soff, 0);
            }
        }
    };

    // One group: the range scale and hi / lo split of the activations (shared by the
    // kNT pairs), then per pair 4 blocks of 2 MFMAs and the scale FMAs.
    auto compute = [&](const St& st) {
        float m = 0.0f;
#pragma unroll
        for (int tt = 0; tt < kXB; ++tt)
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(st.x[tt][j]));
        m = quarter_max(m);
        if constexpr (kRep >= 2) m = fmaxf(m, row_ror<8>(m));  // the parts of a row: lanes li, li ^ 8
        if constexpr (kRep == 4) m = fmaxf(m, row_ror<4>(m));  // and li + 4, li + 12
        // 2^e <= m < 2^(e+1), e = biased exponent - 127; s = 14 - e
        const int sh = 141 - (int)(__float_as_uint(m) >> 23);
        if (kq == 0) my_scale[li] = __builtin_amdgcn_ldexpf(1.0f, -sh);
        if constexpr (F::kMin) {
            // the sums of the lane's activation blocks (the lane's 8 elements, then the
            // four k quarters), one lane per (batch row, block) writing
#pragma unroll
            for (int tt = 0; tt < kXB; ++tt) {
                float v = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) v += st.x[tt][j];
                v = quarter_sum(v);
                if (kq == 0) my_sums[((li / kPartRows) * kXB + tt) * 16 + li % kPartRows] = v;
            }
        }
        f16x8 ah[4], al[4];  // A operands of blocks 0..3 for the batch rows' lanes
#pragma unroll
        for (int tt = 0; tt < kXB; ++tt) split8(st.x[tt], sh, ah[tt], al[tt]);
#pragma unroll
        for (int t = kXB; t < 4; ++t) {  // part t / kXB: lanes li + kPartRows * (t / kXB)
            if (t / kXB == 1) {
                ah[t] = from_lane<kPartRows>(ah[t % kXB]);
                al[t] = from_lane<kPartRows>(al[t % kXB]);
            } else if (t / kXB == 2) {
                ah[t] = from_lane<2 * kPartRows>(ah[t % kXB]);
                al[t] = from_lane<2 * kPartRows>(al[t % kXB]);
            } else {
                ah[t] = from_lane<3 * kPartRows>(ah[t % kXB]);
                al[t] = from_lane<3 * kPartRows>(al[t % kXB]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // 2^-s of the four A rows this lane's D values belong to (rows 4 kq .. 4 kq + 3)
        const f32x4 rs = *reinterpret_cast<const f32x4*>(my_scale + kq * 4);
        // block minimum: the activation-block sums of those rows' batch rows, 4 kq + r
        // modulo the rows per part (A rows repeat the batch rows)
        f32x4 bs[4];
        if constexpr (F::kMin) {
#pragma unroll
            for (int t = 0; t < 4; ++t) bs[t] = *reinterpret_cast<const f32x4*>(my_sums + t * 16 + (kq * 4) % kPartRows);
        }
#pragma unroll
        for (int i = 0; i < kNT; ++i) {
            // lane (kq, i) takes word kq (Q4_0) / words 2 kq, 2 kq + 1 (Q8_0) of slot
            // (t, i) for t = 0..3, and the scales of its column
            uint32_t e[4], o[4];
            if constexpr (!F::kQ8) {
                e[0] = st.c[i][0].x; e[1] = st.c[i][0].y; e[2] = st.c[i][0].z; e[3] = st.c[i][0].w;
                transpose4(e[0], e[1], e[2], e[3]);
                if constexpr (F::kQ5) {
                    // lane (kq, i) takes the high-bit byte of slot (t, i)
                    float hb4[4];
                    broadcast4(__uint_as_float(st.hb[i].x), hb4);
#pragma unroll
                    for (int t = 0; t < 4; ++t) o[t] = __float_as_uint(hb4[t]);
                } else if constexpr (F::kQ6K) {
                    // lane (kq, i) takes top-bit word kq / 2 of slot (t, i): the loader
                    // lane's registers are words 0, 0, 1, 1 before the transpose
                    o[0] = st.hb[i].x; o[1] = st.hb[i].x; o[2] = st.hb[i].y; o[3] = st.hb[i].y;
                    transpose4(o[0], o[1], o[2], o[3]);
                }
            } else {
                e[0] = st.c[i][0].x; o[0] = st.c[i][0].y; e[1] = st.c[i][0].z; o[1] = st.c[i][0].w;
                e[2] = st.c[i][1].x; o[2] = st.c[i][1].y; e[3] = st.c[i][1].z; o[3] = st.c[i][1].w;
                transpose4(e[0], e[1], e[2], e[3]);
                transpose4(o[0], o[1], o[2], o[3]);
            }
            if constexpr (F::kQ6K && !F::kQ5) {
                // Q6_K: the scale changes every 16 elements, inside an MFMA's 32, so it
                // goes into the codes: q * scale, an integer of at most 12 significant
                // bits, as fp16 hi = the rounded product and lo = the exact remainder
                // (an fp16 FMA).  With exact operands the group's 4 blocks chain into
                // one D per tile (hi and lo activations times hi and lo codes), and d
                // (one per row and super-block) applies once, with the range scale.
                // lane (kq, i) takes the scale of half kq / 2 of slot (t, i)
                float sw[4];
                broadcast4(__uint_as_float(st.sc[i]), sw);
                f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const f16x8 b = codes_q6(e[t], o[t], kq);
                    const _Float16 sc = (_Float16)(float)(int8_t)((__float_as_uint(sw[t]) >> ((kq >> 1) * 8)) & 0xFFu);
                    const f16x8 s8 = f16x8{sc, sc, sc, sc, sc, sc, sc, sc};
                    const f16x8 bh = b * s8;
                    const f16x8 bl = __builtin_elementwise_fma(b, s8, -bh);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[t], bh, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t], bh, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[t], bl, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t], bl, d, 0, 0, 0);
                }
                const float dd = f16_bits_to_f32((uint16_t)st.dk[i]);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][r] = fmaf(d[r], rs[r] * dd, acc[i][r]);
                continue;
            }
            // the block factors of column i (slot (t, i) for t = 0..3), exact in fp32:
            // the fp16 scale; Q4_K d * scale; Q5_K d * scale (one per 32-element
            // sub-block: its two scale bytes are equal)
            float ds[4];
            if constexpr (F::kQ4K) {
                broadcast4(f16_bits_to_f32((uint16_t)st.dk[i]) * (float)(st.sc[i] & 0xFFu), ds);
            } else if constexpr (F::kQ6K) {
                broadcast4(f16_bits_to_f32((uint16_t)st.dk[i]) * (float)(int8_t)(st.sc[i] & 0xFFu), ds);
            } else {
                broadcast4(f16_bits_to_f32((uint16_t)st.sc[i]), ds);
            }
            // block minimum offsets of column i's slots: Q4_1 (q - 8) d + (8 d + m),
            // Q5_K dmin * minimum
            float os[4];
            if constexpr (F::kQ41)
                broadcast4(fmaf(8.0f, f16_bits_to_f32((uint16_t)st.sc[i]), f16_bits_to_f32((uint16_t)st.mn[i])), os);
            if constexpr (F::kQ5) broadcast4(f16_bits_to_f32((uint16_t)st.dm[i]) * (float)st.mn[i], os);
            f32x4 gs = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                f16x8 b;
                if constexpr (F::kNib)
                    b = codes_q4_perm(e[t]);  // the activations were loaded in its order
                else if constexpr (F::kQ6K)
                    b = F::kQ5 ? codes_q5(e[t], o[t]) : codes_q6(e[t], o[t], kq);
                else
                    b = codes_q8(e[t], o[t]);
                f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[t], b, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t], b, d, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) gs[r] = fmaf(d[r], ds[t], gs[r]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][r] = fmaf(gs[r], rs[r], acc[i][r]);
            if constexpr (F::kMin) {
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][r] = fmaf(os[t], bs[t][r], acc[i][r]);
            }
        }
        // the next group rewrites my_scale after these reads (in-order LDS per wave)
    };

    if (g0 < g1) {  // uniform per wave
        St sa, sb;
        load(sa, g0);
        // The loads past the slice end re-read its last group (cache hits) and are
        // never consumed, so every path issues the same loads.  One exit, at the loop
        // test: with a break between the two halves the compiler's wait insertion
        // merged the paths conservatively and waited at the loop head for the
        // prefetched stage to land before issuing the next one.
        for (int g = g0; g < g1; g += 2) {
            load(sb, min(g + 1, g1 - 1));
            compute(sa);
            load(sa, min(g + 2, g1 - 1));
            if (g + 1 < g1) compute(sb);
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // the unconsumed prefetch has landed
    }

    // The W K slices meet in LDS and are added in wave order (eight waves: each half
    // in wave order, then the two halves, as the K split adds its splits).
    __syncthreads();  // every wave is done with its scale slots
#pragma unroll
    for (int i = 0; i < kNT; ++i)
        *reinterpret_cast<f32x4*>(lds + ((wave * kNT + i) * 64 + lane) * 4) = acc[i];
    __syncthreads();
    // output (tile i, batch row b): lane (b / 4) * 16 + r, register b % 4
    const size_t n_pad = (size_t)n_tiles * kTileRows;
    for (int f = (int)threadIdx.x; f < T * 256; f += 64 * W) {
        const int i = f >> 8, b = (f >> 4) & 15, r = f & 15;
        const int row = (tile0 + i) * kTileRows + r;
        if (b >= batch || tile0 + i >= n_tiles || row >= n_rows) continue;
        const int src = ((b >> 2) * 16 + r) * 4 + (b & 3);
        float v[kNW];
#pragma unroll
        for (int nw = 0; nw < kNW; ++nw) {
            v[nw] = lds[(nw * T + i) * 256 + src];
#pragma unroll
            for (int w = 1; w < kWH; ++w) v[nw] += lds[((w * kNT) + nw * T + i) * 256 + src];
            if constexpr (W == 8) {
                float h = lds[((4 * kNT) + nw * T + i) * 256 + src];
#pragma unroll
                for (int w = 5; w < 8; ++w) h += lds[((w * kNT) + nw * T + i) * 256 + src];
                v[nw] += h;
            }
        }
        if constexpr (kNW == 2)
            y[(size_t)b * n_rows + row] = v[0] / (1.0f + expf(-v[0])) * v[1];
        else if (splits == 1)
            y[(size_t)b * n_rows + row] = v[0];
        else  // device-coherent store (write-through past this XCD's L2)
            __hip_atomic_store(sums + ((size_t)split * kBatchRows + b) * n_pad + row, v[0], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (kNW == 1) {
        if (splits == 1) return;
        // K split: the last of the tile group's workgroups to finish adds the splits'
        // sums in split order (the same bits whichever finishes last).  No workgroup
        // waits for another.  The group's counter only grows: every call adds exactly
        // `splits` (2 or 4, a divisor of 2^32, so wrap-around keeps the residue), and
        // the workgroup whose increment leaves a multiple of `splits` is the last of
        // its call.  Calls that overlap on one weight (which the interface forbids)
        // could each pick a wrong last workgroup, but leave the count a multiple of
        // `splits`, so later calls are unaffected.
        // Ordering, on gfx950's rules rather than language-level release / acquire:
        //  * the sums are agent-scope atomic stores, which gfx950 issues write-through
        //    past the XCD's L2 (the sc1 bit), and the last workgroup reads them with
        //    agent-scope atomic loads, which miss in its own L2: no L2 write-back or
        //    invalidate is needed for them to meet across XCDs;
        //  * on gfx9 parts vmcnt counts stores as well as loads, so each wave's
        //    s_waitcnt vmcnt(0) returns only once its sum stores are acknowledged, and
        //    the barrier after it makes every wave of the workgroup wait for that
        //    before thread 0 counts the workgroup in;
        //  * the last workgroup issues its loads only after thread 0's count returned
        //    (the barrier orders them after it), in program order.
        // A release count and an acquire fence (an L2 write-back and an L2 invalidate
        // on this part) give the same result and cost 4-5 us per call: 4096 x 4096
        // b = 16 9.5 -> 14.8 us, 4096 x 11008 b = 8 13.7-14.4 -> 19.2-19.5 us (one box).
        // qmm_internal.hpp refuses to build device code for any other target.
        __shared__ uint32_t last;
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
        __syncthreads();
        if (threadIdx.x == 0)
            last = (__hip_atomic_fetch_add(cnt + tgroup, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                    (uint32_t)(splits - 1)) == (uint32_t)(splits - 1);
        __syncthreads();
        if (!last) return;
        for (int f = (int)threadIdx.x; f < T * 256; f += 64 * W) {
            const int i = f >> 8, b = (f >> 4) & 15, r = f & 15;
            const int row = (tile0 + i) * kTileRows + r;
            if (b >= batch || tile0 + i >= n_tiles || row >= n_rows) continue;
            const float* p = sums + (size_t)b * n_pad + row;
            float v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int q = 1; q < splits; ++q)
                v += __hip_atomic_load(p + (size_t)q * kBatchRows * n_pad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            y[(size_t)b * n_rows + row] = v;
        }
    }
}

template <int kFmt, int T, int W, int kNW, int kRep>
hipError_t run(const Weight& w, const uint8_t* w1, const float* x, float* y, int batch, int splits,
               hipStream_t s) {
    const unsigned wgs = (unsigned)((w.n_tiles + T - 1) / T * splits);
    hipLaunchKernelGGL((gemv_batch_kernel<kFmt, T, W, kNW, kRep>), dim3(wgs), dim3(64 * W), 0, s, w.chunks, w1, x,
                       y, (int)w.n, (int)w.n_tiles, (int)w.groups, (int)w.k, batch, w.split_part, w.split_cnt,
                       splits);
    return hipGetLastError();
}

}  // namespace

bool use_batch_kernel(const Weight& w, int64_t batch) {
    return batch >= kBatchMin && (int64_t)kBatchRows * w.k * 4 <= INT32_MAX;
}

hipError_t launch_gemv_rows(const Weight& w, const Weight* up, const float* x, float* y, int64_t batch,
                            hipStream_t s) {
    if (use_batch_kernel(w, batch)) {
        for (int64_t b0 = 0; b0 < batch; b0 += kBatchRows) {
            const int nb = (int)(batch - b0 < kBatchRows ? batch - b0 : kBatchRows);
            const hipError_t e =
                launch_gemv_batch(w, up, x + b0 * w.k, y + b0 * w.n, nb, choose_batch_shape(w, nb, up), s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    for (int64_t b0 = 0; b0 < batch; b0 += kMaxGemvBatch) {
        const int nb = (int)(batch - b0 < kMaxGemvBatch ? batch - b0 : kMaxGemvBatch);
        const Weight* ws[2] = {&w, up};
        float* ys[2] = {y + b0 * w.n, y + b0 * w.n};
        const hipError_t e = launch_gemv_group(ws, ys, up ? 2 : 1, x + b0 * w.k, nb, up != nullptr, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Launch shape, measured on MI355X (Q4_0 / Q8_0 / Q4_K, B = 8, 16, N = 4096 ... 28672):
// four waves per workgroup (one when K has fewer than 8 groups), eight (two per SIMD)
// for one weight when a workgroup walks at least 64 K groups (three interleaved A/B
// passes: Q4_0 28672 x 8192 B = 4 40.1-40.6 -> 38.6-39.0 us, B = 16 43.8-44.5 ->
// 41.8-43.0, 8192 x 28672 (2 K splits) B = 4 42.3-43.0 -> 39.2-41.1, B = 16 even;
// with 32-43 groups per workgroup eight waves lost up to 10%); tiles per workgroup
// so that the grid is one workgroup per CU, all CUs busy: T = ceil(tiles / 256), at
// most 8 (Q4_0 / Q4_K) or 4 (Q8_0 / Q6_K, whose 8-tile registers would leave one
// wave per SIMD).  More tiles share each wave's activation loads and split; more
// workgroups than CUs add activation re-reads.  Against powers of two (1, 2, 4, 8):
// 11008 x 4096 (688 tiles) T = 3 vs 4: Q8_0 B = 8 13.7-15.1 vs 15.8-16.8 us, Q4_0
// B = 16 13.1 vs 15.2 us, Q4_K B = 8 13.0 vs 14.8 us; 28672 x 8192 (1792 tiles) T = 7
// vs 8: 45.4 vs 47.8 us.  A (gate, up) pair takes at most 4 (Q4_0 / Q4_K) or 3 tiles:
// against one tile per workgroup, 11008 x 4096 Q4_0 B = 8 25.5 -> 20.8 us, Q8_0 B = 8
// 30.7 -> 25.2 us, Q4_K B = 16 31.9 -> 22.5 us, 28672 x 8192 Q4_0 B = 16 118 -> 80 us.
constexpr int64_t kCUs = 256;  // MI355X compute units

static int64_t tiles_per_cu(int type, int64_t n_tiles, bool pair) {
    // a pair holds two weights' registers per tile: at most 4 / 3 tiles
    const bool nib = type == OPENMINI_QMM_Q4_0 || type == OPENMINI_QMM_Q4_K || type == OPENMINI_QMM_Q4_1;
    const int64_t cap = pair ? (nib ? 4 : 3) : nib ? 8 : 4;
    const int64_t per_cu = (n_tiles + kCUs - 1) / kCUs;
    return per_cu < 1 ? 1 : per_cu > cap ? cap : per_cu;
}

// K split, measured on MI355X (three interleaved A/B passes on one box): at most 512
// row tiles leave each workgroup 1 or 2 tiles to share its waves' activation split.
// Two workgroups per tile group of twice the tiles, each over half of K, halve that
// share: Q4_0 8192 x 28672 B = 16 60.8 -> 47.9 us, B = 4 45.6 -> 42.8; 8192 x 8192
// B = 16 21.1 -> 18.7-20.0, B = 4 16.4 -> 16.3-17.0; 4096 x 11008 Q8_0 B = 8 18.3 ->
// 16.0-16.9, Q4_0 B = 8 16.1 -> 14.3-14.9; 4096 x 4096 B = 16 10.5 -> 9.9.  Three or
// four splits, or a split at 688 tiles (T = 6), were slower (258 workgroups for 256
// CUs; 3-4 groups per wave).  At most 128 tiles fill at most half the CUs with one
// tile per workgroup; there the K split alone fills them: 1024 x 8192 (64 tiles, 4
// splits) Q4_0 B = 16 17.1 -> 10.0 us, B = 4 10.0 -> 7.8 us, Q8_0 B = 8 11.6 -> 8.4 us
// (2 splits of 2 tiles: 12.9 us, 4 splits of 2 tiles 10.4 us at B = 16).  The choice
// depends on the shape only, so results stay bitwise independent of the batch size
// (choose_batch_shape's eight-wave form of a split at 4 rows computes the same bits).
void batch_split(int type, int64_t n_tiles, int64_t groups, int* t, int* s) {
    const int64_t t0 = tiles_per_cu(type, n_tiles, false);
    const bool nib = type == OPENMINI_QMM_Q4_0 || type == OPENMINI_QMM_Q4_K || type == OPENMINI_QMM_Q4_1;
    *t = (int)t0;
    *s = 1;
    if (groups < 32) return;  // at least 16 groups per split
    if (n_tiles <= kCUs / 4 && groups >= 64) {
        *t = 1;
        *s = 4;
    } else if (n_tiles <= kCUs / 2) {
        *t = 1;
        *s = 2;
    } else if (n_tiles <= 2 * kCUs && 2 * t0 <= (nib ? 8 : 4)) {
        *t = (int)(2 * t0);
        *s = 2;
    }
}

size_t split_workspace_bytes(int64_t n_tiles, int t, int s) {
    if (s <= 1) return 0;
    const size_t part = (size_t)s * kBatchRows * (size_t)n_tiles * kTileRows * 4;
    const size_t cnt = (size_t)((n_tiles + t - 1) / t) * 4;
    return part + (cnt + 255) / 256 * 256;
}

BatchShape choose_batch_shape(const Weight& w, int batch, bool pair) {
    BatchShape sh{};
    if (pair) {
        sh.t = (int)tiles_per_cu(w.type, w.n_tiles, true);
    } else {
        sh.t = w.split_t;
        sh.split = w.split_s;
    }
    // At most 4 rows, a two-way split of 64-127 K groups over tile groups of 2+ tiles
    // runs as one workgroup of eight waves on half the tiles instead: the same K cut
    // and addition order (gemv_batch_kernel), so the bits equal the split's, and no
    // hand-off.  Interleaved A/B passes on two boxes (us, split -> eight waves):
    // Q4_0 8192 x 8192 b = 4 16.0-17.1 -> 13.7-14.5, Q4_K 16.2-16.8 -> 14.3-14.7,
    // 4096 x 8192 10.3-10.6 -> 9.3-9.5, 4096 x 11008 Q8_0 15.0-15.5 -> 14.0-14.5, Q6_K
    // 18.1-20.2 -> 16.8-17.8, Q4_0 even; at 8 rows 4096 x 11008 lost 10-20% and 8192 x
    // 8192 was even, at 16 rows both lost.
    if (!pair && batch <= 4 && sh.split == 2 && sh.t >= 2 && w.groups >= 64 && w.groups < 128) {
        sh.split = 1;
        sh.t /= 2;
    }
    sh.w = w.groups >= 8 ? 4 : 1;
    // at least 64 K groups per workgroup: eight waves of 8+ groups each (two per SIMD)
    if (!pair && w.groups / sh.split >= 64) sh.w = 8;
    sh.rep = batch <= 4 ? 4 : batch <= 8 ? 2 : 1;
    return sh;
}

template <int kFmt, int kNW, int kRep>
static hipError_t dispatch_batch(const Weight& w, const uint8_t* w1, const float* x, float* y, int batch,
                                 const BatchShape& sh, hipStream_t s) {
#define QMM_BATCH_CASE(T_)                                                                          \
    if (sh.t == T_) {                                                                               \
        if constexpr (kNW == 1)                                                                     \
            if (sh.w == 8) return run<kFmt, T_, 8, kNW, kRep>(w, w1, x, y, batch, sh.split, s);      \
        return sh.w == 4 ? run<kFmt, T_, 4, kNW, kRep>(w, w1, x, y, batch, sh.split, s)             \
                         : run<kFmt, T_, 1, kNW, kRep>(w, w1, x, y, batch, sh.split, s);            \
    }
    if (sh.w != 1 && sh.w != 4 && !(kNW == 1 && sh.w == 8)) return hipErrorInvalidValue;
    QMM_BATCH_CASE(1)
    QMM_BATCH_CASE(2)
    if constexpr (kNW == 2) {
        QMM_BATCH_CASE(3)
        if constexpr (BFmt<kFmt>::kNib) {
            QMM_BATCH_CASE(4)
        }
    }
    if constexpr (kNW == 1) {
        QMM_BATCH_CASE(3)
        QMM_BATCH_CASE(4)
        if constexpr (BFmt<kFmt>::kNib) {
            QMM_BATCH_CASE(5)
            QMM_BATCH_CASE(6)
            QMM_BATCH_CASE(7)
            QMM_BATCH_CASE(8)
        }
    }
#undef QMM_BATCH_CASE
    return hipErrorInvalidValue;
}

template <int kFmt, int kNW>
static hipError_t dispatch_rep(const Weight& w, const uint8_t* w1, const float* x, float* y, int batch,
                               const BatchShape& sh, hipStream_t s) {
    if (batch * sh.rep > kBatchRows) return hipErrorInvalidValue;  // 16 / rep batch rows per part
    switch (sh.rep) {
    case 1: return dispatch_batch<kFmt, kNW, 1>(w, w1, x, y, batch, sh, s);
    case 2: return dispatch_batch<kFmt, kNW, 2>(w, w1, x, y, batch, sh, s);
    case 4: return dispatch_batch<kFmt, kNW, 4>(w, w1, x, y, batch, sh, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_batch(const Weight& w, const Weight* up, const float* x, float* y, int batch,
                             const BatchShape& sh, hipStream_t s) {
    if (batch < 1 || batch > kBatchRows) return hipErrorInvalidValue;
    if ((int64_t)batch * w.k * 4 > INT32_MAX) return hipErrorInvalidValue;  // 31-bit x offsets
    // a K split runs on one weight, with the workspace sized for its tile groups
    if (sh.split < 1 || (sh.split != 1 && (up || sh.split != w.split_s || sh.t != w.split_t || !w.split_part)))
        return hipErrorInvalidValue;
    const uint8_t* w1 = up ? up->chunks : nullptr;
    switch (w.type) {
    case OPENMINI_QMM_Q4_0:
        return up ? dispatch_rep<OPENMINI_QMM_Q4_0, 2>(w, w1, x, y, batch, sh, s)
                  : dispatch_rep<OPENMINI_QMM_Q4_0, 1>(w, w1, x, y, batch, sh, s);
    case OPENMINI_QMM_Q8_0:
        return up ? dispatch_rep<OPENMINI_QMM_Q8_0, 2>(w, w1, x, y, batch, sh, s)
                  : dispatch_rep<OPENMINI_QMM_Q8_0, 1>(w, w1, x, y, batch, sh, s);
    case OPENMINI_QMM_Q4_K:
        return up ? dispatch_rep<OPENMINI_QMM_Q4_K, 2>(w, w1, x, y, batch, sh, s)
                  : dispatch_rep<OPENMINI_QMM_Q4_K, 1>(w, w1, x, y, batch, sh, s);
    case OPENMINI_QMM_Q6_K:
        return up ? dispatch_rep<OPENMINI_QMM_Q6_K, 2>(w, w1, x, y, batch, sh, s)
                  : dispatch_rep<OPENMINI_QMM_Q6_K, 1>(w, w1, x, y, batch, sh, s);
    case OPENMINI_QMM_Q4_1:
        return up ? dispatch_rep<OPENMINI_QMM_Q4_1, 2>(w, w1, x, y, batch, sh, s)
                  : dispatch_rep<OPENMINI_QMM_Q4_1, 1>(w, w1, x, y, batch, sh, s);
    case OPENMINI_QMM_Q5_K:
        return up ? dispatch_rep<OPENMINI_QMM_Q5_K, 2>(w, w1, x, y, batch, sh, s)
                  : dispatch_rep<OPENMINI_QMM_Q5_K, 1>(w, w1, x, y, batch, sh, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
