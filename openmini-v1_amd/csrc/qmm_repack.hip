// Upload/repack, dequantization and the streaming-copy yardstick.
//
// Reference semantics (paths relative to openmini-server/):
//   quant::dequantize_q4_0  src/model/inference/quant.rs:152-195
//   quant::dequantize_q8_0  src/model/inference/quant.rs:282-316
//   quant::dequantize_{q4_1, q2_k, q3_k, q4_k, q5_k, q6_k, q8_k}, f32 / f16 arms:
//                           quant.rs:95-133, 216-262, 338-800
//   f16 scale decode        quant.rs:166-167, 296-297 (half::f16::to_f32, exact)
// Q4_0 GGUF byte j of a block holds element 2j in its HIGH nibble and element
// 2j+1 in its LOW nibble (quant.rs:179-188); value = (q - 8) * f32(d).
#include "qmm_device.hpp"

namespace qmm {
namespace {

constexpr int kRepackChunks = 4;  // consecutive chunks (of one row tile) per repack workgroup
constexpr int kRepackThreads = kRepackChunks * kTileEntries;  // one thread per chunk slot

__device__ __forceinline__ uint32_t q4_code(const uint8_t* qs, int e) {
    uint8_t b = qs[e >> 1];
    return (e & 1) ? (b & 0x0Fu) : (b >> 4);
}

// Q4_0 / Q8_0 blocks -> chunks.  A workgroup writes kRepackQuads x kRepackChunks
// consecutive chunks of one row tile, whole: thread t fills slot e = t % 64 of chunk
// t / 64 of each of its quads -- block 4 g + e / 16 of row 16 rt + e % 16 -- so each
// chunk's codes and scales leave as contiguous wave stores.  Slots outside the weight
// (rows past n, blocks past nb: the tile padding) are written as zeros, so every byte of
// the chunk array is written exactly once and no clearing pass is needed.
// When the workgroup's 16 rows are all present and start 16-byte aligned (nb % 8 == 0,
// aligned source), their 16 kQuads blocks are copied to LDS by buffer loads with an LDS
// destination, all issued before the first wait: one memory round trip per workgroup.
// (Pieces past a row's last block hold the next row's bytes, or zeros past the source,
// and are never used.)  Each slot then reads its block as 32-bit words and moves nibbles
// with byte permutes.  Otherwise (the last row tile of a weight whose rows are not a
// multiple of 16, or an unaligned source) each thread reads its own blocks with byte
// loads.  Measured on MI355X, whole upload_device_into calls back to back, 11008 x 4096
// Q4_0: copies through registers (a wait per copy) and a byte loop per slot 15.2 us,
// with word reads 13.5 us, LDS-destination copies 10.2 (one quad per workgroup), 10.1
// (two; Q8_0 19.4-19.6 us) and 14.0 us (four: too few workgroups in flight).
// Q4_1 (20-byte blocks: d, m, then the Q4_0 nibble order) takes the same path with its
// codes stored as Q4_0's and m in the chunk's trailing fp16 array.
template <int kBPB, int kQuads>
__global__ __launch_bounds__(kRepackThreads) void repack_kernel(const uint8_t* __restrict__ gguf, int64_t n,
                                                                int64_t nb, int64_t groups, int64_t wg_per_tile,
                                                                int aligned16, uint8_t* __restrict__ chunks) {
    constexpr bool kQ4 = kBPB != 34;                  // nibble codes: Q4_0, Q4_1
    constexpr bool kMin = kBPB == 20;                 // Q4_1: fp16 m after d
    constexpr int kCB = kQ4 ? 16 : 32;
    constexpr int kCodeOff = kBPB - kCB;              // codes end the block
    constexpr int kChunk = kMin ? kQ41Chunk : chunk_bytes_for(kQ4);
    constexpr int kBlocks = kQuads * kRepackChunks * kTileBlocks;  // blocks of one row in the workgroup
    constexpr int kRowB = kBlocks * kBPB;
    constexpr int kSegs = kRowB / 16;                // 16-byte pieces of one row
    constexpr int kPieces = kTileRows * kSegs;
    constexpr int kPiecesPad = (kPieces + 63) / 64 * 64;  // whole waves of copies
    static_assert(kRowB % 16 == 0, "rows of whole 16-byte pieces");
    // one spare piece: a slot's word reads run up to 2 bytes past its block
    __shared__ uint4 tile[kPiecesPad + 1];
    uint8_t* t8 = reinterpret_cast<uint8_t*>(tile);

    const int64_t rt = (int64_t)blockIdx.x / wg_per_tile, wq = (int64_t)blockIdx.x % wg_per_tile;
    const int64_t row0 = rt * kTileRows, blk0 = wq * kBlocks;
    const bool staged = aligned16 && row0 + kTileRows <= n;
    const int t = threadIdx.x;
    if (staged) {  // uniform per workgroup
        // 32-bit offsets: the source is smaller than the chunk array (< 4 GiB)
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(gguf, (uint32_t)(n * nb * kBPB));
        const int wave = t >> 6, lane = t & 63;
#pragma unroll
        for (int p0 = wave * 64; p0 < kPieces; p0 += kRepackThreads) {  // p0 uniform per wave
            const int p = p0 + lane, r = p / kSegs, j = p % kSegs;
            // pieces past the last one (the padding of a wave) read zeros
            const uint32_t off =
                p < kPieces ? (uint32_t)(((row0 + r) * nb + blk0) * kBPB) + (uint32_t)j * 16u : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(t8 + p0 * 16), 16,
                                                     off, 0, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // this thread's copies have landed
        __syncthreads();
    }
    const int c = t / kTileEntries, e = t % kTileEntries;
    const int64_t row = row0 + (e & 15);
#pragma unroll
    for (int qq = 0; qq < kQuads; ++qq) {
        const int64_t grp = (wq * kQuads + qq) * kRepackChunks + c;
        if (grp >= groups) break;
        const int64_t blk = grp * kTileBlocks + (e >> 4);
        uint8_t* chunk = chunks + (rt * groups + grp) * kChunk;
        uint16_t scale = 0, minv = 0;
        uint32_t w[kCB / 4];
#pragma unroll
        for (int j = 0; j < kCB / 4; ++j) w[j] = 0;
        if (staged && blk < nb) {  // row < n holds for every slot of a staged workgroup
            // The block starts 2-byte aligned (kBPB is even): the scale as one 16-bit
            // read, the codes as 32-bit reads from the word boundary below them, realigned.
            const int src = (e & 15) * kRowB + (int)(blk - blk0) * kBPB;
            scale = *reinterpret_cast<const uint16_t*>(t8 + src);
            if constexpr (kMin) minv = *reinterpret_cast<const uint16_t*>(t8 + src + 2);
            const int a = src + kCodeOff, sh = a & 3;  // codes start; sh is 0 or 2
            const uint32_t* a32 = reinterpret_cast<const uint32_t*>(t8 + (a - sh));
            uint32_t v[kCB / 4 + 1];
#pragma unroll
            for (int j = 0; j <= kCB / 4; ++j) v[j] = a32[j];
            uint32_t q[kCB / 4];  // code bytes 4 j .. 4 j + 3
#pragma unroll
            for (int j = 0; j < kCB / 4; ++j) q[j] = __builtin_amdgcn_alignbyte(v[j + 1], v[j], (uint32_t)sh);
            if constexpr (kQ4) {
                // code word j holds elements 8 j .. 8 j + 7: GGUF bytes s0..s3 = code bytes
                // 4 j .. 4 j + 3 (element 2 m in the high nibble of s_m, 2 m + 1 in the
                // low); chunk byte i = element 8 j + i | element 8 j + 4 + i << 4, i.e.
                // bytes (s0.hi | s2.hi << 4, s0.lo | s2.lo << 4, s1.hi | s3.hi << 4,
                // s1.lo | s3.lo << 4)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t pp = __builtin_amdgcn_perm(0u, q[j], 0x01010000u);  // s0 s0 s1 s1
                    const uint32_t rr = __builtin_amdgcn_perm(0u, q[j], 0x03030202u);  // s2 s2 s3 s3
                    const uint32_t lo = ((pp >> 4) & 0x000F000Fu) | (pp & 0x0F000F00u);
                    const uint32_t hi = (rr & 0x00F000F0u) | ((rr << 4) & 0xF000F000u);
                    w[j] = (lo | hi) ^ 0x88888888u;  // nibble q ^ 8: the two's-complement value q - 8
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) w[j] = q[j];
            }
        } else if (row < n && blk < nb) {
            uint8_t b[kBPB];
            const uint8_t* src = gguf + (row * nb + blk) * kBPB;
#pragma unroll
            for (int i = 0; i < kBPB; ++i) b[i] = src[i];
            scale = (uint16_t)(b[0] | (b[1] << 8));
            if constexpr (kMin) minv = (uint16_t)(b[2] | (b[3] << 8));
            const uint8_t* qs = b + kCodeOff;
            if constexpr (kQ4) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t v = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t lo = q4_code(qs, 8 * j + i);
                        const uint32_t hi = q4_code(qs, 8 * j + 4 + i);
                        v |= (lo | (hi << 4)) << (8 * i);
                    }
                    w[j] = v ^ 0x88888888u;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    w[j] = (uint32_t)qs[4 * j] | ((uint32_t)qs[4 * j + 1] << 8) | ((uint32_t)qs[4 * j + 2] << 16) |
                           ((uint32_t)qs[4 * j + 3] << 24);
            }
        }
        reinterpret_cast<uint16_t*>(chunk + kTileEntries * kCB)[e] = scale;
        if constexpr (kMin) reinterpret_cast<uint16_t*>(chunk + kQ41MinOff)[e] = minv;
        uint4* c4 = reinterpret_cast<uint4*>(chunk + e * kCB);
        c4[0] = make_uint4(w[0], w[1], w[2], w[3]);
        if constexpr (!kQ4) c4[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
}

// 16 GGUF code bytes of a slot as 32-bit words: from LDS byte address a (any
// alignment) by word reads at the boundary below it, realigned.  Reads up to 3 bytes
// past the 16 (within the staged span).
template <int kWords>
__device__ __forceinline__ void lds_words(const uint8_t* base, int a, uint32_t* q) {
    const int sh = a & 3;
    const uint32_t* a32 = reinterpret_cast<const uint32_t*>(base + (a - sh));
    uint32_t v[kWords + 1];
#pragma unroll
    for (int j = 0; j <= kWords; ++j) v[j] = a32[j];
#pragma unroll
    for (int j = 0; j < kWords; ++j) q[j] = __builtin_amdgcn_alignbyte(v[j + 1], v[j], (uint32_t)sh);
}

// K-quant super-blocks -> chunks (layouts in qmm_internal.hpp).  A workgroup fills the
// kRepackChunks consecutive chunks of one row tile that cover two super-blocks (groups
// 4q .. 4q + 3; a group is half a super-block); thread t fills slot t % 64 of chunk
// t / 64, consecutive threads consecutive slots, so a wave writes a chunk's codes as one
// contiguous span; every byte of the chunk array is written (padding rows as zeros).
// A slot's source bytes lie in several places of its super-block (Q6_K: codes, high
// bits, scales; Q4_K: codes, scale, d, dmin), so the 16 rows' two super-blocks are
// first copied to LDS by 4-byte buffer loads with an LDS destination, all issued
// before the first wait.  A row's span starts at any byte (210 is not a multiple of 4,
// and device uploads may start anywhere): the copies run 4-byte aligned from a buffer
// resource based at the source rounded down to 4 bytes; a word past the source reads
// zero, and the source's last word, when partial, is re-read byte by byte, so nothing
// past the source is read.  Each slot then takes its codes as 32-bit LDS words and
// moves nibbles and 2-bit fields with byte permutes and masked shifts.  Measured on
// MI355X at 11008 x 4096 (whole upload calls into caller memory): Q4_K 14.1 us and
// Q6_K 20.3 us with register copies (a wait per copy, Q6_K) or byte loads from HBM
// (Q4_K) and per-element byte loops.
// Super-block reading as the reference's (paths relative to
// openmini-server/src/model/inference/):
//   Q4_K quant.rs:338-410: d = fp16 at 0, dmin = fp16 at 2, scale of sub-block sb =
//        byte 4 + sb & 0x3F, codes from byte 12 (sub-block sb: 16 bytes at 12 + 16 sb,
//        element 2j in the high nibble of byte j as in Q4_0), minimum always 0.
//   Q6_K quant.rs:515-600: d = fp16 at 0; element i: low = nibble of byte 2 + i / 2
//        (even i: low nibble), high = bits 2 (i % 4) of byte 66 + i / 4,
//        q = low + 16 high - 32, scale = int8 byte 130 + i / 16.
//   Q5_K quant.rs:433-505: d = fp16 at 0, dmin = fp16 at 2, scale of sub-block sb =
//        byte 4 + sb & 0x3F, minimum = nibble sb % 2 of byte 12 + sb / 2 (even sb: low),
//        element i: q4 = nibble of byte 36 + 16 sb + i / 2 (even i: high), high bit =
//        bit i % 8 of byte 20 + sb; value (q4 + 16 bit - 16) d scale + dmin minimum.
//        Written as Q6_K's low nibbles (q4), the high-bit byte, scale and minimum per
//        slot, then d and dmin per row.
//   Q8_K quant.rs:768-800: d = fp16 at 0, element i = int8 byte 2 + i, value q d.
//        Written as a Q8_0 chunk: the codes of 32-element sub-block sb as they stand,
//        d as every slot's scale.
template <int kType>
__global__ __launch_bounds__(kRepackThreads) void repack_kquant_kernel(const uint8_t* __restrict__ gguf,
                                                                       uint32_t src_bytes, int64_t n,
                                                                       int64_t supers, int64_t groups,
                                                                       int64_t quads,
                                                                       uint8_t* __restrict__ chunks) {
    constexpr bool kQ5 = kType == OPENMINI_QMM_Q5_K;
    constexpr bool kQ6 = kType == OPENMINI_QMM_Q6_K || kQ5;  // Q6_K chunk layout
    constexpr bool kQ8K = kType == OPENMINI_QMM_Q8_K;        // Q8_0 chunk layout
    constexpr int kBPB = kQ8K ? 258 : kQ5 ? 176 : kType == OPENMINI_QMM_Q6_K ? 210 : 144;
    constexpr int kChunk = kQ8K ? chunk_bytes_for(false) : kQ5 ? kQ5KChunk : kQ6 ? kQ6KChunk : kQ4KChunk;
    constexpr int kScaleOff = kQ6 ? kTileEntries * 24 : kTileEntries * 16;
    constexpr int kDOff = kScaleOff + (kQ6 ? 2 : 1) * kTileEntries;
    constexpr int kSpan = 2 * kBPB;                // one row's bytes in the workgroup
    constexpr int kRowDw = (kSpan + 3 + 3) / 4;    // dwords that cover it from any start
    constexpr int kWords = kTileRows * kRowDw;
    constexpr int kWordsPad = (kWords + 63) / 64 * 64;  // whole waves of copies
    static_assert(kRepackChunks == 4, "a workgroup covers two super-blocks");
    __shared__ uint32_t stage[kWordsPad];
    const uint8_t* st8 = reinterpret_cast<const uint8_t*>(stage);

    const int64_t rt = (int64_t)blockIdx.x / quads, q = (int64_t)blockIdx.x % quads;
    const int64_t row0 = rt * kTileRows, s0 = 2 * q;
    const uint32_t delta = (uint32_t)((uintptr_t)gguf & 3u);
    const uint64_t end = (uint64_t)src_bytes + delta;  // the source's end from the aligned base
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(reinterpret_cast<const void*>((uintptr_t)gguf & ~(uintptr_t)3), (uint32_t)end);
    // byte offset of row r's span from the aligned base (fits: src_bytes + 3 < 2^32)
    auto span_off = [&](int r) {
        return (uint32_t)(((row0 + r) * supers + s0) * kBPB) + delta;
    };
    auto word_off = [&](int i) -> uint64_t {  // source offset of staged word i
        const int r = i / kRowDw, j = i % kRowDw;
        return (uint64_t)(span_off(r) & ~3u) + 4u * (uint32_t)j;
    };
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i0 = wave * 64; i0 < kWords; i0 += kRepackThreads) {  // i0 uniform per wave
        const int i = i0 + lane;
        const uint64_t a = word_off(i);
        const bool live = i < kWords && row0 + i / kRowDw < n && a + 4 <= end;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(stage + i0), 4,
                                                 live ? (uint32_t)a : 0x80000000u, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // this thread's copies have landed
    __syncthreads();
    if ((end & 3u) != 0 && row0 + kTileRows >= n && s0 + 2 >= supers) {  // uniform: may hold the source's last word
        for (int i = threadIdx.x; i < kWords; i += kRepackThreads) {
            const uint64_t a = word_off(i);
            if (row0 + i / kRowDw < n && a < end && a + 4 > end) {
                uint32_t v = 0;
                for (uint32_t b = 0; a + b < end; ++b)
                    v |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, (uint32_t)(a + b), 0, 0) << (8 * b);
                stage[i] = v;
            }
        }
        __syncthreads();
    }

    const int t = threadIdx.x, c = t / kTileEntries, e = t % kTileEntries, r = e & 15;
    const int64_t g = q * kRepackChunks + c;
    if (g >= groups) return;
    const int64_t row = row0 + r;
    const int sub = (c & 1) * kTileBlocks + (e >> 4);  // 32-element sub-block of super-block s0 + c / 2
    uint8_t* ch = chunks + (rt * groups + g) * kChunk;
    uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t sc = 0, mn = 0;
    uint16_t dbits = 0, dmbits = 0;
    if (row < n) {
        const int blk = r * kRowDw * 4 + (int)(span_off(r) & 3u) + (c >> 1) * kBPB;  // LDS byte address
        const uint16_t d = (uint16_t)(st8[blk] | (st8[blk + 1] << 8));
        uint32_t qw[4];
        if constexpr (kQ8K) {
            lds_words<8>(st8, blk + 2 + sub * 32, w);
            dbits = d;
        } else if constexpr (!kQ6) {
            lds_words<4>(st8, blk + 12 + sub * 16, qw);
            // code word j: elements 8 j .. 8 j + 7 from GGUF bytes s0..s3 (element 2 m in
            // the high nibble of s_m): chunk bytes (s0.hi | s2.hi << 4, s0.lo | s2.lo << 4,
            // s1.hi | s3.hi << 4, s1.lo | s3.lo << 4), nibble q ^ 8 (two's-complement q - 8)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t pp = __builtin_amdgcn_perm(0u, qw[j], 0x01010000u);  // s0 s0 s1 s1
                const uint32_t rr = __builtin_amdgcn_perm(0u, qw[j], 0x03030202u);  // s2 s2 s3 s3
                const uint32_t lo = ((pp >> 4) & 0x000F000Fu) | (pp & 0x0F000F00u);
                const uint32_t hi = (rr & 0x00F000F0u) | ((rr << 4) & 0xF000F000u);
                w[j] = (lo | hi) ^ 0x88888888u;
            }
            sc = st8[blk + 4 + sub] & 0x3Fu;
            // dmin * 0 is NaN for an inf / NaN dmin, and so is every value of the block
            const uint16_t dmin = (uint16_t)(st8[blk + 2] | (st8[blk + 3] << 8));
            dbits = (dmin & 0x7C00u) == 0x7C00u ? (uint16_t)0x7E00u : d;
        } else if constexpr (kQ5) {
            lds_words<4>(st8, blk + 36 + sub * 16, qw);
            // low nibbles, element 2 m in the HIGH nibble of s_m (as Q4_0), kept as the
            // code's low 4 bits (no sign flip)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t pp = __builtin_amdgcn_perm(0u, qw[j], 0x01010000u);  // s0 s0 s1 s1
                const uint32_t rr = __builtin_amdgcn_perm(0u, qw[j], 0x03030202u);  // s2 s2 s3 s3
                const uint32_t lo = ((pp >> 4) & 0x000F000Fu) | (pp & 0x0F000F00u);
                const uint32_t hi = (rr & 0x00F000F0u) | ((rr << 4) & 0xF000F000u);
                w[j] = lo | hi;
            }
            w[4] = st8[blk + 20 + sub];  // the high-bit byte, as it stands
            sc = st8[blk + 4 + sub] & 0x3Fu;
            const uint32_t mb = st8[blk + 12 + (sub >> 1)];
            mn = (sub & 1) ? (mb >> 4) : (mb & 0x0Fu);
            dbits = d;
            dmbits = (uint16_t)(st8[blk + 2] | (st8[blk + 3] << 8));
        } else {
            lds_words<4>(st8, blk + 2 + sub * 16, qw);
            // low nibbles, element 2 m in the LOW nibble of s_m: chunk bytes
            // (s0.lo | s2.lo << 4, s0.hi | s2.hi << 4, s1.lo | s3.lo << 4, s1.hi | s3.hi << 4)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t pp = __builtin_amdgcn_perm(0u, qw[j], 0x01010000u);
                const uint32_t rr = __builtin_amdgcn_perm(0u, qw[j], 0x03030202u);
                const uint32_t lo = (pp & 0x000F000Fu) | ((pp >> 4) & 0x0F000F00u);
                const uint32_t hi = ((rr << 4) & 0x00F000F0u) | (rr & 0xF000F000u);
                w[j] = lo | hi;
            }
            // top bits: GGUF word m (bytes f = 0..3) holds elements 16 m + 4 f + i in bit
            // pair i of byte f; the chunk wants them in bit pair f of byte i (a 4 x 4
            // transpose of 2-bit fields), as high ^ 2 (v = q & 63 = low + 16 (high ^ 2))
            uint32_t hw[2];
            lds_words<2>(st8, blk + 66 + sub * 8, hw);
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                uint32_t x = hw[m];
                uint32_t tt = ((x >> 6) ^ x) & 0x00CC00CCu;
                x ^= tt ^ (tt << 6);
                tt = ((x >> 12) ^ x) & 0x0000F0F0u;
                x ^= tt ^ (tt << 12);
                w[4 + m] = x ^ 0xAAAAAAAAu;
            }
            sc = (uint32_t)st8[blk + 130 + 2 * sub] | ((uint32_t)st8[blk + 131 + 2 * sub] << 8);
            dbits = d;
        }
    }
    if constexpr (kQ5) {
        reinterpret_cast<uint4*>(ch)[e] = make_uint4(w[0], w[1], w[2], w[3]);
        ch[kQ5KQhOff + e] = (uint8_t)w[4];
        ch[kQ5KScaleOff + e] = (uint8_t)sc;
        ch[kQ5KMinOff + e] = (uint8_t)mn;
        if ((e >> 4) == 0) {
            reinterpret_cast<uint16_t*>(ch + kQ5KDOff)[r] = dbits;
            reinterpret_cast<uint16_t*>(ch + kQ5KDminOff)[r] = dmbits;
        }
        return;
    } else if constexpr (kQ8K) {
        uint4* c4 = reinterpret_cast<uint4*>(ch + e * 32);
        c4[0] = make_uint4(w[0], w[1], w[2], w[3]);
        c4[1] = make_uint4(w[4], w[5], w[6], w[7]);
        reinterpret_cast<uint16_t*>(ch + kTileEntries * 32)[e] = dbits;
        return;
    } else if constexpr (!kQ6) {
        reinterpret_cast<uint4*>(ch)[e] = make_uint4(w[0], w[1], w[2], w[3]);
        ch[kScaleOff + e] = (uint8_t)sc;
    } else {
        reinterpret_cast<uint4*>(ch)[e] = make_uint4(w[0], w[1], w[2], w[3]);
        reinterpret_cast<uint2*>(ch + kTileEntries * 16)[e] = make_uint2(w[4], w[5]);
        reinterpret_cast<uint16_t*>(ch + kScaleOff)[e] = (uint16_t)sc;
    }
    if ((e >> 4) == 0) reinterpret_cast<uint16_t*>(ch + kDOff)[r] = dbits;
}

// Chunked weight -> f32 [n][k] (8 * nwords outputs, row-major; one code word = 8
// consecutive elements of a row).  A wave covers 512 consecutive outputs: lane l
// decodes the half-word of four at 4 l and the one at 256 + 4 l, so each of its two
// 16-byte streaming stores is one contiguous 1 KB span.
template <bool kQ4>
__global__ __launch_bounds__(256) void dequant_weight_kernel(const uint8_t* __restrict__ chunks,
                                                             int64_t nwords, int64_t nb,
                                                             int64_t groups, float* __restrict__ out) {
    constexpr int kCB = kQ4 ? 16 : 32;
    constexpr int kChunk = chunk_bytes_for(kQ4);
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t ea = (t >> 6) * 512 + (t & 63) * 4, total = nwords * 8;
    typedef float f32x4v __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int64_t e = ea + 256 * half;  // a multiple of 4; total is a multiple of 8
        if (e >= total) return;
        const int64_t g = e >> 3;
        const int hi = (int)((e >> 2) & 1);  // elements 4..7 of the word
        const int64_t row = g / (nb * 4);
        const int64_t rem = g - row * nb * 4;
        const int64_t blk = rem >> 2;
        const uint8_t* chunk = chunks + chunk_of(row, blk, groups) * kChunk;
        const int slot = slot_of(row, blk);
        const int j = (int)(rem & 3);
        const float d = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(chunk + kTileEntries * kCB)[slot]);
        float v[4];
        if constexpr (kQ4) {
            const uint32_t w = reinterpret_cast<const uint32_t*>(chunk + slot * 16)[j];
#pragma unroll
            for (int i = 0; i < 4; ++i)  // sign-extend the nibble to (q - 8) exactly, one fp32 multiply (quant.rs:190)
                v[i] = (float)((int)(w << ((hi ? 24 : 28) - 8 * i)) >> 28) * d;
        } else {
            const uint2 w2 = reinterpret_cast<const uint2*>(chunk + slot * 32)[j];
            const uint32_t w = hi ? w2.y : w2.x;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = (float)(int8_t)(w >> (8 * i)) * d;
        }
        __builtin_nontemporal_store(f32x4v{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4v*>(out + e));
    }
}

// Each value follows the reference's formula
// with one IEEE operation per Rust operator, in its order, and no contraction: every
// product in these formulas is exact in binary32 (at most 23 significant bits), so
// only the final additions round and the results are bit-identical, signed zeros
// included.  Blocks past `avail_blocks` (short input) produce zeros, as the reference
// stops at the first block that does not fit (e.g. quant.rs:224-226).

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    return f16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

// quant.rs:216-262: [d][m][16 B codes]; element 2j high nibble, 2j+1 low; q * d + m.
__device__ float elem_q4_1(const uint8_t* b, int i) {
#pragma clang fp contract(off)
    const float d = f16_at(b), m = f16_at(b + 2);
    const uint8_t c = b[4 + i / 2];
    const float q = (float)((i & 1) ? (c & 0x0F) : (c >> 4));
    return q * d + m;
}
// quant.rs:338-410: the minimum is read past the 8 scale bytes, so it is 0.0.
__device__ float elem_q4_k(const uint8_t* b, int i) {
#pragma clang fp contract(off)
    const float d = f16_at(b), dmin = f16_at(b + 2);
    const int sb = i >> 5, j = i & 31;
    const float scale = (float)(b[4 + sb] & 0x3F);
    const uint8_t c = b[12 + sb * 16 + j / 2];
    const float q = (float)((j & 1) ? (c & 0x0F) : (c >> 4));
    const float t = (q - 8.0f) * d * scale;
    return t + dmin * 0.0f;
}
// quant.rs:433-505
__device__ float elem_q5_k(const uint8_t* b, int i) {
#pragma clang fp contract(off)
    const float d = f16_at(b), dmin = f16_at(b + 2);
    const int sb = i >> 5, j = i & 31;
    const float scale = (float)(b[4 + sb] & 0x3F);
    const uint8_t mb = b[4 + 8 + sb / 2];
    const float min_val = (float)((sb & 1) ? (mb >> 4) : (mb & 0x0F));
    const float qh_bit = (float)((b[20 + sb] >> (j & 7)) & 1);
    const uint8_t c = b[36 + sb * 16 + j / 2];
    const float q4 = (float)((j & 1) ? (c & 0x0F) : (c >> 4));
    const float q = q4 + qh_bit * 16.0f;
    const float t = (q - 16.0f) * d * scale;
    return t + dmin * min_val;
}
// quant.rs:515-600
__device__ float elem_q6_k(const uint8_t* b, int i) {
#pragma clang fp contract(off)
    const float d = f16_at(b);
    const float scale = (float)(int8_t)b[130 + i / 16];
    const uint8_t l = b[2 + i / 2];
    const int low = (i & 1) ? (l >> 4) : (l & 0x0F);
    const int high = (b[66 + i / 4] >> ((i & 3) * 2)) & 0x03;
    const int q = low | ((high << 4) - 32);
    return (float)q * d * scale;
}
// quant.rs:605-660: code bytes past the 32 of the block give q = 1 (:645-649).
__device__ float elem_q2_k(const uint8_t* b, int i) {
#pragma clang fp contract(off)
    const float d = f16_at(b), dmin = f16_at(b + 2);
    const int sb = i >> 4, j = i & 15;
    const float scale = (float)b[4 + sb], min_val = (float)b[20 + sb];
    const int byte_idx = sb * 8 + j / 4;
    const float q = byte_idx < 32 ? (float)((b[36 + byte_idx] >> ((j & 3) * 2)) & 0x03) : 1.0f;
    const float t = (q - 2.0f) * d * scale;
    return t + dmin * min_val;
}
// quant.rs:682-760
__device__ float elem_q3_k(const uint8_t* b, int i) {
#pragma clang fp contract(off)
    const float d = f16_at(b);
    const float scale = (float)(int8_t)b[130 + i / 8];
    const uint8_t l = b[2 + i / 2];
    const int lb = (i & 1) ? ((l >> 4) & 0x07) : (l & 0x07);
    const int hb = (b[66 + i / 4] >> ((i & 3) * 2)) & 0x01;
    const int q = (lb | (hb << 3)) - 16;
    return (float)q * d * scale;
}
// quant.rs:768-800
__device__ float elem_q8_k(const uint8_t* b, int i) { return (float)(int8_t)b[2 + i] * f16_at(b); }

template <int kType>
struct Layout;
template <> struct Layout<OPENMINI_QMM_Q4_0> { static constexpr int kQ = 32, kB = 18; };
template <> struct Layout<OPENMINI_QMM_Q8_0> { static constexpr int kQ = 32, kB = 34; };
template <> struct Layout<OPENMINI_QMM_Q4_1> { static constexpr int kQ = 32, kB = 20; };
template <> struct Layout<OPENMINI_QMM_Q2_K> { static constexpr int kQ = 256, kB = 68; };
template <> struct Layout<OPENMINI_QMM_Q3_K> { static constexpr int kQ = 256, kB = 162; };
template <> struct Layout<OPENMINI_QMM_Q4_K> { static constexpr int kQ = 256, kB = 144; };
template <> struct Layout<OPENMINI_QMM_Q5_K> { static constexpr int kQ = 256, kB = 176; };
template <> struct Layout<OPENMINI_QMM_Q6_K> { static constexpr int kQ = 256, kB = 210; };
template <> struct Layout<OPENMINI_QMM_Q8_K> { static constexpr int kQ = 256, kB = 258; };

template <int kType>
__device__ __forceinline__ float elem(const uint8_t* b, int i) {
    if constexpr (kType == OPENMINI_QMM_Q4_1) return elem_q4_1(b, i);
    if constexpr (kType == OPENMINI_QMM_Q2_K) return elem_q2_k(b, i);
    if constexpr (kType == OPENMINI_QMM_Q3_K) return elem_q3_k(b, i);
    if constexpr (kType == OPENMINI_QMM_Q4_K) return elem_q4_k(b, i);
    if constexpr (kType == OPENMINI_QMM_Q5_K) return elem_q5_k(b, i);
    if constexpr (kType == OPENMINI_QMM_Q6_K) return elem_q6_k(b, i);
    return elem_q8_k(b, i);
}

// Four outputs at element e (a multiple of 4) of one block.  Q4_0 / Q8_0
// (quant.rs:152-195, 282-316) read the scale and codes as halfwords when the source
// starts on an even address (blocks of 18 / 34 bytes then all do), else byte by byte
// (a tensor of the reference's GGUF dialect can sit at an odd file offset).  Past n or
// past the blocks given: zeros.
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p, bool even) {
    return even ? *reinterpret_cast<const uint16_t*>(p) : (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

template <int kType>
__device__ __forceinline__ void four_values(const uint8_t* __restrict__ gguf, size_t e, size_t n,
                                            size_t avail_blocks, bool even, float* v) {
    using L = Layout<kType>;
    const size_t blk = e / L::kQ;
    const int i0 = (int)(e % L::kQ);
    if (e >= n || blk >= avail_blocks) {
        v[0] = v[1] = v[2] = v[3] = 0.0f;
        return;
    }
    const uint8_t* b = gguf + blk * L::kB;
    if constexpr (kType == OPENMINI_QMM_Q4_0) {
        const float d = f16_bits_to_f32((uint16_t)ld_u16(b, even));
        const uint32_t w = ld_u16(b + 2 + 2 * (i0 / 4), even);  // elements 2j (high nibble), 2j + 1 (low) of byte j
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t c = (w >> (8 * t)) & 0xFFu;
            v[2 * t] = (float)((int)(c >> 4) - 8) * d;
            v[2 * t + 1] = (float)((int)(c & 0x0Fu) - 8) * d;
        }
    } else if constexpr (kType == OPENMINI_QMM_Q8_0) {
        const float d = f16_bits_to_f32((uint16_t)ld_u16(b, even));
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t w = ld_u16(b + 2 + 2 * (i0 / 2 + p), even);
            v[2 * p] = (float)(int8_t)(w & 0xFFu) * d;
            v[2 * p + 1] = (float)(int8_t)(w >> 8) * d;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = elem<kType>(b, i0 + j);
    }
}

// A wave covers 512 consecutive outputs: lane l computes the four at 4 l and the four
// at 256 + 4 l, so each of its two store instructions writes one contiguous 1 KB span
// (whole 128-byte lines).  Values are computed before the stores, which are streaming
// (nontemporal): the output is written once and not read back here.
template <int kType>
__global__ __launch_bounds__(256) void dequant_layout_kernel(const uint8_t* __restrict__ gguf, size_t n,
                                                             size_t avail_blocks, float* __restrict__ out) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t ea = (t >> 6) * 512 + (t & 63) * 4;
    if (ea >= n) return;
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    const bool aligned = ((uintptr_t)out & 15) == 0;
    const bool even = ((uintptr_t)gguf & 1) == 0;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const size_t e = ea + 256 * half;
        float v[4];
        four_values<kType>(gguf, e, n, avail_blocks, even, v);
        if (aligned && e + 4 <= n) {
            __builtin_nontemporal_store(f32x4v{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4v*>(out + e));
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (e + j < n) out[e + j] = v[j];
        }
    }
}

// F32 / F16 arms (quant.rs:95-133): element-wise, missing bytes give 0.  Same wave
// layout as the block arms (512 outputs per wave, contiguous 1 KB store spans).  With
// a 16-byte aligned source, a lane's four inputs come in one load; otherwise byte by
// byte.
template <int kEsz>
__global__ __launch_bounds__(256) void dequant_plain_kernel(const uint8_t* __restrict__ src, size_t n,
                                                            size_t avail, float* __restrict__ out) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t ea = (t >> 6) * 512 + (t & 63) * 4;
    if (ea >= n) return;
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    const bool src16 = ((uintptr_t)src & 15) == 0, out16 = ((uintptr_t)out & 15) == 0;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const size_t e = ea + 256 * half;
        float v[4];
        if (src16 && e + 4 <= avail) {
            if constexpr (kEsz == 4) {
                const float4 q = *reinterpret_cast<const float4*>(src + 4 * e);
                v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
            } else {
                const uint2 q = *reinterpret_cast<const uint2*>(src + 2 * e);
                v[0] = f16_bits_to_f32((uint16_t)(q.x & 0xFFFFu));
                v[1] = f16_bits_to_f32((uint16_t)(q.x >> 16));
                v[2] = f16_bits_to_f32((uint16_t)(q.y & 0xFFFFu));
                v[3] = f16_bits_to_f32((uint16_t)(q.y >> 16));
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const size_t i = e + j;
                if (i >= avail) {
                    v[j] = 0.0f;
                } else if constexpr (kEsz == 2) {
                    v[j] = f16_at(src + 2 * i);
                } else {
                    const uint8_t* p = src + 4 * i;
                    v[j] = __uint_as_float((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                                           ((uint32_t)p[3] << 24));
                }
            }
        }
        if (out16 && e + 4 <= n) {
            __builtin_nontemporal_store(f32x4v{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4v*>(out + e));
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (e + j < n) out[e + j] = v[j];
        }
    }
}

__global__ __launch_bounds__(256) void stream_copy_kernel(const uint4* __restrict__ src,
                                                          uint4* __restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

// Read-only streaming yardstick: every 16-byte word of src is read once (kReadU loads in
// flight per lane, workgroups of 512 lanes over consecutive 16 KB spans), folded into a
// register, and nothing is stored unless a lane's fold equals a sentinel (which keeps
// the loads live).  The single-launch floor a read-bound kernel of `bytes` meets.  The
// shape is the fastest of a sweep on MI355X (1-16 loads per lane, 256-1024 lanes per
// workgroup, strided or per-wave spans): at 25.4 MB, 2 loads x 512 lanes took 5.37 us
// against 5.69 us for 4 x 512 and 5.79 us for 8 x 1024.
constexpr int kReadU = 2;
__global__ __launch_bounds__(512) void stream_read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
    const int64_t base = (int64_t)blockIdx.x * (512 * kReadU) + threadIdx.x;
    uint4 v[kReadU];
#pragma unroll
    for (int u = 0; u < kReadU; ++u) {
        const int64_t i = base + (int64_t)u * 512;
        v[u] = i < n16 ? src[i] : make_uint4(0, 0, 0, 0);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < kReadU; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// quant_simd::convert_to_soa_layout's block arms (quant_simd.rs:3300-3397): output byte
// o is byte (o & 1) of fp16 field f (scale; Q4_1 also min) of block b for o below
// 2 * fields * blocks, else code position pos of block b, position-major.  A field is
// copied only when both of its bytes are in the input; missing code bytes are 0.
__global__ __launch_bounds__(256) void soa_kernel(const uint8_t* __restrict__ src, size_t len, size_t blocks,
                                                  int bpb, int fields, uint8_t* __restrict__ out, size_t total) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t hdr = 2 * (size_t)fields * blocks;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
        uint8_t v;
        if (o < hdr) {
            const size_t f = o / (2 * blocks), r = o % (2 * blocks);
            const size_t off = (r >> 1) * bpb + 2 * f;
            v = off + 2 <= len ? src[off + (r & 1)] : 0;
        } else {
            const size_t q = o - hdr, pos = q / blocks, b = q % blocks;
            const size_t off = b * bpb + 2 * (size_t)fields + pos;
            v = off < len ? src[off] : 0;
        }
        out[o] = v;
    }
}

inline unsigned grid_for(int64_t items, int per_block) {
    return (unsigned)((items + per_block - 1) / per_block);
}

// Clears n words: the batched GEMV's split counters of a new weight, on the upload's
// stream (a kernel rather than a memset node, so the upload may be graph-captured).
__global__ void zero_words_kernel(uint32_t* __restrict__ p, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) p[i] = 0;
}

hipError_t launch_repack_chunks(const Weight& w, const uint8_t* gguf, hipStream_t s);

}  // namespace

hipError_t launch_repack(const Weight& w, const uint8_t* gguf, hipStream_t s) {
    const hipError_t e = launch_repack_chunks(w, gguf, s);
    if (e != hipSuccess || !w.split_cnt) return e;
    const int n = (int)((w.n_tiles + w.split_t - 1) / w.split_t);
    hipLaunchKernelGGL(zero_words_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, w.split_cnt, n);
    return hipGetLastError();
}

namespace {

hipError_t launch_repack_chunks(const Weight& w, const uint8_t* gguf, hipStream_t s) {
    if (w.n_tiles <= 0 || w.groups <= 0) return hipSuccess;
    if (is_kquant(w.src_type) || w.src_type == OPENMINI_QMM_Q8_K) {
        const int64_t supers = w.k / 256;
        const int64_t src = w.n * supers * bytes_per_block(w.src_type);
        // 32-bit buffer offsets: the source is smaller than the chunk array (< 4 GiB)
        if (src + 4 > (int64_t)UINT32_MAX) return hipErrorInvalidValue;
        const int64_t quads = (w.groups + kRepackChunks - 1) / kRepackChunks;
        const dim3 grid((unsigned)(w.n_tiles * quads));
        if (w.src_type == OPENMINI_QMM_Q4_K)
            hipLaunchKernelGGL(repack_kquant_kernel<OPENMINI_QMM_Q4_K>, grid, dim3(kRepackThreads), 0, s, gguf,
                               (uint32_t)src, w.n, supers, w.groups, quads, w.chunks);
        else if (w.src_type == OPENMINI_QMM_Q8_K)
            hipLaunchKernelGGL(repack_kquant_kernel<OPENMINI_QMM_Q8_K>, grid, dim3(kRepackThreads), 0, s, gguf,
                               (uint32_t)src, w.n, supers, w.groups, quads, w.chunks);
        else if (w.src_type == OPENMINI_QMM_Q5_K)
            hipLaunchKernelGGL(repack_kquant_kernel<OPENMINI_QMM_Q5_K>, grid, dim3(kRepackThreads), 0, s, gguf,
                               (uint32_t)src, w.n, supers, w.groups, quads, w.chunks);
        else
            hipLaunchKernelGGL(repack_kquant_kernel<OPENMINI_QMM_Q6_K>, grid, dim3(kRepackThreads), 0, s, gguf,
                               (uint32_t)src, w.n, supers, w.groups, quads, w.chunks);
        return hipGetLastError();
    }
    // staged rows start 16-byte aligned: an aligned source and nb * bytes per block a
    // multiple of 16 (Q4_0 / Q8_0: nb % 8 == 0, Q4_1: nb % 4 == 0)
    const int aligned = ((uintptr_t)gguf % 16) == 0 && (w.nb * bytes_per_block(w.type)) % 16 == 0;
    const int64_t quads = (w.groups + kRepackChunks - 1) / kRepackChunks;
    constexpr int kQ4Quads = 2, kQ8Quads = 2;
    if (w.type == OPENMINI_QMM_Q4_1) {
        const int64_t per_tile = (quads + kQ4Quads - 1) / kQ4Quads;
        hipLaunchKernelGGL((repack_kernel<20, kQ4Quads>), dim3((unsigned)(w.n_tiles * per_tile)),
                           dim3(kRepackThreads), 0, s, gguf, w.n, w.nb, w.groups, per_tile, aligned, w.chunks);
    } else if (w.type == OPENMINI_QMM_Q4_0) {
        const int64_t per_tile = (quads + kQ4Quads - 1) / kQ4Quads;
        hipLaunchKernelGGL((repack_kernel<18, kQ4Quads>), dim3((unsigned)(w.n_tiles * per_tile)),
                           dim3(kRepackThreads), 0, s, gguf, w.n, w.nb, w.groups, per_tile, aligned, w.chunks);
    } else {
        const int64_t per_tile = (quads + kQ8Quads - 1) / kQ8Quads;
        hipLaunchKernelGGL((repack_kernel<34, kQ8Quads>), dim3((unsigned)(w.n_tiles * per_tile)),
                           dim3(kRepackThreads), 0, s, gguf, w.n, w.nb, w.groups, per_tile, aligned, w.chunks);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dequant_weight(const Weight& w, float* out, hipStream_t s) {
    const int64_t nwords = w.n * w.nb * 4;
    if (nwords == 0) return hipSuccess;
    const dim3 grid(grid_for((nwords * 8 + 511) / 512 * 64, 256));  // a wave per 512 outputs
    if (w.type == OPENMINI_QMM_Q4_0)
        hipLaunchKernelGGL(dequant_weight_kernel<true>, grid, dim3(256), 0, s, w.chunks, nwords,
                           w.nb, w.groups, out);
    else
        hipLaunchKernelGGL(dequant_weight_kernel<false>, grid, dim3(256), 0, s, w.chunks, nwords,
                           w.nb, w.groups, out);
    return hipGetLastError();
}

size_t soa_bytes(int type, size_t len, size_t n) {
    if (len == 0 || n == 0) return 0;
    if (type == OPENMINI_QMM_F32) return n * 4 < len ? n * 4 : len;
    if (type == OPENMINI_QMM_F16) return n * 2 < len ? n * 2 : len;
    if (type == OPENMINI_QMM_Q4_0 || type == OPENMINI_QMM_Q4_1 || type == OPENMINI_QMM_Q8_0)
        return (n + kQK - 1) / kQK * (size_t)layout_bytes_per_block(type);
    return len;
}

hipError_t launch_convert_to_soa(int type, const uint8_t* src, size_t len, size_t n, uint8_t* out, hipStream_t s) {
    const size_t total = soa_bytes(type, len, n);
    if (total == 0) return hipSuccess;
    if (type != OPENMINI_QMM_Q4_0 && type != OPENMINI_QMM_Q4_1 && type != OPENMINI_QMM_Q8_0)
        return hipMemcpyAsync(out, src, total, hipMemcpyDeviceToDevice, s);  // the copy arms
    const size_t blocks = (n + kQK - 1) / kQK;
    const int64_t wgs = ((int64_t)(total / 256) + 1) < 65536 ? (int64_t)(total / 256) + 1 : 65536;
    hipLaunchKernelGGL(soa_kernel, dim3((unsigned)wgs), dim3(256), 0, s, src, len, blocks, layout_bytes_per_block(type),
                       type == OPENMINI_QMM_Q4_1 ? 2 : 1, out, total);
    return hipGetLastError();
}

hipError_t launch_dequant_layout(int type, const uint8_t* gguf, size_t bytes, size_t n_elems, float* out,
                                 hipStream_t s) {
    // A launch covers fewer than 2^32 work-items: larger tensors go in slices of 2^30
    // elements (a whole number of blocks of every layout), each reading its own
    // blocks and writing its own outputs.
    constexpr size_t kSlice = (size_t)1 << 30;
    if (n_elems > kSlice) {
        const int bs = layout_block_size(type);
        const int bpb = layout_bytes_per_block(type);
        if (bs <= 0 || kSlice % (size_t)bs != 0) return hipErrorInvalidValue;
        for (size_t e0 = 0; e0 < n_elems; e0 += kSlice) {
            const size_t n = n_elems - e0 < kSlice ? n_elems - e0 : kSlice;
            const size_t skip = e0 / (size_t)bs * (size_t)bpb;  // bytes before this slice
            const size_t avail = bytes > skip ? bytes - skip : 0;
            const hipError_t e = launch_dequant_layout(type, avail ? gguf + skip : gguf, avail, n, out + e0, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (n_elems == 0) return hipSuccess;
    if (type == OPENMINI_QMM_F32 || type == OPENMINI_QMM_F16) {
        const dim3 grid(grid_for((int64_t)((n_elems + 511) / 512 * 64), 256));  // a wave per 512 outputs
        if (type == OPENMINI_QMM_F16)
            hipLaunchKernelGGL(dequant_plain_kernel<2>, grid, dim3(256), 0, s, gguf, n_elems, bytes / 2, out);
        else
            hipLaunchKernelGGL(dequant_plain_kernel<4>, grid, dim3(256), 0, s, gguf, n_elems, bytes / 4, out);
        return hipGetLastError();
    }
    const dim3 grid(grid_for((int64_t)((n_elems + 511) / 512 * 64), 256));  // a wave per 512 outputs
    switch (type) {
#define QMM_LAYOUT_CASE(T)                                                                              \
    case T:                                                                                             \
        hipLaunchKernelGGL(dequant_layout_kernel<T>, grid, dim3(256), 0, s, gguf, n_elems,              \
                           bytes / Layout<T>::kB, out);                                                 \
        return hipGetLastError();
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q4_0)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q8_0)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q4_1)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q2_K)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q3_K)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q4_K)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q5_K)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q6_K)
        QMM_LAYOUT_CASE(OPENMINI_QMM_Q8_K)
#undef QMM_LAYOUT_CASE
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s) {
    const int64_t n16 = (int64_t)(bytes / 16);
    if (n16 == 0) return hipSuccess;
    int64_t blocks = grid_for(n16, 256);
    if (blocks > 256 * 32) blocks = 256 * 32;
    hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       reinterpret_cast<const uint4*>(src), reinterpret_cast<uint4*>(dst), n16);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t s) {
    const int64_t n16 = (int64_t)(bytes / 16);
    if (n16 == 0) return hipSuccess;
    const int64_t blocks = (n16 + 512 * kReadU - 1) / (512 * kReadU);
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(512), 0, s,
                       reinterpret_cast<const uint4*>(src), n16, sink);
    return hipGetLastError();
}

}  // namespace qmm
