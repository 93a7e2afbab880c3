// Prefill GEMM: y[m, n] = sum_k x[m, k] * w[n, k], x bf16, y fp32, on bf16 MFMA.
//
// Replaces, per prefill call of linear_gemm() (openmini-server/src/model/inference/
// model.rs:1060-1064), the f32 GEMM over weights dequantized at load
// (gemm_engine.rs:69-71).  Numerics: each code is exact in bf16 (Q4_0 as
// (q-8)/16, Q8_0 as q), bf16 x bf16 products are exact in fp32, and one
// v_mfma_f32_16x16x32_bf16 covers exactly one 32-element block, so every block's
// partial sum is scaled by its fp32 scale and added to an fp32 accumulator:
//   y[m, n] = sum_b d[n, b] * (sum_{k in b} x[m, k] * q[n, k]).
// Weights are never rounded (no bf16 q*d), activations are not requantized.
//
// Tiling: a 256-thread workgroup computes a 128 x 128 tile of y; its four waves
// each own 64 x 64 (4 x 4 MFMA subtiles).  A K step is one 4-block group (128
// elements): the workgroup stages X[128][128] bf16 (rows padded against bank
// conflicts) and the group's eight 16-row weight tiles -- contiguous 1 KB / 2 KB
// runs of the tiled layout -- in LDS; each wave converts its B fragments from the
// LDS codes.
#include "qmm_internal.hpp"

namespace qmm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;                       // 8 weight tiles
constexpr int kNT = kBN / kTileRows;
constexpr int kKStep = kTileBlocks * kQK;      // 128 elements per LDS stage
constexpr int kXRowBytes = kKStep * 2 + 16;    // 272: padded bf16 row
constexpr int kThreads = 256;

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

template <bool kQ4>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const uint16_t* __restrict__ x,
                                                        const uint8_t* __restrict__ chunks,
                                                        float* __restrict__ y, int m_rows,
                                                        int n_rows, int n_tiles, int groups, int k) {
    constexpr int kCB = kQ4 ? 16 : 32;             // code bytes per slot
    constexpr int kTileBytes = kTileEntries * kCB;  // codes of a chunk: 1 KB / 2 KB
    constexpr int kChunk = chunk_bytes_for(kQ4);
    __shared__ __attribute__((aligned(16))) uint8_t xs[kBM * kXRowBytes];
    __shared__ __attribute__((aligned(16))) uint8_t cs[kNT * kTileBytes];
    __shared__ float ds[kNT][kTileEntries];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM;
    const int tile0 = blockIdx.x * kNT;
    const int li = lane & 15;   // row of A / column of B inside a 16 x 16 subtile
    const int lk = lane >> 4;   // which 8-element k group of the 32-element block

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int g = 0; g < groups; ++g) {
        // ---- stage X[128][128] bf16: 8 x 16 B per thread -------------------------------
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = t + i * kThreads;        // 16-byte piece: row q / 16, piece q % 16
            const int r = q >> 4, p = q & 15;
            const int gm = min(m0 + r, m_rows - 1);
            const int kk = g * kKStep + p * 8;     // first element of the piece
            uint4 v = make_uint4(0, 0, 0, 0);
            if (kk < k) v = *reinterpret_cast<const uint4*>(x + (size_t)gm * k + kk);
            *reinterpret_cast<uint4*>(xs + r * kXRowBytes + p * 16) = v;
        }
        // ---- stage the group's 8 weight tiles and their scales -------------------------
#pragma unroll
        for (int i = 0; i < kNT * kTileBytes / 16 / kThreads; ++i) {
            const int q = t + i * kThreads;        // 16-byte piece of the 8 tiles
            const int tl = q / (kTileBytes / 16), p = q % (kTileBytes / 16);
            const int64_t tile = min(tile0 + tl, n_tiles - 1);
            const uint4* src = reinterpret_cast<const uint4*>(chunks + (tile * groups + g) * kChunk);
            reinterpret_cast<uint4*>(cs)[q] = src[p];
        }
        for (int q = t; q < kNT * kTileEntries; q += kThreads) {
            const int tl = q / kTileEntries, e = q % kTileEntries;
            const int64_t tile = min(tile0 + tl, n_tiles - 1);
            const uint16_t* sc = reinterpret_cast<const uint16_t*>(chunks + (tile * groups + g) * kChunk + kTileBytes);
            float d = f16_bits_to_f32(sc[e]);
            if constexpr (kQ4) d *= 16.0f;
            ds[tl][e] = d;
        }
        __syncthreads();

#pragma unroll
        for (int bt = 0; bt < kTileBlocks; ++bt) {  // block slot within the group
            bf16x8 a[4], bfr[4];
            float dsc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = wm * 64 + i * 16 + li;
                a[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                                      xs + r * kXRowBytes + (bt * kQK + lk * 8) * 2));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int tl = wn * 4 + j;                 // the 16 columns are one weight tile
                const int e = bt * kTileRows + li;         // entry (block slot bt, row li)
                const uint8_t* cp = cs + tl * kTileBytes + e * kCB;
                if constexpr (kQ4) {
                    bfr[j] = cvt_q4(*reinterpret_cast<const uint32_t*>(cp + lk * 4));
                } else {
                    const uint32_t* c32 = reinterpret_cast<const uint32_t*>(cp + lk * 8);
                    bfr[j] = cvt_q8(c32[0], c32[1]);
                }
                dsc[j] = ds[tl][e];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        a[i], bfr[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(p[r], dsc[j], acc[i][j][r]);
                }
        }
        __syncthreads();
    }

    // ---- store: lane holds D[4*lk + r][li] of each subtile ---------------------------
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gn = (tile0 + wn * 4 + j) * kTileRows + li;
            if (gn >= n_rows) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * 64 + i * 16 + lk * 4 + r;
                if (gm < m_rows) y[(size_t)gm * n_rows + gn] = acc[i][j][r];
            }
        }
}

}  // namespace

hipError_t launch_gemm_bf16(const Weight& w, const uint16_t* x, float* y, int64_t m,
                            hipStream_t s) {
    if (m <= 0) return hipSuccess;
    const dim3 grid((unsigned)((w.n_tiles + kNT - 1) / kNT), (unsigned)((m + kBM - 1) / kBM));
    if (w.type == OPENMINI_QMM_Q4_0)
        hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(kThreads), 0, s, x, w.chunks, y, (int)m,
                           (int)w.n, (int)w.n_tiles, (int)w.groups, (int)w.k);
    else
        hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(kThreads), 0, s, x, w.chunks, y, (int)m,
                           (int)w.n, (int)w.n_tiles, (int)w.groups, (int)w.k);
    return hipGetLastError();
}

}  // namespace qmm
