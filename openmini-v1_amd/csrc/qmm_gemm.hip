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
// each own 64 x 64 (4 x 4 MFMA subtiles).  Per K step of 64 (two blocks) the
// workgroup stages X[128][64] bf16 and the 128 code rows in LDS (rows padded to
// dodge bank conflicts); each wave converts its B fragments from LDS codes.
#include "qmm_internal.hpp"

namespace qmm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kKStep = 64;                     // elements per LDS stage (2 blocks)
constexpr int kXRowBytes = kKStep * 2 + 16;    // 144: padded bf16 row
constexpr int kThreads = 256;

template <bool kQ4>
struct CodeTile {
    static constexpr int kRowBytes = kQ4 ? 36 : 72;  // 32 / 64 code bytes + pad
};

__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    // bf16 of exactly-representable values = high halves of their fp32 bits.
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 8 Q4_0 nibbles (one code word) -> 8 bf16 (q-8)/16 in k order.
__device__ __forceinline__ bf16x8 cvt_q4(uint32_t w) {
    uint32_t h = w >> 4;
    asm volatile("" : "+v"(h));
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
                                                        const uint8_t* __restrict__ codes,
                                                        const uint16_t* __restrict__ scales,
                                                        float* __restrict__ y, int m_rows,
                                                        int n_rows, int nb, int k) {
    constexpr int kCB = kQ4 ? 16 : 32;            // code bytes per block
    constexpr int kCRow = CodeTile<kQ4>::kRowBytes;
    __shared__ __attribute__((aligned(16))) uint8_t xs[kBM * kXRowBytes];
    __shared__ __attribute__((aligned(16))) uint8_t cs[kBN * kCRow];
    __shared__ float ds[kBN][2];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM;
    const int n0 = blockIdx.x * kBN;
    const int li = lane & 15;   // row of A / column of B inside a 16 x 16 subtile
    const int lk = lane >> 4;   // which 8-element k group of the 32-element block

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int b0 = 0; b0 < nb; b0 += 2) {
        const int nblk = (nb - b0) >= 2 ? 2 : 1;
        // ---- stage X[128][64] bf16: thread t loads 64 B = half a row -------------
        {
            const int r = t >> 1, h = t & 1;
            const int gm = min(m0 + r, m_rows - 1);
            uint4* dst = reinterpret_cast<uint4*>(xs + r * kXRowBytes + h * 64);
            if (h < nblk) {
                const uint4* src =
                    reinterpret_cast<const uint4*>(x + (size_t)gm * k + (size_t)(b0 + h) * kQK);
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[i] = src[i];
            }
        }
        // ---- stage codes of 128 rows x nblk blocks and their scales -----------------
        {
            const int r = t >> 1, h = t & 1;
            const int gn = min(n0 + r, n_rows - 1);
            if (h < nblk) {
                const size_t bi = (size_t)gn * nb + b0 + h;
                const uint32_t* src = reinterpret_cast<const uint32_t*>(codes + bi * kCB);
                uint32_t* dst = reinterpret_cast<uint32_t*>(cs + r * kCRow + h * kCB);
#pragma unroll
                for (int i = 0; i < kCB / 4; ++i) dst[i] = src[i];
                float d = f16_bits_to_f32(scales[bi]);
                if constexpr (kQ4) d *= 16.0f;
                ds[r][h] = d;
            }
        }
        __syncthreads();

        for (int h = 0; h < nblk; ++h) {
            bf16x8 a[4], bfr[4];
            float dsc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = wm * 64 + i * 16 + li;
                a[i] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const uint4*>(xs + r * kXRowBytes + h * 64 + lk * 16));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = wn * 64 + j * 16 + li;
                const uint8_t* cp = cs + c * kCRow + h * kCB;
                if constexpr (kQ4) {
                    bfr[j] = cvt_q4(*reinterpret_cast<const uint32_t*>(cp + lk * 4));
                } else {
                    const uint32_t* c32 = reinterpret_cast<const uint32_t*>(cp + lk * 8);
                    bfr[j] = cvt_q8(c32[0], c32[1]);
                }
                dsc[j] = ds[c][h];
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
            const int gn = n0 + wn * 64 + j * 16 + li;
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
    const dim3 grid((unsigned)((w.n + kBN - 1) / kBN), (unsigned)((m + kBM - 1) / kBM));
    if (w.type == OPENMINI_QMM_Q4_0)
        hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(kThreads), 0, s, x, w.codes, w.scales, y,
                           (int)m, (int)w.n, (int)w.nb, (int)w.k);
    else
        hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(kThreads), 0, s, x, w.codes, w.scales,
                           y, (int)m, (int)w.n, (int)w.nb, (int)w.k);
    return hipGetLastError();
}

}  // namespace qmm
