// Decode GEMV: y[b, n] = sum_k x[b, k] * w[n, k] for batch 1..8, fp32 activations.
//
// Replaces, per call of linear()/linear_gemm() (openmini-server/src/model/inference/
// model.rs:1050-1064), the W^T copy plus f32 sgemm over weights dequantized at load.
// Here W stays quantized in HBM (0.5625 B/weight Q4_0, 1.0625 B/weight Q8_0) and is
// read exactly once; the kernel is HBM-bound.
//
// Mapping.  A wave owns R consecutive rows.  Its 64 lanes sweep the row's blocks:
// a lane takes G groups of 8 elements (G = 4: one whole 32-element block), so one
// wave-wide load is 64 x 16 B of consecutive code bytes (Q4_0, G = 4).  The lane
// loads its x slice once per sweep step and reuses it for all R rows; every row
// contributes one 16-byte (Q4_0) or 32-byte (Q8_0) code load and one fp16 scale
// load per lane.  Per 8 Q4_0 elements the VALU work is one shift, eight SDWA
// v_cvt_off_f32_i4 (nibble -> (q-8)/16) and eight FMAs; the per-block scale (x16)
// is applied once to the block's partial sum.  Lane partials are summed with a
// butterfly at the end.
#include "qmm_internal.hpp"

namespace qmm {
namespace {

constexpr int kWaves = 4;  // waves per workgroup

__device__ __forceinline__ float nib(uint32_t v) {
    // Only bits [3:0] are converted; the explicit byte mask lets the compiler use an
    // SDWA byte select instead of a shift.
    return __builtin_amdgcn_cvt_off_f32_i4(v);
}

// Sum over the 8 elements of one Q4_0 code word (layout in qmm_internal.hpp), in
// units of 1/16: returns sum_i x_i * (q_i - 8) / 16.
__device__ __forceinline__ float dot8_q4(uint32_t w, const float4& xa, const float4& xb) {
    uint32_t hi = w >> 4;
    asm volatile("" : "+v"(hi));  // keep the shift: 1 shift + 4 SDWA converts, not 4 bfe
    float s0 = xa.x * nib(w & 0xFFu);
    float s1 = xa.y * nib((w >> 8) & 0xFFu);
    s0 = fmaf(xa.z, nib((w >> 16) & 0xFFu), s0);
    s1 = fmaf(xa.w, nib(w >> 24), s1);
    s0 = fmaf(xb.x, nib(hi & 0xFFu), s0);
    s1 = fmaf(xb.y, nib((hi >> 8) & 0xFFu), s1);
    s0 = fmaf(xb.z, nib((hi >> 16) & 0xFFu), s0);
    s1 = fmaf(xb.w, nib(hi >> 24), s1);
    return s0 + s1;
}

// Sum over 8 Q8_0 codes (two words, GGUF order): sum_i x_i * q_i.
__device__ __forceinline__ float dot8_q8(uint32_t w0, uint32_t w1, const float4& xa,
                                         const float4& xb) {
    float s0 = xa.x * (float)(int8_t)(w0 & 0xFFu);
    float s1 = xa.y * (float)(int8_t)((w0 >> 8) & 0xFFu);
    s0 = fmaf(xa.z, (float)(int8_t)((w0 >> 16) & 0xFFu), s0);
    s1 = fmaf(xa.w, (float)(int8_t)(w0 >> 24), s1);
    s0 = fmaf(xb.x, (float)(int8_t)(w1 & 0xFFu), s0);
    s1 = fmaf(xb.y, (float)(int8_t)((w1 >> 8) & 0xFFu), s1);
    s0 = fmaf(xb.z, (float)(int8_t)((w1 >> 16) & 0xFFu), s0);
    s1 = fmaf(xb.w, (float)(int8_t)(w1 >> 24), s1);
    return s0 + s1;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// kQ4: Q4_0 (true) or Q8_0.  R rows per wave, B batch rows, G 8-element groups per
// lane (4 = whole block per lane, 2 = half, 1 = quarter).
template <bool kQ4, int R, int B, int G>
__global__ __launch_bounds__(kWaves * 64) void gemv_kernel(const uint8_t* __restrict__ codes,
                                                           const uint16_t* __restrict__ scales,
                                                           const float* __restrict__ x,
                                                           float* __restrict__ y, int n_rows,
                                                           int nb, int k) {
    constexpr int kLanesPerBlock = 4 / G;
    constexpr int kBlocksPerStep = 64 / kLanesPerBlock;
    constexpr int kCodeBytes = kQ4 ? 16 : 32;
    constexpr int kGroupBytes = kQ4 ? 4 : 8;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kWaves + wave) * R;
    if (row0 >= n_rows) return;  // wave-uniform

    const int sub = lane % kLanesPerBlock;  // which G-group slice of the block
    const int g0 = sub * G;                 // first 8-element group of this lane

    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = min(row0 + r, n_rows - 1);

    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.0f;

    for (int blk = lane / kLanesPerBlock; blk < nb; blk += kBlocksPerStep) {
        // x slice: elements [32*blk + 8*g0, +8*G) of every batch row.
        float4 xv[B][2 * G];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float4* xp =
                reinterpret_cast<const float4*>(x + (size_t)b * k + (size_t)blk * kQK + 8 * g0);
#pragma unroll
            for (int i = 0; i < 2 * G; ++i) xv[b][i] = xp[i];
        }
        // code words and scales of all R rows first, so the loads overlap.
        uint32_t cw[R][G * kGroupBytes / 4];
        float d[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t bi = (size_t)rows[r] * nb + blk;
            const uint8_t* cp = codes + bi * kCodeBytes + g0 * kGroupBytes;
            if constexpr (G * kGroupBytes == 16) {
                const uint4 v = *reinterpret_cast<const uint4*>(cp);
                cw[r][0] = v.x; cw[r][1] = v.y; cw[r][2] = v.z; cw[r][3] = v.w;
            } else if constexpr (G * kGroupBytes == 32) {
                const uint4 v0 = reinterpret_cast<const uint4*>(cp)[0];
                const uint4 v1 = reinterpret_cast<const uint4*>(cp)[1];
                cw[r][0] = v0.x; cw[r][1] = v0.y; cw[r][2] = v0.z; cw[r][3] = v0.w;
                cw[r][4] = v1.x; cw[r][5] = v1.y; cw[r][6] = v1.z; cw[r][7] = v1.w;
            } else if constexpr (G * kGroupBytes == 8) {
                const uint2 v = *reinterpret_cast<const uint2*>(cp);
                cw[r][0] = v.x; cw[r][1] = v.y;
            } else {
                cw[r][0] = *reinterpret_cast<const uint32_t*>(cp);
            }
            d[r] = f16_bits_to_f32(scales[bi]);
            if constexpr (kQ4) d[r] *= 16.0f;  // dot8_q4 works in units of 1/16
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float p = 0.0f;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if constexpr (kQ4)
                        p += dot8_q4(cw[r][g], xv[b][2 * g], xv[b][2 * g + 1]);
                    else
                        p += dot8_q8(cw[r][2 * g], cw[r][2 * g + 1], xv[b][2 * g],
                                     xv[b][2 * g + 1]);
                }
                acc[r][b] = fmaf(p, d[r], acc[r][b]);
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float s = wave_sum(acc[r][b]);
            if (lane == ((r * B + b) & 63) && row0 + r < n_rows)
                y[(size_t)b * n_rows + row0 + r] = s;
        }
}

template <bool kQ4, int R, int B, int G>
hipError_t run(const Weight& w, const float* x, float* y, hipStream_t s) {
    const int64_t waves = (w.n + R - 1) / R;
    const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves));
    hipLaunchKernelGGL((gemv_kernel<kQ4, R, B, G>), grid, dim3(kWaves * 64), 0, s, w.codes,
                       w.scales, x, y, (int)w.n, (int)w.nb, (int)w.k);
    return hipGetLastError();
}

template <bool kQ4>
hipError_t dispatch(const Weight& w, const float* x, float* y, int batch, hipStream_t s) {
    switch (batch) {
    case 1: return run<kQ4, 4, 1, 4>(w, x, y, s);
    case 2: return run<kQ4, 4, 2, 4>(w, x, y, s);
    case 3: return run<kQ4, 2, 3, 2>(w, x, y, s);
    case 4: return run<kQ4, 2, 4, 2>(w, x, y, s);
    case 5: return run<kQ4, 2, 5, 1>(w, x, y, s);
    case 6: return run<kQ4, 2, 6, 1>(w, x, y, s);
    case 7: return run<kQ4, 2, 7, 1>(w, x, y, s);
    case 8: return run<kQ4, 2, 8, 1>(w, x, y, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemv(const Weight& w, const float* x, float* y, int batch, hipStream_t s) {
    if (w.type == OPENMINI_QMM_Q4_0) return dispatch<true>(w, x, y, batch, s);
    return dispatch<false>(w, x, y, batch, s);
}

}  // namespace qmm
