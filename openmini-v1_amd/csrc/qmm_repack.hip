// Upload/repack, dequantization and the streaming-copy yardstick.
//
// Reference semantics (paths relative to openmini-server/):
//   quant::dequantize_q4_0  src/model/inference/quant.rs:152-195
//   quant::dequantize_q8_0  src/model/inference/quant.rs:282-316
//   f16 scale decode        quant.rs:166-167, 296-297 (half::f16::to_f32, exact)
// Q4_0 GGUF byte j of a block holds element 2j in its HIGH nibble and element
// 2j+1 in its LOW nibble (quant.rs:179-188); value = (q - 8) * f32(d).
#include "qmm_internal.hpp"

namespace qmm {
namespace {

constexpr int kTile = 256;  // GGUF blocks per workgroup in the repack

__device__ __forceinline__ uint32_t q4_code(const uint8_t* qs, int e) {
    uint8_t b = qs[e >> 1];
    return (e & 1) ? (b & 0x0Fu) : (b >> 4);
}

// One workgroup repacks kTile consecutive GGUF blocks (row-major order).  Full
// tiles of a 16-byte aligned source are staged through LDS with 16-byte loads (a
// tile is 4608 B for Q4_0 and 8704 B for Q8_0, both multiples of 16); the last
// partial tile and unaligned sources fall back to byte loads.  Each block's codes
// (16 / 32 B) and scale then go to its slot of its chunk.
template <int kBPB>
__global__ __launch_bounds__(kTile) void repack_kernel(const uint8_t* __restrict__ gguf,
                                                       int64_t nblocks, int64_t nb, int64_t groups,
                                                       int aligned16, uint8_t* __restrict__ chunks) {
    constexpr bool kQ4 = kBPB == 18;
    constexpr int kCB = kQ4 ? 16 : 32;
    constexpr int kChunk = chunk_bytes_for(kQ4);
    __shared__ uint4 tile[kTile * kBPB / 16];
    uint8_t* t8 = reinterpret_cast<uint8_t*>(tile);
    const int64_t blk0 = (int64_t)blockIdx.x * kTile;
    const int64_t left = nblocks - blk0;
    const int nblk = left < kTile ? (int)left : kTile;
    const uint8_t* src = gguf + blk0 * kBPB;
    if (nblk == kTile && aligned16) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
        for (int i = threadIdx.x; i < kTile * kBPB / 16; i += kTile) tile[i] = s4[i];
    } else {
        for (int i = threadIdx.x; i < nblk * kBPB; i += kTile) t8[i] = src[i];
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t >= nblk) return;
    const uint8_t* b = t8 + t * kBPB;
    const int64_t g = blk0 + t;
    const int64_t row = g / nb, blk = g % nb;
    uint8_t* chunk = chunks + chunk_of(row, blk, groups) * kChunk;
    const int e = slot_of(row, blk);
    reinterpret_cast<uint16_t*>(chunk + kTileEntries * kCB)[e] = (uint16_t)(b[0] | (b[1] << 8));
    const uint8_t* qs = b + 2;
    if constexpr (kQ4) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t v = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t lo = q4_code(qs, 8 * j + i);
                uint32_t hi = q4_code(qs, 8 * j + 4 + i);
                v |= (lo | (hi << 4)) << (8 * i);
            }
            w[j] = v ^ 0x88888888u;  // nibble q ^ 8: the two's-complement value q - 8
        }
        reinterpret_cast<uint4*>(chunk)[e] = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            w[j] = (uint32_t)qs[4 * j] | ((uint32_t)qs[4 * j + 1] << 8) |
                   ((uint32_t)qs[4 * j + 2] << 16) | ((uint32_t)qs[4 * j + 3] << 24);
        uint4* c4 = reinterpret_cast<uint4*>(chunk) + 2 * e;
        c4[0] = make_uint4(w[0], w[1], w[2], w[3]);
        c4[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
}

// Chunked weight -> f32 [n][k].  One thread per 8 consecutive elements of a row
// (one Q4_0 code word / two Q8_0 code words); stores are 2 x float4, contiguous
// across the wave.
template <bool kQ4>
__global__ __launch_bounds__(256) void dequant_weight_kernel(const uint8_t* __restrict__ chunks,
                                                             int64_t nwords, int64_t nb,
                                                             int64_t groups, float* __restrict__ out) {
    constexpr int kCB = kQ4 ? 16 : 32;
    constexpr int kChunk = chunk_bytes_for(kQ4);
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nwords) return;
    const int64_t row = g / (nb * 4);
    const int64_t rem = g - row * nb * 4;
    const int64_t blk = rem >> 2;
    const uint8_t* chunk = chunks + chunk_of(row, blk, groups) * kChunk;
    const int e = slot_of(row, blk);
    const int j = (int)(rem & 3);
    const float d = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(chunk + kTileEntries * kCB)[e]);
    float v[8];
    if constexpr (kQ4) {
        const uint32_t w = reinterpret_cast<const uint32_t*>(chunk + e * 16)[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // sign-extend the nibble to (q - 8) exactly, then one fp32 multiply, as quant.rs:190
            v[i] = (float)((int)(w << (28 - 8 * i)) >> 28) * d;
            v[4 + i] = (float)((int)(w << (24 - 8 * i)) >> 28) * d;
        }
    } else {
        const uint2 w = reinterpret_cast<const uint2*>(chunk + e * 32)[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = (float)(int8_t)(w.x >> (8 * i)) * d;
            v[4 + i] = (float)(int8_t)(w.y >> (8 * i)) * d;
        }
    }
    float4* o = reinterpret_cast<float4*>(out) + 2 * g;
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// Raw GGUF blocks -> f32[n] (GpuQuantOps path).  One thread per 8-element group
// of a block; byte loads because 18/34-byte blocks are only byte aligned in
// general.  Elements >= n are not written (quant.rs:175-177).
template <int kBPB>
__global__ __launch_bounds__(256) void dequant_gguf_kernel(const uint8_t* __restrict__ gguf,
                                                           size_t n, float* __restrict__ out) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = g >> 2;
    const int grp = (int)(g & 3);
    const int64_t e0 = blk * kQK + grp * 8;
    if (e0 >= (int64_t)n) return;
    const uint8_t* b = gguf + blk * kBPB;
    const float d = f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    const uint8_t* qs = b + 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int e = grp * 8 + i;
        float v;
        if constexpr (kBPB == 18) {
            const int q = (int)q4_code(qs, e) - 8;
            v = (float)q * d;
        } else {
            v = (float)(int8_t)qs[e] * d;
        }
        if (e0 + i < (int64_t)n) out[e0 + i] = v;
    }
}

__global__ __launch_bounds__(256) void stream_copy_kernel(const uint4* __restrict__ src,
                                                          uint4* __restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

inline unsigned grid_for(int64_t items, int per_block) {
    return (unsigned)((items + per_block - 1) / per_block);
}

}  // namespace

hipError_t launch_repack(const Weight& w, const uint8_t* gguf, hipStream_t s) {
    const int64_t nblocks = w.n * w.nb;
    if (nblocks <= 0) return hipSuccess;
    const int aligned = ((uintptr_t)gguf % 16) == 0;
    const dim3 grid(grid_for(nblocks, kTile));
    if (w.type == OPENMINI_QMM_Q4_0)
        hipLaunchKernelGGL(repack_kernel<18>, grid, dim3(kTile), 0, s, gguf, nblocks, w.nb,
                           w.groups, aligned, w.chunks);
    else
        hipLaunchKernelGGL(repack_kernel<34>, grid, dim3(kTile), 0, s, gguf, nblocks, w.nb,
                           w.groups, aligned, w.chunks);
    return hipGetLastError();
}

hipError_t launch_dequant_weight(const Weight& w, float* out, hipStream_t s) {
    const int64_t nwords = w.n * w.nb * 4;
    if (nwords == 0) return hipSuccess;
    const dim3 grid(grid_for(nwords, 256));
    if (w.type == OPENMINI_QMM_Q4_0)
        hipLaunchKernelGGL(dequant_weight_kernel<true>, grid, dim3(256), 0, s, w.chunks, nwords,
                           w.nb, w.groups, out);
    else
        hipLaunchKernelGGL(dequant_weight_kernel<false>, grid, dim3(256), 0, s, w.chunks, nwords,
                           w.nb, w.groups, out);
    return hipGetLastError();
}

hipError_t launch_dequant_gguf(int type, const uint8_t* gguf, size_t n_elems, float* out,
                               hipStream_t s) {
    if (n_elems == 0) return hipSuccess;
    const int64_t nblocks = (int64_t)((n_elems + kQK - 1) / kQK);
    const dim3 grid(grid_for(nblocks * 4, 256));
    if (type == OPENMINI_QMM_Q4_0)
        hipLaunchKernelGGL(dequant_gguf_kernel<18>, grid, dim3(256), 0, s, gguf, n_elems, out);
    else
        hipLaunchKernelGGL(dequant_gguf_kernel<34>, grid, dim3(256), 0, s, gguf, n_elems, out);
    return hipGetLastError();
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

}  // namespace qmm
