// Decode GEMV: y[b, n] = sum_k x[b, k] * w[n, k] for 1..4 fp32 activation rows.
//
// Replaces, per call of linear()/linear_gemm() (openmini-server/src/model/inference/
// model.rs:1050-1064), the W^T copy plus f32 sgemm over weights dequantized at load.
// Here W stays quantized in HBM (0.5625 B/weight Q4_0, 1.0625 B/weight Q8_0), is read
// exactly once and streams from HBM; the kernel is HBM-bound.
//
// Arithmetic: exact integer dot products on the matrix cores.
//   * Per 32-element block, x is made block-floating: with M the block's max |x| and
//     2^(e-1) <= M < 2^e, X_k = round-to-nearest-even(x_k * 2^s), s = 22 - e, so
//     |X_k| <= 2^22 and the error is <= 2^(e-23) (fp32-level relative to the block max).
//     The rounding is one fp32 add of 1.5 * 2^23: the sum lies in [2^23, 2^24], where
//     the fp32 spacing is 1, and its bit pattern is 0x4B400000 + X_k.
//   * X_k = a*2^16 + b*2^8 + c with a, b, c balanced int8 digits; they are the low
//     three bytes of (X + 0x808080) ^ 0x808080.
//   * v_mfma_i32_16x16x64_i8 forms sum_k q_k * digit_k exactly in int32.  Q4_0 codes
//     enter as unsigned bytes (w & 0x0F0F0F0F, (w >> 4) & 0x0F0F0F0F: 3 VALU ops per
//     8 weights), Q8_0 codes as they are.
//   * Per block: sum_k (q_k - 8) x_k = 2^-s * (D_c + 2^8 D_b + 2^16 D_a - 8 sum_k X_k)
//     (the -8 term for Q4_0 only; for Q4_0 the bracket is formed exactly in int32),
//     times the block's fp16 scale, accumulated in fp32.
// Versus unpack + convert + FMA on the VALU (about 2.3 instructions per weight, most
// of the VALU budget at HBM speed), this is about 1 per weight.
//
// MFMA mapping (A 16x64 activation digits, B 64x16 codes, D 16x16): the 64 k
// positions are four 16-element parts; part t is block slot t of a 4-block group.
// Lane l = 16t + n feeds row n's block-t codes -- exactly the tiled-layout entry
// l of the group's tile, so a wave-wide load of a tile is one contiguous 1 KB
// (Q4_0) / 2 KB (Q8_0).  A row 4t + h holds digit h of block t (other rows and
// parts zero), so D[4t + h][n] is digit h's block-t dot product for row n, in lane
// (n, t), register h.  Two MFMAs cover a block's 32 elements.  A group's digits are
// computed once per batch row (two elements per lane; block max and sum by DPP
// butterflies within the 16-lane row that holds the block), passed through LDS
// into A fragments, and reused by all RT row tiles of the wave.
//
// Work split: a workgroup owns RT row tiles (16 rows each) and its W waves split
// the K groups into contiguous slices, each a contiguous run of the weight.  Each
// wave keeps two stages of GS groups of loads in flight.  The W partial sums of a
// row meet in LDS and are added in wave order (deterministic).
#include "qmm_internal.hpp"

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

// Butterflies over the 16 lanes of a row (every lane ends with the row result); each
// step compiles to one DPP-modified integer op.  The max runs on the bit patterns of
// non-negative floats, which order like unsigned integers.
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
    v = max(v, dpp<kDppXor1>(v));
    v = max(v, dpp<kDppXor2>(v));
    v = max(v, dpp<kDppHalfMirror>(v));
    v = max(v, dpp<kDppMirror>(v));
    return v;
}
__device__ __forceinline__ uint32_t row16_sum(uint32_t v) {  // wrapping
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return v;
}

// Raw buffer resource (gfx9 descriptor): out-of-range loads return zero, offsets are
// 32-bit with the uniform part in an SGPR.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Loads of one K group for one wave: the lane's tile entry of each row tile, its
// scale, and two activation elements per batch row.
template <bool kQ4, int B, int RT>
struct GroupLoads {
    uint4 c[RT][kQ4 ? 1 : 2];
    uint32_t sc[RT];
    float2 xv[B];
};

template <bool kQ4, int B, int RT, int W, int GS>
__global__ __launch_bounds__(64 * W) void gemv_kernel(const uint8_t* __restrict__ codes,
                                                      const uint16_t* __restrict__ scales,
                                                      const float* __restrict__ x,
                                                      float* __restrict__ y, int n_rows, int n_tiles,
                                                      int groups, int k) {
    constexpr int kCB = kQ4 ? 16 : 32;
    // A-fragment staging per wave: [b][u = block half][t = block slot][h = digit] plus
    // one zero slot read by lanes whose A fragment is zero.
    constexpr int kSlots = B * 2 * 4 * 4 + 1;
    __shared__ uint4 a_lds[W][kSlots];
    __shared__ float red[W][RT][B][16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform per wave
    const int ln = lane & 15, lt = lane >> 4;
    const int tile0 = blockIdx.x * RT;
    const int g0 = (int)((int64_t)groups * wave / W);
    const int g1 = (int)((int64_t)groups * (wave + 1) / W);

    // Weight bytes are < 4 GiB (checked at upload), so 32-bit buffer offsets suffice.
    const uint32_t tile_bytes = (uint32_t)kTileEntries * kCB;
    const __amdgpu_buffer_rsrc_t c_rs = make_rsrc(codes, (uint32_t)n_tiles * groups * tile_bytes);
    const __amdgpu_buffer_rsrc_t s_rs = make_rsrc(scales, (uint32_t)n_tiles * groups * kTileEntries * 2);
    __amdgpu_buffer_rsrc_t x_rs[B];
#pragma unroll
    for (int b = 0; b < B; ++b) x_rs[b] = make_rsrc(x + (size_t)b * k, (uint32_t)k * 4);
    uint32_t tile_off[RT];  // byte offset of (row tile, group 0) in the codes
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) tile_off[rt] = (uint32_t)min(tile0 + rt, n_tiles - 1) * groups * tile_bytes;

    uint4* my_lds = a_lds[wave];
    if (lane == 0) my_lds[kSlots - 1] = make_uint4(0, 0, 0, 0);
    // This lane's A fragment: row m = ln = 4*at + ah of part lt, live iff at == lt, ah < 3.
    const int ah = ln & 3, at = ln >> 2;
    const bool a_live = (at == lt) && (ah < 3);
    // Where this lane writes its two elements' digits: slot (u = ln / 8, t = lt, h),
    // byte 2*(ln % 8); a slot is 8 halfwords.
    uint16_t* wr16 = reinterpret_cast<uint16_t*>(my_lds) + ((ln >> 3) * 4 + lt) * 4 * 8 + (ln & 7);

    auto load_group = [&](GroupLoads<kQ4, B, RT>& L, int g) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint32_t soff = tile_off[rt] + (uint32_t)g * tile_bytes;
            L.c[rt][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(c_rs, lane * kCB, soff, 0));
            if constexpr (!kQ4)
                L.c[rt][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(c_rs, lane * kCB + 16, soff, 0));
            L.sc[rt] = __builtin_amdgcn_raw_buffer_load_b16(s_rs, lane * 2, soff / (kCB / 2), 0);
        }
#pragma unroll
        for (int b = 0; b < B; ++b)
            L.xv[b] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(x_rs[b], lane * 8, (uint32_t)g * 512, 0));
    };

    float acc[RT][B];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[rt][b] = 0.0f;
    // Max of the rounded activations' bit patterns t = 1.5 * 2^23 + X.  Finite x gives
    // t in [2^23, 2^24] (bits <= 0x4B800000); a NaN or +-inf x makes t NaN or +-inf,
    // whose bits lie above.
    uint32_t seen = 0;

    auto process = [&](const GroupLoads<kQ4, B, RT>& L) {
        i32x4 afr[B][2];
        int shift[B], sxn8[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float x0 = L.xv[b].x, x1 = L.xv[b].y;
            const uint32_t mb = row16_max(__float_as_uint(fmaxf(fabsf(x0), fabsf(x1))));
            // 2^(e-1) <= max < 2^e with e = biased exponent - 126; s = 22 - e
            shift[b] = 148 - (int)(mb >> 23);
            // t = 1.5 * 2^23 + round(x * 2^s): bits(t) = 0x4B400000 + X (|X| <= 2^22)
            const uint32_t t0 = __float_as_uint(__builtin_amdgcn_ldexpf(x0, shift[b]) + 12582912.0f);
            const uint32_t t1 = __float_as_uint(__builtin_amdgcn_ldexpf(x1, shift[b]) + 12582912.0f);
            seen = max(seen, max(t0, t1));
            if constexpr (kQ4) {
                // -8 * sum X over the block, in wrapping uint32 (the true value fits int32)
                const uint32_t sum_t = row16_sum(t0 + t1);
                sxn8[b] = (int)(0u - 8u * (sum_t - 32u * 0x4B400000u));
            } else {
                sxn8[b] = 0;
            }
            // low three bytes of (X + 0x808080) ^ 0x808080: digits c, b, a
            const uint32_t z0 = (t0 + (0x808080u - 0x4B400000u)) ^ 0x808080u;
            const uint32_t z1 = (t1 + (0x808080u - 0x4B400000u)) ^ 0x808080u;
            uint16_t* w16 = wr16 + b * 2 * 4 * 4 * 8;
#pragma unroll
            for (int h = 0; h < 3; ++h)
                w16[h * 8] = (uint16_t)__builtin_amdgcn_perm(z1, z0, (uint32_t)(h | ((4 + h) << 8) | 0x0C0C0000u));
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint4 v = my_lds[a_live ? ((b * 2 + u) * 4 + lt) * 4 + ah : kSlots - 1];
                afr[b][u] = i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            i32x4 b0, b1;
            if constexpr (kQ4) {
                const uint4 w = L.c[rt][0];
                b0 = i32x4{(int)(w.x & 0x0F0F0F0Fu), (int)((w.x >> 4) & 0x0F0F0F0Fu),
                           (int)(w.y & 0x0F0F0F0Fu), (int)((w.y >> 4) & 0x0F0F0F0Fu)};
                b1 = i32x4{(int)(w.z & 0x0F0F0F0Fu), (int)((w.z >> 4) & 0x0F0F0F0Fu),
                           (int)(w.w & 0x0F0F0F0Fu), (int)((w.w >> 4) & 0x0F0F0F0Fu)};
            } else {
                const uint4 w0 = L.c[rt][0], w1 = L.c[rt][1];
                b0 = i32x4{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w};
                b1 = i32x4{(int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
            }
            const float d = f16_bits_to_f32((uint16_t)L.sc[rt]);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                // Q4_0: the -8 * sum(X) term enters as the accumulator input of the
                // low digit's row (register 0 of lane (n, t) is D[4t][n])
                i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[b][0], b0, i32x4{sxn8[b], 0, 0, 0}, 0, 0, 0);
                D = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[b][1], b1, D, 0, 0, 0);
                float r;
                if constexpr (kQ4) {
                    // exact: the true value fits int32, so wrap-around in between is harmless
                    const uint32_t lo = ((uint32_t)D[1] << 8) + (uint32_t)D[0];
                    r = (float)(int)(((uint32_t)D[2] << 16) + lo);
                } else {
                    r = fmaf((float)D[2], 65536.0f, fmaf((float)D[1], 256.0f, (float)D[0]));
                }
                acc[rt][b] = fmaf(d, __builtin_amdgcn_ldexpf(r, -shift[b]), acc[rt][b]);
            }
        }
    };

    if (g0 < g1) {
        GroupLoads<kQ4, B, RT> s0[GS], s1[GS];
#pragma unroll
        for (int i = 0; i < GS; ++i)
            if (g0 + i < g1) load_group(s0[i], g0 + i);
        int g = g0;
        while (true) {
#pragma unroll
            for (int i = 0; i < GS; ++i)
                if (g + GS + i < g1) load_group(s1[i], g + GS + i);
#pragma unroll
            for (int i = 0; i < GS; ++i)
                if (g + i < g1) process(s0[i]);
            g += GS;
            if (g >= g1) break;
#pragma unroll
            for (int i = 0; i < GS; ++i)
                if (g + GS + i < g1) load_group(s0[i], g + GS + i);
#pragma unroll
            for (int i = 0; i < GS; ++i)
                if (g + i < g1) process(s1[i]);
            g += GS;
            if (g >= g1) break;
        }
    }

    // Sum the four block slots (lanes n, n+16, n+32, n+48), then the W K slices.
    // Any inf / NaN activation turns the outputs into NaN.
    const bool bad = __builtin_amdgcn_read_exec() && __ballot(seen > 0x4B800000u) != 0;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float v = acc[rt][b];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (bad) v = __builtin_nanf("");
            if (lane < 16) red[wave][rt][b][lane] = v;
        }
    __syncthreads();
    if (wave == 0 && lane < 16) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int row = (tile0 + rt) * kTileRows + lane;
            if (row >= n_rows) continue;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float v = red[0][rt][b][lane];
#pragma unroll
                for (int w = 1; w < W; ++w) v += red[w][rt][b][lane];
                y[(size_t)b * n_rows + row] = v;
            }
        }
    }
}

#ifndef QMM_GEMV_RT
#define QMM_GEMV_RT 1
#endif
#ifndef QMM_GEMV_GS
#define QMM_GEMV_GS 2
#endif

template <bool kQ4, int B, int RT, int W>
hipError_t run(const Weight& w, const float* x, float* y, hipStream_t s) {
    const dim3 grid((unsigned)((w.n_tiles + RT - 1) / RT));
    hipLaunchKernelGGL((gemv_kernel<kQ4, B, RT, W, QMM_GEMV_GS>), grid, dim3(64 * W), 0, s, w.codes,
                       w.scales, x, y, (int)w.n, (int)w.n_tiles, (int)w.groups, (int)w.k);
    return hipGetLastError();
}

// K slices per row tile: about four or more groups per wave, at most 8 waves.
template <bool kQ4, int B>
hipError_t run_w(const Weight& w, const float* x, float* y, hipStream_t s) {
    constexpr int RT = QMM_GEMV_RT;
    if (w.groups >= 32) return run<kQ4, B, RT, 8>(w, x, y, s);
    if (w.groups >= 16) return run<kQ4, B, RT, 4>(w, x, y, s);
    if (w.groups >= 8) return run<kQ4, B, RT, 2>(w, x, y, s);
    return run<kQ4, B, RT, 1>(w, x, y, s);
}

template <bool kQ4>
hipError_t dispatch(const Weight& w, const float* x, float* y, int batch, hipStream_t s) {
    switch (batch) {
    case 1: return run_w<kQ4, 1>(w, x, y, s);
    case 2: return run_w<kQ4, 2>(w, x, y, s);
    case 3: return run_w<kQ4, 3>(w, x, y, s);
    case 4: return run_w<kQ4, 4>(w, x, y, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemv(const Weight& w, const float* x, float* y, int batch, hipStream_t s) {
    if (w.type == OPENMINI_QMM_Q4_0) return dispatch<true>(w, x, y, batch, s);
    return dispatch<false>(w, x, y, batch, s);
}

}  // namespace qmm
