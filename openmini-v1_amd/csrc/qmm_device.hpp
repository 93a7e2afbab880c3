// Device helpers shared by the kernels (gfx950).
#pragma once

#include "qmm_internal.hpp"

namespace qmm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource (gfx9 descriptor): out-of-range loads return zero, offsets are
// 32-bit with the uniform part in an SGPR.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt immediate (gfx9) that waits for vmcnt <= n only.
constexpr int vmcnt_only(int n) { return (n & 0xF) | ((n >> 4) << 14) | 0x0F70; }

// Two code bytes (selector bytes a, b of `u`) -> the fp16 pair (1024 + u_a, 1024 + u_b).
__device__ __forceinline__ uint32_t magic_pair(uint32_t u, uint32_t sel) {
    return __builtin_amdgcn_perm(0x64646464u, u, sel);
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;

__device__ __forceinline__ uint32_t pk_sub(uint32_t v, _Float16 c) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, v) - f16x2{c, c});
}

// Q4_0 code word (elements 8 kq + i in the low nibble of byte i, 8 kq + 4 + i in the
// high nibble; nibble = (q - 8) mod 16) -> 8 fp16 q - 8, elements in order: the 1024 + u
// pattern (0x64XX is the fp16 1024 + XX, spacing 1) and one packed fp16 subtraction.
__device__ __forceinline__ f16x8 codes_q4(uint32_t w) {
    const uint32_t u = w ^ 0x88888888u;  // nibbles q
    const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
    uint32_t p[4] = {pk_sub(magic_pair(lo, kSel01), (_Float16)1032.0f), pk_sub(magic_pair(lo, kSel23), (_Float16)1032.0f),
                     pk_sub(magic_pair(hi, kSel01), (_Float16)1032.0f), pk_sub(magic_pair(hi, kSel23), (_Float16)1032.0f)};
    return __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(p));
}

// The same 8 codes in the element order (0, 2, 1, 3, 4, 6, 5, 7), one operation fewer
// per pair: nibble positions 0 / 4 (elements 0, 2) and 2 / 6 (1, 3) become the fp16
// 1024 + (n ^ 8) = 1024 + q by one bit-field select each (magic bits from both
// constants, bit 3 of the nibble inverted, bits 0-2 kept); positions 1 / 5 (4, 6) and
// 3 / 7 (5, 7) likewise as 1024 + 16 q, scaled by 1/16 in the packed fma that removes
// the offset (exact: 64 + q - 72).  A caller feeds the activations in the same order.
__device__ __forceinline__ f16x8 codes_q4_perm(uint32_t w) {
    constexpr uint32_t kC0 = 0x64076407u, kB0 = 0x64086408u;  // low nibbles of each half
    constexpr uint32_t kC1 = 0x64706470u, kB1 = 0x64806480u;  // high nibbles of each half
    const uint32_t w8 = w >> 8;
    const uint32_t h0 = (w & kC0) | (~w & kB0), h1 = (w8 & kC0) | (~w8 & kB0);
    const uint32_t h2 = (w & kC1) | (~w & kB1), h3 = (w8 & kC1) | (~w8 & kB1);
    const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f}, c72 = {(_Float16)-72.0f, (_Float16)-72.0f};
    const f16x2 v2 = __builtin_bit_cast(f16x2, h2) * s16 + c72, v3 = __builtin_bit_cast(f16x2, h3) * s16 + c72;
    uint32_t p[4] = {pk_sub(h0, (_Float16)1032.0f), pk_sub(h1, (_Float16)1032.0f), __builtin_bit_cast(uint32_t, v2),
                     __builtin_bit_cast(uint32_t, v3)};
    return __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(p));
}

// Bits 0..3 of v (v < 16) to bit 0 of bytes 0..3.
__device__ __forceinline__ uint32_t spread4(uint32_t v) { return (v * 0x00204081u) & 0x01010101u; }

// 8 Q8_0 codes (two words, int8) -> 8 fp16 q.
__device__ __forceinline__ f16x8 codes_q8(uint32_t w0, uint32_t w1) {
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;  // q + 128
    uint32_t p[4] = {pk_sub(magic_pair(u0, kSel01), (_Float16)1152.0f), pk_sub(magic_pair(u0, kSel23), (_Float16)1152.0f),
                     pk_sub(magic_pair(u1, kSel01), (_Float16)1152.0f), pk_sub(magic_pair(u1, kSel23), (_Float16)1152.0f)};
    return __builtin_bit_cast(f16x8, *reinterpret_cast<uint4*>(p));
}

}  // namespace qmm
