// Internal declarations shared by the C-ABI (qmm_api.hip) and the kernels.
//
// GPU weight layout ("repacked", produced by the upload kernels in qmm_repack.hip)
// -------------------------------------------------------------------------------
// A GGUF Q4_0 / Q8_0 tensor W[N, K] arrives as N*nb blocks (nb = K/32), row-major,
// each block = fp16 scale d followed by the codes (16 B of nibbles / 32 int8).
// The 18- and 34-byte blocks are not 16-byte aligned, so the upload splits them
// into two streams, both row-major [N][nb]:
//
//   codes : Q4_0 16 B per block, Q8_0 32 B per block (16-byte aligned rows)
//   scales: fp16 bits, 2 B per block
//
// HBM bytes = GGUF bytes (no padding).  Q8_0 codes keep GGUF order.  Q4_0 codes
// are permuted inside the block so a 32-bit word holds 8 consecutive elements:
//   word j (0..3), byte i (0..3): low nibble  = element 8j + i
//                                 high nibble = element 8j + 4 + i
// and each nibble holds q ^ 8, so its two's-complement reading is q - 8 (the
// Q4_0 value before scaling).  v_cvt_off_f32_i4 then turns a nibble into
// (q - 8) / 16 in one instruction, with SDWA byte selects.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/openmini_qmm.h"

namespace qmm {

constexpr int kQK = 32;

// IEEE binary16 bits -> binary32 (exact; v_cvt_f32_f16).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

inline int bytes_per_block(int type) {
    return type == OPENMINI_QMM_Q4_0 ? 18 : type == OPENMINI_QMM_Q8_0 ? 34 : 0;
}
inline int code_bytes_per_block(int type) {
    return type == OPENMINI_QMM_Q4_0 ? 16 : type == OPENMINI_QMM_Q8_0 ? 32 : 0;
}

struct Weight {
    int type = 0;
    int device = 0;
    int64_t n = 0;   // rows
    int64_t k = 0;   // columns
    int64_t nb = 0;  // blocks per row
    void* base = nullptr;        // single allocation: codes, then scales
    uint8_t* codes = nullptr;    // [n][nb][code_bytes]
    uint16_t* scales = nullptr;  // [n][nb]
    size_t device_bytes = 0;
};

// ---- kernel launchers (qmm_repack.hip, qmm_gemv.hip, qmm_gemm.hip) ----------------

// GGUF blocks (device) -> repacked codes + scales.  nblocks = n * nb.
hipError_t launch_repack(int type, const uint8_t* gguf, int64_t nblocks, uint8_t* codes,
                         uint16_t* scales, hipStream_t s);

// Repacked weight -> f32 [n][k].
hipError_t launch_dequant_weight(const Weight& w, float* out, hipStream_t s);

// Raw GGUF bytes -> f32 [n_elems] (reads only complete blocks; caller validated size).
hipError_t launch_dequant_gguf(int type, const uint8_t* gguf, size_t n_elems, float* out,
                               hipStream_t s);

// y[batch][n] = x[batch][k] . W^T for 1 <= batch <= 8.
hipError_t launch_gemv(const Weight& w, const float* x, float* y, int batch, hipStream_t s);

// y[m][n] = x_bf16[m][k] . W^T.
hipError_t launch_gemm_bf16(const Weight& w, const uint16_t* x, float* y, int64_t m,
                            hipStream_t s);

hipError_t launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s);

}  // namespace qmm
