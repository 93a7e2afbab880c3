// Internal declarations shared by the C-ABI (qmm_api.hip) and the kernels.
//
// GPU weight layout ("tiled", produced by the upload kernels in qmm_repack.hip)
// -------------------------------------------------------------------------------
// A GGUF Q4_0 / Q8_0 tensor W[N, K] arrives as N*nb blocks (nb = K/32), row-major,
// each block = fp16 scale d followed by the codes (16 B of nibbles / 32 int8).
// The upload splits codes from scales and regroups both into tiles of 16 rows x
// 4 consecutive blocks (a "group" of 128 elements):
//
//   entry(row, blk) = ((row/16 * G + blk/4) * 64) + (blk%4) * 16 + row%16,  G = ceil(nb/4)
//   codes : entry * 16 B (Q4_0) or * 32 B (Q8_0)      -> a tile is 1 KB / 2 KB, contiguous
//   scales: entry * 2 B (fp16 bits)                   -> a tile is 128 B
//
// Tiles follow each other along K, so the weight slice a wavefront sweeps is one
// contiguous run of memory, and lane l of a wavefront reading a tile gets entry
// l = (block slot t = l/16, row n = l%16): exactly the B-operand lane of a 16-wide
// MFMA.  Rows are padded to a multiple of 16 and blocks to a multiple of 4 with
// zero codes and zero scales; HBM bytes equal the GGUF bytes when N % 16 == 0 and
// nb % 4 == 0 (all the Llama shapes).
//
// Inside an entry, Q8_0 codes keep GGUF order (int8).  Q4_0 codes (unsigned
// 0..15, value q - 8) are permuted so a 32-bit word holds 8 consecutive elements:
//   word j (0..3), byte i (0..3): low nibble  = element 8j + i
//                                 high nibble = element 8j + 4 + i
// so w & 0x0F0F0F0F and (w >> 4) & 0x0F0F0F0F are elements 8j..8j+3 and
// 8j+4..8j+7 as bytes, in order: ready-made int8 MFMA operands (3 VALU ops per
// 8 weights).  XOR-ing a word with 0x88888888 makes each nibble's two's-complement
// reading q - 8, which v_cvt_off_f32_i4 turns into (q - 8) / 16 in one op.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/openmini_qmm.h"

namespace qmm {

constexpr int kQK = 32;
constexpr int kMaxGemvBatch = 4;  // batch rows per GEMV launch

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

constexpr int kTileRows = 16;   // rows per tile
constexpr int kTileBlocks = 4;  // blocks per tile (one 128-element group)
constexpr int kTileEntries = kTileRows * kTileBlocks;

// Index of (row, blk) in the tiled layout (entries, not bytes).
__host__ __device__ __forceinline__ int64_t tile_entry(int64_t row, int64_t blk, int64_t groups) {
    return (((row >> 4) * groups + (blk >> 2)) << 6) + ((blk & 3) << 4) + (row & 15);
}

struct Weight {
    int type = 0;
    int device = 0;
    int64_t n = 0;        // rows
    int64_t k = 0;        // columns
    int64_t nb = 0;       // blocks per row
    int64_t n_tiles = 0;  // ceil(n / 16)
    int64_t groups = 0;   // ceil(nb / 4)
    void* base = nullptr;        // single allocation: codes, then scales
    uint8_t* codes = nullptr;    // tiled, code_bytes per entry
    uint16_t* scales = nullptr;  // tiled, one fp16 per entry
    size_t device_bytes = 0;
    int64_t entries() const { return n_tiles * groups * kTileEntries; }
};

// ---- kernel launchers (qmm_repack.hip, qmm_gemv.hip, qmm_gemm.hip) ----------------

// GGUF blocks (device, row-major [n][nb]) -> tiled codes + scales of `w` (whose
// padding the caller has zeroed).
hipError_t launch_repack(const Weight& w, const uint8_t* gguf, hipStream_t s);

// Repacked weight -> f32 [n][k].
hipError_t launch_dequant_weight(const Weight& w, float* out, hipStream_t s);

// Raw GGUF bytes -> f32 [n_elems] (reads only complete blocks; caller validated size).
hipError_t launch_dequant_gguf(int type, const uint8_t* gguf, size_t n_elems, float* out,
                               hipStream_t s);

// y[batch][n] = x[batch][k] . W^T for 1 <= batch <= kMaxGemvBatch.
hipError_t launch_gemv(const Weight& w, const float* x, float* y, int batch, hipStream_t s);

// y[m][n] = x_bf16[m][k] . W^T.
hipError_t launch_gemm_bf16(const Weight& w, const uint16_t* x, float* y, int64_t m,
                            hipStream_t s);

hipError_t launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s);

}  // namespace qmm
