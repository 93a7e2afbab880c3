// Internal declarations shared by the C-ABI (qmm_api.hip) and the kernels.
//
// GPU weight layout ("tiled", produced by the upload kernels in qmm_repack.hip)
// -------------------------------------------------------------------------------
// A GGUF Q4_0 / Q8_0 tensor W[N, K] arrives as N*nb blocks (nb = K/32), row-major,
// each block = fp16 scale d followed by the codes (16 B of nibbles / 32 int8).
// The upload regroups the blocks into tiles of 16 rows x 4 consecutive blocks (a
// "group" of 128 elements).  One (row tile, group) pair is a chunk:
//
//   chunk c = (row/16) * G + blk/4,  G = ceil(nb/4),  slot e = (blk%4) * 16 + row%16
//   chunk bytes: [64 x codes: e * 16 B (Q4_0) / e * 32 B (Q8_0)][64 x fp16 scale: e * 2 B]
//   chunk size : 1152 B (Q4_0) / 2176 B (Q8_0), both multiples of 128 B
//
// Chunks follow each other along K, so the weight slice a wavefront sweeps -- codes
// and scales -- is one contiguous run of memory, and lane l of a wavefront reading a
// chunk gets slot l = (block slot t = l/16, row n = l%16): exactly the B-operand lane
// of a 16-wide MFMA.  Rows are padded to a multiple of 16 and blocks to a multiple
// of 4 with zero codes and zero scales; HBM bytes equal the GGUF bytes when
// N % 16 == 0 and nb % 4 == 0 (all the Llama shapes).
//
// Inside a slot, Q8_0 codes keep GGUF order (int8).  Q4_0 codes are stored as the
// 4-bit two's-complement value s = q - 8 (the nibble q ^ 8) and permuted so a
// 32-bit word holds 8 consecutive elements:
//   word j (0..3), byte i (0..3): low nibble  = element 8j + i
//                                 high nibble = element 8j + 4 + i
// so (w << 4) & 0xF0F0F0F0 and w & 0xF0F0F0F0 are 16 * (q - 8) of elements
// 8j..8j+3 and 8j+4..8j+7 as int8 bytes, in order (ready-made int8 MFMA operands),
// and v_cvt_off_f32_i4 turns a nibble into (q - 8) / 16 in one op.
//
// K-quant weights (decode GEMV and prefill GEMM) use the same tiles with 32-element
// sub-blocks as the "blocks" (a 256-element super-block = 8 sub-blocks = 2 groups,
// so K % 256 == 0):
//   Q4_K (144-byte super-blocks, reference reading quant.rs:338-410): element value
//     (q - 8) * d * scale + dmin * 0 (the reference's minimum is always 0); both
//     products are exact, so the value is (q - 8) * (d * scale).  Slot codes as Q4_0
//     (16 B of nibbles q ^ 8); then 64 x u8 scale (scales[sb] & 0x3F); then 16 x fp16 d,
//     one per row of the tile (d becomes NaN when dmin is not finite, as every value
//     of that super-block is then NaN).  1120 B per chunk.
//   Q6_K (210-byte super-blocks, quant.rs:515-600): element value q * d * scale16 with
//     q = low + 16 * high - 32 in [-32, 31] and a signed 8-bit scale per 16 elements,
//     again exact as q * (d * scale16).  Slot codes: 16 B of the low 4 bits of the
//     6-bit two's-complement code v = q & 63, packed as Q4_0's nibbles (word j, byte i:
//     low nibble element 8j + i, high nibble 8j + 4 + i), then 8 B of its top 2 bits
//     (word m, byte i, bits 2f..2f+1: element 16m + 4f + i); then 64 x 2 int8 scales
//     (the slot's two 16-element halves); then 16 x fp16 d.  1696 B per chunk.
//     (w << 2) & 0x3C3C3C3C | (hi << s) & 0xC0C0C0C0 is then 4 q per int8 byte.
//
// Types with a per-block minimum (their matmul adds min * (sum of the block's
// activations) to each block's product):
//   Q4_1 (20-byte blocks, quant.rs:216-262): element value q * d + m, q in [0, 15].
//     Slot codes as Q4_0 (the nibble q ^ 8, i.e. q - 8) and fp16 scales d, then 64 x
//     fp16 m: the value is (q - 8) * d + (8 d + m).  1280 B per chunk.
//   Q5_K (176-byte super-blocks, the reference's reading quant.rs:433-505): element i
//     of sub-block sb has q = (nibble of byte 36 + 16 sb + i / 2, even i high) + 16 *
//     (bit i % 8 of byte 20 + sb) and value (q - 16) * d * (byte 4 + sb & 0x3F) +
//     dmin * (nibble sb % 2 of byte 12 + sb / 2).  In that reading a sub-block's 32
//     high bits are the 8 bits of one byte, each used by 4 elements.  Slot codes: Q6_K's
//     16 B of low nibbles (the nibble of q), then 64 x u8 high-bit bytes (the
//     sub-block's byte 20 + sb as it stands), 64 x u8 scales, 64 x u8 minimum nibbles,
//     16 x fp16 d, 16 x fp16 dmin (per row).  The code term is exact as
//     (q - 16) * (d * scale).  1280 B per chunk (the GGUF bytes: 1408).
#pragma once

#include <hip/hip_runtime.h>

// Device code is written for gfx950 only: its instruction forms (row-swap permutes,
// the gfx950 MFMA shapes, buffer loads to LDS) and the memory-ordering rules the
// batched GEMV's K split relies on (gfx9's store-counting vmcnt, write-through
// agent-scope stores) are those of this part.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "libopenmini_qmm device code targets gfx950 only (--offload-arch=gfx950)"
#endif
#include <stddef.h>
#include <stdint.h>

#include "../../include/openmini_qmm.h"

struct openmini_qweight;

namespace qmm {

constexpr int kQK = 32;
constexpr int kMaxGemvBatch = 4;  // batch rows per launch of the single-row-tuned GEMV
constexpr int kBatchRows = 16;    // batch rows per launch of the batched GEMV (its MFMA rows)
constexpr int kMaxGroup = 4;      // weights sharing one GEMV launch
// linear() on fp32 activations runs the prefill GEMM (split activations, fp16 MFMA)
// from 128 rows on for every weight it takes (gemm_min_rows may choose earlier).
constexpr int64_t kGemmMinRows = 128;
constexpr int64_t kGemmMinRowsLow = 64;  // gemm_min_rows never chooses below this

// IEEE binary16 bits -> binary32 (exact; v_cvt_f32_f16).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// GGUF block geometry of the weight layouts (upload, GEMV; the GEMM takes the types
// without a block minimum): elements and bytes per GGUF block.
inline bool is_kquant(int type) {
    return type == OPENMINI_QMM_Q4_K || type == OPENMINI_QMM_Q5_K || type == OPENMINI_QMM_Q6_K;
}
inline bool has_block_min(int type) { return type == OPENMINI_QMM_Q4_1 || type == OPENMINI_QMM_Q5_K; }
inline int weight_block_elems(int type) { return is_kquant(type) || type == OPENMINI_QMM_Q8_K ? 256 : 32; }
inline int bytes_per_block(int type) {
    switch (type) {
    case OPENMINI_QMM_Q4_0: return 18;
    case OPENMINI_QMM_Q4_1: return 20;
    case OPENMINI_QMM_Q8_0: return 34;
    case OPENMINI_QMM_Q4_K: return 144;
    case OPENMINI_QMM_Q5_K: return 176;
    case OPENMINI_QMM_Q6_K: return 210;
    case OPENMINI_QMM_Q8_K: return 258;
    default: return 0;
    }
}
// The chunk format a weight type is stored and computed in.  The reference reads a
// Q8_K super-block as fp16 d and 256 int8 codes, value q * d (quant.rs:768-800): eight
// Q8_0 blocks that share one d, so Q8_K weights become Q8_0 chunks and run every Q8_0
// kernel with the same values.
inline int chunk_type(int type) { return type == OPENMINI_QMM_Q8_K ? OPENMINI_QMM_Q8_0 : type; }

// The fewest activation rows from which linear() takes the fp32 GEMM on a weight of
// n_rows x k_cols: the first m in [64, 128) where the GEMM's estimated time beats the
// decode GEMVs', else 128.  Estimates (MI355X, graph replay): the GEMM on a grid of at
// most one round takes about 10 ns per K element (its workgroups walk K serially:
// K = 3072 / 4096 / 8192 / 11008 / 13824 -> 31 / 39-46 / 82-90 / 110 / 137 us at
// 64-128 rows), a round being 512 workgroups of 64 x 64; the batched GEMV runs one
// pass per 16 rows of about 6.5 us plus the weight bytes at 5 TB/s (Q8_0 chunks) or
// 3 TB/s (the others).  Over 18 weight shapes x 48-112 rows (Q4_0 / Q8_0 / Q4_K /
// Q6_K, 1024-28672 rows, K 3072-13824) the choice loses at most 9% against the faster
// path (Q4_0 2048 x 4096 at 80 rows), a fixed 128 up to 85% (3072 x 3072 at 112 rows:
// GEMV 60.0 vs GEMM 32.4 us).
inline int64_t gemm_min_rows(int type, int64_t n_rows, int64_t k_cols) {
    const double w_bytes = (double)n_rows * (double)k_cols * bytes_per_block(type) / weight_block_elems(type);
    const double pass_us = 6.5 + w_bytes / (type == OPENMINI_QMM_Q8_0 ? 5.0e6 : 3.0e6);
    for (int64_t m = kGemmMinRowsLow; m < kGemmMinRows; ++m) {
        const int64_t wgs = (n_rows + 63) / 64 * ((m + 63) / 64);
        const double gemm_us = 0.010 * (double)k_cols * (double)((wgs + 511) / 512);
        if (gemm_us < (double)((m + 15) / 16) * pass_us) return m;
    }
    return kGemmMinRows;
}

// GgufTensorType::{block_size, bytes_per_block} (src/model/inference/gguf.rs:348-379)
// for the layouts the dequantization entry points accept; 0 for others.
inline int layout_block_size(int type) {
    switch (type) {
    case OPENMINI_QMM_F32: case OPENMINI_QMM_F16: return 1;
    case OPENMINI_QMM_Q4_0: case OPENMINI_QMM_Q4_1: case OPENMINI_QMM_Q8_0: return 32;
    case OPENMINI_QMM_Q2_K: case OPENMINI_QMM_Q3_K: case OPENMINI_QMM_Q4_K: case OPENMINI_QMM_Q5_K:
    case OPENMINI_QMM_Q6_K: case OPENMINI_QMM_Q8_K: return 256;
    default: return 0;
    }
}
inline int layout_bytes_per_block(int type) {
    switch (type) {
    case OPENMINI_QMM_F32: return 4;
    case OPENMINI_QMM_F16: return 2;
    case OPENMINI_QMM_Q4_0: return 18;
    case OPENMINI_QMM_Q4_1: return 20;
    case OPENMINI_QMM_Q8_0: return 34;
    case OPENMINI_QMM_Q2_K: return 68;
    case OPENMINI_QMM_Q3_K: return 162;
    case OPENMINI_QMM_Q4_K: return 144;
    case OPENMINI_QMM_Q5_K: return 176;
    case OPENMINI_QMM_Q6_K: return 210;
    case OPENMINI_QMM_Q8_K: return 258;
    default: return 0;
    }
}
constexpr int kTileRows = 16;   // rows per tile
constexpr int kTileBlocks = 4;  // blocks per group
constexpr int kTileEntries = kTileRows * kTileBlocks;  // slots per chunk

// Bytes of one chunk: 64 slots of codes, then their 64 fp16 scales.
__host__ __device__ constexpr int chunk_bytes_for(bool q4) { return kTileEntries * (q4 ? 16 : 32) + 2 * kTileEntries; }
// K-quant chunks: codes, per-slot scale bytes, then one fp16 d per tile row.
constexpr int kQ4KChunk = kTileEntries * 16 + kTileEntries + 2 * kTileRows;       // 1120
constexpr int kQ6KChunk = kTileEntries * 24 + 2 * kTileEntries + 2 * kTileRows;   // 1696
// Block-minimum chunks: Q4_1 = a Q4_0 chunk + 64 fp16 m; Q5_K: low nibbles, then
// per-slot high-bit byte, scale and minimum, then per-row d and dmin.
constexpr int kQ41MinOff = kTileEntries * 16 + 2 * kTileEntries;                    // 1152
constexpr int kQ41Chunk = kQ41MinOff + 2 * kTileEntries;                            // 1280
constexpr int kQ5KQhOff = kTileEntries * 16;                                        // 1024
constexpr int kQ5KScaleOff = kQ5KQhOff + kTileEntries;                              // 1088
constexpr int kQ5KMinOff = kQ5KScaleOff + kTileEntries;                             // 1152
constexpr int kQ5KDOff = kQ5KMinOff + kTileEntries;                                 // 1216
constexpr int kQ5KDminOff = kQ5KDOff + 2 * kTileRows;                               // 1248
constexpr int kQ5KChunk = kQ5KDminOff + 2 * kTileRows;                              // 1280
inline int chunk_bytes(int type) {
    switch (type) {
    case OPENMINI_QMM_Q4_K: return kQ4KChunk;
    case OPENMINI_QMM_Q6_K: return kQ6KChunk;
    case OPENMINI_QMM_Q5_K: return kQ5KChunk;
    case OPENMINI_QMM_Q4_1: return kQ41Chunk;
    default: return chunk_bytes_for(type == OPENMINI_QMM_Q4_0);
    }
}

// Chunk index and slot of (row, blk).
__host__ __device__ __forceinline__ int64_t chunk_of(int64_t row, int64_t blk, int64_t groups) {
    return (row >> 4) * groups + (blk >> 2);
}
__host__ __device__ __forceinline__ int slot_of(int64_t row, int64_t blk) {
    return (int)(((blk & 3) << 4) + (row & 15));
}

struct Weight {
    int type = 0;      // chunk format (chunk_type of src_type): what the kernels dispatch on
    int src_type = 0;  // the GGUF block type uploaded
    int device = 0;
    int64_t n = 0;        // rows
    int64_t k = 0;        // columns
    int64_t nb = 0;       // blocks per row
    int64_t n_tiles = 0;  // ceil(n / 16)
    int64_t groups = 0;   // ceil(nb / 4)
    uint8_t* chunks = nullptr;  // n_tiles * groups chunks, tile-major
    size_t chunk_bytes = 0;
    size_t device_bytes = 0;
    // Batched-GEMV K split (split_s > 1, see batch_split): after the chunks, in the
    // same allocation, split_s x kBatchRows x (n_tiles * 16) fp32 partial sums and one
    // arrival counter per workgroup tile group (a multiple of split_s between calls).
    int split_t = 1, split_s = 1;
    float* split_part = nullptr;
    uint32_t* split_cnt = nullptr;
    int64_t n_chunks() const { return n_tiles * groups; }
};

// ---- kernel launchers (qmm_repack.hip, qmm_gemv.hip, qmm_gemm.hip) ----------------

// GGUF blocks (device, row-major [n][nb]) -> the chunks of `w`, every byte written
// (the tile padding as zeros); clears the split counters of a weight that has them.
hipError_t launch_repack(const Weight& w, const uint8_t* gguf, hipStream_t s);

// Repacked weight -> f32 [n][k].
hipError_t launch_dequant_weight(const Weight& w, float* out, hipStream_t s);

// y[batch][n] = x[batch][k] . W^T for 1 <= batch <= kMaxGemvBatch.
hipError_t launch_gemv(const Weight& w, const float* x, float* y, int batch, hipStream_t s);

// One launch for `count` weights of equal type and K sharing x: ys[i][batch][n_i] =
// x . W_i^T (count <= kMaxGroup); or, with swiglu, a (gate, up) pair of equal shape and
// ys[0][batch][n] = silu(x . Wg^T) * (x . Wu^T).
hipError_t launch_gemv_group(const Weight* const* ws, float* const* ys, int count, const float* x, int batch,
                             bool swiglu, hipStream_t s);

// Batches of at least kBatchMin rows use the batched GEMV (qmm_gemv_batch.hip): from
// four rows on, one pass over W beats the single-row kernel (MI355X, b = 4: Q4_0
// 11008 x 4096 11.6 vs 14.0 us, 28672 x 8192 40 vs 50 us, Q8_0 4096 x 11008 16.0-16.9 vs
// 18.7 us; b = 3 is even and b = 2 favours the single-row kernel, 8.5 vs 11.0 us).
constexpr int kBatchMin = 4;
bool use_batch_kernel(const Weight& w, int64_t batch);

// y[batch][n] = x[batch][k] . W^T for any batch >= 1 (with `up`: the SwiGLU pair as in
// launch_gemv_batch), split into launches of the kernel that suits the batch.
hipError_t launch_gemv_rows(const Weight& w, const Weight* up, const float* x, float* y, int64_t batch,
                            hipStream_t s);

// Batched GEMV (qmm_gemv_batch.hip): T row tiles per workgroup, W waves splitting K.
struct BatchShape {
    int t = 1, w = 8;
    int rep = 1;    // lanes per activation row: 1, 2 or 4 (batches of at most 16 / rep rows)
    int split = 1;  // workgroups per tile group, each over 1 / split of K (one weight only)
};
BatchShape choose_batch_shape(const Weight& w, int batch, bool pair);

// Tiles per workgroup (*t) and K splits (*s) of the batched kernel on one weight of
// n_tiles row tiles and `groups` K groups; a weight with *s > 1 carries the split
// workspace (Weight::split_part / split_cnt).
void batch_split(int type, int64_t n_tiles, int64_t groups, int* t, int* s);
// Bytes of that workspace (0 when s == 1).
size_t split_workspace_bytes(int64_t n_tiles, int t, int s);

// y[batch][n] = x[batch][k] . W^T for 1 <= batch <= kBatchRows in one pass over W; with
// `up`, a (gate = w, up) pair of equal shape and y = silu(x . Wg^T) * (x . Wu^T).
hipError_t launch_gemv_batch(const Weight& w, const Weight* up, const float* x, float* y, int batch,
                             const BatchShape& sh, hipStream_t s);

// y[m][n] = x_bf16[m][k] . W^T.
// gate_in_y: y holds gate = x . Wg^T on entry; each element becomes silu(gate) * (x . W^T).
hipError_t launch_gemm_bf16(const Weight& w, const uint16_t* x, float* y, int64_t m, hipStream_t s,
                            bool gate_in_y = false);
// The GEMM's register-only instruction mix on its grid for an m x n x k Q4_0 / Q8_0
// problem (compute-only ceiling); sink[0] is written only if a sentinel is hit.
// Prefill GEMM on fp32 activations (qmm_gemm.hip): split_rows writes x [m, k] as fp16
// hi / lo parts plus a per-row exponent into `work` (gemm_f32_workspace_bytes(m, k)
// bytes, 256-byte aligned), launch_gemm_split runs the GEMM on them.
size_t gemm_f32_workspace_bytes(int64_t m, int64_t k);
// The prefill GEMM's launch shape (0..3, qmm_gemm.hip choose_shape) for m rows of bf16
// (split_x false) or split fp32 (true) activations; -1 for a type it does not take.
int gemm_shape(const Weight& w, int64_t m, bool split_x);
hipError_t split_rows(const float* x, int64_t m, int64_t k, void* work, hipStream_t s);
hipError_t launch_gemm_split(const Weight& w, const void* work, int64_t m, float* y, hipStream_t s, bool gate_in_y);
hipError_t launch_gemm_ceiling(int type, int64_t m, int64_t n, int64_t k, float* sink, hipStream_t s);

// quant_simd::convert_to_soa_layout: output bytes, and the conversion of `len` device
// bytes (n elements) into `out` on stream s.
size_t soa_bytes(int type, size_t len, size_t n);
hipError_t launch_convert_to_soa(int type, const uint8_t* src, size_t len, size_t n, uint8_t* out, hipStream_t s);

// quant::dequantize semantics for every layout the library knows (F32, F16, Q4_0,
// Q4_1, Q8_0, Q2_K..Q8_K): complete blocks of `bytes` are dequantized, the rest of the
// n_elems outputs are zero.  hipErrorInvalidValue for other types.
hipError_t launch_dequant_layout(int type, const uint8_t* gguf, size_t bytes, size_t n_elems, float* out,
                                 hipStream_t s);

hipError_t launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s);
// Reads `bytes` (a multiple of 16) once; stores nothing in practice (a sentinel store to
// sink[0] keeps the loads live).
hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t s);

// ---- shared host helpers (qmm_api.hip) ----------------------------------------------

// Sets the calling thread's openmini_qmm_last_error() message.
void set_last_error(const char* msg);

// Host GGUF blocks of W[n_rows, k_cols] -> a new repacked weight handle (validated like
// openmini_qmm_upload); the copy and repack run on `stream`, which is synchronised.
int upload_from_host(int type, const void* host_blocks, size_t bytes, int64_t n_rows, int64_t k_cols, void* stream,
                     openmini_qweight** out_weight);

// Host bytes of any layout of launch_dequant_layout -> n floats at d_out (device),
// quant::dequantize semantics; synchronous on `stream`.
int dequantize_from_host(int type, const void* host, size_t bytes, size_t n, float* d_out, void* stream);

}  // namespace qmm
