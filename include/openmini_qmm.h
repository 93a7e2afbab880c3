/*
 * openmini_qmm.h -- C ABI of the MI355X (gfx950) quantized linear layer.
 *
 * The GGUF block-quantized matmul (Q4_0 / Q8_0 weight blocks x fp32 / bf16
 * activations) behind OpenMini-V1's matmul operator.  Rust (or any FFI caller)
 * binds these symbols; everything under them is hand-written HIP for gfx950.
 *
 * Conventions follow openmini-server/native/include/openmini.h:
 *   - `openmini_` prefix, `#pragma once`, `extern "C"` (openmini.h:1-9);
 *   - opaque handle typedefs (openmini.h:16-18);
 *   - status codes whose values coincide with openmini_error_t where the meaning is
 *     shared (openmini.h:20-31); the CUDA code (-6) is not reused, HIP failures
 *     report OPENMINI_QMM_ERR_HIP;
 *   - results through out-pointers (openmini.h:90-94), caller frees through
 *     openmini_qmm_free_* (openmini.h:96,108,142).
 * No call aborts: every failure returns a status and leaves a message in the
 * calling thread's openmini_qmm_last_error().
 *
 * Reference paths are relative to openmini-server/ of skin1987/OpenMini-V1.
 *
 * Threading: a weight's quantized data is immutable after upload and its handle may
 * be shared by threads; each call runs on the stream it is given (NULL = the
 * device's null stream).  A weight that splits K in batched calls also carries
 * mutable scratch (see openmini_qmm_gemv) that orders such calls on one weight.
 * Device pointers (d_*) must stay valid until the stream reaches the call.
 * Host-pointer calls (no d_ prefix) are synchronous and safe from any thread.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; only these declarations export. */
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

#define OPENMINI_QMM_VERSION_MAJOR 0
#define OPENMINI_QMM_VERSION_MINOR 1
#define OPENMINI_QMM_VERSION_PATCH 0
#define OPENMINI_QMM_VERSION_STRING "0.1.0"

typedef enum {
    OPENMINI_QMM_OK = 0,
    OPENMINI_QMM_ERR_MEMORY = -1,        /* = OPENMINI_ERR_MEMORY */
    OPENMINI_QMM_ERR_INVALID_PARAM = -2, /* = OPENMINI_ERR_INVALID_PARAM */
    OPENMINI_QMM_ERR_MODEL_LOAD = -3,    /* = OPENMINI_ERR_MODEL_LOAD */
    OPENMINI_QMM_ERR_INFERENCE = -4,     /* = OPENMINI_ERR_INFERENCE */
    OPENMINI_QMM_ERR_UNSUPPORTED = -5,   /* = OPENMINI_ERR_UNSUPPORTED: QuantError::UnsupportedType */
    OPENMINI_QMM_ERR_HIP = -10,          /* HIP runtime failure (no device, launch error, ...) */
    OPENMINI_QMM_ERR_INSUFFICIENT_DATA = -11, /* QuantError::InsufficientData{expected, actual} */
    OPENMINI_QMM_ERR_NOT_FOUND = -12     /* "Tensor not found" / missing metadata key */
} openmini_qmm_status_t;

/* GGUF tensor type ids (src/model/inference/gguf.rs:219-240).  Weight upload and the
 * decode GEMV take Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K and Q8_K; the prefill GEMM the
 * same without Q4_1 and Q5_K (their blocks carry a minimum); the dequantization entry
 * points take every id listed. */
typedef enum {
    OPENMINI_QMM_F32 = 0,
    OPENMINI_QMM_F16 = 1,
    OPENMINI_QMM_Q4_0 = 2,
    OPENMINI_QMM_Q4_1 = 3,
    OPENMINI_QMM_Q8_0 = 7,
    OPENMINI_QMM_Q2_K = 10,
    OPENMINI_QMM_Q3_K = 11,
    OPENMINI_QMM_Q4_K = 12,
    OPENMINI_QMM_Q5_K = 13,
    OPENMINI_QMM_Q6_K = 14,
    OPENMINI_QMM_Q8_K = 15
} openmini_qmm_type_t;

/* A quantized weight W[n_rows, k_cols] resident in HBM in the GPU layout. */
typedef struct openmini_qweight openmini_qweight_t;

typedef struct {
    int32_t type;            /* openmini_qmm_type_t */
    int32_t device;          /* HIP device ordinal holding the weight */
    int64_t n_rows;          /* N: output features */
    int64_t k_cols;          /* K: input features, a multiple of 32 (256 for Q4_K / Q5_K / Q6_K / Q8_K) */
    int64_t blocks_per_row;  /* K / 32 (32-element sub-blocks for the K-quants) */
    size_t gguf_bytes;       /* GGUF data_size: N * K / 32 * 18 | 20 | 34, N * K / 256 * 144 | 176 | 210 | 258 */
    size_t device_bytes;     /* HBM held by the handle */
} openmini_qmm_weight_info_t;

/* ---- library / device ---------------------------------------------------------- */

/* Library version string (cf. openmini_version, openmini.h:87). */
const char* openmini_qmm_version(void);

/* Selects `device` for this thread and checks it is a gfx950 part
 * (cf. openmini_init, openmini.h:85).  Idempotent. */
int openmini_qmm_init(int device);

/* Message of the last failing call on this thread ("" if none). */
const char* openmini_qmm_last_error(void);

/* Log sink (native/include/openmini.h:151-155, openmini_set_log_callback): every
 * failure recorded for openmini_qmm_last_error() is also passed to `callback` as
 * (OPENMINI_QMM_LOG_ERROR, message, user_data), on the failing thread, after the
 * library's own state is updated; callbacks must not call back into the library.
 * A null callback turns logging off.  Process-wide; safe to call from any thread. */
#define OPENMINI_QMM_LOG_ERROR 3
typedef void (*openmini_qmm_log_callback_t)(int level, const char* text, void* user_data);
int openmini_qmm_set_log_callback(openmini_qmm_log_callback_t callback, void* user_data);

/* GpuQuantOps::is_available (src/model/inference/quant_simd.rs:2979): 1 when a
 * gfx950 device is usable, else 0.  Never fails. */
int openmini_qmm_is_available(void);

/* GpuQuantOps::device_info (quant_simd.rs:2982): writes a NUL-terminated
 * description into buf (truncated to buf_len). */
int openmini_qmm_device_info(char* buf, size_t buf_len);

/* GgufTensor::data_size (src/model/inference/gguf.rs:431-438):
 * ceil(n_elements / block_size) * bytes_per_block for every type id above.  Pure host
 * computation.  n_elements above 2^48 -> INVALID_PARAM (every entry point taking an
 * element count has this limit, so no size computed from one wraps around). */
int openmini_qmm_required_bytes(int type, size_t n_elements, size_t* out_bytes);

/* GpuQuantOps::estimate_memory_usage (quant_simd.rs:2985): device bytes a
 * dequantization of n_elements needs (GGUF input + f32 output); SIZE_MAX above 2^48
 * elements. */
size_t openmini_qmm_estimate_memory_usage(int type, size_t n_elements);

/* ---- weight upload / repack (the loader's layout step) ---------------------------
 * Replaces dequantize-at-load: QuantizedWeightLoader::load_tensor_data
 * (src/model/inference/quant_loader.rs:76-92) -> GgufFile::get_tensor_data_by_ref
 * (gguf.rs:2062-2110) -> quant::dequantize (quant.rs:56).  Takes the tensor's raw
 * GGUF blocks (row n = k_cols/32 consecutive blocks, ggml ne0 = K), keeps them
 * quantized and repacks them on the GPU for its access pattern.
 * Types: Q4_0, Q8_0, Q4_K and Q6_K (GEMV and GEMM; Q4_K / Q6_K with the reference's
 * own reading of those blocks, quant.rs:338-410 and :515-600, whose values are exact
 * products of an integer code and an fp32 sub-block factor); Q4_1 and Q5_K (GEMV only:
 * q * d + m, quant.rs:216-262, and the reference's Q5_K reading (q - 16) * d * scale +
 * dmin * minimum, quant.rs:433-505; each block's product gains its minimum times the
 * block's activation sum); Q8_K (the reference's 258-byte reading, fp16 d and 256
 * int8 codes, value q * d, quant.rs:768-800: eight Q8_0 blocks sharing d, stored and
 * served as Q8_0 with the same values).
 * Errors: INVALID_PARAM (k_cols % 32, or % 256 for the K-quants and Q8_K; sizes <= 0),
 * UNSUPPORTED (type), INSUFFICIENT_DATA (gguf_bytes < required). */
int openmini_qmm_upload(int type, const void* gguf_blocks, size_t gguf_bytes,
                        int64_t n_rows, int64_t k_cols, openmini_qweight_t** out_weight);

/* Same, from GGUF blocks already in device memory (e.g. copied straight from the
 * mmap); the repack runs on `stream`, the handle is usable once it completes. */
int openmini_qmm_upload_device(int type, const void* d_gguf_blocks, size_t gguf_bytes,
                               int64_t n_rows, int64_t k_cols, void* stream,
                               openmini_qweight_t** out_weight);

/* The device bytes a weight of this type and shape occupies (its chunks, then the
 * batched GEMV's K-split workspace for weights that have one): what
 * openmini_qmm_upload_device_into needs.  Errors as openmini_qmm_upload's shape checks.
 * No counterpart in the reference (its loader allocates per tensor). */
int openmini_qmm_weight_device_bytes(int type, int64_t n_rows, int64_t k_cols, size_t* out_bytes);

/* openmini_qmm_upload_device into caller-owned device memory, with no device
 * allocation: d_weight_mem (256-byte aligned, device memory of the current device, at
 * least openmini_qmm_weight_device_bytes) holds the weight until
 * openmini_qmm_free_weight, which then frees the handle only; the caller frees the
 * memory after that.  For loaders that place a model's weights in one device arena
 * (one allocation for every layer), where the upload is bound by the repack kernel.
 * No counterpart in the reference (quant_loader.rs:54-138 keeps one allocation per
 * tensor).  Errors: those of openmini_qmm_upload_device; INVALID_PARAM for memory
 * that is null, unaligned, smaller than needed, or not on the current device. */
int openmini_qmm_upload_device_into(int type, const void* d_gguf_blocks, size_t gguf_bytes,
                                    int64_t n_rows, int64_t k_cols, void* d_weight_mem,
                                    size_t weight_mem_bytes, void* stream,
                                    openmini_qweight_t** out_weight);

void openmini_qmm_free_weight(openmini_qweight_t* weight);

int openmini_qmm_weight_info(const openmini_qweight_t* weight,
                             openmini_qmm_weight_info_t* info);

/* ---- the operator -----------------------------------------------------------------
 * linear(x, W) = x . W^T (src/model/inference/model.rs:1050-1064, GemmEngine::matmul
 * gemm_engine.rs:40), on the quantized W without materialising f32 weights. */

/* Decode GEMV: y[batch, N] = x[batch, K] . W^T, fp32 activations, fp32 output.
 * Any batch >= 1.  Up to 3 rows: the single-row-tuned kernel; 4 or more: the
 * batched kernel, one pass over W per 16 rows, in which a row's result does not
 * depend on the other rows of the call nor on the batch size (bitwise).  Every
 * weight type.
 * A weight of at most 8192 rows and K >= 4000 splits K of a batched call over two or
 * four workgroups per row tile; their partial sums and arrival counters live in a
 * mutable workspace after the weight's chunks (counted in device_bytes: 128 or 256 B
 * per row plus one word per tile group).  Batched calls (4+ rows, here and in
 * openmini_qmm_gemv_multi) on one such weight must therefore not overlap in time
 * (two streams with no ordering between them): they would share the workspace and
 * could return wrong sums.  The counters only grow, by the split count per call, so
 * calls after an overlap are correct again.  openmini_qmm_linear_host / _noalloc
 * serialise their own such calls per weight.  Calls of up to 3 rows, the SwiGLU
 * pair and calls on different weights share no state.
 * d_x must be 16-byte aligned. */
int openmini_qmm_gemv(const openmini_qweight_t* weight, const float* d_x, float* d_y,
                      int64_t batch, void* stream);

/* Prefill GEMM: y[m, N] = x[m, K] . W^T with bf16 activations (raw bf16 bits),
 * fp32 output, on bf16 MFMA with exact integer codes and fp32 per-block scales.
 * Q4_0, Q8_0, Q4_K and Q6_K weights (Q6_K: code * 16-element scale, an exact integer,
 * as two bf16 parts, then the fp32 d); UNSUPPORTED for Q4_1 / Q5_K, which run the
 * decode GEMVs at any row count.  d_x must be 16-byte aligned. */
int openmini_qmm_gemm_bf16(const openmini_qweight_t* weight, const uint16_t* d_x, float* d_y,
                           int64_t m, void* stream);

/* Prefill GEMM on fp32 activations, linear_gemm's input type (model.rs:1060-1064):
 * y[m, N] = x[m, K] . W^T, fp32 in and out.  A first kernel writes each row of x,
 * scaled by a power of two per row, as fp16 hi + lo parts (x carried to within
 * 2^-22 of each element; elements more than 2^17 below their row's largest keep an
 * absolute error below 2^-39 of it) into d_work; the GEMM then runs two chained fp16
 * MFMAs per block on exact fp16 codes and rescales per block in fp32.  A row holding
 * inf or NaN gives NaN outputs in that row.  d_work: at least
 * openmini_qmm_gemm_f32_workspace_bytes(m, K) bytes, 256-byte aligned, not shared
 * with another call in flight; d_x 16-byte aligned.  Every weight type of
 * openmini_qmm_gemm_bf16. */
size_t openmini_qmm_gemm_f32_workspace_bytes(int64_t m, int64_t k_cols);

/* Diagnostic, no counterpart in the reference: the launch shape the prefill GEMM picks
 * for m rows on this weight (bf16 activations, or split fp32 ones when split_x != 0):
 * 0 = 128 x 96 tiles, 1 = 128 x 64, 2 = 64 x 96, 3 = 64 x 64 (rows x columns per
 * workgroup), chosen from the problem size alone, so a row's bits depend only on m and
 * the weight.  A negative status on error. */
int openmini_qmm_gemm_launch_shape(const openmini_qweight_t* weight, int64_t m, int split_x);

/* Routing query, no counterpart in the reference: the fewest activation rows from which
 * openmini_qmm_linear_host (and _noalloc) run the fp32 prefill GEMM on this weight
 * rather than the decode GEMVs: the first m in [64, 128) where the GEMM's estimated
 * time (about 10 ns per K element while its grid fits one round) beats the GEMVs' (one
 * pass per 16 rows, about 6.5 us plus the weight bytes at 3-5 TB/s), else 128; 0 for
 * Q4_1 / Q5_K, which have no prefill GEMM.  Depends on the weight's type and shape
 * only.  Engines that call the GEMM and GEMV entry points themselves use it to make
 * the same choice.  A negative status on error. */
int64_t openmini_qmm_gemm_min_rows(const openmini_qweight_t* weight);
int openmini_qmm_gemm_f32(const openmini_qweight_t* weight, const float* d_x, float* d_y, int64_t m,
                          void* d_work, size_t work_bytes, void* stream);

/* ---- projections of one layer (src/model/inference/model.rs) ----------------------- */

/* Weights that share the input: d_ys[i][batch, N_i] = x[batch, K] . W_i^T for
 * i < count (1..4), all of one type and one K; one launch for up to 3 batch rows,
 * or from 4 rows on one batched pass per weight (results identical to
 * openmini_qmm_gemv of each weight).  Replaces the three linear_gemm calls of prepare_qkv
 * (model.rs:1392-1394: q, k, v of one normalised hidden state).  d_x must be
 * 16-byte aligned. */
int openmini_qmm_gemv_multi(const openmini_qweight_t* const* weights, int count, const float* d_x,
                            float* const* d_ys, int64_t batch, void* stream);

/* FFN hidden state of FFNWeights::forward (model.rs:728-731, the silu(gate) * up
 * branch; silu(v) = v / (1 + exp(-v)), model.rs:1187-1189):
 * d_h[batch, N] = silu(x . Wg^T) * (x . Wu^T), gate and up of one type and shape, one
 * launch reading both weights for up to 3 batch rows (per 16 rows from 4 rows on).  d_x
 * must be 16-byte aligned. */
int openmini_qmm_ffn_gate_up(const openmini_qweight_t* gate, const openmini_qweight_t* up,
                             const float* d_x, float* d_h, int64_t batch, void* stream);

/* The same for prefill with bf16 activations (raw bf16 bits): the gate GEMM writes
 * d_h, the up GEMM finishes silu(gate) * up in its epilogue.  d_x 16-byte aligned. */
int openmini_qmm_ffn_gate_up_bf16(const openmini_qweight_t* gate, const openmini_qweight_t* up,
                                  const uint16_t* d_x, float* d_h, int64_t m, void* stream);

/* The same for prefill with fp32 activations: x is split once into d_work (as in
 * openmini_qmm_gemm_f32, same size and alignment rules), then the gate GEMM and the up
 * GEMM with the silu(gate) * up epilogue. */
int openmini_qmm_ffn_gate_up_f32(const openmini_qweight_t* gate, const openmini_qweight_t* up,
                                 const float* d_x, float* d_h, int64_t m, void* d_work, size_t work_bytes,
                                 void* stream);

/* GemmEngine::matmul-shaped convenience on host memory: y[m, N] = x[m, K] . W^T,
 * fp32 in/out, synchronous.  Below openmini_qmm_gemm_min_rows rows (64-128, by the
 * weight's shape) the decode GEMVs, from there on the fp32 prefill GEMM
 * (openmini_qmm_gemm_f32; Q4_1 / Q5_K weights: the batched GEMV at any row count); x,
 * y and the GEMM's workspace are allocated per call. */
int openmini_qmm_linear_host(const openmini_qweight_t* weight, const float* x, float* y,
                             int64_t m);

/* openmini_qmm_linear_host without any allocation.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  x and y are staged through a
 * fixed 16 MiB device array that the library holds on every device it runs on until
 * the process ends: x, then (from openmini_qmm_gemm_min_rows rows on, for the types
 * the GEMM takes) the fp32 GEMM's workspace, then y, each from a 256-byte boundary.  About m * (K + N) * 4
 * bytes without the GEMM and m * (2 K + N + 1) * 4 with it must fit in 16 MiB, else
 * INVALID_PARAM naming the row limit.  Same kernels and results as openmini_qmm_linear_host, synchronous
 * on the null stream.
 * All calls on one device share the array: the library holds a per-device lock from
 * the copy in to the copy out, so calls from several threads are safe and run one at
 * a time per device.  Nothing in the array needs clearing (x and y are written whole
 * by every call). */
int openmini_qmm_linear_host_noalloc(const openmini_qweight_t* weight, const float* x, float* y,
                                     int64_t m);

/* ---- dequantization (GpuQuantOps, src/model/inference/quant_simd.rs:2944-2986) ----- */

/* Dequantizes an uploaded Q4_0 / Q8_0 / Q8_K weight to f32 W[N, K] (row-major) in device memory
 * (d_out 16-byte aligned).  Bit-identical to quant::dequantize of the original GGUF bytes.
 * UNSUPPORTED for the other weight types: their GGUF bytes dequantize through
 * openmini_qmm_dequantize_any_device. */
int openmini_qmm_dequant_weight(const openmini_qweight_t* weight, float* d_out, void* stream);

/* quant_simd::safe_dequantize semantics (quant_simd.rs:150-302) on raw GGUF bytes in
 * device memory, for Q4_0, Q8_0 and Q4_1: n == 0 -> OK (nothing written); gguf_bytes
 * < ceil(n/32)*bpb -> INSUFFICIENT_DATA with *expected_bytes set; other types ->
 * UNSUPPORTED (QuantError::UnsupportedType).  Writes n floats.  expected_bytes may be
 * NULL. */
int openmini_qmm_dequantize_device(int type, const void* d_gguf, size_t gguf_bytes, size_t n,
                                   float* d_out, void* stream, size_t* expected_bytes);

/* GpuQuantOps::dequantize_{q4_0,q8_0}_gpu(&[u8], n) -> Vec<f32> (quant_simd.rs:2955-2958):
 * host bytes in, host floats out, synchronous, same validation as above. */
int openmini_qmm_dequantize(int type, const void* gguf, size_t gguf_bytes, size_t n,
                            float* out, size_t* expected_bytes);

/* quant::dequantize semantics (src/model/inference/quant.rs:56-79), the CPU path that
 * GpuQuantOps::batch_dequantize_gpu falls back to (quant_simd.rs:3104-3118 via
 * dequantize_simd :304-313), for F32, F16, Q4_0, Q4_1, Q8_0 and Q2_K..Q8_K: the blocks
 * that fit in gguf_bytes are dequantized, the rest of the n outputs are 0.0 (the
 * reference stops at the first incomplete block).  Bit-identical to the reference,
 * signed zeros included.  F32 / F16 input with fewer than n whole elements: those
 * elements, then 0.0 -- dequantize_simd's fixed-length result (quant_simd.rs:332-340);
 * quant::dequantize_f32 / _f16 (quant.rs:95-133) return the same leading values as a
 * shorter vector.  Other type ids -> UNSUPPORTED (the reference returns zeros
 * for types it does not implement; the IQ types are not implemented here). */
int openmini_qmm_dequantize_any_device(int type, const void* d_gguf, size_t gguf_bytes, size_t n,
                                       float* d_out, void* stream);

/* Same on host memory, synchronous. */
int openmini_qmm_dequantize_any(int type, const void* gguf, size_t gguf_bytes, size_t n, float* out);

/* quant_simd::convert_to_soa_layout (src/model/inference/quant_simd.rs:3245-3397), the
 * reference's AoS -> SoA byte permutation:
 *   - empty input or n == 0: 0 bytes;
 *   - F32 / F16: the first min(n * 4 | 2, len) bytes, copied;
 *   - Q4_0 / Q8_0: [the fp16 scale of each of ceil(n / 32) blocks][byte position 0 of
 *     every block] ... [the last position]; Q4_1: [scales][mins][16 positions]; a
 *     field is copied only when both its bytes are in the input, missing code bytes
 *     are 0;
 *   - any other GgufTensorType id: the input, copied.
 * soa_bytes gives the output length (UNSUPPORTED for ids GgufTensorType does not have;
 * n above 2^48 -> INVALID_PARAM).  The device call runs on `stream`; the host call is
 * synchronous.  The reference's unused `_block_size` argument is dropped. */
int openmini_qmm_soa_bytes(int type, size_t len, size_t n, size_t* out_bytes);
int openmini_qmm_convert_to_soa_device(int type, const void* d_data, size_t len, size_t n,
                                       void* d_out, void* stream);
int openmini_qmm_convert_to_soa(int type, const void* data, size_t len, size_t n, void* out);

/* ---- GGUF files: the loader's raw-block path ----------------------------------------
 * GgufFile (src/model/inference/gguf.rs:1357-2110) and QuantizedWeightLoader
 * (quant_loader.rs:54-138) without dequantize-at-load.  The file is memory-mapped once;
 * tensor bytes are views of the mapping; a Q4_0 / Q8_0 projection goes to the GPU as
 * its raw blocks.  Host-only calls (open, header, lookups, metadata, data views) touch
 * no device. */

typedef struct openmini_qmm_gguf openmini_qmm_gguf_t;

typedef enum {
    OPENMINI_QMM_GGUF_AUTO = 0,      /* standard, else the reference's dialect */
    OPENMINI_QMM_GGUF_REFERENCE = 1, /* 1-byte type fields, absolute tensor offsets (gguf.rs:1795,
                                        2009, 2037) -- what the reference reads and writes */
    OPENMINI_QMM_GGUF_STANDARD = 2   /* GGUF v2/v3: uint32 type fields, offsets relative to the
                                        data section aligned to general.alignment (default 32) */
} openmini_qmm_gguf_dialect_t;

typedef struct {
    uint32_t version;            /* GgufHeader (gguf.rs:1687-1702) */
    int32_t dialect;             /* the dialect the file was read in */
    uint64_t tensor_count;
    uint64_t metadata_kv_count;
    uint64_t distinct_tensors;   /* after later definitions replace earlier ones */
    uint64_t distinct_keys;
    uint32_t alignment;          /* standard dialect; 0 for the reference's */
    uint64_t file_size;
} openmini_qmm_gguf_header_t;

typedef struct {
    int32_t type;                /* GgufTensorType id (gguf.rs:219-247) */
    uint32_t n_dims;
    uint64_t dims[8];            /* GGUF order: dims[0] = ne0 (the contiguous dimension) */
    uint64_t offset;             /* absolute file offset of the data */
    uint64_t n_elements;         /* GgufTensor::num_elements (gguf.rs:425-427) */
    uint64_t data_size;          /* GgufTensor::data_size (gguf.rs:431-438) */
} openmini_qmm_gguf_tensor_info_t;

/* GgufFile::open + parse (gguf.rs:1357-1364, 1658-2032).  Errors (MODEL_LOAD, message as
 * the reference's): file missing, "File too small", "Invalid GGUF magic number",
 * "Unexpected EOF", "String too long", "Unknown value type", "Too many dimensions",
 * "Unknown tensor type".  Never reads past the file. */
int openmini_qmm_gguf_open(const char* path, int dialect, openmini_qmm_gguf_t** out_gguf);
void openmini_qmm_gguf_close(openmini_qmm_gguf_t* gguf);
int openmini_qmm_gguf_header(const openmini_qmm_gguf_t* gguf, openmini_qmm_gguf_header_t* header);

/* Tensors in file order (index < distinct_tensors) and by name (GgufFile::tensors). */
int openmini_qmm_gguf_tensor_name(const openmini_qmm_gguf_t* gguf, size_t index, char* buf, size_t buf_len);
int openmini_qmm_gguf_tensor_info(const openmini_qmm_gguf_t* gguf, const char* name,
                                  openmini_qmm_gguf_tensor_info_t* info);

/* GgufFile::get_tensor_data (gguf.rs:2034-2045): a view of the tensor's data_size bytes
 * inside the mapping, valid until openmini_qmm_gguf_close.  NOT_FOUND; MODEL_LOAD
 * "Tensor data out of bounds". */
int openmini_qmm_gguf_tensor_data(const openmini_qmm_gguf_t* gguf, const char* name, const void** data,
                                  size_t* bytes);

/* GgufMetadata (gguf.rs:133-209): keys in file order, value type (0..12, gguf.rs:73-101)
 * and the typed getters get_u32 (UInt32 | Int32), get_u64 (UInt64 | Int64 | UInt32 |
 * Int32), get_f32 (Float32), get_string.  NOT_FOUND when absent or of another type. */
int openmini_qmm_gguf_meta_key(const openmini_qmm_gguf_t* gguf, size_t index, char* buf, size_t buf_len);
int openmini_qmm_gguf_meta_type(const openmini_qmm_gguf_t* gguf, const char* key, int* value_type,
                                uint64_t* array_len);
int openmini_qmm_gguf_get_u32(const openmini_qmm_gguf_t* gguf, const char* key, uint32_t* out);
int openmini_qmm_gguf_get_u64(const openmini_qmm_gguf_t* gguf, const char* key, uint64_t* out);
int openmini_qmm_gguf_get_f32(const openmini_qmm_gguf_t* gguf, const char* key, float* out);
int openmini_qmm_gguf_get_string(const openmini_qmm_gguf_t* gguf, const char* key, char* buf, size_t buf_len,
                                 size_t* out_len);

/* QuantizedWeightLoader::load_tensor (quant_loader.rs:66-92) without dequantization: the
 * 2-D tensor [ne0 = K, ne1 = N] becomes the weight W[N, K] (row n = K consecutive
 * elements, the semantic layout linear() multiplies by); the weight types of
 * openmini_qmm_upload (UNSUPPORTED otherwise).  Copy and repack run on `stream`, synchronised before returning. */
int openmini_qmm_gguf_upload_weight(const openmini_qmm_gguf_t* gguf, const char* name, void* stream,
                                    openmini_qweight_t** out_weight);

/* GgufFile::get_tensor_data_by_ref (gguf.rs:2062-2110) on the GPU: the tensor as
 * n_elements f32 in device memory at d_out, bit-identical to the reference for F32, F16,
 * Q4_0, Q4_1, Q8_0 and Q2_K..Q8_K (UNSUPPORTED for other types).  Synchronous.
 * As the reference, an F32 tensor whose data does not start 4-byte aligned in the file,
 * or an F16 tensor not 2-byte aligned, is MODEL_LOAD "F32 data is not properly aligned" /
 * "F16 data is not properly aligned" (gguf.rs:2076-2078, 2090-2092; the reference's
 * size-mismatch errors cannot occur: data_size is n_elements * 4 | 2 by definition). */
int openmini_qmm_gguf_dequantize_tensor(const openmini_qmm_gguf_t* gguf, const char* name, float* d_out,
                                        void* stream);

/* ---- device memory and streams for callers without a HIP binding of their own ----- */

int openmini_qmm_malloc(void** d_ptr, size_t bytes);
int openmini_qmm_free(void* d_ptr);
int openmini_qmm_memcpy_h2d(void* d_dst, const void* src, size_t bytes, void* stream);
int openmini_qmm_memcpy_d2h(void* dst, const void* d_src, size_t bytes, void* stream);
int openmini_qmm_memset(void* d_dst, int value, size_t bytes, void* stream);
int openmini_qmm_stream_create(void** out_stream);
int openmini_qmm_stream_destroy(void* stream);
int openmini_qmm_stream_synchronize(void* stream);

/* Bandwidth calibration: a plain streaming copy kernel of `bytes` (multiple of 16,
 * 16-byte aligned pointers) on `stream`; the yardstick that HBM traffic counters
 * of the GEMV are scaled against.  No counterpart in the reference. */
int openmini_qmm_stream_copy(void* d_dst, const void* d_src, size_t bytes, void* stream);

/* Single-launch floor: a read-only streaming kernel over `bytes` (multiple of 16,
 * 16-byte aligned source) on `stream`, 16-byte loads, workgroups of 512 lanes over
 * consecutive 16 KB spans (the fastest read shape measured on MI355X).  Nothing is
 * written in practice; d_sink (4 bytes, 4-byte aligned) receives a word only if the
 * data fold hits a sentinel.  The time a read-bound kernel of that many bytes cannot
 * beat in one launch; the decode GEMV is measured against it.  No counterpart in the
 * reference. */
int openmini_qmm_stream_read(const void* d_src, size_t bytes, void* d_sink, void* stream);

/* Compute-only ceiling of the prefill GEMM: for an m x n x k problem on a Q4_0 or
 * Q8_0 weight (type), the grid and waves openmini_qmm_gemm_bf16 would launch, each
 * running only its per-block register work (code conversion, MFMAs, rescale FMAs) on
 * operands held in registers: no loads, LDS traffic, barriers or stores.  d_sink
 * (4 bytes, 4-byte aligned) receives a word only if a sentinel is hit.  Its time is
 * what the GEMM's instruction mix alone costs; the GEMM is measured against it.
 * INVALID_PARAM for sizes <= 0, k % 32 != 0; UNSUPPORTED for other types.  No
 * counterpart in the reference. */
int openmini_qmm_gemm_ceiling(int type, int64_t m, int64_t n, int64_t k, void* d_sink, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif
