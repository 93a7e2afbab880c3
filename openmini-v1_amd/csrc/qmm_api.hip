// C-ABI of libopenmini_qmm.so (declarations and reference citations in
// include/openmini_qmm.h).  Host code only: validation, device selection, memory
// management and kernel dispatch.  Every failure returns a status and records a
// message for openmini_qmm_last_error(); nothing aborts.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "qmm_internal.hpp"

struct openmini_qweight {
    qmm::Weight w;
    // Serialises the synchronous host-memory calls of 4+ rows on a weight with a K
    // split workspace, so concurrent host threads may share one handle there (their
    // launches go to the null stream, which orders them too; the lock keeps that
    // guarantee independent of the stream).
    mutable std::mutex batch_mu;
    // false for openmini_qmm_upload_device_into: the caller's memory, not freed here
    bool owns_memory = true;
};

namespace {

thread_local std::string g_last_error;

// The log sink of openmini_qmm_set_log_callback (callback and its user data change
// together under the mutex; the call itself runs outside it).
std::mutex g_log_mu;
openmini_qmm_log_callback_t g_log_cb = nullptr;
void* g_log_user = nullptr;

void log_error(const char* msg) {
    openmini_qmm_log_callback_t cb;
    void* user;
    {
        std::lock_guard<std::mutex> lk(g_log_mu);
        cb = g_log_cb;
        user = g_log_user;
    }
    if (cb) cb(OPENMINI_QMM_LOG_ERROR, msg, user);
}

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    log_error(buf);
    return code;
}

int ok() {
    g_last_error.clear();
    return OPENMINI_QMM_OK;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(OPENMINI_QMM_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(expr, what)                         \
    do {                                            \
        hipError_t e_ = (expr);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

// Weight layouts of the upload and the decode GEMV; the prefill GEMM takes those
// without a block minimum (not Q4_1 / Q5_K), dequant_weight Q4_0 and Q8_0 (Q8_K
// weights are stored as Q8_0 chunks: chunk_type).
bool type_supported(int type) {
    return type == OPENMINI_QMM_Q4_0 || type == OPENMINI_QMM_Q4_1 || type == OPENMINI_QMM_Q8_0 ||
           qmm::is_kquant(type) || type == OPENMINI_QMM_Q8_K;
}
int check_gemm_type(const qmm::Weight& w) {
    if (qmm::has_block_min(w.type))
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED,
                    "no prefill GEMM for type %d (Q4_1 / Q5_K weights run the decode GEMVs at any row count)", w.type);
    return OPENMINI_QMM_OK;
}
// Rows that linear() hands to the fp32 prefill GEMM rather than the decode GEMVs.
bool gemm_rows(const qmm::Weight& w, int64_t m) {
    return !qmm::has_block_min(w.type) && m >= qmm::gemm_min_rows(w.type, w.n, w.k);
}
bool plain_type(int type) { return type == OPENMINI_QMM_Q4_0 || type == OPENMINI_QMM_Q8_0; }
// quant_simd::safe_dequantize's types (quant_simd.rs:284-302, F16/F32 aside).
bool safe_type(int type) {
    return type == OPENMINI_QMM_Q4_0 || type == OPENMINI_QMM_Q8_0 || type == OPENMINI_QMM_Q4_1;
}
// ceil(n / block_size) * bytes_per_block (gguf.rs:431-438); 0 for unknown types.
// Element counts above 2^48 (1 PB of f32) are rejected, so every size computed
// from one (bytes of any layout, n * sizeof(float)) fits in 64 bits.
constexpr size_t kMaxElements = (size_t)1 << 48;

size_t layout_bytes(int type, size_t n) {
    const int bs = qmm::layout_block_size(type);
    return bs ? (n + bs - 1) / bs * (size_t)qmm::layout_bytes_per_block(type) : 0;
}

int check_elements(size_t n) {
    if (n > kMaxElements)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "n_elements=%zu exceeds the maximum 2^48", n);
    return OPENMINI_QMM_OK;
}

// Device probing is done once per device; the result is cached.
constexpr int kMaxDevices = 64;  // device ordinals the per-device tables cover
std::mutex g_dev_mu;
int g_dev_state[kMaxDevices];  // 0 unknown, 1 gfx950, -1 unusable

int ensure_device(int* out_dev) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(OPENMINI_QMM_ERR_HIP, "device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if (g_dev_state[dev] == 0) {
        hipDeviceProp_t p;
        e = hipGetDeviceProperties(&p, dev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        g_dev_state[dev] = (std::strncmp(p.gcnArchName, "gfx950", 6) == 0) ? 1 : -1;
        if (g_dev_state[dev] < 0)
            return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950",
                        dev, p.gcnArchName);
    }
    if (g_dev_state[dev] < 0)
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "device %d is not a gfx950 part", dev);
    if (out_dev) *out_dev = dev;
    return OPENMINI_QMM_OK;
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int validate_weight_args(int type, size_t gguf_bytes, int64_t n_rows, int64_t k_cols) {
    if (!type_supported(type))
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED,
                    "unsupported tensor type %d (Q4_0=2, Q4_1=3, Q8_0=7, Q4_K=12, Q5_K=13, Q6_K=14, Q8_K=15)",
                    type);
    if (n_rows <= 0 || k_cols <= 0)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "invalid shape [%lld, %lld]", (long long)n_rows,
                    (long long)k_cols);
    const int be = qmm::weight_block_elems(type);  // 32, or 256 for the K-quant super-blocks
    if (k_cols % be != 0)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "k_cols=%lld is not a multiple of %d", (long long)k_cols, be);
    if (n_rows > INT32_MAX || k_cols / qmm::kQK > INT32_MAX / 64)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "shape [%lld, %lld] too large", (long long)n_rows,
                    (long long)k_cols);
    // The decode kernels address the weight with 32-bit buffer offsets: the chunks
    // (padding included) must stay below 4 GiB (a Q4_0 matrix of ~7.5 G elements; the
    // largest Llama-70B projection is 0.23 G).
    const size_t chunked = (size_t)((n_rows + qmm::kTileRows - 1) / qmm::kTileRows) *
                           (size_t)((k_cols / qmm::kQK + qmm::kTileBlocks - 1) / qmm::kTileBlocks) *
                           (size_t)qmm::chunk_bytes(qmm::chunk_type(type));
    if (chunked >= ((size_t)1 << 32))
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "shape [%lld, %lld]: %zu weight bytes exceed 4 GiB",
                    (long long)n_rows, (long long)k_cols, chunked);
    const size_t need = (size_t)n_rows * (size_t)(k_cols / be) * qmm::bytes_per_block(type);
    if (gguf_bytes < need)
        return fail(OPENMINI_QMM_ERR_INSUFFICIENT_DATA,
                    "InsufficientData: expected %zu bytes, actual %zu", need, gguf_bytes);
    return OPENMINI_QMM_OK;
}

// The weight's geometry and device size (chunks, then the K-split workspace).
void plan_weight(int type, int64_t n_rows, int64_t k_cols, int dev, qmm::Weight& w) {
    w.src_type = type;
    w.type = qmm::chunk_type(type);
    w.device = dev;
    w.n = n_rows;
    w.k = k_cols;
    w.nb = k_cols / qmm::kQK;
    w.n_tiles = (w.n + qmm::kTileRows - 1) / qmm::kTileRows;
    w.groups = (w.nb + qmm::kTileBlocks - 1) / qmm::kTileBlocks;
    w.chunk_bytes = (size_t)qmm::chunk_bytes(w.type);
    qmm::batch_split(w.type, w.n_tiles, w.groups, &w.split_t, &w.split_s);
    w.device_bytes = round_up((size_t)w.n_chunks() * w.chunk_bytes, 256) +
                     qmm::split_workspace_bytes(w.n_tiles, w.split_t, w.split_s);
}

// Places a planned weight at `base` (device_bytes, 256-byte aligned).
void bind_weight(qmm::Weight& w, void* base) {
    w.chunks = static_cast<uint8_t*>(base);
    const size_t chunks_bytes = round_up((size_t)w.n_chunks() * w.chunk_bytes, 256);
    if (w.device_bytes > chunks_bytes) {
        w.split_part = reinterpret_cast<float*>(w.chunks + chunks_bytes);
        w.split_cnt = reinterpret_cast<uint32_t*>(
            w.chunks + chunks_bytes + (size_t)w.split_s * qmm::kBatchRows * (size_t)w.n_tiles * qmm::kTileRows * 4);
    }
}

int alloc_weight(int type, int64_t n_rows, int64_t k_cols, int dev, openmini_qweight** out) {
    openmini_qweight* h = new (std::nothrow) openmini_qweight();
    if (!h) return fail(OPENMINI_QMM_ERR_MEMORY, "host allocation failed");
    qmm::Weight& w = h->w;
    plan_weight(type, n_rows, k_cols, dev, w);
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, w.device_bytes);
    if (e != hipSuccess) {
        delete h;
        return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc(%zu) for weight failed: %s", w.device_bytes,
                    hipGetErrorString(e));
    }
    bind_weight(w, base);
    *out = h;
    return OPENMINI_QMM_OK;
}

int check_weight(const openmini_qweight* h) {
    if (!h) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null weight handle");
    int dev = 0;
    int rc = ensure_device(&dev);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (dev != h->w.device)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "weight lives on device %d, current device is %d",
                    h->w.device, dev);
    return OPENMINI_QMM_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ---- device staging of openmini_qmm_linear_host_noalloc ----------------------------
// x, then y at the next 256-byte boundary, in one file-scope array that every device
// the library runs on holds until the process ends.  Its name is a host-side stand-in:
// the device address of each device's copy comes from hipGetSymbolAddress, resolved
// once per device with that device current and kept in g_scratch_ptr.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices];  // per device ordinal; nullptr until resolved
// One staging user per device at a time: openmini_qmm_linear_host_noalloc holds its
// device's lock across the copy in, the launch and the copy out (the call is
// synchronous, so the lock costs nothing beyond the serialisation the shared array
// needs anyway).
std::mutex g_staging_mu[kMaxDevices];

// The current device's address of `scratch` (dev = the current device).
int scratch_on_device(int dev, uint8_t** out) {
    if (dev < 0 || dev >= kMaxDevices) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "device ordinal %d out of range", dev);
    hipError_t e = hipSuccess;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (!g_scratch_ptr[dev]) {
            void* p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e == hipSuccess) g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
        }
        *out = g_scratch_ptr[dev];
    }
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    return OPENMINI_QMM_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace

namespace qmm {

void set_last_error(const char* msg) { g_last_error = msg ? msg : ""; }

int upload_from_host(int type, const void* host_blocks, size_t bytes, int64_t n_rows, int64_t k_cols, void* stream,
                     openmini_qweight** out_weight) {
    *out_weight = nullptr;
    int rc = validate_weight_args(type, bytes, n_rows, k_cols);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!host_blocks) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null gguf_blocks");
    int dev = 0;
    rc = ensure_device(&dev);
    if (rc != OPENMINI_QMM_OK) return rc;
    const size_t need = (size_t)n_rows * (size_t)(k_cols / weight_block_elems(type)) * bytes_per_block(type);
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, need);
    if (e != hipSuccess)
        return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc(%zu) staging failed: %s", need, hipGetErrorString(e));
    openmini_qweight* h = nullptr;
    rc = alloc_weight(type, n_rows, k_cols, dev, &h);
    if (rc != OPENMINI_QMM_OK) {
        (void)hipFree(staging);
        return rc;
    }
    hipStream_t s = as_stream(stream);
    e = hipMemcpyAsync(staging, host_blocks, need, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = launch_repack(h->w, static_cast<const uint8_t*>(staging), s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(staging);
    if (e != hipSuccess) {
        openmini_qmm_free_weight(h);
        return hip_fail(e, "upload/repack");
    }
    *out_weight = h;
    return ok();
}

int dequantize_from_host(int type, const void* host, size_t bytes, size_t n, float* d_out, void* stream) {
    if (n == 0) return ok();
    int rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    const size_t used = bytes;
    void* din = nullptr;
    hipError_t e = hipMalloc(&din, used ? used : 1);
    if (e != hipSuccess)
        return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc(%zu) for dequantize failed: %s", used, hipGetErrorString(e));
    hipStream_t s = as_stream(stream);
    if (used) e = hipMemcpyAsync(din, host, used, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = launch_dequant_layout(type, static_cast<const uint8_t*>(din), used, n, d_out, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(din);
    if (e != hipSuccess) return hip_fail(e, "dequantize");
    return ok();
}

}  // namespace qmm

extern "C" {

const char* openmini_qmm_version(void) { return OPENMINI_QMM_VERSION_STRING; }

const char* openmini_qmm_last_error(void) { return g_last_error.c_str(); }

int openmini_qmm_init(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) return fail(OPENMINI_QMM_ERR_HIP, "no HIP device available");
    if (device < 0 || device >= count)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "device %d out of range (count %d)", device, count);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    int rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    uint8_t* staging = nullptr;  // resolve the no-allocation staging while `device` is current
    rc = scratch_on_device(device, &staging);
    if (rc != OPENMINI_QMM_OK) return rc;
    return ok();
}

int openmini_qmm_set_log_callback(openmini_qmm_log_callback_t callback, void* user_data) {
    {
        std::lock_guard<std::mutex> lk(g_log_mu);
        g_log_cb = callback;
        g_log_user = user_data;
    }
    return ok();
}

int openmini_qmm_is_available(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return 0;
    std::string saved = g_last_error;
    const int rc = ensure_device(nullptr);
    g_last_error = saved;
    return rc == OPENMINI_QMM_OK ? 1 : 0;
}

int openmini_qmm_device_info(char* buf, size_t buf_len) {
    if (!buf || buf_len == 0) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null buffer");
    int dev = 0;
    int rc = ensure_device(&dev);
    if (rc != OPENMINI_QMM_OK) {
        std::snprintf(buf, buf_len, "HipQuantOps { device: unavailable }");
        return rc;
    }
    hipDeviceProp_t p;
    HIP_TRY(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
    std::snprintf(buf, buf_len, "HipQuantOps { device: %d, name: %s, arch: %s, cus: %d, hbm_bytes: %zu }",
                  dev, p.name, p.gcnArchName, p.multiProcessorCount, (size_t)p.totalGlobalMem);
    return ok();
}

int openmini_qmm_required_bytes(int type, size_t n_elements, size_t* out_bytes) {
    if (!out_bytes) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_bytes");
    if (!qmm::layout_block_size(type)) return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "unsupported tensor type %d", type);
    const int rc = check_elements(n_elements);
    if (rc != OPENMINI_QMM_OK) return rc;
    *out_bytes = layout_bytes(type, n_elements);
    return ok();
}

size_t openmini_qmm_estimate_memory_usage(int type, size_t n_elements) {
    if (n_elements > kMaxElements) return SIZE_MAX;
    const size_t in = qmm::layout_block_size(type) ? layout_bytes(type, n_elements) : n_elements * sizeof(float);
    return in + n_elements * sizeof(float);
}

int openmini_qmm_upload(int type, const void* gguf_blocks, size_t gguf_bytes, int64_t n_rows,
                        int64_t k_cols, openmini_qweight_t** out_weight) {
    if (!out_weight) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_weight");
    return qmm::upload_from_host(type, gguf_blocks, gguf_bytes, n_rows, k_cols, nullptr, out_weight);
}

int openmini_qmm_upload_device(int type, const void* d_gguf_blocks, size_t gguf_bytes, int64_t n_rows,
                               int64_t k_cols, void* stream, openmini_qweight_t** out_weight) {
    if (!out_weight) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_weight");
    *out_weight = nullptr;
    int rc = validate_weight_args(type, gguf_bytes, n_rows, k_cols);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_gguf_blocks) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null d_gguf_blocks");
    int dev = 0;
    rc = ensure_device(&dev);
    if (rc != OPENMINI_QMM_OK) return rc;
    openmini_qweight* h = nullptr;
    rc = alloc_weight(type, n_rows, k_cols, dev, &h);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipError_t e = qmm::launch_repack(h->w, static_cast<const uint8_t*>(d_gguf_blocks), as_stream(stream));
    if (e != hipSuccess) {
        openmini_qmm_free_weight(h);
        return hip_fail(e, "repack launch");
    }
    *out_weight = h;
    return ok();
}

int openmini_qmm_weight_device_bytes(int type, int64_t n_rows, int64_t k_cols, size_t* out_bytes) {
    if (!out_bytes) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_bytes");
    *out_bytes = 0;
    const int rc = validate_weight_args(type, SIZE_MAX, n_rows, k_cols);  // the shape only
    if (rc != OPENMINI_QMM_OK) return rc;
    qmm::Weight w;
    plan_weight(type, n_rows, k_cols, 0, w);
    *out_bytes = w.device_bytes;
    return ok();
}

int openmini_qmm_upload_device_into(int type, const void* d_gguf_blocks, size_t gguf_bytes, int64_t n_rows,
                                    int64_t k_cols, void* d_weight_mem, size_t weight_mem_bytes, void* stream,
                                    openmini_qweight_t** out_weight) {
    if (!out_weight) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_weight");
    *out_weight = nullptr;
    int rc = validate_weight_args(type, gguf_bytes, n_rows, k_cols);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_gguf_blocks) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null d_gguf_blocks");
    if (!d_weight_mem || ((uintptr_t)d_weight_mem & 255u))
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "d_weight_mem must be a non-null 256-byte aligned device address");
    int dev = 0;
    rc = ensure_device(&dev);
    if (rc != OPENMINI_QMM_OK) return rc;
    openmini_qweight* h = new (std::nothrow) openmini_qweight();
    if (!h) return fail(OPENMINI_QMM_ERR_MEMORY, "host allocation failed");
    plan_weight(type, n_rows, k_cols, dev, h->w);
    if (weight_mem_bytes < h->w.device_bytes) {
        const size_t need = h->w.device_bytes;
        delete h;
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "weight memory of %zu bytes, %zu needed", weight_mem_bytes, need);
    }
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, d_weight_mem) != hipSuccess || attr.type != hipMemoryTypeDevice ||
        attr.device != dev) {
        (void)hipGetLastError();
        delete h;
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "d_weight_mem is not device memory of the current device %d", dev);
    }
    bind_weight(h->w, d_weight_mem);
    h->owns_memory = false;
    hipError_t e = qmm::launch_repack(h->w, static_cast<const uint8_t*>(d_gguf_blocks), as_stream(stream));
    if (e != hipSuccess) {
        delete h;
        return hip_fail(e, "repack launch");
    }
    *out_weight = h;
    return ok();
}

void openmini_qmm_free_weight(openmini_qweight_t* weight) {
    if (!weight) return;
    if (weight->w.chunks && weight->owns_memory) {
        int cur = 0;
        const bool switch_dev = hipGetDevice(&cur) == hipSuccess && cur != weight->w.device;
        if (switch_dev) (void)hipSetDevice(weight->w.device);
        (void)hipFree(weight->w.chunks);
        if (switch_dev) (void)hipSetDevice(cur);
    }
    delete weight;
}

int openmini_qmm_weight_info(const openmini_qweight_t* weight, openmini_qmm_weight_info_t* info) {
    if (!weight || !info) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null argument");
    const qmm::Weight& w = weight->w;
    info->type = w.src_type;
    info->device = w.device;
    info->n_rows = w.n;
    info->k_cols = w.k;
    info->blocks_per_row = w.nb;
    info->gguf_bytes =
        (size_t)w.n * (size_t)(w.k / qmm::weight_block_elems(w.src_type)) * qmm::bytes_per_block(w.src_type);
    info->device_bytes = w.device_bytes;
    return ok();
}

int openmini_qmm_gemv(const openmini_qweight_t* weight, const float* d_x, float* d_y, int64_t batch,
                      void* stream) {
    int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_x || !d_y) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x or y");
    if (batch <= 0) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "batch=%lld must be >= 1", (long long)batch);
    if (!aligned16(d_x)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "x must be 16-byte aligned");
    hipError_t e = qmm::launch_gemv_rows(weight->w, nullptr, d_x, d_y, batch, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "gemv launch");
    return ok();
}

int openmini_qmm_gemm_bf16(const openmini_qweight_t* weight, const uint16_t* d_x, float* d_y, int64_t m,
                           void* stream) {
    int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_x || !d_y) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x or y");
    if (m <= 0 || m > INT32_MAX) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "m=%lld out of range", (long long)m);
    if (!aligned16(d_x)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "x must be 16-byte aligned");
    rc = check_gemm_type(weight->w);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipError_t e = qmm::launch_gemm_bf16(weight->w, d_x, d_y, m, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "gemm launch");
    return ok();
}

int64_t openmini_qmm_gemm_min_rows(const openmini_qweight_t* weight) {
    const int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    const qmm::Weight& w = weight->w;
    return qmm::has_block_min(w.type) ? 0 : qmm::gemm_min_rows(w.type, w.n, w.k);
}

int openmini_qmm_gemm_launch_shape(const openmini_qweight_t* weight, int64_t m, int split_x) {
    int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (m <= 0 || m > INT32_MAX) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "m=%lld out of range", (long long)m);
    const int shape = qmm::gemm_shape(weight->w, m, split_x != 0);
    if (shape < 0) return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "no prefill GEMM for type %d", weight->w.type);
    return shape;
}

size_t openmini_qmm_gemm_f32_workspace_bytes(int64_t m, int64_t k_cols) {
    if (m <= 0 || k_cols <= 0 || m > INT32_MAX || k_cols > INT32_MAX / 2) return 0;
    return qmm::gemm_f32_workspace_bytes(m, k_cols);
}

namespace {
// Shared checks of the fp32-activation GEMM entry points.
int check_f32_gemm_args(const qmm::Weight& w, const float* d_x, const void* d_out, int64_t m, const void* d_work,
                        size_t work_bytes) {
    const int rc = check_gemm_type(w);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_x || !d_out || !d_work) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x, output or workspace");
    if (m <= 0 || m > INT32_MAX) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "m=%lld out of range", (long long)m);
    if (!aligned16(d_x)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "x must be 16-byte aligned");
    if (((uintptr_t)d_work & 255u) != 0) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "workspace must be 256-byte aligned");
    const size_t need = qmm::gemm_f32_workspace_bytes(m, w.k);
    if (work_bytes < need)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "workspace of %zu bytes, %zu needed for m=%lld, K=%lld", work_bytes,
                    need, (long long)m, (long long)w.k);
    return OPENMINI_QMM_OK;
}
}  // namespace

int openmini_qmm_gemm_f32(const openmini_qweight_t* weight, const float* d_x, float* d_y, int64_t m, void* d_work,
                          size_t work_bytes, void* stream) {
    int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    rc = check_f32_gemm_args(weight->w, d_x, d_y, m, d_work, work_bytes);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipError_t e = qmm::split_rows(d_x, m, weight->w.k, d_work, as_stream(stream));
    if (e == hipSuccess) e = qmm::launch_gemm_split(weight->w, d_work, m, d_y, as_stream(stream), false);
    if (e != hipSuccess) return hip_fail(e, "gemm_f32 launch");
    return ok();
}

int openmini_qmm_gemv_multi(const openmini_qweight_t* const* weights, int count, const float* d_x,
                            float* const* d_ys, int64_t batch, void* stream) {
    if (!weights || !d_ys) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null weights or outputs");
    if (count < 1 || count > qmm::kMaxGroup)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "count=%d must be in [1, %d]", count, qmm::kMaxGroup);
    const qmm::Weight* ws[qmm::kMaxGroup];
    for (int i = 0; i < count; ++i) {
        int rc = check_weight(weights[i]);
        if (rc != OPENMINI_QMM_OK) return rc;
        if (!d_ys[i]) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null output %d", i);
        ws[i] = &weights[i]->w;
        if (ws[i]->type != ws[0]->type || ws[i]->k != ws[0]->k || ws[i]->device != ws[0]->device)
            return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "weight %d differs from weight 0 in type, K or device", i);
    }
    if (!d_x) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x");
    if (batch <= 0) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "batch=%lld must be >= 1", (long long)batch);
    if (!aligned16(d_x)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "x must be 16-byte aligned");
    int64_t tiles = 0;
    for (int i = 0; i < count; ++i) tiles += ws[i]->n_tiles;
    if (tiles > INT32_MAX) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "too many rows in one group");
    const int64_t k = ws[0]->k;
    if (qmm::use_batch_kernel(*ws[0], batch)) {
        // several rows: one batched pass per weight
        for (int i = 0; i < count; ++i) {
            hipError_t e = qmm::launch_gemv_rows(*ws[i], nullptr, d_x, d_ys[i], batch, as_stream(stream));
            if (e != hipSuccess) return hip_fail(e, "gemv_multi launch");
        }
        return ok();
    }
    for (int64_t b0 = 0; b0 < batch; b0 += qmm::kMaxGemvBatch) {
        const int nb = (int)((batch - b0) < qmm::kMaxGemvBatch ? (batch - b0) : qmm::kMaxGemvBatch);
        float* ys[qmm::kMaxGroup];
        for (int i = 0; i < count; ++i) ys[i] = d_ys[i] + b0 * ws[i]->n;
        hipError_t e = qmm::launch_gemv_group(ws, ys, count, d_x + b0 * k, nb, false, as_stream(stream));
        if (e != hipSuccess) return hip_fail(e, "gemv_multi launch");
    }
    return ok();
}

static int check_pair(const openmini_qweight_t* gate, const openmini_qweight_t* up) {
    int rc = check_weight(gate);
    if (rc == OPENMINI_QMM_OK) rc = check_weight(up);
    if (rc != OPENMINI_QMM_OK) return rc;
    const qmm::Weight &g = gate->w, &u = up->w;
    if (g.type != u.type || g.n != u.n || g.k != u.k || g.device != u.device)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM,
                    "gate [%lld, %lld] and up [%lld, %lld] differ in shape, type or device", (long long)g.n,
                    (long long)g.k, (long long)u.n, (long long)u.k);
    return OPENMINI_QMM_OK;
}

int openmini_qmm_ffn_gate_up(const openmini_qweight_t* gate, const openmini_qweight_t* up, const float* d_x,
                             float* d_h, int64_t batch, void* stream) {
    int rc = check_pair(gate, up);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_x || !d_h) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x or h");
    if (batch <= 0) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "batch=%lld must be >= 1", (long long)batch);
    if (!aligned16(d_x)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "x must be 16-byte aligned");
    hipError_t e = qmm::launch_gemv_rows(gate->w, &up->w, d_x, d_h, batch, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "ffn_gate_up launch");
    return ok();
}

int openmini_qmm_ffn_gate_up_bf16(const openmini_qweight_t* gate, const openmini_qweight_t* up,
                                  const uint16_t* d_x, float* d_h, int64_t m, void* stream) {
    int rc = check_pair(gate, up);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_x || !d_h) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x or h");
    if (m <= 0 || m > INT32_MAX) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "m=%lld out of range", (long long)m);
    if (!aligned16(d_x)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "x must be 16-byte aligned");
    rc = check_gemm_type(gate->w);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipError_t e = qmm::launch_gemm_bf16(gate->w, d_x, d_h, m, as_stream(stream), false);
    if (e == hipSuccess) e = qmm::launch_gemm_bf16(up->w, d_x, d_h, m, as_stream(stream), true);
    if (e != hipSuccess) return hip_fail(e, "ffn_gate_up_bf16 launch");
    return ok();
}

int openmini_qmm_ffn_gate_up_f32(const openmini_qweight_t* gate, const openmini_qweight_t* up, const float* d_x,
                                 float* d_h, int64_t m, void* d_work, size_t work_bytes, void* stream) {
    int rc = check_pair(gate, up);
    if (rc != OPENMINI_QMM_OK) return rc;
    rc = check_f32_gemm_args(gate->w, d_x, d_h, m, d_work, work_bytes);
    if (rc != OPENMINI_QMM_OK) return rc;
    // one split of x for both weights; the up GEMM finishes silu(gate) * up
    hipError_t e = qmm::split_rows(d_x, m, gate->w.k, d_work, as_stream(stream));
    if (e == hipSuccess) e = qmm::launch_gemm_split(gate->w, d_work, m, d_h, as_stream(stream), false);
    if (e == hipSuccess) e = qmm::launch_gemm_split(up->w, d_work, m, d_h, as_stream(stream), true);
    if (e != hipSuccess) return hip_fail(e, "ffn_gate_up_f32 launch");
    return ok();
}

namespace {
// linear(x, W) on device buffers: the decode GEMVs below qmm::gemm_min_rows rows (and for
// block-minimum types at any count), else the fp32-activation prefill GEMM (its
// workspace at d_work).
hipError_t linear_rows(const qmm::Weight& w, const float* dx, float* dy, int64_t m, void* d_work) {
    if (gemm_rows(w, m)) {
        hipError_t e = qmm::split_rows(dx, m, w.k, d_work, nullptr);
        return e == hipSuccess ? qmm::launch_gemm_split(w, d_work, m, dy, nullptr, false) : e;
    }
    return qmm::launch_gemv_rows(w, nullptr, dx, dy, m, nullptr);
}
}  // namespace

int openmini_qmm_linear_host(const openmini_qweight_t* weight, const float* x, float* y, int64_t m) {
    int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!x || !y) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x or y");
    if (m <= 0) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "m=%lld must be >= 1", (long long)m);
    const qmm::Weight& w = weight->w;
    std::unique_lock<std::mutex> lk(weight->batch_mu, std::defer_lock);
    if (w.split_s > 1 && !gemm_rows(w, m) && qmm::use_batch_kernel(w, m)) lk.lock();
    if (m > INT32_MAX) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "m=%lld out of range", (long long)m);
    const size_t xb = round_up((size_t)m * w.k * sizeof(float), 256), yb = (size_t)m * w.n * sizeof(float);
    const size_t wb = gemm_rows(w, m) ? qmm::gemm_f32_workspace_bytes(m, w.k) : 0;
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, xb + wb + yb);
    if (e != hipSuccess) return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc for linear_host failed: %s", hipGetErrorString(e));
    float* dx = static_cast<float*>(base);
    uint8_t* work = static_cast<uint8_t*>(base) + xb;
    float* dy = reinterpret_cast<float*>(work + wb);
    e = hipMemcpy(dx, x, (size_t)m * w.k * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = linear_rows(w, dx, dy, m, work);
    if (e == hipSuccess) e = hipMemcpy(y, dy, yb, hipMemcpyDeviceToHost);
    (void)hipFree(base);
    if (e != hipSuccess) return hip_fail(e, "linear_host");
    return ok();
}

int openmini_qmm_linear_host_noalloc(const openmini_qweight_t* weight, const float* x, float* y, int64_t m) {
    int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!x || !y) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null x or y");
    if (m <= 0) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "m=%lld must be >= 1", (long long)m);
    const qmm::Weight& w = weight->w;
    // staging: x, the GEMM's workspace (where gemm_rows), y, each 256-aligned
    auto staged_bytes = [&](int64_t rows) {
        const size_t wb = gemm_rows(w, rows) ? qmm::gemm_f32_workspace_bytes(rows, w.k) : 0;
        return round_up((size_t)rows * w.k * sizeof(float), 256) + wb + (size_t)rows * w.n * sizeof(float);
    };
    if (m > INT32_MAX || staged_bytes(m) > kScratchBytes) {
        int64_t rows_max = 0;  // the largest accepted m (staged_bytes grows with m)
        for (int64_t step = (int64_t)1 << 30; step > 0; step >>= 1)
            if (staged_bytes(rows_max + step) <= kScratchBytes) rows_max += step;
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM,
                    "linear_host_noalloc: m=%lld rows of x[K=%lld] and y[N=%lld] need more than the %zu-byte "
                    "staging (at most %lld rows for this weight)",
                    (long long)m, (long long)w.k, (long long)w.n, kScratchBytes, (long long)rows_max);
    }
    uint8_t* base = nullptr;
    rc = scratch_on_device(w.device, &base);
    if (rc != OPENMINI_QMM_OK) return rc;
    std::lock_guard<std::mutex> staging(g_staging_mu[w.device]);
    std::unique_lock<std::mutex> lk(weight->batch_mu, std::defer_lock);
    if (w.split_s > 1 && !gemm_rows(w, m) && qmm::use_batch_kernel(w, m)) lk.lock();
    const size_t xb = round_up((size_t)m * w.k * sizeof(float), 256), yb = (size_t)m * w.n * sizeof(float);
    const size_t wb = gemm_rows(w, m) ? qmm::gemm_f32_workspace_bytes(m, w.k) : 0;
    float* dx = reinterpret_cast<float*>(base);
    uint8_t* work = base + xb;
    float* dy = reinterpret_cast<float*>(work + wb);
    hipError_t e = hipMemcpy(dx, x, (size_t)m * w.k * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = linear_rows(w, dx, dy, m, work);
    if (e == hipSuccess) e = hipMemcpy(y, dy, yb, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "linear_host_noalloc");
    return ok();
}

int openmini_qmm_dequant_weight(const openmini_qweight_t* weight, float* d_out, void* stream) {
    int rc = check_weight(weight);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (!d_out) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out");
    if (!aligned16(d_out)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "out must be 16-byte aligned");
    if (!plain_type(weight->w.type))
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED,
                    "dequant_weight takes Q4_0, Q8_0 and Q8_K weights (K-quant bytes: openmini_qmm_dequantize_any_device)");
    hipError_t e = qmm::launch_dequant_weight(weight->w, d_out, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return ok();
}

static int validate_dequant(int type, size_t gguf_bytes, size_t n, size_t* expected_bytes) {
    if (expected_bytes) *expected_bytes = 0;
    if (!safe_type(type))
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "UnsupportedType(%d)", type);
    const int rc = check_elements(n);
    if (rc != OPENMINI_QMM_OK) return rc;
    const size_t need = layout_bytes(type, n);
    if (gguf_bytes < need) {
        if (expected_bytes) *expected_bytes = need;
        return fail(OPENMINI_QMM_ERR_INSUFFICIENT_DATA, "InsufficientData: expected %zu bytes, actual %zu",
                    need, gguf_bytes);
    }
    return OPENMINI_QMM_OK;
}

int openmini_qmm_dequantize_device(int type, const void* d_gguf, size_t gguf_bytes, size_t n, float* d_out,
                                   void* stream, size_t* expected_bytes) {
    int rc = validate_dequant(type, gguf_bytes, n, expected_bytes);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (n == 0) return ok();
    if (!d_gguf || !d_out) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipError_t e = qmm::launch_dequant_layout(type, static_cast<const uint8_t*>(d_gguf), gguf_bytes, n, d_out,
                                              as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    return ok();
}

int openmini_qmm_dequantize(int type, const void* gguf, size_t gguf_bytes, size_t n, float* out,
                            size_t* expected_bytes) {
    int rc = validate_dequant(type, gguf_bytes, n, expected_bytes);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (n == 0) return ok();
    if (!gguf || !out) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    const size_t need = layout_bytes(type, n);
    void *din = nullptr, *dout = nullptr;
    hipError_t e = hipMalloc(&din, need);
    if (e == hipSuccess) e = hipMalloc(&dout, n * sizeof(float));
    if (e != hipSuccess) {
        (void)hipFree(din);
        return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc for dequantize failed: %s", hipGetErrorString(e));
    }
    e = hipMemcpy(din, gguf, need, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = qmm::launch_dequant_layout(type, static_cast<const uint8_t*>(din), need, n, static_cast<float*>(dout),
                                       nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, dout, n * sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(din);
    (void)hipFree(dout);
    if (e != hipSuccess) return hip_fail(e, "dequantize");
    return ok();
}

int openmini_qmm_dequantize_any_device(int type, const void* d_gguf, size_t gguf_bytes, size_t n, float* d_out,
                                       void* stream) {
    if (!qmm::layout_block_size(type))
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "tensor type %d is not implemented", type);
    int rc = check_elements(n);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (n == 0) return ok();
    if (!d_out || (!d_gguf && gguf_bytes)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    const size_t used = std::min(gguf_bytes, layout_bytes(type, n));
    hipError_t e = qmm::launch_dequant_layout(type, static_cast<const uint8_t*>(d_gguf), used, n, d_out,
                                              as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    return ok();
}

int openmini_qmm_dequantize_any(int type, const void* gguf, size_t gguf_bytes, size_t n, float* out) {
    if (!qmm::layout_block_size(type))
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "tensor type %d is not implemented", type);
    int rc = check_elements(n);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (n == 0) return ok();
    if (!out || (!gguf && gguf_bytes)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    const size_t used = std::min(gguf_bytes, layout_bytes(type, n));
    void *din = nullptr, *dout = nullptr;
    hipError_t e = hipMalloc(&din, used ? used : 1);
    if (e == hipSuccess) e = hipMalloc(&dout, n * sizeof(float));
    if (e != hipSuccess) {
        (void)hipFree(din);
        return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc for dequantize failed: %s", hipGetErrorString(e));
    }
    if (used) e = hipMemcpy(din, gguf, used, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = qmm::launch_dequant_layout(type, static_cast<const uint8_t*>(din), used, n, static_cast<float*>(dout),
                                       nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, dout, n * sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(din);
    (void)hipFree(dout);
    if (e != hipSuccess) return hip_fail(e, "dequantize");
    return ok();
}

// GgufTensorType ids (gguf.rs:219-276): 0..29 except 6 and 9.
static bool gguf_type_id(int t) { return t >= 0 && t <= 29 && t != 6 && t != 9; }

int openmini_qmm_soa_bytes(int type, size_t len, size_t n, size_t* out_bytes) {
    if (!out_bytes) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_bytes");
    *out_bytes = 0;
    if (!gguf_type_id(type)) return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "unknown tensor type %d", type);
    const int rc = check_elements(n);
    if (rc != OPENMINI_QMM_OK) return rc;
    *out_bytes = qmm::soa_bytes(type, len, n);
    return ok();
}

int openmini_qmm_convert_to_soa_device(int type, const void* d_data, size_t len, size_t n, void* d_out,
                                       void* stream) {
    size_t total = 0;
    int rc = openmini_qmm_soa_bytes(type, len, n, &total);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (total == 0) return ok();
    if (!d_data || !d_out) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipError_t e = qmm::launch_convert_to_soa(type, static_cast<const uint8_t*>(d_data), len, n,
                                              static_cast<uint8_t*>(d_out), as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "convert_to_soa launch");
    return ok();
}

int openmini_qmm_convert_to_soa(int type, const void* data, size_t len, size_t n, void* out) {
    size_t total = 0;
    int rc = openmini_qmm_soa_bytes(type, len, n, &total);
    if (rc != OPENMINI_QMM_OK) return rc;
    if (total == 0) return ok();
    if (!data || !out) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    void *din = nullptr, *dout = nullptr;
    hipError_t e = hipMalloc(&din, len);
    if (e == hipSuccess) e = hipMalloc(&dout, total);
    if (e != hipSuccess) {
        (void)hipFree(din);
        return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc for convert_to_soa failed: %s", hipGetErrorString(e));
    }
    e = hipMemcpy(din, data, len, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = qmm::launch_convert_to_soa(type, static_cast<const uint8_t*>(din), len, n, static_cast<uint8_t*>(dout),
                                       nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, dout, total, hipMemcpyDeviceToHost);
    (void)hipFree(din);
    (void)hipFree(dout);
    if (e != hipSuccess) return hip_fail(e, "convert_to_soa");
    return ok();
}

int openmini_qmm_malloc(void** d_ptr, size_t bytes) {
    if (!d_ptr) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null d_ptr");
    *d_ptr = nullptr;
    int rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipError_t e = hipMalloc(d_ptr, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(OPENMINI_QMM_ERR_MEMORY, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return ok();
}

int openmini_qmm_free(void* d_ptr) {
    if (!d_ptr) return ok();
    HIP_TRY(hipFree(d_ptr), "hipFree");
    return ok();
}

int openmini_qmm_memcpy_h2d(void* d_dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return ok();
    if (!d_dst || !src) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    HIP_TRY(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "hipMemcpyAsync H2D");
    HIP_TRY(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    return ok();
}

int openmini_qmm_memcpy_d2h(void* dst, const void* d_src, size_t bytes, void* stream) {
    if (bytes == 0) return ok();
    if (!dst || !d_src) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    HIP_TRY(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "hipMemcpyAsync D2H");
    HIP_TRY(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    return ok();
}

int openmini_qmm_memset(void* d_dst, int value, size_t bytes, void* stream) {
    if (bytes == 0) return ok();
    if (!d_dst) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    HIP_TRY(hipMemsetAsync(d_dst, value, bytes, as_stream(stream)), "hipMemsetAsync");
    return ok();
}

int openmini_qmm_stream_create(void** out_stream) {
    if (!out_stream) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null out_stream");
    int rc = ensure_device(nullptr);
    if (rc != OPENMINI_QMM_OK) return rc;
    hipStream_t s = nullptr;
    HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *out_stream = s;
    return ok();
}

int openmini_qmm_stream_destroy(void* stream) {
    if (!stream) return ok();
    HIP_TRY(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
    return ok();
}

int openmini_qmm_stream_synchronize(void* stream) {
    HIP_TRY(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    return ok();
}

int openmini_qmm_stream_copy(void* d_dst, const void* d_src, size_t bytes, void* stream) {
    if (!d_dst || !d_src) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    if (bytes % 16 || !aligned16(d_dst) || !aligned16(d_src))
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "stream_copy needs 16-byte sizes and alignment");
    hipError_t e = qmm::launch_stream_copy(d_dst, d_src, bytes, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "stream_copy launch");
    return ok();
}

int openmini_qmm_stream_read(const void* d_src, size_t bytes, void* d_sink, void* stream) {
    if (!d_src || !d_sink) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null pointer");
    if (bytes % 16 || !aligned16(d_src) || ((uintptr_t)d_sink & 3u))
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "stream_read needs 16-byte sizes and source alignment");
    hipError_t e = qmm::launch_stream_read(d_src, bytes, static_cast<uint32_t*>(d_sink), as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "stream_read launch");
    return ok();
}

int openmini_qmm_gemm_ceiling(int type, int64_t m, int64_t n, int64_t k, void* d_sink, void* stream) {
    if (!d_sink || ((uintptr_t)d_sink & 3u)) return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "null or unaligned sink");
    if (!plain_type(type))
        return fail(OPENMINI_QMM_ERR_UNSUPPORTED, "gemm_ceiling takes Q4_0 and Q8_0, not type %d", type);
    if (m <= 0 || n <= 0 || k <= 0 || k % 32 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
        return fail(OPENMINI_QMM_ERR_INVALID_PARAM, "gemm_ceiling sizes m=%lld n=%lld k=%lld", (long long)m,
                    (long long)n, (long long)k);
    hipError_t e = qmm::launch_gemm_ceiling(type, m, n, k, static_cast<float*>(d_sink), as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "gemm_ceiling launch");
    return ok();
}

}  // extern "C"
