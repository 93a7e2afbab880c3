/* A plain-C consumer of libopenmini_qmm.so, compiled with gcc against
 * include/openmini_qmm.h only: what a Rust / cgo / JNI binding of the C-ABI links
 * to.  Test code, built and run by tests/test_c_consumer.py.
 *
 *   c_consumer host     argument validation, error codes, last-error text and the
 *                       log callback (no device needed)
 *   c_consumer device   upload a Q4_0 weight from host GGUF blocks, run the decode
 *                       GEMV on device buffers (3 and 8 activation rows), compare with a C reference of
 *                       quant::dequantize_q4_0 (openmini-server/src/model/inference/
 *                       quant.rs:152-195) and linear() (model.rs:1050-1064)
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "openmini_qmm.h"

static int g_logged = 0;
static void on_log(int level, const char *text, void *user) {
    (void)user;
    if (level == OPENMINI_QMM_LOG_ERROR && text && text[0]) ++g_logged;
}

#define CHECK(cond)                                                  \
    do {                                                             \
        if (!(cond)) {                                               \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            return 1;                                                \
        }                                                            \
    } while (0)

static int host_checks(void) {
    size_t bytes = 0;
    CHECK(strlen(openmini_qmm_version()) > 0);
    CHECK(openmini_qmm_required_bytes(OPENMINI_QMM_Q4_0, 4096 * 11008, &bytes) == OPENMINI_QMM_OK);
    CHECK(bytes == 25362432u);
    CHECK(openmini_qmm_set_log_callback(on_log, NULL) == OPENMINI_QMM_OK);
    openmini_qweight_t *w = NULL;
    uint8_t buf[64] = {0};
    /* K not a multiple of 32 */
    CHECK(openmini_qmm_upload(OPENMINI_QMM_Q4_0, buf, sizeof buf, 1, 48, &w) == OPENMINI_QMM_ERR_INVALID_PARAM);
    CHECK(w == NULL && strstr(openmini_qmm_last_error(), "multiple of 32") != NULL);
    /* InsufficientData{expected 36, actual 20} */
    CHECK(openmini_qmm_upload(OPENMINI_QMM_Q4_0, buf, 20, 1, 64, &w) == OPENMINI_QMM_ERR_INSUFFICIENT_DATA);
    CHECK(strstr(openmini_qmm_last_error(), "expected 36") != NULL);
    CHECK(g_logged == 2);
    CHECK(openmini_qmm_set_log_callback(NULL, NULL) == OPENMINI_QMM_OK);
    printf("host ok\n");
    return 0;
}

/* fp16 bits -> float (normal and zero values only; the generator makes no others) */
static float f16_to_f32(uint16_t h) {
    const int e = (h >> 10) & 0x1F, m = h & 0x3FF;
    const float v = e ? ldexpf(1.0f + m / 1024.0f, e - 15) : ldexpf(m / 1024.0f, -14);
    return (h & 0x8000) ? -v : v;
}

static int device_checks(const int B) {
    enum { N = 80, K = 256 };
    const int nb = K / 32;
    uint8_t *blocks = malloc((size_t)N * nb * 18);
    float *x = malloc(sizeof(float) * B * K), *y = malloc(sizeof(float) * B * N);
    CHECK(blocks && x && y);
    uint32_t s = 12345u;
    for (int i = 0; i < N * nb; ++i) {
        uint8_t *b = blocks + (size_t)i * 18;
        const uint16_t d = (uint16_t)(0x1C00 + (i * 37) % 0x0800); /* fp16 in [2^-8, 2^-7) */
        b[0] = (uint8_t)(d & 0xFF);
        b[1] = (uint8_t)(d >> 8);
        for (int j = 0; j < 16; ++j) {
            s = s * 1664525u + 1013904223u;
            b[2 + j] = (uint8_t)(s >> 24);
        }
    }
    for (int i = 0; i < B * K; ++i) {
        s = s * 1664525u + 1013904223u;
        x[i] = (float)((int)(s >> 16) % 2001 - 1000) / 500.0f;
    }
    CHECK(openmini_qmm_init(0) == OPENMINI_QMM_OK);
    openmini_qweight_t *w = NULL;
    CHECK(openmini_qmm_upload(OPENMINI_QMM_Q4_0, blocks, (size_t)N * nb * 18, N, K, &w) == OPENMINI_QMM_OK);
    void *dx = NULL, *dy = NULL, *stream = NULL;
    CHECK(openmini_qmm_stream_create(&stream) == OPENMINI_QMM_OK);
    CHECK(openmini_qmm_malloc(&dx, sizeof(float) * B * K) == OPENMINI_QMM_OK);
    CHECK(openmini_qmm_malloc(&dy, sizeof(float) * B * N) == OPENMINI_QMM_OK);
    CHECK(openmini_qmm_memcpy_h2d(dx, x, sizeof(float) * B * K, stream) == OPENMINI_QMM_OK);
    CHECK(openmini_qmm_gemv(w, dx, dy, B, stream) == OPENMINI_QMM_OK);
    CHECK(openmini_qmm_memcpy_d2h(y, dy, sizeof(float) * B * N, stream) == OPENMINI_QMM_OK);
    CHECK(openmini_qmm_stream_synchronize(stream) == OPENMINI_QMM_OK);
    /* reference: element 2j of a block = high nibble of byte j, 2j+1 = low nibble */
    double worst = 0.0, scale = 0.0;
    for (int r = 0; r < B; ++r)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int blk = 0; blk < nb; ++blk) {
                const uint8_t *b = blocks + ((size_t)n * nb + blk) * 18;
                const float d = f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
                for (int i = 0; i < 32; ++i) {
                    const uint8_t byte = b[2 + i / 2];
                    const int q = (i % 2 == 0) ? (byte >> 4) : (byte & 0x0F);
                    acc += (double)((float)(q - 8) * d) * x[r * K + blk * 32 + i];
                }
            }
            const double err = fabs(acc - y[r * N + n]);
            if (err > worst) worst = err;
            if (fabs(acc) > scale) scale = fabs(acc);
        }
    printf("device batch %d normwise error %.3g\n", B, worst / scale);
    CHECK(worst <= 1e-3 * scale);
    openmini_qmm_free(dx);
    openmini_qmm_free(dy);
    openmini_qmm_stream_destroy(stream);
    openmini_qmm_free_weight(w);
    free(blocks);
    free(x);
    free(y);
    printf("device ok\n");
    return 0;
}

int main(int argc, char **argv) {
    /* 3 rows: the int8 decode kernel; 8 rows: the batched kernel */
    if (argc > 1 && strcmp(argv[1], "device") == 0) return device_checks(3) || device_checks(8);
    return host_checks();
}
