/*
 * CPU oracle of qwenny's quantized-weight matrix products — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's semantics for this path, used by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker. The product library never links, loads or calls it. Every function
 * cites the reference file:line it follows (paths relative to the reference repository).
 *
 * Pinning (what checks each function against something other than itself) is listed per function; the tests in
 * tests/test_oracle.py hold those checks.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* bf16 bits -> f32 (checkpoint.rs:188 float_format BF16: the bits shifted up 16) */
static float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/*
 * Checkpoint::packed_matrix (src/checkpoint.rs:408-453): compressed-tensors pack-quantized -> Quant.
 * Returns 0 on success, -1 if the zero-point shape fits neither packing. Writes bits, group and cols.
 * Pinned by: hand-built words with known values; zero points packed along rows and along groups.
 */
EXPORT int or_packed_matrix(const uint32_t* packed, size_t rows, size_t words, size_t cols_in, int bits_cfg,
                            int group_cfg, const float* scale, const uint32_t* zp, size_t zp_rows, size_t zp_cols,
                            float* scales, float* offsets, int* bits_out, size_t* group_out, size_t* cols_out) {
    size_t cols = cols_in ? cols_in : words * 32 / (size_t)bits_cfg;                  /* :411 */
    int bits = (words * 32) % cols == 0 ? (int)(words * 32 / cols) : bits_cfg;         /* :413 */
    if ((bits != 4 && bits != 8) || cols != words * 32 / (size_t)bits) return -1;    /* :414-419 */
    size_t group = group_cfg == 0 ? cols : (size_t)group_cfg;                          /* :420 */
    if (cols % group) return -1;
    size_t groups = cols / group, per = 32 / (size_t)bits;
    uint32_t mask = (1u << bits) - 1;
    int along_rows = 0;
    if (zp) {
        along_rows = zp_rows == (rows + per - 1) / per && zp_cols == groups;           /* :436 */
        if (!along_rows && !(zp_rows == rows && zp_cols == (groups + per - 1) / per)) return -1;
    }
    for (size_t r = 0; r < rows; r++)
        for (size_t g = 0; g < groups; g++) {
            size_t i = r * groups + g;
            float z;
            if (!zp)
                z = (float)(1 << (bits - 1));                                           /* :430 */
            else if (along_rows)
                z = (float)((zp[(r / per) * groups + g] >> ((r % per) * bits)) & mask); /* :445 */
            else
                z = (float)((zp[r * zp_cols + g / per] >> ((g % per) * bits)) & mask);  /* :447 */
            scales[i] = scale[i];
            offsets[i] = -scale[i] * z;                                                 /* :451 */
        }
    *bits_out = bits;
    *group_out = group;
    *cols_out = cols;
    return 0;
}

/*
 * Quant::row_into (src/checkpoint.rs:39-47): w = v * scale + offset in f32.
 * Pinned by: known codes/scales with exact results; symmetric offset gives (q - 8) s.
 */
EXPORT void or_row_into(int bits, size_t group, size_t cols, const uint32_t* q, const float* scales,
                        const float* offsets, size_t r, float* out) {
    size_t per = 32 / (size_t)bits, words = cols * (size_t)bits / 32, groups = cols / group;
    uint32_t mask = (1u << bits) - 1;
    const uint32_t* w = q + r * words;
    for (size_t c = 0; c < cols; c++) {
        uint32_t v = (w[c / per] >> ((c % per) * (size_t)bits)) & mask;
        size_t g = r * groups + c / group;
        out[c] = (float)v * scales[g] + offsets[g];
    }
}

/*
 * Quant::zero_points (src/checkpoint.rs:72-82). Returns 1 and fills z if all integer, else 0.
 * Pinned by: symmetric -> all 2^(bits-1); stored zero points recovered; a non-integer offset (beyond 1e-3) -> none.
 */
EXPORT int or_zero_points(int bits, size_t n, const float* scales, const float* offsets, uint8_t* z) {
    float max = (float)((1u << bits) - 1);
    for (size_t i = 0; i < n; i++) {
        float s = scales[i], o = offsets[i];
        float v = s == 0.0f ? 0.0f : -o / s;
        float r = roundf(v);
        if (!(r >= 0.0f && r <= max && fabsf(v - r) < 1e-3f)) return 0;
        z[i] = (uint8_t)r;
    }
    return 1;
}

/*
 * row_order (src/cuda/core.rs:108-114). Pinned by: its closed form on 32 rows written out by hand, bijection.
 */
EXPORT void or_row_order(size_t rows, int silu, size_t* out) {
    for (size_t i = 0; i < rows; i++) out[i] = silu ? (i / 16) * 8 + i % 8 + (i % 16 >= 8 ? rows / 2 : 0) : i;
}

/*
 * Mat::new / pack int8 branch (src/cuda/core.rs:356-369): per row and 128 columns, scale = max|w| / 127 (1 if 0),
 * q = round(w / scale) (half away from zero, Rust f32::round) clamped to +-127, stored q + 128.
 * vals [rows][cols] stored values, scales [rows][cols / 128]. Rows in their own order (the layout is not the oracle's
 * concern). Pinned by: ties 2.5 -> 3 and -2.5 -> -3, an all-zero group (scale 1), clamping, max element -> +-127.
 */
EXPORT void or_requant_int8(const uint16_t* bf16, size_t rows, size_t cols, uint8_t* vals, float* scales) {
    size_t groups = cols / 128;
    for (size_t r = 0; r < rows; r++)
        for (size_t g = 0; g < groups; g++) {
            const uint16_t* src = bf16 + r * cols + g * 128;
            float m = 0.0f;
            for (int c = 0; c < 128; c++) {
                float a = fabsf(bf16f(src[c]));
                m = a > m ? a : m;
            }
            float s = m > 0.0f ? m / 127.0f : 1.0f;
            scales[r * groups + g] = s;
            for (int c = 0; c < 128; c++) {
                float v = roundf(bf16f(src[c]) / s);
                if (isnan(v)) v = 0.0f;
                if (v < -127.0f) v = -127.0f;
                if (v > 127.0f) v = 127.0f;
                vals[r * cols + g * 128 + c] = (uint8_t)((int)v + 128);
            }
        }
}

/* ---- products ------------------------------------------------------------------------------------------------ */

typedef struct {
    int bits;
    size_t group, rows, cols, m;
    const uint32_t* q;
    const float* scales;
    const float* offsets;
    const uint16_t* x; /* bf16 [m][cols] */
    void* y;           /* [m][rows] */
    size_t r0, r1;
    int f32;
} gemm_job;

static void* gemm_rows(void* arg) {
    gemm_job* j = (gemm_job*)arg;
    size_t cols = j->cols;
    float* w32 = (float*)malloc(cols * sizeof(float));
    double* w64 = (double*)malloc(cols * sizeof(double));
    float* x32 = (float*)malloc(j->m * cols * sizeof(float));
    for (size_t i = 0; i < j->m * cols; i++) x32[i] = bf16f(j->x[i]);
    size_t per = 32 / (size_t)j->bits, words = cols * (size_t)j->bits / 32, groups = cols / j->group;
    uint32_t mask = (1u << j->bits) - 1;
    for (size_t r = j->r0; r < j->r1; r++) {
        if (j->f32) {
            /* the reference's CPU form: the row dequantized to f32 (Quant::row_into), then a plain f32 dot */
            or_row_into(j->bits, j->group, cols, j->q, j->scales, j->offsets, r, w32);
            for (size_t t = 0; t < j->m; t++) {
                const float* xt = x32 + t * cols;
                float acc = 0.0f;
                for (size_t c = 0; c < cols; c++) acc += w32[c] * xt[c];
                ((float*)j->y)[t * j->rows + r] = acc;
            }
        } else {
            /* exact: w = v s + offset = (q - z) s in f64, products and sums in f64 */
            const uint32_t* wr = j->q + r * words;
            for (size_t c = 0; c < cols; c++) {
                uint32_t v = (wr[c / per] >> ((c % per) * (size_t)j->bits)) & mask;
                size_t g = r * groups + c / j->group;
                w64[c] = (double)v * (double)j->scales[g] + (double)j->offsets[g];
            }
            for (size_t t = 0; t < j->m; t++) {
                const float* xt = x32 + t * cols;
                double acc = 0.0;
                for (size_t c = 0; c < cols; c++) acc += w64[c] * (double)xt[c];
                ((double*)j->y)[t * j->rows + r] = acc;
            }
        }
    }
    free(w32);
    free(w64);
    free(x32);
    return NULL;
}

static void gemm(int bits, size_t group, size_t rows, size_t cols, const uint32_t* q, const float* scales,
                 const float* offsets, const uint16_t* x, size_t m, void* y, int threads, int f32) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = (int)rows;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    gemm_job* jobs = (gemm_job*)malloc(sizeof(gemm_job) * (size_t)threads);
    size_t per = (rows + (size_t)threads - 1) / (size_t)threads;
    int started = 0;
    for (int i = 0; i < threads; i++) {
        size_t r0 = (size_t)i * per, r1 = r0 + per > rows ? rows : r0 + per;
        if (r0 >= r1) break;
        jobs[i] = (gemm_job){bits, group, rows, cols, m, q, scales, offsets, x, y, r0, r1, f32};
        if (threads == 1)
            gemm_rows(&jobs[i]);
        else
            pthread_create(&th[started++], NULL, gemm_rows, &jobs[i]);
    }
    for (int i = 0; i < started; i++) pthread_join(th[i], NULL);
    free(th);
    free(jobs);
}

/*
 * The dequantize-then-matmul semantics of every product (Quant::row_into, src/checkpoint.rs:39-47, as the kernels
 * compute it: kernels/marlin.cuh:102-133, kernels/gemm.cuh:176-200, kernels/qwen_train.cu:84-103):
 * y[t][r] = sum_c x[t][c] ((q - z) s) in f64, x bf16 taken as given. y f64 [m][rows].
 * Pinned by: numpy f64 matmul of independently dequantized weights; one-hot x selects a weight column; q == z gives 0;
 * s = 1, z = 0 gives exact integers; the closed-form known-answer generator of src/mlx/metal.rs:375-384.
 */
EXPORT void or_gemm_f64(int bits, size_t group, size_t rows, size_t cols, const uint32_t* q, const float* scales,
                        const float* offsets, const uint16_t* x, size_t m, double* y, int threads) {
    gemm(bits, group, rows, cols, q, scales, offsets, x, m, y, threads, 0);
}

/* The reference's own CPU form (Quant::row_into then an f32 dot), threaded over rows: the cpu_baseline of the
 * benchmark. y f32 [m][rows]. */
EXPORT void or_gemm_f32(int bits, size_t group, size_t rows, size_t cols, const uint32_t* q, const float* scales,
                        const float* offsets, const uint16_t* x, size_t m, float* y, int threads) {
    gemm(bits, group, rows, cols, q, scales, offsets, x, m, y, threads, 1);
}
