// Host side of libqwenny_hip: the checkpoint's weight formats (Quant) and the load-time repacker into the gfx950
// tile layout (layout.h). Nothing here touches the GPU, so all of it runs and is tested without one.
#include <math.h>
#include <stdarg.h>

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "internal.h"
#include "layout.h"

namespace qh {

static thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

void parallel_for(size_t n, void (*fn)(void*, size_t, size_t), void* arg) {
    size_t threads = std::max(1u, std::thread::hardware_concurrency());
    threads = std::min(threads, n);
    if (threads <= 1) {
        if (n) fn(arg, 0, n);
        return;
    }
    size_t per = (n + threads - 1) / threads;
    std::vector<std::thread> pool;
    for (size_t i = 0; i < threads; i++) {
        size_t lo = i * per, hi = std::min(n, lo + per);
        if (lo >= hi) break;
        pool.emplace_back(fn, arg, lo, hi);
    }
    for (auto& t : pool) t.join();
}

}  // namespace qh

using namespace qh;

extern "C" const char* qh_last_error(void) { return g_error.c_str(); }

// Checkpoint::packed_matrix (checkpoint.rs:408-453)
extern "C" int qh_quant_from_packed(const uint32_t* packed, size_t rows, size_t words, size_t cols, int bits,
                                    int group, const float* scale, const uint32_t* zp, size_t zp_rows, size_t zp_cols,
                                    float* scales_out, float* offsets_out, qh_quant* out) {
    if (!packed || !scale || !scales_out || !offsets_out || !out || rows == 0 || words == 0)
        return fail(QH_EINVAL, "packed matrix: null buffer or empty shape");
    if (cols == 0) cols = words * 32 / (size_t)bits;
    // the matrix's own bits (config groups may differ in them)
    if ((words * 32) % cols == 0) bits = (int)(words * 32 / cols);
    if (bits != 4 && bits != 8) return fail(QH_EINVAL, "%zu words per row for %zu columns", words, cols);
    if (cols != words * 32 / (size_t)bits)
        return fail(QH_EINVAL, "%zu columns in %zu words of %d-bit values (padded rows are not supported)", cols,
                    words, bits);
    size_t g = group == 0 ? cols : (size_t)group;
    if (cols % g) return fail(QH_EINVAL, "%zu columns in groups of %zu", cols, g);
    size_t groups = cols / g;
    size_t per = 32 / (size_t)bits;
    uint32_t mask = (1u << bits) - 1;
    bool along_rows = false;
    if (zp) {
        along_rows = zp_rows == (rows + per - 1) / per && zp_cols == groups;
        if (!along_rows && !(zp_rows == rows && zp_cols == (groups + per - 1) / per))
            return fail(QH_EINVAL, "weight_zero_point [%zu, %zu] for %zu x %zu groups", zp_rows, zp_cols, rows,
                        groups);
    }
    for (size_t i = 0; i < rows * groups; i++) {
        size_t r = i / groups, gi = i % groups;
        float z;
        if (!zp) {
            z = (float)(1u << (bits - 1));
        } else {
            uint32_t v = along_rows ? zp[(r / per) * groups + gi] >> ((r % per) * bits)
                                    : zp[r * zp_cols + gi / per] >> ((gi % per) * bits);
            z = (float)(v & mask);
        }
        scales_out[i] = scale[i];
        offsets_out[i] = -scale[i] * z;
    }
    out->bits = bits;
    out->group = (int32_t)g;
    out->rows = rows;
    out->cols = cols;
    out->q = packed;
    out->scales = scales_out;
    out->offsets = offsets_out;
    return QH_OK;
}

static int check_quant(const qh_quant* q) {
    if (!q || !q->q || !q->scales || !q->offsets) return fail(QH_EINVAL, "quant: null buffer");
    if (q->bits != 4 && q->bits != 8) return fail(QH_EINVAL, "quant: %d bits (4 or 8)", q->bits);
    if (q->group <= 0 || q->cols == 0 || q->cols % (size_t)q->group || (q->cols * q->bits) % 32)
        return fail(QH_EINVAL, "quant: %zu columns in groups of %d", q->cols, q->group);
    return QH_OK;
}

// Quant::zero_points (checkpoint.rs:72-82)
extern "C" int qh_quant_zero_points(const qh_quant* q, uint8_t* z) {
    if (int e = check_quant(q)) return e;
    if (!z) return fail(QH_EINVAL, "zero points: null output");
    float max = (float)((1u << q->bits) - 1);
    size_t n = q->rows * (q->cols / (size_t)q->group);
    for (size_t i = 0; i < n; i++) {
        float s = q->scales[i], o = q->offsets[i];
        float v = s == 0.0f ? 0.0f : -o / s;
        float r = roundf(v);
        if (!(r >= 0.0f && r <= max && fabsf(v - r) < 1e-3f)) return 0;
        z[i] = (uint8_t)r;
    }
    return 1;
}

// Quant::row_into (checkpoint.rs:39-47)
extern "C" int qh_quant_row_into(const qh_quant* q, size_t r, float* out) {
    if (int e = check_quant(q)) return e;
    if (r >= q->rows || !out) return fail(QH_EINVAL, "row %zu of %zu", r, q->rows);
    size_t per = 32 / (size_t)q->bits, words = q->cols * (size_t)q->bits / 32, groups = q->cols / (size_t)q->group;
    uint32_t mask = (1u << q->bits) - 1;
    const uint32_t* w = q->q + r * words;
    for (size_t c = 0; c < q->cols; c++) {
        uint32_t v = (w[c / per] >> ((c % per) * (size_t)q->bits)) & mask;
        size_t g = r * groups + c / (size_t)q->group;
        out[c] = (float)v * q->scales[g] + q->offsets[g];
    }
    return QH_OK;
}

// Quant::to_bf16 (checkpoint.rs:50-68): every row through row_into, rounded to bf16 nearest even, threaded over rows
extern "C" int qh_quant_to_bf16(const qh_quant* q, uint16_t* out) {
    if (int e = check_quant(q)) return e;
    if (!out) return fail(QH_EINVAL, "to_bf16: null output");
    parallel(q->rows, [&](size_t lo, size_t hi) {
        std::vector<float> row(q->cols);
        for (size_t r = lo; r < hi; r++) {
            qh_quant_row_into(q, r, row.data());
            for (size_t c = 0; c < q->cols; c++) out[r * q->cols + c] = f32_to_bf16(row[c]);
        }
    });
    return QH_OK;
}

// row_order (cuda/core.rs:108-114)
extern "C" int qh_row_order(size_t rows, int silu, size_t* out) {
    if (!out) return fail(QH_EINVAL, "row order: null output");
    if (silu && rows % 16) return fail(QH_EINVAL, "row order: %zu rows for SwiGLU tiles of 16", rows);
    for (size_t i = 0; i < rows; i++)
        out[i] = silu ? (i / 16) * 8 + i % 8 + (i % 16 >= 8 ? rows / 2 : 0) : i;
    return QH_OK;
}

extern "C" int qh_packed_sizes(int wt, size_t rows, size_t cols, size_t* code_bytes, size_t* scale_bytes,
                               size_t* zero_bytes) {
    if (!valid_wt(wt)) return fail(QH_EINVAL, "storage %d", wt);
    if (rows == 0 || rows % TILE || cols == 0 || cols % QG)
        return fail(QH_EINVAL, "%zu x %zu: rows must be a multiple of 16, columns of 128", rows, cols);
    size_t tiles = rows / TILE, blocks = tiles * (cols / QG), qd = tiles * quads(cols / QG);
    // the kernels address codes and scales with 32-bit byte offsets from the matrix's base
    if (rows > (1u << 30) || cols > (1u << 30) || blocks * block_bytes(wt) > 0xffffffffu)
        return fail(QH_EINVAL, "%zu x %zu: the codes must fit in 4 GiB", rows, cols);
    if (code_bytes) *code_bytes = blocks * block_bytes(wt);
    if (scale_bytes) *scale_bytes = has_scales(wt) ? qd * TILE * 4 * (f32_scales(wt) ? 4 : 2) : 0;
    if (zero_bytes) *zero_bytes = has_zeros(wt) ? qd * TILE * 2 : 0;
    return QH_OK;
}

// One tile (16 packed rows) of the layout from per-row accessors. word(row, k) gives the source word holding columns
// k .. k + 32 / bits - 1 of `row` in the checkpoint's order (value c at bits c * bits); scale(row, g), zero(row, g) per
// 128-column group.
template <class Word, class Scale, class Zero>
static void pack_tile(int wt, size_t cols, const size_t* rows16, size_t t, size_t T, Word word, Scale scale, Zero zero,
                      void* codes, void* scales, void* zeros) {
    const size_t G = cols / QG;
    for (size_t g = 0; g < G; g++) {
        size_t blk = t * G + g;
        if (is_i8(wt)) {
            uint32_t* out = (uint32_t*)codes + blk * 512;
            for (int h = 0; h < 2; h++)
                for (int l = 0; l < LANES; l++)
                    for (int w = 0; w < 4; w++) {
                        size_t k = g * QG + 32 * (2 * h + w / 2) + 8 * (l / 16) + 4 * (w % 2);
                        out[(h * LANES + l) * 4 + w] = word(rows16[l % 16], k);
                    }
        } else {
            uint32_t* out = (uint32_t*)codes + blk * 256;
            for (int l = 0; l < LANES; l++)
                for (int j = 0; j < 4; j++) {
                    uint32_t src = word(rows16[l % 16], g * QG + 32 * j + 8 * (l / 16)), dst = 0;
                    for (int c = 0; c < 8; c++) dst |= ((src >> (4 * c)) & 15u) << (4 * nib_pos(c));
                    out[l * 4 + j] = dst;
                }
        }
    }
    // scales and zero points by quads of 4 groups; the padding past G holds zeros
    for (size_t g = 0; g < quads(G) * 4; g++)
        for (int r = 0; r < TILE; r++) {
            const float sc = g < G ? scale(rows16[r], g) : 0.0f;
            if (f32_scales(wt))
                ((float*)scales)[scale_idx(t, T, g, r)] = sc;
            else
                ((uint16_t*)scales)[scale_idx(t, T, g, r)] = f32_to_bf16(sc);
        }
    if (has_zeros(wt))
        for (size_t q4 = 0; q4 < quads(G); q4++)
            for (int r = 0; r < TILE; r++) {
                uint16_t z = 0;
                for (size_t g = 4 * q4; g < std::min(G, 4 * q4 + 4); g++) z |= (uint16_t)((zero(rows16[r], g) & 15u) << (4 * (g % 4)));
                ((uint16_t*)zeros)[zero_idx(t, T, 4 * q4, r)] = z;
            }
}

extern "C" int qh_pack_quant(const qh_quant* q, const uint8_t* zeros, const size_t* order, size_t n, int wt,
                             void* codes, void* scales, void* zeros_out) {
    if (int e = check_quant(q)) return e;
    if (!order || !codes || !scales) return fail(QH_EINVAL, "pack: null buffer");
    if (!valid_wt(wt) || is_bf16(wt) || is_i8(wt) != (q->bits == 8))
        return fail(QH_EINVAL, "pack: storage %d for %d-bit values", wt, q->bits);
    if (has_zeros(wt) && (!zeros || !zeros_out)) return fail(QH_EINVAL, "pack: zero points needed");
    if (q->group % QG || q->cols % QG || n == 0 || n % TILE)
        return fail(QH_EINVAL, "pack: %zu rows of %zu columns in groups of %d: rows must be a multiple of 16, "
                    "groups and columns of 128", n, q->cols, q->group);
    for (size_t i = 0; i < n; i++)
        if (order[i] >= q->rows) return fail(QH_EINVAL, "pack: row %zu of %zu", order[i], q->rows);
    size_t words = q->cols * (size_t)q->bits / 32, qgroups = q->cols / (size_t)q->group, per = 32 / (size_t)q->bits;
    size_t gstep = (size_t)q->group / QG;  // 128-column groups per stored group
    auto word = [&](size_t row, size_t k) { return q->q[row * words + k / per]; };
    auto scale = [&](size_t row, size_t g) { return q->scales[row * qgroups + g / gstep]; };
    auto zero = [&](size_t row, size_t g) -> uint32_t { return zeros ? zeros[row * qgroups + g / gstep] : 8; };
    parallel(n / TILE, [&](size_t lo, size_t hi) {
        for (size_t t = lo; t < hi; t++)
            pack_tile(wt, q->cols, order + t * TILE, t, n / TILE, word, scale, zero, codes, scales, zeros_out);
    });
    return QH_OK;
}

extern "C" int qh_unpack_row(int wt, size_t rows, size_t cols, const void* codes, const void* scales,
                             const void* zeros, size_t p, uint8_t* vals, float* sc, uint8_t* z) {
    if (int e = qh_packed_sizes(wt, rows, cols, nullptr, nullptr, nullptr)) return e;
    if (is_bf16(wt)) return fail(QH_EINVAL, "unpack: dense bf16 rows unpack with qh_unpack_row_bf16");
    if (p >= rows || !codes || !scales || !vals || !sc || !z || (has_zeros(wt) && !zeros))
        return fail(QH_EINVAL, "unpack: row %zu of %zu or null buffer", p, rows);
    size_t G = cols / QG, t = p / TILE, T = rows / TILE;
    int r = (int)(p % TILE);
    for (size_t g = 0; g < G; g++) {
        size_t blk = t * G + g;
        for (int l = r; l < LANES; l += 16) {
            if (is_i8(wt)) {
                const uint32_t* in = (const uint32_t*)codes + blk * 512;
                for (int h = 0; h < 2; h++)
                    for (int w = 0; w < 4; w++) {
                        uint32_t v = in[(h * LANES + l) * 4 + w];
                        size_t k = g * QG + 32 * (2 * h + w / 2) + 8 * (l / 16) + 4 * (w % 2);
                        for (int b = 0; b < 4; b++) vals[k + b] = (uint8_t)(v >> (8 * b));
                    }
            } else {
                const uint32_t* in = (const uint32_t*)codes + blk * 256;
                for (int j = 0; j < 4; j++) {
                    uint32_t v = in[l * 4 + j];
                    size_t k = g * QG + 32 * j + 8 * (l / 16);
                    for (int c = 0; c < 8; c++) vals[k + c] = (uint8_t)((v >> (4 * nib_pos(c))) & 15u);
                }
            }
        }
        sc[g] = f32_scales(wt) ? ((const float*)scales)[scale_idx(t, T, g, r)]
                               : bf16_to_f32(((const uint16_t*)scales)[scale_idx(t, T, g, r)]);
        z[g] = is_i8(wt)       ? 128
               : has_zeros(wt) ? (uint8_t)((((const uint16_t*)zeros)[zero_idx(t, T, g, r)] >> (4 * (g % 4))) & 15u)
                               : 8;
    }
    return QH_OK;
}

// Mat::new / pack, int8 branch (cuda/core.rs:127-135, :338-389)
extern "C" int qh_pack_dense_int8(const uint16_t* bf16, size_t rows, size_t cols, const size_t* order, size_t n,
                                  void* codes, void* scales) {
    if (!bf16 || !order || !codes || !scales) return fail(QH_EINVAL, "dense int8: null buffer");
    if (int e = qh_packed_sizes(QH_WT_I8, n, cols, nullptr, nullptr, nullptr)) return e;
    for (size_t i = 0; i < n; i++)
        if (order[i] >= rows) return fail(QH_EINVAL, "dense int8: row %zu of %zu", order[i], rows);
    size_t G = cols / QG;
    parallel(n / TILE, [&](size_t lo, size_t hi) {
        std::vector<uint32_t> qw(TILE * cols / 4);  // the tile's requantized rows, 4 values per word
        std::vector<float> sc(TILE * G);
        for (size_t t = lo; t < hi; t++) {
            const size_t* rows16 = order + t * TILE;
            for (int r = 0; r < TILE; r++) {
                const uint16_t* src = bf16 + rows16[r] * cols;
                for (size_t g = 0; g < G; g++) {
                    float max = 0.0f;
                    for (int c = 0; c < QG; c++) max = fmaxf(max, fabsf(bf16_to_f32(src[g * QG + c])));
                    float s = max > 0.0f ? max / 127.0f : 1.0f;
                    sc[r * G + g] = s;
                    for (int c = 0; c < QG; c += 4) {
                        uint32_t w = 0;
                        for (int b = 0; b < 4; b++) {
                            float v = roundf(bf16_to_f32(src[g * QG + c + b]) / s);
                            v = isnan(v) ? 0.0f : fminf(fmaxf(v, -127.0f), 127.0f);  // Rust: NaN as i32 == 0
                            w |= (uint32_t)((int)v + 128) << (8 * b);
                        }
                        qw[(r * cols + g * QG + c) / 4] = w;
                    }
                }
            }
            static const size_t local[TILE] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15};
            auto word = [&](size_t r, size_t k) { return qw[(r * cols + k) / 4]; };
            auto scale = [&](size_t r, size_t g) { return sc[r * G + g]; };
            auto zero = [](size_t, size_t) -> uint32_t { return 128; };
            pack_tile(QH_WT_I8, cols, local, t, n / TILE, word, scale, zero, codes, scales, nullptr);
        }
    });
    return QH_OK;
}

// Mat::new / pack, 16-bit branch (cuda/core.rs:127-135, :370-381): the reference stores f16 tiles; here the weights stay
// bf16 (the checkpoint's own values, bit for bit) in the QH_WT_BF16 layout.
extern "C" int qh_pack_dense_bf16(const uint16_t* bf16, size_t rows, size_t cols, const size_t* order, size_t n,
                                  void* codes) {
    if (!bf16 || !order || !codes) return fail(QH_EINVAL, "dense bf16: null buffer");
    if (int e = qh_packed_sizes(QH_WT_BF16, n, cols, nullptr, nullptr, nullptr)) return e;
    for (size_t i = 0; i < n; i++)
        if (order[i] >= rows) return fail(QH_EINVAL, "dense bf16: row %zu of %zu", order[i], rows);
    const size_t G = cols / QG;
    uint16_t* out = (uint16_t*)codes;
    parallel(n / TILE, [&](size_t lo, size_t hi) {
        for (size_t t = lo; t < hi; t++)
            for (size_t g = 0; g < G; g++)
                for (int j = 0; j < 4; j++)
                    for (int l = 0; l < LANES; l++) {
                        const uint16_t* src = bf16 + order[t * TILE + l % 16] * cols + g * QG + 32 * j + 8 * (l / 16);
                        std::memcpy(out + (((t * G + g) * 4 + j) * LANES + l) * 8, src, 16);
                    }
    });
    return QH_OK;
}

// The inverse for one packed row p of a QH_WT_BF16 matrix: its bf16 values into out[cols].
extern "C" int qh_unpack_row_bf16(size_t rows, size_t cols, const void* codes, size_t p, uint16_t* out) {
    if (int e = qh_packed_sizes(QH_WT_BF16, rows, cols, nullptr, nullptr, nullptr)) return e;
    if (p >= rows || !codes || !out) return fail(QH_EINVAL, "unpack bf16: row %zu of %zu or null buffer", p, rows);
    const size_t G = cols / QG, t = p / TILE;
    const uint16_t* in = (const uint16_t*)codes;
    for (size_t g = 0; g < G; g++)
        for (int j = 0; j < 4; j++)
            for (int l = (int)(p % TILE); l < LANES; l += 16)
                std::memcpy(out + g * QG + 32 * j + 8 * (l / 16), in + (((t * G + g) * 4 + j) * LANES + l) * 8, 16);
    return QH_OK;
}
