// Device side of the C ABI (include/qwenny_hip.h): contexts, device matrices and the product dispatch by token count
// (and, at 33-48 tokens, matrix size).
// Mirrors the reference's Gemm / Mat runtime (cuda/core.rs:94-681) over HIP: the matrix owns its device buffers, the
// product only launches (no allocation, no host synchronisation), errors come back as status codes.
#include <hip/hip_runtime.h>

#include <stdlib.h>

#include <algorithm>
#include <vector>

#include "gemm.h"
#include "internal.h"
#include "kernels.h"
#include "layout.h"

using namespace qh;

struct qh_ctx {
    int device;
    // the argmax epilogue's scratch: table [ARGMAX_SPREAD][ARGMAX_MAX_TOK] u64, then the workgroup counter; zeroed
    // here and left zero by every launch
    void* argmax_scratch;
    int cus;             // compute units
    int skinny_max_w;       // skinny kernel: most waves per workgroup (non-plain epilogues)
    int skinny_fill;        // skinny kernel, non-plain epilogues: waves per CU a launch aims for
    int skinny_tile_waves;  // skinny kernel, plain products: waves side by side over tiles (0: by token count)
    int pf_shape;           // prefill workgroup shape (0: by tail waste; QH_PF_SHAPE for tuning sweeps)
    // prefill stream-K: partial tiles, then PF_SK_ITEMS_MAX item counters (zeroed here, left zero by every launch);
    // QH_PF_SK=0 turns it off, a value above 1 replaces the launcher's fix-up cost (tuning); then the f16 activations
    // of prefill launches with f16 operands (X16_SCRATCH_BYTES)
    void* sk_scratch;
    int stream_k;
    int skinny_plain_wk;    // skinny kernel, plain products: wave rows over K per workgroup (1; QH_SKINNY_PLAIN_WK)
    int pf_from;            // products from this many tokens take the prefill kernel (QH_PF_FROM, tuning; 49: off)
    int skinny_few;         // plain products with fewer 4-group waves than this many per CU take 1-group waves (0: by
                            // token count; QH_SKINNY_FEW, tuning)
};

int qh::ctx_device(const qh_ctx* ctx) { return ctx->device; }

// The context's own launch scratch.
static Scratch ctx_scratch(const qh_ctx* ctx) {
    return Scratch{ctx->argmax_scratch, ctx->sk_scratch, (uint8_t*)ctx->sk_scratch + PF_SK_SCRATCH_BYTES};
}

static int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

struct qh_mat {
    int wt;
    bool per_channel;  // int8 with one scale per row (every group's equal): exact integer prefill products
    size_t rows, cols, valid;
    size_t code_bytes, scale_bytes, zero_bytes;
    void* codes;
    void* scales;
    void* zeros;
    // put_block staging (one tile: codes, scales, zeros), pinned, reused after `staged` completes
    uint8_t* stage;
    hipEvent_t staged;
};

#define HIP_TRY(call)                                                                              \
    do {                                                                                           \
        hipError_t e_ = (call);                                                                    \
        if (e_ != hipSuccess) return fail(QH_EHIP, "%s: %s", #call, hipGetErrorString(e_));        \
    } while (0)

extern "C" int qh_open(int device, qh_ctx** out) {
    if (!out) return fail(QH_EINVAL, "open: null output");
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(QH_EINVAL, "device %d of %d", device, count);
    HIP_TRY(hipSetDevice(device));
    int cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    // QH_SKINNY_MAX_W / QH_SKINNY_TILE_WAVES override the skinny partition (tuning sweeps)
    void* scratch = nullptr;
    const size_t scratch_bytes = ARGMAX_SCRATCH_BYTES;
    HIP_TRY(hipMalloc(&scratch, scratch_bytes));
    if (hipMemset(scratch, 0, scratch_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(scratch);
        return fail(QH_EHIP, "argmax scratch: clear failed");
    }
    void* sk = nullptr;
    const size_t sk_bytes = PF_SK_SCRATCH_BYTES + X16_SCRATCH_BYTES;
    if (hipMalloc(&sk, sk_bytes) != hipSuccess) {
        (void)hipFree(scratch);
        return fail(QH_ENOMEM, "prefill scratch of %zu bytes: allocation failed", sk_bytes);
    }
    if (hipMemset((uint8_t*)sk + PF_SK_PART_BYTES, 0, PF_SK_ITEMS_MAX * sizeof(unsigned)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(scratch);
        (void)hipFree(sk);
        return fail(QH_EHIP, "prefill scratch: clear failed");
    }
    if (int e = noalloc_init(device)) {
        (void)hipFree(scratch);
        (void)hipFree(sk);
        return e;
    }
    *out = new qh_ctx{device, scratch, std::max(cus, 1), std::min(16, std::max(1, env_int("QH_SKINNY_MAX_W", 16))),
                      std::min(64, std::max(1, env_int("QH_SKINNY_FILL", 8))),
                      std::min(16, std::max(0, env_int("QH_SKINNY_TILE_WAVES", 0))),
                      std::min(9, std::max(0, env_int("QH_PF_SHAPE", 0))), sk, std::max(0, env_int("QH_PF_SK", 1)),
                      std::min(4, std::max(1, env_int("QH_SKINNY_PLAIN_WK", 1))),
                      std::max(1, env_int("QH_PF_FROM", SKINNY_MAX_M + 1)),
                      std::min(64, std::max(0, env_int("QH_SKINNY_FEW", 0)))};
    return QH_OK;
}

extern "C" void qh_close(qh_ctx* ctx) {
    if (!ctx) return;
    if (ctx->argmax_scratch) (void)hipFree(ctx->argmax_scratch);
    if (ctx->sk_scratch) (void)hipFree(ctx->sk_scratch);
    delete ctx;
}

static void mat_release(qh_mat* m) {
    if (!m) return;
    if (m->codes) (void)hipFree(m->codes);
    if (m->scales) (void)hipFree(m->scales);
    if (m->zeros) (void)hipFree(m->zeros);
    if (m->stage) (void)hipHostFree(m->stage);
    if (m->staged) (void)hipEventDestroy(m->staged);
    delete m;
}

extern "C" void qh_mat_free(qh_mat* m) { mat_release(m); }

static int mat_alloc(int wt, size_t rows, size_t cols, size_t valid, qh_mat** out) {
    qh_mat* m = new qh_mat{};
    m->wt = wt;
    m->rows = rows;
    m->cols = cols;
    m->valid = valid;
    if (int e = qh_packed_sizes(wt, rows, cols, &m->code_bytes, &m->scale_bytes, &m->zero_bytes)) {
        delete m;
        return e;
    }
    if (valid > rows) {
        delete m;
        return fail(QH_EINVAL, "%zu valid rows of %zu", valid, rows);
    }
    size_t tiles = rows / TILE;
    size_t stage = (m->code_bytes + m->scale_bytes + m->zero_bytes) / tiles;
    if (hipMalloc(&m->codes, m->code_bytes) != hipSuccess ||
        (m->scale_bytes && hipMalloc(&m->scales, m->scale_bytes) != hipSuccess) ||
        (m->zero_bytes && hipMalloc(&m->zeros, m->zero_bytes) != hipSuccess) ||
        hipHostMalloc((void**)&m->stage, stage, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&m->staged, hipEventDisableTiming) != hipSuccess) {
        mat_release(m);
        return fail(QH_ENOMEM, "device matrix of %zu x %zu: allocation failed", rows, cols);
    }
    *out = m;
    return QH_OK;
}

extern "C" int qh_mat_upload(qh_ctx* ctx, int wt, size_t rows, size_t cols, const void* codes, const void* scales,
                             const void* zeros, size_t valid, qh_mat** out) {
    if (!ctx || !codes || (has_scales(wt) && !scales) || !out || (has_zeros(wt) && !zeros))
        return fail(QH_EINVAL, "upload: null");
    qh_mat* m = nullptr;
    if (int e = mat_alloc(wt, rows, cols, valid, &m)) return e;
    if (hipMemcpy(m->codes, codes, m->code_bytes, hipMemcpyHostToDevice) != hipSuccess ||
        (m->scale_bytes && hipMemcpy(m->scales, scales, m->scale_bytes, hipMemcpyHostToDevice) != hipSuccess) ||
        (m->zero_bytes && hipMemcpy(m->zeros, zeros, m->zero_bytes, hipMemcpyHostToDevice) != hipSuccess)) {
        mat_release(m);
        return fail(QH_EHIP, "upload of %zu x %zu failed", rows, cols);
    }
    if (wt == QH_WT_I8) {
        const float* s = (const float*)scales;
        const size_t G = cols / QG, tiles = rows / TILE;
        m->per_channel = true;
        for (size_t t = 0; t < tiles && m->per_channel; t++)
            for (int r = 0; r < TILE && m->per_channel; r++)
                for (size_t g = 1; g < G && m->per_channel; g++)
                    m->per_channel = s[scale_idx(t, tiles, g, r)] == s[scale_idx(t, tiles, 0, r)];
    }
    *out = m;
    return QH_OK;
}

// int4 storage of q: bf16 scales when every scale is exact in bf16, else f32.
static int int4_storage(const qh_quant* q, bool sym) {
    const size_t n = q->rows * (q->cols / (size_t)q->group);
    bool bf16 = true;
    for (size_t i = 0; i < n && bf16; i++) bf16 = bf16_to_f32(f32_to_bf16(q->scales[i])) == q->scales[i];
    if (sym) return bf16 ? QH_WT_I4 : QH_WT_I4_S32;
    return bf16 ? QH_WT_I4Z : QH_WT_I4Z_S32;
}

// Pack `order` rows of q and upload them.
static int pack_upload(qh_ctx* ctx, const qh_quant* q, const uint8_t* zeros, const size_t* order, size_t n, int wt,
                       size_t valid, qh_mat** out) {
    size_t cb, sb, zb;
    if (int e = qh_packed_sizes(wt, n, q->cols, &cb, &sb, &zb)) return e;
    std::vector<uint8_t> codes(cb), scales(sb), zs(zb);
    if (int e = qh_pack_quant(q, zeros, order, n, wt, codes.data(), scales.data(), zs.data())) return e;
    return qh_mat_upload(ctx, wt, n, q->cols, codes.data(), scales.data(), zs.data(), valid, out);
}

extern "C" int qh_mat_quant(qh_ctx* ctx, const qh_quant* q, int silu, qh_mat** out) {
    if (!ctx || !q || !out) return fail(QH_EINVAL, "mat quant: null");
    if (q->rows % TILE || q->cols % QG || q->group <= 0 || q->group % QG)
        return fail(QH_ENOTFIT, "%d-bit %zu x %zu in groups of %d: rows must be a multiple of 16, columns and "
                    "groups of 128", q->bits, q->rows, q->cols, q->group);
    std::vector<uint8_t> z(q->rows * (q->cols / (size_t)q->group));
    int zp = qh_quant_zero_points(q, z.data());
    if (zp < 0) return zp;
    if (zp == 0) return fail(QH_ENOTFIT, "%d-bit %zu x %zu: zero points are not integers", q->bits, q->rows, q->cols);
    std::vector<size_t> order(q->rows);
    if (int e = qh_row_order(q->rows, silu, order.data())) return e;
    int wt;
    if (q->bits == 8) {
        if (std::any_of(z.begin(), z.end(), [](uint8_t v) { return v != 128; }))
            return fail(QH_ENOTFIT, "int8 %zu x %zu: zero points other than 128", q->rows, q->cols);
        wt = QH_WT_I8;
    } else {
        wt = int4_storage(q, std::all_of(z.begin(), z.end(), [](uint8_t v) { return v == 8; }));
    }
    return pack_upload(ctx, q, has_zeros(wt) ? z.data() : nullptr, order.data(), q->rows, wt, q->rows, out);
}

extern "C" int qh_mat_quant_rows(qh_ctx* ctx, const qh_quant* q, const uint8_t* zeros, const size_t* rows, size_t n,
                                 size_t cap, qh_mat** out) {
    if (!ctx || !q || !zeros || !rows || !out) return fail(QH_EINVAL, "mat rows: null");
    if (q->bits != 4) return fail(QH_EINVAL, "int4 rows only, not %d-bit ones", q->bits);
    if (n == 0 || n % TILE || cap % TILE || n > cap) return fail(QH_EINVAL, "%zu rows (room for %zu)", n, cap);
    size_t nz = q->rows * (q->cols / (size_t)q->group);
    bool sym = std::all_of(zeros, zeros + nz, [](uint8_t v) { return v == 8; });
    std::vector<size_t> order(cap, rows[0]);
    std::copy(rows, rows + n, order.begin());
    const int wt = int4_storage(q, sym);
    return pack_upload(ctx, q, has_zeros(wt) ? zeros : nullptr, order.data(), cap, wt, n, out);
}

extern "C" int qh_mat_dense_int8(qh_ctx* ctx, const uint16_t* bf16, size_t rows, size_t cols, int silu,
                                 qh_mat** out) {
    if (!ctx || !bf16 || !out) return fail(QH_EINVAL, "dense int8: null");
    size_t cb, sb;
    if (int e = qh_packed_sizes(QH_WT_I8, rows, cols, &cb, &sb, nullptr)) return e;
    std::vector<size_t> order(rows);
    if (int e = qh_row_order(rows, silu, order.data())) return e;
    std::vector<uint8_t> codes(cb), scales(sb);
    if (int e = qh_pack_dense_int8(bf16, rows, cols, order.data(), rows, codes.data(), scales.data())) return e;
    return qh_mat_upload(ctx, QH_WT_I8, rows, cols, codes.data(), scales.data(), nullptr, rows, out);
}

extern "C" int qh_mat_dense(qh_ctx* ctx, const uint16_t* bf16, size_t rows, size_t cols, int silu, qh_mat** out) {
    if (!ctx || !bf16 || !out) return fail(QH_EINVAL, "dense bf16: null");
    size_t cb;
    if (int e = qh_packed_sizes(QH_WT_BF16, rows, cols, &cb, nullptr, nullptr)) return e;
    std::vector<size_t> order(rows);
    if (int e = qh_row_order(rows, silu, order.data())) return e;
    std::vector<uint8_t> codes(cb);
    if (int e = qh_pack_dense_bf16(bf16, rows, cols, order.data(), rows, codes.data())) return e;
    return qh_mat_upload(ctx, QH_WT_BF16, rows, cols, codes.data(), nullptr, nullptr, rows, out);
}

extern "C" int qh_mat_describe(const qh_mat* m, qh_mat_desc* out) {
    if (!m || !out) return fail(QH_EINVAL, "describe: null");
    *out = qh_mat_desc{m->wt, m->rows, m->cols, m->valid, m->code_bytes, m->scale_bytes, m->zero_bytes,
                       m->per_channel ? 1 : 0};
    return QH_OK;
}

extern "C" int qh_mat_download(const qh_mat* m, void* codes, void* scales, void* zeros) {
    if (!m || !codes || (m->scale_bytes && !scales)) return fail(QH_EINVAL, "download: null");
    HIP_TRY(hipMemcpy(codes, m->codes, m->code_bytes, hipMemcpyDeviceToHost));
    if (m->scale_bytes) HIP_TRY(hipMemcpy(scales, m->scales, m->scale_bytes, hipMemcpyDeviceToHost));
    if (zeros && m->zero_bytes) HIP_TRY(hipMemcpy(zeros, m->zeros, m->zero_bytes, hipMemcpyDeviceToHost));
    return QH_OK;
}

// The skinny kernel's K partition: waves per workgroup and grid split for a product of m tokens. Enough waves
// (about 12 per CU) to keep HBM busy, at least a few groups per wave so that its pipeline fills; non-plain epilogues
// need whole sums in one workgroup (split 1).
struct Partition {
    int tile_waves, waves, split, groups_per_wave, tiles_per_wave;
};

// The skinny kernel's partition of a product of m tokens (kernels.hip skinny_kernel): each wave takes SKINNY_TILES
// tiles (plain int8 and bf16 products of 1-2 tokens: one) and 4 groups (1 when the group count is not a multiple of 4); a
// workgroup stages the activations of its super-chunk of K once for all its waves, so the more wave columns
// (tile_waves) share it, the less that costs relative to the weights (m / (4 * tile_waves * SKINNY_TILES) of the int4
// bytes).
// Plain products: workgroups of wave columns side by side over tiles, the grid split over every chunk of K (split-K
// partials the consumer sums). Other epilogues need whole sums in one workgroup: its wave rows split K (reduced
// through LDS), as few as give the launch enough waves to fill the CUs, dividing the chunks evenly and fitting the wave
// and LDS limits; longer K is walked in super-chunks.
static Partition skinny_partition(const qh_ctx* ctx, const qh_mat* m, size_t tokens, bool plain) {
    const int tiles = (int)(m->rows / TILE), G = (int)(m->cols / QG);
    // tiles per wave: one for plain int8 and bf16 products of 1-2 tokens (8 KiB of one tile, half the registers of a
    // two-tile wave, 5 waves per SIMD for int8: same-box graph replays, int8 per channel 27B set at M = 1 5.39 -> 5.49
    // TB/s, grouped int8 5.49 -> 5.69, dense bf16 6.12 -> 6.17; at M = 2 int8 5.04 -> 5.19 TB/s, grouped 5.00 ->
    // 5.17; from 3 tokens two tiles stay level or ahead, -0.5% at 5)
    const int tpw = plain && tokens <= 2 && (is_i8(m->wt) || is_bf16(m->wt)) ? 1 : SKINNY_TILES;
    const int cols = (tiles + tpw - 1) / tpw;  // wave columns over the tiles
    // groups per wave: 4 (int4 and int8: 4 KiB or 8 KiB of a tile per wave), 1 for bf16 (4 KiB per group)
    // (plain products whose 4-group waves would number fewer than the chip's SIMDs take one group per wave instead:
    // 4x the waves in flight; measured +5% at M = 1 and +10% at M = 8 on the 4B layer set, the 27B set unchanged;
    // at 1-2 tokens up to 6 waves per CU: configs[0] (2560, 9728) 4.33 -> 4.10 us, the 4B set at M = 2 3.94 -> 3.90
    // us, the 27B set the same, while at 5 tokens the 4B set lost 10% and 8 per CU cost the 27B set 1% at 1 token)
    const int few_per_cu = ctx->skinny_few > 0 ? ctx->skinny_few : (tokens <= 2 ? 6 : 4);
    const bool few = plain && (long)cols * (G / 4) < (long)few_per_cu * ctx->cus;
    const int ng = !is_bf16(m->wt) && G % 4 == 0 && !few ? 4 : 1;
    const int want_wt = ctx->skinny_tile_waves > 0 ? ctx->skinny_tile_waves : (tokens <= 2 ? 4 : 8);
    if (plain) {
        const int wt = std::max(1, std::min({want_wt, cols, tokens > 16 ? 8 : 16}));
        // QH_SKINNY_PLAIN_WK (tuning): wave rows over K within the workgroup, dividing the partials
        const int pk = ctx->skinny_plain_wk;
        if (pk > 1 && (G / ng) % pk == 0 && wt * pk <= (tokens > 16 ? 8 : 16))
            return Partition{wt, wt * pk, G / ng / pk, ng, tpw};
        return Partition{wt, wt, G / ng, ng, tpw};
    }
    const size_t per_group = std::max<size_t>(tokens, 1) * QG * 2;  // LDS bytes of one group's activations
    // above 16 tokens (several 16-token blocks per wave) workgroups of at most 8 waves: the kernel's register budget
    const int max_w = tokens > 16 ? std::min(ctx->skinny_max_w, 8) : ctx->skinny_max_w;
    const int wt = std::max(1, std::min({tokens <= 2 ? 2 : 8, cols, max_w}));
    const long wgs = (cols + wt - 1) / wt;
    // wave rows: dividing the chunks of K, within the wave and LDS limits; the fewest that make a workgroup of at least
    // 4 waves, more only while the launch has fewer than skinny_fill waves per CU (measured: extra rows add LDS
    // reductions and lose occupancy; fewer than 4 waves walk K in too many barrier-separated super-chunks)
    const int nchunks = G / ng, wmax = std::min(max_w / wt, nchunks);
    int wk = 1;
    for (int w = 1; w <= wmax; w++) {
        if (nchunks % w || (size_t)w * ng * per_group > SKINNY_X_LDS) continue;
        wk = w;
        if (wt * w >= 4 && wgs * wt * w >= (long)ctx->skinny_fill * ctx->cus) break;
    }
    return Partition{wt, wt * wk, 1, ng, tpw};
}

// Whether the skinny kernel takes a product of m tokens (else the prefill kernel): up to SKINNY_MAX_M tokens, except
// split-K plain and SwiGLU products of int4 or grouped int8 matrices of at least PF_FROM33_WEIGHTS weights from 33
// tokens (three 16-token blocks per skinny wave), where the prefill kernel is faster (measured at 33-48 tokens on the
// 27B shapes (5120, 17408) and (17408, 5120), plain: 1.10-1.29x per product for int4 with zero points, 1.17-1.27x
// symmetric, 1.36-1.50x grouped int8, more with the partials summed; the [gate; up] SwiGLU product 1.14-1.36x; on
// the smaller 27B shapes, 31M weights, the skinny kernel stays ahead). The argmax epilogue (the 27B head: 238 against
// 254 us at 48 tokens), whole plain products, per-channel int8 and bf16 matrices stay on the skinny kernel.
// QH_PF_FROM (tuning) moves every product from that many tokens to the prefill kernel instead.
static bool use_skinny(const qh_ctx* ctx, const qh_mat* w, size_t m, int epi, int whole) {
    if (m > (size_t)SKINNY_MAX_M) return false;
    if (ctx->pf_from <= SKINNY_MAX_M) return m < (size_t)ctx->pf_from;
    if (epi == QH_EPI_ARGMAX || (epi == QH_EPI_PLAIN && whole)) return true;
    const bool fmt = (!is_i8(w->wt) && !is_bf16(w->wt)) || (is_i8(w->wt) && !w->per_channel);
    return !(m > 32 && fmt && w->rows * w->cols >= PF_FROM33_WEIGHTS);
}

// The launch of a product of m tokens (epi, x, y and keys as qh_gemm takes them; `whole`: one partial).
static Launch make_launch(const qh_ctx* ctx, const qh_mat* w, const void* x, size_t ldx, size_t m,
                          const int32_t* out_rows, void* y, int epi, uint64_t* keys, int whole, void* stream,
                          const Scratch& sc) {
    Launch l{};
    l.codes = w->codes;
    l.scales = w->scales;
    l.zeros = (const uint16_t*)w->zeros;
    l.fmt = is_bf16(w->wt) ? F_BF16
                           : (is_i8(w->wt) ? F_I8 | (w->per_channel ? F_PERCH : 0) : 0) | (has_zeros(w->wt) ? F_ZP : 0) |
                                 (f32_scales(w->wt) ? F_S32 : 0);
    l.rows = (int)w->rows;
    l.cols = (int)w->cols;
    l.valid = (int)w->valid;
    l.x = x;
    l.ldx = (int)ldx;
    l.xrows = epi == QH_EPI_ARGMAX ? out_rows : nullptr;
    l.m = (int)m;
    l.y = y;
    l.ldy = (int)(epi == QH_EPI_SILU ? w->rows / 2 : w->rows);
    l.keys = (unsigned long long*)keys;
    l.argmax_table = (unsigned long long*)sc.argmax;
    l.epi = epi;
    l.stream = (hipStream_t)stream;
    l.bf16_magic = 0x43004300u;
    l.cus = ctx->cus;
    l.pf_shape = ctx->pf_shape;
    l.sk_part = (float*)sc.stream_k;
    l.sk_count = (unsigned*)((uint8_t*)sc.stream_k + PF_SK_PART_BYTES);
    l.x16 = sc.x16;
    l.x16_bytes = X16_SCRATCH_BYTES;
    l.lora_ldm = (int)m;
    l.stream_k = ctx->stream_k;
    l.nib_mask = 0x000F000Fu;
    l.ks = 1;
    l.whole = whole;
    l.skinny = use_skinny(ctx, w, m, epi, whole);
    if (l.skinny) {
        Partition p = skinny_partition(ctx, w, m, epi == QH_EPI_PLAIN && !whole);
        l.tile_waves = p.tile_waves;
        l.waves = p.waves;
        l.split = p.split;
        l.groups_per_wave = p.groups_per_wave;
        l.tiles_per_wave = p.tiles_per_wave;
        // 16-byte row runs need a 16-byte aligned y (its rows are: the row count is a multiple of 16)
        // (one token: the LDS round trip costs more than it saves, measured 3% on small matrices)
        l.stage_out = epi == QH_EPI_PLAIN && m > 1 && ((uintptr_t)y & 15) == 0;
    } else {
        l.tile_waves = 4;
        l.waves = 4;
        l.tiles_per_wave = SKINNY_TILES;
        l.split = 1;  // the prefill launcher sets it (K-sliced plain products write several partials)
    }
    return l;
}

extern "C" int qh_mat_split(const qh_ctx* ctx, const qh_mat* m, size_t n) {
    if (!ctx || !m) return fail(QH_EINVAL, "split: null");
    if (n == 0) return 1;
    if (use_skinny(ctx, m, n, QH_EPI_PLAIN, 0)) return skinny_partition(ctx, m, n, true).split;
    if (n > (size_t)PF_KS_MAX_M || n > (1u << 24)) return 1;
    Launch l = make_launch(ctx, m, nullptr, m->cols, n, nullptr, nullptr, QH_EPI_PLAIN, nullptr, 0, nullptr,
                           ctx_scratch(ctx));
    l.dry_run = 1;
    if (hipError_t e = launch(l); e != hipSuccess) return fail(QH_EHIP, "split: %s", hipGetErrorString(e));
    return l.split;
}

extern "C" int qh_mat_kernel(const qh_ctx* ctx, const qh_mat* m, size_t n, int epi, int whole) {
    if (!ctx || !m) return fail(QH_EINVAL, "kernel: null");
    if (epi != QH_EPI_PLAIN && epi != QH_EPI_SILU && epi != QH_EPI_ARGMAX) return fail(QH_EINVAL, "epilogue %d", epi);
    return use_skinny(ctx, m, n, epi, whole) ? QH_KERNEL_SKINNY : QH_KERNEL_PREFILL;
}

extern "C" size_t qh_part_len(const qh_ctx* ctx, const qh_mat* const* mats, size_t count, size_t max_tok) {
    size_t len = 0;
    for (size_t i = 0; ctx && mats && i < count; i++) {
        if (!mats[i]) continue;
        // decode sizes: the largest split x tokens over every token count the skinny kernel takes (its partition
        // can depend on the token count, e.g. under QH_SKINNY_PLAIN_WK); prefill sizes up to PF_KS_MAX_M tokens: at
        // most PF_KS_MAX partials and PF_KS_ROWS partial rows; beyond: one
        size_t rows = std::max(max_tok, std::min((size_t)PF_KS_MAX * std::min(max_tok, (size_t)PF_KS_MAX_M),
                                                 (size_t)PF_KS_ROWS));
        for (size_t n = 1; n <= std::min(max_tok, (size_t)SKINNY_MAX_M); n++)
            if (use_skinny(ctx, mats[i], n, QH_EPI_PLAIN, 0))
                rows = std::max(rows, (size_t)skinny_partition(ctx, mats[i], n, true).split * n);
        len = std::max(len, rows * mats[i]->rows);
    }
    return len;
}

// qh_gemm's checks and launch, with the scratch (argmax table, stream-K partials and counters) at `sc`.
int qh::gemm_with_scratch(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n,
                          const int32_t* out_rows, size_t n_out, void* y, int epi, uint64_t* keys, int whole,
                          const Scratch& sc, const qh_lora* lora) {
    if (!ctx || !w || !x || !y) return fail(QH_EINVAL, "gemm: null");
    if (epi != QH_EPI_PLAIN && epi != QH_EPI_SILU && epi != QH_EPI_ARGMAX) return fail(QH_EINVAL, "epilogue %d", epi);
    if (epi == QH_EPI_ARGMAX && !keys) return fail(QH_EINVAL, "argmax without keys");
    if (epi == QH_EPI_SILU && w->rows % 16) return fail(QH_EINVAL, "SwiGLU of %zu rows", w->rows);
    if (ldx == 0) ldx = w->cols;
    if (ldx < w->cols || ldx % 8 || (uintptr_t)x % 16)
        return fail(QH_EINVAL, "x rows of %zu elements at %p: 16-byte aligned rows of at least %zu", ldx, x, w->cols);
    const size_t m = epi == QH_EPI_ARGMAX ? n_out : n;
    if (m == 0) return 1;
    if (epi == QH_EPI_ARGMAX && m > (size_t)ARGMAX_MAX_TOK)
        return fail(QH_EINVAL, "argmax over %zu logit rows: at most %d", m, ARGMAX_MAX_TOK);
    if (m > (1u << 24) || w->rows > (1u << 30) || ldx > (1u << 30)) return fail(QH_EINVAL, "gemm: sizes too large");
    // the prefill kernel addresses activation rows (the n token rows, also those the argmax gathers) with 32-bit byte
    // offsets from x
    if (!use_skinny(ctx, w, m, epi, whole) && ((std::max(n, m) - 1) * ldx + w->cols) * 2 > 0xffffffffu)
        return fail(QH_EINVAL, "gemm: %zu token rows of %zu elements: x must fit in 4 GiB", n, ldx);
    Launch l = make_launch(ctx, w, x, ldx, m, out_rows, y, epi, keys, whole, stream, sc);
    if (lora) {
        if (epi == QH_EPI_ARGMAX) return fail(QH_EINVAL, "gemm lora: the argmax epilogue takes no adapter");
        if (!lora->xa || !lora->b_f16 || !lora->tab || !lora->tok_slot || !lora->slot_scale || lora->split < 1)
            return fail(QH_EINVAL, "gemm lora: null or %d splits", lora->split);
        if (lora->rank != 8 && lora->rank != 16 && lora->rank != 32 && lora->rank != 64)
            return fail(QH_EINVAL, "LoRA rank %d: ranks 8, 16, 32 and 64 are served", lora->rank);
        if (lora->m_cols < 1 || lora->m_cols > 256)
            return fail(QH_EINVAL, "gemm lora: %d columns of xa (at most 256)", lora->m_cols);
        l.lora_xa = lora->xa;
        l.lora_split = lora->split;
        l.lora_cols = lora->m_cols;
        l.lora_rank = lora->rank;
        l.lora_b = lora->b_f16;
        l.lora_tab = lora->tab;
        l.lora_tok_slot = lora->tok_slot;
        l.lora_slot_scale = lora->slot_scale;
        l.lora_stage = lora->split == 1 && (lora->m_cols == 4 || lora->m_cols == 8 || lora->m_cols == 16 ||
                                            lora->m_cols == 32) && ((uintptr_t)lora->xa & 15) == 0;
    }
    hipError_t e = launch(l);
    if (e != hipSuccess) return fail(QH_EHIP, "gemm launch: %s", hipGetErrorString(e));
    return l.split;
}

extern "C" int qh_gemm(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n,
                       const int32_t* out_rows, size_t n_out, void* y, int epi, uint64_t* keys, int whole) {
    if (!ctx) return fail(QH_EINVAL, "gemm: null");
    return gemm_with_scratch(ctx, stream, w, x, ldx, n, out_rows, n_out, y, epi, keys, whole,
                             ctx_scratch(ctx));
}

extern "C" int qh_gemm_lora(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n, void* y,
                            int epi, int whole, const qh_lora* lora) {
    if (!ctx) return fail(QH_EINVAL, "gemm lora: null");
    return gemm_with_scratch(ctx, stream, w, x, ldx, n, nullptr, 0, y, epi, nullptr, whole,
                             ctx_scratch(ctx), lora);
}

extern "C" int qh_put_block(qh_ctx* ctx, void* stream, qh_mat* m, const qh_quant* q, const uint8_t* zeros,
                            size_t block, const size_t* rows16) {
    if (!ctx || !m || !q || !zeros || !rows16) return fail(QH_EINVAL, "put block: null");
    if (is_i8(m->wt) || is_bf16(m->wt) || q->bits != 4) return fail(QH_EINVAL, "put block: int4 matrices only");
    if (q->cols != m->cols || (block + 1) * TILE > m->rows)
        return fail(QH_EINVAL, "block %zu of a matrix of %zu rows", block, m->rows);
    const size_t qgroups = q->cols / (size_t)q->group;
    for (int r = 0; r < TILE; r++) {
        if (rows16[r] >= q->rows) return fail(QH_EINVAL, "put block: row %zu of %zu", rows16[r], q->rows);
        if (!has_zeros(m->wt))
            for (size_t g = 0; g < qgroups; g++)
                if (zeros[rows16[r] * qgroups + g] != 8)
                    return fail(QH_EINVAL, "rows with zero points for a symmetric matrix");
    }
    // one tile's codes are contiguous; its scales and zero points are one run per quad of 4 groups, a quad's tiles
    // side by side (layout.h), so they go as strided copies
    const size_t tiles = m->rows / TILE, nq = quads(m->cols / QG);
    const size_t cb = m->code_bytes / tiles, sb = m->scale_bytes / tiles, zb = m->zero_bytes / tiles;
    const size_t sq = sb / nq, zq = zb / nq;  // bytes of one tile's run in one quad
    HIP_TRY(hipEventSynchronize(m->staged));  // the previous block's copies have left the staging buffer
    uint8_t* st = m->stage;
    if (!f32_scales(m->wt))
        for (int r = 0; r < TILE; r++)
            for (size_t g = 0; g < qgroups; g++) {
                const float sc = q->scales[rows16[r] * qgroups + g];
                if (bf16_to_f32(f32_to_bf16(sc)) != sc)
                    return fail(QH_EINVAL, "put block: a scale bf16 does not hold in a bf16-scaled matrix");
            }
    if (int e = qh_pack_quant(q, has_zeros(m->wt) ? zeros : nullptr, rows16, TILE, m->wt, st, st + cb, st + cb + sb))
        return e;
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(hipMemcpyAsync((uint8_t*)m->codes + block * cb, st, cb, hipMemcpyHostToDevice, s));
    // the staged tile was packed alone (one tile: its quads' runs are consecutive)
    HIP_TRY(hipMemcpy2DAsync((uint8_t*)m->scales + block * sq, tiles * sq, st + cb, sq, sq, nq, hipMemcpyHostToDevice,
                             s));
    if (zb)
        HIP_TRY(hipMemcpy2DAsync((uint8_t*)m->zeros + block * zq, tiles * zq, st + cb + sb, zq, zq, nq,
                                 hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(m->staged, s));
    m->valid = std::max(m->valid, (block + 1) * TILE);
    return QH_OK;
}
