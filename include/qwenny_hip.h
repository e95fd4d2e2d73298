/*
 * qwenny_hip.h — C ABI of the MI355X (gfx950) quantized-weight matrix products.
 *
 * This is the boundary that replaces qwenny's CUDA product runtime (`src/cuda/core.rs`) behind the same Rust call
 * sites (`Stack::gemm`, `Mat::stack`, `Mat::marlin_rows`, `Gemm::put_block`). Every entry point takes plain pointers
 * and sizes; device pointers are opaque `void*` (HIP device memory), streams are `hipStream_t` passed as `void*`.
 * No C++ exception crosses this boundary: functions return an int status (>= 0 success, < 0 error) and
 * `qh_last_error()` describes the last failure of the calling thread.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   Quant (checkpoint.rs:21-31), Quant::row_into (:39-47), Quant::zero_points (:72-82), Quant::stack (:85-99),
 *   Checkpoint::packed_matrix (:408-453), row_order (cuda/core.rs:108-114), Mat (:94-104),
 *   Mat::new / pack (:127-135, :338-389), Mat::marlin_rows (:140-153), Mat::marlin (:159-164), Mat::int8 (:168-191),
 *   part_len (:315-318), Gemm::load (:436-481), Gemm::run / run_split (:485-561), Gemm::put_block (:619-657),
 *   Gemm::block_stage (:675-680); the kernels the engine launches on the products' partials: add_rmsnorm and
 *   sum_parts (kernels/qwen.cu:57-80, :141-143), the LoRA epilogue (kernels/lora.cuh:52-113); and the trainer's
 *   dequant (kernels/qwen_train.cu:84-103).
 */
#ifndef QWENNY_HIP_H
#define QWENNY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (negative = error). */
#define QH_OK 0
#define QH_EINVAL -1   /* bad argument or shape the layout does not take */
#define QH_EHIP -2     /* a HIP runtime call failed */
#define QH_ENOMEM -3   /* device or host allocation failed */
#define QH_ENOTFIT -4  /* the matrix does not fit this storage (e.g. non-integer zero points) */

/* How a matrix is stored for the kernels (core.rs:65-79 `Wt`; its F16 is QH_WT_BF16 here). */
enum qh_wt {
    QH_WT_I8 = 1,  /* int8 stored q + 128, an f32 scale per row and 128 columns (core.rs Wt::I8) */
    QH_WT_I4 = 2,  /* symmetric int4 (zero point 8), bf16 scale per row and 128 columns (core.rs Wt::Marlin) */
    QH_WT_I4Z = 3, /* int4 with a 4-bit zero point per row and 128 columns (core.rs Wt::MarlinZ) */
    QH_WT_I4_S32 = 4, /* QH_WT_I4 with f32 scales: scales that bf16 does not hold exactly (f16 / f32 checkpoints) */
    QH_WT_I4Z_S32 = 5, /* QH_WT_I4Z with f32 scales */
    QH_WT_BF16 = 6     /* dense 16-bit weights kept bf16, no scales (core.rs Wt::F16, which rounds them to f16) */
};

/* Epilogue of a product (core.rs:52-58 `Epi`). */
enum qh_epi {
    QH_EPI_PLAIN = 0,  /* f32 y[split][n][rows], split-K partials the consumer sums */
    QH_EPI_SILU = 1,   /* bf16 y[n][rows/2] = silu(gate) * up over row_order's interleaved tiles */
    QH_EPI_ARGMAX = 2  /* f32 logits y[n_out][rows] and the running argmax key per logit row in keys[] */
};

/* A quantized matrix [rows][cols] as stored (checkpoint.rs:21-31 `Quant`): w = q * scale + offset per group of a
 * row. q: [rows][cols * bits / 32] words, value c of a row in word c * bits / 32 at bit (c % (32 / bits)) * bits.
 * scales, offsets: [rows][cols / group] f32. */
typedef struct qh_quant {
    int32_t bits;
    int32_t group;
    size_t rows;
    size_t cols;
    const uint32_t* q;
    const float* scales;
    const float* offsets;
} qh_quant;

typedef struct qh_ctx qh_ctx;
typedef struct qh_mat qh_mat;

/* Read-only description of a device matrix (core.rs:94-104 `Mat`). */
typedef struct qh_mat_desc {
    int32_t wt;         /* enum qh_wt */
    size_t rows;        /* packed rows (outputs), a multiple of 16 */
    size_t cols;        /* columns (K), a multiple of 128 */
    size_t valid;       /* rows that count for the argmax (core.rs Mat::valid) */
    size_t code_bytes;  /* device bytes of the packed codes */
    size_t scale_bytes; /* device bytes of the scales */
    size_t zero_bytes;  /* device bytes of the zero points (0 unless QH_WT_I4Z or QH_WT_I4Z_S32) */
    int32_t per_channel; /* QH_WT_I8 with one scale per row (every group's equal): prefill products in exact
                          * integers with the row's scale after the sum; 0: a scale per row and 128 columns */
} qh_mat_desc;

/* The last error of the calling thread ("" if none). */
const char* qh_last_error(void);

/* ---- host-side weight formats (no GPU needed) ----------------------------------------------------------------- */

/* Checkpoint::packed_matrix (checkpoint.rs:408-453): compressed-tensors pack-quantized tensors into Quant fields.
 * packed: weight_packed [rows][words] int32; scale: weight_scale as f32 [rows * groups] (callers convert bf16/f16);
 * zp: weight_zero_point words or NULL (symmetric: zero 2^(bits-1)); zp_rows/zp_cols its shape (packed along rows:
 * [ceil(rows/per)][groups], or along groups: [rows][ceil(groups/per)]); cols: weight_shape[1] or 0 (from words);
 * group: 0 = one group per row (strategy "channel"). Writes bits/group/cols to *out and scales/offsets to the
 * caller's arrays [rows * groups]; out->q points at `packed`. */
int qh_quant_from_packed(const uint32_t* packed, size_t rows, size_t words, size_t cols, int bits, int group,
                         const float* scale, const uint32_t* zp, size_t zp_rows, size_t zp_cols, float* scales_out,
                         float* offsets_out, qh_quant* out);

/* Quant::zero_points (checkpoint.rs:72-82): z[rows * groups] if every offset is -z * scale for an integer z in
 * [0, 2^bits - 1] (within 1e-3). Returns 1 if so, 0 if not (z unspecified), < 0 on error. */
int qh_quant_zero_points(const qh_quant* q, uint8_t* z);

/* Quant::row_into (checkpoint.rs:39-47): row r dequantized into out[cols] (f32). */
int qh_quant_row_into(const qh_quant* q, size_t r, float* out);

/* Quant::to_bf16 (checkpoint.rs:50-68): all rows dequantized (row_into) and rounded to bf16 nearest even into
 * out[rows * cols], threaded over rows. */
int qh_quant_to_bf16(const qh_quant* q, uint16_t* out);

/* row_order (core.rs:108-114): packed row i <- original row out[i]. silu: gate/up interleaved per 16 rows. */
int qh_row_order(size_t rows, int silu, size_t* out);

/* Byte sizes of the gfx950 tile layout for a matrix of `rows` packed rows (a multiple of 16) and `cols` columns (a
 * multiple of 128). The codes of one matrix must fit in 4 GiB (the kernels use 32-bit offsets): QH_EINVAL beyond. */
int qh_packed_sizes(int wt, size_t rows, size_t cols, size_t* code_bytes, size_t* scale_bytes, size_t* zero_bytes);

/* The load-time repacker: rows `order[0..n)` of `q` (a Quant of bits 4 or 8, group a multiple of 128 or a whole row)
 * into the gfx950 tile layout (replaces pack_marlin, core.rs:245-311, and frags_int8, :223-242). wt QH_WT_I4 needs
 * zero points 8 everywhere, QH_WT_I4Z takes `zeros` [rows * groups] (Quant::zero_points), QH_WT_I8 needs zero points
 * 128; the _S32 storages keep f32 scales. codes / scales / zeros: buffers of qh_packed_sizes. Host-side,
 * multithreaded. */
int qh_pack_quant(const qh_quant* q, const uint8_t* zeros, const size_t* order, size_t n, int wt, void* codes,
                  void* scales, void* zeros_out);

/* The repacker's inverse for one packed row p: its stored values (int4 0..15 or int8 q + 128) into vals[cols], its
 * per-128-column scales as f32 into sc[cols / 128] and zero points into z[cols / 128] (8 or 128 when symmetric). */
int qh_unpack_row(int wt, size_t rows, size_t cols, const void* codes, const void* scales, const void* zeros,
                  size_t p, uint8_t* vals, float* sc, uint8_t* z);

/* Mat::new / pack int8 branch (core.rs:127-135, :338-389): dense bf16 [rows][cols] rows `order` requantized to
 * symmetric int8 per row and 128 columns (scale max|w| / 127, 1 if 0; q = round half away from zero, clamped to
 * +-127, stored + 128) into the QH_WT_I8 layout. */
int qh_pack_dense_int8(const uint16_t* bf16, size_t rows, size_t cols, const size_t* order, size_t n, void* codes,
                       void* scales);

/* Mat::new / pack 16-bit branch (core.rs:127-135, :370-381): dense bf16 [rows][cols] rows `order` into the
 * QH_WT_BF16 layout, bit for bit (the reference rounds them to f16). codes: qh_packed_sizes bytes. */
int qh_pack_dense_bf16(const uint16_t* bf16, size_t rows, size_t cols, const size_t* order, size_t n, void* codes);

/* The inverse for one packed row p of a QH_WT_BF16 matrix: its bf16 values into out[cols]. */
int qh_unpack_row_bf16(size_t rows, size_t cols, const void* codes, size_t p, uint16_t* out);

/* ---- device: context, matrices, products ---------------------------------------------------------------------- */

/* Gemm::load (core.rs:436-481): a context on `device` (makes it current on this thread). It holds the argmax scratch
 * table, the prefill's stream-K scratch (128 MiB of partial tiles and 4096 item counters) and 32 MiB
 * for the f16 activations of the prefill's SwiGLU launches, all returned to zero by every launch that uses them;
 * products on one context must therefore not run concurrently on two streams. */
int qh_open(int device, qh_ctx** out);
void qh_close(qh_ctx* ctx);

/* Mat::upload (core.rs:117-124): a device matrix from packed host buffers (qh_pack_*); `valid` rows count. */
int qh_mat_upload(qh_ctx* ctx, int wt, size_t rows, size_t cols, const void* codes, const void* scales,
                  const void* zeros, size_t valid, qh_mat** out);

/* Mat::marlin / Mat::int8 (core.rs:159-191): a stored int4 / int8 Quant, packed in row_order(silu) and uploaded.
 * int4 gives QH_WT_I4 (all zero points 8) or QH_WT_I4Z, their _S32 forms when a scale is not exact in bf16; int8
 * needs zero points 128. QH_ENOTFIT if it does not fit. */
int qh_mat_quant(qh_ctx* ctx, const qh_quant* q, int silu, qh_mat** out);

/* Mat::marlin_rows (core.rs:140-153): rows `rows[0..n)` (n a multiple of 16) of an int4 Quant with zero points
 * `zeros`, in a matrix of `cap` rows (a multiple of 16); the rest are room for qh_put_block and not valid. */
int qh_mat_quant_rows(qh_ctx* ctx, const qh_quant* q, const uint8_t* zeros, const size_t* rows, size_t n, size_t cap,
                      qh_mat** out);

/* Mat::new int8 (core.rs:127-135): dense bf16 [rows][cols] requantized to int8 (qh_pack_dense_int8), uploaded. */
int qh_mat_dense_int8(qh_ctx* ctx, const uint16_t* bf16, size_t rows, size_t cols, int silu, qh_mat** out);

/* Mat::new with int8 false (core.rs:127-135, Wt::F16): dense bf16 [rows][cols] packed in row_order(silu) as
 * QH_WT_BF16 (qh_pack_dense_bf16) and uploaded; the 16-bit matrices of a pre-quantized checkpoint (in_ba). */
int qh_mat_dense(qh_ctx* ctx, const uint16_t* bf16, size_t rows, size_t cols, int silu, qh_mat** out);

void qh_mat_free(qh_mat* m);
int qh_mat_describe(const qh_mat* m, qh_mat_desc* out);

/* Copy a device matrix's packed buffers back to the host (sizes from qh_mat_describe); zeros may be NULL. */
int qh_mat_download(const qh_mat* m, void* codes, void* scales, void* zeros);

/* Split-K factor a plain product of n tokens uses on m (core.rs Mat::split): the skinny kernel's K chunks where it
 * takes the product (qh_mat_kernel), 1-16 K slices (slices x tokens <= 2048) on the prefill kernel up to 512
 * tokens, 1 above. No launch; the same value qh_gemm returns. */
int qh_mat_split(const qh_ctx* ctx, const qh_mat* m, size_t n);

/* Which kernel a product of n tokens (qh_gemm's n, or n_out for QH_EPI_ARGMAX) with epilogue `epi` runs on m:
 * QH_KERNEL_SKINNY (exact products of the dequantized weights) or QH_KERNEL_PREFILL (weights rounded to bf16 once;
 * both within the bf16-operand bound). No counterpart in the reference, whose Marlin kernel serves every token count:
 * for callers and tests that need to know which numerics a product has. The skinny kernel takes up to 48 tokens,
 * except split-K plain and SwiGLU products of int4 and grouped int8 matrices of at least 2^26 weights from 33
 * tokens. No launch. */
#define QH_KERNEL_SKINNY 1
#define QH_KERNEL_PREFILL 2
int qh_mat_kernel(const qh_ctx* ctx, const qh_mat* m, size_t n, int epi, int whole);

/* part_len (core.rs:315-318): floats the plain products of `mats` write at most, for up to `max_tok` tokens. */
size_t qh_part_len(const qh_ctx* ctx, const qh_mat* const* mats, size_t count, size_t max_tok);

/* Gemm::run_split (core.rs:485-561): y = w . x on `stream`.
 *   x: bf16 [.][ldx] device (ldx = 0: cols); n tokens (rows of x);
 *   epi QH_EPI_PLAIN: y f32 [split][n][rows], returns split (1 when `whole`);
 *   epi QH_EPI_SILU: y bf16 [n][rows / 2];
 *   epi QH_EPI_ARGMAX: logit rows: token t reads x row out_rows[t] (int32 device, NULL: t) for t < n_out; y f32
 *     [n_out][rows]; keys[t] (u64 device, cleared by the caller) = max(keys[t], (ordered(v) << 32) | ~o) over the
 *     valid rows o (one launch for one int4 token row, n_out = 1, without an adapter; otherwise two: the product,
 *     then a one-workgroup fold of its per-workgroup maxima into keys).
 * Above 48 tokens x's rows 0 .. max(n, n_out) - 1 must lie within 4 GiB of x (32-bit offsets): QH_EINVAL beyond.
 * Returns the split (>= 1) or < 0. Launches only: no host synchronisation, no allocation (graph-capturable). */
int qh_gemm(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n, const int32_t* out_rows,
            size_t n_out, void* y, int epi, uint64_t* keys, int whole);

/* An unmerged LoRA adapter on a product (the arguments of the reference's lora_add / lora_silu kernels,
 * kernels/lora.cuh:52-113, src/cuda/qwen/lora.rs:143-190): xa, the stacked A product's partials f32
 * [split][n][m_cols] (m_cols <= 256) of the product's n tokens; b_f16, B f16 [rows][rank] in the product's row order
 * (rank 8, 16, 32 or 64); tab, 8 int32: each module's end row (ascending; unused INT_MAX), then its first column of xa
 * (-1: not adapted); for a SwiGLU product module 0 is the gate and 1 the up rows; the token's slot scale
 * slot_scale[tok_slot[t]] (0: no delta). All device pointers. */
typedef struct qh_lora {
    const float* xa;
    int32_t split;
    int32_t m_cols;
    const uint16_t* b_f16;
    int32_t rank;
    const int32_t* tab;
    const int32_t* tok_slot;
    const float* slot_scale;
} qh_lora;

/* qh_gemm with the LoRA delta s_t * B (A x) fused into the product's epilogue, computed in f32: QH_EPI_PLAIN adds it to
 * split 0 of the partials (what qh_gemm then qh_lora_add on y[0] make); QH_EPI_SILU adds it to gate and up before the
 * activation (what a whole plain product, then qh_lora_silu, make), with no f32 [gate; up] pass through memory.
 * Outputs whose delta is exactly zero (unadapted rows, tokens of slot scale 0) are the product's bit for bit.
 * QH_EPI_ARGMAX takes no adapter (QH_EINVAL). lora NULL: qh_gemm. Returns the split or < 0. Launch only. */
int qh_gemm_lora(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n, void* y, int epi,
                 int whole, const qh_lora* lora);

/* qh_gemm without allocation: no counterpart in the reference. For callers that cannot allocate device memory around
 * a product (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments,
 * checks, launch plans and results as qh_gemm, but the launch scratch (argmax table, stream-K partials
 * and counters, the f16 activations of prefill SwiGLU launches) lives in a static device array of the library
 * (160 MiB + 48.25 KiB per GPU, held until the process ends, set up by qh_open; every process that loads the library
 * reserves it) instead of the context's allocations; it calls no allocating routine. Products never need more scratch
 * than that (the launch planner sizes stream-K to it; longer SwiGLU steps run in token chunks; argmax takes at most 64
 * logit rows, QH_EINVAL beyond). Calls that overlap on one GPU share the array and race: serialise them (one
 * stream). */
int qh_gemm_noalloc(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n,
                    const int32_t* out_rows, size_t n_out, void* y, int epi, uint64_t* keys, int whole);

/* Gemm::put_block (core.rs:619-657): rewrite the 16-row block `block` of an int4 matrix made by qh_mat_quant_rows
 * with stored rows rows16[0..16) of q (zero points `zeros`), counting it as valid. Stages through the matrix's own
 * staging buffer (allocated at upload, like Gemm::block_stage): no allocation. */
int qh_put_block(qh_ctx* ctx, void* stream, qh_mat* m, const qh_quant* q, const uint8_t* zeros, size_t block,
                 const size_t* rows16);

/* The trainer's dequant (kernels/qwen_train.cu:84-103, called by src/cuda/qwen/train.rs:490-520): rows
 * [r0, r0 + n) of a quantized matrix in the checkpoint's layout (q [rows][words] u32, value c in word c * bits / 32
 * from the low bits; scales f32 and zero points u8 per (row, group)) into dense rows out [n][cols] on `stream`:
 * w = (q - zero) * scale in f32, stored bf16 (nearest even; out_f32 = 0) or f32. All pointers are device addresses,
 * q 4-byte and out 16-byte aligned; group a multiple of 32 / bits. Launch only. */
int qh_dequant(void* stream, const uint32_t* q, const float* scales, const uint8_t* zeros, size_t rows, size_t words,
               size_t cols, int group, int bits, size_t r0, size_t n, void* out, int out_f32);

/* Consumers of the plain products' partials x [splits][n][.] f32 (device pointers, 16-byte aligned), on `stream`:
 * sum_parts (kernels/qwen.cu:141-143): y [n][ld] = sum over s of x[s] (ld a multiple of 4);
 * add_rmsnorm (kernels/qwen.cu:57-80), the residual step: h [n][hidden] += sum over s of x[s] (h + x[0] first, then
 * x[1], ..), then y [n][hidden] bf16 = w_next * h / sqrt(mean(h^2) + eps) (hidden a multiple of 4). The sums are
 * those of the reference, in its order. Launch only. */
int qh_sum_parts(void* stream, const float* x, int splits, size_t n, size_t ld, float* y);
int qh_add_rmsnorm(void* stream, float* h, const float* x, int splits, size_t n, size_t hidden, const float* w_next,
                   void* y_bf16, float eps);

/* The LoRA consumers (kernels/lora.cuh:52-113, launched by src/cuda/qwen/lora.rs:143-190): an unmerged adapter adds
 * s_t * B (A x) to a plain product for the tokens t whose slot uses it (s_t = slot_scale[tok_slot[t]]; 0: nothing
 * added). xa: the stacked A product's partials f32 [split][n][m_cols] (m_cols <= 256); b_f16: B f16 [rows][rank] in
 * the product's row order (rank 8, 16, 32 or 64; 16-byte aligned); tab: 8 int32, each module's end row (ascending;
 * unused INT_MAX), then its first column of xa (-1: not adapted; a column range must lie within m_cols). rows: a
 * multiple of 16 (the products' row count). y 16-byte aligned with ldy a multiple of 4, mid 8-byte aligned (QH_EINVAL
 * otherwise). All pointers are device addresses. The delta is computed in f32.
 * lora_add: y [n][ldy] f32, the plain product's split 0, row o += s_t * B[o] . xa[t][off(o) ..].
 * lora_silu: y [n][ldy] f32, a plain [gate; up] product packed in row_order(rows, 1) (split 1), read; mid [n][rows / 2]
 * bf16 = silu(gate + delta) * (up + delta) for every token t < n, as the SwiGLU epilogue writes it.
 * Launch only. */
int qh_lora_add(void* stream, const float* xa, int split, int m_cols, const uint16_t* b_f16, int rank, size_t rows,
                const int32_t* tab, const int32_t* tok_slot, const float* slot_scale, size_t n, float* y, size_t ldy);
int qh_lora_silu(void* stream, const float* xa, int split, int m_cols, const uint16_t* b_f16, int rank, size_t rows,
                 const int32_t* tab, const int32_t* tok_slot, const float* slot_scale, size_t n, const float* y,
                 size_t ldy, void* mid_bf16);

/* ---- graph capture --------------------------------------------------------------------------------------------- */

/* Replaces the capture and replay inside Graphs::run (src/cuda/core.rs:1151-1192); the graph cache around it (keys,
 * LRU, memory floor) stays with the caller. The launches the calling thread makes on `stream` (not the null stream)
 * between qh_graph_begin and qh_graph_end become one graph (thread-local capture mode), instantiated for replay with
 * qh_graph_launch on any stream; qh_graph_free releases it. Every launch entry point of this library may be captured:
 * none allocates, synchronises or records a memset. Buffers and arguments are those of the capture at every replay;
 * argmax keys keep their running maximum, so a caller resets them between replays as between eager calls. */
typedef struct qh_graph qh_graph;
int qh_graph_begin(void* stream);
int qh_graph_end(void* stream, qh_graph** out);
int qh_graph_launch(const qh_graph* g, void* stream);
void qh_graph_free(qh_graph* g);

/* ---- measurement aid ------------------------------------------------------------------------------------------ */

/* No counterpart in the reference: a read-only kernel for the benchmark and its profiles. It reads `tiles` x `groups`
 * 1 KiB blocks at buf (device, 16-byte aligned) with the decode kernel's 16-byte non-temporal loads and stores
 * nothing (sink: device u32 scratch, never written in practice). pattern 0: contiguous, 8 KiB per wave (tiles x
 * groups a multiple of 32; the FETCH_SIZE calibration); pattern 1: the tile-layout walk and partition of the
 * one-token plain product (2 tiles x 4 groups per wave; tiles even, groups a multiple of 4; the read floor of a
 * product over the same code bytes). Launch only. */
int qh_diag_read(void* stream, const void* buf, size_t tiles, size_t groups, int pattern, uint32_t* sink);

#ifdef __cplusplus
}
#endif

#endif /* QWENNY_HIP_H */
