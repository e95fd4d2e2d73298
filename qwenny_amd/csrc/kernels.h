// Launch interface of the product kernels (kernels.hip), used by the C ABI (api.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qh {

// Kernel storage format: bit flags. int4 symmetric with bf16 scales is F_I4 (0).
enum {
    F_I4 = 0,
    F_I8 = 1,     // int8 codes (stored q + 128), 2 KiB blocks
    F_ZP = 2,     // int4 with zero points
    F_S32 = 4,    // f32 scales (else bf16)
    F_PERCH = 8,  // int8 with one scale per row: exact integer weights, the row's scale after the sum
    F_BF16 = 16,  // dense bf16 weights (4 KiB blocks, no scales): B fragments as loaded
};

struct Launch {
    const void* codes;
    const void* scales;
    const uint16_t* zeros;  // F_ZP only
    int fmt;                // F_* flags
    int rows;               // packed rows (outputs), multiple of 16
    int cols;               // K, multiple of 128
    int valid;              // rows that count for the argmax
    const void* x;          // bf16 activations
    int ldx;                // elements between x rows
    const int32_t* xrows;   // x row of token t (argmax logit rows), or null: t
    int m;                  // tokens
    void* y;
    int ldy;                // elements between y rows
    unsigned long long* keys;
    unsigned long long* argmax_table;  // [ARGMAX_SPREAD][ARGMAX_MAX_TOK], zero between launches
    int epi;                // enum qh_epi
    int split;              // grid split-K (plain products only)
    int waves;              // waves per workgroup (skinny kernel): tile_waves over tiles x waves / tile_waves over K
    int tile_waves;
    int groups_per_wave;    // skinny kernel: 4, or 1 when the group count is not a multiple of 4
    int tiles_per_wave;     // skinny kernel: SKINNY_TILES, or 1 (plain int8 and bf16 products of 1-2 tokens)
    int nc;                 // skinny kernel: super-chunks of K (groups / (wave rows x groups_per_wave)); set at launch
    int stage_out;          // skinny kernel, plain products: partials written through LDS in 16-byte row runs
    int cus;                // compute units (the prefill shape choice)
    int pf_shape;           // prefill workgroup shape: 0 chosen by size, else forced (kernels.hip prefill_epi)
    // prefill stream-K (kernels.hip prefill_kernel): scratch of partial tiles (PF_SK_PART_BYTES) and PF_SK_ITEMS_MAX
    // item counters (zero between launches); stream_k = 0 turns it off, above 1 it is the fix-up cost (tuning). Set by the launcher: dp_items, sk_items,
    // sk_wgs and the stream-K ranges (sk_q units per workgroup, one more for the first sk_r).
    float* sk_part;
    unsigned* sk_count;
    int stream_k;
    int dp_items, sk_items, sk_wgs, sk_q, sk_r;
    // plain prefill products of few tokens: whole items cut into ks slices of K, slice s writing partial y[s] (the
    // split-K contract; ks = 1: none). whole: the caller wants one partial. dry_run: plan only (l.split), no launch.
    int ks, whole, dry_run;
    // an unmerged LoRA adapter's delta fused into the epilogue (lora_rank 0: none): plain products add it to split 0,
    // SwiGLU products to gate and up before the activation (kernels.hip lora_delta16 / lora_delta32)
    const float* lora_xa;        // the stacked A product's partials [lora_split][lora_ldm][lora_cols]
    int lora_split, lora_cols, lora_rank;
    int lora_ldm;                // token rows between xa's partials (m, or the whole step's when run in token chunks)
    int skinny;                  // the skinny kernel takes the product (else the prefill kernel)
    int lora_stage;              // prefill: the item's xa rows staged in LDS (one split, 4 to 32 columns, aligned)
    const uint16_t* lora_b;      // B f16 [rows][lora_rank], the product's row order
    const int* lora_tab;         // module end rows (3 used), then each module's first column of xa (-1: none)
    const int* lora_tok_slot;
    const float* lora_slot_scale;
    // f16 copies of the activations for prefill launches with f16 operands (kernels.hip prefill_h16): x16_bytes of
    // scratch; longer steps run in token chunks that fit it
    void* x16;
    size_t x16_bytes;
    uint32_t bf16_magic;    // 0x43004300: the bf16 pair (128, 128) (see kernels.hip i4_biased)
    uint32_t nib_mask;      // 0x000F000F
    hipStream_t stream;
};

// The argmax epilogue's scratch table: rows the workgroups spread their maxima over, and the logit rows of a step
// it takes at most (the reference's MAX_OUT).
constexpr int ARGMAX_SPREAD = 64;
constexpr int ARGMAX_MAX_TOK = 64;

// Prefill stream-K scratch: bytes of partial tiles (two slots per stream-K workgroup of a launch) and item counters.
constexpr size_t PF_SK_PART_BYTES = (size_t)128 << 20;
constexpr int PF_SK_ITEMS_MAX = 4096;
// Cost of stream-K's partials in units of one group's compute (the launcher's choice between whole items and stream-K).
constexpr int PF_SK_FIXUP = 12;
constexpr double PF_SK_PIECE_S = 1e-6;  // stream-K fix-up: seconds per partial summed beyond three (measured)
// K slices of plain prefill products (at most PF_KS_MAX, up to PF_KS_MAX_M tokens, slices x tokens at most PF_KS_ROWS
// partial rows), and the estimated cost of a slice's extra pipeline start and partial, in the same units.
constexpr int PF_KS_MAX = 16;
constexpr int PF_KS_ROWS = 2048;
// More than 4 slices only when each keeps this many groups of K (a slice's start and partial are not amortised over
// fewer: 8 slices of 40 groups measured 3-17% slower than 4 at 49-64 tokens).
constexpr int PF_KS_MIN_G = 8;
constexpr int PF_KS_MAX_M = 512;
constexpr int PF_KS_COST = 2;
// The rates that price the slices' extra partials in those units: one CU's MFMA rate under load, and HBM.
constexpr double PF_KS_CU_FLOPS = 4e12, PF_KS_HBM = 5e12;

// Tokens the skinny kernel takes at most (three 16-token blocks per MFMA pass); larger steps go to the prefill kernel.
constexpr int SKINNY_MAX_M = 48;
// Split-K plain and SwiGLU products of 33-48 tokens on int4 and grouped int8 matrices of at least this many weights
// take the prefill kernel (faster there; api.hip use_skinny).
constexpr size_t PF_FROM33_WEIGHTS = (size_t)1 << 26;
// 16-row tiles per wave in the skinny kernel, and its pipeline depth (groups whose loads are in flight + 1).
#ifndef QH_SKINNY_TILES
#define QH_SKINNY_TILES 2
#endif
constexpr int SKINNY_TILES = QH_SKINNY_TILES;
// Most bytes of LDS the skinny kernel stages activations in.
constexpr size_t SKINNY_X_LDS = 64 * 1024;

// Dynamic LDS of a skinny launch: the staged activations and the K reduction.
size_t skinny_lds(const Launch& l);

enum { EPI_PLAIN = 0, EPI_SILU = 1, EPI_ARGMAX = 2 };

// Scratch of a product launch: the argmax table (ARGMAX_SPREAD x ARGMAX_MAX_TOK u64, and 256 bytes more:
// ARGMAX_SCRATCH_BYTES in all), and the stream-K partials (PF_SK_PART_BYTES) followed by PF_SK_ITEMS_MAX item counters
// (PF_SK_SCRATCH_BYTES in all); every counter and table entry zero between launches.
struct Scratch {
    void* argmax;
    void* stream_k;
    void* x16;  // X16_SCRATCH_BYTES: f16 activations of prefill launches with f16 operands
};
constexpr size_t ARGMAX_SCRATCH_BYTES = (size_t)ARGMAX_SPREAD * ARGMAX_MAX_TOK * 8 + 256;
constexpr size_t PF_SK_SCRATCH_BYTES = PF_SK_PART_BYTES + PF_SK_ITEMS_MAX * sizeof(unsigned);
// f16 activations of a prefill launch with f16 operands: 3276 tokens of K = 5120 (the 27B [gate; up] product) at once
constexpr size_t X16_SCRATCH_BYTES = (size_t)32 << 20;

// The kernels of one storage format F and epilogue EPI: the skinny kernel for m <= SKINNY_MAX_M, else the prefill
// kernel.
template <int F, int EPI>
hipError_t launch_epi(Launch& l);

// launch_epi for l.fmt and l.epi; sets l.split to the partials the launch writes.
hipError_t launch(Launch& l);

}  // namespace qh
