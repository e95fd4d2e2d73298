// The quantized-weight matrix products on gfx950 (MI355X): y = W . x for bf16 activations x [m][K] and int4 / int8 /
// dense bf16 weights W [rows][K] in the tile layout of layout.h, f32 accumulation.
//
// Both kernels compute D = X . W^T with the activations as the MFMA A operand and the weights as the B operand, so the
// packed tile block is the B operand as loaded. The skinny kernel runs v_mfma_f32_16x16x32_bf16 (A 16 tokens x 32 k,
// B 32 k x 16 outputs; lane l of a wave holds D[row 4 (l / 16) + r][output l % 16], r = 0..3, MFMA row 4 (t % 4) +
// t / 4 holding token t from two tokens, so that row r of lane l is token 4 r + l / 16), the prefill kernel
// v_mfma_f32_32x32x16_bf16 (its layout below).
//
// skinny_kernel (m <= 48, decode, MTP verify and small batches; from 33 tokens not the plain and SwiGLU products of
// matrices of 2^26 weights and more, which the prefill kernel takes): HBM-bound. The weights are streamed once with 16-byte loads (a wave
// reads each (tile, group) block as one contiguous KiB) and turned into bf16 (128 + q) with one and-or per two values;
// the MFMA sums x (128 + q) exactly in f32 per 128-column group, and the group's scale and zero point are applied
// after it: acc += s (D - (128 + z) sum_k x), where sum_k x comes from one more MFMA against ones per k32 step (shared
// by the wave's tiles). K is split over the waves of a workgroup (reduced through LDS) and, for plain products, over
// the grid (the split-K partials of the output contract). The activations are staged in LDS once per workgroup, or,
// for one token of int4 without zero points, by each wave for itself (no workgroup barrier).
//
// prefill_kernel (m > 48, and those 33-48-token products): MFMA-bound. A workgroup computes up to 256 tokens x 256 outputs (8 waves of 256 x 32, or
// 256 x 192 on 12 waves of 128 x 32, or smaller tiles for short steps); the activation tile goes global -> LDS directly
// (global_load_lds) into double-buffered, XOR-swizzled 64-column stages, each wave dequantizes its own outputs'
// weights straight from global memory into bf16 registers ((q - z) s in f32, rounded once), the workgroups are mapped
// XCD-aware (an XCD's workgroups share a token tile's activations in its L2), and a badly filled last round is spread
// over the resident workgroups by groups of K (stream-K). On 256 x 256 items the two waves of each SIMD ping-pong: one
// runs a group's MFMAs while the other dequantizes its next group's weights.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "kernels.h"
#include "layout.h"

namespace qh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Kernel format F: bit flags of the storage (kernels.h F_*).

__device__ __forceinline__ f32x4 mfma(u32x4 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
}

// int4 word (layout.h nibble order) -> bf16 (128 + q) of columns 0..7: each 16-bit half's nibble put under the
// exponent of 128 by one and-or (v_and_or_b32) per pair: 3 shifts and 4 and-ors for 8 values. The mask (0x000F000F)
// and the bf16 pair (128, 128) = 0x43004300 come from the host: with both known, the compiler would split each and-or
// into an and and an or (a gfx9 VOP3 instruction takes no literal).
__device__ __forceinline__ bf16x8 i4_biased(uint32_t w, uint32_t mask, uint32_t magic) {
    u32x4 v;
    v.x = (w & mask) | magic;
    v.y = ((w >> 4) & mask) | magic;
    v.z = ((w >> 8) & mask) | magic;
    v.w = ((w >> 12) & mask) | magic;
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float byte_f(uint32_t w, int b) { return (float)((w >> (8 * b)) & 255u); }

// int8 words (columns 0..3, 4..7; stored q + 128) -> bf16 (128 + q), exact (integers below 256)
__device__ __forceinline__ bf16x8 i8_biased(uint32_t a, uint32_t b) {
    auto pair = [](uint32_t v, int b0) {  // one v_cvt_pk_bf16_f32 per pair
        const f32x2 f = {byte_f(v, b0), byte_f(v, b0 + 1)};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
    };
    const u32x4 r = {pair(a, 0), pair(a, 2), pair(b, 0), pair(b, 2)};
    return __builtin_bit_cast(bf16x8, r);
}

// two f32 -> the 16-bit pair of the prefill operands: bf16 (v_cvt_pk_bf16_f32) or, H16, f16 (v_cvt_pk_f16_f32), both
// nearest even
template <bool H16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    const f32x2 f = {a, b};
    if constexpr (H16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// int4 word -> 16-bit (bf16, or f16 with H16) of (q - z) s = q s + off, in f32 then rounded once
template <bool H16 = false>
__device__ __forceinline__ bf16x8 i4_scaled(uint32_t w, float s, float off) {
    uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    // opaque to the optimizer: otherwise it folds the nibble mask into each byte extraction and loses the one-op
    // byte-to-float conversions (v_cvt_f32_ubyte0..3)
    asm("" : "+v"(lo));
    asm("" : "+v"(hi));
    // each pair is one two-wide conversion (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32), so no halves are spliced afterwards
    auto pair = [&](uint32_t v, int b0, int b1) {
        return pack2<H16>(__builtin_fmaf(byte_f(v, b0), s, off), __builtin_fmaf(byte_f(v, b1), s, off));
    };
    const u32x4 r = {pair(lo, 0, 2), pair(hi, 0, 2), pair(lo, 1, 3), pair(hi, 1, 3)};
    return __builtin_bit_cast(bf16x8, r);
}

template <bool H16 = false>
__device__ __forceinline__ bf16x8 i8_scaled(uint32_t a, uint32_t b, float s, float off) {
    auto pair = [&](uint32_t v, int b0) {  // one two-wide conversion per pair, as i4_scaled
        return pack2<H16>(__builtin_fmaf(byte_f(v, b0), s, off), __builtin_fmaf(byte_f(v, b0 + 1), s, off));
    };
    const u32x4 r = {pair(a, 0), pair(a, 2), pair(b, 0), pair(b, 2)};
    return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ float bf16_bits_f(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// Order-preserving map of a float to an unsigned int; the argmax key (value, then lowest index on ties).
__device__ __forceinline__ unsigned long long argmax_key(float v, int o) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (0xffffffffu - (uint32_t)o);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

// The max over the 16 lanes of a lane's row group (lanes that share l / 16).
__device__ __forceinline__ unsigned long long group16_max(unsigned long long k) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) k = max_u64(k, __shfl_xor(k, o));
    return k;
}

// The argmax across workgroups without every workgroup hitting the same cache line of keys[]: a workgroup folds its
// per-token maxima into one of ARGMAX_SPREAD rows of a scratch table (row = its index mod ARGMAX_SPREAD) with
// non-returning device-scope atomics, and a one-workgroup kernel launched right after the product on the same stream
// (argmax_fold_kernel; the kernel boundary orders the table updates before its reads) folds the table into keys[]
// (one atomicMax per token), zeroing it as it reads: the next launch (or graph replay) starts from a clean table. One
// product at a time per context uses the table (launches on one stream). Against a last-workgroup protocol in the
// product itself (each workgroup's table updates returned, then a returning count on one counter), the extra launch
// measured faster: the 27B head 3.8 us per step less. The one-token argmax on skinny_m1w_kernel needs neither: each
// workgroup reads keys[0] once at its start (a lower bound of the final key, as keys only grow) and sends its maximum
// straight to keys[0] only when above it, so after the first round of workgroups few atomics reach the line (the 27B
// headline step 0.2517 -> 0.2495 ms against the table and the fold launch).
__device__ __forceinline__ void argmax_spread_max(unsigned long long* table, int tok, unsigned long long k) {
    const int row = (blockIdx.y * gridDim.x + blockIdx.x) % ARGMAX_SPREAD;
    (void)__hip_atomic_fetch_max(table + row * ARGMAX_MAX_TOK + tok, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void argmax_spread_max(const Launch& a, int tok, unsigned long long k) {
    argmax_spread_max(a.argmax_table, tok, k);
}

static __global__ __launch_bounds__(1024) void argmax_fold_kernel(unsigned long long* table, unsigned long long* keys,
                                                                 int m) {
    __shared__ unsigned long long best[ARGMAX_MAX_TOK];
    for (int t = threadIdx.x; t < m; t += blockDim.x) best[t] = 0;
    __syncthreads();
    // read and cleared at the coherence point where the product's atomics were performed (agent-scope exchanges)
    for (int i = threadIdx.x; i < ARGMAX_SPREAD * m; i += blockDim.x) {
        const int row = i / m, tok = i - row * m;
        const unsigned long long k =
            __hip_atomic_exchange(table + row * ARGMAX_MAX_TOK + tok, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (k) atomicMax(best + tok, k);
    }
    __syncthreads();
    for (int t = threadIdx.x; t < m; t += blockDim.x)
        if (best[t]) (void)__hip_atomic_fetch_max(keys + t, best[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// the fold after an argmax product's launch (m logit rows)
static hipError_t argmax_fold(const Launch& l, int m) {
    // a thread per table entry up to 1024 (m <= 16: one exchange round trip per thread)
    const int threads = std::min(1024, (ARGMAX_SPREAD * m + 63) / 64 * 64);
    hipLaunchKernelGGL(argmax_fold_kernel, dim3(1), dim3(threads), 0, l.stream, l.argmax_table, l.keys, m);
    return hipGetLastError();
}

// Words of a (tile, group) code block per lane (16 bytes each).
template <int F>
struct CodeWords {
    static constexpr int N = (F & F_BF16) ? 4 : (F & F_I8) ? 2 : 1;
};

// The scale of row r of `tile`, group g (T tiles; layout.h scale_idx)
template <int F>
__device__ __forceinline__ float scale_of(const void* scales, int tile, int T, int g, int r) {
    if (F & F_S32) return ((const float*)scales)[scale_idx(tile, T, g, r)];
    return bf16_bits_f(((const uint16_t*)scales)[scale_idx(tile, T, g, r)]);
}

// ---------------------------------------------------------------------------------------------------------------
// skinny_kernel
//
// A wave owns T tiles and NG consecutive groups (one "chunk"): it issues all of that chunk's loads at once (its
// scales, one load per tile for 4 groups, then the codes), so that many short waves keep HBM saturated, and computes
// them as they arrive. The workgroup's waves are WT side by side over tiles (x) times WK over consecutive chunks of K
// (y); together they cover a super-chunk of CH = WK * NG groups, whose activations the workgroup stages once in LDS
// (every wave of it reads them with ds_read_b128 instead of fetching them from L2). The grid's y dimension splits the
// super-chunks of K (plain products: split-K partials); WK waves' partial sums are reduced through LDS.


// ---------------------------------------------------------------------------------------------------------------
// The LoRA delta fused into the products' epilogues (the reference applies it as separate kernels after the product,
// kernels/lora.cuh:52-113): delta[t][o] = s_t B[o] . xa_t[off(o) .. off(o) + R), s_t the token's slot scale, xa_t the
// token's A product summed over its split-K partials, off(o) the first column of o's module (routing as
// lora_module: module ends tab[0..2], column offsets tab[4..7]; SwiGLU products: rows 0..7 of each 16-row tile are
// the gate (tab[4]), rows 8..15 the up rows (tab[5])). It runs on the f32 matrix cores, in the layout of each kernel's
// accumulators: D = (s xa) (tokens x R) . B^T (R x outputs), the contraction index laid out so that a lane group
// reads contiguous runs of xa and B. A tile (or 32-row block) that straddles a module end takes one pass per module
// with the other rows' B masked to zero. The MFMAs accumulate straight into the product's accumulators (no registers
// held for a separate delta): rows of unadapted modules are not touched, and the products of tokens of slot scale 0
// or of masked rows add exact zeros.

template <bool SILU>
__device__ __forceinline__ int lora_module_of(const Launch& a, int o) {
    if (SILU) return (o >> 3) & 1;  // gate / up halves of a 16-row tile
    return (o >= a.lora_tab[0]) + (o >= a.lora_tab[1]) + (o >= a.lora_tab[2]);
}
__device__ __forceinline__ int lora_off(const Launch& a, int m) { return a.lora_tab[4 + m]; }

// s_t * sum over splits of xa[.][tok][c .. c + N), N consecutive columns into v
template <int N>
__device__ __forceinline__ void lora_xs_run(const Launch& a, int tok, int c, float s, float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = 0.0f;
    for (int sp = 0; sp < a.lora_split; sp++) {
        const float* p = a.lora_xa + ((size_t)sp * a.lora_ldm + tok) * a.lora_cols + c;
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += p[i];
    }
#pragma unroll
    for (int i = 0; i < N; i++) v[i] *= s;
}

// B[o][c .. c + N) (f16 -> f32), zero when `keep` is false
template <int N>
__device__ __forceinline__ void lora_b_run(const Launch& a, int o, int c, bool keep, float (&v)[N]) {
    const _Float16* p = (const _Float16*)a.lora_b + (size_t)o * a.lora_rank + c;
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = keep ? (float)p[i] : 0.0f;
}

__device__ __forceinline__ float lora_scale_of(const Launch& a, int tok) {
    return a.lora_slot_scale[a.lora_tok_slot[tok]];
}

// The decode kernel's layout (v_mfma_f32_16x16x4_f32): the delta of 16-row tile `tile` for 16 tokens starting at
// tok0 (A rows: tokens tok0 + lane % 16, clamped to m - 1); lane l gets D[token tok0 + 4 (l / 16) + i][row l % 16].
template <bool SILU>
__device__ void lora_delta16(const Launch& a, int tile, int tok0, f32x4& d) {
    constexpr int C = 2;  // steps whose operands are in registers at a time (R / 4 is a multiple)
    const int Q = a.lora_rank / 4;  // contraction steps; lane group q takes k = q Q + i
    const int lane = threadIdx.x & 63, l16 = lane & 15, q = lane >> 4;
    const int o = tile * TILE + l16, mod = lora_module_of<SILU>(a, o);
    const int mlo = lora_module_of<SILU>(a, tile * TILE), mhi = lora_module_of<SILU>(a, tile * TILE + TILE - 1);
    const int tok = min(tok0 + (((l16 & 3) << 2) | (l16 >> 2)), a.m - 1);  // skinny_kernel's token rows
    const float s = lora_scale_of(a, tok);
    for (int m = mlo; m <= mhi; m++) {
        const int c0 = lora_off(a, m);
        if (c0 < 0) continue;  // wave-uniform
        for (int i0 = 0; i0 < Q; i0 += C) {
            float xv[C], bv[C];
            lora_xs_run<C>(a, tok, c0 + q * Q + i0, s, xv);
            lora_b_run<C>(a, o, q * Q + i0, mod == m, bv);
#pragma unroll
            for (int i = 0; i < C; i++) d = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], bv[i], d, 0, 0, 0);
        }
    }
}

// The prefill kernel's layout (v_mfma_f32_32x32x2_f32): the deltas of a wave's TN blocks of 32 output rows (block t:
// rows (tile0 + 2 t) 16 ..) for its BMB blocks of 32 tokens (block bb: tokens tok0 + 32 bb ..), accumulated into
// acc[bb][t]; lane l holds D[token 8 (v / 4) + 4 (l / 32) + v % 4][row l % 32], v = 0..15. Loads are batched for
// latency: the tokens' slot scales for every block at once, each lane's B run once, and xa either from the item's rows
// staged in LDS (xs: one split, 4-32 columns; row r's 16-byte chunk k at slot k ^ (r mod chunks per row), rows from
// xs_row0) or, otherwise, the xa runs of NBB token blocks at a time from global memory.
template <bool SILU, int BMB, int TN>
__device__ void lora_item32(const Launch& a, int tile0, int tok0, f32x16 (&acc)[BMB][TN], const uint8_t* xs = nullptr,
                            int xs_row0 = 0) {
    // one code path for every rank (a switch over ranks multiplies the epilogue's code and spills registers): the
    // H = R / 2 contraction steps run C at a time, lane group h taking k = h H + i
    constexpr int C = 4;                     // steps whose operands are in registers at a time (H is a multiple)
    constexpr int NBB = BMB < 4 ? BMB : 4;   // token blocks whose xa runs are loaded together
    const int H = a.lora_rank / 2;
    const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    int tok[BMB];
    float s[BMB];
#pragma unroll
    for (int bb = 0; bb < BMB; bb++) tok[bb] = min(tok0 + 32 * bb + l32, a.m - 1);
#pragma unroll
    for (int bb = 0; bb < BMB; bb++) s[bb] = (float)a.lora_tok_slot[tok[bb]];  // slot index, exact as a float
#pragma unroll
    for (int bb = 0; bb < BMB; bb++) s[bb] = a.lora_slot_scale[(int)s[bb]];
#pragma unroll
    for (int t = 0; t < TN; t++) {
        const int o0 = (tile0 + 2 * t) * TILE;
        if (o0 >= a.rows) break;  // wave-uniform
        const int o = min(o0 + l32, a.rows - 1), mod = lora_module_of<SILU>(a, o);
        const int mlo = lora_module_of<SILU>(a, o0), mhi = lora_module_of<SILU>(a, min(o0 + 31, a.rows - 1));
        // this lane's B run (row o, columns h H .. h H + H), loaded once for every module and step as f16 pairs (H is 4 to
        // 32): one load instead of a dependent one per module and step
        uint32_t bw[16];
        {
            const _Float16* bp = (const _Float16*)a.lora_b + (size_t)o * a.lora_rank + h * H;
            if (H == 4) {  // rank 8: the run is 8 bytes (a 16-byte load would pass the last row's end)
                const unsigned long long v = *(const unsigned long long*)bp;
                bw[0] = (uint32_t)v, bw[1] = (uint32_t)(v >> 32);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (8 * q < H) {
                        const u32x4 v = ((const u32x4*)bp)[q];
                        bw[4 * q] = v.x, bw[4 * q + 1] = v.y, bw[4 * q + 2] = v.z, bw[4 * q + 3] = v.w;
                    }
            }
        }
        for (int m = mlo; m <= mhi; m++) {
            const int c0 = lora_off(a, m);
            if (c0 < 0) continue;  // wave-uniform
            for (int i0 = 0; i0 < H; i0 += C) {
                float bv[C];
                const bool keep = mod == m && o0 + l32 < a.rows;
#pragma unroll
                for (int i = 0; i < C; i += 2) {
                    uint32_t w = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++)
                        if (q == (i0 + i) >> 1) w = bw[q];
                    const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)w),
                                   hi = __builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
                    bv[i] = keep ? (float)lo : 0.0f;
                    bv[i + 1] = keep ? (float)hi : 0.0f;
                }
                // (loops over accumulators fully unrolled: an indexed register array would live in scratch memory)
#pragma unroll
                for (int b0 = 0; b0 < BMB; b0 += NBB) {
                    float xv[NBB][C];
                    if (xs) {  // staged in LDS: row r's 16-byte chunk k at slot k ^ (r mod chunks per row)
                        const int cpr = a.lora_cols >> 2, k = (c0 + h * H + i0) >> 2;
#pragma unroll
                        for (int j = 0; j < NBB; j++) {
                            const int r = xs_row0 + 32 * (b0 + j) + l32;
                            const f32x4 v = *(const f32x4*)(xs + (r * cpr + (k ^ (r & (cpr - 1)))) * 16);
#pragma unroll
                            for (int i = 0; i < C; i++) xv[j][i] = v[i] * s[b0 + j];
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < NBB; j++)
                            lora_xs_run<C>(a, tok[b0 + j], c0 + h * H + i0, s[b0 + j], xv[j]);
                    }
#pragma unroll
                    for (int j = 0; j < NBB; j++)
#pragma unroll
                        for (int i = 0; i < C; i++)
                            acc[b0 + j][t] = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[j][i], bv[i], acc[b0 + j][t], 0, 0, 0);
                }
            }
        }
    }
}

// Whether a skinny launch stages the activations per wave instead of per workgroup: one token, int4 without zero
// points, 4-group waves. Each wave then loads its own 1 KiB of x (from L2: the x reads grow by the workgroup's wave
// count, against the 8 KiB of weights per wave) and waits for no other wave before it computes. Same-box A/B, per
// launch: the 27B set 8.00 -> 7.90 us, configs[0] 4.81 -> 4.73 us; with zero points (the 4B set) it measured 3% slower,
// int8 and bf16 1-2% slower, so those keep the workgroup's staging.
__host__ __device__ constexpr bool skinny_wave_x(int m, int fmt, int ng) {
    return m == 1 && ng == 4 && !(fmt & (F_I8 | F_BF16 | F_ZP));
}

template <int F, int EPI, int NR, int T, int NG, int TB>
__global__ __launch_bounds__(TB == 1 ? 1024 : 512) __attribute__((amdgpu_waves_per_eu(NG == 1 && TB > 1 ? 4 : 1))) void skinny_kernel(Launch a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int CW = CodeWords<F>::N;
    // the workgroup is WT wave columns (x) by WK wave rows (y): no division in the index set-up, which every wave
    // runs before its first load
    const int lane = threadIdx.x & 63, nthr = blockDim.x * blockDim.y, tid = threadIdx.y * blockDim.x + threadIdx.x;
    const int WT = blockDim.x >> 6, WK = blockDim.y;
    const int wt = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), wk = __builtin_amdgcn_readfirstlane(threadIdx.y);
    const int l16 = lane & 15, kq = lane >> 4;
    const int tiles = a.rows / TILE, G = a.cols / QG, M = a.m;
    const int CH = WK * NG, NC = a.nc;  // groups per super-chunk, super-chunks in K
    // super-chunks [c0, c1) of this split: one each (split-K plain products: split == NC), else all (split 1; the
    // launcher makes no other split), chosen without a branch so that no scalar load waits ahead of the next
    const bool per_chunk = a.split == NC;
    const int c0 = per_chunk ? (int)blockIdx.y : 0, c1 = per_chunk ? c0 + 1 : NC;
    // activation rows are gathered (out_rows) only by the argmax epilogue
    const int32_t* const xrows = EPI == EPI_ARGMAX ? a.xrows : nullptr;
    // the loop's operands loaded here with the fields above, in one batch of scalar loads and one wait, rather than
    // a second round trip in the loop's preheader
    {
        const void* const ops[4] = {a.codes, a.scales, a.x, (F & F_ZP) ? (const void*)a.zeros : a.y};
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" ::"s"(ops[i]));
        asm volatile("" ::"s"(a.ldx));
    }
    const int tile0 = (blockIdx.x * WT + wt) * T;
    const int xpitch = CH * QG + 8;  // bf16 per staged x row (+16 bytes: rows start 4 banks apart)
    __bf16* xs_lds = (__bf16*)smem;
    // one token (int4 without zero points, 4-group waves): each wave stages its own groups' activations (1 KiB, one
    // direct-to-LDS load per lane) in its own LDS slot, and no workgroup barrier separates its loads from its compute
    constexpr bool PRIV = NR == 1 && TB == 1 && skinny_wave_x(1, F, NG);
    __bf16* xw = xs_lds + (size_t)(wk * WT + wt) * NG * QG;
    const size_t xbytes = PRIV ? std::max((size_t)M * xpitch * 2, (size_t)WT * WK * NG * QG * 2) : (size_t)M * xpitch * 2;
    float* red = (float*)(smem + ((xbytes + 15) & ~(size_t)15));

    int tt[T];
#pragma unroll
    for (int t = 0; t < T; t++) tt[t] = min(tile0 + t, tiles - 1);
    // token block b (16 tokens): MFMA row l16 holds token 16 b + 4 (l16 % 4) + l16 / 4, so that a lane's accumulator
    // row r holds token 16 b + 4 r + lane / 16 and NR = ceil(tokens / 4) rows per lane suffice in a partial block (one
    // token: row order); rows past M read row M - 1 (their results are never stored)
    int xtok[TB];
#pragma unroll
    for (int b = 0; b < TB; b++) xtok[b] = min(16 * b + (NR > 1 ? (((l16 & 3) << 2) | (l16 >> 2)) : l16), M - 1);

    const uint32_t magic_s = a.bf16_magic, mask = a.nib_mask;
    uint32_t magic;  // in a VGPR (copied once; only VALU reads it) so that each pair is one v_and_or_b32
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(magic_s));
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

    float acc[TB][T][NR];
#pragma unroll
    for (int b = 0; b < TB; b++)
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int r = 0; r < NR; r++) acc[b][t][r] = 0.0f;

    // the activation pieces this thread stages (the same in every super-chunk): the first XPT of its pieces are loaded
    // ahead of the weights; their rows (the argmax's gathered rows) are looked up once, here, not in every super-chunk
    const int rowc = CH * 16;  // 16-byte pieces per staged row
    const int npieces = M * rowc;
    constexpr int XPT = PRIV ? 0 : TB;
    int xo[XPT > 0 ? XPT : 1];            // LDS offset (-1: none)
    const __bf16* xsrc[XPT > 0 ? XPT : 1];  // source, before the super-chunk's column offset
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int p = tid + i * nthr;
        const int tok = min(p / rowc, M - 1), pc = p - (p / rowc) * rowc;
        xo[i] = p < npieces ? tok * xpitch + 8 * pc : -1;
        xsrc[i] = (const __bf16*)a.x + (size_t)(xrows ? xrows[tok] : tok) * a.ldx + 8 * (p < npieces ? pc : 0);
    }
    const __bf16* xwsrc = (const __bf16*)a.x + (size_t)(PRIV && xrows ? xrows[0] : 0) * a.ldx + 8 * lane;

    for (int c = c0; c < c1; c++) {
        const int gs = c * CH;              // first group of the super-chunk
        const int gw = gs + wk * NG;        // this wave's first group
        // 1. the super-chunk's activations (M rows of CH * 128 columns): the first XPT pieces per thread are loaded
        //    before the weights (loads complete in order, so staging them afterwards would wait for every weight),
        //    the rest, if any, afterwards
        u32x4 xv[XPT > 0 ? XPT : 1];
        if constexpr (PRIV) {  // the wave's own 4 groups (64 pieces of 16 bytes), global -> LDS directly
            __builtin_amdgcn_global_load_lds((const void*)(xwsrc + (size_t)gw * QG),
                                             (__attribute__((address_space(3))) void*)xw, 16, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < XPT; i++) xv[i] = *(const u32x4*)(xsrc[i] + (size_t)gs * QG);
        // 2. this wave's weights: scales (4 groups per load), zero points, then codes group by group, all streamed
        //    (non-temporal: read once; measured 1-2% faster for the scales, 10% for the codes, than cached loads)
        uint32_t sraw[T][NG == 4 ? ((F & F_S32) ? 4 : 2) : 1];
        uint32_t zraw[T];
        u32x4 code[NG][T][CW];
#pragma unroll
        for (int t = 0; t < T && !(F & F_BF16); t++) {
            const size_t si = scale_idx(tt[t], tiles, gw, l16);
            if constexpr (NG == 4) {
                if constexpr ((F & F_S32) != 0) {
                    const u32x4 v = __builtin_nontemporal_load((const u32x4*)((const float*)a.scales + si));
                    sraw[t][0] = v.x, sraw[t][1] = v.y, sraw[t][2] = v.z, sraw[t][3] = v.w;
                } else {
                    const unsigned long long v =
                        __builtin_nontemporal_load((const unsigned long long*)((const uint16_t*)a.scales + si));
                    sraw[t][0] = (uint32_t)v, sraw[t][1] = (uint32_t)(v >> 32);
                }
            } else {
                sraw[t][0] = (F & F_S32) ? __builtin_nontemporal_load((const uint32_t*)a.scales + si)
                                         : __builtin_nontemporal_load((const uint16_t*)a.scales + si);
            }
            if (F & F_ZP) zraw[t] = __builtin_nontemporal_load(a.zeros + zero_idx(tt[t], tiles, gw, l16));
        }
#pragma unroll
        for (int gi = 0; gi < NG; gi++)
#pragma unroll
            for (int t = 0; t < T; t++) {
                const u32x4* cp = (const u32x4*)a.codes + ((size_t)tt[t] * G + gw + gi) * 64 * CW;
#pragma unroll
                for (int h = 0; h < CW; h++) code[gi][t][h] = __builtin_nontemporal_load(cp + h * 64 + lane);
            }
        // 3. stage the activations
        if constexpr (PRIV) {
            // the wave's own activation load done: the weight loads issued after it (a scale load and NG code loads
            // per tile) may stay in flight. Its previous super-chunk's LDS reads were all consumed by its MFMAs.
            constexpr int WL = T * (1 + NG * CW);
            __builtin_amdgcn_s_waitcnt((WL & 15) | ((WL >> 4) << 14) | (7 << 4) | (15 << 8));
        } else {
            if (c > c0) __syncthreads();  // the previous super-chunk's readers are done
#pragma unroll
            for (int i = 0; i < XPT; i++)
                if (xo[i] >= 0) *(u32x4*)(xs_lds + xo[i]) = xv[i];
            for (int p = tid + XPT * nthr; p < npieces; p += nthr) {
                const int tok = p / rowc, pc = p - tok * rowc;
                const __bf16* src =
                    (const __bf16*)a.x + (size_t)(xrows ? xrows[tok] : tok) * a.ldx + (size_t)gs * QG + 8 * pc;
                *(u32x4*)(xs_lds + (size_t)tok * xpitch + 8 * pc) = *(const u32x4*)src;
            }
            __syncthreads();
        }
        // 3. compute the wave's groups: each tile's B fragments once, against every token block
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            u32x4 xa[TB][4];
            f32x4 xsum[TB];
#pragma unroll
            for (int b = 0; b < TB; b++) {
                const __bf16* xrow = PRIV ? xw + gi * QG + 8 * kq
                                          : xs_lds + (size_t)xtok[b] * xpitch + (wk * NG + gi) * QG + 8 * kq;
#pragma unroll
                for (int j = 0; j < 4; j++) xa[b][j] = *(const u32x4*)(xrow + 32 * j);
                xsum[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4 && !(F & F_BF16); j++) xsum[b] = mfma(xa[b][j], ones, xsum[b]);
            }
#pragma unroll
            for (int t = 0; t < T; t++) {
                // B fragment j of tile t (one token block dequantizes it next to its MFMA, fewer live registers;
                // several keep all four for their blocks)
                auto frag = [&](int j) -> bf16x8 {
                    if (F & F_BF16) return __builtin_bit_cast(bf16x8, code[gi][t][j]);
                    if (F & F_I8)
                        return i8_biased(code[gi][t][j >> 1][2 * (j & 1)], code[gi][t][j >> 1][2 * (j & 1) + 1]);
                    return i4_biased(code[gi][t][0][j], mask, magic);
                };
                f32x4 d[TB];
                if constexpr (TB == 1) {
                    d[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < 4; j++) d[0] = mfma(xa[0][j], frag(j), d[0]);
                } else {
                    bf16x8 bw[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) bw[j] = frag(j);
#pragma unroll
                    for (int b = 0; b < TB; b++) {
                        d[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int j = 0; j < 4; j++) d[b] = mfma(xa[b][j], bw[j], d[b]);
                    }
                }
                if (F & F_BF16) {  // the weights themselves: no scale, no zero point
#pragma unroll
                    for (int b = 0; b < TB; b++)
#pragma unroll
                        for (int r = 0; r < NR; r++) acc[b][t][r] += d[b][r];
                    continue;
                }
                const int g = gw + gi;
                // the group's scale from the raw scale words: f32 one per word; bf16 two per word (NG == 4) or one
                float sc;
                if (F & F_S32) {
                    sc = __uint_as_float(sraw[t][NG == 4 ? gi : 0]);
                } else if (NG == 4) {
                    const uint32_t w = sraw[t][gi >> 1];
                    sc = __uint_as_float((gi & 1) ? (w & 0xffff0000u) : (w << 16));
                } else {
                    sc = __uint_as_float(sraw[t][0] << 16);
                }
                const float cz = (F & F_ZP) ? (float)(128 + (int)((zraw[t] >> (4 * (g & 3))) & 15u))
                                            : ((F & F_I8) ? 128.0f : 136.0f);  // 128 + zero point
#pragma unroll
                for (int b = 0; b < TB; b++)
#pragma unroll
                    for (int r = 0; r < NR; r++)  // two explicit fmas (the one-token kernel's too: equal results)
                        acc[b][t][r] = __builtin_fmaf(sc, __builtin_fmaf(-cz, xsum[b][r], d[b][r]), acc[b][t][r]);
            }
        }
    }

    // reduce the K chunks of a column's waves into its first (the others stay for the workgroup's barriers)
    bool lead = true;
    if (WK > 1) {
        if (wk > 0) {
#pragma unroll
            for (int b = 0; b < TB; b++)
#pragma unroll
                for (int t = 0; t < T; t++)
#pragma unroll
                    for (int r = 0; r < NR; r++)
                        red[(((((wk - 1) * WT + wt) * TB + b) * T + t) * NR + r) * 64 + lane] = acc[b][t][r];
        }
        __syncthreads();
        lead = wk == 0;
        if (lead)
            for (int w = 1; w < WK; w++)
#pragma unroll
                for (int b = 0; b < TB; b++)
#pragma unroll
                    for (int t = 0; t < T; t++)
#pragma unroll
                        for (int r = 0; r < NR; r++)
                            acc[b][t][r] += red[(((((w - 1) * WT + wt) * TB + b) * T + t) * NR + r) * 64 + lane];
    }

    const int sp = blockIdx.y;
    // the LoRA delta: on split 0 of a plain product, before the activation of a SwiGLU one
    if ((EPI == EPI_SILU || (EPI == EPI_PLAIN && sp == 0)) && a.lora_rank && lead) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int tile = tile0 + t;
            if (tile >= tiles) break;
#pragma unroll
            for (int b = 0; b < TB; b++) {
                f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int r = 0; r < NR; r++) d[r] = acc[b][t][r];
                lora_delta16<EPI == EPI_SILU>(a, tile, 16 * b, d);
#pragma unroll
                for (int r = 0; r < NR; r++) acc[b][t][r] = d[r];
            }
        }
    }
    unsigned long long key[TB][NR];
#pragma unroll
    for (int b = 0; b < TB; b++)
#pragma unroll
        for (int r = 0; r < NR; r++) key[b][r] = 0;
    if (EPI == EPI_PLAIN && a.stage_out) {
        if (WK > 1) __syncthreads();  // every lead wave has read the K-wave partials that the staging overwrites
        // plain partials through LDS: the wave's block (m tokens x T 16-row tiles) is written to its own LDS slot in
        // the MFMA layout and read back along the rows, so that y is written with 16-byte stores of whole row runs
        // (one store instruction for up to 8 tokens, against one per tile and token row of 16 lanes: small scattered
        // stores cost far more per byte than the reads they follow)
        constexpr int RW = T * TILE;  // rows of the wave's block
        float* stg = red + (size_t)wt * M * RW;  // the lead wave of tile column wt
        if (lead) {
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int b = 0; b < TB; b++)
#pragma unroll
                    for (int r = 0; r < NR; r++) {
                        const int tok = 16 * b + (NR > 1 ? 4 * r + kq : 4 * kq + r);
                        if (tok < M) stg[tok * RW + t * TILE + l16] = acc[b][t][r];
                    }
            const int row0 = tile0 * TILE;
            for (int i = lane; i < M * (RW / 4); i += 64) {
                const int tok = i / (RW / 4), c = 4 * (i - tok * (RW / 4));
                if (row0 + c < a.rows)  // streamed past the caches (measured 7% faster on the 4B set at M = 2-8)
                    __builtin_nontemporal_store(*(const f32x4*)(stg + tok * RW + c),
                                                (f32x4*)((float*)a.y + ((size_t)sp * M + tok) * a.ldy + row0 + c));
            }
        }
    } else if (lead) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int tile = tile0 + t;
            if (tile >= tiles) break;
            const int out = tile * TILE + l16;
#pragma unroll
            for (int b = 0; b < TB; b++)
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    const int tok = 16 * b + (NR > 1 ? 4 * r + kq : 4 * kq + r);
                    const float v = acc[b][t][r];
                    if (EPI == EPI_SILU) {
                        const float up = __shfl_xor(v, 8);
                        if (l16 < 8 && tok < M)
                            ((__bf16*)a.y)[(size_t)tok * a.ldy + tile * 8 + l16] = (__bf16)(silu(v) * up);
                    } else {
                        if (tok < M) ((float*)a.y)[((size_t)sp * M + tok) * a.ldy + out] = v;
                        if (EPI == EPI_ARGMAX && tok < M && out < a.valid)
                            key[b][r] = max_u64(key[b][r], argmax_key(v, out));
                    }
                }
        }
    }
    if (EPI == EPI_ARGMAX) {
#pragma unroll
        for (int b = 0; b < TB; b++)
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const unsigned long long k = group16_max(key[b][r]);
                const int tok = 16 * b + (NR > 1 ? 4 * r + kq : 4 * kq + r);
                if (lead && l16 == 0 && tok < M && k) argmax_spread_max(a, tok, k);
            }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// skinny_m1_kernel: the one-token plain product of int4 with bf16 scales, symmetric or with zero points (ZP), with
// no adapter, the decode hot path, as skinny_kernel runs it (the same partition, loads, arithmetic and partials, so the
// same results bit for bit) with a compact argument block and no paths for other cases. skinny_kernel reads a
// 300-byte Launch and carries every other case's set-up ahead of its first global load. Same-box graph replays, per
// launch: the 27B set 8.15 -> 7.40 us (symmetric; (5120, 17408) and (17408, 5120) 10.1-10.3 -> 9.7 us, (5120, 6144)
// 5.55 -> 5.1 us), configs[0] 4.93 -> 4.49 us.
struct M1Args {
    const u32x4* codes;
    const uint16_t* scales;
    const uint16_t* zeros;  // ZP only
    const __bf16* x;
    float* y;  // [G / NG][tiles * 16]: the partial of each NG-group chunk of K
    int tiles, G;
    uint32_t mask, magic;  // 0x000F000F and the bf16 pair (128, 128): see i4_biased
};

// workgroups of 4 waves side by side over tiles (2 tiles each), the grid over tile columns x NG-group chunks of K
// (NG = 4, or 1 when 4-group waves would not fill the chip; skinny_partition).
// At least two waves per SIMD (amdgpu_waves_per_eu(2)) caps the kernel at 256 registers, which lets the compiler keep
// the MFMA accumulators in ordinary VGPRs: without it the compiler gave them 48 accumulation registers beside 62 VGPRs,
// 4 waves per SIMD; with it 68 VGPRs, 7 waves per SIMD (74 and 6 with zero points), so that the whole grid of a 27B
// product is resident at once. Same box, three A/B pairs: the 27B set 7.43 -> 7.32 us per launch, configs[0] 4.49 ->
// 4.35 us. (Eight waves per SIMD, 64 VGPRs, spills 16-56 bytes per lane.)
template <bool ZP, int NG>
static __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void skinny_m1_kernel(M1Args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63, wt = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, kq = lane >> 4;
    const int T = a.tiles, G = a.G;
    const int tile0 = (blockIdx.x * 4 + wt) * 2, gw = NG * blockIdx.y;
    if (tile0 >= T) return;
    const int t1 = min(tile0 + 1, T - 1);  // an odd last tile: its wave reads the same tile twice, stores once
    __bf16* xw = (__bf16*)smem + wt * 4 * QG;
    uint32_t magic;  // in a VGPR, so that each pair is one v_and_or_b32
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(a.magic));
    const uint32_t mask = a.mask;
    // the wave's groups of activations, global -> LDS directly, first, into its own slot (no workgroup barrier);
    // one group (NG = 1): each quarter of the wave loads the same 256 bytes, read from the first copy
    const int xl = NG == 4 ? lane : l16;
    __builtin_amdgcn_global_load_lds((const void*)(a.x + (size_t)gw * QG + 8 * xl),
                                     (__attribute__((address_space(3))) void*)xw, 16, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    // scales (4 groups per 8-byte load, or the one group's), zero points, then the codes group by group, streamed
    // past the caches
    constexpr int SW = NG == 4 ? 2 : 1;
    uint32_t sraw[2][SW], zraw[2];
    const int tl[2] = {tile0, t1};
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const uint16_t* sp = a.scales + scale_idx(tl[t], T, gw, l16);
        if constexpr (NG == 4) {
            const unsigned long long v = __builtin_nontemporal_load((const unsigned long long*)sp);
            sraw[t][0] = (uint32_t)v, sraw[t][1] = (uint32_t)(v >> 32);
        } else {
            sraw[t][0] = __builtin_nontemporal_load(sp);
        }
        if (ZP) zraw[t] = __builtin_nontemporal_load(a.zeros + zero_idx(tl[t], T, gw, l16));
    }
    u32x4 code[NG][2];
#pragma unroll
    for (int gi = 0; gi < NG; gi++)
#pragma unroll
        for (int t = 0; t < 2; t++) code[gi][t] = __builtin_nontemporal_load(a.codes + ((size_t)tl[t] * G + gw + gi) * 64 + lane);
    // the activations landed (the weight loads issued after them may stay in flight)
    constexpr int WL = 2 + (ZP ? 2 : 0) + 2 * NG;
    __builtin_amdgcn_s_waitcnt((WL & 15) | ((WL >> 4) << 14) | (7 << 4) | (15 << 8));
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    float acc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        u32x4 xa[4];
        const __bf16* xrow = xw + gi * QG + 8 * kq;
#pragma unroll
        for (int j = 0; j < 4; j++) xa[j] = *(const u32x4*)(xrow + 32 * j);
        f32x4 xsum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) xsum = mfma(xa[j], ones, xsum);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) d = mfma(xa[j], i4_biased(code[gi][t][j], mask, magic), d);
            float sc;
            if constexpr (NG == 4) {
                const uint32_t w = sraw[t][gi >> 1];
                sc = __uint_as_float((gi & 1) ? (w & 0xffff0000u) : (w << 16));
            } else {
                sc = __uint_as_float(sraw[t][0] << 16);
            }
            const float cz = ZP ? (float)(128 + (int)((zraw[t] >> (4 * ((gw + gi) & 3))) & 15u)) : 136.0f;
            acc[t] = __builtin_fmaf(sc, __builtin_fmaf(-cz, xsum[0], d[0]), acc[t]);  // as skinny_kernel
        }
    }
    if (kq == 0) {
        float* yo = a.y + (size_t)blockIdx.y * T * TILE + tile0 * TILE + l16;
        yo[0] = acc[0];
        if (tile0 + 1 < T) yo[TILE] = acc[1];
    }
}

// skinny_m1w_kernel: one-token products that need whole sums (the SwiGLU epilogue, plain products asked for whole
// rows, the argmax epilogue) of int4 with bf16 scales, symmetric or with zero points, no adapter, on the lean
// terms of skinny_m1_kernel: a workgroup takes one pair of tiles over all of K, one wave per 4-group chunk up to 8
// chunks, beyond that WK = 8 waves each taking every WK-th chunk (mw_waves), each chunk as short-lived as a plain
// product's wave; the waves' sums meet in LDS and the first wave adds them in wave order. (skinny_kernel runs these with 2 x 2-wave workgroups whose waves each walk G / 8 chunks, one after another.)
struct M1wArgs {
    const u32x4* codes;
    const uint16_t* scales;
    const uint16_t* zeros;  // ZP only
    const __bf16* x;        // the token's row: x row xrows[0] (xrows null: row 0)
    void* y;                // SwiGLU: bf16 [rows / 2]; argmax: f32 logits [rows]
    unsigned long long* keys;  // argmax: the token's running key, keys[0]
    int tiles, G, valid;
    uint32_t mask, magic;
    const int32_t* xrows;  // argmax: the token's activations are x row xrows[0] (null: row 0), rows ldx apart
    int ldx;
};

template <int EPI, bool ZP>
static __global__ __launch_bounds__(1024) void skinny_m1w_kernel(M1wArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63, wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int WK = blockDim.x >> 6;
    const int l16 = lane & 15, kq = lane >> 4;
    const int T = a.tiles, G = a.G;
    const int tile0 = blockIdx.x * 2;
    const int t1 = min(tile0 + 1, T - 1);
    __bf16* xw = (__bf16*)smem + wk * 4 * QG;
    float* red = (float*)(smem + (size_t)WK * 4 * QG * 2);  // [WK][32]: each wave's sums of the 32 rows
    uint32_t magic;
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(a.magic));
    const uint32_t mask = a.mask;
    const int tl[2] = {tile0, t1};
    // the token's row index through the scalar cache (a uniform load: a vector load here made every wave wait for it
    // before issuing anything else)
    const int32_t xrow = a.xrows ? *(const __attribute__((address_space(4))) int32_t*)a.xrows : 0;
    const __bf16* const x0 = a.x + (size_t)xrow * a.ldx;
    float acc[2] = {0.0f, 0.0f};
    // argmax: a lower bound of the token's final key (keys only grow during the launch), read at the coherence point
    // while the chunks load; the workgroup's maximum is sent only when above it
    unsigned long long seen = 0;
    if (EPI == EPI_ARGMAX && wk == 0) seen = __hip_atomic_load(a.keys, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the wave's chunks of 4 groups: wk, wk + WK, ... (one when K has at most 8 chunks)
    for (int gw = 4 * wk; gw < G; gw += 4 * WK) {
        __builtin_amdgcn_global_load_lds((const void*)(x0 + (size_t)gw * QG + 8 * lane),
                                         (__attribute__((address_space(3))) void*)xw, 16, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t sraw[2][2], zraw[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const unsigned long long v =
                __builtin_nontemporal_load((const unsigned long long*)(a.scales + scale_idx(tl[t], T, gw, l16)));
            sraw[t][0] = (uint32_t)v, sraw[t][1] = (uint32_t)(v >> 32);
            if (ZP) zraw[t] = __builtin_nontemporal_load(a.zeros + zero_idx(tl[t], T, gw, l16));
        }
        u32x4 code[4][2];
#pragma unroll
        for (int gi = 0; gi < 4; gi++)
#pragma unroll
            for (int t = 0; t < 2; t++)
                code[gi][t] = __builtin_nontemporal_load(a.codes + ((size_t)tl[t] * G + gw + gi) * 64 + lane);
        constexpr int WL = 2 + (ZP ? 2 : 0) + 8;
        __builtin_amdgcn_s_waitcnt((WL & 15) | ((WL >> 4) << 14) | (7 << 4) | (15 << 8));
        const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            u32x4 xa[4];
            const __bf16* xrow = xw + gi * QG + 8 * kq;
#pragma unroll
            for (int j = 0; j < 4; j++) xa[j] = *(const u32x4*)(xrow + 32 * j);
            f32x4 xsum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) xsum = mfma(xa[j], ones, xsum);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) d = mfma(xa[j], i4_biased(code[gi][t][j], mask, magic), d);
                const uint32_t w = sraw[t][gi >> 1];
                const float sc = __uint_as_float((gi & 1) ? (w & 0xffff0000u) : (w << 16));
                const float cz = ZP ? (float)(128 + (int)((zraw[t] >> (4 * gi)) & 15u)) : 136.0f;
                acc[t] = __builtin_fmaf(sc, __builtin_fmaf(-cz, xsum[0], d[0]), acc[t]);
            }
        }
    }
    if (kq == 0) {
        red[wk * 32 + l16] = acc[0];
        red[wk * 32 + TILE + l16] = acc[1];
    }
    __syncthreads();
    if (wk == 0) {
        // row tile0 * 16 + lane of the pair (lanes 0..31): the chunks in K order
        float v = 0.0f;
        for (int c = 0; c < WK; c++) v += red[c * 32 + (lane & 31)];
        const int tile = tile0 + (lane >> 4 & 1), out = tile * TILE + l16;
        const bool ok = lane < 32 && tile < T;
        if (EPI == EPI_SILU) {
            const float up = __shfl_xor(v, 8);  // rows 8..15 of a tile are the up rows of rows 0..7
            if (ok && l16 < 8) ((__bf16*)a.y)[tile * 8 + l16] = (__bf16)(silu(v) * up);
        } else if (EPI == EPI_PLAIN) {
            if (ok) ((float*)a.y)[out] = v;
        } else {
            unsigned long long k = 0;
            if (ok) {
                // streamed past the caches (1 MB of logits on the 27B head; the headline step 0.2427 -> 0.2424 ms)
                __builtin_nontemporal_store(v, (float*)a.y + out);
                if (out < a.valid) k = argmax_key(v, out);
            }
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) k = max_u64(k, __shfl_xor(k, o));
            if (lane == 0 && k > seen)
                (void)__hip_atomic_fetch_max(a.keys, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// skinny_mt_kernel: the plain product of 2-8 tokens on the same terms as skinny_m1_kernel (int4 with bf16 scales,
// symmetric or with zero points, no adapter): the partition of skinny_kernel's plain products (WT wave columns of 2
// tiles per workgroup, one chunk of NG groups of K per wave, split = the chunks) and its arithmetic per token (one
// MFMA row block of 16 rows), bit for bit. Token t sits in MFMA row 4 (t % 4) + t / 4, so that a lane's accumulator
// row r holds token 4 r + lane / 16: 2-4 tokens need one accumulator row per lane and 5-8 two (against 2-4 with
// tokens in row order), which holds the kernel at 74-78 VGPRs, 6 waves per SIMD (5 before). Same-box A/B, three
// pairs: the 27B step at M = 5 0.2822 -> 0.2788 ms, the 4B set with zero points at M = 4 / 5 4.59 / 4.67 -> 4.23 /
// 4.41 us per launch, at M = 2 3.91 -> 3.89 us. Each wave stages its own tokens' activations (M rows of NG groups,
// rows 16 bytes apart, global -> LDS directly), so no workgroup barrier separates its loads from its compute, and
// writes its partials through its LDS slot as 16-byte row runs.
struct MtArgs {
    const u32x4* codes;
    const uint16_t* scales;
    const uint16_t* zeros;  // ZP only
    const __bf16* x;
    int ldx;
    float* y;  // [G / NG][m][tiles * 16]
    int tiles, G, m;
    uint32_t mask, magic;
};

template <int NG>
__host__ __device__ constexpr int mt_xpitch() { return NG * QG + 8; }  // bf16 per staged row (16 bytes of padding)

template <bool ZP, int NG, int NR>
static __global__ __launch_bounds__(512) void skinny_mt_kernel(MtArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int XP = mt_xpitch<NG>();
    const int lane = threadIdx.x & 63, wt = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int WT = blockDim.x >> 6;
    const int l16 = lane & 15, kq = lane >> 4;
    const int T = a.tiles, G = a.G, M = a.m;
    const int tile0 = (blockIdx.x * WT + wt) * 2, gw = NG * blockIdx.y;
    if (tile0 >= T) return;
    const int t1 = min(tile0 + 1, T - 1);
    __bf16* xw = (__bf16*)smem + (size_t)wt * M * XP;  // the wave's slot: its M rows (and then its partials)
    uint32_t magic;
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(a.magic));
    const uint32_t mask = a.mask;
    // the activations first: row r into slot row r (NG = 4: 64 lanes x 16 bytes; NG = 1: 16 lanes)
    for (int r = 0; r < M; r++) {
        if (NG == 4 || lane < 16)
            __builtin_amdgcn_global_load_lds((const void*)(a.x + (size_t)r * a.ldx + (size_t)gw * QG + 8 * lane),
                                             (__attribute__((address_space(3))) void*)(xw + r * XP), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr int SW = NG == 4 ? 2 : 1;
    uint32_t sraw[2][SW], zraw[2];
    const int tl[2] = {tile0, t1};
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const uint16_t* sp = a.scales + scale_idx(tl[t], T, gw, l16);
        if constexpr (NG == 4) {
            const unsigned long long v = __builtin_nontemporal_load((const unsigned long long*)sp);
            sraw[t][0] = (uint32_t)v, sraw[t][1] = (uint32_t)(v >> 32);
        } else {
            sraw[t][0] = __builtin_nontemporal_load(sp);
        }
        if (ZP) zraw[t] = __builtin_nontemporal_load(a.zeros + zero_idx(tl[t], T, gw, l16));
    }
    u32x4 code[NG][2];
#pragma unroll
    for (int gi = 0; gi < NG; gi++)
#pragma unroll
        for (int t = 0; t < 2; t++) code[gi][t] = __builtin_nontemporal_load(a.codes + ((size_t)tl[t] * G + gw + gi) * 64 + lane);
    // the activations landed (the weight loads issued after them may stay in flight)
    constexpr int WL = 2 + (ZP ? 2 : 0) + 2 * NG;
    __builtin_amdgcn_s_waitcnt((WL & 15) | ((WL >> 4) << 14) | (7 << 4) | (15 << 8));
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    float acc[2][NR];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < NR; r++) acc[t][r] = 0.0f;
    // MFMA row l16 holds token 4 (l16 % 4) + l16 / 4; rows past M read row M - 1 (never stored)
    const __bf16* xrow0 = xw + min(((l16 & 3) << 2) | (l16 >> 2), M - 1) * XP + 8 * kq;
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        u32x4 xa[4];
#pragma unroll
        for (int j = 0; j < 4; j++) xa[j] = *(const u32x4*)(xrow0 + gi * QG + 32 * j);
        f32x4 xsum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) xsum = mfma(xa[j], ones, xsum);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            bf16x8 bw[4];
#pragma unroll
            for (int j = 0; j < 4; j++) bw[j] = i4_biased(code[gi][t][j], mask, magic);
            f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) d = mfma(xa[j], bw[j], d);
            float sc;
            if constexpr (NG == 4) {
                const uint32_t w = sraw[t][gi >> 1];
                sc = __uint_as_float((gi & 1) ? (w & 0xffff0000u) : (w << 16));
            } else {
                sc = __uint_as_float(sraw[t][0] << 16);
            }
            const float cz = ZP ? (float)(128 + (int)((zraw[t] >> (4 * ((gw + gi) & 3))) & 15u)) : 136.0f;
#pragma unroll
            for (int r = 0; r < NR; r++) acc[t][r] = __builtin_fmaf(sc, __builtin_fmaf(-cz, xsum[r], d[r]), acc[t][r]);
        }
    }
    // the partials through the wave's own slot (its activation reads are done: LDS reads complete in order, and the
    // compiler waits for each before its MFMA): M tokens x 32 rows, then 16-byte stores of 128-byte row runs
    float* stg = (float*)xw;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int tok = 4 * r + kq;
            if (tok < M) stg[tok * 32 + t * TILE + l16] = acc[t][r];
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes before its reads
    const int rows = a.tiles * TILE, nrow = min(32, rows - tile0 * TILE);
    float* yb = a.y + (size_t)blockIdx.y * M * rows + tile0 * TILE;
    for (int i = lane; i < M * 8; i += 64) {
        const int tok = i >> 3, c = 4 * (i & 7);
        if (c < nrow)
            __builtin_nontemporal_store(*(const f32x4*)(stg + tok * 32 + c), (f32x4*)(yb + (size_t)tok * rows + c));
    }
}

// ---------------------------------------------------------------------------------------------------------------
// skinny_mw_kernel: whole rows (split 1) of a plain product of 2-8 tokens, int4 with bf16 scales, symmetric or with
// zero points, no adapter: skinny_m1w_kernel's partition (a workgroup per tile pair over all of K, each wave taking
// every WK-th chunk of 4 groups) with skinny_mt_kernel's arithmetic and token rows (each wave stages its tokens' rows
// of its chunk, 16 bytes apart; token 4 r + lane / 16 in row r of a lane's accumulators). The waves' sums meet in LDS
// and the first wave adds them in wave order (the 27B step at M = 5 with whole rows 0.3268 -> 0.3243 ms with the
// token rows above).
template <bool ZP, int NR>
static __global__ __launch_bounds__(1024) void skinny_mw_kernel(MtArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int XP = mt_xpitch<4>();
    const int lane = threadIdx.x & 63, wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int WK = blockDim.x >> 6;
    const int l16 = lane & 15, kq = lane >> 4;
    const int T = a.tiles, G = a.G, M = a.m;
    const int tile0 = blockIdx.x * 2, t1 = min(tile0 + 1, T - 1);
    __bf16* xw = (__bf16*)smem + (size_t)wk * M * XP;                // the wave's M staged rows
    float* red = (float*)(smem + (size_t)WK * M * XP * 2);          // [WK][M][32]: each wave's sums
    uint32_t magic;
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "s"(a.magic));
    const uint32_t mask = a.mask;
    const int tl[2] = {tile0, t1};
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    float acc[2][NR];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < NR; r++) acc[t][r] = 0.0f;
    // MFMA row l16 holds token 4 (l16 % 4) + l16 / 4; rows past M read row M - 1 (never stored)
    const __bf16* xrow0 = xw + min(((l16 & 3) << 2) | (l16 >> 2), M - 1) * XP + 8 * kq;
    for (int gw = 4 * wk; gw < G; gw += 4 * WK) {
        for (int r = 0; r < M; r++)
            __builtin_amdgcn_global_load_lds((const void*)(a.x + (size_t)r * a.ldx + (size_t)gw * QG + 8 * lane),
                                             (__attribute__((address_space(3))) void*)(xw + r * XP), 16, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t sraw[2][2], zraw[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const unsigned long long v =
                __builtin_nontemporal_load((const unsigned long long*)(a.scales + scale_idx(tl[t], T, gw, l16)));
            sraw[t][0] = (uint32_t)v, sraw[t][1] = (uint32_t)(v >> 32);
            if (ZP) zraw[t] = __builtin_nontemporal_load(a.zeros + zero_idx(tl[t], T, gw, l16));
        }
        u32x4 code[4][2];
#pragma unroll
        for (int gi = 0; gi < 4; gi++)
#pragma unroll
            for (int t = 0; t < 2; t++)
                code[gi][t] = __builtin_nontemporal_load(a.codes + ((size_t)tl[t] * G + gw + gi) * 64 + lane);
        // the activations landed (the weight loads issued after them may stay in flight)
        constexpr int WL = 2 + (ZP ? 2 : 0) + 8;
        __builtin_amdgcn_s_waitcnt((WL & 15) | ((WL >> 4) << 14) | (7 << 4) | (15 << 8));
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            u32x4 xa[4];
#pragma unroll
            for (int j = 0; j < 4; j++) xa[j] = *(const u32x4*)(xrow0 + gi * QG + 32 * j);
            f32x4 xsum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) xsum = mfma(xa[j], ones, xsum);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) d = mfma(xa[j], i4_biased(code[gi][t][j], mask, magic), d);
                const uint32_t w = sraw[t][gi >> 1];
                const float sc = __uint_as_float((gi & 1) ? (w & 0xffff0000u) : (w << 16));
                const float cz = ZP ? (float)(128 + (int)((zraw[t] >> (4 * gi)) & 15u)) : 136.0f;
#pragma unroll
                for (int r = 0; r < NR; r++)
                    acc[t][r] = __builtin_fmaf(sc, __builtin_fmaf(-cz, xsum[r], d[r]), acc[t][r]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int tok = 4 * r + kq;
            if (tok < M) red[(wk * M + tok) * 32 + t * TILE + l16] = acc[t][r];
        }
    __syncthreads();
    if (wk == 0) {
        const int rows = T * TILE;
        for (int i = lane; i < M * 32; i += 64) {
            const int tok = i >> 5, row = i & 31, tile = tile0 + (row >> 4);
            float v = 0.0f;
            for (int c = 0; c < WK; c++) v += red[(c * M + tok) * 32 + row];
            if (tile < T) __builtin_nontemporal_store(v, a.y + (size_t)tok * rows + tile * TILE + (row & 15));
        }
    }
}

// prefill_kernel
//
// On v_mfma_f32_32x32x16_bf16 (on gfx950 it sustains about twice the rate of the 16x16x32 form). A: 32 tokens x 16
// columns of activations, lane l holding token l % 32, columns 8 (l / 32) .. + 7; B: 16 columns x 32 outputs (two
// tiles), lane l holding output l % 32, the same columns; D: lane l holds output l % 32 of tokens
// 8 (v / 4) + 4 (l / 32) + v % 4, v = 0..15.
//
// The same packed blocks as the skinny kernel serve as B: for a 32-output block (tiles 2p, 2p + 1) and a group, lane
// l reads two 16-byte pieces of its tile's block, those of block lanes 16 (l / 32) + l % 16 and 32 + the same, which
// hold its output row's columns for k16 steps 2i (first piece, word i) and 2i + 1 (second piece, word i).
//
// A workgroup of WM x WN waves computes WM * BMB * 32 tokens x WN * TN * 32 outputs; wave (wm, wn) owns BMB token
// blocks x TN output blocks (BMB * TN accumulators of 16 registers). Activations go global -> LDS directly
// (global_load_lds_dwordx4, no register round trip) into double-buffered, XOR-swizzled stages of 64 columns; each wave
// dequantizes its outputs' weights straight from global memory into bf16 registers ((q - z) s in f32, rounded once).
//
// Work distribution. A work item is one workgroup tile. Whole items go to the first dp_items workgroups, ordered
// XCD-aware, weight tiles fastest (an XCD's workgroups then share one token tile's activations in its L2; measured
// 0-8% faster than token tiles fastest at M = 512 and 2048). When whole items would leave the last round of
// resident workgroups badly underfilled, the last sk_items items are instead spread evenly
// over sk_wgs = P workgroups (one per resident slot) by groups of K ("stream-K"): of the U = sk_items * G
// (item, group) units, range s takes a contiguous q = U / P of them, one more for the first r = U % P; ranges are
// dealt to the workgroups XCD-aware too.
// An item cut between workgroups is finished by the last of them to arrive: each writes its partial accumulators to
// its own slot of a scratch buffer (device-coherent stores), then counts itself on the item's counter (a returning
// device-scope atomic); the one that counts last adds the partials in segment order (so the sum does not depend on
// who arrives last; its own share from its registers when it is the item's first segment, the usual case), runs the
// epilogue and clears the counter. No workgroup ever waits for another.

// H16: the operands are f16 (v_mfma_f32_32x32x16_f16, the same rate), else bf16
template <bool H16 = false>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, bf16x8 b, f32x16 c) {
    if constexpr (H16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
}

// Whether a prefill launch runs f16 operands: SwiGLU products of int4 and grouped int8 weights. Their activations come
// converted to f16 (x16_kernel) and each dequantized weight (q - z) s rounds once to f16, the reference's own operands
// (f16 activations, weights rounded to f16 in its Marlin dequant): 8 times finer than bf16 rounding, which the
// epilogue's product of two outputs would otherwise carry beyond the bar. Other products keep bf16: dense bf16 and
// per-channel int8 weights are exact there, and plain outputs hold the bar with bf16 weights.
__host__ __device__ constexpr bool prefill_h16(int fmt, int epi) {
    return epi == EPI_SILU && !(fmt & (F_BF16 | F_PERCH));
}

constexpr int PF_BK = 64;            // columns per LDS stage (half a group; 128-column stages measured the same)
constexpr int PF_ROW = PF_BK * 2;    // LDS bytes per token row of a stage
constexpr int PF_K16 = PF_BK / 16;   // k16 steps per stage

// LDS byte offset of 16-byte chunk kc (0..7) of token row `row` in a stage: XOR-swizzled so that 16 lanes reading
// 16 consecutive rows at one chunk hit all 64 banks once (rows of 128 bytes pair up in one 256-byte bank line).
__device__ __forceinline__ int pf_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int pf_lds_off(int row, int kc) { return row * PF_ROW + 16 * (kc ^ pf_swz(row)); }

typedef __attribute__((address_space(3))) void* lds_ptr;

// 16 bytes per lane global -> LDS (global_load_lds_dwordx4: wave-uniform base + 32-bit lane offset) into the 1 KiB at
// dst. In inline assembly: with its own form of this load in flight the compiler cannot order the wave's LDS reads
// against it and waits for every outstanding LDS operation (lgkmcnt(0)) at the next read's use, which in the
// ping-pong's MFMA phase drains the A-fragment ring before the first MFMA. The data's readers are ordered by the
// s_waitcnt and workgroup barrier that follow every stage's loads.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, lds_ptr dst) {
    // both wave-uniform by construction; read from the first lane so that they are in scalar registers whatever the
    // compiler could prove
    const uint64_t b = (uint64_t)(uintptr_t)base;
    // (readfirstlane returns a signed int: each half is zero-extended before it is put in place)
    const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t d = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(bs), "{m0}"(d) : "memory");
}

// buffer resource word 3 (gfx9: 32-bit data format, no swizzle) and the sc1 cache-policy bit of buffer operations
constexpr int BUF_RSRC_WORD3 = 0x00020000;
constexpr int CPOL_SC1 = 16;

// Stream-K ranges: U units over P workgroups, q = U / P (at least 1) each and one more for the first r = U % P.
// The first unit of workgroup s, and the workgroup whose range holds unit u:
__device__ __forceinline__ int sk_begin(int s, int q, int r) { return s * q + min(s, r); }
__device__ __forceinline__ int sk_owner(int u, int q, int r) {
    return u < r * (q + 1) ? u / (q + 1) : r + (u - r * (q + 1)) / q;
}

template <int F, int EPI, int BMB, int TN, int WM, int WN, int MINB, bool LORA>
__global__ __launch_bounds__(WM * WN * 64, MINB) void prefill_kernel(Launch a) {
    constexpr int BM = WM * BMB * 32;                // tokens per workgroup
    constexpr int WTILES = WN * TN * 2;              // 16-row tiles per workgroup
    constexpr int CW = CodeWords<F>::N;
    constexpr int STAGE = BM * PF_ROW;               // LDS bytes of one stage
    constexpr int NW = WM * WN;                      // waves
    constexpr int NACC = BMB * TN * 16;              // accumulator registers per lane
    constexpr bool H16 = prefill_h16(F, EPI);        // f16 operands (activations converted by x16_kernel)
    // two objects, so that the compiler can tell the direct-to-LDS loads into one from the reads of the other
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[STAGE];
    // the ping-pong schedule (below) keeps a whole group's two stages and the next group's in flight: two more stage
    // buffers
    constexpr bool PP = NW == 8 && WM == 1 && TN == 1;
    __shared__ __attribute__((aligned(PP ? 1024 : 16))) uint8_t lds2[PP ? STAGE : 16];
    __shared__ __attribute__((aligned(PP ? 1024 : 16))) uint8_t lds3[PP ? STAGE : 16];
    constexpr int NB = STAGE / 1024;           // 1 KiB blocks of a stage
    constexpr int NI = (NB + NW - 1) / NW;     // direct-to-LDS loads per wave per stage (block i NW + wave < NB)
    static_assert(NB * 1024 == STAGE, "stages of whole 1 KiB blocks");
    uint32_t xd[NI];                       // per-lane global byte offsets of those loads (stage 0)
    // LoRA: the item's xa rows ([BM][lora_cols] f32, 16-byte chunks XOR-swizzled by row), staged while the item runs
    __shared__ __attribute__((aligned(16))) uint8_t xa_lds[LORA ? BM * 32 * 4 : 16];
    // the stream-K counter's answer, in lds2: no load writes it in kernels without the ping-pong schedule, and in
    // those with it the next run first writes it after its prologue's barrier, which every wave passes only after
    // reading the answer
    int* const sk_last_p = (int*)lds2;

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int l32 = lane & 31, lh = lane >> 5, l16 = lane & 15;
    const int tiles = a.rows / TILE, G = a.cols / QG, M = a.m;

    const int nwt = (tiles + WTILES - 1) / WTILES;  // weight tiles (of WTILES 16-row tiles); items: weight tiles fastest
    const int wtok0 = wm * BMB * 32;  // the wave's first token row in the stage
    int tok0 = 0, tile0 = 0;          // the current item's first token and the wave's first tile
    int kslice = 0;                   // the partial a K-sliced whole item writes (a.ks > 1)

    // Global loads take a wave-uniform base plus a 32-bit per-lane byte offset fixed for the item (no 64-bit address
    // arithmetic per load).
    const uint8_t* xbase = (const uint8_t*)a.x;
    // LDS reads of A fragments: row wtok0 + 32 bb + l32, chunk 2 s16 + lh; the swizzle of rows 32 bb + l32 depends on
    // l32 only, so the per-lane part is 4 offsets and the token block is an immediate
    int xr[PF_K16];
#pragma unroll
    for (int s16 = 0; s16 < PF_K16; s16++) xr[s16] = pf_lds_off(wtok0 + l32, 2 * s16 + lh);

    // this lane's output row: tile tt[t] (of output block t), row l16; its code pieces and scales as offsets
    int tt[TN];
    uint32_t cg[TN], sg[TN], zg[TN];
    // the per-lane offsets of an item
    auto set_item = [&](int item) __attribute__((always_inline)) {
        tok0 = (item / nwt) * BM;
        tile0 = (item % nwt) * WTILES + wn * TN * 2;
        // activations: load i of this wave fills LDS block i NW + wave, whose lane l writes row 8 block + l / 8, slot
        // l % 8; that slot holds column chunk slot ^ swizzle(row), so the lane fetches that chunk (rows past M read
        // row M - 1: their results are never stored)
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = 8 * (i * NW + wave) + (lane >> 3), kc = (lane & 7) ^ pf_swz(row);
            const int tok = min(tok0 + row, M - 1);
            xd[i] = (uint32_t)(((size_t)(a.xrows ? a.xrows[tok] : tok) * a.ldx + 8 * kc) * 2);
        }
#pragma unroll
        for (int t = 0; t < TN; t++) {
            tt[t] = min(tile0 + 2 * t + (l32 >> 4), tiles - 1);
            cg[t] = (uint32_t)(((size_t)tt[t] * G * 64 * CW + 16 * lh + l16) * 16);
            sg[t] = (uint32_t)(scale_idx(tt[t], tiles, 0, l16) * ((F & F_S32) ? 4 : 2));
            zg[t] = (uint32_t)(zero_idx(tt[t], tiles, 0, l16) * 2);
        }
    };
    // a group's weights as loaded: codes, and the raw scale and zero-point words, converted only where the group is
    // dequantized (converted at the load, the compiler would hold the wave there for every load in flight)
    struct WFrag {
        u32x4 c[TN][2][CW];  // per output block: the two pieces (x CW words for int8)
        uint32_t sr[TN], zr[TN];
        int zs;  // the group's zero point: bits zs .. zs + 3 of zr
    };
    auto wload = [&](int g, WFrag& f) __attribute__((always_inline)) {
        const uint8_t* cb = (const uint8_t*)a.codes + (size_t)g * 64 * CW * 16;
        const size_t sq = ((size_t)(g >> 2) * tiles * TILE * 4 + (g & 3)) * ((F & F_S32) ? 4 : 2);
        f.zs = 4 * (g & 3);
#pragma unroll
        for (int t = 0; t < TN; t++) {
#pragma unroll
            for (int pc = 0; pc < 2; pc++)
#pragma unroll
                for (int h = 0; h < CW; h++) f.c[t][pc][h] = *(const u32x4*)(cb + cg[t] + (h * 64 + 32 * pc) * 16);
            f.sr[t] = f.zr[t] = 0;
            if (!(F & (F_BF16 | F_PERCH))) {
                const uint8_t* sp = (const uint8_t*)a.scales + sq + sg[t];
                f.sr[t] = (F & F_S32) ? *(const uint32_t*)sp : (uint32_t)*(const uint16_t*)sp;
                if (F & F_ZP)
                    f.zr[t] = *(const uint16_t*)((const uint8_t*)a.zeros + (size_t)(g >> 2) * tiles * TILE * 2 + zg[t]);
            }
        }
    };
    // the scale s and offset -z s of output block t
    auto scale_off = [&](const WFrag& f, int t, float& sc, float& off) __attribute__((always_inline)) {
        if (F & F_BF16) {
            sc = 1.0f;  // the weights themselves
            off = 0.0f;
        } else if (F & F_PERCH) {
            sc = 1.0f;  // exact integers q = stored - 128; the row scale comes after the sum
            off = -128.0f;
        } else {
            sc = __uint_as_float((F & F_S32) ? f.sr[t] : f.sr[t] << 16);
            const int z = (F & F_ZP) ? (int)((f.zr[t] >> f.zs) & 15u) : ((F & F_I8) ? 128 : 8);
            off = -(float)z * sc;
        }
    };
    // B fragment of output block t for k16 step kk (0..7) of the group
    auto dequant = [&](const WFrag& f, int t, int kk, float sc, float off) __attribute__((always_inline)) -> bf16x8 {
        const int pc = kk & 1, i = kk >> 1;
        if (F & F_BF16) return __builtin_bit_cast(bf16x8, f.c[t][pc][i]);  // step kk's piece as stored
        if (F & F_I8)  // int8: word pair (2e, 2e + 1) of half h, for k32 step i = 2h + e
            return i8_scaled<H16>(f.c[t][pc][i >> 1][2 * (i & 1)], f.c[t][pc][i >> 1][2 * (i & 1) + 1], sc, off);
        return i4_scaled<H16>(f.c[t][pc][0][i], sc, off);
    };

    f32x16 acc[BMB][TN];
    auto clear = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int bb = 0; bb < BMB; bb++)
#pragma unroll
            for (int t = 0; t < TN; t++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[bb][t][e] = 0.0f;
    };

    // one stage (64 columns, half hh of the group) from LDS buffer `buf`: the A fragments of k16 step s16 + 1 are read
    // while step s16's MFMAs run
    auto compute = [&](int buf, int hh, const WFrag& w) __attribute__((always_inline)) {
        const uint8_t* lb = buf ? lds1 : lds0;
        float wsc[TN], woff[TN];
#pragma unroll
        for (int t = 0; t < TN; t++) scale_off(w, t, wsc[t], woff[t]);
        // raised issue priority while this wave's MFMAs run: of the SIMD's waves, the one in its MFMA phase issues
        // first and the other fills the gaps with its loads, LDS stores and barrier (measured: equal or faster on
        // every prefill shape, +9% on (17408, 5120) at 512 tokens)
        __builtin_amdgcn_s_setprio(1);
        u32x4 xa[2][BMB];
#pragma unroll
        for (int bb = 0; bb < BMB; bb++) xa[0][bb] = *(const u32x4*)(lb + xr[0] + bb * 32 * PF_ROW);
#pragma unroll
        for (int s16 = 0; s16 < PF_K16; s16++) {
            if (s16 < PF_K16 - 1) {
#pragma unroll
                for (int bb = 0; bb < BMB; bb++)
                    xa[(s16 + 1) & 1][bb] = *(const u32x4*)(lb + xr[s16 + 1] + bb * 32 * PF_ROW);
            }
            bf16x8 bw[TN];
#pragma unroll
            for (int t = 0; t < TN; t++) bw[t] = dequant(w, t, PF_K16 * hh + s16, wsc[t], woff[t]);
#pragma unroll
            for (int bb = 0; bb < BMB; bb++)
#pragma unroll
                for (int t = 0; t < TN; t++) acc[bb][t] = mfma32<H16>(xa[s16 & 1][bb], bw[t], acc[bb][t]);
        }
        __builtin_amdgcn_s_setprio(0);
    };

    // acc = the current item's product over groups [g0, g1). The activations go global -> LDS directly
    // (global_load_lds_dwordx4): stage 2g (the group's first 64 columns) is computed from lds0 while stage 2g + 1 loads
    // into lds1 and the next group's weights into registers, then stage 2g + 1 from lds1 while stage 2g + 2 loads into
    // lds0; each stage ends with a wait for this wave's loads in flight (the next stage's activations and the next
    // group's weights) and one workgroup barrier.
    auto stage_issue = [&](int st, uint8_t* buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NI; i++)
            if (NB % NW == 0 || i * NW + wave < NB) {  // wave-uniform
                // the ping-pong schedule issues them in inline assembly (measured +3% at 2048 tokens); the shared one
                // in the compiler's form (1-3% faster there at 256 tokens)
                if constexpr (PP)
                    lds_dma16((const void*)(xbase + (size_t)st * PF_ROW), xd[i], (lds_ptr)(buf + (i * NW + wave) * 1024));
                else
                    __builtin_amdgcn_global_load_lds((const void*)(xbase + (size_t)st * PF_ROW + xd[i]),
                                                     (lds_ptr)(buf + (i * NW + wave) * 1024), 16, 0, 0);
            }
    };
    // LoRA: the item's xa rows (tokens tok0 .., clamped to m - 1) go global -> LDS while the item runs; the run's
    // barriers make them the workgroup's before the epilogue reads them
    auto xa_stage = [&]() __attribute__((always_inline)) {
        if constexpr (LORA) {
            if (a.lora_stage) {
                const int cpr = a.lora_cols >> 2, nblk = BM * cpr / 64;  // 16-byte chunks per row; 1 KiB blocks
                for (int blk = wave; blk < nblk; blk += NW) {
                    const int e = blk * 64 + lane, row = e / cpr, k = (e - row * cpr) ^ (row & (cpr - 1));
                    const float* src = a.lora_xa + (size_t)min(tok0 + row, M - 1) * a.lora_cols + 4 * k;
                    __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr)(xa_lds + blk * 1024), 16, 0, 0);
                }
            }
        }
    };
    auto run = [&](int g0, int g1) __attribute__((always_inline)) {
        clear();
        WFrag wcur, wnxt;
        stage_issue(2 * g0, lds0);
        wload(g0, wcur);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        xa_stage();
        for (int g = g0; g < g1; g++) {
            const bool more = g + 1 < g1;
            // stage 2g from lds0 while stage 2g + 1 loads into lds1 (the next group's weights behind it)
            stage_issue(2 * g + 1, lds1);
            __builtin_amdgcn_sched_barrier(0);  // the weight loads behind the activation loads
            wload(more ? g + 1 : g, wnxt);
            compute(0, 0, wcur);
            __builtin_amdgcn_s_waitcnt(0);  // stage 2g + 1, read after the barrier, has landed (and the weights)
            __syncthreads();
            if (more) stage_issue(2 * g + 2, lds0);
            compute(1, 1, wcur);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            wcur = wnxt;
        }
    };
    // Ping-pong (PP: 256 x 256 items on 8 waves). The SIMD's two waves (w and w + 4) take turns: while one runs a
    // group's 64 MFMAs (raised issue priority, A fragments read six ahead through a register ring), the other
    // dequantizes its weights for its next group into registers; a workgroup barrier ends each half. Activations: a
    // group's two stages in one pair of LDS buffers while the next group's load into the other pair (issued at the
    // group's start, waited for only at its end: the barrier between the halves carries no wait for them). Against the shared schedule above, same box, M = 2048: int4 (5120, 17408) / (17408, 5120) +2-3%,
    // int8 +1-3.5%, zero points +3-5%, the fused LoRA delta 0 to +5% (MFMA busy 0.540 -> 0.564 and 0.564 -> 0.599, at a
    // slightly lower clock).
    bf16x8 bwg[2 * PF_K16][TN];  // a group's B fragments, dequantized a half ahead of their MFMAs
    auto deq_group = [&](const WFrag& w) __attribute__((always_inline)) {
        float wsc[TN], woff[TN];
#pragma unroll
        for (int t = 0; t < TN; t++) scale_off(w, t, wsc[t], woff[t]);
#pragma unroll
        for (int kk = 0; kk < 2 * PF_K16; kk++)
#pragma unroll
            for (int t = 0; t < TN; t++) bwg[kk][t] = dequant(w, t, kk, wsc[t], woff[t]);
    };
    // the group's 16 k16 steps from the two stage buffers
    auto mfma_group = [&](const uint8_t* la, const uint8_t* lb2) __attribute__((always_inline)) {
        __builtin_amdgcn_s_setprio(1);
        constexpr int NF = 2 * PF_K16 * BMB, LA = 6;  // A fragments (k16 step f / BMB, token block f % BMB); ring
        auto addr = [&](int f) __attribute__((always_inline)) -> const u32x4* {
            const int kk = f / BMB, bb = f % BMB;
            return (const u32x4*)((kk < PF_K16 ? la : lb2) + xr[kk % PF_K16] + bb * 32 * PF_ROW);
        };
        u32x4 ring[LA];
#pragma unroll
        for (int f = 0; f < LA; f++) ring[f] = *addr(f);
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const u32x4 cur = ring[f % LA];
            if (f + LA < NF) ring[f % LA] = *addr(f + LA);
#pragma unroll
            for (int t = 0; t < TN; t++) acc[f % BMB][t] = mfma32<H16>(cur, bwg[f / BMB][t], acc[f % BMB][t]);
        }
        // the order above, kept by the scheduler: LA reads, then each MFMA followed by the next read
        __builtin_amdgcn_sched_group_barrier(0x100, LA, 0);
#pragma unroll
        for (int f = 0; f < NF - LA; f++) {
            __builtin_amdgcn_sched_group_barrier(0x8, TN, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x8, TN * LA, 0);
        __builtin_amdgcn_s_setprio(0);
    };
    // group g of a run for ping-pong role GRP (0: MFMAs first): its stages in buffers (a0, a1), the next group's
    // loading into (b0, b1), whose last readers passed the previous barrier
    auto pp_group = [&](auto GRP, int g, int g1, uint8_t* a0, uint8_t* a1, uint8_t* b0, uint8_t* b1, WFrag& wcur,
                        WFrag& wnxt) __attribute__((always_inline)) {
        constexpr int grp = decltype(GRP)::value;
        const bool more = g + 1 < g1;
        if (more) {
            stage_issue(2 * g + 2, b0);
            stage_issue(2 * g + 3, b1);
        }
        __builtin_amdgcn_sched_barrier(0);  // the weight loads stay behind the activation loads
        wload(more ? g + 1 : g, wnxt);
        if (grp == 0) mfma_group(a0, a1);
        else deq_group(wcur);
        __syncthreads();
        if (grp == 0) {
            if (more) deq_group(wnxt);
        } else {
            mfma_group(a0, a1);
        }
        __builtin_amdgcn_s_waitcnt(0);  // the next group's activations (and weights) landed
        __syncthreads();
        wcur = wnxt;
    };
    // acc = the current item's product over groups [g0, g1), ping-pong role GRP
    auto run_pp = [&](auto GRP, int g0, int g1) __attribute__((always_inline)) {
        constexpr int grp = decltype(GRP)::value;
        clear();
        WFrag wcur, wnxt;
        stage_issue(2 * g0, lds0);
        stage_issue(2 * g0 + 1, lds1);
        wload(g0, wcur);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        xa_stage();
        if (grp == 0) deq_group(wcur);
        for (int g = g0; g < g1; g += 2) {  // two groups per pass: the buffer pairs stay known at compile time
            pp_group(GRP, g, g1, lds0, lds1, lds2, lds3, wcur, wnxt);
            if (g + 1 < g1) pp_group(GRP, g + 1, g1, lds2, lds3, lds0, lds1, wcur, wnxt);
        }
    };
    // epilogue of the current item: acc[bb][t][v] = D[token tok0 + wtok0 + 32 bb + 8 (v / 4) + 4 lh + v % 4]
    // [output 32-block t, l32]
    auto epilogue = [&]() __attribute__((always_inline)) {
        if (F & F_PERCH) {  // the row's scale after the exact integer sum
#pragma unroll
            for (int t = 0; t < TN; t++) {
                const float rs = scale_of<F>(a.scales, tt[t], tiles, 0, l16);
#pragma unroll
                for (int bb = 0; bb < BMB; bb++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[bb][t][e] *= rs;
            }
        }
        // the LoRA delta: on partial 0 of a plain product, before the activation of a SwiGLU one
        if constexpr (LORA) {
            if (EPI == EPI_SILU || kslice == 0) {
                lora_item32<EPI == EPI_SILU, BMB, TN>(a, tile0, tok0 + wtok0, acc, a.lora_stage ? xa_lds : nullptr,
                                                      wtok0);
            }
        }
        unsigned long long key[BMB][16];
#pragma unroll
        for (int bb = 0; bb < BMB; bb++)
#pragma unroll
            for (int v = 0; v < 16; v++) key[bb][v] = 0;
#pragma unroll
        for (int t = 0; t < TN; t++) {
            const int tile = tile0 + 2 * t + (l32 >> 4);
            const bool tile_ok = tile < tiles;
            const int out = tile * TILE + l16;
#pragma unroll
            for (int bb = 0; bb < BMB; bb++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int tok = tok0 + wtok0 + 32 * bb + 8 * (v >> 2) + 4 * lh + (v & 3);
                    const float val = acc[bb][t][v];
                    if (EPI == EPI_SILU) {
                        const float up = __shfl_xor(val, 8);
                        if (tile_ok && l16 < 8 && tok < M)
                            ((__bf16*)a.y)[(size_t)tok * a.ldy + tile * 8 + l16] = (__bf16)(silu(val) * up);
                    } else {
                        // streamed past the caches: the outputs are not read again here, the tiles still are
                        if (tile_ok && tok < M)
                            __builtin_nontemporal_store(val, (float*)a.y + ((size_t)kslice * M + tok) * a.ldy + out);
                        if (EPI == EPI_ARGMAX && tile_ok && tok < M && out < a.valid)
                            key[bb][v] = max_u64(key[bb][v], argmax_key(val, out));
                    }
                }
        }
        if (EPI == EPI_ARGMAX) {
            // the max over the 32 lanes that share a token (one lane half)
#pragma unroll
            for (int bb = 0; bb < BMB; bb++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    unsigned long long k = key[bb][v];
#pragma unroll
                    for (int o = 1; o < 32; o <<= 1) k = max_u64(k, __shfl_xor(k, o));
                    const int tok = tok0 + wtok0 + 32 * bb + 8 * (v >> 2) + 4 * lh + (v & 3);
                    if (l32 == 0 && tok < M && k) argmax_spread_max(a, tok, k);
                }
        }
    };

    // This workgroup's units (item * G + group): one whole item for the first dp_items workgroups, XCD-aware
    // (workgroup b runs on XCD b % 8; each XCD gets a contiguous run of items), else its stream-K range.
    const int b = blockIdx.x, dp = a.dp_items;
    int u, u1, s = -1;
    if (b < dp) {
        const int xcd = b & 7, q8 = dp >> 3, r8 = dp & 7, ui = xcd * q8 + min(xcd, r8) + (b >> 3);
        if (a.ks > 1) {  // slice kslice of K of item ui / ks, written as partial kslice
            const int item = ui / a.ks;
            kslice = ui - item * a.ks;
            u = item * G + kslice * G / a.ks;
            u1 = item * G + (kslice + 1) * G / a.ks;
        } else {
            u = ui * G;
            u1 = u + G;
        }
    } else {
        // stream-K range s, XCD-aware like whole items: workgroups b and b + 8 run on one XCD, and each XCD takes a
        // contiguous run of ranges (so the items they cut share its L2)
        const int c = b - dp, xcd = c & 7, q8 = a.sk_wgs >> 3, r8 = a.sk_wgs & 7;
        s = xcd * q8 + min(xcd, r8) + (c >> 3);
        u = dp * G + sk_begin(s, a.sk_q, a.sk_r);
        u1 = dp * G + sk_begin(s + 1, a.sk_q, a.sk_r);
    }
    // the stream-K partials, as a buffer resource: 16-byte loads and stores with the agent-coherence cache policy
    // (sc1, what agent-scope atomics use), at byte offsets [slot][wave][register / 4][lane][4] f32
    constexpr int NQ = NACC / 4, SK_QC = NQ >= 32 ? 16 : NQ / 2;
    const __amdgpu_buffer_rsrc_t skr = __builtin_amdgcn_make_buffer_rsrc(a.sk_part, 0, (int)PF_SK_PART_BYTES,
                                                                         BUF_RSRC_WORD3);
    auto sk_off = [&](int slot, int w, int l) __attribute__((always_inline)) -> uint32_t {
        return (uint32_t)((((size_t)slot * NW + w) * NQ * 64 + l) * 16);
    };
    const int first_item = u / G;
    // the work loop, instantiated once per ping-pong role (a role known at compile time keeps the compiler from
    // merging the two roles' live registers, which spilled)
    auto work = [&](auto GRP) __attribute__((always_inline)) {
    while (u < u1) {
        const int it = u / G, g0 = u - it * G, g1 = min(G, g0 + (u1 - u));
        set_item(it);
        if constexpr (PP) run_pp(GRP, g0, g1);
        else run(g0, g1);
        u += g1 - g0;
        if (a.ks == 1 && (g0 != 0 || g1 != G)) {
            // a cut item (stream-K): write this segment's partial to slot 2 s (+1 unless it is this workgroup's
            // first item), as [wave][register / 4][lane][4] f32, with 16-byte device-coherent stores
            const uint32_t part = sk_off(2 * s + (it != first_item), wave, lane);
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                const f32x16& v = acc[(q >> 2) / TN][(q >> 2) % TN];
                const int e = (q & 3) * 4;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{v[e], v[e + 1], v[e + 2], v[e + 3]}),
                                                       skr, part + q * 1024, 0, CPOL_SC1);
            }
            __builtin_amdgcn_s_waitcnt(0);  // this wave's partial has been performed
            __syncthreads();
            const int sit = it - dp, su = sit * G;  // the item among the stream-K ones, its first unit
            const int sa = sk_owner(su, a.sk_q, a.sk_r), sb = sk_owner(su + G - 1, a.sk_q, a.sk_r);
            if (threadIdx.x == 0)
                *sk_last_p = __hip_atomic_fetch_add(a.sk_count + sit, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(sb - sa);
            __syncthreads();
            if (!*sk_last_p) continue;  // uniform over the workgroup
            // the last segment to arrive: the sum of all segments' partials in segment order from zero (so that it does
            // not depend on the order of arrival), 16 registers at a time. When it is the item's first segment (the
            // usual case: it reached the item at the end of its range), its own share, the sum's first term, stays in
            // its registers; otherwise it reads its own back like the others. Each addition is followed by + 0, which
            // gives the sum from zero exactly in both cases: (0 + a) + b = (a + b) + 0 for all a, b, and no later sum
            // from zero is -0 (x + (-x) is +0), so the further + 0 change nothing.
            const bool own_first = s == sa;
            if (!own_first) clear();
            for (int o = own_first ? sa + 1 : sa; o <= sb; o++) {
                const uint32_t src = sk_off(2 * o + (sk_begin(o, a.sk_q, a.sk_r) < su), wave, lane);
#pragma unroll
                for (int q0 = 0; q0 < NQ; q0 += SK_QC) {
                    f32x4 v[SK_QC];
#pragma unroll
                    for (int i = 0; i < SK_QC; i++)
                        v[i] = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(skr, src + (q0 + i) * 1024, 0, CPOL_SC1));
#pragma unroll
                    for (int i = 0; i < SK_QC; i++) {
                        const int q = q0 + i, e = (q & 3) * 4;
                        f32x16& d = acc[(q >> 2) / TN][(q >> 2) % TN];
#pragma unroll
                        for (int c = 0; c < 4; c++) d[e + c] = (d[e + c] + v[i][c]) + 0.0f;
                    }
                    __builtin_amdgcn_sched_barrier(0);  // one chunk of loads in flight at a time (registers)
                }
            }
            if (threadIdx.x == 0)
                (void)__hip_atomic_exchange(a.sk_count + sit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        epilogue();
    }
    };
    if (PP && (wave >> 2) != 0) work(std::integral_constant<int, 1>{});
    else work(std::integral_constant<int, 0>{});
}

// ---------------------------------------------------------------------------------------------------------------
// launchers

template <int F, int EPI, int NR, int NG, int TB>
static hipError_t skinny_ng(const Launch& l) {
    if (64 * l.waves > (TB == 1 ? 1024 : 512)) return hipErrorInvalidConfiguration;  // the kernel's launch bound
    const int tiles = l.rows / TILE;
    const int per_wg = l.tiles_per_wave * l.tile_waves;
    dim3 grid((tiles + per_wg - 1) / per_wg, l.split);
    Launch k = l;
    const int wk = l.waves / l.tile_waves;
    k.nc = l.cols / QG / (wk * NG);
    if (l.split != 1 && l.split != k.nc) return hipErrorInvalidConfiguration;  // the kernel's two cases
    // one tile per wave: plain int8 and bf16 products of 1-2 tokens (the partition's choice)
    constexpr bool T1 = EPI == EPI_PLAIN && NR <= 2 && TB == 1 && (F & (F_I8 | F_BF16));
    if (T1 && l.tiles_per_wave == 1)
        hipLaunchKernelGGL((skinny_kernel<F, EPI, NR, 1, NG, TB>), grid, dim3(64 * l.tile_waves, wk), skinny_lds(l),
                           l.stream, k);
    else if (l.tiles_per_wave == SKINNY_TILES)
        hipLaunchKernelGGL((skinny_kernel<F, EPI, NR, SKINNY_TILES, NG, TB>), grid, dim3(64 * l.tile_waves, wk),
                           skinny_lds(l), l.stream, k);
    else
        return hipErrorInvalidConfiguration;
    if (EPI == EPI_ARGMAX) {
        const hipError_t e = hipGetLastError();
        return e != hipSuccess ? e : argmax_fold(l, l.m);
    }
    return hipGetLastError();
}

template <int F, int EPI, int NR, int TB = 1>
static hipError_t skinny_nr(const Launch& l) {
    if constexpr ((F & F_BF16) != 0)
        return skinny_ng<F, EPI, NR, 1, TB>(l);  // one 4 KiB group of a tile per wave
    else
        return l.groups_per_wave == 4 ? skinny_ng<F, EPI, NR, 4, TB>(l) : skinny_ng<F, EPI, NR, 1, TB>(l);
}

// Waves per workgroup of the workgroup-per-tile-pair kernels for nc chunks of K: a wave per 4-group chunk up to 8,
// beyond that the chunks dealt out in turn. Eight-wave workgroups fill a CU's 24 wave slots (6 waves per SIMD) with
// three workgroups, where 10- or 5-wave ones leave 4 idle. Same-box graph replays, us per whole-row product, against
// the earlier rule (a wave per chunk up to 16, two chunks a wave when the grid would not fit one round of resident
// workgroups: 10 / 5, 12 and 12 waves here): one token (5120, 17408) 10.70 -> 10.09, (17408, 5120) 11.17 -> 10.88,
// (5120, 6144) 5.40 -> 5.31, (6144, 5120) 5.52 -> 5.42; five tokens 12.31 -> 11.79, 14.04 -> 12.65, 6.32 -> 6.10,
// 6.70 -> 6.39; the 27B step with every plain product as whole rows 0.2736 -> 0.2638 ms, the decode layer with its
// consumers 0.1888 -> 0.1853 ms (its [gate; up] SwiGLU and in-projection on these kernels), the head the same. 6, 4
// or 16 waves were slower.
static int mw_waves(int nc) { return std::min(nc, 8); }

// token rows per lane (NR, of a 16-token block: tokens 4 r + lane / 16) and 16-token blocks (TB) for m tokens
template <int F, int EPI>
static hipError_t skinny_epi(const Launch& l) {
    if constexpr (F == F_I4 || F == F_ZP) {
        // Products that need whole sums of their rows, on the workgroup-per-tile-pair kernels (skinny_m1w_kernel at one
        // token, skinny_mw_kernel for whole plain rows of 2-8 tokens): the one-token argmax, whole plain products, and
        // the one-token SwiGLU product when K has at most 16 chunks of 4 groups. Same-box graph replays: the 27B
        // [gate; up] product (2 x 17408 rows, K 5120) 20.6 -> 18.9 us; the 27B head with its argmax, once the fold
        // became a launch of its own (while each workgroup counted itself done with a returning atomic, twice the
        // workgroups made it 20% slower), the headline step 0.2509 -> 0.2497 ms, and with keys[0] as the workgroups'
        // filter and target (no fold launch) 0.2495 ms against 0.2517 on another box (at 5 tokens the head on
        // skinny_mw_kernel made the step 0.2852 -> 0.3011 ms: it stays on skinny_kernel); whole plain products below
        // the split product plus the sum of its partials (see qh_gemm's `whole`).
        const int G = l.cols / QG;
        const bool fits = !l.lora_rank && G % 4 == 0 &&
                          ((EPI == EPI_ARGMAX && l.m == 1) || (EPI == EPI_PLAIN && l.split == 1) ||
                           (EPI == EPI_SILU && l.m == 1 && G / 4 <= 16 && !l.xrows));
        if (fits && l.m == 1) {
            const int tiles = l.rows / TILE, wk = mw_waves(G / 4);
            const M1wArgs a{(const u32x4*)l.codes, (const uint16_t*)l.scales, l.zeros, (const __bf16*)l.x, l.y,
                            l.keys, tiles, G, l.valid, l.nib_mask, l.bf16_magic, l.xrows, l.ldx};
            const size_t lds = (size_t)wk * 4 * QG * 2 + (size_t)wk * 32 * 4;
            hipLaunchKernelGGL((skinny_m1w_kernel<EPI, F == F_ZP>), dim3((tiles + 1) / 2), dim3(64 * wk), lds, l.stream,
                               a);
            return hipGetLastError();
        }
        if constexpr (EPI == EPI_PLAIN) {
            if (fits && l.m >= 2 && l.m <= 8) {
                const int tiles = l.rows / TILE, nc = G / 4, wk = mw_waves(nc);
                const MtArgs a{(const u32x4*)l.codes, (const uint16_t*)l.scales, l.zeros, (const __bf16*)l.x, l.ldx,
                               (float*)l.y, tiles, G, l.m, l.nib_mask, l.bf16_magic};
                const size_t lds = (size_t)wk * l.m * mt_xpitch<4>() * 2 + (size_t)wk * l.m * 32 * 4;
                const dim3 grid((tiles + 1) / 2), block(64 * wk);
                // accumulator rows per lane: ceil(m / 4)
                if (l.m <= 4) hipLaunchKernelGGL((skinny_mw_kernel<F == F_ZP, 1>), grid, block, lds, l.stream, a);
                else hipLaunchKernelGGL((skinny_mw_kernel<F == F_ZP, 2>), grid, block, lds, l.stream, a);
                return hipGetLastError();
            }
        }
    }
    if constexpr ((F == F_I4 || F == F_ZP) && EPI == EPI_PLAIN) {
        // the lean one-token kernel: the partition skinny_partition gives a plain one-token product (4 wave columns of
        // 2 tiles, one chunk of 4 groups, or of one, of K per wave, split = the chunks), no adapter, activations in
        // their own rows
        const int G = l.cols / QG, ng = l.groups_per_wave;
        if (l.m == 1 && !l.lora_rank && !l.xrows && (ng == 4 || ng == 1) && l.tile_waves == 4 && l.waves == 4 &&
            l.split == G / ng && !l.stage_out) {
            const int tiles = l.rows / TILE;
            const M1Args a{(const u32x4*)l.codes, (const uint16_t*)l.scales, l.zeros, (const __bf16*)l.x,
                           (float*)l.y, tiles, G, l.nib_mask, l.bf16_magic};
            const dim3 grid((tiles + 7) / 8, G / ng);
            if (ng == 4)
                hipLaunchKernelGGL((skinny_m1_kernel<F == F_ZP, 4>), grid, dim3(256), 4 * 4 * QG * 2, l.stream, a);
            else
                hipLaunchKernelGGL((skinny_m1_kernel<F == F_ZP, 1>), grid, dim3(256), 4 * 4 * QG * 2, l.stream, a);
            return hipGetLastError();
        }
        // the lean kernel for 2-8 tokens, on the same partition. Same-box graph replays: the 27B step at M = 5
        // 0.302 -> 0.282 ms, the 4B set with zero points at M = 2 4.28 -> 3.95 us per launch, at M = 4 and 5 level;
        // at 6-8 tokens it lost 3% to skinny_kernel's shared staging until its token rows (two accumulator rows per
        // lane from 5 tokens): then the 27B set (no head) at M = 6 / 8 3.68 / 3.69 -> 4.07 / 3.90 TB/s, the 4B set
        // with zero points at M = 8 4.74 -> 4.69 us per launch
        const int wt = l.tile_waves;
        if (l.m >= 2 && l.m <= 8 && !l.lora_rank && !l.xrows && (ng == 4 || ng == 1) && l.waves == wt &&
            wt <= 8 && l.split == G / ng && ((uintptr_t)l.y & 15) == 0) {
            const int tiles = l.rows / TILE;
            const MtArgs a{(const u32x4*)l.codes, (const uint16_t*)l.scales, l.zeros, (const __bf16*)l.x, l.ldx,
                           (float*)l.y, tiles, G, l.m, l.nib_mask, l.bf16_magic};
            const dim3 grid((tiles + 2 * wt - 1) / (2 * wt), G / ng), block(64 * wt);
            // per wave: m staged rows, which also hold its m x 32 partials (m x 128 bytes) afterwards
            const size_t lds = (size_t)wt * l.m * (ng == 4 ? mt_xpitch<4>() : mt_xpitch<1>()) * 2;
            auto go = [&](auto NGc, auto NRc) {
                hipLaunchKernelGGL((skinny_mt_kernel<F == F_ZP, decltype(NGc)::value, decltype(NRc)::value>), grid,
                                   block, lds, l.stream, a);
            };
            using I1 = std::integral_constant<int, 1>;
            using I4 = std::integral_constant<int, 4>;
            using I2 = std::integral_constant<int, 2>;
            // accumulator rows per lane: ceil(m / 4)
            if (ng == 4) {
                if (l.m <= 4) go(I4{}, I1{});
                else go(I4{}, I2{});
            } else {
                if (l.m <= 4) go(I1{}, I1{});
                else go(I1{}, I2{});
            }
            return hipGetLastError();
        }
    }
    if (l.m > 32) return skinny_nr<F, EPI, 4, 3>(l);
    if (l.m > 16) return skinny_nr<F, EPI, 4, 2>(l);
    // accumulator rows per lane: ceil(m / 4), at least 2 from 2 tokens (one row is the one-token form); same-box A/B
    // against rows in token order (2-4 rows from 2 tokens), three pairs: the 27B step at M = 5 0.2813 -> 0.2780 ms
    // (its head), int8 per channel at M = 5 0.1490 -> 0.1466 ms per step, one token unchanged
    if (l.m == 1) return skinny_nr<F, EPI, 1>(l);
    if (l.m <= 8) return skinny_nr<F, EPI, 2>(l);
    if (l.m <= 12) return skinny_nr<F, EPI, 3>(l);
    return skinny_nr<F, EPI, 4>(l);
}

// The launch plan of one prefill shape: whole items or stream-K for the tail, in l.dp_items / sk_*; returns the
// estimated time in units of one group of K on one item of this shape.
// Stream-K: the last P < sk_items <= 2 P items (all of them when there are at most 2 P) are spread over P = the
// resident workgroups, when that is estimated faster: whole items take rounds * G; stream-K takes (rounds - 2) * G for
// the whole rounds, ceil(U / P) for the spread units and PF_SK_FIXUP for the cut items (pipeline refills, writing and
// summing partials; measured on MI355X: about 12 groups of K for 256 x 256 items, so a 75%-full single round of
// K = 5120 stays whole).
template <int F, int EPI, int BMB, int TN, int WM, int WN, int MINB = 1>
static long prefill_plan(Launch& l) {
    l.ks = 1;
    l.split = 1;
    const int tiles = l.rows / TILE, G = l.cols / QG;
    const int wg_tiles = WN * TN * 2, bm = WM * BMB * 32, threads = WM * WN * 64;
    const long items = (long)((tiles + wg_tiles - 1) / wg_tiles) * ((l.m + bm - 1) / bm);
    // resident workgroups per CU (per instantiation; the same on every MI355X; thread-safe static initialisation)
    static const int per_cu = [] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_kernel<F, EPI, BMB, TN, WM, WN, MINB, false>,
                                                         threads, 0) != hipSuccess)
            n = 0;
        return n;
    }();
    const long P = (long)per_cu * l.cus;
    l.dp_items = (int)items;
    l.sk_items = 0;
    l.sk_wgs = 0;
    if (P <= 0) return 1l << 40;
    const long rounds = (items + P - 1) / P, t_dp = rounds * G;
    if (!l.stream_k) return t_dp;
    const size_t slot = (size_t)bm * wg_tiles * TILE * 4;
    const long sk = rounds >= 2 ? items - (rounds - 2) * P : items;
    const long U = sk * G;
    // one group of one item on a CU running per_cu of them at PF_KS_CU_FLOPS (seconds)
    const double unit_s = 2.0 * bm * wg_tiles * TILE * QG * per_cu / PF_KS_CU_FLOPS;
    // the fix-up reads an item's partials one after another, so each piece beyond three adds PF_SK_PIECE_S: with q
    // units per workgroup an item is cut in about ceil(G / q) pieces (measured: 64 x 128 items of 48 groups cut in
    // 48 pieces took 48 us, in 16 pieces 31 us, against 13 and 19 us in 4 K slices)
    const long q = std::max(1l, U / P), pieces = (G + q - 1) / q;
    const long fixup = (l.stream_k > 1 ? l.stream_k : PF_SK_FIXUP) +
                       (long)(std::max(0l, pieces - 3) * PF_SK_PIECE_S / unit_s + 0.5);
    const long t_sk = (rounds >= 2 ? (rounds - 2) * G : 0) + (U + P - 1) / P + fixup;
    if (t_sk * 20 < t_dp * 19 && 2 * P * slot <= PF_SK_PART_BYTES && sk <= PF_SK_ITEMS_MAX && U >= P &&
        items * G < (1l << 31)) {
        l.dp_items = (int)(items - sk);
        l.sk_items = (int)sk;
        l.sk_wgs = (int)P;
        l.sk_q = (int)(U / P);
        l.sk_r = (int)(U % P);
    }
    long t = l.sk_items ? t_sk : t_dp;
    // plain products of few tokens: K slices of whole items, each writing a partial (no stream-K fix-up)
    if (EPI == EPI_PLAIN && !l.whole && l.m <= PF_KS_MAX_M)
        for (int ks = 2; ks <= PF_KS_MAX && ks <= G && (ks <= 4 || G / ks >= PF_KS_MIN_G) && (long)ks * l.m <= PF_KS_ROWS;
             ks *= 2) {
            // the extra partials (ks - 1 more f32 outputs per token and row, written here and read back by the
            // consumer) at PF_KS_HBM bytes/s, in units of unit_s
            const double extra_s = (double)(ks - 1) * l.m * l.rows * 8 / PF_KS_HBM;
            const long units = items * ks,
                       t_ks = (units + P - 1) / P * ((G + ks - 1) / ks) + PF_KS_COST + (long)(extra_s / unit_s + 0.5);
            if (t_ks < t && units < (1l << 31)) {
                t = t_ks;
                l.ks = ks;
                l.split = ks;
                l.dp_items = (int)units;
                l.sk_items = 0;
                l.sk_wgs = 0;
            }
        }
    return t;
}

template <int F, int EPI, int BMB, int TN, int WM, int WN, int MINB = 1>
static hipError_t prefill_cfg(Launch& l) {
    (void)prefill_plan<F, EPI, BMB, TN, WM, WN, MINB>(l);
    if (l.dry_run) return hipSuccess;
    // the LoRA epilogue in kernels of its own (its code would otherwise weigh on every product's registers)
    if constexpr (EPI == EPI_PLAIN || EPI == EPI_SILU)
        if (l.lora_rank) {
            hipLaunchKernelGGL((prefill_kernel<F, EPI, BMB, TN, WM, WN, MINB, true>), dim3(l.dp_items + l.sk_wgs),
                               dim3(WM * WN * 64), 0, l.stream, l);
            return hipGetLastError();
        }
    hipLaunchKernelGGL((prefill_kernel<F, EPI, BMB, TN, WM, WN, MINB, false>), dim3(l.dp_items + l.sk_wgs),
                       dim3(WM * WN * 64), 0, l.stream, l);
    if (EPI == EPI_ARGMAX) {
        const hipError_t e = hipGetLastError();
        return e != hipSuccess ? e : argmax_fold(l, l.m);
    }
    return hipGetLastError();
}

// The prefill workgroup shape (tokens x outputs; waves): 256 token rows (256 x 256 on 8 waves of 256 x 32, or 256 x 192
// on 12 waves when that fills the CUs better), else 128 x 128 on 4 waves, else 64 x 128 on 4 waves; QH_PF_SHAPE forces
// one in tuning sweeps (256 x 128 on 4 waves, 1, and the wider wave tiles 3 and 4 only then).
template <int F, int EPI>
static hipError_t prefill_epi(Launch& l) {
    const int tiles = l.rows / TILE;
    auto items = [&](int bm, int wg_tiles) {
        return (long)((tiles + wg_tiles - 1) / wg_tiles) * ((l.m + bm - 1) / bm);
    };
    // token rows a tile height pads the step to, against the next smaller height (at most 15% more)
    auto pads_ok = [&](int bm) {
        const long h = bm / 2;
        return (l.m + bm - 1) / bm * bm * 20 <= (l.m + h - 1) / h * h * 23;
    };
    // 256-token tiles want four waves per CU, or two where K is long (stream-K's fix-up amortised over 64+ groups);
    // 128 x 128 tiles one (measured over M = 130..2048 on the 27B and 4B shapes)
    const long waves2 = items(256, 16) * 8;
    int shape = l.pf_shape;
    if (shape == 0) {
        if (l.m > 128 && (waves2 >= 4 * l.cus || (waves2 >= 2 * l.cus && l.cols / QG >= 64)) && pads_ok(256)) {
            shape = 2;
            // 256 x 192 on 12 waves when its rounds fill the CUs enough better to outweigh its lower rate (items of
            // 3/4 the work at about 0.85 of the rate of 256 x 256), and only where 256 x 256 items would fill at most
            // 5/8 of the CUs: beside the ping-pong 256 x 256 kernel it won only up to there (measured at 768-4096
            // tokens: at 50-62.5% fill +2-11%, e.g. (2560, 4096) at 2048, (5120, 10240) at 1024, (6144, 5120) at
            // 2048; at 75-150% fill, (5120, 6144) at 2048 and 4096 tokens, it lost 3-6%)
            Launch a = l, b = l;
            a.dry_run = b.dry_run = 1;
            if (items(256, 16) * 8 <= (long)l.cus * 5 &&
                prefill_plan<F, EPI, 4, 1, 2, 6>(a) * 15 < prefill_plan<F, EPI, 8, 1, 1, 8>(b) * 17)
                shape = 7;
        } else if (l.m > 64 && items(128, 8) * 4 >= l.cus && pads_ok(128)) shape = 5;
        else shape = 6;
    }
    switch (shape) {
        case 1: return prefill_cfg<F, EPI, 8, 1, 1, 4>(l);   // 256 x 128; 4 waves of 256 x 32
        case 2: return prefill_cfg<F, EPI, 8, 1, 1, 8>(l);   // 256 x 256; 8 waves of 256 x 32
        case 3: return prefill_cfg<F, EPI, 4, 2, 2, 4>(l);   // 256 x 256; 8 waves of 128 x 64
        case 4: return prefill_cfg<F, EPI, 8, 2, 1, 4>(l);   // 256 x 256; 4 waves of 256 x 64
        case 5: return prefill_cfg<F, EPI, 4, 1, 1, 4>(l);   // 128 x 128; 4 waves of 128 x 32
        case 7: return prefill_cfg<F, EPI, 4, 1, 2, 6>(l);   // 256 x 192; 12 waves of 128 x 32
        default: return prefill_cfg<F, EPI, 2, 1, 1, 4>(l);  // 64 x 128; 4 waves of 64 x 32
    }
}

#if defined(QH_PART_F) && defined(QH_PART_EPI)
// This object holds the kernels of one (format, epilogue) pair: the library compiles kernels.hip once per pair, in
// parallel, plus once with QH_PART_DISPATCH for the dispatcher.
template <int F, int EPI>
hipError_t launch_epi(Launch& l) {
    if (l.skinny) return l.dry_run ? hipSuccess : skinny_epi<F & ~F_PERCH, EPI>(l);
    return prefill_epi<F, EPI>(l);
}
template hipError_t launch_epi<QH_PART_F, QH_PART_EPI>(Launch& l);
#endif

#ifdef QH_PART_DISPATCH
size_t skinny_lds(const Launch& l) {
    const int wk = l.waves / l.tile_waves, tb = (l.m + 15) / 16;
    const size_t x0 = (size_t)l.m * (wk * l.groups_per_wave * QG + 8) * 2;  // the workgroup's staged rows
    const size_t xw = skinny_wave_x(l.m, l.fmt, l.groups_per_wave) ? (size_t)l.waves * l.groups_per_wave * QG * 2 : 0;
    const size_t x = (std::max(x0, xw) + 15) & ~(size_t)15;
    const size_t red = (size_t)(wk - 1) * l.tile_waves * tb * l.tiles_per_wave * 4 * 64 * sizeof(float);
    // plain partials staged per tile column's lead wave: m tokens x tiles_per_wave tiles of f32
    const size_t out = l.stage_out ? (size_t)l.tile_waves * l.m * l.tiles_per_wave * TILE * sizeof(float) : 0;
    return x + std::max(red, out);
}

template <int F>
static hipError_t launch_fmt(Launch& l) {
    switch (l.epi) {
        case EPI_SILU: return launch_epi<F, EPI_SILU>(l);
        case EPI_ARGMAX: return launch_epi<F, EPI_ARGMAX>(l);
        default: return launch_epi<F, EPI_PLAIN>(l);
    }
}

// bf16 activations rows [0, m) (ldx elements apart) -> f16 [m][cols], nearest even (v_cvt_pk_f16_f32; beyond f16's
// range to infinity, as the reference's f16 activations would be): 8 values per thread
__global__ __launch_bounds__(256) void x16_kernel(const uint16_t* x, int ldx, int m, int cols, uint16_t* out) {
    const int per_row = cols / 8;
    const size_t n = (size_t)m * per_row;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / per_row, c = 8 * (i - r * per_row);
        const u32x4 v = *(const u32x4*)(x + r * ldx + c);
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; j++)
            o[j] = pack2<true>(__uint_as_float(v[j] << 16), __uint_as_float(v[j] & 0xffff0000u));
        *(u32x4*)(out + r * cols + c) = o;
    }
}

static hipError_t launch_any(Launch& l) {
    switch (l.fmt) {
        case F_I4: return launch_fmt<F_I4>(l);
        case F_I4 | F_S32: return launch_fmt<F_I4 | F_S32>(l);
        case F_ZP: return launch_fmt<F_ZP>(l);
        case F_ZP | F_S32: return launch_fmt<F_ZP | F_S32>(l);
        case F_I8 | F_S32: return launch_fmt<F_I8 | F_S32>(l);
        case F_I8 | F_S32 | F_PERCH: return launch_fmt<F_I8 | F_S32 | F_PERCH>(l);
        case F_BF16: return launch_fmt<F_BF16>(l);
        default: return hipErrorInvalidValue;
    }
}

// A prefill launch with f16 operands: the activations converted into the x16 scratch first, in token chunks that fit
// it (each chunk one conversion and one product launch, on the same stream; the LoRA adapter's rows follow the chunk).
static hipError_t launch_h16(Launch& l) {
    const size_t per = l.x16 ? l.x16_bytes / ((size_t)l.cols * 2) : 0;
    if (per == 0 || l.xrows) return hipErrorInvalidValue;
    for (int t0 = 0; t0 < l.m; t0 += (int)per) {
        Launch c = l;
        c.m = (int)std::min<size_t>(per, (size_t)(l.m - t0));
        const unsigned blocks = (unsigned)std::min<size_t>(((size_t)c.m * l.cols / 8 + 255) / 256, 2048);
        hipLaunchKernelGGL(x16_kernel, dim3(blocks), dim3(256), 0, l.stream, (const uint16_t*)l.x + (size_t)t0 * l.ldx,
                           l.ldx, c.m, l.cols, (uint16_t*)l.x16);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        c.x = l.x16;
        c.ldx = l.cols;
        c.y = (uint16_t*)l.y + (size_t)t0 * l.ldy;
        if (l.lora_rank) {
            c.lora_xa = l.lora_xa + (size_t)t0 * l.lora_cols;
            c.lora_tok_slot = l.lora_tok_slot + t0;
        }
        if (hipError_t e = launch_any(c); e != hipSuccess) return e;
        l.split = c.split;
    }
    return hipSuccess;
}

hipError_t launch(Launch& l) {
    if (!l.skinny && !l.dry_run && prefill_h16(l.fmt, l.epi)) return launch_h16(l);
    return launch_any(l);
}
#endif

}  // namespace qh
