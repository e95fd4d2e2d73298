// Consumers of the plain products' split-K partials (the output contract y [split][n][ld] f32): the reference's
// sum_parts (kernels/qwen.cu:141-143, part_sum kernels/common.cuh:66-70) and add_rmsnorm (kernels/qwen.cu:57-80),
// the residual step after the o_proj / out_proj / down products, and the LoRA epilogue (kernels/lora.cuh) that adds an
// unmerged adapter's delta to them. The sums are HBM-bound, in f32 in the reference's order (h + x[0], then x[1], x[2],
// ..), so they are bit-identical to it; the LoRA delta runs on the f32 matrix cores.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "internal.h"

using namespace qh;

namespace {

// v += x[0][i] + x[1][i] + .. + x[splits - 1][i], in that order; the partials load B at a time ahead of their adds
// (the sum of 34 partials of a decode product is then 3-5 memory round trips, not 34). Decode sizes, where few
// workgroups each wait on their loads: B = 16 (the 10-12 partials of most decode products in one round trip; 32
// measured slower); streaming sizes: B = 8.
template <int B = 8>
__device__ __forceinline__ void add_splits(float4& v, const float4* __restrict__ x, int splits, long n4, long i) {
    for (int s0 = 0; s0 < splits; s0 += B) {
        float4 p[B];
#pragma unroll
        for (int j = 0; j < B; j++)
            if (s0 + j < splits) p[j] = x[(size_t)(s0 + j) * n4 + i];
#pragma unroll
        for (int j = 0; j < B; j++)
            if (s0 + j < splits) v.x += p[j].x, v.y += p[j].y, v.z += p[j].z, v.w += p[j].w;
    }
}

// y [n][ld] = sum over s of x [s][n][ld] (from 0; h = nullptr), or h [n][ld] += that sum (h + x[0] first, as the
// residual step adds); one thread per 4 columns (ld % 4 == 0), grid-stride over n * ld / 4
template <int B>
__global__ __launch_bounds__(256) void sum_parts_kernel(const float4* __restrict__ x, int splits, long n4, float4* y,
                                                        float4* h) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x) {
        float4 v = h ? h[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        add_splits<B>(v, x, splits, n4, i);
        (h ? h : y)[i] = v;
    }
}

constexpr int AR_THREADS = 256;
// add_rmsnorm spreads the partials' sum over workgroups below this many float4 per step (n * hidden / 4): 64 tokens
// of a 5120-wide row, where a workgroup per token leaves most CUs idle
constexpr long AR_SPREAD_BELOW = 64l * 1280;

// y[t] = bf16(w * (h[t] / rms(h[t]))) with the row held in registers: each of the T threads loads its C float4 of h
// and of w at once (one memory round trip), then the sum of squares and the output (H4 <= T * C)
template <int T, int C>
__global__ __launch_bounds__(T) void rmsnorm_kernel(const float* __restrict__ h, int H, const float* __restrict__ w,
                                                    __bf16* __restrict__ y, float eps) {
    __shared__ float wsum[T / 64];
    const size_t base = (size_t)blockIdx.x * H;
    const int H4 = H / 4;
    float4 v[C], wn[C];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < C; i++) {
        const int c = threadIdx.x + i * T;
        v[i] = c < H4 ? ((const float4*)(h + base))[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        wn[i] = c < H4 ? ((const float4*)w)[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int i = 0; i < C; i++) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < T / 64; i++) tot += wsum[i];
    const float r = rsqrtf(tot / (float)H + eps);
#pragma unroll
    for (int i = 0; i < C; i++) {
        const int c = threadIdx.x + i * T;
        if (c >= H4) break;
        __bf16* yo = y + base + 4 * c;
        yo[0] = (__bf16)(wn[i].x * (v[i].x * r));
        yo[1] = (__bf16)(wn[i].y * (v[i].y * r));
        yo[2] = (__bf16)(wn[i].z * (v[i].z * r));
        yo[3] = (__bf16)(wn[i].w * (v[i].w * r));
    }
}

// token t (one workgroup of T threads): h[t] += the sum of the partials x[.][t]; y[t] = bf16(w * (h[t] / rms(h[t])))
template <int T>
__global__ __launch_bounds__(T) void add_rmsnorm_kernel(float* __restrict__ h, const float* __restrict__ x, int splits,
                                                        int n, int H, const float* __restrict__ w,
                                                        __bf16* __restrict__ y, float eps) {
    __shared__ float wsum[T / 64];
    const size_t base = (size_t)blockIdx.x * H;
    const int H4 = H / 4;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < H4; c += T) {
        float4 v = ((const float4*)(h + base))[c];
        if (splits) {
            add_splits(v, (const float4*)x, splits, (long)n * H4, (long)blockIdx.x * H4 + c);
            ((float4*)(h + base))[c] = v;
        }
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < T / 64; i++) tot += wsum[i];
    const float r = rsqrtf(tot / (float)H + eps);
    // the second pass re-reads this workgroup's own h row (written above by the same threads, same columns)
    for (int c = threadIdx.x; c < H4; c += T) {
        const float4 v = ((const float4*)(h + base))[c], wn = ((const float4*)w)[c];
        __bf16* yo = y + base + 4 * c;
        yo[0] = (__bf16)(wn.x * (v.x * r));
        yo[1] = (__bf16)(wn.y * (v.y * r));
        yo[2] = (__bf16)(wn.z * (v.z * r));
        yo[3] = (__bf16)(wn.w * (v.w * r));
    }
}

// ---------------------------------------------------------------------------------------------------------------
// LoRA consumers (the reference's lora_add / lora_silu, kernels/lora.cuh:52-113, launched by
// src/cuda/qwen/lora.rs:143-190): an unmerged adapter adds s_t B (A x) to a plain product for the tokens t of the slots
// that use it. A x arrives as the split-K partials xa [split][n][cols] of the stacked A product (cols = adapted modules
// x rank); B is f16 [rows][R] in the product's row order; tab (8 ints) holds each module's end row (ascending; unused
// INT_MAX), then its first column of xa (-1: not adapted). Kept from the reference: this interface and its meaning.
//
// The delta of a 16-row tile for 16 tokens is a rank-R update D = Xs . B^T, done on the f32 matrix cores
// (v_mfma_f32_16x16x4_f32: full f32 products and sums, R / 4 steps): A operand = the tokens' xa columns scaled by
// s_t (staged in LDS, summed over the splits once per workgroup), B operand = the tile's B rows (f16, exact in f32).
// The contraction index is laid out so that each lane reads its B values as one contiguous run of R / 4 halves: lane
// group q = lane / 16 takes k = q R / 4 + i for step i. Module routing is per tile: a tile whose rows lie in one
// module (every tile, when module ends are multiples of 16) takes one pass; a tile that straddles a module end takes
// one pass per module with the other modules' B rows masked to zero. The D layout is the one the decode product's
// accumulators have: lane l holds D[token 4 (l / 16) + i][row l % 16], i = 0..3.
//
// A workgroup takes WT * 64 rows (LORA_WAVES waves of WT tiles each: 4 for 17 tokens and more, 1 for fewer, where the
// launch would otherwise have too few waves) and up to LORA_TOK tokens (one 16-token block). The deltas reuse the LDS
// of the staged xa (at most 17 KiB per workgroup), so that 8 workgroups per CU hide each other's memory round trips. The deltas go through LDS so that y is read and written along its rows (whole
// cache lines), not in the MFMA's 16-row pieces.

constexpr int LORA_COLS_MAX = 256;  // columns of xa at most (four modules of rank 64)
constexpr int LORA_TOK = 16;        // tokens per workgroup at most (one 16-token block)
constexpr int LORA_WAVES = 4;
// LDS row pitches (floats): off a multiple of the 64 banks, so that the 16 lanes reading 16 token rows of xs (or the
// lane groups writing 4 token rows of the deltas) hit distinct banks
constexpr int LORA_XS_LD = LORA_COLS_MAX + 1;
template <int WT>
constexpr int lora_dl_ld() { return WT * 64 + 4; }

typedef float lf32x4 __attribute__((ext_vector_type(4)));

struct LoraArgs {
    const float* xa;
    int split, cols;
    const uint16_t* b;
    int rank;
    int rows;
    const int* tab;
    const int* tok_slot;
    const float* slot_scale;
    int n;
    int ldy;
};

// module of output row o: how many module ends lie at or below it
__device__ __forceinline__ int lora_module(const int* tab, int o) {
    int m = 0;
#pragma unroll
    for (int i = 0; i < 3; i++) m += o >= tab[i];
    return m;
}

// xs[t][c] = s_t * sum over splits of xa[.][t0 + t][c] for the workgroup's tokens (0 without the adapter),
// sc[t] = s_t (0 past n). Every thread's xa loads are issued at once, before the slot scales are known (they only
// multiply the sums): one memory round trip beside the scales' two.
__device__ void lora_stage_xs(const LoraArgs& a, int t0, float* xs, float* sc) {
    constexpr int PER = LORA_TOK * LORA_COLS_MAX / (64 * LORA_WAVES);  // elements per thread at most
    const int tn = min(LORA_TOK, a.n - t0), ne = tn * a.cols;
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) v[k] = 0.0f;
    for (int s = 0; s < a.split; s++) {
        const float* xp = a.xa + ((size_t)s * a.n + t0) * a.cols;  // [tn][cols] contiguous
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = threadIdx.x + k * 64 * LORA_WAVES;
            if (i < ne) v[k] += xp[i];
        }
    }
    if (threadIdx.x < LORA_TOK) {
        const int t = t0 + threadIdx.x;
        sc[threadIdx.x] = t < a.n ? a.slot_scale[a.tok_slot[t]] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = threadIdx.x + k * 64 * LORA_WAVES;
        if (i < ne) {
            const int t = i / a.cols, c = i - t * a.cols;
            xs[t * LORA_XS_LD + c] = sc[t] != 0.0f ? v[k] * sc[t] : 0.0f;
        }
    }
    __syncthreads();
}

// The lane's raw B words for row o, columns q R / 4 .. + R / 4 (f16 pairs)
template <int R>
__device__ __forceinline__ void lora_b_load(const uint16_t* b, int o, uint32_t (&w)[R / 8]) {
    const int q = (threadIdx.x & 63) >> 4;
    const uint16_t* p = b + (size_t)o * R + q * (R / 4);
    if constexpr (R / 4 >= 8) {
#pragma unroll
        for (int i = 0; i < R / 8; i += 4) {
            const uint4 u = *(const uint4*)(p + 2 * i);
            w[i] = u.x, w[i + 1] = u.y, w[i + 2] = u.z, w[i + 3] = u.w;
        }
    } else if constexpr (R / 4 == 4) {
        const uint2 u = *(const uint2*)p;
        w[0] = u.x, w[1] = u.y;
    } else {
        w[0] = *(const uint32_t*)p;
    }
}

// The workgroup's part of a LoRA launch: B words of the wave's tiles and the workgroup's y values are loaded first (in
// flight while the tokens' xa is staged), then the deltas of each tile (one masked MFMA pass per module present,
// module_of(row) and off[module]) go through LDS to the threads that own y's rows.
template <int R, int WT>
struct LoraTiles {
    static constexpr int DL_LD = lora_dl_ld<WT>();
    uint32_t bw[WT][R / 8];

    __device__ void load(const LoraArgs& a, int o0) {
        const int wave = threadIdx.x >> 6, l16 = threadIdx.x & 15;
#pragma unroll
        for (int wt = 0; wt < WT; wt++) {
            const int o = min(o0 + (wave * WT + wt) * 16 + l16, a.rows - 1);
            lora_b_load<R>(a.b, o, bw[wt]);
        }
    }

    // xs and dl are the same LDS: every wave's MFMAs read xs before any delta is written
    template <class ModuleOf>
    __device__ void deltas(const LoraArgs& a, int o0, const float* xs, const int* off, ModuleOf module_of,
                           float* dl) const {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, q = lane >> 4;
        lf32x4 d[WT];
#pragma unroll
        for (int wt = 0; wt < WT; wt++) {
            const int r0 = (wave * WT + wt) * 16;  // tile's first row in the workgroup
            d[wt] = lf32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (o0 + r0 >= a.rows) continue;            // wave-uniform
            const int mod = module_of(o0 + r0 + l16), mlo = module_of(o0 + r0), mhi = module_of(o0 + r0 + 15);
            float bv[R / 4];
#pragma unroll
            for (int i = 0; i < R / 8; i++) {
                bv[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(bw[wt][i] & 0xffffu));
                bv[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(bw[wt][i] >> 16));
            }
            for (int m = mlo; m <= mhi; m++) {
                const int c0 = off[m];
                if (c0 < 0) continue;  // wave-uniform: module not adapted
                const bool mine = mod == m;
                const float* xr = xs + l16 * LORA_XS_LD + c0 + q * (R / 4);
#pragma unroll
                for (int i = 0; i < R / 4; i++)
                    d[wt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xr[i], mine ? bv[i] : 0.0f, d[wt], 0, 0, 0);
            }
        }
        __syncthreads();
#pragma unroll
        for (int wt = 0; wt < WT; wt++) {
            const int r0 = (wave * WT + wt) * 16;
#pragma unroll
            for (int i = 0; i < 4; i++) dl[(4 * q + i) * DL_LD + r0 + l16] = d[wt][i];
        }
        __syncthreads();
    }
};

// y [n][ldy] (a plain product's split 0) row o += delta for the adapter tokens; rows of unadapted modules and tokens
// without the adapter are left as they are. Thread i owns rows o0 + 4 (i % QUADS) .. + 3 (one 16-byte access per
// token) of tokens i / QUADS + TS k.
template <int R, int WT>
__global__ __launch_bounds__(64 * LORA_WAVES) void lora_add_kernel(LoraArgs a, float* __restrict__ y) {
    constexpr int ROWS = WT * 64, QUADS = ROWS / 4, DL_LD = lora_dl_ld<WT>(), TS = 64 * LORA_WAVES / QUADS,
                  TPT = LORA_TOK / TS;
    __shared__ float xs[LORA_TOK * (LORA_XS_LD > DL_LD ? LORA_XS_LD : DL_LD)];  // the staged xa, then the deltas
    float* const dl = xs;
    __shared__ float sc[LORA_TOK];
    const int t0 = blockIdx.y * LORA_TOK, o0 = blockIdx.x * ROWS;
    const int tn = min(LORA_TOK, a.n - t0);
    const int c = 4 * (threadIdx.x % QUADS), tp = threadIdx.x / QUADS, o = min(o0 + c, a.rows - 4);
    LoraTiles<R, WT> tiles;
    tiles.load(a, o0);
    float4 v[TPT];
    float* yc = y + (size_t)t0 * a.ldy + o;
#pragma unroll
    for (int k = 0; k < TPT; k++) {
        const int t = min(tp + TS * k, tn - 1);
        v[k] = *(const float4*)(yc + (size_t)t * a.ldy);
    }
    lora_stage_xs(a, t0, xs, sc);
    const int off[4] = {a.tab[4], a.tab[5], a.tab[6], a.tab[7]};
    tiles.deltas(a, o0, xs, off, [&](int r) { return lora_module(a.tab, r); }, dl);
    if (o0 + c >= a.rows) return;
    bool ad[4];  // rows of adapted modules (the others keep their bits, -0.0 included)
#pragma unroll
    for (int i = 0; i < 4; i++) ad[i] = off[lora_module(a.tab, o + i)] >= 0;
    if (!(ad[0] | ad[1] | ad[2] | ad[3])) return;
#pragma unroll
    for (int k = 0; k < TPT; k++) {
        const int t = tp + TS * k;
        if (t >= tn || sc[t] == 0.0f) continue;
        const float4 d = *(const float4*)(dl + t * DL_LD + c);
        float4 r = v[k];
        r.x = ad[0] ? r.x + d.x : r.x;
        r.y = ad[1] ? r.y + d.y : r.y;
        r.z = ad[2] ? r.z + d.z : r.z;
        r.w = ad[3] ? r.w + d.w : r.w;
        *(float4*)(yc + (size_t)t * a.ldy) = r;
    }
}

// mid [n][rows / 2] (bf16) = SwiGLU of the plain [gate; up] product y [n][ldy] (split 1, packed in the SwiGLU
// epilogue's row order: 16-row tile p holds gate rows 8p .. 8p + 7, then their up rows) with the delta added first:
// in a tile, rows 0..7 are module 0 (gate, columns from tab[4]) and rows 8..15 module 1 (up, tab[5]). Thread i owns
// outputs j .. j + 3, j = 4 (i % OQ), of the workgroup (gate rows 16 (j / 8) + j % 8 .. + 3, up rows 8 further: one
// 16-byte load each, one 8-byte store) for tokens i / OQ + TS k.
template <int R, int WT>
__global__ __launch_bounds__(64 * LORA_WAVES) void lora_silu_kernel(LoraArgs a, const float* __restrict__ y,
                                                                   __bf16* __restrict__ mid) {
    constexpr int ROWS = WT * 64, OQ = ROWS / 8, DL_LD = lora_dl_ld<WT>(), TS = 64 * LORA_WAVES / OQ,
                  TPT = TS < LORA_TOK ? LORA_TOK / TS : 1;
    __shared__ float xs[LORA_TOK * (LORA_XS_LD > DL_LD ? LORA_XS_LD : DL_LD)];  // the staged xa, then the deltas
    float* const dl = xs;
    __shared__ float sc[LORA_TOK];
    const int t0 = blockIdx.y * LORA_TOK, o0 = blockIdx.x * ROWS;
    const int tn = min(LORA_TOK, a.n - t0);
    const int half = a.rows / 2, j = 4 * (threadIdx.x % OQ), tp = threadIdx.x / OQ;
    const int rg = 16 * (j >> 3) + (j & 7), og = o0 + rg < a.rows ? o0 + rg : a.rows - 16;  // in bounds
    LoraTiles<R, WT> tiles;
    tiles.load(a, o0);
    float4 g[TPT], u[TPT];
#pragma unroll
    for (int k = 0; k < TPT; k++) {
        const float* yr = y + (size_t)(t0 + min(tp + TS * k, tn - 1)) * a.ldy + og;
        g[k] = *(const float4*)yr;
        u[k] = *(const float4*)(yr + 8);
    }
    lora_stage_xs(a, t0, xs, sc);
    const int off[2] = {a.tab[4], a.tab[5]};
    tiles.deltas(a, o0, xs, off, [](int r) { return (r >> 3) & 1; }, dl);
    if (o0 + rg >= a.rows) return;
#pragma unroll
    for (int k = 0; k < TPT; k++) {
        const int t = tp + TS * k;
        if (t >= tn) break;
        const float4 dg = *(const float4*)(dl + t * DL_LD + rg), du = *(const float4*)(dl + t * DL_LD + rg + 8);
        const float gg[4] = {g[k].x + dg.x, g[k].y + dg.y, g[k].z + dg.z, g[k].w + dg.w};
        const float uu[4] = {u[k].x + du.x, u[k].y + du.y, u[k].z + du.z, u[k].w + du.w};
        uint32_t w[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float lo = gg[2 * i] / (1.0f + __expf(-gg[2 * i])) * uu[2 * i];
            const float hi = gg[2 * i + 1] / (1.0f + __expf(-gg[2 * i + 1])) * uu[2 * i + 1];
            w[i] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
        }
        *(uint2*)(mid + (size_t)(t0 + t) * half + o0 / 2 + j) = uint2{w[0], w[1]};
    }
}

int lora_launch(void* stream, const LoraArgs& a, float* y_add, const float* y_silu, __bf16* mid) {
    const bool silu = mid != nullptr;
    hipStream_t s = (hipStream_t)stream;
    auto go = [&](auto rank, auto wt) {
        constexpr int R = decltype(rank)::value, WT = decltype(wt)::value;
        const dim3 grid((unsigned)((a.rows + WT * 64 - 1) / (WT * 64)), (unsigned)((a.n + LORA_TOK - 1) / LORA_TOK));
        if (silu)
            hipLaunchKernelGGL((lora_silu_kernel<R, WT>), grid, dim3(64 * LORA_WAVES), 0, s, a, y_silu, mid);
        else
            hipLaunchKernelGGL((lora_add_kernel<R, WT>), grid, dim3(64 * LORA_WAVES), 0, s, a, y_add);
    };
    auto by_rank = [&](auto wt) -> bool {
        switch (a.rank) {
            case 8: go(std::integral_constant<int, 8>{}, wt); return true;
            case 16: go(std::integral_constant<int, 16>{}, wt); return true;
            case 32: go(std::integral_constant<int, 32>{}, wt); return true;
            case 64: go(std::integral_constant<int, 64>{}, wt); return true;
            default: return false;
        }
    };
    // decode-sized steps: one tile per wave (4x the workgroups of a launch that would otherwise leave most CUs idle)
    const bool ok = a.n <= LORA_TOK ? by_rank(std::integral_constant<int, 1>{}) : by_rank(std::integral_constant<int, 4>{});
    if (!ok) return fail(QH_EINVAL, "LoRA rank %d: ranks 8, 16, 32 and 64 are served", a.rank);
    if (hipError_t e = hipGetLastError(); e != hipSuccess)
        return fail(QH_EHIP, "lora launch: %s", hipGetErrorString(e));
    return QH_OK;
}

int lora_check(const float* xa, int split, int m_cols, const uint16_t* b, size_t rows, const int32_t* tab,
               const int32_t* tok_slot, const float* slot_scale, size_t n, const void* y, size_t ldy) {
    if (!xa || !b || !tab || !tok_slot || !slot_scale || !y || split < 1)
        return fail(QH_EINVAL, "lora: null or %d splits", split);
    if (m_cols < 1 || m_cols > LORA_COLS_MAX)
        return fail(QH_EINVAL, "lora: %d columns of xa (at most %d)", m_cols, LORA_COLS_MAX);
    if (rows == 0 || rows % 16 || rows > (1u << 30) || n > (1u << 24) || ldy < rows || ldy > (1u << 30) || ldy % 4 ||
        (uintptr_t)b % 16 || (uintptr_t)y % 16)
        return fail(QH_EINVAL,
                    "lora: %zu rows (ld %zu), %zu tokens: rows a multiple of 16, ld of 4, B and y 16-byte aligned", rows,
                    ldy, n);
    return QH_OK;
}

}  // namespace

extern "C" int qh_lora_add(void* stream, const float* xa, int split, int m_cols, const uint16_t* b_f16, int rank,
                           size_t rows, const int32_t* tab, const int32_t* tok_slot, const float* slot_scale, size_t n,
                           float* y, size_t ldy) {
    if (n == 0) return QH_OK;
    if (int e = lora_check(xa, split, m_cols, b_f16, rows, tab, tok_slot, slot_scale, n, y, ldy)) return e;
    const LoraArgs a{xa, split, m_cols, b_f16, rank, (int)rows, tab, tok_slot, slot_scale, (int)n, (int)ldy};
    return lora_launch(stream, a, y, nullptr, nullptr);
}

extern "C" int qh_lora_silu(void* stream, const float* xa, int split, int m_cols, const uint16_t* b_f16, int rank,
                            size_t rows, const int32_t* tab, const int32_t* tok_slot, const float* slot_scale,
                            size_t n, const float* y, size_t ldy, void* mid_bf16) {
    if (n == 0) return QH_OK;
    if (!mid_bf16 || (uintptr_t)mid_bf16 % 8) return fail(QH_EINVAL, "lora silu: null or unaligned output (8 bytes)");
    if (int e = lora_check(xa, split, m_cols, b_f16, rows, tab, tok_slot, slot_scale, n, y, ldy)) return e;
    const LoraArgs a{xa, split, m_cols, b_f16, rank, (int)rows, tab, tok_slot, slot_scale, (int)n, (int)ldy};
    return lora_launch(stream, a, nullptr, y, (__bf16*)mid_bf16);
}

// launch sum_parts_kernel over n4 float4: workgroups of 64 threads for decode-sized rows (one float4 per thread over
// 4x as many CUs), 256 otherwise
static int sum_launch(hipStream_t s, const float* x, int splits, long n4, float* y, float* h) {
    const unsigned t = n4 < 64l * 1024 ? 64 : 256, blocks = (unsigned)std::min<long>((n4 + t - 1) / t, 4096);
    if (t == 64)
        hipLaunchKernelGGL(sum_parts_kernel<16>, dim3(blocks), dim3(t), 0, s, (const float4*)x, splits, n4,
                           (float4*)y, (float4*)h);
    else
        hipLaunchKernelGGL(sum_parts_kernel<8>, dim3(blocks), dim3(t), 0, s, (const float4*)x, splits, n4,
                           (float4*)y, (float4*)h);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_EHIP;
}

extern "C" int qh_sum_parts(void* stream, const float* x, int splits, size_t n, size_t ld, float* y) {
    if (n == 0 || ld == 0) return QH_OK;
    if (!x || !y || splits < 1) return fail(QH_EINVAL, "sum_parts: null or %d splits", splits);
    if (ld % 4 || (uintptr_t)x % 16 || (uintptr_t)y % 16)
        return fail(QH_EINVAL, "sum_parts: rows of %zu floats must be a multiple of 4, buffers 16-byte aligned", ld);
    if (sum_launch((hipStream_t)stream, x, splits, (long)(n * ld / 4), y, nullptr))
        return fail(QH_EHIP, "sum_parts launch failed");
    return QH_OK;
}

extern "C" int qh_add_rmsnorm(void* stream, float* h, const float* x, int splits, size_t n, size_t hidden,
                              const float* w_next, void* y_bf16, float eps) {
    if (n == 0) return QH_OK;
    if (!h || !x || !w_next || !y_bf16 || splits < 1) return fail(QH_EINVAL, "add_rmsnorm: null or %d splits", splits);
    if (hidden == 0 || hidden % 4 || hidden > (1u << 24) || n > 0x7fffffffu || (uintptr_t)h % 16 ||
        (uintptr_t)x % 16 || (uintptr_t)w_next % 16)
        return fail(QH_EINVAL, "add_rmsnorm: hidden %zu must be a multiple of 4, f32 buffers 16-byte aligned", hidden);
    // few tokens (decode): the partials' sum, the bulk of the bytes, over many workgroups first (a workgroup per token
    // would read a 34-split partial set of a 5120-wide row alone, about 20 us), then the norm with no partials left
    const long n4 = (long)(n * hidden / 4);
    if (splits > 1 && (long)n * (hidden / 4) < (long)AR_SPREAD_BELOW) {
        if (sum_launch((hipStream_t)stream, x, splits, n4, nullptr, h)) return fail(QH_EHIP, "add_rmsnorm launch failed");
        // the norm alone, a wide workgroup per token with the row in registers
        if (hidden / 4 <= 1024 * 4)
            hipLaunchKernelGGL((rmsnorm_kernel<1024, 4>), dim3((unsigned)n), dim3(1024), 0, (hipStream_t)stream, h,
                               (int)hidden, w_next, (__bf16*)y_bf16, eps);
        else
            hipLaunchKernelGGL(add_rmsnorm_kernel<1024>, dim3((unsigned)n), dim3(1024), 0, (hipStream_t)stream, h, x,
                               0, (int)n, (int)hidden, w_next, (__bf16*)y_bf16, eps);
    } else {
        hipLaunchKernelGGL(add_rmsnorm_kernel<AR_THREADS>, dim3((unsigned)n), dim3(AR_THREADS), 0, (hipStream_t)stream,
                           h, x, splits, (int)n, (int)hidden, w_next, (__bf16*)y_bf16, eps);
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess)
        return fail(QH_EHIP, "add_rmsnorm launch: %s", hipGetErrorString(e));
    return QH_OK;
}
