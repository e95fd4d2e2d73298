// The quantized-weight matrix products on gfx950 (MI355X): y = W . x for bf16 activations x [m][K] and int4 / int8
// weights W [rows][K] in the tile layout of layout.h, f32 accumulation, on v_mfma_f32_16x16x32_bf16.
//
// Both kernels compute D = X . W^T with the activations as the MFMA A operand (16 tokens x 32 k) and the weights as
// the B operand (32 k x 16 outputs), so the packed tile block is the B operand as loaded. Lane l of a wave holds
// D[token 4 (l / 16) + r][output l % 16], r = 0..3.
//
// skinny_kernel (m <= 16, decode and MTP verify): HBM-bound. The weights are streamed once with 16-byte loads (a wave
// reads each (tile, group) block as one contiguous KiB) and turned into bf16 (128 + q) with one and-or per two values;
// the MFMA sums x (128 + q) exactly in f32 per 128-column group, and the group's scale and zero point are applied
// after it: acc += s (D - (128 + z) sum_k x), where sum_k x comes from one more MFMA against ones per k32 step (shared
// by the wave's tiles). K is split over the waves of a workgroup (reduced through LDS) and, for plain products, over
// the grid (the split-K partials of the output contract).
//
// prefill_kernel (m > 16): MFMA-bound. A workgroup of 4 waves computes 16 * BMB tokens x 128 outputs; the activation
// tile goes through double-buffered, XOR-swizzled LDS in 64-column stages, each wave dequantizes its own 32 outputs'
// weights straight from global memory into bf16 registers ((q - z) s in f32, rounded once), and the workgroups are
// mapped XCD-aware so that those sharing a weight tile run on one XCD's L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "layout.h"

namespace qh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Kernel format F: bit flags of the storage (kernels.h F_*).
enum { EPI_PLAIN = 0, EPI_SILU = 1, EPI_ARGMAX = 2 };

__device__ __forceinline__ f32x4 mfma(u32x4 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
}

// int4 word (layout.h nibble order) -> bf16 (128 + q) of columns 0..7
__device__ __forceinline__ bf16x8 i4_biased(uint32_t w) {
    u32x4 v;
    v.x = (w & 0x000F000Fu) | 0x43004300u;
    v.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
    v.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
    v.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float byte_f(uint32_t w, int b) { return (float)((w >> (8 * b)) & 255u); }

// int8 words (columns 0..3, 4..7; stored q + 128) -> bf16 (128 + q), exact (integers below 256)
__device__ __forceinline__ bf16x8 i8_biased(uint32_t a, uint32_t b) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[i] = (__bf16)byte_f(a, i);
        r[4 + i] = (__bf16)byte_f(b, i);
    }
    return r;
}

// int4 word -> bf16 of (q - z) s = q s + off, in f32 then rounded once
__device__ __forceinline__ bf16x8 i4_scaled(uint32_t w, float s, float off) {
    uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    bf16x8 r;
    r[0] = (__bf16)__builtin_fmaf(byte_f(lo, 0), s, off);
    r[1] = (__bf16)__builtin_fmaf(byte_f(lo, 2), s, off);
    r[2] = (__bf16)__builtin_fmaf(byte_f(hi, 0), s, off);
    r[3] = (__bf16)__builtin_fmaf(byte_f(hi, 2), s, off);
    r[4] = (__bf16)__builtin_fmaf(byte_f(lo, 1), s, off);
    r[5] = (__bf16)__builtin_fmaf(byte_f(lo, 3), s, off);
    r[6] = (__bf16)__builtin_fmaf(byte_f(hi, 1), s, off);
    r[7] = (__bf16)__builtin_fmaf(byte_f(hi, 3), s, off);
    return r;
}

__device__ __forceinline__ bf16x8 i8_scaled(uint32_t a, uint32_t b, float s, float off) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[i] = (__bf16)__builtin_fmaf(byte_f(a, i), s, off);
        r[4 + i] = (__bf16)__builtin_fmaf(byte_f(b, i), s, off);
    }
    return r;
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

// Words of a (tile, group) code block per lane (16 bytes each).
template <int F>
struct CodeWords {
    static constexpr int N = (F & F_I8) ? 2 : 1;
};

template <int F>
__device__ __forceinline__ float scale_of(const void* scales, size_t blk, int r) {
    if (F & F_S32) return ((const float*)scales)[blk * TILE + r];
    return bf16_bits_f(((const uint16_t*)scales)[blk * TILE + r]);
}

template <int F>
__device__ __forceinline__ int zero_of(const uint64_t* zeros, size_t blk, int r) {
    if (F & F_ZP) return (int)((zeros[blk] >> (4 * r)) & 15u);
    return (F & F_I8) ? 128 : 8;
}

// ---------------------------------------------------------------------------------------------------------------
// skinny_kernel

template <int F, int T>
struct SkinnyFrag {
    u32x4 c[T][CodeWords<F>::N];
    float s[T];
    float cz[T];  // 128 + zero point
    u32x4 xa[4];
};

template <int F, int EPI, int NR, int T>
__global__ __launch_bounds__(1024) void skinny_kernel(Launch a) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int l16 = lane & 15, kq = lane >> 4;
    const int tiles = a.rows / TILE, G = a.cols / QG, S = a.split, M = a.m;
    const int tile0 = blockIdx.x * T, sp = blockIdx.y;
    const int gs0 = (int)((long)sp * G / S), gs1 = (int)((long)(sp + 1) * G / S);
    const int g0 = gs0 + wave * (gs1 - gs0) / W, g1 = gs0 + (wave + 1) * (gs1 - gs0) / W;

    // this lane's x row (A operand: token l16, columns 8 kq .. 8 kq + 7 of each k32 step)
    const __bf16* xr = nullptr;
    if (l16 < M) xr = (const __bf16*)a.x + (size_t)(a.xrows ? a.xrows[l16] : l16) * a.ldx + 8 * kq;
    size_t tb[T];
#pragma unroll
    for (int t = 0; t < T; t++) tb[t] = (size_t)min(tile0 + t, tiles - 1) * G;

    auto load = [&](int g, SkinnyFrag<F, T>& f) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            size_t blk = tb[t] + g;
            const u32x4* cp = (const u32x4*)a.codes + blk * 64 * CodeWords<F>::N;
#pragma unroll
            for (int h = 0; h < CodeWords<F>::N; h++) f.c[t][h] = __builtin_nontemporal_load(cp + h * 64 + lane);
            f.s[t] = scale_of<F>(a.scales, blk, l16);
            f.cz[t] = (float)(128 + ((F & F_I8) ? 0 : zero_of<F>(a.zeros, blk, l16)));
        }
#pragma unroll
        for (int j = 0; j < 4; j++) f.xa[j] = xr ? *(const u32x4*)(xr + (size_t)g * QG + 32 * j) : u32x4{0, 0, 0, 0};
    };

    float acc[T][NR];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < NR; r++) acc[t][r] = 0.0f;

    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    if (g0 < g1) {
        SkinnyFrag<F, T> cur, nxt;
        load(g0, cur);
        for (int g = g0; g < g1; g++) {
            load(min(g + 1, g1 - 1), nxt);
            f32x4 xs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) xs = mfma(cur.xa[j], ones, xs);
#pragma unroll
            for (int t = 0; t < T; t++) {
                f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    bf16x8 b;
                    if (F & F_I8)
                        b = i8_biased(cur.c[t][j >> 1][2 * (j & 1)], cur.c[t][j >> 1][2 * (j & 1) + 1]);
                    else
                        b = i4_biased(cur.c[t][0][j]);
                    d = mfma(cur.xa[j], b, d);
                }
#pragma unroll
                for (int r = 0; r < NR; r++) acc[t][r] += cur.s[t] * (d[r] - cur.cz[t] * xs[r]);
            }
            cur = nxt;
        }
    }

    // reduce the waves' K ranges into wave 0
    if (W > 1) {
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int r = 0; r < NR; r++) red[(((wave - 1) * T + t) * NR + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        if (wave > 0) return;
        for (int w = 1; w < W; w++)
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int r = 0; r < NR; r++) acc[t][r] += red[(((w - 1) * T + t) * NR + r) * 64 + lane];
    }

    unsigned long long key[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) key[r] = 0;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int tile = tile0 + t;
        if (tile >= tiles) break;
        const int out = tile * TILE + l16;
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int tok = 4 * kq + r;
            const float v = acc[t][r];
            if (EPI == EPI_SILU) {
                const float up = __shfl_xor(v, 8);
                if (l16 < 8 && tok < M) ((__bf16*)a.y)[(size_t)tok * a.ldy + tile * 8 + l16] = (__bf16)(silu(v) * up);
            } else {
                if (tok < M) ((float*)a.y)[((size_t)sp * M + tok) * a.ldy + out] = v;
                if (EPI == EPI_ARGMAX && tok < M && out < a.valid) key[r] = max_u64(key[r], argmax_key(v, out));
            }
        }
    }
    if (EPI == EPI_ARGMAX) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const unsigned long long k = group16_max(key[r]);
            const int tok = 4 * kq + r;
            if (l16 == 0 && tok < M && k) atomicMax(a.keys + tok, k);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// prefill_kernel

constexpr int PF_WAVES = 4;
constexpr int PF_TILES_PER_WAVE = 2;
constexpr int PF_TILES = PF_WAVES * PF_TILES_PER_WAVE;  // 128 outputs per workgroup
constexpr int PF_BK = 64;                               // columns per LDS stage (half a group)
constexpr int PF_ROW = PF_BK * 2;                       // LDS bytes per token row of a stage

// LDS byte offset of 16-byte chunk kc (0..7) of token row `row` in a stage: XOR-swizzled so that the 16 lanes of a
// row group (16 tokens, one chunk) hit all 64 banks once.
__device__ __forceinline__ int pf_lds_off(int row, int kc) { return row * PF_ROW + 16 * (kc ^ ((row >> 1) & 7)); }

template <int F, int EPI, int BMB>
__global__ __launch_bounds__(256) void prefill_kernel(Launch a) {
    constexpr int BM = 16 * BMB;
    constexpr int CPT = BM * (PF_ROW / 16) / 256;  // 16-byte x chunks each thread stages per stage
    constexpr int CW = CodeWords<F>::N;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][BM * PF_ROW];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
    const int l16 = lane & 15, kq = lane >> 4;
    const int tiles = a.rows / TILE, G = a.cols / QG, M = a.m;

    // XCD-aware order: workgroup b runs on XCD b % 8; give each XCD a contiguous run of work items, token tiles
    // fastest, so the workgroups sharing a weight tile share that XCD's L2.
    const int nb = gridDim.x, b = blockIdx.x, xcd = b & 7, q8 = nb >> 3, r8 = nb & 7;
    const int item = xcd * q8 + min(xcd, r8) + (b >> 3);
    const int ntok = (M + BM - 1) / BM;
    const int tok0 = (item % ntok) * BM, otile = (item / ntok) * PF_TILES + wave * PF_TILES_PER_WAVE;

    // staging of the activation tile: chunk c = tid + 256 i -> row c / 8, column chunk c % 8
    const __bf16* xsrc[CPT];
    int xoff[CPT];
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int c = tid + 256 * i, row = c >> 3, kc = c & 7;
        const int tok = min(tok0 + row, M - 1);
        xsrc[i] = (const __bf16*)a.x + (size_t)(a.xrows ? a.xrows[tok] : tok) * a.ldx + 8 * kc;
        xoff[i] = pf_lds_off(row, kc);
    }
    auto stage_load = [&](int s, u32x4 (&v)[CPT]) {
#pragma unroll
        for (int i = 0; i < CPT; i++) v[i] = *(const u32x4*)(xsrc[i] + (size_t)s * PF_BK);
    };
    auto stage_store = [&](int buf, const u32x4 (&v)[CPT]) {
#pragma unroll
        for (int i = 0; i < CPT; i++) *(u32x4*)(&lds[buf][xoff[i]]) = v[i];
    };

    size_t tb[PF_TILES_PER_WAVE];
#pragma unroll
    for (int t = 0; t < PF_TILES_PER_WAVE; t++) tb[t] = (size_t)min(otile + t, tiles - 1) * G;
    struct WFrag {
        u32x4 c[PF_TILES_PER_WAVE][CW];
        float s[PF_TILES_PER_WAVE], off[PF_TILES_PER_WAVE];
    };
    auto wload = [&](int g, WFrag& f) {
#pragma unroll
        for (int t = 0; t < PF_TILES_PER_WAVE; t++) {
            const size_t blk = tb[t] + g;
            const u32x4* cp = (const u32x4*)a.codes + blk * 64 * CW;
#pragma unroll
            for (int h = 0; h < CW; h++) f.c[t][h] = cp[h * 64 + lane];
            if (F & F_PERCH) {
                f.s[t] = 1.0f;  // exact integers q = stored - 128; the row scale comes after the sum
                f.off[t] = -128.0f;
            } else {
                f.s[t] = scale_of<F>(a.scales, blk, l16);
                f.off[t] = -(float)zero_of<F>(a.zeros, blk, l16) * f.s[t];
            }
        }
    };

    f32x4 acc[BMB][PF_TILES_PER_WAVE];
#pragma unroll
    for (int bb = 0; bb < BMB; bb++)
#pragma unroll
        for (int t = 0; t < PF_TILES_PER_WAVE; t++) acc[bb][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int stages = 2 * G;
    u32x4 xv[CPT];
    WFrag wcur, wnxt;
    stage_load(0, xv);
    wload(0, wcur);
    stage_store(0, xv);
    __syncthreads();
    for (int s = 0; s < stages; s++) {
        const bool more = s + 1 < stages;
        if (more) stage_load(s + 1, xv);
        if (s & 1) wload(min(s / 2 + 1, G - 1), wnxt);
        const uint8_t* buf = lds[s & 1];
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            const int j = 2 * (s & 1) + jj;  // k32 step within the group
            bf16x8 bw[PF_TILES_PER_WAVE];
#pragma unroll
            for (int t = 0; t < PF_TILES_PER_WAVE; t++) {
                if (F & F_I8)
                    bw[t] = i8_scaled(wcur.c[t][j >> 1][2 * (j & 1)], wcur.c[t][j >> 1][2 * (j & 1) + 1], wcur.s[t],
                                      wcur.off[t]);
                else
                    bw[t] = i4_scaled(wcur.c[t][0][j], wcur.s[t], wcur.off[t]);
            }
#pragma unroll
            for (int bb = 0; bb < BMB; bb++) {
                const u32x4 xa = *(const u32x4*)(buf + pf_lds_off(16 * bb + l16, 4 * jj + kq));
#pragma unroll
                for (int t = 0; t < PF_TILES_PER_WAVE; t++) acc[bb][t] = mfma(xa, bw[t], acc[bb][t]);
            }
        }
        if (more) stage_store((s + 1) & 1, xv);
        __syncthreads();
        if (s & 1) wcur = wnxt;
    }

    // epilogue: acc[bb][t][r] = D[token tok0 + 16 bb + 4 kq + r][output 16 (otile + t) + l16]
    float rs[PF_TILES_PER_WAVE];
#pragma unroll
    for (int t = 0; t < PF_TILES_PER_WAVE; t++) rs[t] = (F & F_PERCH) ? scale_of<F>(a.scales, tb[t], l16) : 1.0f;
#pragma unroll
    for (int bb = 0; bb < BMB; bb++) {
        unsigned long long key[4] = {0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < PF_TILES_PER_WAVE; t++) {
            const int tile = otile + t;
            if (tile >= tiles) break;
            const int out = tile * TILE + l16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tok = tok0 + 16 * bb + 4 * kq + r;
                const float v = (F & F_PERCH) ? acc[bb][t][r] * rs[t] : acc[bb][t][r];
                if (EPI == EPI_SILU) {
                    const float up = __shfl_xor(v, 8);
                    if (l16 < 8 && tok < M)
                        ((__bf16*)a.y)[(size_t)tok * a.ldy + tile * 8 + l16] = (__bf16)(silu(v) * up);
                } else {
                    if (tok < M) ((float*)a.y)[(size_t)tok * a.ldy + out] = v;
                    if (EPI == EPI_ARGMAX && tok < M && out < a.valid) key[r] = max_u64(key[r], argmax_key(v, out));
                }
            }
        }
        if (EPI == EPI_ARGMAX) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const unsigned long long k = group16_max(key[r]);
                const int tok = tok0 + 16 * bb + 4 * kq + r;
                if (l16 == 0 && tok < M && k) atomicMax(a.keys + tok, k);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// launchers

template <int F, int EPI, int NR>
static hipError_t skinny_nr(const Launch& l) {
    const int tiles = l.rows / TILE;
    dim3 grid((tiles + SKINNY_TILES - 1) / SKINNY_TILES, l.split);
    size_t lds = (size_t)(l.waves - 1) * SKINNY_TILES * NR * 64 * sizeof(float);
    hipLaunchKernelGGL((skinny_kernel<F, EPI, NR, SKINNY_TILES>), grid, dim3(64 * l.waves), lds, l.stream, l);
    return hipGetLastError();
}

template <int F, int EPI>
static hipError_t skinny_epi(const Launch& l) {
    switch (l.m) {
        case 1: return skinny_nr<F, EPI, 1>(l);
        case 2: return skinny_nr<F, EPI, 2>(l);
        case 3: return skinny_nr<F, EPI, 3>(l);
        default: return skinny_nr<F, EPI, 4>(l);
    }
}

template <int F, int EPI, int BMB>
static hipError_t prefill_bm(const Launch& l) {
    const int tiles = l.rows / TILE;
    const int items = ((tiles + PF_TILES - 1) / PF_TILES) * ((l.m + 16 * BMB - 1) / (16 * BMB));
    hipLaunchKernelGGL((prefill_kernel<F, EPI, BMB>), dim3(items), dim3(256), 0, l.stream, l);
    return hipGetLastError();
}

template <int F, int EPI>
static hipError_t launch_epi(const Launch& l) {
    if (l.m <= SKINNY_MAX_M) return skinny_epi<F & ~F_PERCH, EPI>(l);
    return l.m > 128 ? prefill_bm<F, EPI, 16>(l) : prefill_bm<F, EPI, 4>(l);
}

template <int F>
static hipError_t launch_fmt(const Launch& l) {
    switch (l.epi) {
        case EPI_SILU: return launch_epi<F, EPI_SILU>(l);
        case EPI_ARGMAX: return launch_epi<F, EPI_ARGMAX>(l);
        default: return launch_epi<F, EPI_PLAIN>(l);
    }
}

hipError_t launch(const Launch& l) {
    switch (l.fmt) {
        case F_I4: return launch_fmt<F_I4>(l);
        case F_I4 | F_S32: return launch_fmt<F_I4 | F_S32>(l);
        case F_ZP: return launch_fmt<F_ZP>(l);
        case F_ZP | F_S32: return launch_fmt<F_ZP | F_S32>(l);
        case F_I8 | F_S32: return launch_fmt<F_I8 | F_S32>(l);
        case F_I8 | F_S32 | F_PERCH: return launch_fmt<F_I8 | F_S32 | F_PERCH>(l);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qh
