// Consumers of the plain products' split-K partials (the output contract y [split][n][ld] f32): the reference's
// sum_parts (kernels/qwen.cu:141-143, part_sum kernels/common.cuh:66-70) and add_rmsnorm (kernels/qwen.cu:57-80),
// the residual step after the o_proj / out_proj / down products, and the LoRA epilogue (kernels/lora.cuh) that adds an
// unmerged adapter's delta to them. HBM-bound; f32 sums in the reference's order (h + x[0], then x[1], x[2], ..), so
// the sums are bit-identical to it.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"

using namespace qh;

namespace {

// v += x[0][i] + x[1][i] + .. + x[splits - 1][i], in that order; the partials load 8 at a time ahead of their adds
// (the sum of 34 partials of a decode product is then 5 memory round trips, not 34)
__device__ __forceinline__ void add_splits(float4& v, const float4* __restrict__ x, int splits, long n4, long i) {
    constexpr int B = 8;
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
__global__ __launch_bounds__(256) void sum_parts_kernel(const float4* __restrict__ x, int splits, long n4, float4* y,
                                                        float4* h) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x) {
        float4 v = h ? h[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        add_splits(v, x, splits, n4, i);
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
// LoRA consumers (kernels/lora.cuh:52-113, launched by src/cuda/qwen/lora.rs:143-190): an unmerged adapter adds
// s_t B (A x) to a plain product for the tokens t of the slots that use it. A x arrives as the split-K partials xa
// [split][n][M] of the stacked A product (M = adapted modules x rank, at most 256 columns); B is f16 [rows][R] in the
// product's row order; tab (8 ints) holds each module's end row (ascending; unused INT_MAX), then its first column of
// xa (-1: not adapted). A workgroup takes LORA_TT tokens and 256 rows (add) or 256 SwiGLU outputs (silu): the tokens'
// scales and their xa (the partials summed in split order) are staged in LDS once, each thread reads its B row as
// 16-byte loads and dots it with the staged xa in f32, in column order.

constexpr int LORA_TT = 8;
constexpr int LORA_MAXM = 256;

struct LoraArgs {
    const float* xa;
    int split, M;
    const uint16_t* b;
    int rows;
    const int* tab;
    const int* tok_slot;
    const float* slot_scale;
    int n;
    int ldy;
};

// the block's token scales (0 past n) and, for the tokens with a nonzero scale, xa summed over the splits
__device__ void lora_stage(const LoraArgs& a, int t0, float (*xs)[LORA_MAXM], float* sc) {
    if (threadIdx.x < LORA_TT) {
        const int t = t0 + threadIdx.x;
        sc[threadIdx.x] = t < a.n ? a.slot_scale[a.tok_slot[t]] : 0.0f;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < LORA_TT * a.M; i += blockDim.x) {
        const int tl = i / a.M, c = i - tl * a.M, t = t0 + tl;
        float v = 0.0f;
        if (sc[tl] != 0.0f)
            for (int s = 0; s < a.split; s++) v += a.xa[((size_t)s * a.n + t) * a.M + c];
        xs[tl][c] = v;
    }
    __syncthreads();
}

// B row o (f16 [R]) as f32
template <int R>
__device__ __forceinline__ void lora_b_row(const uint16_t* b, int o, float (&w)[R]) {
    const uint4* p = (const uint4*)(b + (size_t)o * R);
#pragma unroll
    for (int i = 0; i < R / 8; i++) {
        const uint4 u = p[i];
        const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            w[8 * i + 2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(h[k] & 0xffffu));
            w[8 * i + 2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(h[k] >> 16));
        }
    }
}

template <int R>
__device__ __forceinline__ float lora_dot(const float (&w)[R], const float* x) {
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < R; j++) d = __builtin_fmaf(w[j], x[j], d);
    return d;
}

// y [n][ldy] (a plain product's split 0) row o += s_t B[o] . xa[t][off(o) ..] for the adapter tokens
template <int R>
__global__ __launch_bounds__(256) void lora_add_kernel(LoraArgs a, float* __restrict__ y) {
    __shared__ float xs[LORA_TT][LORA_MAXM];
    __shared__ float sc[LORA_TT];
    const int t0 = blockIdx.y * LORA_TT;
    lora_stage(a, t0, xs, sc);
    bool any = false;
#pragma unroll
    for (int i = 0; i < LORA_TT; i++) any |= sc[i] != 0.0f;
    const int o = blockIdx.x * 256 + threadIdx.x;
    if (!any || o >= a.rows) return;
    const int mod = (o >= a.tab[0]) + (o >= a.tab[1]) + (o >= a.tab[2]), off = a.tab[4 + mod];
    if (off < 0) return;
    float w[R];
    lora_b_row<R>(a.b, o, w);
#pragma unroll
    for (int tl = 0; tl < LORA_TT; tl++)
        if (sc[tl] != 0.0f) {
            float* yo = y + (size_t)(t0 + tl) * a.ldy + o;
            *yo = __builtin_fmaf(sc[tl], lora_dot<R>(w, &xs[tl][off]), *yo);
        }
}

// mid [n][rows / 2] (bf16) = SwiGLU of the plain [gate; up] product y [n][ldy] (split 1, packed in the SwiGLU
// epilogue's row order: 16-row tile p holds gate rows 8p .. 8p + 7, then their up rows) with the delta added first
template <int R>
__global__ __launch_bounds__(256) void lora_silu_kernel(LoraArgs a, const float* __restrict__ y, __bf16* mid) {
    __shared__ float xs[LORA_TT][LORA_MAXM];
    __shared__ float sc[LORA_TT];
    const int t0 = blockIdx.y * LORA_TT;
    lora_stage(a, t0, xs, sc);
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= a.rows / 2) return;
    const int og = 16 * (j / 8) + j % 8, ou = og + 8, offg = a.tab[4], offu = a.tab[5];
    float wg[R], wu[R];
    if (offg >= 0) lora_b_row<R>(a.b, og, wg);
    if (offu >= 0) lora_b_row<R>(a.b, ou, wu);
    for (int tl = 0; tl < LORA_TT && t0 + tl < a.n; tl++) {
        const size_t r = (size_t)(t0 + tl) * a.ldy;
        float g = y[r + og], u = y[r + ou];
        if (sc[tl] != 0.0f) {
            if (offg >= 0) g = __builtin_fmaf(sc[tl], lora_dot<R>(wg, &xs[tl][offg]), g);
            if (offu >= 0) u = __builtin_fmaf(sc[tl], lora_dot<R>(wu, &xs[tl][offu]), u);
        }
        mid[(size_t)(t0 + tl) * (a.rows / 2) + j] = (__bf16)(g / (1.0f + __expf(-g)) * u);
    }
}

int lora_launch(void* stream, const LoraArgs& a, int rank, float* y_add, const float* y_silu, __bf16* mid) {
    const bool silu = mid != nullptr;
    const unsigned per = 256, outs = (unsigned)(silu ? a.rows / 2 : a.rows);
    const dim3 grid((outs + per - 1) / per, (unsigned)((a.n + LORA_TT - 1) / LORA_TT));
    hipStream_t s = (hipStream_t)stream;
#define QH_LORA_CASE(R)                                                                      \
    case R:                                                                                  \
        if (silu)                                                                            \
            hipLaunchKernelGGL(lora_silu_kernel<R>, grid, dim3(256), 0, s, a, y_silu, mid);  \
        else                                                                                 \
            hipLaunchKernelGGL(lora_add_kernel<R>, grid, dim3(256), 0, s, a, y_add);         \
        break;
    switch (rank) {
        QH_LORA_CASE(8)
        QH_LORA_CASE(16)
        QH_LORA_CASE(32)
        QH_LORA_CASE(64)
        default: return fail(QH_EINVAL, "LoRA rank %d: ranks 8, 16, 32 and 64 are served", rank);
    }
#undef QH_LORA_CASE
    if (hipError_t e = hipGetLastError(); e != hipSuccess)
        return fail(QH_EHIP, "lora launch: %s", hipGetErrorString(e));
    return QH_OK;
}

int lora_check(const float* xa, int split, int m_cols, const uint16_t* b, size_t rows, const int32_t* tab,
               const int32_t* tok_slot, const float* slot_scale, size_t n, const void* y, size_t ldy, bool silu) {
    if (!xa || !b || !tab || !tok_slot || !slot_scale || !y || split < 1)
        return fail(QH_EINVAL, "lora: null or %d splits", split);
    if (m_cols < 1 || m_cols > LORA_MAXM)
        return fail(QH_EINVAL, "lora: %d columns of xa (at most %d)", m_cols, LORA_MAXM);
    if (rows == 0 || rows > (1u << 30) || n > (1u << 24) || ldy < rows || ldy > (1u << 30) || (uintptr_t)b % 16 ||
        (silu && rows % 16))
        return fail(QH_EINVAL, "lora: %zu rows (ld %zu), %zu tokens, B 16-byte aligned%s", rows, ldy, n,
                    silu ? ", rows a multiple of 16" : "");
    return QH_OK;
}

}  // namespace

extern "C" int qh_lora_add(void* stream, const float* xa, int split, int m_cols, const uint16_t* b_f16, int rank,
                           size_t rows, const int32_t* tab, const int32_t* tok_slot, const float* slot_scale, size_t n,
                           float* y, size_t ldy) {
    if (n == 0) return QH_OK;
    if (int e = lora_check(xa, split, m_cols, b_f16, rows, tab, tok_slot, slot_scale, n, y, ldy, false)) return e;
    const LoraArgs a{xa, split, m_cols, b_f16, (int)rows, tab, tok_slot, slot_scale, (int)n, (int)ldy};
    return lora_launch(stream, a, rank, y, nullptr, nullptr);
}

extern "C" int qh_lora_silu(void* stream, const float* xa, int split, int m_cols, const uint16_t* b_f16, int rank,
                            size_t rows, const int32_t* tab, const int32_t* tok_slot, const float* slot_scale,
                            size_t n, const float* y, size_t ldy, void* mid_bf16) {
    if (n == 0) return QH_OK;
    if (!mid_bf16) return fail(QH_EINVAL, "lora silu: null output");
    if (int e = lora_check(xa, split, m_cols, b_f16, rows, tab, tok_slot, slot_scale, n, y, ldy, true)) return e;
    const LoraArgs a{xa, split, m_cols, b_f16, (int)rows, tab, tok_slot, slot_scale, (int)n, (int)ldy};
    return lora_launch(stream, a, rank, nullptr, y, (__bf16*)mid_bf16);
}

// launch sum_parts_kernel over n4 float4: workgroups of 64 threads for decode-sized rows (one float4 per thread over
// 4x as many CUs), 256 otherwise
static int sum_launch(hipStream_t s, const float* x, int splits, long n4, float* y, float* h) {
    const unsigned t = n4 < 64l * 1024 ? 64 : 256, blocks = (unsigned)std::min<long>((n4 + t - 1) / t, 4096);
    hipLaunchKernelGGL(sum_parts_kernel, dim3(blocks), dim3(t), 0, s, (const float4*)x, splits, n4, (float4*)y,
                       (float4*)h);
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
