// Consumers of the plain products' split-K partials (the output contract y [split][n][ld] f32): the reference's
// sum_parts (kernels/qwen.cu:141-143, part_sum kernels/common.cuh:66-70) and add_rmsnorm (kernels/qwen.cu:57-80),
// the residual step after the o_proj / out_proj / down products. HBM-bound; f32 sums in the reference's order
// (h + x[0], then x[1], x[2], ..), so the sums are bit-identical to it.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"

using namespace qh;

namespace {

// y [n][ld] = sum over s of x [s][n][ld]; one thread per 4 columns (ld % 4 == 0), grid-stride over n * ld / 4
__global__ __launch_bounds__(256) void sum_parts_kernel(const float4* __restrict__ x, int splits, long n4, float4* y) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int s = 0; s < splits; s++) {
            const float4 p = x[(size_t)s * n4 + i];
            v.x += p.x, v.y += p.y, v.z += p.z, v.w += p.w;
        }
        y[i] = v;
    }
}

constexpr int AR_THREADS = 256;

// token t (one workgroup): h[t] += the sum of the partials x[.][t]; y[t] = bf16(w * (h[t] / rms(h[t])))
__global__ __launch_bounds__(AR_THREADS) void add_rmsnorm_kernel(float* __restrict__ h, const float* __restrict__ x,
                                                                 int splits, int n, int H, const float* __restrict__ w,
                                                                 __bf16* __restrict__ y, float eps) {
    __shared__ float wsum[AR_THREADS / 64];
    const size_t base = (size_t)blockIdx.x * H;
    const int H4 = H / 4;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < H4; c += AR_THREADS) {
        float4 v = ((const float4*)(h + base))[c];
        for (int s = 0; s < splits; s++) {
            const float4 p = ((const float4*)(x + (size_t)s * n * H + base))[c];
            v.x += p.x, v.y += p.y, v.z += p.z, v.w += p.w;
        }
        ((float4*)(h + base))[c] = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < AR_THREADS / 64; i++) tot += wsum[i];
    const float r = rsqrtf(tot / (float)H + eps);
    // the second pass re-reads this workgroup's own h row (written above by the same threads, same columns)
    for (int c = threadIdx.x; c < H4; c += AR_THREADS) {
        const float4 v = ((const float4*)(h + base))[c], wn = ((const float4*)w)[c];
        __bf16* yo = y + base + 4 * c;
        yo[0] = (__bf16)(wn.x * (v.x * r));
        yo[1] = (__bf16)(wn.y * (v.y * r));
        yo[2] = (__bf16)(wn.z * (v.z * r));
        yo[3] = (__bf16)(wn.w * (v.w * r));
    }
}

}  // namespace

extern "C" int qh_sum_parts(void* stream, const float* x, int splits, size_t n, size_t ld, float* y) {
    if (n == 0 || ld == 0) return QH_OK;
    if (!x || !y || splits < 1) return fail(QH_EINVAL, "sum_parts: null or %d splits", splits);
    if (ld % 4 || (uintptr_t)x % 16 || (uintptr_t)y % 16)
        return fail(QH_EINVAL, "sum_parts: rows of %zu floats must be a multiple of 4, buffers 16-byte aligned", ld);
    const long n4 = (long)(n * ld / 4);
    const unsigned blocks = (unsigned)std::min<long>((n4 + 255) / 256, 4096);
    hipLaunchKernelGGL(sum_parts_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const float4*)x, splits, n4,
                       (float4*)y);
    if (hipError_t e = hipGetLastError(); e != hipSuccess)
        return fail(QH_EHIP, "sum_parts launch: %s", hipGetErrorString(e));
    return QH_OK;
}

extern "C" int qh_add_rmsnorm(void* stream, float* h, const float* x, int splits, size_t n, size_t hidden,
                              const float* w_next, void* y_bf16, float eps) {
    if (n == 0) return QH_OK;
    if (!h || !x || !w_next || !y_bf16 || splits < 1) return fail(QH_EINVAL, "add_rmsnorm: null or %d splits", splits);
    if (hidden == 0 || hidden % 4 || hidden > (1u << 24) || n > 0x7fffffffu || (uintptr_t)h % 16 ||
        (uintptr_t)x % 16 || (uintptr_t)w_next % 16)
        return fail(QH_EINVAL, "add_rmsnorm: hidden %zu must be a multiple of 4, f32 buffers 16-byte aligned", hidden);
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)n), dim3(AR_THREADS), 0, (hipStream_t)stream, h, x, splits,
                       (int)n, (int)hidden, w_next, (__bf16*)y_bf16, eps);
    if (hipError_t e = hipGetLastError(); e != hipSuccess)
        return fail(QH_EHIP, "add_rmsnorm launch: %s", hipGetErrorString(e));
    return QH_OK;
}
