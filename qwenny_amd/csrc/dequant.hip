// The trainer's dequantization (kernels/qwen_train.cu:84-103, called from src/cuda/qwen/train.rs:490-520): rows
// r0 .. r0 + n of a quantized matrix in the checkpoint's own layout (not the product kernels' tile layout) written as
// dense rows, w = (q - zero) * scale in f32, then bf16 (round to nearest even) or f32. The trainer multiplies the dense
// rows with a library GEMM (hipBLASLt here, cuBLAS in the reference).
//
// Layout read: q [rows][words] u32, value c of a row in word c * bits / 32 from the low bits up; scales f32 and zero
// points u8 per (row, group of `group` columns). HBM-bound byte work: each thread reads 16 bytes of words (4 words;
// one when a row's words are not a multiple of 4) and writes their values with 16-byte stores, consecutive threads
// covering consecutive memory.
#include <hip/hip_runtime.h>

#include "internal.h"

using namespace qh;

namespace {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

template <int BITS, int VW, bool F32>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ q, const float* __restrict__ sc,
                                                       const uint8_t* __restrict__ zp, int words, int cols, int group,
                                                       int r0, long chunks, void* __restrict__ out) {
    constexpr int PER = 32 / BITS;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= chunks) return;
    const int cpr = words / VW;  // chunks per row
    const int rr = (int)(i / cpr), w0 = (int)(i - (long)rr * cpr) * VW, r = r0 + rr;
    uint32_t v[VW];
    if (VW == 4) {
        const u32x4v x = *(const u32x4v*)(q + (size_t)r * words + w0);
        v[0] = x.x, v[1] = x.y, v[VW > 2 ? 2 : 0] = x.z, v[VW > 3 ? 3 : 0] = x.w;
    } else {
        v[0] = q[(size_t)r * words + w0];
    }
    const int groups = cols / group;
#pragma unroll
    for (int k = 0; k < VW; k++) {
        const int c0 = (w0 + k) * PER;  // a word's values share one group (group % PER == 0)
        const size_t gi = (size_t)r * groups + c0 / group;
        const float s = sc[gi], z = (float)zp[gi];
        float f[PER];
#pragma unroll
        for (int e = 0; e < PER; e++) f[e] = ((float)((v[k] >> (e * BITS)) & ((1u << BITS) - 1u)) - z) * s;
        const size_t o = (size_t)rr * cols + c0;
        if (F32) {
#pragma unroll
            for (int e = 0; e < PER; e += 4)
                *(float4*)((float*)out + o + e) = make_float4(f[e], f[e + 1], f[e + 2], f[e + 3]);
        } else {
            uint32_t b[PER / 2];
#pragma unroll
            for (int e = 0; e < PER; e += 2) {
                const __bf16 lo = (__bf16)f[e], hi = (__bf16)f[e + 1];  // round to nearest even
                b[e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
            }
            if (PER == 8)
                *(u32x4v*)((uint16_t*)out + o) = u32x4v{b[0], b[1], b[PER / 2 > 2 ? 2 : 0], b[PER / 2 > 3 ? 3 : 0]};
            else
                *(uint2*)((uint16_t*)out + o) = make_uint2(b[0], b[1]);
        }
    }
}

template <int BITS, bool F32>
hipError_t launch_bits(hipStream_t s, const uint32_t* q, const float* sc, const uint8_t* zp, int words, int cols,
                       int group, int r0, size_t n, void* out) {
    const int vw = words % 4 == 0 ? 4 : 1;
    const long chunks = (long)n * (words / vw);
    const unsigned blocks = (unsigned)((chunks + 255) / 256);
    if (vw == 4)
        hipLaunchKernelGGL((dequant_kernel<BITS, 4, F32>), dim3(blocks), dim3(256), 0, s, q, sc, zp, words, cols,
                           group, r0, chunks, out);
    else
        hipLaunchKernelGGL((dequant_kernel<BITS, 1, F32>), dim3(blocks), dim3(256), 0, s, q, sc, zp, words, cols,
                           group, r0, chunks, out);
    return hipGetLastError();
}

}  // namespace

extern "C" int qh_dequant(void* stream, const uint32_t* q, const float* scales, const uint8_t* zeros, size_t rows,
                          size_t words, size_t cols, int group, int bits, size_t r0, size_t n, void* out,
                          int out_f32) {
    if (n == 0) return QH_OK;
    if (!q || !scales || !zeros || !out) return fail(QH_EINVAL, "dequant: null");
    if (bits != 4 && bits != 8) return fail(QH_EINVAL, "dequant: %d bits", bits);
    const size_t per = 32 / (size_t)bits;
    if (words * per != cols || group <= 0 || group % (int)per || cols % (size_t)group)
        return fail(QH_EINVAL, "dequant: %zu words for %zu columns in groups of %d", words, cols, group);
    if (r0 + n > rows || rows > (1u << 30) || cols > (1u << 24))
        return fail(QH_EINVAL, "dequant: rows %zu..%zu of %zu", r0, r0 + n, rows);
    if ((uintptr_t)q % 16 || (uintptr_t)out % 16)
        return fail(QH_EINVAL, "dequant: q and out must be 16-byte aligned");
    const hipStream_t s = (hipStream_t)stream;
    const int w = (int)words, c = (int)cols, r = (int)r0;
    hipError_t e;
    if (bits == 4)
        e = out_f32 ? launch_bits<4, true>(s, q, scales, zeros, w, c, group, r, n, out)
                    : launch_bits<4, false>(s, q, scales, zeros, w, c, group, r, n, out);
    else
        e = out_f32 ? launch_bits<8, true>(s, q, scales, zeros, w, c, group, r, n, out)
                    : launch_bits<8, false>(s, q, scales, zeros, w, c, group, r, n, out);
    if (e != hipSuccess) return fail(QH_EHIP, "dequant launch: %s", hipGetErrorString(e));
    return QH_OK;
}
