// The trainer's dequantization (kernels/qwen_train.cu:84-103, called from src/cuda/qwen/train.rs:490-520): rows
// r0 .. r0 + n of a quantized matrix in the checkpoint's own layout (not the product kernels' tile layout) written as
// dense rows, w = (q - zero) * scale in f32, then bf16 (round to nearest even) or f32. The trainer multiplies the dense
// rows with a library GEMM (hipBLASLt here, cuBLAS in the reference).
//
// Layout read: q [rows][words] u32, value c of a row in word c * bits / 32 from the low bits up; scales f32 and zero
// points u8 per (row, group of `group` columns). HBM-bound byte work over the range's words as one flat array
// (non-temporal loads and stores: the rows are streamed once).
#include <hip/hip_runtime.h>

#include "internal.h"

using namespace qh;

namespace {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

// Words per workgroup: 4 per thread, at a stride of 256 so that every load and store instruction of a wave covers one
// contiguous span.
constexpr int DQ_WORDS = 1024;

template <int BITS, bool F32>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ q, const float* __restrict__ sc,
                                                       const uint8_t* __restrict__ zp, long total, int group,
                                                       void* __restrict__ out) {
    // q, sc, zp and out start at row r0; rows are contiguous in q and in out, so word gw of the range holds columns
    // gw * PER .. of the flattened rows, its output starts at element gw * PER and its group is gw * PER / group
    constexpr int PER = 32 / BITS;
    const long base = (long)blockIdx.x * DQ_WORDS + threadIdx.x;
    uint32_t v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const long gw = base + 256 * k;
        v[k] = gw < total ? __builtin_nontemporal_load(q + gw) : 0u;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const long gw = base + 256 * k;
        if (gw >= total) break;
        const size_t e0 = (size_t)gw * PER, gi = e0 / group;  // a word's values share one group (group % PER == 0)
        const float s = sc[gi], z = (float)zp[gi];
        float f[PER];
#pragma unroll
        for (int e = 0; e < PER; e++) f[e] = ((float)((v[k] >> (e * BITS)) & ((1u << BITS) - 1u)) - z) * s;
        if (F32) {
#pragma unroll
            for (int e = 0; e < PER; e += 4)
                __builtin_nontemporal_store(f32x4v{f[e], f[e + 1], f[e + 2], f[e + 3]}, (f32x4v*)((float*)out + e0 + e));
        } else {
            uint32_t b[PER / 2];
#pragma unroll
            for (int e = 0; e < PER; e += 2) {
                const __bf16 lo = (__bf16)f[e], hi = (__bf16)f[e + 1];  // round to nearest even
                b[e / 2] =
                    (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
            }
            if constexpr (PER == 8)
                __builtin_nontemporal_store(u32x4v{b[0], b[1], b[2], b[3]}, (u32x4v*)((uint16_t*)out + e0));
            else
                __builtin_nontemporal_store(u32x2v{b[0], b[1]}, (u32x2v*)((uint16_t*)out + e0));
        }
    }
}

template <int BITS, bool F32>
hipError_t launch_bits(hipStream_t s, const uint32_t* q, const float* sc, const uint8_t* zp, long total, int group,
                       void* out) {
    hipLaunchKernelGGL((dequant_kernel<BITS, F32>), dim3((unsigned)((total + DQ_WORDS - 1) / DQ_WORDS)), dim3(256), 0, s,
                       q, sc, zp, total, group, out);
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
    if (r0 + n > rows || rows > (1u << 30) || cols > (1u << 24) || n * words > ((size_t)DQ_WORDS << 31) - DQ_WORDS)
        return fail(QH_EINVAL, "dequant: rows %zu..%zu of %zu", r0, r0 + n, rows);
    if ((uintptr_t)q % 4 || (uintptr_t)out % 16)
        return fail(QH_EINVAL, "dequant: q must be 4-byte and out 16-byte aligned");
    const hipStream_t s = (hipStream_t)stream;
    // the range's first row: words, and scales and zero points per group
    const uint32_t* q0 = q + r0 * words;
    const size_t g0 = r0 * (cols / (size_t)group);
    const long total = (long)(n * words);
    hipError_t e;
    if (bits == 4)
        e = out_f32 ? launch_bits<4, true>(s, q0, scales + g0, zeros + g0, total, group, out)
                    : launch_bits<4, false>(s, q0, scales + g0, zeros + g0, total, group, out);
    else
        e = out_f32 ? launch_bits<8, true>(s, q0, scales + g0, zeros + g0, total, group, out)
                    : launch_bits<8, false>(s, q0, scales + g0, zeros + g0, total, group, out);
    if (e != hipSuccess) return fail(QH_EHIP, "dequant launch: %s", hipGetErrorString(e));
    return QH_OK;
}
