// A read-only streaming kernel with the decode kernel's own memory access: the measurement aid behind two figures of
// the benchmark (no counterpart in the reference).
//  - The HBM read floor of a decode product: the same bytes, the same 16-byte non-temporal loads, the same wave and
//    workgroup partition over the same tile layout as skinny_kernel's plain one-token launch (2 tiles x 4 groups of
//    1 KiB blocks per wave, 4 wave columns per workgroup, the grid over tile columns x 4-group chunks of K), with no
//    arithmetic beyond folding the loaded words, no activations, no scales and no stores. A product cannot run in
//    less time than this kernel takes on its code bytes.
//  - The calibration of rocprofv3's FETCH_SIZE counter for exactly these loads (a contiguous read of known size).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qwenny_hip.h"
#include "internal.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// pattern 0: wave w reads the 8 KiB at w * 8 KiB. pattern 1: the skinny layout walk (tiles x groups 1 KiB blocks,
// block (t, g) at (t G + g) KiB): wave column wt of workgroup (bx, by) reads tiles 2 (4 bx + wt) + 0..1, groups
// 4 by + 0..3. The folded words are stored only if they equal `never` (they do not: the stores never happen, but the
// compiler cannot drop the loads).
__global__ __launch_bounds__(256) void diag_read_kernel(const u32x4* p, int tiles, int groups, int pattern,
                                                        uint32_t never, uint32_t* sink) {
    const int lane = threadIdx.x & 63, wt = threadIdx.x >> 6;
    // block offsets (in 16-byte units) of the wave's 8 blocks; loads straight off `p`, so that they stay global loads
    size_t o[8];
    if (pattern == 0) {
        const size_t w = (size_t)blockIdx.x * (blockDim.x >> 6) + wt;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (w * 8 + i) * 64 + lane;
    } else {
        const int t0 = 2 * (blockIdx.x * (blockDim.x >> 6) + wt), g0 = 4 * blockIdx.y;
        if (t0 >= tiles) return;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = ((size_t)(t0 + (i & 1)) * groups + g0 + (i >> 1)) * 64 + lane;
    }
    u32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = __builtin_nontemporal_load(p + o[i]);
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (s == never) sink[blockIdx.x] = s;
}

}  // namespace

using namespace qh;

extern "C" int qh_diag_read(void* stream, const void* buf, size_t tiles, size_t groups, int pattern, uint32_t* sink) {
    if (!buf || !sink || (uintptr_t)buf % 16) return fail(QH_EINVAL, "diag read: null or unaligned buffer");
    if (pattern != 0 && pattern != 1) return fail(QH_EINVAL, "diag read: pattern %d", pattern);
    const size_t blocks = tiles * groups;
    if (tiles == 0 || groups == 0 || tiles > (1u << 24) || groups > (1u << 20) || blocks > (1ull << 32))
        return fail(QH_EINVAL, "diag read: %zu x %zu blocks", tiles, groups);
    dim3 grid;
    if (pattern == 0) {
        if (blocks % 32) return fail(QH_EINVAL, "diag read: %zu KiB, not whole 32 KiB", blocks);
        grid = dim3((unsigned)(blocks / 32));
    } else {
        if (tiles % 2 || groups % 4) return fail(QH_EINVAL, "diag read: %zu tiles x %zu groups", tiles, groups);
        grid = dim3((unsigned)((tiles / 2 + 3) / 4), (unsigned)(groups / 4));
    }
    hipLaunchKernelGGL(diag_read_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const u32x4*)buf, (int)tiles,
                       (int)groups, pattern, 0x9e3779b9u, sink);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? QH_OK : fail(QH_EHIP, "diag read: %s", hipGetErrorString(e));
}
