// The product entry points' shared core (api.hip) and the allocation-free entry point's set-up (noalloc.hip).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "../../include/qwenny_hip.h"
#include "kernels.h"

namespace qh {

// qh_gemm's argument checks and launch, with the launch scratch at `sc` (device addresses; zero between launches).
int gemm_with_scratch(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n,
                      const int32_t* out_rows, size_t n_out, void* y, int epi, uint64_t* keys, int whole,
                      const Scratch& sc, const qh_lora* lora = nullptr);

// The device a context was opened on.
int ctx_device(const qh_ctx* ctx);

// Set-up of the allocation-free entry point on `device` (current on the calling thread): resolves the device address
// of its static scratch once per device and clears it. Called by qh_open.
int noalloc_init(int device);

}  // namespace qh
