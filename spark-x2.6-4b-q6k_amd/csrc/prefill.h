/* prefill.h — host-side launchers of the prefill GEMM kernels (prefill.hip). */
#pragma once

#include "common.h"

namespace sparkmv {

/* y[t * ldy + r] (+)= sum over stages of the stage GEMV of token t, with x
 * element (t, k) at x[t * xs_t + k * xs_k] (bf16 bits or f32). Any geometry. */
int prefill_simple_launch(const void * const * stages, int nst, const Layout & L, const void * x, int xf32,
                          size_t xs_t, size_t xs_k, int ntok, float * y, int ldy, int accumulate, hipStream_t s);

}  // namespace sparkmv
