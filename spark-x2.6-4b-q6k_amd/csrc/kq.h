/* kq.h — host-side launchers of the ggml k-quant kernels (kq_kernels.hip). */
#pragma once

#include "common.h"

namespace sparkmv {

/* y[n*ldy + r] (+)= sum_c W[r][c] * x[n*ldx + c], W in ggml Q6_K (kind 6) or
 * Q8_0 (kind 8) blocks, row-major. x is bf16 bits or f32 (xf32). */
int kq_gemv_launch(int kind, const void * blocks, int rows, int cols, const void * x, int xf32, int ldx, int ncol,
                   float * y, int ldy, int accumulate, hipStream_t s);
/* Exact decode to f32 (overwrites out). */
int kq_dequant_launch(int kind, const void * blocks, int rows, int cols, float * out, hipStream_t s);

}  // namespace sparkmv
