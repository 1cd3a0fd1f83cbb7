/* prefill.h — host-side launchers of the prefill GEMM kernels (prefill.hip). */
#pragma once

#include "common.h"

namespace sparkmv {

/* y[t * ldy + r] (+)= sum over stages of the stage GEMV of token t, with x
 * element (t, k) at x[t * xs_t + k * xs_k] (bf16 bits or f32). Any geometry. */
int prefill_simple_launch(const void * const * stages, int nst, const Layout & L, const void * x, int xf32,
                          size_t xs_t, size_t xs_k, int ntok, float * y, int ldy, int accumulate, hipStream_t s);

/* The MFMA GEMM: DQV3 dim 4, 12/13-bit indices, 1 or 2 stages, x in
 * 16-byte aligned rows, y[t * ldy + r] (+)= W x_t. x is token-major
 * (x[t * ldx + k], bf16 or f32) or, with xt, K-major f32 of one stage
 * (x[k * ldx + t], the reference's xT layout, ntok >= 4). Two stages enter
 * the MFMA as one f16 weight (one rounding of the f32 decode); one stage as
 * its exact codewords, scaled by the row gain in f32. x enters as f16. Short
 * matrices split K through a stream-ordered workspace and a fixed-order
 * reduction. */
int prefill_mfma_ready(const Layout & L, int nst, const void * x, int xf32, int ldx, int xt, int ntok);
/* fixed_ws: NULL takes split slices from the library's pool; otherwise the
 * device address of the no-allocation scratch (prefill_scratch), whose size
 * bounds the split slices. */
int prefill_mfma_launch(const void * const * stages, int nst, const Layout & L, const void * x, int xf32, int ldx,
                        int xt, int ntok, float * y, int ldy, int accumulate, hipStream_t s,
                        void * fixed_ws = nullptr);

/* Whether two-stage prefills fold their stages into one f16 weight (the
 * default; off: each stage's exact codewords accumulate apart).
 * Process-wide. */
int prefill_fold_on();
int prefill_fold_set(int on);   /* returns the previous setting */

/* Bytes of the no-allocation prefill's scratch (split-K partial sums), one
 * array per GPU: the 2560 x 10240 FFN down matrix at 512 tokens needs 26 MB. */
constexpr size_t kPrefillScratchBytes = 32u << 20;
/* The scratch array's device address on the current device (looked up once
 * per device); 0, or -1 with the message set. */
int prefill_scratch(void ** ptr);

}  // namespace sparkmv
