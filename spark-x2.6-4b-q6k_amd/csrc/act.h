/* act.h — the MLP activation, shared by every kernel that produces it, so
 * that each computes it with the same instructions. */
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace sparkmv {

/* gelu(g) * u with the exact-erf gelu of tools/vq-runtime/src/model.rs:253-258:
 * erf evaluated in f64 and rounded to f32, then 0.5 * g * (1 + erf) * u in
 * f32, left to right. Not inlined: a caller inside a loop would otherwise
 * hold erf's constants in registers across it. */
static __device__ __attribute__((noinline)) float gelu_mul(float g, float u) {
    const double e = erf((double) g * 0.70710678118654752440);
    return 0.5f * g * (1.0f + (float) e) * u;
}

}  // namespace sparkmv
