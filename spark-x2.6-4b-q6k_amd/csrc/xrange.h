/* xrange.h — the activation range check shared by the GEMV kernels that stage
 * x as f16 (device code only).
 *
 * The matrix-core and dot2 kernels take x as f16 operands. f16 is exact for
 * every bf16 value between 2^-14 and 65504 (and keeps the hi + lo split of an
 * f32 value to about 22 bits there), but bf16 and f32 activations reach far
 * outside that range, where a plain conversion turns |x| >= 65520 into
 * infinity and rounds values below 2^-14 to the f16 subnormal grid. The
 * reference's decode arithmetic keeps x in f32 (tools/vq-format/src/
 * lib.rs:215-227; its GPU GEMV reads f32 x, tools/vq/gpu/decode-gpu.cu:
 * 228-260), so the kernels must not change the result there.
 *
 * Each workgroup converts x as usual and records, per wave, whether the
 * values it staged include one of |x| >= 2^15 (or a non-finite one), one of
 * |x| >= 2^-4, and a nonzero one (three ballots and one LDS word per wave,
 * inside the staging it already does). After the staging barrier the
 * workgroup reads the words. In range (some |x| >= 2^-4 and none >= 2^15,
 * or all zero) it goes on unchanged and the results are exactly those of the
 * plain conversion. Otherwise, a uniform branch: the workgroup reads x again
 * for its largest finite |x|; unless that is in range after all (the flag
 * came from an infinity or NaN), x is staged again as x * 2^-k (a power of
 * two, exact) so that the largest lands in [2^14, 2^15), and the kernel
 * multiplies its sums by 2^k, which is exact as well. Non-finite x stays
 * non-finite, and y with it, as in an f32 product; other columns keep their
 * precision.
 *
 * LDS: kXrWords words per workgroup (16 wave flag words, 16 wave maxima), at
 * a 16-byte aligned offset (xr_off): the VQ kernels read all flag words in
 * four 16-byte reads (xr_out), the k-quant kernels one word per lane
 * (xr_out_lanes). */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sparkmv {

constexpr int kXrWords = 32;
constexpr uint32_t kXrBytes = kXrWords * 4 + 16;   /* with room to align */

/* the area's byte offset in LDS, given the end of what precedes it */
__host__ __device__ constexpr uint32_t xr_off(uint32_t end) { return (end + 15u) & ~15u; }
constexpr uint32_t kXrOver = 0x47000000u;   /* 2^15, as f32 bits */
constexpr uint32_t kXrLow = 0x3d800000u;    /* 2^-4 */
constexpr uint32_t kXrInf = 0x7f800000u;

/* |x| as f32 bits (monotonic in |x|; NaN above infinity) */
__device__ __forceinline__ uint32_t xr_mag(float f) { return __float_as_uint(f) & 0x7fffffffu; }
__device__ __forceinline__ uint32_t xr_mag_f32w(uint32_t w) { return w & 0x7fffffffu; }
/* the larger |x| of a bf16 pair, as f32 bits */
__device__ __forceinline__ uint32_t xr_mag_bf16x2(uint32_t w) {
    return max((w << 16) & 0x7fffffffu, w & 0x7fff0000u);
}
/* The largest |x| of bf16 pairs, two lanes at a time (one packed u16 max per
 * pair); xr_bf16_max turns it into f32 bits. */
typedef uint16_t xr_u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void xr_acc_bf16x2(xr_u16x2 & m, uint32_t w) {
    m = __builtin_elementwise_max(m, __builtin_bit_cast(xr_u16x2, w & 0x7fff7fffu));
}
__device__ __forceinline__ uint32_t xr_bf16_max(xr_u16x2 m) { return (uint32_t) max(m.x, m.y) << 16; }

/* |x| as f32 bits for the finite maximum: non-finite values count as zero */
__device__ __forceinline__ uint32_t xr_fin(uint32_t mag) { return mag < kXrInf ? mag : 0u; }

__device__ __forceinline__ void xr_put(uint32_t * xr, bool over, bool big, bool nonzero) {
    const uint32_t b = (__builtin_amdgcn_ballot_w64(over) ? 1u : 0u) | (__builtin_amdgcn_ballot_w64(big) ? 2u : 0u) |
                       (__builtin_amdgcn_ballot_w64(nonzero) ? 4u : 0u);
    if ((threadIdx.x & 63u) == 0u) xr[threadIdx.x >> 6] = b;
}

/* Every wave, in uniform control flow, before the staging barrier: its
 * flags from the largest |x| m that each lane staged, as f32 bits. */
__device__ __forceinline__ void xr_note(uint32_t * xr, uint32_t m) { xr_put(xr, m >= kXrOver, m >= kXrLow, m != 0u); }

/* The same from the largest converted value, as f16 bits (2^15 is 0x7800,
 * 2^-4 is 0x2c00; infinity and NaN lie above). A value below 2^-25 converts
 * to zero, so x whose every |x| is below 2^-25 reads as zero. */
__device__ __forceinline__ void xr_note_f16(uint32_t * xr, uint32_t m16) {
    xr_put(xr, m16 >= 0x7800u, m16 >= 0x2c00u, m16 != 0u);
}

/* After the barrier: whether the workgroup must look at x again (the same
 * answer in every thread). Waves first .. staged x and noted it. */
__device__ __forceinline__ bool xr_out(const uint32_t * xr, int first = 0) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const int nw = (int) (blockDim.x >> 6);
    uint32_t b = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u4 v = ((const u4 *) xr)[i];
#pragma unroll
        for (int j = 0; j < 4; j++) b |= 4 * i + j >= first && 4 * i + j < nw ? v[j] : 0u;
    }
    return (b & 1u) || (!(b & 2u) && (b & 4u));
}

/* The same from one word per lane, lane i holding wave i's flags: one
 * LDS read and three ballots. */
__device__ __forceinline__ bool xr_out_lanes(uint32_t w, int first = 0) {
    const int lane = (int) (threadIdx.x & 63u), nw = (int) (blockDim.x >> 6);
    const uint32_t b = lane >= first && lane < nw ? w : 0u;
    const bool over = __builtin_amdgcn_ballot_w64(b & 1u) != 0;
    const bool big = __builtin_amdgcn_ballot_w64(b & 2u) != 0;
    const bool nonzero = __builtin_amdgcn_ballot_w64(b & 4u) != 0;
    return over || (!big && nonzero);
}

__device__ __forceinline__ uint32_t xr_wave_max(uint32_t m) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t) __shfl_xor((int) m, o, 64));
    return m;
}

/* The largest m over the four lanes that share lane & 15: in the MFMA
 * layouts here, the lanes of one B column (and of one output column). */
__device__ __forceinline__ uint32_t xr_col_max(uint32_t m) {
    m = max(m, (uint32_t) __shfl_xor((int) m, 16, 64));
    return max(m, (uint32_t) __shfl_xor((int) m, 32, 64));
}

/* The rescale exponent k for the largest finite |x|, as f32 bits M: 0 when
 * M is zero or in range, else the k that brings M to exponent 14. */
__device__ __forceinline__ int xr_shift_of(uint32_t M) {
    return M == 0u || (M >= kXrLow && M < kXrOver) ? 0 : (int) (M >> 23) - 141;
}

/* Out of range, every thread of the workgroup: the workgroup's largest
 * finite |x| from each thread's m (a barrier inside) and from it k. */
__device__ __forceinline__ int xr_shift(uint32_t * xr, uint32_t m) {
    const uint32_t wm = xr_wave_max(m);
    if ((threadIdx.x & 63u) == 0u) xr[16 + (threadIdx.x >> 6)] = wm;
    __syncthreads();
    const int nw = (int) (blockDim.x >> 6);
    uint32_t M = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) M = max(M, i < nw ? xr[16 + i] : 0u);
    return xr_shift_of(M);
}

/* sum * 2^k, exact; k = 0 leaves the value as it is */
__device__ __forceinline__ float xr_unscale(float v, int k) { return k ? __builtin_ldexpf(v, k) : v; }

}  // namespace sparkmv
