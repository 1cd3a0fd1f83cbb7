/* prefill.hip — VQ GEMM for prompt prefill (many tokens against one matrix).
 *
 * Computes, for every token t and row r, y[t][r] (+)= sum_s g_s[r] * sum_i
 * cb_s[idx_s(r, i)] . x[t][dim*i ..] — the reference's per-token GEMV summed
 * over stages (tools/vq/gpu/decode-gpu.cu:359-501 is its tiled form).
 *
 * prefill_simple_kernel: one thread per (row, token), the row's indices staged
 * in LDS; any geometry and any x layout (strided), f32 arithmetic. It backs
 * variant 3 of the reference-compatible prefill entry points.
 */
#include "prefill.h"

#include <string.h>

namespace sparkmv {

__device__ __forceinline__ float pf_f16(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float) v;
}

__device__ __forceinline__ float pf_x(const void * x, int xf32, size_t k) {
    return xf32 ? ((const float *) x)[k] : __uint_as_float((uint32_t) ((const uint16_t *) x)[k] << 16);
}

__device__ __forceinline__ uint32_t pf_index(const uint8_t * st, const Layout & L, size_t row, size_t i) {
    auto byte = [&](size_t k) -> uint32_t { return k < L.idx_bytes ? (uint32_t) st[k] : 0u; };
    uint32_t v;
    if (L.v3) {
        const size_t bit = i * (size_t) L.mb;
        const size_t qb = row * L.mrow + (bit >> 3);
        const uint32_t w = byte(qb) | byte(qb + 1) << 8 | byte(qb + 2) << 16 | byte(qb + 3) << 24;
        v = (w >> (bit & 7)) & ((1u << L.mb) - 1u);
        if (L.prow) v |= ((byte(L.mrow * (size_t) L.rows + row * L.prow + (i >> 3)) >> (i & 7)) & 1u) << 12;
    } else {
        const size_t gi = row * L.nidx_row + i;
        if (L.nbit == 8) {
            v = byte(gi);
        } else {
            const size_t bit = gi * (size_t) L.nbit;
            const uint32_t w = byte(bit >> 3) | byte((bit >> 3) + 1) << 8 | byte((bit >> 3) + 2) << 16;
            v = (w >> (bit & 7)) & ((1u << L.nbit) - 1u);
        }
    }
    return v < (uint32_t) L.nc ? v : (uint32_t) L.nc - 1u;
}

struct SimpleArgs {
    const uint8_t * st[kMaxStages];
    int nst;
    Layout L;
    const void * x;
    int xf32;
    size_t xs_t, xs_k;   /* x element (t, k) sits at x[t * xs_t + k * xs_k] */
    int ntok;
    float * y;
    int ldy, accumulate;
};

__global__ __launch_bounds__(256) void prefill_simple_kernel(const SimpleArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint16_t * sidx = (uint16_t *) lds;   /* [nst][nidx_row] indices of this block's row */
    const Layout & L = A.L;
    const int row = blockIdx.x;
    for (int s = 0; s < A.nst; s++)
        for (size_t i = threadIdx.x; i < L.nidx_row; i += blockDim.x)
            sidx[s * L.nidx_row + i] = (uint16_t) pf_index(A.st[s] + L.stream_off, L, (size_t) row, i);
    __syncthreads();
    const int t = blockIdx.y * blockDim.x + threadIdx.x;
    if (t >= A.ntok) return;
    float * yp = A.y + (size_t) t * A.ldy + row;
    float v = A.accumulate ? *yp : 0.0f;
    for (int s = 0; s < A.nst; s++) {
        const uint16_t * cb = (const uint16_t *) (A.st[s] + L.cb_off);
        float acc = 0.0f;
        for (size_t i = 0; i < L.nidx_row; i++) {
            const uint32_t vv = sidx[s * L.nidx_row + i];
            for (int d = 0; d < L.dim; d++)
                acc += pf_f16(cb[(size_t) vv * L.dim + d]) * pf_x(A.x, A.xf32, (size_t) t * A.xs_t + (i * L.dim + d) * A.xs_k);
        }
        v += pf_f16(((const uint16_t *) (A.st[s] + L.gain_off))[row]) * acc;
    }
    *yp = v;
}

int prefill_simple_launch(const void * const * stages, int nst, const Layout & L, const void * x, int xf32,
                          size_t xs_t, size_t xs_k, int ntok, float * y, int ldy, int accumulate, hipStream_t s) {
    if (nst < 1 || nst > kMaxStages) { set_error("stage count %d is outside 1..%d", nst, kMaxStages); return -1; }
    if (ntok <= 0) { set_error("prefill needs at least one token"); return -1; }
    SimpleArgs A;
    memset(&A, 0, sizeof A);
    for (int i = 0; i < nst; i++) A.st[i] = (const uint8_t *) stages[i];
    A.nst = nst;
    A.L = L;
    A.x = x;
    A.xf32 = xf32;
    A.xs_t = xs_t;
    A.xs_k = xs_k;
    A.ntok = ntok;
    A.y = y;
    A.ldy = ldy;
    A.accumulate = accumulate;
    const size_t lds = (size_t) nst * L.nidx_row * 2;
    if (lds > 64 * 1024) { set_error("a row of %zu indices does not fit the simple prefill kernel", L.nidx_row); return -1; }
    const int threads = 256;
    hipLaunchKernelGGL(prefill_simple_kernel, dim3((unsigned) L.rows, (unsigned) ((ntok + threads - 1) / threads)),
                       dim3(threads), lds, s, A);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("prefill launch", e);
}

}  // namespace sparkmv
