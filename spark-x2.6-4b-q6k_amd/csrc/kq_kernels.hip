/* kq_kernels.hip — ggml Q6_K and Q8_0 dequant-GEMV for gfx950.
 *
 * Block layouts (ggml's published structs; sizes match tools/kquant/stubs.c:25-30):
 *   block_q6_K (210 B / 256 weights): ql[128] | qh[64] | int8 scales[16] | fp16 d
 *     weight 128h + 32k + l (h half, k quarter, l 0..31) =
 *       d * scales[8h + l/16 + 2k] * (q - 32),
 *       q = (ql[64h + l + 32(k&1)] >> 4(k>>1)) & 15 | ((qh[32h + l] >> 2k) & 3) << 4
 *   block_q8_0 (34 B / 32 weights): fp16 d | int8 qs[32];  weight j = d * qs[j]
 * Every decoded weight is exact in f32 (d has 11 significant bits, the
 * integer factor at most 11 more), so the dequant kernels are bit-exact and the
 * GEMVs only round in the f32 accumulation.
 *
 * GEMV mapping: 16 lanes per row (a wave covers 4 rows), each lane a run of
 * blocks (Q8_0) or superblock halves (Q6_K) spaced 16 apart; partial sums meet
 * in a 16-lane butterfly. Blocks are 2-byte aligned, so a lane reads the
 * dword-aligned window around its bytes with dwordx4 loads and realigns with
 * v_alignbit; the window never leaves the block except where the next
 * block's bytes follow, and the buffer's final block reads only its own bytes.
 */
#include "kq.h"

#include <string.h>

namespace sparkmv {

__device__ __forceinline__ float kq_f16(uint32_t h) {
    _Float16 v;
    const uint16_t b = (uint16_t) h;
    __builtin_memcpy(&v, &b, 2);
    return (float) v;
}

__device__ __forceinline__ float kq_x(const void * x, int xf32, size_t k) {
    return xf32 ? ((const float *) x)[k] : __uint_as_float((uint32_t) ((const uint16_t *) x)[k] << 16);
}

/* N dwords of the byte stream starting at `addr` (2-byte aligned): loads the
 * covering aligned dwords and funnel-shifts them. `last_ok` false forbids the
 * extra trailing dword (the stream's end is the buffer's end). */
template <int N>
__device__ __forceinline__ void load_stream(const uint8_t * addr, uint32_t * out, bool last_ok) {
    const uintptr_t a = (uintptr_t) addr;
    const uint32_t * p = (const uint32_t *) (a & ~(uintptr_t) 3);
    const uint32_t sh = (uint32_t) (a & 3) * 8u;
    uint32_t w[N + 1];
#pragma unroll
    for (int k = 0; k < N; k++) w[k] = p[k];
    if (sh && last_ok) w[N] = p[N];
    else if (sh) w[N] = (uint32_t) *(const uint16_t *) (p + N);
    else w[N] = 0;
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
}

__device__ __forceinline__ float sum16(float v) {
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

/* ---------------------------------- Q8_0 --------------------------------- */

__global__ __launch_bounds__(256) void q8_0_gemv_kernel(const uint8_t * blocks, int rows, int cols, const void * x,
                                                        int xf32, int ldx, int ncol, float * y, int ldy, int accumulate) {
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int bpr = cols / 32;
    const size_t total = (size_t) rows * bpr;
    const int row_step = gridDim.x * (blockDim.x >> 6) * 4;
    for (int r0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4; r0 < rows; r0 += row_step) {
        const int row = r0 + g;
        float acc[kMaxCols];
#pragma unroll
        for (int n = 0; n < kMaxCols; n++) acc[n] = 0.0f;
        if (row < rows) {
            for (int c = j; c < bpr; c += 16) {
                const size_t b = (size_t) row * bpr + c;
                const uint8_t * blk = blocks + b * 34;
                const float d = kq_f16(*(const uint16_t *) blk);
                uint32_t q[8];
                load_stream<8>(blk + 2, q, b + 1 < total);
                float qf[32];
#pragma unroll
                for (int k = 0; k < 8; k++) {
#pragma unroll
                    for (int e = 0; e < 4; e++) qf[4 * k + e] = (float) (int) (int8_t) (q[k] >> (8 * e));
                }
#pragma unroll
                for (int n = 0; n < kMaxCols; n++) {
                    if (n < ncol) {
                        float s = 0.0f;
#pragma unroll
                        for (int e = 0; e < 32; e++) s += qf[e] * kq_x(x, xf32, (size_t) n * ldx + 32 * (size_t) c + e);
                        acc[n] += d * s;
                    }
                }
            }
        }
#pragma unroll
        for (int n = 0; n < kMaxCols; n++) {
            if (n < ncol) {
                const float s = sum16(acc[n]);
                if (j == 0 && row < rows) {
                    float * yp = y + (size_t) n * ldy + row;
                    *yp = (accumulate ? *yp : 0.0f) + s;
                }
            }
        }
    }
}

/* ---------------------------------- Q6_K --------------------------------- */

__global__ __launch_bounds__(256) void q6k_gemv_kernel(const uint8_t * blocks, int rows, int cols, const void * x,
                                                       int xf32, int ldx, int ncol, float * y, int ldy, int accumulate) {
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int bpr = cols / 256, units = 2 * bpr;   /* a unit is one 128-weight half */
    const int row_step = gridDim.x * (blockDim.x >> 6) * 4;
    for (int r0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4; r0 < rows; r0 += row_step) {
        const int row = r0 + g;
        float acc[kMaxCols];
#pragma unroll
        for (int n = 0; n < kMaxCols; n++) acc[n] = 0.0f;
        if (row < rows) {
            for (int u = j; u < units; u += 16) {
                const int sb = u >> 1, h = u & 1;
                const uint8_t * blk = blocks + ((size_t) row * bpr + sb) * 210;
                const float d = kq_f16(*(const uint16_t *) (blk + 208));
                uint32_t ql[16], qh[8], scw[2];
                load_stream<16>(blk + 64 * h, ql, true);
                load_stream<8>(blk + 128 + 32 * h, qh, true);
                load_stream<2>(blk + 192 + 8 * h, scw, true);
                const size_t col0 = (size_t) sb * 256 + 128 * h;
#pragma unroll
                for (int k = 0; k < 4; k++) {
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        const int sci = p + 2 * k;
                        const float dsc = d * (float) (int) (int8_t) (scw[sci >> 2] >> (8 * (sci & 3)));
                        float qf[16];
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            const int l = 16 * p + e;
                            const uint32_t lo = (ql[(l + 32 * (k & 1)) >> 2] >> (8 * (l & 3) + 4 * (k >> 1))) & 15u;
                            const uint32_t hi = (qh[l >> 2] >> (8 * (l & 3) + 2 * k)) & 3u;
                            qf[e] = (float) ((int) (lo | (hi << 4)) - 32);
                        }
#pragma unroll
                        for (int n = 0; n < kMaxCols; n++) {
                            if (n < ncol) {
                                float s = 0.0f;
#pragma unroll
                                for (int e = 0; e < 16; e++)
                                    s += qf[e] * kq_x(x, xf32, (size_t) n * ldx + col0 + 32 * k + 16 * p + e);
                                acc[n] += dsc * s;
                            }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int n = 0; n < kMaxCols; n++) {
            if (n < ncol) {
                const float s = sum16(acc[n]);
                if (j == 0 && row < rows) {
                    float * yp = y + (size_t) n * ldy + row;
                    *yp = (accumulate ? *yp : 0.0f) + s;
                }
            }
        }
    }
}

/* ------------------------------- dequant --------------------------------- */

__global__ void q8_0_dequant_kernel(const uint8_t * blocks, size_t nblocks, float * out) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks * 32) return;
    const uint8_t * blk = blocks + (i >> 5) * 34;
    out[i] = (float) (int8_t) blk[2 + (i & 31)] * kq_f16(*(const uint16_t *) blk);
}

__global__ void q6k_dequant_kernel(const uint8_t * blocks, size_t nblocks, float * out) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks * 256) return;
    const uint8_t * blk = blocks + (i >> 8) * 210;
    const int w = (int) (i & 255), h = w >> 7, k = (w >> 5) & 3, l = w & 31;
    const uint32_t lo = (blk[64 * h + l + 32 * (k & 1)] >> (4 * (k >> 1))) & 15u;
    const uint32_t hi = (blk[128 + 32 * h + l] >> (2 * k)) & 3u;
    const int sc = (int8_t) blk[192 + 8 * h + l / 16 + 2 * k];
    const float d = kq_f16(*(const uint16_t *) (blk + 208));
    out[i] = d * (float) sc * (float) ((int) (lo | (hi << 4)) - 32);
}

/* -------------------------------- host ----------------------------------- */

int kq_gemv_launch(int kind, const void * blocks, int rows, int cols, const void * x, int xf32, int ldx, int ncol,
                   float * y, int ldy, int accumulate, hipStream_t s) {
    const int blk = kind == 6 ? 256 : 32;
    if (kind != 6 && kind != 8) { set_error("unknown k-quant kind %d", kind); return -1; }
    if (rows <= 0 || cols <= 0 || cols % blk) {
        set_error("%s needs rows > 0 and cols a multiple of %d (got %d x %d)", kind == 6 ? "Q6_K" : "Q8_0", blk, rows, cols);
        return -1;
    }
    if (!blocks || !x || !y) { set_error("null pointer passed to the k-quant GEMV"); return -1; }
    if (((uintptr_t) blocks) & 1) { set_error("k-quant blocks must be 2-byte aligned"); return -1; }
    if (ncol < 1 || ncol > kMaxCols) { set_error("column count %d is outside 1..%d", ncol, kMaxCols); return -1; }
    if (ncol > 1 && (ldx < cols || ldy < rows)) { set_error("ldx/ldy below the matrix extent"); return -1; }
    const int threads = 256;
    const int rows_per_block = (threads / 64) * 4;
    int grid = (rows + rows_per_block - 1) / rows_per_block;
    const int cap = cu_count() * 8;
    if (grid > cap) grid = cap;
    if (kind == 6)
        hipLaunchKernelGGL(q6k_gemv_kernel, dim3(grid), dim3(threads), 0, s, (const uint8_t *) blocks, rows, cols, x,
                           xf32, ldx, ncol, y, ldy, accumulate);
    else
        hipLaunchKernelGGL(q8_0_gemv_kernel, dim3(grid), dim3(threads), 0, s, (const uint8_t *) blocks, rows, cols, x,
                           xf32, ldx, ncol, y, ldy, accumulate);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("k-quant gemv launch", e);
}

int kq_dequant_launch(int kind, const void * blocks, int rows, int cols, float * out, hipStream_t s) {
    const int blk = kind == 6 ? 256 : 32;
    if ((kind != 6 && kind != 8) || rows <= 0 || cols <= 0 || cols % blk || !blocks || !out) {
        set_error("k-quant dequant needs a valid kind, shape and pointers");
        return -1;
    }
    const size_t nb = (size_t) rows * (cols / blk);
    const size_t n = nb * blk;
    const int threads = 256;
    if (kind == 6)
        hipLaunchKernelGGL(q6k_dequant_kernel, dim3((unsigned) ((n + threads - 1) / threads)), dim3(threads), 0, s,
                           (const uint8_t *) blocks, nb, out);
    else
        hipLaunchKernelGGL(q8_0_dequant_kernel, dim3((unsigned) ((n + threads - 1) / threads)), dim3(threads), 0, s,
                           (const uint8_t *) blocks, nb, out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("k-quant dequant launch", e);
}

}  // namespace sparkmv
