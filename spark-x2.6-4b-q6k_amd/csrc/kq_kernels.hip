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
 * Q8_0 runs on the matrix cores (q8_0_mfma_kernel) wherever rows are whole
 * 512-column chunks in a 16-byte aligned buffer, for every column count, so
 * the columns of a speculative verify equal one-column launches bit for bit;
 * other shapes take the dot2 kernels below, again for every column count.
 *
 * Dot2 GEMV mapping: 16 lanes per row (a wave covers 4 rows), each lane a run
 * of blocks (Q8_0) or superblock halves (Q6_K) spaced 16 apart; partial sums
 * meet in a 16-lane butterfly. Blocks are 2-byte aligned, so a lane reads the
 * dword-aligned window around its bytes with dwordx4 loads and realigns with
 * v_alignbit; the window never leaves the block except where the next
 * block's bytes follow, and the buffer's final block reads only its own bytes.
 */
#include "kq.h"
#include "xrange.h"

#include <string.h>

#include <atomic>
#include <type_traits>

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
    /* global address space (a pointer rebuilt from an integer would be a
     * flat one: flat loads wait on both counters) */
    typedef const __attribute__((address_space(1))) uint32_t gu32;
    typedef const __attribute__((address_space(1))) uint16_t gu16;
    const uintptr_t a = (uintptr_t) addr;
    gu32 * p = (gu32 *) (a & ~(uintptr_t) 3);
    const uint32_t sh = (uint32_t) (a & 3) * 8u;
    uint32_t w[N + 1];
#pragma unroll
    for (int k = 0; k < N; k++) w[k] = p[k];
    if (sh && last_ok) w[N] = p[N];
    else if (sh) w[N] = (uint32_t) *(gu16 *) (p + N);
    else w[N] = 0;
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
}

/* N dwords of LDS bytes from byte `off` of the shared array (2-byte
 * aligned): the covering aligned dwords, funnel-shifted. Offsets from the
 * array itself keep the reads in the LDS address space. */
template <int N>
__device__ __forceinline__ void lds_stream(const uint8_t * lds_base, uint32_t off, uint32_t * out) {
    const uint32_t * p = (const uint32_t *) (lds_base + (off & ~3u));
    const uint32_t sh = (off & 3u) * 8u;
    uint32_t w[N + 1];
#pragma unroll
    for (int k = 0; k <= N; k++) w[k] = p[k];
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
}

__device__ __forceinline__ float sum16(float v) {
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

typedef _Float16 kq_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 kq_h4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ kq_h2 as_h2(uint32_t v) {
    kq_h2 r;
    __builtin_memcpy(&r, &v, 4);
    return r;
}

/* Two f16 pairs holding the four bytes of w (each biased by 1024: the f16
 * with exponent field 25 and the byte as significand is exactly 1024 + b)
 * minus `bias`: exact integers in f16. */
__device__ __forceinline__ void bytes_to_h2(uint32_t w, _Float16 bias, kq_h2 & lo, kq_h2 & hi) {
    const kq_h2 b2 = {bias, bias};
    lo = as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)) - b2;
    hi = as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)) - b2;
}

/* Activations staged once per workgroup as f16, 32 columns per 72-byte slot
 * (64 bytes of data and 8 of pad, so the 16 lanes of a row, 16 slots apart,
 * hit distinct LDS banks). f32 activations also stage the residual
 * lo = f16(x - hi) one array further on, and the dot runs over both. */
/* x to LDS as f16 (and the f32 remainder as a second f16 array), 72-byte
 * slots of 32 columns. With 4-byte aligned rows (x aligned, ldx even) the
 * columns go in groups of 8 through batches of unconditional 16-byte loads
 * (groups past the end re-read the last one), so the staging costs a few
 * memory latencies rather than one per element; otherwise one element per
 * thread and step. PADU adds 8 bytes after every 4 slots (128 columns): the
 * Q6_K kernels' lanes read 128-column units, and the pad puts neighbouring
 * units on different LDS banks. FLAT instead stores each column's values
 * contiguously (column k at byte 2k of its xst-byte row). */
template <int XF32, int PADU = 0, int FLAT = 0>
__device__ __forceinline__ uint32_t kq_stage_x_by(uint8_t * lds, const void * x, int ldx, int ncol, int cols, int xst,
                                                  int tid, int nthr) {
    typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));
    const bool vec = !((uintptr_t) x & 3) && (ncol == 1 || !(ldx & 1));
    /* the largest staged |f16(x)|, as f16 bits (two lanes of a pair) */
    typedef uint16_t ush2 __attribute__((ext_vector_type(2)));
    ush2 m16 = {0, 0};
    if (vec) {
        constexpr int KB = 8, NV = XF32 ? 2 : 1;
        const int ng = cols >> 3, total = ncol * ng;
        for (int base = 0; base < total; base += KB * nthr) {
            u4a v[KB][NV];
            int gi[KB];
#pragma unroll
            for (int k = 0; k < KB; k++) {
                gi[k] = min(base + k * nthr + tid, total - 1);
                const int n = gi[k] / ng, c8 = gi[k] - n * ng;
                const uint8_t * src = (const uint8_t *) x + ((size_t) n * ldx + 8 * c8) * (XF32 ? 4 : 2);
#pragma unroll
                for (int q = 0; q < NV; q++) v[k][q] = ((const u4a *) src)[q];
            }
#pragma unroll
            for (int k = 0; k < KB; k++) {
                const int n = gi[k] / ng, e = 8 * (gi[k] - n * ng);
                const int off = FLAT ? 2 * e : (e >> 5) * 72 + (PADU ? (e >> 7) * 8 : 0) + 2 * (e & 31);
                float f[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const uint32_t w = XF32 ? v[k][q >> 2][q & 3] : v[k][0][q >> 1];
                    f[q] = XF32 ? __uint_as_float(w) : __uint_as_float((q & 1) ? (w & 0xffff0000u) : (w << 16));
                }
                kq_h4 h0, h1;
#pragma unroll
                for (int q = 0; q < 4; q++) { h0[q] = (_Float16) f[q]; h1[q] = (_Float16) f[4 + q]; }
                {
                    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
                    const u2v a = __builtin_bit_cast(u2v, h0), b = __builtin_bit_cast(u2v, h1);
                    m16 = __builtin_elementwise_max(m16, __builtin_bit_cast(ush2, (a.x & 0x7fff7fffu)));
                    m16 = __builtin_elementwise_max(m16, __builtin_bit_cast(ush2, (a.y & 0x7fff7fffu)));
                    m16 = __builtin_elementwise_max(m16, __builtin_bit_cast(ush2, (b.x & 0x7fff7fffu)));
                    m16 = __builtin_elementwise_max(m16, __builtin_bit_cast(ush2, (b.y & 0x7fff7fffu)));
                }
                *(kq_h4 *) (lds + n * xst + off) = h0;
                *(kq_h4 *) (lds + n * xst + off + 8) = h1;
                if (XF32) {
                    kq_h4 l0, l1;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        l0[q] = (_Float16) (f[q] - (float) h0[q]);
                        l1[q] = (_Float16) (f[4 + q] - (float) h1[q]);
                    }
                    *(kq_h4 *) (lds + (ncol + n) * xst + off) = l0;
                    *(kq_h4 *) (lds + (ncol + n) * xst + off + 8) = l1;
                }
            }
        }
        return max(m16.x, m16.y);
    }
    uint32_t m = 0;
    for (int e = tid; e < ncol * cols; e += nthr) {
        const int n = e / cols, k = e - n * cols;
        const float v = kq_x(x, XF32, (size_t) n * ldx + k);
        const _Float16 hi = (_Float16) v;
        m = max(m, (uint32_t) __builtin_bit_cast(uint16_t, hi) & 0x7fffu);
        const int off = FLAT ? 2 * k : (k >> 5) * 72 + (PADU ? (k >> 7) * 8 : 0) + 2 * (k & 31);
        *(_Float16 *) (lds + n * xst + off) = hi;
        if (XF32) *(_Float16 *) (lds + (ncol + n) * xst + off) = (_Float16) (v - (float) hi);
    }
    return m;
}

/* The whole workgroup stages x. */
template <int XF32, int PADU = 0, int FLAT = 0>
__device__ __forceinline__ uint32_t kq_stage_x(uint8_t * lds, const void * x, int ldx, int ncol, int cols, int xst) {
    return kq_stage_x_by<XF32, PADU, FLAT>(lds, x, ldx, ncol, cols, xst, (int) threadIdx.x, (int) blockDim.x);
}

/* After the staging barrier, every thread of the workgroup: when the staged
 * x looks out of f16's comfortable range, find the workgroup's largest
 * finite |x| (x read again) and, unless that is in range, stage x again as
 * x * 2^-k (one element per thread and step, the same layout) and return k;
 * otherwise return 0 with x as staged. */
template <int XF32, int PADU = 0, int FLAT = 0>
__device__ __forceinline__ int kq_x_range(uint8_t * lds, uint32_t * xr, const void * x, int ldx, int ncol, int cols,
                                          int xst, int first = 0) {
    if (!xr_out_lanes(xr[threadIdx.x & 15u], first)) return 0;
    uint32_t m = 0;
    for (int e = threadIdx.x; e < ncol * cols; e += blockDim.x) {
        const int n = e / cols, c = e - n * cols;
        m = max(m, xr_fin(xr_mag(kq_x(x, XF32, (size_t) n * ldx + c))));
    }
    const int k = xr_shift(xr, m);
    if (!k) return 0;
    for (int e = threadIdx.x; e < ncol * cols; e += blockDim.x) {
        const int n = e / cols, c = e - n * cols;
        const float v = __builtin_ldexpf(kq_x(x, XF32, (size_t) n * ldx + c), -k);
        const _Float16 hi = (_Float16) v;
        const int off = FLAT ? 2 * c : (c >> 5) * 72 + (PADU ? (c >> 7) * 8 : 0) + 2 * (c & 31);
        *(_Float16 *) (lds + n * xst + off) = hi;
        if (XF32) *(_Float16 *) (lds + (ncol + n) * xst + off) = (_Float16) (v - (float) hi);
    }
    __syncthreads();
    return k;
}

/* ---------------------------------- Q8_0 --------------------------------- */

/* Lane (j, g) of a wave sums blocks j, j + 16, j + 32, ... of RPL rows, the
 * rows of a wave being 4 RPL consecutive ones, and 16 lanes reduce each row
 * (sum16). Per row and column the arithmetic is the same for every RPL and
 * NC: 16 fdot2 per block in column order, acc += d * s in block order, the
 * same reduction tree, so each column of a several-column launch equals a
 * one-column launch bit for bit. With RPL = 4 a lane reads each activation
 * of a block once for four rows (several columns read x from LDS once per
 * four rows instead of once per row); one column keeps RPL = 1 and four
 * blocks of one row in flight. */
template <int NC, int XF32, int RPL = 1>
__global__ __launch_bounds__(256) void q8_0_gemv_kernel(const uint8_t * blocks, int rows, int cols, const void * x,
                                                        int ldx, int ncol, float * y, int ldy, int accumulate) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int UB = 4 / RPL;   /* blocks of each row per pass: four loads in flight per lane */
    const int bpr = cols / 32, xst = bpr * 72;
    uint32_t * xr = (uint32_t *) (lds + xr_off((XF32 ? 2 : 1) * ncol * xst));
    const uint32_t xm = kq_stage_x<XF32>(lds, x, ldx, ncol, cols, xst);
    xr_note_f16(xr, xm);
    __syncthreads();
    const int xk = kq_x_range<XF32>(lds, xr, x, ldx, ncol, cols, xst);
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const size_t total = (size_t) rows * bpr;
    const int row_step = gridDim.x * (blockDim.x >> 6) * 4 * RPL;
    for (int r0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4 * RPL; r0 < rows; r0 += row_step) {
        float acc[RPL][NC];
#pragma unroll
        for (int i = 0; i < RPL; i++)
#pragma unroll
            for (int n = 0; n < NC; n++) acc[i][n] = 0.0f;
        for (int cb = j; cb < bpr; cb += 16 * UB) {
            uint32_t qw[UB][RPL][8];
            float d[UB][RPL];
#pragma unroll
            for (int u = 0; u < UB; u++) {
                const int c = cb + 16 * u;
                if (c < bpr) {
#pragma unroll
                    for (int i = 0; i < RPL; i++) {
                        const size_t b = (size_t) min(r0 + RPL * g + i, rows - 1) * bpr + c;
                        const uint8_t * blk = blocks + b * 34;
                        d[u][i] = kq_f16(*(const uint16_t *) blk);
                        load_stream<8>(blk + 2, qw[u][i], b + 1 < total);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < UB; u++) {
                const int c = cb + 16 * u;
                if (c < bpr) {
                    /* the block's quants as f16 pairs, once for every column */
                    kq_h2 qa[RPL][8], qb[RPL][8];
#pragma unroll
                    for (int i = 0; i < RPL; i++)
#pragma unroll
                        for (int k = 0; k < 8; k++) bytes_to_h2(qw[u][i][k] ^ 0x80808080u, (_Float16) 1152.0f, qa[i][k], qb[i][k]);
                    /* every column slot, branch-free (slots past ncol re-read
                     * the last column and are not stored), so the compiler
                     * can read the next column's x while this one computes */
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        const uint8_t * xp = lds + min(n, ncol - 1) * xst + c * 72;
                        float s[RPL];
#pragma unroll
                        for (int i = 0; i < RPL; i++) s[i] = 0.0f;
#pragma unroll
                        for (int k = 0; k < 8; k++) {
                            const kq_h4 xv = *(const kq_h4 *) (xp + 8 * k);
                            kq_h4 xl;
                            if (XF32) xl = *(const kq_h4 *) (xp + ncol * xst + 8 * k);
#pragma unroll
                            for (int i = 0; i < RPL; i++) {
                                s[i] = __builtin_amdgcn_fdot2(qa[i][k], kq_h2{xv[0], xv[1]}, s[i], false);
                                s[i] = __builtin_amdgcn_fdot2(qb[i][k], kq_h2{xv[2], xv[3]}, s[i], false);
                                if (XF32) {
                                    s[i] = __builtin_amdgcn_fdot2(qa[i][k], kq_h2{xl[0], xl[1]}, s[i], false);
                                    s[i] = __builtin_amdgcn_fdot2(qb[i][k], kq_h2{xl[2], xl[3]}, s[i], false);
                                }
                            }
                        }
#pragma unroll
                        for (int i = 0; i < RPL; i++) acc[i][n] += d[u][i] * s[i];
                    }
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NC; n++) {
            if (n < ncol) {
#pragma unroll
                for (int i = 0; i < RPL; i++) {
                    const float v = xr_unscale(sum16(acc[i][n]), xk);
                    const int row = r0 + RPL * g + i;
                    if (j == 0 && row < rows) {
                        float * yp = y + (size_t) n * ldy + row;
                        *yp = (accumulate ? *yp : 0.0f) + v;
                    }
                }
            }
        }
    }
}

/* Q8_0 on the matrix cores (v_mfma_f32_16x16x32_f16), every column count.
 * A wave owns tiles of 16 rows; per 32-weight block it forms
 *   D = A B from zero, A[i][k] = x[i][k] as f16 (activation columns past
 *   ncol zero), B[k][j] = q(row j, weight k) (exact in f16),
 * and then acc[i][j] = fma(d(row j), D[i][j], acc[i][j]), blocks in row
 * order. Row i of D depends on row i of A alone, so each column of a
 * several-column launch equals a one-column launch bit for bit.
 * Rows stream through LDS in chunks of 16 blocks: a chunk (16 rows x 544
 * bytes) is loaded with coalesced 16-byte loads into registers PD chunks
 * ahead, stored into the wave's own LDS slot (rows 560 bytes apart, so the
 * lanes' fragment reads hit distinct banks) and read back in MFMA layout:
 * lane (m, g) = m + 16 g takes weights 8g .. 8g + 7 of the block, of row m
 * (B) and of activation column m (A); D[i][j] lands in lane j + 16 (i / 4),
 * so a lane scales its four sums by one row's d. x is staged once per
 * workgroup as f16, each column contiguous. Only the x staging uses a
 * barrier: the waves then run on their own. */
constexpr int kQ8Chunk = 16;                  /* blocks per chunk */
constexpr int kQ8PR = kQ8Chunk * 34 / 16;     /* 16-byte pieces per row of a chunk */
/* LDS bytes per row of a chunk slot: the row's 544 bytes and a pad, so
 * that the 16 rows' fragment reads spread over the banks */
constexpr int kQ8Row = 560;
constexpr int kQ8Slot = 16 * kQ8Row;

template <int NC, int XF32, int PD>
__global__ __launch_bounds__(PD == 1 ? 1024 : 512) void q8_0_mfma_kernel(const uint8_t * blocks, int rows, int cols,
                                                                        const void * x, int ldx, int ncol, float * y,
                                                                        int ldy, int accumulate) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int bpr = cols / 32, nch = bpr / kQ8Chunk;
    const size_t rowbytes = (size_t) bpr * 34;
    const int xs = 2 * cols + 16;                                /* LDS bytes per staged column */
    const uint32_t xbytes = (uint32_t) ((XF32 ? 2 : 1) * ncol * xs);
    const int nwv = blockDim.x >> 6;
    uint32_t * xr = (uint32_t *) (lds + xr_off(xbytes + (uint32_t) nwv * kQ8Slot));
    const uint32_t xm = kq_stage_x<XF32, 0, 1>(lds, x, ldx, ncol, cols, xs);
    xr_note_f16(xr, xm);
    __syncthreads();
    const int xk = kq_x_range<XF32, 0, 1>(lds, xr, x, ldx, ncol, cols, xs);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = lane & 15, g = lane >> 4;
    const uint32_t slot = xbytes + (uint32_t) wave * kQ8Slot;
    const int ntiles = (rows + 15) >> 4, nw = gridDim.x * nwv, w0 = blockIdx.x * nwv + wave;
    const int S = (w0 < ntiles ? (ntiles - 1 - w0) / nw + 1 : 0) * nch;   /* chunks this wave streams */
    /* piece p = 64 k + lane of a chunk: row p / kQ8PR of the tile, 16 bytes at 16 (p % kQ8PR) */
    constexpr int NP = (16 * kQ8PR + 63) / 64;
    const bool plast = 64 * (NP - 1) + lane < 16 * kQ8PR;
    u4 R[PD][NP];
    auto load = [&](int s, int b) {
        const int tile = w0 + (s / nch) * nw, c = s - (s / nch) * nch;
        const uint8_t * base = blocks + (size_t) c * (kQ8Chunk * 34);
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int p = 64 * k + lane, pr = p / kQ8PR;
            if (k < NP - 1 || plast) {
                const int row = min(16 * tile + pr, rows - 1);
                R[b][k] = *(const u4 *) (base + (size_t) row * rowbytes + 16 * (p - kQ8PR * pr));
            }
        }
    };
    auto put = [&](int b) {
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int p = 64 * k + lane, pr = p / kQ8PR;
            if (k < NP - 1 || plast) *(u4 *) (lds + slot + (uint32_t) pr * kQ8Row + 16u * (p - kQ8PR * pr)) = R[b][k];
        }
    };
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool xact = NC == 1 ? m == 0 : m < ncol;
    /* the A operand of lanes past the columns stays zero: they never load */
    h8 A = {}, Al = {};
    auto compute = [&](int s) {
        const int tile = w0 + (s / nch) * nw, c = s - (s / nch) * nch;
        const uint32_t wrow = slot + (uint32_t) m * kQ8Row;   /* 16-byte aligned */
        /* blocks 4i .. 4i + 3 of the chunk start 136 bytes apart from a lane
         * base that is a multiple of 8, so each block's quant bytes 8g .. 8g
         * + 7 sit 2, 4, 2 and 0 bytes past a dword: 3, 2, 3 and 2 dword
         * reads, and a fixed shift */
        auto frag = [&](const uint32_t * pw, auto J, uint32_t * q) {
            constexpr int j = decltype(J)::value;
            if constexpr (j == 0 || j == 2) {
                constexpr int o = j == 0 ? 0 : 17;
                const uint32_t a = pw[o], b = pw[o + 1], c2 = pw[o + 2];
                q[0] = __builtin_amdgcn_alignbit(b, a, 16);
                q[1] = __builtin_amdgcn_alignbit(c2, b, 16);
            } else {
                constexpr int o = j == 1 ? 9 : 26;
                q[0] = pw[o];
                q[1] = pw[o + 1];
            }
        };
        auto block = [&](const uint32_t * pw, int bb, auto J) {
            uint32_t qw[2];
            frag(pw, J, qw);
            kq_h2 w0h, w1h, w2h, w3h;
            bytes_to_h2(qw[0] ^ 0x80808080u, (_Float16) 1152.0f, w0h, w1h);
            bytes_to_h2(qw[1] ^ 0x80808080u, (_Float16) 1152.0f, w2h, w3h);
            const h8 B = {w0h[0], w0h[1], w1h[0], w1h[1], w2h[0], w2h[1], w3h[0], w3h[1]};
            const uint32_t xo = (uint32_t) m * xs + 2u * (32u * (kQ8Chunk * c + bb) + 8u * g);
            if (xact) A = *(const h8 *) (lds + xo);
            f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            if (XF32) {
                if (xact) Al = *(const h8 *) (lds + (uint32_t) ncol * xs + xo);
                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, B, D, 0, 0, 0);
            }
            const float d = kq_f16(*(const uint16_t *) (lds + wrow + 34u * (uint32_t) bb));
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = __builtin_fmaf(d, D[e], acc[e]);
        };
        static_assert(kQ8Chunk % 4 == 0, "chunks of whole block quads");
#pragma unroll 1
        for (int b4 = 0; b4 < kQ8Chunk; b4 += 4) {
            /* the lane's dword base, its 8-byte alignment hidden so that the
             * reads stay dword reads (wider unaligned LDS reads measured slower) */
            uint32_t pb = wrow + 8u * g + 34u * (uint32_t) b4;
            asm volatile("" : "+v"(pb));
            const uint32_t * pw = (const uint32_t *) (lds + pb);
            block(pw, b4, std::integral_constant<int, 0>{});
            block(pw, b4 + 1, std::integral_constant<int, 1>{});
            block(pw, b4 + 2, std::integral_constant<int, 2>{});
            block(pw, b4 + 3, std::integral_constant<int, 3>{});
        }
        if (c == nch - 1) {
            const int row = 16 * tile + m;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int n = 4 * g + e;
                if ((NC == 1 ? n == 0 : n < ncol) && row < rows) {
                    float * yp = y + (size_t) n * ldy + row;
                    *yp = (accumulate ? *yp : 0.0f) + xr_unscale(acc[e], xk);
                }
                acc[e] = 0.0f;
            }
        }
    };
#pragma unroll
    for (int b = 0; b < PD; b++)
        if (b < S) load(b, b);
    for (int s = 0; s < S; s += PD) {
#pragma unroll
        for (int b = 0; b < PD; b++) {
            if (s + b < S) {
                put(b);
                if (s + b + PD < S) load(s + b + PD, b);
                compute(s + b);
            }
        }
    }
}

/* ---------------------------------- Q6_K --------------------------------- */

/* A unit is one 128-weight half of a superblock: 64 ql bytes, 32 qh bytes,
 * 8 scales. Weight (quarter k, l) is lo4(ql[l + 32(k&1)] >> 4(k>>1)) |
 * ((qh[l] >> 2k) & 3) << 4, minus 32, times d * scale[l/16 + 2k]. */
template <int NC, int XF32>
__global__ __launch_bounds__(256) void q6k_gemv_kernel(const uint8_t * blocks, int rows, int cols, const void * x,
                                                       int ldx, int ncol, float * y, int ldy, int accumulate) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int bpr = cols / 256, units = 2 * bpr, xst = (cols / 32) * 72 + (cols / 128) * 8;
    uint32_t * xr = (uint32_t *) (lds + xr_off((XF32 ? 2 : 1) * ncol * xst));
    const uint32_t xm = kq_stage_x<XF32, 1>(lds, x, ldx, ncol, cols, xst);
    xr_note_f16(xr, xm);
    __syncthreads();
    const int xk = kq_x_range<XF32, 1>(lds, xr, x, ldx, ncol, cols, xst);
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int row_step = gridDim.x * (blockDim.x >> 6) * 4;
    for (int r0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4; r0 < rows; r0 += row_step) {
        const int row = r0 + g, rowc = min(row, rows - 1);
        float acc[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) acc[n] = 0.0f;
        for (int u = j; u < units; u += 16) {
            const int sb = u >> 1, h = u & 1;
            const uint8_t * blk = blocks + ((size_t) rowc * bpr + sb) * 210;
            const float d = kq_f16(*(const uint16_t *) (blk + 208));
            uint32_t ql[16], qh[8], scw[2];
            load_stream<16>(blk + 64 * h, ql, true);
            load_stream<8>(blk + 128 + 32 * h, qh, true);
            load_stream<2>(blk + 192 + 8 * h, scw, true);
            const int chunk0 = (sb * 256 + 128 * h) >> 5;   /* first 32-column LDS slot of the unit */
#pragma unroll
            for (int k = 0; k < 4; k++) {
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    const int sci = p + 2 * k;
                    const float dsc = d * (float) (int) (int8_t) (scw[sci >> 2] >> (8 * (sci & 3)));
                    kq_h2 qv[8];
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        const int l = 16 * p + 4 * w;   /* four consecutive l in one dword */
                        const uint32_t lo = (ql[(l + 32 * (k & 1)) >> 2] >> (4 * (k >> 1))) & 0x0F0F0F0Fu;
                        const uint32_t hi = ((qh[l >> 2] >> (2 * k)) & 0x03030303u) << 4;
                        bytes_to_h2(lo | hi, (_Float16) 1056.0f, qv[2 * w], qv[2 * w + 1]);
                    }
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        if (n < ncol) {
                            const uint8_t * xp = lds + n * xst + (chunk0 + k) * 72 + (chunk0 >> 2) * 8 + 32 * p;
                            float s = 0.0f;
#pragma unroll
                            for (int w = 0; w < 4; w++) {
                                const kq_h4 xv = *(const kq_h4 *) (xp + 8 * w);
                                s = __builtin_amdgcn_fdot2(qv[2 * w], kq_h2{xv[0], xv[1]}, s, false);
                                s = __builtin_amdgcn_fdot2(qv[2 * w + 1], kq_h2{xv[2], xv[3]}, s, false);
                                if (XF32) {
                                    const kq_h4 xl = *(const kq_h4 *) (xp + ncol * xst + 8 * w);
                                    s = __builtin_amdgcn_fdot2(qv[2 * w], kq_h2{xl[0], xl[1]}, s, false);
                                    s = __builtin_amdgcn_fdot2(qv[2 * w + 1], kq_h2{xl[2], xl[3]}, s, false);
                                }
                            }
                            acc[n] += dsc * s;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NC; n++) {
            if (n < ncol) {
                const float v = xr_unscale(sum16(acc[n]), xk);
                if (j == 0 && row < rows) {
                    float * yp = y + (size_t) n * ldy + row;
                    *yp = (accumulate ? *yp : 0.0f) + v;
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

/* Q6_K, wide form: 32 lanes per row (two rows per wave), every lane issues
 * the loads of all its half superblocks (at most 3, so rows of up to 96
 * half superblocks = 12288 columns) before any of them is used, which keeps
 * a whole row's blocks in flight per wave instead of one at a time. The
 * arithmetic per half superblock is the one of q6k_gemv_kernel. */
template <int NC, int XF32>
__global__ __launch_bounds__(256) void q6k_gemv_wide_kernel(const uint8_t * blocks, int rows, int cols, const void * x,
                                                            int ldx, int ncol, float * y, int ldy, int accumulate) {
    constexpr int NU = 3;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int bpr = cols / 256, units = 2 * bpr, xst = (cols / 32) * 72 + (cols / 128) * 8;
    const int lane = threadIdx.x & 63, j = lane & 31, g = lane >> 5;
    const int row = ((int) blockIdx.x * (int) (blockDim.x >> 6) + (int) (threadIdx.x >> 6)) * 2 + g;
    const int rowc = min(row, rows - 1);
    uint32_t ql[NU][16], qh[NU][8], scw[NU][2];
    float d[NU];
#pragma unroll
    for (int k = 0; k < NU; k++) {
        const int u = min(j + 32 * k, units - 1), sb = u >> 1, h = u & 1;
        const uint8_t * blk = blocks + ((size_t) rowc * bpr + sb) * 210;
        d[k] = kq_f16(*(const uint16_t *) (blk + 208));
        load_stream<16>(blk + 64 * h, ql[k], true);
        load_stream<8>(blk + 128 + 32 * h, qh[k], true);
        load_stream<2>(blk + 192 + 8 * h, scw[k], true);
    }
    /* x after the blocks are requested: both latencies overlap */
    uint32_t * xr = (uint32_t *) (lds + xr_off((XF32 ? 2 : 1) * ncol * xst));
    const uint32_t xm = kq_stage_x<XF32, 1>(lds, x, ldx, ncol, cols, xst);
    xr_note_f16(xr, xm);
    __syncthreads();
    const int xk = kq_x_range<XF32, 1>(lds, xr, x, ldx, ncol, cols, xst);
    float acc[NC];
#pragma unroll
    for (int n = 0; n < NC; n++) acc[n] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < NU; kk++) {
        const int u = j + 32 * kk;
        if (u >= units) continue;
        const int sb = u >> 1, h = u & 1;
        const int chunk0 = (sb * 256 + 128 * h) >> 5;
#pragma unroll
        for (int k = 0; k < 4; k++) {
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const int sci = p + 2 * k;
                const float dsc = d[kk] * (float) (int) (int8_t) (scw[kk][sci >> 2] >> (8 * (sci & 3)));
                kq_h2 qv[8];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const int l = 16 * p + 4 * w;
                    const uint32_t lo = (ql[kk][(l + 32 * (k & 1)) >> 2] >> (4 * (k >> 1))) & 0x0F0F0F0Fu;
                    const uint32_t hi = ((qh[kk][l >> 2] >> (2 * k)) & 0x03030303u) << 4;
                    bytes_to_h2(lo | hi, (_Float16) 1056.0f, qv[2 * w], qv[2 * w + 1]);
                }
#pragma unroll
                for (int n = 0; n < NC; n++) {
                    if (n < ncol) {
                        const uint8_t * xp = lds + n * xst + (chunk0 + k) * 72 + (chunk0 >> 2) * 8 + 32 * p;
                        float sacc = 0.0f;
#pragma unroll
                        for (int w = 0; w < 4; w++) {
                            const kq_h4 xv = *(const kq_h4 *) (xp + 8 * w);
                            sacc = __builtin_amdgcn_fdot2(qv[2 * w], kq_h2{xv[0], xv[1]}, sacc, false);
                            sacc = __builtin_amdgcn_fdot2(qv[2 * w + 1], kq_h2{xv[2], xv[3]}, sacc, false);
                            if (XF32) {
                                const kq_h4 xl = *(const kq_h4 *) (xp + ncol * xst + 8 * w);
                                sacc = __builtin_amdgcn_fdot2(qv[2 * w], kq_h2{xl[0], xl[1]}, sacc, false);
                                sacc = __builtin_amdgcn_fdot2(qv[2 * w + 1], kq_h2{xl[2], xl[3]}, sacc, false);
                            }
                        }
                        acc[n] += dsc * sacc;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NC; n++) {
        if (n < ncol) {
            float v = acc[n];
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
            v = xr_unscale(v, xk);
            if (j == 0 && row < rows) {
                float * yp = y + (size_t) n * ldy + row;
                *yp = (accumulate ? *yp : 0.0f) + v;
            }
        }
    }
}


/* Q6_K, staged form. Compute waves each own one row: a wave copies its row
 * into its own LDS region by 1 KB direct-to-LDS loads and then works it,
 * waiting only for its own copy, so rows that land early are decoded while
 * the others still stream in. Further waves stage x, one batch of loads per
 * lane (a wave that had issued direct-to-LDS loads would wait for them before
 * its own LDS stores). The
 * row is split into units of 32 weights, an 8-wide l range of one half
 * superblock in ggml's layout (l0 .. l0 + 7 of y[l], y[l + 32], y[l + 64],
 * y[l + 96]): 8 units per superblock, five per lane at 10240 columns. Rows
 * are a multiple of 4 bytes and at least 1 KB long, blocks 4-byte aligned
 * (the host checks). Every column gets the same arithmetic whatever the
 * column count. */
/* One 32-weight unit u of the Q6_K row at LDS byte offset row (ggml's
 * block_q6_K: ql, qh, scales, d), against ncol activation columns staged
 * as f16 from LDS offset xoff: acc[n] += d * scale * (q . x) over its four
 * 8-weight groups, in group order. */
template <int NC, int XF32>
__device__ __forceinline__ void q6k_unit(const uint8_t * lds, uint32_t row, int u, uint32_t xoff, int xst, int ncol,
                                         float * acc) {
    const int sb = u >> 3, h = (u >> 2) & 1, l0 = 8 * (u & 3);
    const uint32_t blk = row + (uint32_t) sb * 210u;
    uint32_t qa[2], qb[2], qc[2], scw[2], dw[1];
    lds_stream<2>(lds, blk + 64 * h + l0, qa);
    lds_stream<2>(lds, blk + 64 * h + 32 + l0, qb);
    lds_stream<2>(lds, blk + 128 + 32 * h + l0, qc);
    lds_stream<2>(lds, blk + 192 + 8 * h, scw);
    lds_stream<1>(lds, blk + 208, dw);
    const float d = kq_f16((uint16_t) dw[0]);
    const int e0 = 256 * sb + 128 * h + l0;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int sci = (l0 >> 4) + 2 * g;
        const float dsc = d * (float) (int) (int8_t) (scw[sci >> 2] >> (8 * (sci & 3)));
        kq_h2 qv[4];
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t lo = ((g & 1 ? qb[w] : qa[w]) >> (4 * (g >> 1))) & 0x0F0F0F0Fu;
            const uint32_t hi = ((qc[w] >> (2 * g)) & 0x03030303u) << 4;
            bytes_to_h2(lo | hi, (_Float16) 1056.0f, qv[2 * w], qv[2 * w + 1]);
        }
        const int e = e0 + 32 * g;
        const int xo = (e >> 5) * 72 + (e >> 7) * 8 + 2 * (e & 31);
#pragma unroll
        for (int n = 0; n < NC; n++) {
            if (n < ncol) {
                const uint8_t * xp = lds + xoff + n * xst + xo;
                float sacc = 0.0f;
#pragma unroll
                for (int w = 0; w < 2; w++) {
                    const kq_h4 xv = *(const kq_h4 *) (xp + 8 * w);
                    sacc = __builtin_amdgcn_fdot2(qv[2 * w], kq_h2{xv[0], xv[1]}, sacc, false);
                    sacc = __builtin_amdgcn_fdot2(qv[2 * w + 1], kq_h2{xv[2], xv[3]}, sacc, false);
                    if (XF32) {
                        const kq_h4 xl = *(const kq_h4 *) (xp + ncol * xst + 8 * w);
                        sacc = __builtin_amdgcn_fdot2(qv[2 * w], kq_h2{xl[0], xl[1]}, sacc, false);
                        sacc = __builtin_amdgcn_fdot2(qv[2 * w + 1], kq_h2{xl[2], xl[3]}, sacc, false);
                    }
                }
                acc[n] += dsc * sacc;
            }
        }
    }
}

template <int NC, int XF32, int RPV>
__global__ __launch_bounds__(1024) void q6k_gemv_staged_kernel(const uint8_t * blocks, int rows, int cols,
                                                                const void * x, int ldx, int ncol, float * y, int ldy,
                                                                int accumulate, int rpw) {
    constexpr int rpv = RPV;
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int bpr = cols / 256, units = 8 * bpr, xst = (cols / 32) * 72 + (cols / 128) * 8;
    const uint32_t rowbytes = (uint32_t) bpr * 210;
    const int nrw = (rpw + rpv - 1) / rpv;                     /* waves with rows; waves nrw .. stage x */
    const int xw = (blockDim.x >> 6) - nrw;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = blockIdx.x * rpw, nrow = min(rpw, rows - row0);
    const int wr0 = wv * rpv, wnr = min(rpv, nrow - wr0);     /* this wave's first row in the workgroup, its row count */
    const uint32_t xoff = (uint32_t) ((rpw * rowbytes + 15) & ~15u);
    const uint32_t reg = (uint32_t) wr0 * rowbytes;           /* this wave's rows, a byte offset in LDS */
    uint32_t * xr = (uint32_t *) (lds + xoff + xr_off((XF32 ? 2 : 1) * ncol * xst));
    uint32_t xm = 0;
    if (wv >= nrw) {
        /* x: the x waves' loads, LDS stores and range flags, complete
         * before the barrier */
        xm = kq_stage_x_by<XF32, 1>(lds + xoff, x, ldx, ncol, cols, xst, threadIdx.x - 64 * nrw, 64 * xw);
        xr_note_f16(xr, xm);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else if (wnr > 0) {
        /* the wave's rows are contiguous, in memory and in LDS */
        const uint32_t bytes = (uint32_t) wnr * rowbytes;
        const uint8_t * src = blocks + (size_t) (row0 + wr0) * rowbytes;
        const int nchunk = (int) ((bytes + 1023) >> 10);
        for (int b = 0; b < nchunk; b++) {
            const uint32_t o = min((uint32_t) b * 1024u, bytes - 1024u);   /* the last chunk overlaps its neighbour */
            __builtin_amdgcn_global_load_lds((const void *) (src + o + 16 * lane), (lds_void *) (lds + reg + o), 16, 0, 0);
        }
    }
    /* x is in LDS after this barrier. An execution barrier only (the asm
     * keeps the compiler from moving LDS reads above it): no wave waits for
     * its row copy here. */
    asm volatile("s_barrier" ::: "memory");
    /* every wave takes the (uniform) range decision before any leaves */
    const int xk = kq_x_range<XF32, 1>(lds + xoff, xr, x, ldx, ncol, cols, xst, nrw);
    if (wnr <= 0) return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   /* this wave's rows */
    /* rpv rows per wave, each on L = 64 / rpv lanes; the lane l of its row's
     * L takes units l, l + L, ..., k = rpv * units / 64 of them (the host
     * picks rpv so that k is whole), so every lane has the same work. With
     * one row per wave that is units lane, lane + 64, ... */
    constexpr int L = 64 / RPV;
    const int k = RPV * units / 64;
    const int rl = lane / L, ul = lane - rl * L;
    const bool live = rl < wnr;
    const uint32_t rreg = reg + (uint32_t) (live ? rl : 0) * rowbytes;
    float acc[NC];
#pragma unroll
    for (int n = 0; n < NC; n++) acc[n] = 0.0f;
    if (live)
        for (int i = 0; i < k; i++) q6k_unit<NC, XF32>(lds, rreg, ul + L * i, xoff, xst, ncol, acc);
#pragma unroll
    for (int n = 0; n < NC; n++) {
        if (n < ncol) {
            float v = acc[n];
#pragma unroll
            for (int o = L >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
            v = xr_unscale(v, xk);
            if (live && lane == rl * L) {
                float * yp = y + (size_t) n * ldy + row0 + wr0 + rl;
                *yp = (accumulate ? *yp : 0.0f) + v;
            }
        }
    }
}

static inline const uint8_t * bp_in(const void * p) { return (const uint8_t *) p; }

/* Rows per wave of the staged kernel: the fewest that give its 64 lanes a
 * whole, equal number of 32-weight units (8 per 256 columns): 4 rows of
 * 2560 columns (80 units each, 5 per lane), 1 of 4096 or 10240. */
static int q6k_rows_per_wave(int cols) {
    const int units = 8 * (cols / 256);
    int g = 64;
    while (units % g) g >>= 1;
    return 64 / g;
}

template <int NC, int XF32, int RPV>
static int kq_q6k_staged_k(const uint8_t * bp, int rows, int cols, const void * x, int ldx, int ncol, float * y,
                           int ldy, int accumulate, int rpw, size_t lds, hipStream_t s) {
    static size_t opted = 0;
    const void * fn = (const void *) q6k_gemv_staged_kernel<NC, XF32, RPV>;
    if (lds > 65536 && lds > opted) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return fail_hip("LDS opt-in for the staged Q6_K kernel", e);
        opted = lds;
    }
    /* x waves: enough for one batch of eight 16-byte groups per lane, within 16 waves */
    const int nrw = (rpw + RPV - 1) / RPV;
    int xw = (ncol * cols + 4095) / 4096;
    xw = xw < 1 ? 1 : (xw > 16 - nrw ? 16 - nrw : xw);
    const dim3 grid((unsigned) ((rows + rpw - 1) / rpw)), block((unsigned) (64 * (nrw + xw)));
    launch_kernel(q6k_gemv_staged_kernel<NC, XF32, RPV>, grid, block, (uint32_t) lds, s, bp, rows, cols, x, ldx, ncol, y,
                  ldy, accumulate, rpw);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("staged Q6_K launch", e);
}

template <int NC, int XF32>
static int kq_q6k_staged_r(const uint8_t * bp, int rows, int cols, const void * x, int ldx, int ncol, float * y,
                           int ldy, int accumulate, int rpw, size_t lds, hipStream_t s) {
    switch (q6k_rows_per_wave(cols)) {
        case 1: return kq_q6k_staged_k<NC, XF32, 1>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s);
        case 2: return kq_q6k_staged_k<NC, XF32, 2>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s);
        default: return kq_q6k_staged_k<NC, XF32, 4>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s);
    }
}

template <int XF32>
static int kq_q6k_staged_t(const uint8_t * bp, int rows, int cols, const void * x, int ldx, int ncol, float * y,
                           int ldy, int accumulate, int rpw, size_t lds, hipStream_t s) {
    if (ncol == 1) return kq_q6k_staged_r<1, XF32>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s);
    if (ncol <= 4) return kq_q6k_staged_r<4, XF32>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s);
    return kq_q6k_staged_r<16, XF32>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s);
}

static int kq_q6k_staged(const uint8_t * bp, int rows, int cols, const void * x, int xf32, int ldx, int ncol, float * y,
                         int ldy, int accumulate, int rpw, size_t lds, hipStream_t s) {
    return xf32 ? kq_q6k_staged_t<1>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s)
                : kq_q6k_staged_t<0>(bp, rows, cols, x, ldx, ncol, y, ldy, accumulate, rpw, lds, s);
}

/* The matrix-core Q8_0 kernel: rows of whole 16-block chunks (cols a multiple
 * of 512) from a 16-byte aligned buffer. Waves per workgroup: as many
 * 8960-byte row slots as fit beside x, in fours, at most 16; one workgroup
 * per CU, each wave a strided share of the 16-row tiles. Returns 1 when the
 * shape does not fit it. */
template <int NC, int XF32, int PD>
static int kq_q8_mfma_k(const uint8_t * bp, int rows, int cols, const void * x, int ldx, int ncol, float * y, int ldy,
                        int accumulate, int nwv, int persist, size_t lds, hipStream_t s) {
    static std::atomic<size_t> opted{0};
    const void * fn = (const void *) q8_0_mfma_kernel<NC, XF32, PD>;
    if (lds > 65536 && lds > opted.load()) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return fail_hip("LDS opt-in for the matrix-core Q8_0 kernel", e);
        opted.store(lds);
    }
    const int ntiles = (rows + 15) / 16;
    int grid = (ntiles + nwv - 1) / nwv;
    if (persist && grid > cu_count()) grid = cu_count();
    launch_kernel(q8_0_mfma_kernel<NC, XF32, PD>, dim3((unsigned) grid), dim3((unsigned) (64 * nwv)), (uint32_t) lds, s,
                  bp, rows, cols, x, ldx, ncol, y, ldy, accumulate);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("matrix-core Q8_0 launch", e);
}

/* The matrix-core Q8_0 GEMV for rows of whole 16-block chunks (cols a
 * multiple of 512) in a 16-byte aligned buffer; returns 1 when the shape
 * does not fit it. Columns per launch: as many as fit LDS beside four row
 * slots; a shape where one column does not fit never takes this kernel, and
 * wider launches go in groups, so every column count of a shape gets the
 * same arithmetic. Launch shapes (measured on the 151936 x 2560 head):
 *  - one column: eight waves per workgroup, one 16-row tile per wave, the
 *    next chunk's loads in flight (78.0-78.5 us; before the block quads,
 *    80.5 against whole-grid persistent waves 82.5-84.5, two tiles per wave
 *    91.6 and two chunks ahead 85);
 *  - several columns: at most one workgroup of eight waves per CU, each
 *    wave a strided share of the tiles, two chunks ahead (8 columns:
 *    88.4-89.2 us; one tile per wave would stage 41 KB of x per tile;
 *    twelve waves, whose slots LDS also holds, 103.5 us). */
static int kq_q8_mfma(const uint8_t * bp, int rows, int cols, const void * x, int xf32, int ldx, int ncol, float * y,
                      int ldy, int accumulate, hipStream_t s) {
    if (cols % (32 * kQ8Chunk) || ((uintptr_t) bp & 15u)) return 1;
    const size_t xcol = (size_t) (xf32 ? 2 : 1) * (2 * cols + 16);
    const size_t room = 160 * 1024 - kXrBytes - 16;
    if (xcol + 4 * (size_t) kQ8Slot > room) return 1;
    const int gmax = (int) ((room - 4 * (size_t) kQ8Slot) / xcol);
    for (int n0 = 0; n0 < ncol; n0 += gmax) {
        const int nc = ncol - n0 < gmax ? ncol - n0 : gmax;
        const size_t xbytes = (size_t) nc * xcol;
        int nwv = (int) ((room - xbytes) / kQ8Slot);
        nwv = nwv > 8 ? 8 : nwv & ~3;
        const size_t lds = xr_off((uint32_t) (xbytes + (size_t) nwv * kQ8Slot)) + kXrBytes;
        const void * xg = (const uint8_t *) x + (size_t) n0 * ldx * (xf32 ? 4 : 2);
        float * yg = y + (size_t) n0 * ldy;
        int rc;
        if (nc == 1)
            rc = xf32 ? kq_q8_mfma_k<1, 1, 1>(bp, rows, cols, xg, ldx, nc, yg, ldy, accumulate, nwv, 0, lds, s)
                      : kq_q8_mfma_k<1, 0, 1>(bp, rows, cols, xg, ldx, nc, yg, ldy, accumulate, nwv, 0, lds, s);
        else
            rc = xf32 ? kq_q8_mfma_k<16, 1, 2>(bp, rows, cols, xg, ldx, nc, yg, ldy, accumulate, nwv, 1, lds, s)
                      : kq_q8_mfma_k<16, 0, 2>(bp, rows, cols, xg, ldx, nc, yg, ldy, accumulate, nwv, 1, lds, s);
        if (rc) return rc;
    }
    return 0;
}

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
    if (kind == 8) {
        /* the matrix cores where the shape allows (any column count) */
        const int mr = kq_q8_mfma((const uint8_t *) blocks, rows, cols, x, xf32, ldx, ncol, y, ldy, accumulate, s);
        if (mr != 1) return mr;
    }
    const int threads = 256;
    const int rows_per_block = (threads / 64) * 4;
    /* Q6_K slots carry 8 bytes of pad per 128 columns */
    const size_t lds = (size_t) (xf32 ? 2 : 1) * ncol * ((cols / 32) * 72 + (kind == 6 ? (cols / 128) * 8 : 0)) +
                       kXrBytes;
    if (lds > 160 * 1024) { set_error("%d activation columns of %d do not fit LDS", ncol, cols); return -1; }
    int grid = (rows + rows_per_block - 1) / rows_per_block;
    const int cap = cu_count() * 16;
    if (grid > cap) grid = cap;
    const uint8_t * bp = (const uint8_t *) blocks;
#define KQ_LAUNCH(K, NC, XF) launch_kernel(K<NC, XF>, dim3(grid), dim3(threads), (uint32_t) lds, s, bp, rows, cols, x, \
                                           ldx, ncol, y, ldy, accumulate)
#define KQ_PICK(K, XF)                          \
    do {                                        \
        if (ncol == 1) KQ_LAUNCH(K, 1, XF);     \
        else if (ncol <= 4) KQ_LAUNCH(K, 4, XF); \
        else if (ncol <= 8) KQ_LAUNCH(K, 8, XF); \
        else KQ_LAUNCH(K, 16, XF);              \
    } while (0)
    if (kind == 6 && cols >= 1280 && cols <= 16384 && (cols / 256) % 2 == 0 && !((uintptr_t) blocks & 3) &&
        !(xf32 && ncol > 4)) {
        /* rows per workgroup: about one workgroup per CU, one row per wave
         * (rows of at least 1 KB, the size of one copy) plus the wave that
         * stages x, the rows' blocks and x within LDS */
        const size_t rowbytes = (size_t) (cols / 256) * 210;
        const size_t xbytes = (size_t) (xf32 ? 2 : 1) * ncol * ((cols / 32) * 72 + (cols / 128) * 8) + kXrBytes;
        const int rpv = q6k_rows_per_wave(cols);
        int rpw = (rows + cu_count() - 1) / cu_count();
        rpw = rpw < 2 ? 2 : (rpw > 12 ? 12 : rpw);
        rpw = (rpw + rpv - 1) / rpv * rpv;
        while (rpw > rpv && ((rpw * rowbytes + 15) & ~(size_t) 15) + xbytes > 160 * 1024) rpw -= rpv;
        const size_t slds = ((rpw * rowbytes + 15) & ~(size_t) 15) + xbytes;
        if (slds <= 160 * 1024) {
            return kq_q6k_staged(bp_in(blocks), rows, cols, x, xf32, ldx, ncol, y, ldy, accumulate, rpw, slds, s);
        }
    }
    if (kind == 6 && cols <= 12288) {
        /* eight rows per workgroup, every row's blocks requested at once */
        grid = (rows + 7) / 8;
        if (xf32) KQ_PICK(q6k_gemv_wide_kernel, 1);
        else KQ_PICK(q6k_gemv_wide_kernel, 0);
    } else if (kind == 6) {
        if (xf32) KQ_PICK(q6k_gemv_kernel, 1);
        else KQ_PICK(q6k_gemv_kernel, 0);
    } else if (ncol == 1) {
        /* one pass of 16 rows per workgroup, no cap: measured 75.8 against
         * 78.3 us for the 151936-row head with 16 workgroups per CU looping */
        grid = (rows + rows_per_block - 1) / rows_per_block;
        if (xf32) KQ_LAUNCH(q8_0_gemv_kernel, 1, 1);
        else KQ_LAUNCH(q8_0_gemv_kernel, 1, 0);
    } else {
        /* four rows per lane: 64 rows per workgroup */
        grid = (rows + 63) / 64;
        if (grid > cap) grid = cap;
#define KQ_LAUNCH4(NC, XF) launch_kernel(q8_0_gemv_kernel<NC, XF, 4>, dim3(grid), dim3(threads), (uint32_t) lds, s, bp, \
                                         rows, cols, x, ldx, ncol, y, ldy, accumulate)
        if (xf32) {
            if (ncol <= 4) KQ_LAUNCH4(4, 1);
            else if (ncol <= 8) KQ_LAUNCH4(8, 1);
            else KQ_LAUNCH4(16, 1);
        } else {
            if (ncol <= 4) KQ_LAUNCH4(4, 0);
            else if (ncol <= 8) KQ_LAUNCH4(8, 0);
            else KQ_LAUNCH4(16, 0);
        }
#undef KQ_LAUNCH4
    }
#undef KQ_PICK
#undef KQ_LAUNCH
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
