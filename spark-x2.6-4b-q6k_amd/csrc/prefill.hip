/* prefill.hip — VQ GEMM for prompt prefill (many tokens against one matrix).
 *
 * Computes, for every token t and row r, y[t][r] (+)= sum_s g_s[r] * sum_i
 * cb_s[idx_s(r, i)] . x[t][dim*i ..] — the reference's per-token GEMV summed
 * over stages (tools/vq/gpu/decode-gpu.cu:359-501 is its tiled form).
 *
 * prefill_cw_kernel: the DQV3 dim-4 GEMM on the matrix cores with the
 * codewords gathered straight into the MFMA operands (no weight tile in LDS),
 * 256 rows x 128 tokens per workgroup, split K for short matrices. It takes
 * every MFMA-shaped call whose LDS fits.
 *
 * prefill_mfma_kernel: the same GEMM through a decoded f16 weight tile in
 * LDS (64 or 128 rows x 128 tokens); it takes what the codeword kernel's LDS
 * does not fit (two stages of an 8192-entry codebook) and y rows that are not
 * 16-byte aligned.
 *
 * prefill_simple_kernel: one thread per (row, token), the row's indices staged
 * in LDS; any geometry and any x layout (strided), f32 arithmetic. It backs
 * variant 3 of the reference-compatible prefill entry points and every call
 * the MFMA kernel does not take.
 */
#include "prefill.h"

#include <string.h>

#include <atomic>
#include <mutex>

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

/* ------------------------------------------------------------------------ */
/* MFMA prefill                                                              */
/* ------------------------------------------------------------------------ */

typedef _Float16 pf_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 pf_h8 __attribute__((ext_vector_type(8)));
typedef float pf_f4 __attribute__((ext_vector_type(4)));
typedef float pf_f16v __attribute__((ext_vector_type(16)));
typedef uint32_t pf_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t pf_u4a __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kPR = 128;   /* rows per workgroup tile (the larger of the two tile heights) */
constexpr int kPT = 128;   /* tokens per workgroup tile */
constexpr int kPK = 64;    /* columns per chunk */
constexpr int kPS = 72;    /* LDS row stride of a tile in halves (64 + 8 pad: conflict-free 16-byte reads) */

struct MfmaArgs {
    const uint8_t * st[2];
    const void * x;      /* token-major: x[t * ldx + k], bf16 bits or f32; K-major (XT): f32 x[k * ldx + t] */
    float * y;           /* y[t * ldy + r] */
    int rows, cols, nc, ntok, ldx, ldy, accumulate;
    uint32_t gain_off, stream_off, mrow, prow;
};

/* field j of 8 12-bit fields packed LSB-first in three words */
__device__ __forceinline__ uint32_t pf_field12(uint32_t w0, uint32_t w1, uint32_t w2, int j) {
    switch (j) {
        case 0: return w0 & 0xfffu;
        case 1: return (w0 >> 12) & 0xfffu;
        case 2: return __builtin_amdgcn_alignbit(w1, w0, 24) & 0xfffu;
        case 3: return (w1 >> 4) & 0xfffu;
        case 4: return (w1 >> 16) & 0xfffu;
        case 5: return __builtin_amdgcn_alignbit(w2, w1, 28) & 0xfffu;
        case 6: return (w2 >> 8) & 0xfffu;
        default: return w2 >> 20;
    }
}

constexpr int kPThreads = 512;   /* 8 waves: two per SIMD, so one wave's decode hides another's latency */

template <int NST, int EXT, int XF32, int PF, int XT, int RT>
__global__ __launch_bounds__(kPThreads) void prefill_mfma_kernel(const MfmaArgs P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t cbb = (uint32_t) P.nc * 8u;
    _Float16 * At = (_Float16 *) (lds + NST * cbb);   /* [2][RT][kPS] decoded weights */
    _Float16 * Bt = At + 2 * RT * kPS;                 /* [2][kPT][kPS] tokens */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * RT, t0 = blockIdx.y * kPT;
    const int nk = P.cols / kPK;

    /* codebooks to LDS in batches of unconditional 16-byte loads */
    {
        const int n16 = (int) (cbb >> 4), ncb = NST * n16;
        for (int base = 0; base < ncb; base += 4 * kPThreads) {
            pf_u4 v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = min(base + k * kPThreads + tid, ncb - 1), s = i >= n16 ? 1 : 0;
                v[k] = ((const pf_u4a *) (P.st[NST > 1 ? s : 0] + 24))[i - s * n16];
            }
#pragma unroll
            for (int k = 0; k < 4; k++) ((pf_u4 *) lds)[min(base + k * kPThreads + tid, ncb - 1)] = v[k];
        }
    }

    /* decode role: row dr of the tile, IPT indices (4 IPT columns) of a chunk
     * per thread, TPR threads per row: bits 12 IPT h .. of the chunk's 24
     * stream bytes, from the dword holding the first of them (and the next
     * one within the chunk), shifted into place */
    constexpr int TPR = kPThreads / RT, IPT = 16 / TPR;
    const int dr = tid / TPR, h = tid % TPR;
    const int drow = min(r0 + dr, P.rows - 1);
    const int wo = (3 * IPT * h) >> 1;                 /* byte of the first index */
    const int wd = wo >> 2, wd1 = min(wd + 1, 5);
    const uint32_t wsh = (uint32_t) (wo & 3) * 8u;
    /* x role (token-major): token xt of the tile, columns 16 xh .. 16 xh + 15 */
    const int xtk = tid >> 2, xh = tid & 3;
    const int dtok = min(t0 + xtk, P.ntok - 1);
    float g[NST];
    const uint32_t * rs[NST];
    const uint8_t * ps[NST];
#pragma unroll
    for (int s = 0; s < NST; s++) {
        g[s] = (float) *(const _Float16 *) (P.st[s] + P.gain_off + 2 * (size_t) drow);
        rs[s] = (const uint32_t *) (P.st[s] + P.stream_off + (size_t) drow * P.mrow) + wd;
        ps[s] = P.st[s] + P.stream_off + (size_t) P.rows * P.mrow + (size_t) drow * P.prow + ((IPT * h) >> 3);
    }
    const uint8_t * xr = (const uint8_t *) P.x + ((size_t) dtok * P.ldx + 16 * xh) * (XF32 ? 4 : 2);
    /* K-major x role (the reference's xT[cols][ntok]): tokens 4 tq .. 4 tq + 3
     * of the tile, columns 4 cg .. 4 cg + 3 of a chunk; lanes run along the
     * tokens, so each 16-byte load of a wave reads 512 contiguous bytes */
    const int tq = tid & 31, cg = tid >> 5;
    const float * xk = (const float *) P.x + (size_t) (4 * cg) * P.ldx + min(t0 + 4 * tq, P.ntok - 4);

    /* PF chunks of index words and x in flight: a ring of register slots,
     * slot kc % PF holding chunk kc until it is decoded */
    constexpr int NXV = XT ? 4 : (XF32 ? 4 : 2);
    uint32_t wv[PF][NST][2], pb[PF][NST];
    pf_u4 xv[PF][NXV];
    auto fetch = [&](int kc, int sl) {
#pragma unroll
        for (int s = 0; s < NST; s++) {
            wv[sl][s][0] = rs[s][6 * kc];
            wv[sl][s][1] = rs[s][6 * kc + wd1 - wd];
            pb[sl][s] = EXT ? ps[s][2 * kc] : 0u;
        }
        if constexpr (XT) {
#pragma unroll
            for (int k = 0; k < NXV; k++) xv[sl][k] = *(const pf_u4 *) (xk + (size_t) (kPK * kc + k) * P.ldx);
        } else {
#pragma unroll
            for (int k = 0; k < NXV; k++) xv[sl][k] = ((const pf_u4 *) (xr + kPK * kc * (XF32 ? 4 : 2)))[k];
        }
    };
    auto store = [&](int b, int sl) {
        pf_h8 w8[IPT / 2];
#pragma unroll
        for (int j = 0; j < IPT; j++) {
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NST; s++) {
                const uint32_t lo = __builtin_amdgcn_alignbit(wv[sl][s][1], wv[sl][s][0], wsh);
                const uint32_t hi = wv[sl][s][1] >> wsh;
                uint32_t idx = j == 0 ? lo : j == 1 ? lo >> 12 : j == 2 ? __builtin_amdgcn_alignbit(hi, lo, 24) : hi >> 4;
                idx &= 0xfffu;
                if (EXT) idx |= ((pb[sl][s] >> ((IPT * h) % 8 + j)) & 1u) << 12;
                const pf_h4 c = *(const pf_h4 *) (lds + s * cbb + 8 * idx);
#pragma unroll
                for (int d = 0; d < 4; d++) acc[d] = __builtin_fmaf((float) c[d], g[s], acc[d]);
            }
#pragma unroll
            for (int d = 0; d < 4; d++) w8[j >> 1][4 * (j & 1) + d] = (_Float16) acc[d];
        }
        _Float16 * ad = At + (b * RT + dr) * kPS + 4 * IPT * h;
#pragma unroll
        for (int k = 0; k < IPT / 2; k++) *(pf_h8 *) (ad + 8 * k) = w8[k];
        if constexpr (XT) {
            /* xv[c] holds tokens 4 tq .. +3 of column 4 cg + c: four
             * columns (8 bytes) per token */
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pf_h4 v4;
#pragma unroll
                for (int c = 0; c < 4; c++) v4[c] = (_Float16) __uint_as_float(xv[sl][c][i]);
                *(pf_h4 *) (Bt + (b * kPT + 4 * tq + i) * kPS + 4 * cg) = v4;
            }
            return;
        }
        _Float16 * bd = Bt + (b * kPT + xtk) * kPS + 16 * xh;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            pf_h8 v8;
            if (XF32) {
                const pf_u4 lo = xv[sl][2 * k], hi = xv[sl][2 * k + 1];
                v8[0] = (_Float16) __uint_as_float(lo.x); v8[1] = (_Float16) __uint_as_float(lo.y);
                v8[2] = (_Float16) __uint_as_float(lo.z); v8[3] = (_Float16) __uint_as_float(lo.w);
                v8[4] = (_Float16) __uint_as_float(hi.x); v8[5] = (_Float16) __uint_as_float(hi.y);
                v8[6] = (_Float16) __uint_as_float(hi.z); v8[7] = (_Float16) __uint_as_float(hi.w);
            } else {
                const pf_u4 q = xv[sl][k];
                v8[0] = (_Float16) __uint_as_float(q.x << 16); v8[1] = (_Float16) __uint_as_float(q.x & 0xffff0000u);
                v8[2] = (_Float16) __uint_as_float(q.y << 16); v8[3] = (_Float16) __uint_as_float(q.y & 0xffff0000u);
                v8[4] = (_Float16) __uint_as_float(q.z << 16); v8[5] = (_Float16) __uint_as_float(q.z & 0xffff0000u);
                v8[6] = (_Float16) __uint_as_float(q.w << 16); v8[7] = (_Float16) __uint_as_float(q.w & 0xffff0000u);
            }
            *(pf_h8 *) (bd + 8 * k) = v8;
        }
    };

    /* MFMA role: wave (wm, wn) owns rows RT/2 wm .. + RT/2 - 1 and tokens
     * 32 wn .. +31 of the tile as NB blocks of 32 x 32 (v_mfma_f32_32x32x16_f16: each
     * operand element serves 32 outputs, half the LDS reads of 16 x 16
     * blocks). A lane's operand is 8 consecutive columns of one row (A) or
     * one token (B); A and B assign columns to lanes the same way, so each
     * block is a plain dot over the chunk's columns. */
    constexpr int NB = RT / 64;
    const int wm = wave & 1, wn = wave >> 1, m32 = lane & 31, kh = lane >> 5;
    pf_f16v acc[NB];
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][e] = 0.0f;

    __syncthreads();   /* codebooks staged */
#pragma unroll
    for (int u = 0; u < PF; u++) fetch(min(u, nk - 1), u);
    store(0, 0);
    __syncthreads();
    /* nk is a multiple of PF (even), so chunk kc0 + u uses buffer u & 1 and
     * slot u; the body has no branches (chunks past the end are clamped and
     * their decode lands in a buffer nobody reads), so the compiler counts
     * the ring's loads exactly across iterations */
    for (int kc0 = 0; kc0 < nk; kc0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int kc = kc0 + u, b = u & 1;
            /* keep each chunk's decode in its own step: hoisted above, it
             * would wait for loads that are meant to stay in flight */
            __builtin_amdgcn_sched_barrier(0);
            fetch(min(kc + PF, nk - 1), u);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                pf_h8 a[NB];
#pragma unroll
                for (int i = 0; i < NB; i++)
                    a[i] = *(const pf_h8 *) (At + (b * RT + (RT / 2) * wm + 32 * i + m32) * kPS + 16 * ks + 8 * kh);
                const pf_h8 bb = *(const pf_h8 *) (Bt + (b * kPT + 32 * wn + m32) * kPS + 16 * ks + 8 * kh);
#pragma unroll
                for (int i = 0; i < NB; i++) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bb, acc[i], 0, 0, 0);
            }
            store(b ^ 1, (u + 1) % PF);
            __syncthreads();
        }
    }

    /* block i: entry e of a lane is row 8 (e / 4) + 4 kh + e % 4 of the
     * block, token m32 */
    const int tok = t0 + 32 * wn + m32;
    if (tok < P.ntok) {
#pragma unroll
        for (int i = 0; i < NB; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = r0 + (RT / 2) * wm + 32 * i + 8 * (e >> 2) + 4 * kh + (e & 3);
                if (row < P.rows) {
                    float * yp = P.y + (size_t) tok * P.ldy + row;
                    *yp = (P.accumulate ? *yp : 0.0f) + acc[i][e];
                }
            }
    }
}

/* ------------------------------------------------------------------------ */
/* Codeword-operand MFMA prefill                                             */
/* ------------------------------------------------------------------------ */

/* prefill_cw_kernel: the same GEMM with no decoded weight tile. Since a row's
 * gain is constant along the row, sum_k (g0 c0_k + g1 c1_k) x_k =
 * g0 (c0 . x) + g1 (c1 . x): each stage's f16 codewords go straight from the
 * LDS codebook into the A operand of v_mfma_f32_32x32x16_f16 (a lane's 8
 * columns are two dim-4 codewords), each stage accumulates in its own f32
 * registers, and the gains are applied once in the epilogue (the decode
 * GEMV's form, exact codewords, no rounding of W). Two stages instead fold
 * in the lane that gathered them: W = g0 c0 + g1 c1 in f32 (one rounding,
 * the reference decode's rule) rounded to f16, one MFMA per block. Either
 * way a weight costs one LDS gather per stage and no trip through an LDS
 * weight tile.
 *
 * A workgroup owns 256 rows x 128 tokens: wave w owns rows 32 w .. 32 w + 31
 * against all 128 tokens (four 32 x 32 blocks), so every codeword is gathered
 * once per workgroup, and the token tile (f16, staged by all threads, three
 * buffers) is shared by the eight waves. The columns a lane
 * reads are permuted so that its index words are contiguous: for MFMA step
 * ks, lane half kh takes codewords 8 kh + 2 ks and 8 kh + 2 ks + 1 of the
 * 16-codeword chunk, i.e. columns 32 kh + 8 ks .. + 7, on the A and the B side
 * alike. Lane half kh therefore needs the three dwords at byte 12 kh of the
 * row's 24-byte chunk (and bits 8 kh .. 8 kh + 7 of its 13th-bit plane).
 *
 * Split K (grid z): when the row and token tiles alone leave the CUs idle
 * (the 2560-row matrix), each split covers nkc consecutive chunks and writes
 * its partial sums to its own slice of a workspace; prefill_cw_reduce then
 * adds the slices in split order, so the result does not depend on timing. */
constexpr int kCT = 128;            /* tokens per workgroup tile */
constexpr int kCR = 256;            /* rows per workgroup tile: 8 waves x 32 */
constexpr int kCThreads = 512;

struct CwArgs {
    const uint8_t * st[2];
    const void * x;      /* token-major: x[t * ldx + k], bf16 bits or f32; K-major (XT): f32 x[k * ldx + t] */
    float * y;           /* y[t * ldy + r]; split z writes y + z * ysplit */
    size_t ysplit;
    int rows, cols, nc, ntok, ldx, ldy, accumulate, nkc;
    uint32_t gain_off, stream_off, mrow, prow;
};

template <int NST, int EXT, int XF32, int XT, int FOLD>
__global__ __launch_bounds__(kCThreads) void prefill_cw_kernel(const CwArgs P) {
    /* FOLD (two stages): W = g0 c0 + g1 c1 formed in f32 (one rounding) and
     * rounded to f16 in the lane that feeds it to the MFMA, one accumulator
     * set; else each stage's exact codewords accumulate apart and the gains
     * apply in the epilogue */
    constexpr int NA = FOLD ? 1 : NST;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t cbb = (uint32_t) P.nc * 8u;
    _Float16 * Bt = (_Float16 *) (lds + NST * cbb);   /* [3][kCT][kPS] tokens */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m32 = lane & 31, kh = lane >> 5;
    const int r0 = blockIdx.x * kCR, t0 = blockIdx.y * kCT;
    const int kcb = blockIdx.z * P.nkc;               /* this split's first chunk */
    const int nkc = P.nkc;

    /* codebooks to LDS in batches of unconditional 16-byte loads */
    {
        const int n16 = (int) (cbb >> 4), ncb = NST * n16;
        for (int base = 0; base < ncb; base += 4 * kCThreads) {
            pf_u4 v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = min(base + k * kCThreads + tid, ncb - 1), s = i >= n16 ? 1 : 0;
                v[k] = ((const pf_u4a *) (P.st[NST > 1 ? s : 0] + 24))[i - s * n16];
            }
#pragma unroll
            for (int k = 0; k < 4; k++) ((pf_u4 *) lds)[min(base + k * kCThreads + tid, ncb - 1)] = v[k];
        }
    }

    /* A role: row arow of the tile; per chunk, three index dwords per stage */
    const int arow = min(r0 + 32 * wave + m32, P.rows - 1);
    const uint32_t * rs[NST];
    const uint8_t * ps[NST];
#pragma unroll
    for (int s = 0; s < NST; s++) {
        rs[s] = (const uint32_t *) (P.st[s] + P.stream_off + (size_t) arow * P.mrow) + 6 * kcb + 3 * kh;
        ps[s] = P.st[s] + P.stream_off + (size_t) P.rows * P.mrow + (size_t) arow * P.prow + 2 * kcb + kh;
    }
    /* x role (token-major): token xtk of the tile, columns 16 xh .. 16 xh + 15 */
    const int xtk = tid >> 2, xh = tid & 3;
    const int dtok = min(t0 + xtk, P.ntok - 1);
    const uint8_t * xr = (const uint8_t *) P.x + ((size_t) dtok * P.ldx + (size_t) kPK * kcb + 16 * xh) * (XF32 ? 4 : 2);
    /* x role (K-major f32, ntok >= 4): tokens 4 tq .. 4 tq + 3, columns 4 cg .. 4 cg + 3 of a chunk */
    const int tq = tid & 31, cg = tid >> 5;
    const float * xk = (const float *) P.x + (size_t) (kPK * kcb + 4 * cg) * P.ldx + min(t0 + 4 * tq, P.ntok - 4);

    /* register rings of two slots: index words of chunk c in slot c & 1
     * (loaded two chunks ahead), x of chunk c in slot c & 1 (loaded three
     * chunks ahead, staged two ahead) */
    constexpr int NXV = XT ? 4 : (XF32 ? 4 : 2);
    uint32_t iw[2][NST][3], pb[2][NST];
    pf_u4 xv[2][NXV];
    auto fetch_idx = [&](int kc, int sl) {
#pragma unroll
        for (int s = 0; s < NST; s++) {
            iw[sl][s][0] = rs[s][6 * kc];
            iw[sl][s][1] = rs[s][6 * kc + 1];
            iw[sl][s][2] = rs[s][6 * kc + 2];
            pb[sl][s] = EXT ? (uint32_t) ps[s][2 * kc] : 0u;
        }
    };
    auto fetch_x = [&](int kc, int sl) {
        if constexpr (XT) {
#pragma unroll
            for (int k = 0; k < NXV; k++) xv[sl][k] = *(const pf_u4 *) (xk + (size_t) (kPK * kc + k) * P.ldx);
        } else {
#pragma unroll
            for (int k = 0; k < NXV; k++) xv[sl][k] = ((const pf_u4 *) (xr + kPK * kc * (XF32 ? 4 : 2)))[k];
        }
    };
    /* the token tile of the chunk in x slot sl, as f16, into buffer b */
    auto stage_x = [&](int b, int sl) {
        if constexpr (XT) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pf_h4 v4;
#pragma unroll
                for (int c = 0; c < 4; c++) v4[c] = (_Float16) __uint_as_float(xv[sl][c][i]);
                *(pf_h4 *) (Bt + (b * kCT + 4 * tq + i) * kPS + 4 * cg) = v4;
            }
            return;
        }
        _Float16 * bd = Bt + (b * kCT + xtk) * kPS + 16 * xh;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            pf_h8 v8;
            if (XF32) {
                const pf_u4 lo = xv[sl][2 * k], hi = xv[sl][2 * k + 1];
                v8[0] = (_Float16) __uint_as_float(lo.x); v8[1] = (_Float16) __uint_as_float(lo.y);
                v8[2] = (_Float16) __uint_as_float(lo.z); v8[3] = (_Float16) __uint_as_float(lo.w);
                v8[4] = (_Float16) __uint_as_float(hi.x); v8[5] = (_Float16) __uint_as_float(hi.y);
                v8[6] = (_Float16) __uint_as_float(hi.z); v8[7] = (_Float16) __uint_as_float(hi.w);
            } else {
                const pf_u4 q = xv[sl][k];
                v8[0] = (_Float16) __uint_as_float(q.x << 16); v8[1] = (_Float16) __uint_as_float(q.x & 0xffff0000u);
                v8[2] = (_Float16) __uint_as_float(q.y << 16); v8[3] = (_Float16) __uint_as_float(q.y & 0xffff0000u);
                v8[4] = (_Float16) __uint_as_float(q.z << 16); v8[5] = (_Float16) __uint_as_float(q.z & 0xffff0000u);
                v8[6] = (_Float16) __uint_as_float(q.w << 16); v8[7] = (_Float16) __uint_as_float(q.w & 0xffff0000u);
            }
            *(pf_h8 *) (bd + 8 * k) = v8;
        }
    };
    /* step ks's A operand of each stage (codewords 2 ks and 2 ks + 1 of the
     * lane's eight), from index slot sl */
    auto gather_a = [&](int sl, int ks, pf_h8 * a) {
#pragma unroll
        for (int s = 0; s < NST; s++) {
            uint32_t i0 = pf_field12(iw[sl][s][0], iw[sl][s][1], iw[sl][s][2], 2 * ks);
            uint32_t i1 = pf_field12(iw[sl][s][0], iw[sl][s][1], iw[sl][s][2], 2 * ks + 1);
            if (EXT) {
                i0 |= ((pb[sl][s] >> (2 * ks)) & 1u) << 12;
                i1 |= ((pb[sl][s] >> (2 * ks + 1)) & 1u) << 12;
            }
            const pf_h4 lo = *(const pf_h4 *) (lds + s * cbb + 8u * i0);
            const pf_h4 hi = *(const pf_h4 *) (lds + s * cbb + 8u * i1);
            a[s] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };
    /* step ks's B operands (four token blocks) from token buffer b */
    auto read_b = [&](int b, int ks, pf_h8 * bb) {
#pragma unroll
        for (int j = 0; j < 4; j++) bb[j] = *(const pf_h8 *) (Bt + (b * kCT + 32 * j + m32) * kPS + 32 * kh + 8 * ks);
    };

    pf_f16v acc[NA][4];
#pragma unroll
    for (int s = 0; s < NA; s++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[s][j][e] = 0.0f;
    /* FOLD: the gains of the lane's row */
    float ga[NST];
#pragma unroll
    for (int s = 0; s < NST; s++) ga[s] = FOLD ? (float) *(const _Float16 *) (P.st[s] + P.gain_off + 2 * (size_t) arow) : 0.0f;

    /* Three token buffers: chunk c sits in buffer c % 3. While chunk kc's
     * MFMAs run, chunk kc + 2 is staged, and the first operands of chunk
     * kc + 1 (staged a chunk earlier) are read before the barrier; each
     * step's operands are read one step ahead of its MFMAs. */
    __syncthreads();   /* codebooks staged */
    fetch_idx(0, 0);
    fetch_idx(min(1, nkc - 1), 1);
    fetch_x(0, 0);
    fetch_x(min(1, nkc - 1), 1);
    stage_x(0, 0);
    stage_x(1, 1);
    fetch_x(min(2, nkc - 1), 0);
    __syncthreads();
    int b0 = 0;
    if constexpr (FOLD) {
        /* Steps t = 4 kc + ks run a three-deep pipeline in each wave: at step
         * t the wave gathers the codewords of step t + 2, reads the token
         * operands of step t + 1, folds step t + 1's weights and runs step
         * t's MFMAs, the folding VALU interleaved between the MFMAs so the
         * matrix pipe runs while the same wave decodes. */
        auto fold = [&](const pf_h8 * c) {
            pf_h8 w;
#pragma unroll
            for (int d = 0; d < 8; d++)   /* c0 g0 is exact in f32: both products map to v_fma_mix_f32 */
                w[d] = (_Float16) __builtin_fmaf((float) c[1][d], ga[1], __builtin_fmaf((float) c[0][d], ga[0], 0.0f));
            return w;
        };
        pf_h8 raw[2][NST], wv[2], bq[2][4];
        gather_a(0, 0, raw[0]);
        gather_a(0, 1, raw[1]);
        read_b(0, 0, bq[0]);
        wv[0] = fold(raw[0]);
        for (int kc0 = 0; kc0 < nkc; kc0 += 2) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int kc = kc0 + u;
                const int b1 = b0 == 2 ? 0 : b0 + 1, b2 = b1 == 2 ? 0 : b1 + 1;
                __builtin_amdgcn_sched_barrier(0);
                fetch_x(min(kc + 3, nkc - 1), u ^ 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    /* step t + 2's codewords into the slot step t's have left */
                    if (ks < 2) gather_a(u, ks + 2, raw[ks & 1]);
                    else gather_a(u ^ 1, ks - 2, raw[ks & 1]);
                    if (ks == 2) fetch_idx(min(kc + 2, nkc - 1), u);   /* slot u is done */
                    if (ks < 3) read_b(b0, ks + 1, bq[(ks + 1) & 1]);
                    else read_b(b1, 0, bq[0]);
                    wv[(ks + 1) & 1] = fold(raw[(ks + 1) & 1]);
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wv[ks & 1], bq[ks & 1][j], acc[0][j], 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                stage_x(b2, u);
                __syncthreads();
                b0 = b1;
            }
        }
    } else {
    pf_h8 aa[2][NST], bq[2][4];
    gather_a(0, 0, aa[0]);
    read_b(0, 0, bq[0]);
    /* nkc is even: chunk kc0 + u uses index slot u and x slot u */
    for (int kc0 = 0; kc0 < nkc; kc0 += 2) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int kc = kc0 + u;
            const int b1 = b0 == 2 ? 0 : b0 + 1, b2 = b1 == 2 ? 0 : b1 + 1;
            /* the scheduler keeps each group in place: reads stay a step
             * ahead of the MFMAs that use them, loads at their slot */
            __builtin_amdgcn_sched_barrier(0);
            fetch_x(min(kc + 3, nkc - 1), u ^ 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                if (ks < 3) {
                    gather_a(u, ks + 1, aa[(ks + 1) & 1]);
                    read_b(b0, ks + 1, bq[(ks + 1) & 1]);
                } else {
                    /* slot u is done: it takes chunk kc + 2's index words */
                    fetch_idx(min(kc + 2, nkc - 1), u);
                    gather_a(u ^ 1, 0, aa[0]);
                    read_b(b1, 0, bq[0]);
                }
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int s = 0; s < NST; s++)
                        acc[s][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aa[ks & 1][s], bq[ks & 1][j], acc[s][j], 0, 0, 0);
                /* the next step's operand reads spread between the MFMAs,
                 * one read between consecutive MFMAs, so the LDS queue is fed
                 * evenly rather than in bursts */
#pragma unroll
                for (int q = 0; q < 4 * NST; q++) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            stage_x(b2, u);
            __syncthreads();
            b0 = b1;
        }
    }
    }

    /* block j: entry e of a lane is row 8 (e / 4) + 4 kh + e % 4 of the
     * wave's 32 rows, token 32 j + m32; four consecutive rows per store */
    float g[NST][4][4];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = min(r0 + 32 * wave + 8 * q + 4 * kh + i, P.rows - 1);
#pragma unroll
            for (int s = 0; s < NST; s++) g[s][q][i] = (float) *(const _Float16 *) (P.st[s] + P.gain_off + 2 * (size_t) row);
        }
    float * yb = P.y + blockIdx.z * P.ysplit;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int tok = t0 + 32 * j + m32;
        if (tok >= P.ntok) continue;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int row = r0 + 32 * wave + 8 * q + 4 * kh;
            if (row >= P.rows) continue;
            pf_f4 v;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float t = 0.0f;
                if (FOLD) t = acc[0][j][4 * q + i];
                else
#pragma unroll
                    for (int s = 0; s < NST; s++) t = __builtin_fmaf(g[s][q][i], acc[s][j][4 * q + i], t);
                v[i] = t;
            }
            float * yp = yb + (size_t) tok * P.ldy + row;
            if (row + 4 <= P.rows && !((uintptr_t) yp & 15u)) {
                if (P.accumulate) v += *(const pf_f4 *) yp;
                *(pf_f4 *) yp = v;
            } else {
                for (int i = 0; i < 4 && row + i < P.rows; i++) yp[i] = (P.accumulate ? yp[i] : 0.0f) + v[i];
            }
        }
    }
}

/* y[t][r] (+)= the sum of the splits' partial sums, in split order */
__global__ __launch_bounds__(256) void prefill_cw_reduce(const float * ws, int nsplit, int rows, int ntok, float * y,
                                                          int ldy, int accumulate) {
    const size_t n4 = (size_t) ntok * (rows >> 2);
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const int t = (int) (i / (size_t) (rows >> 2)), r = 4 * (int) (i % (size_t) (rows >> 2));
    const size_t slice = (size_t) ntok * rows;
    float * yp = y + (size_t) t * ldy + r;
    pf_f4 v = accumulate ? *(const pf_f4 *) yp : pf_f4{0.f, 0.f, 0.f, 0.f};
    for (int z = 0; z < nsplit; z++) v += *(const pf_f4 *) (ws + z * slice + (size_t) t * rows + r);
    *(pf_f4 *) yp = v;
}

/* The MFMA kernel takes DQV3 dim-4 stages with 12- or 13-bit indices, 1 or
 * 2 stages, an even codebook, columns a multiple of 128, dword-aligned row
 * streams, and x in 16-byte aligned rows: token-major, or K-major f32 of one
 * stage with at least 4 tokens (xt). */
int prefill_mfma_ready(const Layout & L, int nst, const void * x, int xf32, int ldx, int xt, int ntok) {
    if (!L.v3 || L.dim != 4 || L.nbit < 12 || L.nbit > 13 || nst < 1 || nst > 2) return 0;
    if (L.nc % 2 || L.cols % 128 || L.stream_off % 4 || L.mrow % 4) return 0;
    if ((uintptr_t) x & 15u) return 0;
    if (ldx % (xf32 ? 4 : 8)) return 0;
    if (xt && (!xf32 || nst != 1 || ntok < 4 || ldx < ntok)) return 0;
    const size_t lds = (size_t) nst * L.nc * 8 + (size_t) 4 * kPR * kPS * 2;
    return lds <= 160 * 1024;
}

/* LDS of a workgroup: codebooks, two weight tiles of rt rows, two token tiles */
static size_t prefill_lds(int nst, int nc, int rt) {
    return (size_t) nst * nc * 8 + (size_t) (2 * rt + 2 * kPT) * kPS * 2;
}

/* Tile height. A workgroup fills a CU (its LDS leaves no room for a second),
 * so the time is rounds of workgroups over the CUs times a workgroup's time.
 * 128-row tiles decode each weight for 128 tokens; 64-row tiles halve the
 * decode and the MFMAs of a workgroup (not its token conversion), measured at
 * about 0.65 of a 128-row workgroup's time, and double the workgroups. */
static int prefill_rt(int rows, int ntok) {
    const long ttiles = (ntok + kPT - 1) / kPT, G = cu_count();
    const long r128 = ((rows + 127) / 128 * ttiles + G - 1) / G;
    const long r64 = ((rows + 63) / 64 * ttiles + G - 1) / G;
    return r64 * 65 < r128 * 100 ? 64 : 128;
}

template <int NST, int EXT, int XF32, int PF, int XT, int RT>
static int prefill_mfma_rt(const MfmaArgs & P, size_t lds, hipStream_t s) {
    static size_t opted = 0;
    const void * fn = (const void *) prefill_mfma_kernel<NST, EXT, XF32, PF, XT, RT>;
    if (lds > 65536 && lds > opted) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return fail_hip("LDS opt-in for the MFMA prefill kernel", e);
        opted = lds;
    }
    const dim3 grid((unsigned) ((P.rows + RT - 1) / RT), (unsigned) ((P.ntok + kPT - 1) / kPT));
    launch_kernel(prefill_mfma_kernel<NST, EXT, XF32, PF, XT, RT>, grid, dim3(kPThreads), (uint32_t) lds, s, P);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("MFMA prefill launch", e);
}

template <int NST, int EXT, int XF32, int PF, int XT = 0>
static int prefill_mfma_t(const MfmaArgs & P, int nc, hipStream_t s) {
    if (prefill_rt(P.rows, P.ntok) == 64)
        return prefill_mfma_rt<NST, EXT, XF32, PF, XT, 64>(P, prefill_lds(NST, nc, 64), s);
    return prefill_mfma_rt<NST, EXT, XF32, PF, XT, 128>(P, prefill_lds(NST, nc, 128), s);
}

/* LDS of a codeword-operand workgroup: codebooks and three token tiles */
static size_t prefill_cw_lds(int nst, int nc) { return (size_t) nst * nc * 8 + (size_t) 3 * kCT * kPS * 2; }

/* The codeword-operand kernel takes what the tile kernel takes, with y in
 * 16-byte aligned rows (four rows per store), K-major x of whole token
 * quads, and its LDS within the CU's 160 KB. */
static int prefill_cw_ready(const Layout & L, int nst, const void * x, int xf32, int ldx, int xt, int ntok,
                            const float * y, int ldy) {
    if (!prefill_mfma_ready(L, nst, x, xf32, ldx, xt, ntok)) return 0;
    if (xt && ntok % 4) return 0;
    (void) y;
    (void) ldy;
    return prefill_cw_lds(nst, L.nc) <= 160 * 1024;
}

/* K splits: a split costs its chunks times the rounds of workgroups over the
 * CUs, plus, past one split, the reduction's traffic (the slices written and
 * read back, and y) at about 8 bytes per ns, in chunk times of about 0.9 us. */
static int prefill_cw_splits(int rows, int ntok, int nk) {
    const long tiles = (long) ((rows + kCR - 1) / kCR) * ((ntok + kCT - 1) / kCT), G = cu_count();
    int best = 1;
    double best_cost = (double) ((tiles + G - 1) / G) * nk;
    if (rows % 4) return 1;
    for (int S = 2; S <= 16; S++) {
        if (nk % S || (nk / S) % 2) continue;
        const double red_us = (double) (2 * S + 2) * ntok * rows * 4 / 8e3 / 1e3;
        const double cost = (double) ((tiles * S + G - 1) / G) * (nk / S) + red_us / 0.9;
        if (cost < best_cost) { best_cost = cost; best = S; }
    }
    return best;
}

static std::atomic<int> g_prefill_fold{1};

int prefill_fold_on() { return g_prefill_fold.load(std::memory_order_relaxed); }

int prefill_fold_set(int on) { return g_prefill_fold.exchange(on ? 1 : 0); }

/* The no-allocation form's split slices: one file-scope device array of
 * kPrefillScratchBytes, which every GPU the library runs on holds until the
 * process ends. Host code never passes the array's name to a kernel (on the
 * host it is a stand-in, not a device address): the address comes from
 * hipGetSymbolAddress, asked once per device with that device current. */
static __device__ __align__(256) float scratch[kPrefillScratchBytes / sizeof(float)];

int prefill_scratch(void ** ptr) {
    static void * addr[64] = {};
    static std::mutex mu;   /* the first calls on a device may come from several threads */
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail_hip("get device", e);
    if (dev < 0 || dev >= 64) { set_error("device %d is outside the scratch table", dev); return -1; }
    std::lock_guard<std::mutex> hold(mu);
    if (!addr[dev]) {
        void * p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return fail_hip("prefill scratch address", e);
        if (!p) { set_error("prefill scratch has no device address"); return -1; }
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return 0;
}

/* the split slices come from a pool owned by the library (stream ordered,
 * kept between calls), one per device */
static int cw_workspace(size_t bytes, hipStream_t s, void ** out) {
    static hipMemPool_t pools[64] = {};
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail_hip("get device", e);
    if (dev < 0 || dev >= 64) { set_error("device %d is outside the pool table", dev); return -1; }
    std::unique_lock<std::mutex> hold(mu);
    if (!pools[dev]) {
        hipMemPoolProps props;
        memset(&props, 0, sizeof props);
        props.allocType = hipMemAllocationTypePinned;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t p = nullptr;
        e = hipMemPoolCreate(&p, &props);
        if (e != hipSuccess) return fail_hip("memory pool create", e);
        uint64_t keep = ~0ull;
        e = hipMemPoolSetAttribute(p, hipMemPoolAttrReleaseThreshold, &keep);
        if (e != hipSuccess) return fail_hip("memory pool attribute", e);
        pools[dev] = p;
    }
    hipMemPool_t pool = pools[dev];
    hold.unlock();
    e = hipMallocFromPoolAsync(out, bytes, pool, s);
    return e == hipSuccess ? 0 : fail_hip("split workspace", e);
}

template <int NST, int EXT, int XF32, int XT, int FOLD>
static int prefill_cw_tf(const CwArgs & P, int nsplit, hipStream_t s) {
    static size_t opted = 0;
    const size_t lds = prefill_cw_lds(NST, P.nc);
    const void * fn = (const void *) prefill_cw_kernel<NST, EXT, XF32, XT, FOLD>;
    if (lds > 65536 && lds > opted) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return fail_hip("LDS opt-in for the codeword prefill kernel", e);
        opted = lds;
    }
    const dim3 grid((unsigned) ((P.rows + kCR - 1) / kCR), (unsigned) ((P.ntok + kCT - 1) / kCT), (unsigned) nsplit);
    launch_kernel(prefill_cw_kernel<NST, EXT, XF32, XT, FOLD>, grid, dim3(kCThreads), (uint32_t) lds, s, P);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("codeword prefill launch", e);
}

/* Two stages fold by default into one f16 weight (one MFMA per block, 16 %
 * faster on the FFN pair than running them apart, and one more rounding of
 * each weight). With the fold switched off each stage's exact codewords
 * accumulate in their own registers and the gains apply in f32 at the end,
 * the reference's per-stage arithmetic (decode-gpu.cu:359-501). One stage
 * always keeps its exact codewords. */
template <int NST, int EXT, int XF32, int XT>
static int prefill_cw_t(const CwArgs & P, int nsplit, hipStream_t s) {
    if constexpr (NST == 2) {
        if (prefill_fold_on()) return prefill_cw_tf<2, EXT, XF32, XT, 1>(P, nsplit, s);
    }
    return prefill_cw_tf<NST, EXT, XF32, XT, 0>(P, nsplit, s);
}

static int prefill_cw_launch(const void * const * stages, int nst, const Layout & L, const void * x, int xf32,
                             int ldx, int xt, int ntok, float * y, int ldy, int accumulate, hipStream_t s,
                             void * fixed_ws) {
    CwArgs P;
    memset(&P, 0, sizeof P);
    P.st[0] = (const uint8_t *) stages[0];
    P.st[1] = (const uint8_t *) stages[nst > 1 ? 1 : 0];
    P.x = x;
    P.rows = L.rows; P.cols = L.cols; P.nc = L.nc; P.ntok = ntok;
    P.ldx = ldx;
    P.gain_off = (uint32_t) L.gain_off;
    P.stream_off = (uint32_t) L.stream_off;
    P.mrow = (uint32_t) L.mrow;
    P.prow = (uint32_t) L.prow;
    /* the split reduction stores four rows at once: y in 16-byte aligned rows */
    const int y_vec = !((uintptr_t) y & 15u) && ldy % 4 == 0;
    const int nk = L.cols / kPK, nsplit = y_vec ? prefill_cw_splits(L.rows, ntok, nk) : 1;
    P.nkc = nk / nsplit;
    void * ws = nullptr;
    if (nsplit > 1) {
        P.ysplit = (size_t) ntok * L.rows;
        const size_t need = P.ysplit * nsplit * sizeof(float);
        if (fixed_ws) {
            /* every slice is written whole by its split before the reduction
             * reads it, so the scratch needs no clearing */
            if (need > kPrefillScratchBytes) {
                set_error("this prefill splits K %d ways and needs %zu bytes of scratch; the no-allocation "
                          "prefill holds %zu", nsplit, need, (size_t) kPrefillScratchBytes);
                return -1;
            }
            ws = fixed_ws;
        } else if (cw_workspace(need, s, &ws)) {
            return -1;
        }
        P.y = (float *) ws;
        P.ldy = L.rows;
        P.accumulate = 0;
    } else {
        P.y = y;
        P.ldy = ldy;
        P.accumulate = accumulate;
    }
    const int ext = L.nbit > 12;
    int rc;
    if (xt) rc = ext ? prefill_cw_t<1, 1, 1, 1>(P, nsplit, s) : prefill_cw_t<1, 0, 1, 1>(P, nsplit, s);
    else if (nst == 2) {
        if (xf32) rc = ext ? prefill_cw_t<2, 1, 1, 0>(P, nsplit, s) : prefill_cw_t<2, 0, 1, 0>(P, nsplit, s);
        else rc = ext ? prefill_cw_t<2, 1, 0, 0>(P, nsplit, s) : prefill_cw_t<2, 0, 0, 0>(P, nsplit, s);
    } else {
        if (xf32) rc = ext ? prefill_cw_t<1, 1, 1, 0>(P, nsplit, s) : prefill_cw_t<1, 0, 1, 0>(P, nsplit, s);
        else rc = ext ? prefill_cw_t<1, 1, 0, 0>(P, nsplit, s) : prefill_cw_t<1, 0, 0, 0>(P, nsplit, s);
    }
    if (nsplit > 1) {
        if (!rc) {
            const size_t n4 = (size_t) ntok * (L.rows / 4);
            launch_kernel(prefill_cw_reduce, dim3((unsigned) ((n4 + 255) / 256)), dim3(256), 0u, s, (const float *) ws,
                          nsplit, L.rows, ntok, y, ldy, accumulate);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) rc = fail_hip("split reduction launch", e);
        }
        if (!fixed_ws) {
            hipError_t e = hipFreeAsync(ws, s);
            if (!rc && e != hipSuccess) rc = fail_hip("split workspace release", e);
        }
    }
    return rc;
}

int prefill_mfma_launch(const void * const * stages, int nst, const Layout & L, const void * x, int xf32, int ldx,
                        int xt, int ntok, float * y, int ldy, int accumulate, hipStream_t s, void * fixed_ws) {
    if (!prefill_mfma_ready(L, nst, x, xf32, ldx, xt, ntok)) {
        set_error("the MFMA prefill kernel does not take this geometry, stage count or x layout");
        return -1;
    }
    if (ntok <= 0) { set_error("prefill needs at least one token"); return -1; }
    if (prefill_cw_ready(L, nst, x, xf32, ldx, xt, ntok, y, ldy))
        return prefill_cw_launch(stages, nst, L, x, xf32, ldx, xt, ntok, y, ldy, accumulate, s, fixed_ws);
    MfmaArgs P;
    memset(&P, 0, sizeof P);
    P.st[0] = (const uint8_t *) stages[0];
    P.st[1] = (const uint8_t *) stages[nst > 1 ? 1 : 0];
    P.x = x;
    P.y = y;
    P.rows = L.rows; P.cols = L.cols; P.nc = L.nc; P.ntok = ntok;
    P.ldx = ldx; P.ldy = ldy; P.accumulate = accumulate;
    P.gain_off = (uint32_t) L.gain_off;
    P.stream_off = (uint32_t) L.stream_off;
    P.mrow = (uint32_t) L.mrow;
    P.prow = (uint32_t) L.prow;
    const int nc = L.nc, ext = L.nbit > 12;
    /* four chunks in flight when the chunk count allows, else two */
    const int pf4 = (L.cols / kPK) % 4 == 0;
#define PF_PICK(N, E, X) return pf4 ? prefill_mfma_t<N, E, X, 4>(P, nc, s) : prefill_mfma_t<N, E, X, 2>(P, nc, s)
    if (xt) {   /* one stage, f32 (checked above) */
        if (ext) return pf4 ? prefill_mfma_t<1, 1, 1, 4, 1>(P, nc, s) : prefill_mfma_t<1, 1, 1, 2, 1>(P, nc, s);
        return pf4 ? prefill_mfma_t<1, 0, 1, 4, 1>(P, nc, s) : prefill_mfma_t<1, 0, 1, 2, 1>(P, nc, s);
    }
    if (nst == 2) {
        if (xf32) { if (ext) PF_PICK(2, 1, 1); PF_PICK(2, 0, 1); }
        if (ext) PF_PICK(2, 1, 0);
        PF_PICK(2, 0, 0);
    }
    if (xf32) { if (ext) PF_PICK(1, 1, 1); PF_PICK(1, 0, 1); }
    if (ext) PF_PICK(1, 1, 0);
    PF_PICK(1, 0, 0);
#undef PF_PICK
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
