/* vq_kernels.hip — VQ codebook-index GEMV, dequant and row dequant for gfx950.
 *
 * Semantics (what every kernel here computes) follow the reference's Rust
 * reader: a stage contributes y[n][r] += g[r] * sum_i dot(cb[idx(r, i)], x[n][dim*i ..])
 * (tools/vq-format/src/lib.rs:215-227), stages in order, and a decoded weight is
 * W[r][dim*i + d] += cb[idx][d] * g[r] (lib.rs:197-211).
 *
 * Kernels
 *   vq_mfma_kernel  the hot path (variant 3): DQV3, dim 4, 12- or 13-bit
 *                   indices. Codebooks of every stage sit in LDS; a wave owns
 *                   16 rows, gathers each raw f16 codeword with one ds_read_b64
 *                   straight into the A operand of v_mfma_f32_16x16x16_f16, and
 *                   x (f16 in LDS) is the B operand, one column per N lane.
 *                   Gains are applied per stage in the epilogue, so products
 *                   of codeword and activation are exact and only the f32
 *                   accumulation rounds. The same kernel serves N = 1..16
 *                   activation columns: a weight is decoded once for all of them.
 *   vq_wave_kernel  variants 1 and 2: one wave per row, any dim, any index
 *                   width, DQVQ or DQV3; codebook in LDS (2) or read through
 *                   the cache (1). f32 arithmetic.
 *   vq_dequant_kernel / vq_row_dequant_kernel: bit-exact decode (each
 *                   codeword times gain is exact in f32, one rounding per add).
 */
#include "vq.h"

#include <hip/hip_fp16.h>
#include <string.h>

namespace sparkmv {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float) v;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t) h << 16);
}

__device__ __forceinline__ float load_x(const void * x, int xf32, size_t k) {
    return xf32 ? ((const float *) x)[k] : bf16_to_f32(((const uint16_t *) x)[k]);
}

/* ------------------------------------------------------------------------ */
/* Variant 3: the MFMA block kernel.                                         */
/* ------------------------------------------------------------------------ */

struct FastMat {
    const uint8_t * st[2];
    float * y;
    int rows;
    int group0;   /* first tile group of this matrix within the launch */
};

struct FastArgs {
    FastMat mat[kMaxMats];
    const void * x;
    int nmat, ngroups, cols, nc, ncol, ldx, ldy, accumulate;
    uint32_t gain_off;   /* 24 + nc * 8: the same for every matrix of a launch */
    uint32_t mrow, prow;
    int kc;              /* columns per LDS x chunk, a multiple of 128 */
    int xstride;         /* bytes per x column row in LDS (kc * 2 + 8: the pad spreads N over banks) */
};

/* Byte address (index * 8) of field t of the 8 12-bit indices packed
 * LSB-first into three little-endian words. */
template <int T>
__device__ __forceinline__ uint32_t cw_addr(uint32_t w0, uint32_t w1, uint32_t w2) {
    switch (T) {
        case 0: return (w0 << 3) & 0x7ff8u;
        case 1: return (w0 >> 9) & 0x7ff8u;
        case 2: return __builtin_amdgcn_alignbit(w1, w0, 21) & 0x7ff8u;
        case 3: return (w1 >> 1) & 0x7ff8u;
        case 4: return (w1 >> 13) & 0x7ff8u;
        case 5: return __builtin_amdgcn_alignbit(w2, w1, 25) & 0x7ff8u;
        case 6: return (w2 >> 5) & 0x7ff8u;
        default: return (w2 >> 17) & 0x7ff8u;
    }
}

template <int NST, int EXT>
struct Words {
    uint32_t w[NST][3];
    uint32_t pb[NST];
};

template <int NST, int EXT>
__device__ __forceinline__ void load_words(Words<NST, EXT> & W, const uint8_t * const * rp,
                                           const uint8_t * const * pp, int ms) {
#pragma unroll
    for (int s = 0; s < NST; s++) {
        const uint32_t * p = (const uint32_t *) (rp[s] + 48 * ms);
        W.w[s][0] = p[0];
        W.w[s][1] = p[1];
        W.w[s][2] = p[2];
        if (EXT) W.pb[s] = pp[s][4 * ms];
    }
}

/* One macro-step: 32 indices of each of the wave's 16 rows, 8 per lane
 * quarter, 8 MFMAs per stage. k-slot (quarter q, step t) holds index
 * 32 * msl + 8q + t of the chunk, i.e. columns 4 * that .. + 3; A and B use the
 * same assignment, so the contraction is over the row's true columns. */
template <int NST, int XF32, int EXT, int T>
__device__ __forceinline__ void mstep_t(const Words<NST, EXT> & W, const uint8_t * lds, uint32_t cbb,
                                        const uint8_t * xb, const uint8_t * xbl, f4 * acc) {
    const h4 b = *(const h4 *) (xb + 8 * T);
    h4 bl;
    if (XF32) bl = *(const h4 *) (xbl + 8 * T);
#pragma unroll
    for (int s = 0; s < NST; s++) {
        uint32_t a = cw_addr<T>(W.w[s][0], W.w[s][1], W.w[s][2]);
        if (EXT) a |= (W.pb[s] << (15 - T)) & 0x8000u;
        const h4 cw = *(const h4 *) (lds + (uint32_t) s * cbb + a);
        acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(cw, b, acc[s], 0, 0, 0);
        if (XF32) acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(cw, bl, acc[s], 0, 0, 0);
    }
}

template <int NST, int XF32, int EXT>
__device__ __forceinline__ void mstep(const Words<NST, EXT> & W, const uint8_t * lds, uint32_t cbb,
                                      const uint8_t * xb, const uint8_t * xbl, f4 * acc) {
    mstep_t<NST, XF32, EXT, 0>(W, lds, cbb, xb, xbl, acc);
    mstep_t<NST, XF32, EXT, 1>(W, lds, cbb, xb, xbl, acc);
    mstep_t<NST, XF32, EXT, 2>(W, lds, cbb, xb, xbl, acc);
    mstep_t<NST, XF32, EXT, 3>(W, lds, cbb, xb, xbl, acc);
    mstep_t<NST, XF32, EXT, 4>(W, lds, cbb, xb, xbl, acc);
    mstep_t<NST, XF32, EXT, 5>(W, lds, cbb, xb, xbl, acc);
    mstep_t<NST, XF32, EXT, 6>(W, lds, cbb, xb, xbl, acc);
    mstep_t<NST, XF32, EXT, 7>(W, lds, cbb, xb, xbl, acc);
}

/* Cooperative conversion of x columns [c0, c1) of every activation column to
 * f16 in LDS (hi, and for f32 input also the residual lo = f16(x - hi)). */
template <int XF32>
__device__ __forceinline__ void stage_x(const FastArgs & A, uint8_t * lx, int c0, int c1) {
    const int w = c1 - c0;
    for (int e = threadIdx.x; e < A.ncol * w; e += blockDim.x) {
        const int n = e / w, cc = e - n * w;
        const float v = load_x(A.x, XF32, (size_t) n * A.ldx + c0 + cc);
        const _Float16 h = (_Float16) v;
        *(_Float16 *) (lx + n * A.xstride + 2 * cc) = h;
        if (XF32) *(_Float16 *) (lx + (A.ncol + n) * A.xstride + 2 * cc) = (_Float16) (v - (float) h);
    }
}

template <int NST, int XF32, int EXT>
__global__ __launch_bounds__(512) void vq_mfma_kernel(const FastArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t cbb = (uint32_t) A.nc * 8u;
    uint8_t * lx = lds + NST * cbb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const int r16 = lane & 15, q = lane >> 4;
    const int ncx = (A.cols + A.kc - 1) / A.kc;
    const int g0 = (int) (((long long) A.ngroups * blockIdx.x) / gridDim.x);
    const int g1 = (int) (((long long) A.ngroups * (blockIdx.x + 1)) / gridDim.x);
    const int bn = r16 < A.ncol ? r16 : A.ncol - 1;
    int m = 0, loaded = -1;
    for (int g = g0; g < g1; g++) {
        while (m + 1 < A.nmat && g >= A.mat[m + 1].group0) m++;
        if (m != loaded) {
            __syncthreads();
            /* codebooks: nc * 8 bytes per stage, 16 bytes per thread step
             * and the last 8 bytes when nc is odd */
            const int n16 = (int) (cbb >> 4);
#pragma unroll
            for (int s = 0; s < NST; s++) {
                const uint32_t * src = (const uint32_t *) (A.mat[m].st[s] + 24);
                uint32_t * dst = (uint32_t *) (lds + s * cbb);
                for (int i = threadIdx.x; i < n16; i += blockDim.x) {
                    const uint32_t a0 = src[4 * i], a1 = src[4 * i + 1], a2 = src[4 * i + 2], a3 = src[4 * i + 3];
                    dst[4 * i] = a0; dst[4 * i + 1] = a1; dst[4 * i + 2] = a2; dst[4 * i + 3] = a3;
                }
                if ((cbb & 8u) && threadIdx.x < 2) dst[4 * n16 + threadIdx.x] = src[4 * n16 + threadIdx.x];
            }
            if (loaded < 0 && ncx == 1) stage_x<XF32>(A, lx, 0, A.cols);
            __syncthreads();
            loaded = m;
        }
        const int rows = A.mat[m].rows;
        const int trow = (g - A.mat[m].group0) * nwave * 16 + wave * 16;
        const bool active = trow < rows;
        const int row = min(trow + r16, rows - 1);
        const uint8_t * rp[NST];
        const uint8_t * pp[NST];
#pragma unroll
        for (int s = 0; s < NST; s++) {
            const uint8_t * sbase = A.mat[m].st[s] + A.gain_off + (size_t) rows * 2;
            rp[s] = sbase + (size_t) row * A.mrow + 12 * q;
            pp[s] = sbase + (size_t) rows * A.mrow + (size_t) row * A.prow + q;
        }
        f4 acc[NST];
#pragma unroll
        for (int s = 0; s < NST; s++) acc[s] = f4{0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < ncx; c++) {
            const int c0 = c * A.kc, c1 = min(A.cols, c0 + A.kc);
            if (ncx > 1) {
                __syncthreads();
                stage_x<XF32>(A, lx, c0, c1);
                __syncthreads();
            }
            if (active) {
                const int ms0 = c0 >> 7, ms1 = c1 >> 7;
                const uint8_t * xb = lx + bn * A.xstride + 64 * q;
                const uint8_t * xbl = lx + (A.ncol + bn) * A.xstride + 64 * q;
                Words<NST, EXT> cur, nxt;
                load_words<NST, EXT>(cur, rp, pp, ms0);
                for (int ms = ms0; ms < ms1; ms++) {
                    if (ms + 1 < ms1) load_words<NST, EXT>(nxt, rp, pp, ms + 1);
                    const int off = 256 * (ms - ms0);
                    mstep<NST, XF32, EXT>(cur, lds, cbb, xb + off, xbl + off, acc);
                    cur = nxt;
                }
            }
        }
        if (active && r16 < A.ncol) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = trow + 4 * q + i;
                if (r < rows) {
                    float * yp = A.mat[m].y + (size_t) r16 * A.ldy + r;
                    float v = A.accumulate ? *yp : 0.0f;
#pragma unroll
                    for (int s = 0; s < NST; s++) {
                        const float gs = f16_to_f32(*(const uint16_t *) (A.mat[m].st[s] + A.gain_off + 2 * (size_t) r));
                        v += gs * acc[s][i];
                    }
                    *yp = v;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Variants 1 and 2: one wave per row, any geometry.                         */
/* ------------------------------------------------------------------------ */

/* Index of group i in `row`, reading bytes only inside the stage's stream;
 * bytes past it read as zero, as tools/vq-format/src/lib.rs:175-186 does. */
__device__ __forceinline__ uint32_t rd_index(const uint8_t * st, const Layout & L, size_t row, size_t i) {
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
    /* A corrupt stream must never address past the codebook. */
    return v < (uint32_t) L.nc ? v : (uint32_t) L.nc - 1u;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int LDSCB>
__global__ __launch_bounds__(256) void vq_wave_kernel(const uint8_t * p, const Layout L, const void * x, int ldx,
                                                       int xf32, int ncol, float * y, int ldy, int accumulate) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint16_t * gcb = (const uint16_t *) (p + L.cb_off);
    const uint16_t * cb = gcb;
    if (LDSCB) {
        uint16_t * s = (uint16_t *) lds;
        for (int i = threadIdx.x; i < L.nc * L.dim; i += blockDim.x) s[i] = gcb[i];
        __syncthreads();
        cb = s;
    }
    const uint8_t * st = p + L.stream_off;
    const uint16_t * gr = (const uint16_t *) (p + L.gain_off);
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int row = blockIdx.x * nw + (threadIdx.x >> 6); row < L.rows; row += gridDim.x * nw) {
        float acc[kMaxCols];
#pragma unroll
        for (int n = 0; n < kMaxCols; n++) acc[n] = 0.0f;
        for (size_t i = lane; i < L.nidx_row; i += 64) {
            const uint32_t v = rd_index(st, L, (size_t) row, i);
            for (int d = 0; d < L.dim; d++) {
                const float c = f16_to_f32(cb[(size_t) v * L.dim + d]);
                const size_t k = i * (size_t) L.dim + d;
#pragma unroll
                for (int n = 0; n < kMaxCols; n++)
                    if (n < ncol) acc[n] += c * load_x(x, xf32, (size_t) n * ldx + k);
            }
        }
        const float g = f16_to_f32(gr[row]);
#pragma unroll
        for (int n = 0; n < kMaxCols; n++) {
            if (n < ncol) {
                const float s = wave_sum(acc[n]);
                if (lane == 0) {
                    float * yp = y + (size_t) n * ldy + row;
                    *yp = (accumulate ? *yp : 0.0f) + s * g;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Dequant (bit-exact), row dequant, plain f32 GEMV.                          */
/* ------------------------------------------------------------------------ */

__global__ void vq_dequant_kernel(const uint8_t * p, const Layout L, float * out, int accumulate) {
    const size_t gi = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= (size_t) L.rows * L.nidx_row) return;
    const size_t row = gi / L.nidx_row, i = gi - row * L.nidx_row;
    const uint16_t * cb = (const uint16_t *) (p + L.cb_off);
    const float g = f16_to_f32(((const uint16_t *) (p + L.gain_off))[row]);
    const uint32_t v = rd_index(p + L.stream_off, L, row, i);
    float * o = out + row * (size_t) L.cols + i * (size_t) L.dim;
    /* accumulate 0 starts from +0.0, exactly as adding into a zeroed matrix */
    for (int d = 0; d < L.dim; d++)
        o[d] = __fadd_rn(accumulate ? o[d] : 0.0f, __fmul_rn(f16_to_f32(cb[(size_t) v * L.dim + d]), g));
}

__global__ void vq_row_dequant_kernel(const uint8_t * p, const Layout L, int row, float * out) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= L.nidx_row) return;
    const uint16_t * cb = (const uint16_t *) (p + L.cb_off);
    const float g = f16_to_f32(((const uint16_t *) (p + L.gain_off))[row]);
    const uint32_t v = rd_index(p + L.stream_off, L, (size_t) row, i);
    float * o = out + i * (size_t) L.dim;
    for (int d = 0; d < L.dim; d++) o[d] = __fadd_rn(o[d], __fmul_rn(f16_to_f32(cb[(size_t) v * L.dim + d]), g));
}

__global__ __launch_bounds__(256) void f32_gemv_kernel(const float * w, const float * x, float * y, int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float * wr = w + (size_t) row * cols;
    float acc = 0.0f;
    for (int c = lane; c < cols; c += 64) acc += wr[c] * x[c];
    acc = wave_sum(acc);
    if (lane == 0) y[row] += acc;
}

/* ------------------------------------------------------------------------ */
/* Host side.                                                                */
/* ------------------------------------------------------------------------ */

static const int kLdsMax = 160 * 1024;

static int fast_geometry_ok(int dim, int nc, int rows, int cols, int v3) {
    if (!v3 || dim != 4 || rows <= 0 || cols <= 0 || cols % 4) return 0;
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    if (L.nbit < 12 || L.nbit > 13) return 0;     /* 12-bit fields (+ plane bit) */
    if (L.nidx_row % 32) return 0;                /* whole 32-index macro steps */
    if (L.stream_off % 4 || L.mrow % 4) return 0; /* dword-aligned row streams */
    return 1;
}

int vq_variant_ready(int dim, int nc, int rows, int cols, int v3, int variant) {
    if (dim <= 0 || nc <= 0 || rows <= 0 || cols <= 0 || cols % dim) return 0;
    if (v3 && bits_for(nc) > 13) return 0;
    switch (variant) {
        case 0: return 1;
        case 1: return 1;
        case 2: return (size_t) nc * dim * 2 <= 65536;
        case 3: return fast_geometry_ok(dim, nc, rows, cols, v3);
        default: return 0;
    }
}

static int aligned4(const void * p) { return ((uintptr_t) p & 3u) == 0; }

template <int NST, int XF32, int EXT>
static int launch_fast_t(const FastArgs & A, int grid, int threads, size_t lds, hipStream_t s) {
    static size_t opted = 0;
    const void * fn = (const void *) vq_mfma_kernel<NST, XF32, EXT>;
    if (lds > 65536 && lds > opted) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return fail_hip("LDS opt-in for the VQ block kernel", e);
        opted = lds;
    }
    hipLaunchKernelGGL((vq_mfma_kernel<NST, XF32, EXT>), dim3(grid), dim3(threads), lds, s, A);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail_hip("VQ block kernel launch", e);
    return 0;
}

static int launch_fast(const VqCall & c, int st0, int nst, int accumulate) {
    const Layout L0 = make_layout(c.dim, c.nc, c.mats[0].rows, c.cols, 1);
    const int ext = L0.nbit > 12;
    const int threads = c.threads ? c.threads : 512;
    if (threads > 512) { set_error("the VQ block kernel runs at most 512 threads per workgroup, not %d", threads); return -1; }
    const int nwave = threads / 64;
    FastArgs A;
    memset(&A, 0, sizeof A);
    A.x = c.x;
    A.nmat = c.nmat;
    A.cols = c.cols;
    A.nc = c.nc;
    A.ncol = c.ncol;
    A.ldx = c.ldx;
    A.ldy = c.ldy;
    A.accumulate = accumulate;
    A.gain_off = (uint32_t) L0.gain_off;
    A.mrow = (uint32_t) L0.mrow;
    A.prow = (uint32_t) L0.prow;
    int groups = 0;
    for (int m = 0; m < c.nmat; m++) {
        for (int s = 0; s < nst; s++) A.mat[m].st[s] = (const uint8_t *) c.mats[m].stages[st0 + s];
        A.mat[m].y = c.mats[m].y;
        A.mat[m].rows = c.mats[m].rows;
        A.mat[m].group0 = groups;
        groups += (c.mats[m].rows + 16 * nwave - 1) / (16 * nwave);
    }
    A.ngroups = groups;
    const size_t cbb = (size_t) nst * c.nc * 8;
    const int xmul = c.xf32 ? 2 : 1;
    /* x chunk: every column resident when it fits, else the widest multiple of
     * 128 columns that does. */
    const size_t room = kLdsMax - cbb;
    int kc = c.cols;
    if ((size_t) xmul * c.ncol * ((size_t) kc * 2 + 8) > room) {
        kc = (int) (((room / ((size_t) xmul * c.ncol)) - 8) / 2);
        kc &= ~127;
        if (kc < 128) { set_error("x of %d columns does not fit LDS beside the codebooks", c.ncol); return -1; }
    }
    A.kc = kc;
    A.xstride = kc * 2 + 8;
    const size_t lds = cbb + (size_t) xmul * c.ncol * A.xstride;
    int grid = c.grid;
    if (grid <= 0) {
        const int per_cu = (int) (kLdsMax / lds) > 0 ? (int) (kLdsMax / lds) : 1;
        grid = cu_count() * (per_cu < 2 ? per_cu : 2);
    }
    if (grid > groups) grid = groups;
    if (grid < 1) grid = 1;
    const int key = (nst == 2 ? 4 : 0) | (c.xf32 ? 2 : 0) | (ext ? 1 : 0);
    switch (key) {
        case 0: return launch_fast_t<1, 0, 0>(A, grid, threads, lds, c.stream);
        case 1: return launch_fast_t<1, 0, 1>(A, grid, threads, lds, c.stream);
        case 2: return launch_fast_t<1, 1, 0>(A, grid, threads, lds, c.stream);
        case 3: return launch_fast_t<1, 1, 1>(A, grid, threads, lds, c.stream);
        case 4: return launch_fast_t<2, 0, 0>(A, grid, threads, lds, c.stream);
        case 5: return launch_fast_t<2, 0, 1>(A, grid, threads, lds, c.stream);
        case 6: return launch_fast_t<2, 1, 0>(A, grid, threads, lds, c.stream);
        default: return launch_fast_t<2, 1, 1>(A, grid, threads, lds, c.stream);
    }
}

static int launch_wave(const VqCall & c, int variant) {
    /* A wider request runs as more 256-thread workgroups: the width only
     * changes how many row-waves share a workgroup, never the arithmetic. */
    const int threads = c.threads && c.threads < 256 ? c.threads : 256;
    const int nw = threads / 64;
    for (int m = 0; m < c.nmat; m++) {
        const Layout L = make_layout(c.dim, c.nc, c.mats[m].rows, c.cols, c.v3);
        const size_t lds = variant == 2 ? (size_t) c.nc * c.dim * 2 : 0;
        int grid = c.grid > 0 ? c.grid : (L.rows + nw - 1) / nw;
        for (int s = 0; s < c.nst; s++) {
            const int acc = s > 0 || c.accumulate;
            const uint8_t * p = (const uint8_t *) c.mats[m].stages[s];
            if (variant == 2)
                hipLaunchKernelGGL(vq_wave_kernel<1>, dim3(grid), dim3(threads), lds, c.stream, p, L, c.x, c.ldx,
                                   c.xf32, c.ncol, c.mats[m].y, c.ldy, acc);
            else
                hipLaunchKernelGGL(vq_wave_kernel<0>, dim3(grid), dim3(threads), 0, c.stream, p, L, c.x, c.ldx,
                                   c.xf32, c.ncol, c.mats[m].y, c.ldy, acc);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return fail_hip("VQ wave kernel launch", e);
        }
    }
    return 0;
}

int vq_launch(const VqCall & c) {
    if (c.dim <= 0 || c.nc <= 0 || c.cols <= 0 || c.cols % c.dim) {
        set_error("VQ geometry dim %d, nc %d, cols %d is inconsistent", c.dim, c.nc, c.cols);
        return -1;
    }
    if (c.v3 && bits_for(c.nc) > 13) {
        set_error("DQV3 carries 13 index bits, nc %d needs %d", c.nc, bits_for(c.nc));
        return -1;
    }
    if (c.nst < 1 || c.nst > kMaxStages) { set_error("stage count %d is outside 1..%d", c.nst, kMaxStages); return -1; }
    if (c.nmat < 1 || c.nmat > kMaxMats) { set_error("matrix count %d is outside 1..%d", c.nmat, kMaxMats); return -1; }
    if (c.ncol < 1 || c.ncol > kMaxCols) { set_error("column count %d is outside 1..%d", c.ncol, kMaxCols); return -1; }
    if (!c.x) { set_error("x is null"); return -1; }
    if (c.ncol > 1 && c.ldx < c.cols) { set_error("ldx %d is below cols %d", c.ldx, c.cols); return -1; }
    if (c.threads && (c.threads < 64 || c.threads > 1024 || c.threads % 64)) {
        set_error("launch width %d is not a multiple of 64 up to 1024", c.threads);
        return -1;
    }
    int all_fast = 1;
    for (int m = 0; m < c.nmat; m++) {
        if (c.mats[m].rows <= 0) { set_error("matrix %d has %d rows", m, c.mats[m].rows); return -1; }
        if (!c.mats[m].y) { set_error("matrix %d has a null y", m); return -1; }
        if (c.ncol > 1 && c.ldy < c.mats[m].rows) { set_error("ldy %d is below rows %d", c.ldy, c.mats[m].rows); return -1; }
        for (int s = 0; s < c.nst; s++) {
            if (!c.mats[m].stages[s]) { set_error("matrix %d stage %d payload is null", m, s); return -1; }
            if (!aligned4(c.mats[m].stages[s])) all_fast = 0;
        }
        if (!fast_geometry_ok(c.dim, c.nc, c.mats[m].rows, c.cols, c.v3)) all_fast = 0;
    }
    int variant = c.variant;
    if (variant == 0) variant = all_fast ? 3 : ((size_t) c.nc * c.dim * 2 <= 65536 ? 2 : 1);
    if (variant == 3) {
        if (!all_fast) { set_error("the VQ block kernel does not take this geometry or alignment"); return -1; }
        for (int st0 = 0; st0 < c.nst; st0 += 2) {
            const int n = c.nst - st0 < 2 ? c.nst - st0 : 2;
            if (launch_fast(c, st0, n, st0 > 0 || c.accumulate)) return -1;
        }
        return 0;
    }
    if (variant == 2 && (size_t) c.nc * c.dim * 2 > 65536) {
        set_error("a codebook of %d x %d does not fit the LDS variant", c.nc, c.dim);
        return -1;
    }
    if (variant != 1 && variant != 2) { set_error("unknown VQ variant %d", variant); return -1; }
    return launch_wave(c, variant);
}

int vq_dequant_launch(const void * payload, const Layout & L, float * out, int accumulate, hipStream_t s) {
    const size_t n = (size_t) L.rows * L.nidx_row;
    const int threads = 256;
    hipLaunchKernelGGL(vq_dequant_kernel, dim3((unsigned) ((n + threads - 1) / threads)), dim3(threads), 0, s,
                       (const uint8_t *) payload, L, out, accumulate);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("dequant launch", e);
}

int vq_row_dequant_launch(const void * payload, const Layout & L, int row, float * out, hipStream_t s) {
    const int threads = 256;
    hipLaunchKernelGGL(vq_row_dequant_kernel, dim3((unsigned) ((L.nidx_row + threads - 1) / threads)), dim3(threads),
                       0, s, (const uint8_t *) payload, L, row, out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("row dequant launch", e);
}

int f32_gemv_launch(const float * w, const float * x, float * y, int rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL(f32_gemv_kernel, dim3((unsigned) ((rows + 3) / 4)), dim3(256), 0, s, w, x, y, rows, cols);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("f32 gemv launch", e);
}

}  // namespace sparkmv
