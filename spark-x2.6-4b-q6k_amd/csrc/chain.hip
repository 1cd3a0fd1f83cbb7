/* chain.hip — a chain of VQ matvecs as ONE persistent launch (gfx950).
 *
 * The reference's GPU runtime issues each token's matvecs one launch at a
 * time, every matvec depending on the one before it through the residual,
 * the norms and the activations (tools/vq/gpu/vq-model-gpu.cu:776-835). On
 * gfx950 every launch pays a fixed cost before its first multiply: dispatch,
 * staging 64 KB of codebooks into LDS, the first index words' memory round
 * trip, and the epilogue. A chain replaces the per-matvec launches with one
 * launch of one workgroup per CU that walks the whole op list:
 *
 *  - Each op is split over the workgroups by whole MFMA tiles (one matrix per
 *    workgroup, or, for a gate/up pair, the same rows of both matrices), and
 *    each workgroup's units (tile x K chunk) over its waves.
 *  - Weights never depend on activations, so every wave streams its index
 *    words through a ring of R macro steps that runs straight across
 *    unit and op boundaries: while a workgroup waits for the previous op's
 *    output, its next op's first index words, codebooks and gains are already
 *    in flight.
 *  - An op that reads an earlier op's output waits until every workgroup has
 *    published it: each workgroup's writes are acknowledged (s_waitcnt
 *    vmcnt(0) on agent-coherent stores), then it stores its count of finished
 *    ops into its own flag word; a waiting workgroup polls all flags with
 *    agent-coherent loads. Every wait is bounded: past kChainSpin polls the
 *    workgroup sets the error word and goes on, so the launch always ends and
 *    the host reports the failure.
 *  - Staging applies the op's input transform while it writes x to LDS: bf16
 *    as is, f32 rounded to bf16, or rms_norm (f64 sum of squares, as
 *    tools/vq-runtime/src/model.rs:236-245) then bf16. A gate/up pair's
 *    epilogue writes bf16(gelu(gate) * up) (model.rs:253-258, erf in f64), the
 *    input of down, so no workgroup recomputes it.
 *
 * The arithmetic of one tile is the block kernel's (vq_tile.h): raw f16
 * codewords gathered from LDS into the A operand of v_mfma_f32_16x16x16_f16,
 * x as f16 in the B operand, f32 accumulation, gains applied per stage after
 * the K chunks of a row are added in a fixed order. Results do not depend on
 * timing.
 *
 * A chain assumes it has the GPU to itself while it runs: all its workgroups
 * must be resident at once (one per CU, held there by its LDS size).
 */
#include "../../include/sparkmv.h"
#include "common.h"
#include "vq_tile.h"
#include "xrange.h"

#include <math.h>
#include <string.h>

#include <vector>

namespace sparkmv {

constexpr int kChainMats = 4;
constexpr uint32_t kChainSpin = 1u << 19; /* polls before a wait gives up (about half a second) */
constexpr uint32_t kChainLds = 160 * 1024;
constexpr uint32_t kChainTop = 512;      /* range flags and norm partials at the top of LDS */
constexpr int kChainMaxCols = 16384;     /* columns a chain op stages (x in registers, then LDS) */
constexpr int kChainMaxChunks = 8192;    /* 16-byte codebook chunks: 2 matrices x 2 stages x 32 KB */

struct ChainMat {
    const uint8_t * st[2];   /* stage payloads */
    float * y;               /* f32 output */
    uint16_t * ybf;          /* bf16 copy of the output (may be null) */
    const float * yadd;      /* y = yadd + W x when set */
    int rows, tiles, wg0, nwg;
    uint32_t stream_off;     /* gain_off + 2 * rows */
    uint32_t pad;
};

struct ChainOp {
    ChainMat mat[kChainMats];
    const void * x;
    const float * nw;        /* rms_norm weight (null = 1) */
    uint16_t * xout;         /* workgroup 0 writes the staged bf16 x here (may be null) */
    uint16_t * act;          /* a pair's bf16 gelu(y0) * y1 */
    float eps;
    int nmat, pair, cols, M, lgS, C, msc, dep, xmode;
    int yadd_early;                 /* every y_add is published before this op's wait is entered */
    uint32_t gain_off, mrow, cbb;   /* cbb: bytes per stage codebook, nc * 8 */
    uint32_t xoff, roff, poff;      /* LDS byte offsets of x, the reduction area, the partials */
};

enum { kXBf16 = 0, kXF32 = 1, kXNorm = 2 };

/* The op table is read through the constant address space: it does not
 * change during a launch, so every field is a scalar load even after the
 * kernel's own agent-scope stores (which would otherwise keep the compiler
 * from proving the table unchanged, and turn the reads into vector loads
 * that wait for every outstanding load). */
typedef const __attribute__((address_space(4))) ChainOp KOp;

__device__ __forceinline__ uint32_t ld_agent(const uint32_t * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldf_agent(const float * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t * p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stf_agent(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sth_agent(uint16_t * p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* f32 -> bf16, round to nearest even; NaN stays a (quiet) NaN */
__device__ __forceinline__ uint32_t chain_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float chain_f16(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float) v;
}

/* bf16(gelu(g) * u) with the exact-erf gelu of model.rs:253-258 (erf in
 * f64, cast to f32). Not inlined: the erf polynomial's constants would
 * otherwise be hoisted out of the op loop and held in registers for the
 * whole launch. */
__device__ __attribute__((noinline)) uint32_t chain_gelu_mul_bf16(float g, float u) {
    const double e = erf((double) g * 0.70710678118654752440);
    return chain_bf16(0.5f * g * (1.0f + (float) e) * u);
}

/* One macro step of a two-stage unit (vq_tile.h's mstep for one bf16
 * column): every LDS read of the step, the 16 codeword gathers and the x
 * operands, is issued before the first MFMA, so the gathers' latencies
 * overlap instead of each MFMA waiting for its own. */
__device__ __forceinline__ void chain_step(const Words<2, 0, 0> & Wd, const uint8_t * cb, uint32_t cbb,
                                           const uint8_t * xb, f4 * acc) {
    h4 cw[8][2], b[8];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint8_t * c = cb + s * cbb;
        const uint32_t w0 = Wd.w[s][0], w1 = Wd.w[s][1], w2 = Wd.w[s][2];
        cw[0][s] = *(const h4 *) (c + cw_addr<0>(w0, w1, w2));
        cw[1][s] = *(const h4 *) (c + cw_addr<1>(w0, w1, w2));
        cw[2][s] = *(const h4 *) (c + cw_addr<2>(w0, w1, w2));
        cw[3][s] = *(const h4 *) (c + cw_addr<3>(w0, w1, w2));
        cw[4][s] = *(const h4 *) (c + cw_addr<4>(w0, w1, w2));
        cw[5][s] = *(const h4 *) (c + cw_addr<5>(w0, w1, w2));
        cw[6][s] = *(const h4 *) (c + cw_addr<6>(w0, w1, w2));
        cw[7][s] = *(const h4 *) (c + cw_addr<7>(w0, w1, w2));
    }
#pragma unroll
    for (int t = 0; t < 8; t++) b[t] = *(const h4 *) (xb + 8 * t);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 8; t++) {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x16f16(cw[t][0], b[t], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x16f16(cw[t][1], b[t], acc[1], 0, 0, 0);
    }
}

/* A workgroup's share of an op: ns matrix slots (0, 1, or 2 for a pair), the
 * matrix of each, and the tile range [t0, t0 + nt) it owns in each. */
struct Share {
    int ns, m0, m1, t0, nt;
};

__device__ __forceinline__ Share share_of(KOp & O, int wg, int G) {
    Share S;
    S.ns = 0; S.m0 = 0; S.m1 = 0; S.t0 = 0; S.nt = 0;
    if (O.pair) {
        const int T = O.mat[0].tiles;
        S.t0 = (int) ((uint32_t) (wg * T) / (uint32_t) G);
        S.nt = (int) ((uint32_t) ((wg + 1) * T) / (uint32_t) G) - S.t0;
        S.ns = S.nt > 0 ? 2 : 0;
        S.m1 = 1;
        return S;
    }
    for (int k = 0; k < O.nmat; k++) {
        const int w0 = O.mat[k].wg0, nw = O.mat[k].nwg;
        if (wg >= w0 && wg < w0 + nw) {
            const int lw = wg - w0, T = O.mat[k].tiles;
            S.m0 = k;
            S.t0 = (int) ((uint32_t) (lw * T) / (uint32_t) nw);
            S.nt = (int) ((uint32_t) ((lw + 1) * T) / (uint32_t) nw) - S.t0;
            S.ns = S.nt > 0 ? 1 : 0;
        }
    }
    return S;
}

template <int W, int R>
__global__ __launch_bounds__(W * 64) void vq_chain_kernel(const ChainOp * __restrict__ ops, int nops,
                                                           uint32_t * flags, uint32_t * err) {
    constexpr int NT = W * 64;
    constexpr int XGk = (kChainMaxCols / 4 + NT - 1) / NT;   /* 4-element groups of x per thread */
    constexpr int KC = (kChainMaxChunks + NT - 65) / (NT - 64);  /* codebook chunks per staging thread: one batch */
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint32_t * xr = (uint32_t *) (lds + kChainLds - kChainTop);       /* range flags (32 words) */
    double * nrm = (double *) (lds + kChainLds - kChainTop + 256);    /* norm partials, one per wave */
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   /* uniform in the wave */
    const int m16 = lane & 15, q = lane >> 4;
    const int wg = blockIdx.x, G = gridDim.x;
    /* ops every workgroup had published before this launch (all equal) */
    const uint32_t base = ld_agent(flags + wg);
    KOp * kops = (KOp *) ops;

    /* ---- index-word streaming. Each wave keeps R macro steps of index
     * words in flight in a ring, slot k always holding a step k mod R of the
     * current op. An op gives every wave pad >= R steps (its real steps
     * rounded up to a multiple of R; a wave with no unit re-reads one
     * address), so during op i's loop the refills load op i's own steps R ..
     * pad - 1 (cursor A) and then op i + 1's first R steps (cursor B). Both
     * cursors keep their op's record in registers; B's is read during op i's
     * staging, where the workgroup waits anyway, so no table read falls
     * inside a step loop, and every step issues exactly two loads, so each
     * use waits only for its own words. ---- */
    struct Cur {
        const uint8_t * s00;   /* stream bases: slot 0 stage 0, slot 0 stage 1, slot 1 ... */
        const uint8_t * s01;
        const uint8_t * s10;
        const uint8_t * s11;
        const uint8_t * p0;    /* lane pointers of the current unit at step 0 */
        const uint8_t * p1;
        int rows0, rows1, t0, nt, C, lgS, MP, msc, mrow, real, pad, k, j, pos;
    };
    auto units_of = [&](KOp & O, const Share & S) {
        const int U = S.ns * S.nt * O.C;
        return U > wave ? (U - wave + W - 1) / W : 0;
    };
    auto enter_unit = [&](Cur & c) {
        const int us = c.nt * c.C;
        const int u = wave + c.k * W;
        const int slot = u >= us ? 1 : 0;
        const int rem = u - slot * us;
        const int tl = rem / c.C, cc = rem - tl * c.C;
        const int rows = slot ? c.rows1 : c.rows0;
        const int row = min((c.t0 + tl) * (16 >> c.lgS) + (m16 >> c.lgS), rows - 1);
        const int ms0 = (m16 & ((1 << c.lgS) - 1)) * c.MP + cc * c.msc;
        const size_t off = (size_t) row * c.mrow + 48 * ms0 + 12 * q;
        c.p0 = (slot ? c.s10 : c.s00) + off;
        c.p1 = (slot ? c.s11 : c.s01) + off;
    };
    /* cursor at step 0 of op j (j >= nops: a cursor that re-reads the op table) */
    auto cur_init = [&](Cur & c, int j) {
        c.k = 0; c.j = 0; c.pos = 0;
        c.real = 0; c.pad = R;
        c.p0 = (const uint8_t *) ops;
        c.p1 = (const uint8_t *) ops;
        if (j >= nops) return;
        KOp & O = kops[j];
        const Share S = share_of(O, wg, G);
        const int nu = units_of(O, S);
        c.msc = O.msc; c.C = O.C; c.lgS = O.lgS; c.MP = O.M >> O.lgS; c.mrow = (int) O.mrow;
        c.t0 = S.t0; c.nt = S.nt;
        c.rows0 = O.mat[S.m0].rows; c.rows1 = O.mat[S.m1].rows;
        c.s00 = O.mat[S.m0].st[0] + O.mat[S.m0].stream_off;
        c.s01 = O.mat[S.m0].st[1] + O.mat[S.m0].stream_off;
        c.s10 = O.mat[S.m1].st[0] + O.mat[S.m1].stream_off;
        c.s11 = O.mat[S.m1].st[1] + O.mat[S.m1].stream_off;
        c.real = nu * c.msc;
        c.pad = max(R, (c.real + R - 1) & ~(R - 1));
        if (nu > 0) enter_unit(c);
    };
    /* the step a cursor points at, as two stream addresses */
    auto cur_p0 = [&](const Cur & c) { return c.p0 + 48 * c.j; };
    auto cur_p1 = [&](const Cur & c) { return c.p1 + 48 * c.j; };
    /* advance a cursor by one step (past the op's last real step it stays) */
    auto cur_next = [&](Cur & c) {
        if (c.pos + 1 < c.real && ++c.j == c.msc) {
            c.j = 0;
            c.k++;
            enter_unit(c);
        }
        c.pos++;
    };
    /* one ring slot's two loads (stage 0 and stage 1 words) */
    auto ring_load = [&](Words<2, 0, 0> & Wd, const uint8_t * a0, const uint8_t * a1) {
        const uint32_t * p0 = (const uint32_t *) a0;
        const uint32_t * p1 = (const uint32_t *) a1;
        Wd.w[0][0] = p0[0]; Wd.w[0][1] = p0[1]; Wd.w[0][2] = p0[2];
        Wd.w[1][0] = p1[0]; Wd.w[1][1] = p1[1]; Wd.w[1][2] = p1[2];
    };
    auto cur_load = [&](Cur & c, Words<2, 0, 0> & Wd) {
        ring_load(Wd, cur_p0(c), cur_p1(c));
        cur_next(c);
    };

    bool dead = false;
    Cur A, B;
    cur_init(A, 0);
    Words<2, 0, 0> w[R];
#pragma unroll
    for (int k = 0; k < R; k++) cur_load(A, w[k]);

    for (int i = 0; i < nops; i++) {
        KOp & O = kops[i];
        const Share S = share_of(O, wg, G);
        const int nu = units_of(O, S);
        const int msc = O.msc, C = O.C, lgS = O.lgS, rpt = 16 >> lgS;
        const int nreal = nu * msc, npad = max(R, (nreal + R - 1) & ~(R - 1));
        const int nrow = S.nt * rpt;          /* rows per slot */
        const uint32_t cbb = O.cbb, cbm = 2 * cbb;
        uint8_t * lx = lds + O.xoff;
        float * red = (float *) (lds + O.roff) + wave * (16 * 17);
        float * P = (float *) (lds + O.poff);

        /* cursor B: the next op's first steps */
        cur_init(B, i + 1);

        /* (c) the epilogue's row constants: gains of both stages and, when it
         * was published two or more ops back, the addend (read before the wait) */
        const int erow = tid < nrow ? S.t0 * rpt + tid : 0;
        float g00 = 0.f, g01 = 0.f, g10 = 0.f, g11 = 0.f, ya = 0.f;
        if (S.ns > 0 && tid < nrow) {
            const __attribute__((address_space(4))) ChainMat & A = O.mat[S.m0];
            const int r0 = min(erow, A.rows - 1);
            g00 = chain_f16(*(const uint16_t *) (A.st[0] + O.gain_off + 2 * r0));
            g01 = chain_f16(*(const uint16_t *) (A.st[1] + O.gain_off + 2 * r0));
            if (A.yadd && O.yadd_early) ya = ldf_agent(A.yadd + r0);
            if (S.ns > 1) {
                const __attribute__((address_space(4))) ChainMat & B = O.mat[S.m1];
                const int r1 = min(erow, B.rows - 1);
                g10 = chain_f16(*(const uint16_t *) (B.st[0] + O.gain_off + 2 * r1));
                g11 = chain_f16(*(const uint16_t *) (B.st[1] + O.gain_off + 2 * r1));
            }
        }

        /* (a) wave 0 waits until every workgroup has finished the ops this
         * one reads (after one wait has given up, the workgroup waits no
         * more); meanwhile the other waves stage this op's codebooks: the
         * previous op's gathers ended before its epilogue barrier */
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));
        if (wave == 0) {
            if (O.dep > 0 && !dead) {
                const uint32_t target = base + (uint32_t) O.dep;
                uint32_t n = 0;
                while (true) {
                    /* four flags per lane, all requested before any is looked at */
                    uint32_t fv[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) fv[k] = ld_agent(flags + min(4 * lane + k, G - 1));
                    bool ok = true;
#pragma unroll
                    for (int k = 0; k < 4; k++) ok &= (int) (fv[k] - target) >= 0;
                    if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
                    if (++n > kChainSpin) {
                        if (lane == 0) st_agent(err, 1u);
                        dead = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        } else if (S.ns > 0) {
            const int n16 = (int) (cbb >> 4);        /* 16-byte chunks per stage codebook */
            const int ncb = S.ns * 2 * n16;
            const uint8_t * c00 = O.mat[S.m0].st[0] + 24;
            const uint8_t * c01 = O.mat[S.m0].st[1] + 24;
            const uint8_t * c10 = O.mat[S.m1].st[0] + 24;
            const uint8_t * c11 = O.mat[S.m1].st[1] + 24;
            const int t = tid - 64;
            for (int b0 = 0; b0 < ncb; b0 += KC * (NT - 64)) {
                u4v cv[KC];
#pragma unroll
                for (int k = 0; k < KC; k++) {
                    const int ci = min(b0 + k * (NT - 64) + t, ncb - 1);
                    const int sl = ci >= 2 * n16 ? 1 : 0, r = ci - sl * 2 * n16, st = r >= n16 ? 1 : 0;
                    const uint8_t * src = sl ? (st ? c11 : c10) : (st ? c01 : c00);
                    cv[k] = ((const u4a *) src)[r - st * n16];
                }
#pragma unroll
                for (int k = 0; k < KC; k++) {
                    const int ci = b0 + k * (NT - 64) + t;
                    if (ci < ncb) ((u4v *) lds)[ci] = cv[k];
                }
            }
        }
        __syncthreads();
        if (S.ns == 1 && tid < nrow && !O.yadd_early) {
            const __attribute__((address_space(4))) ChainMat & A = O.mat[S.m0];
            if (A.yadd) ya = ldf_agent(A.yadd + min(erow, A.rows - 1));
        }

        /* (d) x: the transform, bf16, then f16 into LDS (264 bytes per 128
         * columns); every workgroup stages all of it */
        const int n4 = O.cols >> 2;
        uint32_t xb2[XGk][2];   /* bf16 pairs of this thread's groups */
        {
            /* every load of every group first, in one uniform branch, so the
             * groups share one memory round trip */
            uint32_t raw[XGk][4];
            if (O.xmode == kXBf16) {
#pragma unroll
                for (int k = 0; k < XGk; k++) {
                    const uint32_t * p = (const uint32_t *) O.x + 2 * min(k * NT + tid, n4 - 1);
                    raw[k][0] = ld_agent(p);
                    raw[k][1] = ld_agent(p + 1);
                }
            } else {
#pragma unroll
                for (int k = 0; k < XGk; k++) {
                    const uint32_t * p = (const uint32_t *) O.x + 4 * min(k * NT + tid, n4 - 1);
#pragma unroll
                    for (int e = 0; e < 4; e++) raw[k][e] = ld_agent(p + e);
                }
            }
            float xv[XGk][4];
#pragma unroll
            for (int k = 0; k < XGk; k++) {
                if (O.xmode == kXBf16) {
                    xv[k][0] = __uint_as_float(raw[k][0] << 16); xv[k][1] = __uint_as_float(raw[k][0] & 0xffff0000u);
                    xv[k][2] = __uint_as_float(raw[k][1] << 16); xv[k][3] = __uint_as_float(raw[k][1] & 0xffff0000u);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) xv[k][e] = __uint_as_float(raw[k][e]);
                }
            }
            float inv = 1.0f;
            if (O.xmode == kXNorm) {
                double ss = 0.0;
#pragma unroll
                for (int k = 0; k < XGk; k++)
                    if (k * NT + tid < n4)
#pragma unroll
                        for (int e = 0; e < 4; e++) ss += (double) xv[k][e] * (double) xv[k][e];
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
                if (lane == 0) nrm[wave] = ss;
                __syncthreads();
                double tot = 0.0;
#pragma unroll
                for (int k = 0; k < W; k++) tot += nrm[k];
                inv = (float) (1.0 / sqrt(tot / (double) O.cols + (double) O.eps));
            }
            uint32_t xm = 0;
#pragma unroll
            for (int k = 0; k < XGk; k++) {
                const int e4 = k * NT + tid;
                uint32_t b[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float v = xv[k][e];
                    if (O.xmode == kXNorm) v = v * inv * (O.nw ? O.nw[4 * min(e4, n4 - 1) + e] : 1.0f);
                    b[e] = O.xmode == kXBf16 ? __float_as_uint(v) >> 16 : chain_bf16(v);
                    if (e4 < n4) xm = max(xm, (b[e] << 16) & 0x7fffffffu);
                }
                xb2[k][0] = b[0] | (b[1] << 16);
                xb2[k][1] = b[2] | (b[3] << 16);
                if (O.xout && wg == 0 && e4 < n4) {
                    uint32_t * xo = (uint32_t *) O.xout + 2 * e4;
                    st_agent(xo, xb2[k][0]);
                    st_agent(xo + 1, xb2[k][1]);
                }
            }
            xr_note(xr, xm);
        }
        auto put_x = [&](int k, float sc) {
            const int e4 = k * NT + tid;
            if (e4 >= n4) return;
            const int e = 4 * e4;
            h4 v;
            v[0] = (_Float16) (__uint_as_float(xb2[k][0] << 16) * sc);
            v[1] = (_Float16) (__uint_as_float(xb2[k][0] & 0xffff0000u) * sc);
            v[2] = (_Float16) (__uint_as_float(xb2[k][1] << 16) * sc);
            v[3] = (_Float16) (__uint_as_float(xb2[k][1] & 0xffff0000u) * sc);
            *(h4 *) (lx + 264 * (e >> 7) + 2 * (e & 127)) = v;
        };
#pragma unroll
        for (int k = 0; k < XGk; k++) put_x(k, 1.0f);
        __syncthreads();
        /* x outside f16's comfortable range: stage it again as x * 2^-xk and
         * scale the sums back (both exact) */
        int xk = 0;
        if (xr_out(xr)) {
            uint32_t fm = 0;
#pragma unroll
            for (int k = 0; k < XGk; k++)
                if (k * NT + tid < n4) {
                    fm = max(fm, xr_fin((xb2[k][0] << 16) & 0x7fffffffu));
                    fm = max(fm, xr_fin(xb2[k][0] & 0x7fff0000u));
                    fm = max(fm, xr_fin((xb2[k][1] << 16) & 0x7fffffffu));
                    fm = max(fm, xr_fin(xb2[k][1] & 0x7fff0000u));
                }
            xk = xr_shift(xr, fm);
            if (xk) {
                const float sc = __builtin_ldexpf(1.0f, -xk);
#pragma unroll
                for (int k = 0; k < XGk; k++) put_x(k, sc);
                __syncthreads();
            }
        }

        /* (e) the wave's units: its nreal steps of this op, padded to npad */
        f4 acc[2];
        acc[0] = f4{0.f, 0.f, 0.f, 0.f};
        acc[1] = acc[0];
        int ck = 0, cj = 0;
        int cslot = 0, ctl = 0, cc = 0;
        const uint8_t * xbase = lx;
        auto enter_cunit = [&]() {
            const int us = S.nt * C;
            const int u = wave + ck * W;
            cslot = u >= us ? 1 : 0;
            const int rem = u - cslot * us;
            ctl = rem / C;
            cc = rem - ctl * C;
            const int hp = m16 < (1 << lgS) ? m16 : 0;   /* B column m16 carries part m16 */
            xbase = lx + 264 * (hp * (O.M >> lgS) + cc * msc) + 64 * q;
        };
        auto end_unit = [&]() {
            /* C[m][n] -> red; row r of the tile is the sum over parts h of
             * C[r*S + h][h], added in part order, per stage */
#pragma unroll
            for (int s = 0; s < 2; s++) {
#pragma unroll
                for (int k = 0; k < 4; k++) red[(4 * q + k) * 17 + m16] = acc[s][k];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (lane < rpt) {
                    float v = 0.0f;
                    for (int h = 0; h < (1 << lgS); h++) v += red[((lane << lgS) + h) * 17 + h];
                    P[((cslot * nrow + ctl * rpt + lane) * C + cc) * 2 + s] = v;
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            acc[0] = f4{0.f, 0.f, 0.f, 0.f};
            acc[1] = acc[0];
            cj = 0;
            if (++ck < nu) enter_cunit();
        };
        if (nu > 0) enter_cunit();
        /* every ring load was issued before the staging, which waited for
         * later loads: say so to the compiler, whose count of outstanding
         * loads then starts from zero and stays exact around the loop */
        __builtin_amdgcn_s_waitcnt(0);
        for (int g = 0; g < npad; g += R) {
#pragma unroll
            for (int k = 0; k < R; k++) {
                if (g + k < nreal) {
                    chain_step(w[k], lds + cslot * cbm, cbb, xbase + 264 * cj, acc);
                    if (++cj == msc) end_unit();
                }
                /* one load pair from either cursor (a select, not a branch,
                 * so the slot is written by one instruction pair) */
                const bool fromA = g + k + R < npad;
                ring_load(w[k], fromA ? cur_p0(A) : cur_p0(B), fromA ? cur_p1(A) : cur_p1(B));
                if (fromA) cur_next(A);
                else cur_next(B);
            }
        }
        A = B;

        /* (f) the epilogue: K chunks added in order, gains per stage, the
         * addend; then publish */
        __syncthreads();
        if (S.ns > 0 && tid < nrow) {
            float sum[2][2];
#pragma unroll
            for (int sl = 0; sl < 2; sl++)
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    float v = 0.0f;
                    if (sl < S.ns)
                        for (int c = 0; c < C; c++) v += P[((sl * nrow + tid) * C + c) * 2 + s];
                    sum[sl][s] = v;
                }
            const float v0 = xr_unscale(g00 * sum[0][0] + g01 * sum[0][1], xk);
            if (S.ns == 1) {
                const __attribute__((address_space(4))) ChainMat & A = O.mat[S.m0];
                if (erow < A.rows) {
                    const float y = ya + v0;
                    if (A.y) stf_agent(A.y + erow, y);
                    if (A.ybf) sth_agent(A.ybf + erow, (uint16_t) chain_bf16(y));
                }
            } else {
                const float v1 = xr_unscale(g10 * sum[1][0] + g11 * sum[1][1], xk);
                const __attribute__((address_space(4))) ChainMat & A = O.mat[0];
                const __attribute__((address_space(4))) ChainMat & B = O.mat[1];
                if (erow < A.rows) {
                    if (A.y) stf_agent(A.y + erow, v0);
                    if (B.y) stf_agent(B.y + erow, v1);
                    if (O.act) sth_agent(O.act + erow, (uint16_t) chain_gelu_mul_bf16(v0, v1));
                }
            }
        }
        /* every store of this workgroup acknowledged, then the flag */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) st_agent(flags + wg, base + (uint32_t) (i + 1));
    }
}

/* ------------------------------------------------------------------------ */
/* Host side.                                                                */
/* ------------------------------------------------------------------------ */

struct Chain {
    std::vector<ChainOp> ops;
    ChainOp * dops = nullptr;
    uint32_t * flags = nullptr;   /* one word per workgroup, then the error word */
    int dev = -1;
    int G = 0;
    int built = 0;
    int waves = 16;
    int look = 2;                 /* macro steps of index words in flight per wave */
    int umin = 16;                /* units per workgroup the shape search aims for */
};

static int chain_alloc(Chain * c) {
    if (c->flags) return 0;
    hipError_t e = hipGetDevice(&c->dev);
    if (e != hipSuccess) return fail_hip("chain device", e);
    c->G = cu_count();
    if (c->G < 1 || c->G > 256) { set_error("a chain runs on 1..256 CUs, this device has %d", c->G); return -1; }
    e = hipMalloc((void **) &c->flags, 4 * (size_t) (c->G + 1));
    if (e != hipSuccess) return fail_hip("chain flags", e);
    e = hipMemset(c->flags, 0, 4 * (size_t) (c->G + 1));
    if (e != hipSuccess) return fail_hip("chain flags", e);
    return 0;
}

static int divides(int a, int b) { return b > 0 && a % b == 0; }

/* Shape of one op: parts per tile S, K chunks C and the unit length, plus
 * the workgroups of each matrix; the LDS offsets. */
static int chain_shape(Chain * c, ChainOp & O) {
    const int G = c->G, W = c->waves;
    const int M = O.M;
    long best = -1;
    int bS = 0, bC = 0;
    std::vector<int> bnwg(O.nmat, 0);
    for (int S = 1; S <= 16; S *= 2) {
        if (!divides(M, S)) continue;
        const int MP = M / S;
        std::vector<int> tiles(O.nmat), nwg(O.nmat, 1);
        for (int m = 0; m < O.nmat; m++) tiles[m] = (int) ((O.mat[m].rows * (long) S + 15) / 16);
        long maxT;
        if (O.pair) {
            maxT = (tiles[0] + G - 1) / G;
        } else {
            if (O.nmat > G) continue;
            /* give each next workgroup to the matrix with the most tiles per workgroup */
            for (int used = O.nmat; used < G; used++) {
                int wm = 0;
                long wv = -1;
                for (int m = 0; m < O.nmat; m++) {
                    const long v = (tiles[m] + nwg[m] - 1) / nwg[m];
                    if (v > wv) { wv = v; wm = m; }
                }
                if ((tiles[wm] + nwg[wm] - 1) / nwg[wm] <= 1 && nwg[wm] >= tiles[wm]) break;
                nwg[wm]++;
            }
            maxT = 0;
            for (int m = 0; m < O.nmat; m++) maxT = std::max(maxT, (long) (tiles[m] + nwg[m] - 1) / nwg[m]);
        }
        const int ns = O.pair ? 2 : 1;
        const long steps = maxT * MP * ns;
        if ((long) maxT * (16 / S) > (long) W * 64) continue;   /* one epilogue thread per row */
        /* the fewest K chunks that give every wave of the workgroup a unit */
        int Cc = 0;
        for (int cc = 1; cc <= MP; cc++) {
            if (!divides(MP, cc)) continue;
            Cc = cc;
            if (maxT * cc * ns >= c->umin) break;
        }
        const long cost = steps * 64 + S;   /* fewest steps on the busiest workgroup, then the smallest S */
        if (best < 0 || cost < best) {
            best = cost;
            bS = S; bC = Cc;
            for (int m = 0; m < O.nmat; m++) bnwg[m] = nwg[m];
        }
    }
    if (best < 0) { set_error("no chain shape for a %d-column op", O.cols); return -1; }
    O.lgS = 0;
    while ((1 << O.lgS) < bS) O.lgS++;
    O.C = bC;
    O.msc = M / bS / bC;
    int wg = 0;
    for (int m = 0; m < O.nmat; m++) {
        O.mat[m].tiles = (int) ((O.mat[m].rows * (long) bS + 15) / 16);
        if (O.pair) {
            O.mat[m].wg0 = 0;
            O.mat[m].nwg = G;
        } else {
            O.mat[m].wg0 = wg;
            O.mat[m].nwg = bnwg[m];
            wg += bnwg[m];
        }
    }
    /* LDS: codebooks of each slot, x, the reduction area, the partials */
    const int ns = O.pair ? 2 : 1;
    long maxT = 0;
    for (int m = 0; m < O.nmat; m++)
        maxT = std::max(maxT, (long) (O.mat[m].tiles + O.mat[m].nwg - 1) / O.mat[m].nwg);
    const uint32_t cb = ns * 2 * O.cbb;
    O.xoff = (cb + 15) & ~15u;
    O.roff = O.xoff + ((264 * (uint32_t) M + 8 + 15) & ~15u);
    O.poff = O.roff + (uint32_t) W * 16 * 17 * 4;
    const uint32_t pend = O.poff + (uint32_t) (ns * maxT * (16 >> O.lgS) * O.C * 2 * 4);
    if (pend > kChainLds - kChainTop) {
        set_error("a chain op of %d columns needs %u bytes of LDS", O.cols, pend);
        return -1;
    }
    return 0;
}

static int chain_build(Chain * c) {
    if (chain_alloc(c)) return -1;
    for (auto & O : c->ops) {
        if (O.nmat == 0) {
            O.lgS = 0; O.C = 1; O.msc = 1;
            O.xoff = 0;
            O.roff = O.poff = (uint32_t) (264 * O.M + 16);
            continue;
        }
        if (chain_shape(c, O)) return -1;
    }
    if (c->dops) { (void) hipFree(c->dops); c->dops = nullptr; }
    if (!c->ops.empty()) {
        const size_t bytes = sizeof(ChainOp) * c->ops.size();
        hipError_t e = hipMalloc((void **) &c->dops, bytes);
        if (e != hipSuccess) return fail_hip("chain op table", e);
        e = hipMemcpy(c->dops, c->ops.data(), bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail_hip("chain op table", e);
    }
    c->built = 1;
    return 0;
}

template <int W, int R>
static int chain_launch_w(Chain * c, hipStream_t s) {
    static int opted[64] = {0};
    const void * fn = (const void *) vq_chain_kernel<W, R>;
    if (c->dev >= 0 && c->dev < 64 && !opted[c->dev]) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) kChainLds);
        if (e != hipSuccess) return fail_hip("chain LDS opt-in", e);
        opted[c->dev] = 1;
    }
    launch_kernel(vq_chain_kernel<W, R>, dim3(c->G), dim3(W * 64), kChainLds, s, (const ChainOp *) c->dops,
                  (int) c->ops.size(), c->flags, c->flags + c->G);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("chain launch", e);
}

}  // namespace sparkmv

using namespace sparkmv;

extern "C" {

void * sparkmv_chain_create(void) { return new Chain(); }

void sparkmv_chain_destroy(void * chain) {
    Chain * c = (Chain *) chain;
    if (!c) return;
    if (c->dops) (void) hipFree(c->dops);
    if (c->flags) (void) hipFree(c->flags);
    delete c;
}

int sparkmv_chain_size(void * chain) { return chain ? (int) ((Chain *) chain)->ops.size() : -1; }

int sparkmv_chain_tune(void * chain, int waves, int look, int min_units) {
    Chain * c = (Chain *) chain;
    if (!c) { set_error("chain is null"); return -1; }
    if (waves != 8 && waves != 12 && waves != 16) { set_error("a chain runs 8, 12 or 16 waves per workgroup, not %d", waves); return -1; }
    if (look != 2 && look != 4) { set_error("a chain keeps 2 or 4 macro steps in flight per wave, not %d", look); return -1; }
    if (min_units < 1 || min_units > 1024) { set_error("min_units %d is outside 1..1024", min_units); return -1; }
    c->waves = waves;
    c->look = look;
    c->umin = min_units;
    c->built = 0;
    return 0;
}

int sparkmv_chain_add_vq(void * chain, const sparkmv_chain_matrix * mats, int nmat, int nstages, int dim, int nc,
                         int cols, int v3, const void * x, int x_mode, const float * norm_w, float eps,
                         uint16_t * x_out, uint16_t * act, int wait) {
    Chain * c = (Chain *) chain;
    if (!c || !mats) { set_error("chain or matrix list is null"); return -1; }
    if (nmat < 1 || nmat > kChainMats) { set_error("matrix count %d is outside 1..%d", nmat, kChainMats); return -1; }
    if (nstages != 2) { set_error("a chain op takes two residual stages, not %d", nstages); return -1; }
    if (dim != 4 || !v3) { set_error("a chain op takes DQV3 dim-4 stages (dim %d, v3 %d)", dim, v3); return -1; }
    if (bits_for(nc) != 12 || nc % 2) {
        set_error("a chain op takes 12-bit indices (an even codebook of 2050..4096 entries), not nc %d", nc);
        return -1;
    }
    if (cols < 128 || cols % 128 || cols > kChainMaxCols) {
        set_error("a chain op takes a multiple of 128 columns up to %d, not %d", kChainMaxCols, cols);
        return -1;
    }
    if (x_mode != 0 && x_mode != 1 && x_mode != 2) { set_error("unknown chain x mode %d", x_mode); return -1; }
    if (!x) { set_error("x is null"); return -1; }
    if (((uintptr_t) x & 3u)) { set_error("chain x must be 4-byte aligned"); return -1; }
    if (act && nmat != 2) { set_error("a gate/up pair has two matrices, not %d", nmat); return -1; }
    if (act && mats[0].rows != mats[1].rows) { set_error("a gate/up pair has equal row counts (%d, %d)", mats[0].rows, mats[1].rows); return -1; }
    ChainOp O;
    memset(&O, 0, sizeof O);
    const Layout L0 = make_layout(dim, nc, 1, cols, 1);
    for (int m = 0; m < nmat; m++) {
        const sparkmv_chain_matrix & A = mats[m];
        if (A.rows < 1) { set_error("matrix %d has %d rows", m, A.rows); return -1; }
        for (int s = 0; s < 2; s++) {
            if (!A.stages[s]) { set_error("matrix %d stage %d payload is null", m, s); return -1; }
            if ((uintptr_t) A.stages[s] & 3u) { set_error("matrix %d stage %d payload is not 4-byte aligned", m, s); return -1; }
        }
        if (!act && !A.y && !A.y_bf16) { set_error("matrix %d has no output", m); return -1; }
        O.mat[m].st[0] = (const uint8_t *) A.stages[0];
        O.mat[m].st[1] = (const uint8_t *) A.stages[1];
        O.mat[m].y = A.y;
        O.mat[m].ybf = A.y_bf16;
        O.mat[m].yadd = act ? nullptr : A.y_add;
        O.mat[m].rows = A.rows;
        O.mat[m].stream_off = (uint32_t) (L0.gain_off + 2 * (size_t) A.rows);
    }
    if (L0.mrow % 4 || L0.gain_off % 4) { set_error("chain row streams are not dword aligned"); return -1; }
    O.x = x;
    O.nw = norm_w;
    O.xout = x_out;
    O.act = act;
    O.eps = eps;
    O.nmat = nmat;
    O.pair = act ? 1 : 0;
    O.cols = cols;
    O.M = cols / 128;
    O.dep = wait ? (int) c->ops.size() : 0;
    O.xmode = x_mode;
    /* an addend written by the op just before this one is read after the
     * wait; any other (external, or two or more ops back) before it */
    O.yadd_early = 1;
    if (!c->ops.empty()) {
        const ChainOp & P = c->ops.back();
        for (int m = 0; m < nmat; m++) {
            if (!O.mat[m].yadd) continue;
            for (int k = 0; k < P.nmat; k++)
                if ((const void *) O.mat[m].yadd == (const void *) P.mat[k].y) O.yadd_early = 0;
        }
        if (!wait) O.yadd_early = 1;
    }
    O.gain_off = (uint32_t) L0.gain_off;
    O.mrow = (uint32_t) L0.mrow;
    O.cbb = (uint32_t) nc * 8u;
    c->ops.push_back(O);
    c->built = 0;
    return 0;
}

int sparkmv_chain_add_norm(void * chain, const float * x, int n, const float * norm_w, float eps, uint16_t * out,
                           int wait) {
    Chain * c = (Chain *) chain;
    if (!c || !x || !out) { set_error("chain, x or out is null"); return -1; }
    if (n < 128 || n % 128 || n > kChainMaxCols) { set_error("a chain norm takes a multiple of 128 values, not %d", n); return -1; }
    ChainOp O;
    memset(&O, 0, sizeof O);
    O.x = x;
    O.nw = norm_w;
    O.xout = out;
    O.eps = eps;
    O.cols = n;
    O.M = n / 128;
    O.msc = 1;
    O.C = 1;
    O.dep = wait ? (int) c->ops.size() : 0;
    O.xmode = kXNorm;
    c->ops.push_back(O);
    c->built = 0;
    return 0;
}

int sparkmv_chain_launch(void * chain, void * stream) {
    Chain * c = (Chain *) chain;
    if (!c) { set_error("chain is null"); return -1; }
    if (c->ops.empty()) { set_error("chain has no ops"); return -1; }
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail_hip("chain device", e);
    if (c->flags && dev != c->dev) { set_error("a chain runs on the device it was built on (%d, not %d)", c->dev, dev); return -1; }
    if (!c->built && chain_build(c)) return -1;
    hipStream_t s = (hipStream_t) stream;
    const int k = c->waves * 8 + c->look;
    switch (k) {
        case 8 * 8 + 2: return chain_launch_w<8, 2>(c, s);
        case 8 * 8 + 4: return chain_launch_w<8, 4>(c, s);
        case 12 * 8 + 2: return chain_launch_w<12, 2>(c, s);
        case 12 * 8 + 4: return chain_launch_w<12, 4>(c, s);
        case 16 * 8 + 4: return chain_launch_w<16, 4>(c, s);
        default: return chain_launch_w<16, 2>(c, s);
    }
}

/* 0 when every wait of every launch so far ended in time; -1 (message set)
 * after a wait gave up, with the flags cleared so the chain can run again.
 * Synchronizes the device. */
int sparkmv_chain_status(void * chain) {
    Chain * c = (Chain *) chain;
    if (!c) { set_error("chain is null"); return -1; }
    if (!c->flags) return 0;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail_hip("chain status", e);
    uint32_t w = 0;
    e = hipMemcpy(&w, c->flags + c->G, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail_hip("chain status", e);
    if (!w) return 0;
    (void) hipMemset(c->flags, 0, 4 * (size_t) (c->G + 1));
    set_error("a chain workgroup waited too long for the others (were all %d resident?)", c->G);
    return -1;
}

/* the shape the chain chose for op i: S, C, unit length, workgroups of matrix 0 */
int sparkmv_chain_op_shape(void * chain, int i, int * S, int * C, int * msc) {
    Chain * c = (Chain *) chain;
    if (!c || i < 0 || i >= (int) c->ops.size()) { set_error("no chain op %d", i); return -1; }
    if (!c->built && chain_build(c)) return -1;
    const ChainOp & O = c->ops[i];
    if (S) *S = 1 << O.lgS;
    if (C) *C = O.C;
    if (msc) *msc = O.msc;
    return 0;
}

}  // extern "C"
