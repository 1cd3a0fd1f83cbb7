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
 *    words through a ring of R macro steps that runs straight across unit and
 *    op boundaries: while a workgroup waits for the previous op's output, its
 *    next op's first index words are already in flight.
 *  - Outputs that a later op of the chain reads travel as self-validating
 *    words: 8 bytes, {payload, epoch}, written with one agent-scope vector
 *    store (an f32 value per word, or a pair of bf16 values). The epoch is
 *    the launch's base plus the producing op's index plus one, so a word is
 *    current exactly when its upper half equals the epoch its reader
 *    expects. A reader's load of its input IS its wait: it loads its words
 *    with agent-scope loads and loads again those whose epoch is not yet
 *    there. No acknowledgement, flag or fence sits between a producer's
 *    multiply and its reader's (one memory round trip per dependent op).
 *    Which outputs are published, and where each op's input comes from, is
 *    found when the chain is built by matching pointers: an input that is
 *    an earlier op's output is read from that op's words, anything else is
 *    external and read as plain memory.
 *  - Every wait is bounded: past kChainSpin polls the workgroup sets the
 *    error word and stops waiting for the rest of the launch, so the launch
 *    always ends and the host reports the failure.
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

#include <algorithm>
#include <vector>

namespace sparkmv {

constexpr int kChainMats = 4;
constexpr uint32_t kChainSpin = 1u << 19; /* polls before a wait gives up (about half a second) */
constexpr uint32_t kChainLds = 160 * 1024;
constexpr uint32_t kChainTop = 512;      /* range flags, norm partials and the give-up flag at the top of LDS */
constexpr int kChainMaxXw = 6144;        /* words of x an op reads: f32 values, or bf16 pairs */
constexpr int kChainStamps = 10;         /* trace words per workgroup and op */

enum { kXBf16 = 0, kXF32 = 1, kXNorm = 2 };
/* where an op's x comes from: external bf16 pairs or f32 values, or an
 * earlier op's published words (f32 values or bf16 pairs) */
enum { kSrcBf16 = 0, kSrcF32 = 1, kSrcWordF32 = 2, kSrcWordBf16 = 3 };

struct ChainMat {
    const uint8_t * st[2];   /* stage payloads */
    float * y;               /* f32 output (may be null) */
    uint16_t * ybf;          /* bf16 copy of the output (may be null) */
    uint64_t * pf;           /* published y: {f32, epoch} per row (null: no op of the chain reads y) */
    uint64_t * pb;           /* published bf16(y): {bf16 pair, epoch} per two rows */
    const void * yadd;       /* y = yadd + W x when set: f32 values, or published f32 words */
    int yadd_op;             /* 0: yadd is external; else the producing op's index + 1 */
    int rows, tiles, wg0, nwg;
    uint32_t stream_off;     /* gain_off + 2 * rows */
};

struct ChainOp {
    ChainMat mat[kChainMats];
    const void * x;          /* external x, or the producer's published words */
    const float * nw;        /* rms_norm weight (null = 1) */
    uint16_t * xout;         /* workgroup 0 writes the staged bf16 x here (may be null) */
    uint16_t * act;          /* a pair's bf16 gelu(y0) * y1 (may be null) */
    uint64_t * pact;         /* the same, published: {bf16 pair, epoch} per two rows */
    float eps;
    int nmat, pair, cols, M, lgS, C, msc, xmode;
    int xsrc, x_op, nxw;     /* x's source kind, producing op's index + 1, words to read */
    uint32_t gain_off, mrow, cbb;   /* cbb: LDS bytes per stage codebook, nc * 8 rounded up to 1 KB */
    uint32_t cbr;                   /* codebook bytes, nc * 8 */
    uint32_t xoff, roff, poff;      /* LDS byte offsets of x, the reduction area, the partials */
};

/* The op table is read through the constant address space: it does not
 * change during a launch, so every field is a scalar load even after the
 * kernel's own agent-scope stores (which would otherwise keep the compiler
 * from proving the table unchanged, and turn the reads into vector loads
 * that wait for every outstanding load). */
typedef const __attribute__((address_space(4))) ChainOp KOp;
typedef const __attribute__((address_space(4))) ChainMat KMat;

__device__ __forceinline__ uint32_t ld_agent(const uint32_t * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t * p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* A published word: one 8-byte agent-scope access, so its two halves are
 * always seen together. */
template <typename P>
__device__ __forceinline__ uint64_t ld_word(P p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename P>
__device__ __forceinline__ void st_word(P p, uint32_t payload, uint32_t ep) {
    __hip_atomic_store(p, ((uint64_t) ep << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t word_ep(uint64_t w) { return (uint32_t) (w >> 32); }

/* A table field read once and then held in a scalar register: the asm keeps
 * the compiler from re-reading it from the table (a scalar load and a wait
 * each time) where it would rather not hold a register. */
template <typename T>
__device__ __forceinline__ T pin(T v) {
    asm volatile("" : "+s"(v));
    return v;
}
/* the same for a pointer, which stays a global-memory pointer */
template <typename T>
using gptr = __attribute__((address_space(1))) T *;
template <typename T>
__device__ __forceinline__ gptr<T> gpin(T * p) {
    uint64_t u = (uint64_t) p;
    asm volatile("" : "+s"(u));
    return (gptr<T>) u;
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

/* One workgroup's share of one op, resolved when the chain is built so
 * the kernel reads it as one burst of independent scalar loads: ns matrix
 * slots (0, 1, or 2 for a gate/up pair), the tile range [t0, t0 + nt) it
 * owns in each, and the pointers of the slots' matrices. */
struct ChainWg {
    const uint8_t * strm[4];   /* index streams: slot 0 stage 0, slot 0 stage 1, slot 1 stage 0, slot 1 stage 1 */
    const uint8_t * cb[4];     /* codebooks, in the same order */
    const uint8_t * gain[4];   /* gains, in the same order */
    float * y[2];              /* the slots' f32 outputs (may be null) */
    uint16_t * ybf;            /* slot 0's bf16 copy (may be null) */
    uint64_t * pf;             /* slot 0's published f32 words (may be null) */
    uint64_t * pb;             /* slot 0's published bf16 pairs (may be null) */
    const void * yadd;         /* slot 0's addend: f32 values, or published words (yadd_op > 0) */
    int ns, t0, nt, rows0, rows1, yadd_op;
    int pad[6];
};
static_assert(sizeof(ChainWg) == 192, "a workgroup record is three 64-byte scalar loads");
typedef const __attribute__((address_space(4))) ChainWg KWg;

template <int W, int R>
__global__ __launch_bounds__(W * 64) void vq_chain_kernel(const ChainOp * __restrict__ ops,
                                                           const ChainWg * __restrict__ wgs, int nops,
                                                           uint32_t * flags, uint32_t * err, uint32_t * trace) {
    constexpr int NT = W * 64;
    constexpr int NXK = (kChainMaxXw + NT - 1) / NT;         /* x words per thread */
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint32_t * xr = (uint32_t *) (lds + kChainLds - kChainTop);          /* range flags (32 words) */
    double * nrm = (double *) (lds + kChainLds - kChainTop + 256);       /* norm partials, one per wave */
    uint32_t * gaveup = (uint32_t *) (lds + kChainLds - kChainTop + 384);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   /* uniform in the wave */
    const int m16 = lane & 15, q = lane >> 4;
    const int wg = blockIdx.x, G = gridDim.x;
    /* ops every workgroup had published before this launch (all equal); op
     * i of this launch publishes epoch base + i + 1 */
    const uint32_t base = ld_agent(flags + wg);
    KOp * kops = (KOp *) ops;
    KWg * kwgs = (KWg *) wgs;
    /* phase trace (null: off): per workgroup and op, the 100 MHz clock at
     * the op's start (0), x arrived (1), x staged (2), the step loop entered
     * (3), wave 0's steps done (4), every unit done (5), the epilogue's
     * stores issued (6), x requested (7) */
    auto stamp = [&](int i, int k) {
        if (trace && tid == 0) {
            uint32_t * t = trace + ((size_t) wg * nops + i) * kChainStamps;
            t[k] = (uint32_t) __builtin_amdgcn_s_memrealtime();
            /* the shader clock beside the 100 MHz one at the op's start and end */
            if (k == 0) t[8] = (uint32_t) __builtin_amdgcn_s_memtime();
            if (k == 6) t[9] = (uint32_t) __builtin_amdgcn_s_memtime();
        }
    };
    if (tid == 0) *gaveup = 0u;
    __syncthreads();

    /* ---- index-word streaming. Each wave keeps R macro steps of index
     * words in flight in a ring, slot k always holding a step k mod R of the
     * current op. An op gives every wave pad >= R steps (its real steps
     * rounded up to a multiple of R; a wave with no unit re-reads one
     * address), so during op i's loop the refills load op i's own steps R ..
     * pad - 1 (cursor A) and then op i + 1's first R steps (cursor B). Both
     * cursors keep their op's record in registers; B's is read before op i's
     * staging, so no table read falls inside a step loop, and every step
     * issues exactly two loads, so each use waits only for its own words. */
    struct Cur {
        const uint8_t * p0;    /* lane pointers of the current unit at step 0 */
        const uint8_t * p1;
        int op, real, msc, k, j, pos;
    };
    auto units_of = [&](KOp & O, KWg & Wr) {
        const int U = Wr.ns * Wr.nt * O.C;
        return U > wave ? (U - wave + W - 1) / W : 0;
    };
    /* the lane pointers of unit k of op c.op (its fields reread from the
     * tables, which the scalar cache holds by then) */
    auto enter_unit = [&](Cur & c) {
        KOp & O = kops[c.op];
        KWg & Wr = kwgs[(size_t) c.op * G + wg];
        const int C = O.C, lgS = O.lgS, MP = O.M >> lgS;
        const int us = Wr.nt * C;
        const int u = wave + c.k * W;
        const int slot = u >= us ? 1 : 0;
        const int rem = u - slot * us;
        const int tl = rem / C, cc = rem - tl * C;
        const int rows = slot ? Wr.rows1 : Wr.rows0;
        const int row = min((Wr.t0 + tl) * (16 >> lgS) + (m16 >> lgS), rows - 1);
        const int ms0 = (m16 & ((1 << lgS) - 1)) * MP + cc * c.msc;
        const size_t off = (size_t) row * O.mrow + 48 * ms0 + 12 * q;
        c.p0 = (slot ? Wr.strm[2] : Wr.strm[0]) + off;
        c.p1 = (slot ? Wr.strm[3] : Wr.strm[1]) + off;
    };
    /* cursor at step 0 of op j (j >= nops: a cursor that re-reads the op table) */
    auto cur_init = [&](Cur & c, int j) {
        c.k = 0; c.j = 0; c.pos = 0;
        c.real = 0; c.msc = 1; c.op = j;
        c.p0 = (const uint8_t *) ops;
        c.p1 = (const uint8_t *) ops;
        if (j >= nops) return;
        KOp & O = kops[j];
        KWg & Wr = kwgs[(size_t) j * G + wg];
        const int nu = units_of(O, Wr);
        c.msc = O.msc;
        c.real = nu * c.msc;
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

    /* The epilogue's row constants of op j: the raw gains of both stages of
     * each slot and the addend (its published word, or its plain value).
     * Requested one op ahead, after the previous op's steps, so that they
     * have landed by the time x has. */
    auto load_consts = [&](int j, uint32_t * g, uint64_t & yw, float & yp) {
        g[0] = g[1] = g[2] = g[3] = 0u;
        yw = 0;
        yp = 0.f;
        if (j >= nops) return;
        KOp & O = kops[j];
        KWg & Wr = kwgs[(size_t) j * G + wg];
        const int rp = 16 >> O.lgS, nr = Wr.nt * rp;
        if (Wr.ns > 0 && tid < nr) {
            const int r0 = min(Wr.t0 * rp + tid, Wr.rows0 - 1);
            g[0] = *(const uint16_t *) (Wr.gain[0] + 2 * r0);
            g[1] = *(const uint16_t *) (Wr.gain[1] + 2 * r0);
            if (Wr.ns == 1 && Wr.yadd) {
                if (Wr.yadd_op) yw = ld_word((const uint64_t *) Wr.yadd + r0);
                else yp = ((const float *) Wr.yadd)[r0];
            }
            if (Wr.ns > 1) {
                const int r1 = min(Wr.t0 * rp + tid, Wr.rows1 - 1);
                g[2] = *(const uint16_t *) (Wr.gain[2] + 2 * r1);
                g[3] = *(const uint16_t *) (Wr.gain[3] + 2 * r1);
            }
        }
    };
    uint32_t gr[4];
    uint64_t yword;
    float yplain;
    load_consts(0, gr, yword, yplain);

    bool dead = false;   /* a wait of this workgroup gave up: wait no more in this launch */
    Cur A, B;
    cur_init(A, 0);
    Words<2, 0, 0> w[R];
#pragma unroll
    for (int k = 0; k < R; k++) cur_load(A, w[k]);

    typedef __attribute__((address_space(3))) void lds_void;

    for (int i = 0; i < nops; i++) {
        KOp & O = kops[i];
        KWg & Wr = kwgs[(size_t) i * G + wg];
        const int ns = Wr.ns;
        const int nu = units_of(O, Wr);
        const int msc = O.msc, C = O.C, lgS = O.lgS, rpt = 16 >> lgS;
        const int nreal = nu * msc, npad = max(R, (nreal + R - 1) & ~(R - 1));
        const int nrow = Wr.nt * rpt;         /* rows per slot */
        const uint32_t cbb = O.cbb, cbm = 2 * cbb;
        const uint32_t ep = base + (uint32_t) (i + 1);
        /* workgroups with rows stage x; so does workgroup 0 when x_out is
         * set (it writes the copy) and for a norm op (no matrix) */
        const bool stages_x = ns > 0 || (wg == 0 && (O.xout || O.nmat == 0));
        uint8_t * lx = lds + O.xoff;
        float * red = (float *) (lds + O.roff) + wave * (16 * 17);
        float * P = (float *) (lds + O.poff);
        stamp(i, 0);

        /* (a) x first: its words (this read is the wait for a published
         * input); every load unconditional, so the waits count exactly */
        const int nxw = O.nxw, xsrc = O.xsrc;
        const bool words = xsrc >= kSrcWordF32;
        const bool f32v = xsrc == kSrcF32 || xsrc == kSrcWordF32;   /* one value per word */
        uint64_t xw[NXK];
        if (stages_x) {
            if (words) {
                const uint64_t * xp = (const uint64_t *) O.x;
#pragma unroll
                for (int k = 0; k < NXK; k++) xw[k] = ld_word(xp + min(k * NT + tid, nxw - 1));
            } else {
                const uint32_t * xp = (const uint32_t *) O.x;
#pragma unroll
                for (int k = 0; k < NXK; k++) xw[k] = xp[min(k * NT + tid, nxw - 1)];
            }
        }
        /* the norm's weights with x (they do not depend on it), so that no
         * load falls between x's arrival and its staging; a norm without
         * weights (a null pointer) multiplies by 1 */
        float nv[NXK];
#pragma unroll
        for (int k = 0; k < NXK; k++) nv[k] = 1.0f;
        if (stages_x && O.xmode == kXNorm && O.nw) {
            const gptr<const float> nwp = gpin(O.nw);
#pragma unroll
            for (int k = 0; k < NXK; k++) nv[k] = nwp[min(k * NT + tid, nxw - 1)];
        }
        stamp(i, 7);

        /* cursor B: the next op's first steps */
        cur_init(B, i + 1);

        /* (b) the epilogue's row constants (gains of both stages, the
         * addend's word) were requested after the previous op's steps */
        const int erow = tid < nrow ? Wr.t0 * rpt + tid : 0;

        /* (c) this op's codebooks, straight into LDS (no registers): one
         * 1 KB piece per wave instruction, every piece requested at once.
         * Each stage's LDS slot is padded to whole pieces: lanes past a
         * short codebook re-read its last 16 bytes into the padding. The
         * previous op's gathers ended before its epilogue barrier. */
        if (ns > 0) {
            const int pps = (int) (cbb >> 10);        /* pieces per stage */
            const int np = ns * 2 * pps;
            for (int pc = wave; pc < np; pc += W) {
                const int q2 = pc / pps, j = pc - q2 * pps;   /* q2: slot * 2 + stage */
                const uint8_t * src = Wr.cb[q2] + min(1024u * j + 16u * lane, O.cbr - 16u);
                __builtin_amdgcn_global_load_lds((const void *) src, (lds_void *) (lds + 1024 * pc), 16, 0, 0);
            }
        }

        /* (d) wait for x */
        if (stages_x && words && !dead) {
            const uint32_t want = base + (uint32_t) O.x_op;
            const uint64_t * xp = (const uint64_t *) O.x;
            uint32_t n = 0;
            while (true) {
                bool ok = true;
#pragma unroll
                for (int k = 0; k < NXK; k++) ok &= word_ep(xw[k]) == want;
                if (ok) break;
                if (++n > kChainSpin) {
                    st_agent(err, 1u);
                    dead = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int k = 0; k < NXK; k++)
                    if (word_ep(xw[k]) != want) xw[k] = ld_word(xp + min(k * NT + tid, nxw - 1));
            }
        }
        if (stages_x && O.xmode == kXNorm) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < NXK; k++)
                if (k * NT + tid < nxw) {
                    const double v = (double) __uint_as_float((uint32_t) xw[k]);
                    ss += v * v;
                }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            if (lane == 0) nrm[wave] = ss;
        }
        if (dead) *gaveup = 1u;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   /* this wave's codebook pieces are in LDS */
        __syncthreads();
        stamp(i, 1);
        dead = *gaveup != 0u;
        /* every earlier load has landed (the wait above): take the row
         * constants now, so no wait for them falls after the steps, whose
         * refills of the next op's index words are then in flight */
        asm volatile("" : "+v"(gr[0]), "+v"(gr[1]), "+v"(gr[2]), "+v"(gr[3]), "+v"(yword), "+v"(yplain));
#pragma unroll
        for (int k = 0; k < NXK; k++) asm volatile("" : "+v"(nv[k]));
        const float g00 = chain_f16((uint16_t) gr[0]), g01 = chain_f16((uint16_t) gr[1]);
        const float g10 = chain_f16((uint16_t) gr[2]), g11 = chain_f16((uint16_t) gr[3]);
        int xk = 0;
        uint32_t xb[NXK];   /* bf16 per word (f32 sources) or bf16 pairs */
        if (stages_x) {
            const int xmode = pin(O.xmode);
            const gptr<uint16_t> xo = wg == 0 ? gpin(O.xout) : nullptr;
            float inv = 1.0f;
            if (xmode == kXNorm) {
                double tot = 0.0;
#pragma unroll
                for (int k = 0; k < W; k++) tot += nrm[k];
                inv = (float) (1.0 / sqrt(tot / (double) pin(O.cols) + (double) pin(O.eps)));
            }
            uint32_t xm = 0;
            if (f32v) {
#pragma unroll
                for (int k = 0; k < NXK; k++) {
                    const int wi = k * NT + tid;
                    float v = __uint_as_float((uint32_t) xw[k]);
                    if (xmode == kXNorm) v = v * inv * nv[k];
                    const uint32_t b = chain_bf16(v);
                    xb[k] = b;
                    if (wi < nxw) {
                        xm = max(xm, (b << 16) & 0x7fffffffu);
                        *(_Float16 *) (lx + 264 * (wi >> 7) + 2 * (wi & 127)) = (_Float16) __uint_as_float(b << 16);
                        if (xo) xo[wi] = (uint16_t) b;
                    }
                }
            } else {
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
                for (int k = 0; k < NXK; k++) {
                    const int wi = k * NT + tid;
                    const uint32_t p = (uint32_t) xw[k];
                    xb[k] = p;
                    if (wi < nxw) {
                        xm = max(xm, xr_mag_bf16x2(p));
                        const int e = 2 * wi;
                        h2 hv;
                        hv[0] = (_Float16) __uint_as_float(p << 16);
                        hv[1] = (_Float16) __uint_as_float(p & 0xffff0000u);
                        *(h2 *) (lx + 264 * (e >> 7) + 2 * (e & 127)) = hv;
                        if (xo) ((gptr<uint32_t>) xo)[wi] = p;
                    }
                }
            }
            xr_note(xr, xm);
        }
        __syncthreads();
        /* x outside f16's comfortable range: stage it again as x * 2^-xk and
         * scale the sums back (both exact) */
        if (stages_x && xr_out(xr)) {
            uint32_t fm = 0;
#pragma unroll
            for (int k = 0; k < NXK; k++)
                if (k * NT + tid < nxw) fm = max(fm, f32v ? xr_fin((xb[k] << 16) & 0x7fffffffu)
                                                          : max(xr_fin((xb[k] << 16) & 0x7fffffffu),
                                                                xr_fin(xb[k] & 0x7fff0000u)));
            xk = xr_shift(xr, fm);
            if (xk && O.nmat > 0) {
                const float sc = __builtin_ldexpf(1.0f, -xk);
#pragma unroll
                for (int k = 0; k < NXK; k++) {
                    const int wi = k * NT + tid;
                    if (wi >= nxw) continue;
                    if (f32v) {
                        *(_Float16 *) (lx + 264 * (wi >> 7) + 2 * (wi & 127)) =
                            (_Float16) (__uint_as_float(xb[k] << 16) * sc);
                    } else {
                        const int e = 2 * wi;
                        *(_Float16 *) (lx + 264 * (e >> 7) + 2 * (e & 127)) = (_Float16) (__uint_as_float(xb[k] << 16) * sc);
                        *(_Float16 *) (lx + 264 * (e >> 7) + 2 * (e & 127) + 2) =
                            (_Float16) (__uint_as_float(xb[k] & 0xffff0000u) * sc);
                    }
                }
                __syncthreads();
            }
        }

        stamp(i, 2);
        /* (d) the wave's units: its nreal steps of this op, padded to npad */
        f4 acc[2];
        acc[0] = f4{0.f, 0.f, 0.f, 0.f};
        acc[1] = acc[0];
        int ck = 0, cj = 0;
        int cslot = 0, ctl = 0, cc = 0;
        const uint8_t * xbase = lx;
        auto enter_cunit = [&]() {
            const int us = Wr.nt * C;
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
                    /* all S reads issued together (parts past S re-read the
                     * last one and add nothing), added in part order */
                    float part[16];
#pragma unroll
                    for (int h = 0; h < 16; h++) {
                        const int hc = min(h, (1 << lgS) - 1);
                        part[h] = red[((lane << lgS) + hc) * 17 + hc];
                    }
                    float v = 0.0f;
#pragma unroll
                    for (int h = 0; h < 16; h++)
                        if (h < (1 << lgS)) v += part[h];
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
        stamp(i, 3);
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
        stamp(i, 4);
        /* the next op's row constants, in flight through this epilogue */
        uint32_t ngr[4];
        uint64_t nyword;
        float nyplain;
        load_consts(i + 1, ngr, nyword, nyplain);

        /* (e) the epilogue: K chunks added in order, gains per stage, the
         * addend; then the plain outputs and the published words */
        __syncthreads();
        stamp(i, 5);
        if (ns > 0) {
            const bool have = tid < nrow;
            float sum[2][2];
#pragma unroll
            for (int sl = 0; sl < 2; sl++)
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    float v = 0.0f;
                    if (have && sl < ns)
                        for (int c = 0; c < C; c++) v += P[((sl * nrow + tid) * C + c) * 2 + s];
                    sum[sl][s] = v;
                }
            const float v0 = xr_unscale(g00 * sum[0][0] + g01 * sum[0][1], xk);
            if (ns == 1) {
                const bool ok = have && erow < pin(Wr.rows0);
                const gptr<float> yo = gpin(Wr.y[0]);
                const gptr<uint16_t> ybo = gpin(Wr.ybf);
                const gptr<uint64_t> pfo = gpin(Wr.pf);
                const gptr<uint64_t> pbo = gpin(Wr.pb);
                const gptr<const void> ya = gpin(Wr.yadd);
                const int yaop = pin(Wr.yadd_op);
                float y = v0;
                if (ya) {
                    if (yaop) {
                        const uint32_t want = base + (uint32_t) yaop;
                        uint32_t n = 0;
                        while (ok && !dead && word_ep(yword) != want) {
                            if (++n > kChainSpin) {
                                st_agent(err, 1u);
                                dead = true;
                                break;
                            }
                            __builtin_amdgcn_s_sleep(1);
                            yword = ld_word((gptr<const uint64_t>) ya + erow);
                        }
                        y = __uint_as_float((uint32_t) yword) + v0;
                    } else {
                        y = yplain + v0;
                    }
                }
                const uint32_t yb = chain_bf16(y);
                if (ok && yo) yo[erow] = y;
                if (ok && ybo) ybo[erow] = (uint16_t) yb;
                if (ok && pfo) st_word(pfo + erow, __float_as_uint(y), ep);
                if (pbo) {
                    /* rows 2j and 2j + 1 are neighbouring lanes (a published
                     * bf16 op's workgroups start at even rows) */
                    const uint32_t hi = (uint32_t) __shfl_xor((int) (ok ? yb : 0u), 1, 64);
                    if (ok && !(erow & 1)) st_word(pbo + (erow >> 1), yb | (hi << 16), ep);
                }
            } else {
                const float v1 = xr_unscale(g10 * sum[1][0] + g11 * sum[1][1], xk);
                const bool ok = have && erow < pin(Wr.rows0);
                const gptr<float> y0 = gpin(Wr.y[0]);
                const gptr<float> y1 = gpin(Wr.y[1]);
                const gptr<uint16_t> ao = gpin(O.act);
                const gptr<uint64_t> pao = gpin(O.pact);
                uint32_t a = 0;
                if (ok) {
                    if (y0) y0[erow] = v0;
                    if (y1) y1[erow] = v1;
                    if (ao || pao) a = chain_gelu_mul_bf16(v0, v1);
                    if (ao) ao[erow] = (uint16_t) a;
                }
                if (pao) {
                    const uint32_t hi = (uint32_t) __shfl_xor((int) a, 1, 64);
                    if (ok && !(erow & 1)) st_word(pao + (erow >> 1), a | (hi << 16), ep);
                }
            }
        }
        stamp(i, 6);
        gr[0] = ngr[0]; gr[1] = ngr[1]; gr[2] = ngr[2]; gr[3] = ngr[3];
        yword = nyword;
        yplain = nyplain;
    }
    if (tid == 0) st_agent(flags + wg, base + (uint32_t) nops);
}

/* ------------------------------------------------------------------------ */
/* Host side.                                                                */
/* ------------------------------------------------------------------------ */

struct Chain {
    std::vector<ChainOp> ops;     /* as added: external pointers only */
    std::vector<ChainOp> built_ops;
    ChainOp * dops = nullptr;
    ChainWg * dwgs = nullptr;     /* per op and workgroup: its share, resolved */
    uint64_t * words = nullptr;   /* every published output's words */
    uint32_t * flags = nullptr;   /* one epoch base per workgroup, then the error word */
    uint32_t * trace = nullptr;   /* phase trace (caller's device memory; null: off) */
    int dev = -1;
    int G = 0;
    int built = 0;
    int waves = 12;
    int look = 2;                 /* macro steps of index words in flight per wave */
    int umin = 0;                 /* units per workgroup the shape search aims for (0: its cost model) */
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
 * the workgroups of each matrix; the LDS offsets. An op that publishes bf16
 * pairs keeps S <= 8, so every workgroup's rows start at an even row. */
static int chain_shape(Chain * c, ChainOp & O) {
    const int G = c->G, W = c->waves;
    const int M = O.M;
    bool pairs = O.pact != nullptr;
    for (int m = 0; m < O.nmat; m++) pairs |= O.mat[m].pb != nullptr;
    long best = -1;
    int bS = 0, bC = 0;
    std::vector<int> bnwg(O.nmat, 0);
    for (int S = 1; S <= (pairs ? 8 : 16); S *= 2) {
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
        /* K chunks: with umin set, the fewest that give the workgroup umin
         * units; else the fewest rounds of units per wave, each unit costing
         * its steps plus about one step for its partial sums */
        int Cc = 0;
        long ccost = -1;
        for (int cc = 1; cc <= MP; cc++) {
            if (!divides(MP, cc)) continue;
            if (c->umin > 0) {
                Cc = cc;
                if (maxT * cc * ns >= c->umin) break;
                continue;
            }
            const long units = maxT * cc * ns;
            const long v = (units + W - 1) / W * (MP / cc + 1);
            if (ccost < 0 || v < ccost) { ccost = v; Cc = cc; }
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

/* An output of the chain: the op and matrix (-1: a pair's act) that writes
 * it, and whether it holds f32 values (y) or bf16 ones (y_bf16, act). */
struct ChainOut {
    uintptr_t p, bytes;
    int op, mat, f32;
};

static bool overlaps(uintptr_t a, uintptr_t na, uintptr_t b, uintptr_t nb) { return a < b + nb && b < a + na; }

/* Where every input comes from and what every op publishes: an input that
 * is exactly an earlier op's output (same start, same type, same length) is
 * read from that op's published words; one that only overlaps an output is
 * refused; anything else is external. An output that overlaps an earlier
 * external input or another output is refused too: within a launch, no
 * order holds between such accesses. Then one allocation holds every
 * published word, zeroed (epoch 0 is never current). */
static int chain_link(Chain * c) {
    std::vector<ChainOp> & B = c->built_ops;
    B = c->ops;
    std::vector<ChainOut> outs;
    struct In {
        uintptr_t p, bytes;
        int op;
    };
    std::vector<In> ext;
    size_t nwords = 0;
    std::vector<size_t> pf_at(B.size() * kChainMats, (size_t) -1), pb_at(B.size() * kChainMats, (size_t) -1),
        act_at(B.size(), (size_t) -1);
    auto need = [&](size_t & at, int rows) {
        if (at == (size_t) -1) {
            at = nwords;
            nwords += (((size_t) rows + 1) / 2 * 2 + 63) & ~(size_t) 63;
        }
    };
    /* find the producer of [p, p + bytes) among ops before i: -1 external,
     * -2 refused (message set), else its index into outs */
    auto producer = [&](uintptr_t p, uintptr_t bytes, int f32, const char * what, int i) -> int {
        for (int k = (int) outs.size() - 1; k >= 0; k--) {
            const ChainOut & o = outs[k];
            if (!overlaps(p, bytes, o.p, o.bytes)) continue;
            if (o.p == p && o.bytes == bytes && o.f32 == f32) return k;
            set_error("chain op %d reads its %s from part of op %d's output (or in another type or length)", i, what,
                      o.op);
            return -2;
        }
        return -1;
    };
    for (int i = 0; i < (int) B.size(); i++) {
        ChainOp & O = B[i];
        /* x */
        const int xf32 = O.xmode != kXBf16;
        const uintptr_t xbytes = (uintptr_t) O.cols * (xf32 ? 4 : 2);
        const int px = producer((uintptr_t) O.x, xbytes, xf32, "x", i);
        if (px == -2) return -1;
        if (px >= 0) {
            const ChainOut & o = outs[px];
            ChainOp & Pd = B[o.op];
            O.x_op = o.op + 1;
            if (xf32) {
                need(pf_at[o.op * kChainMats + o.mat], Pd.mat[o.mat].rows);
                O.xsrc = kSrcWordF32;
            } else if (o.mat >= 0) {
                need(pb_at[o.op * kChainMats + o.mat], Pd.mat[o.mat].rows);
                O.xsrc = kSrcWordBf16;
            } else {
                need(act_at[o.op], Pd.mat[0].rows);
                O.xsrc = kSrcWordBf16;
            }
        } else {
            O.x_op = 0;
            O.xsrc = xf32 ? kSrcF32 : kSrcBf16;
            ext.push_back({(uintptr_t) O.x, xbytes, i});
        }
        O.nxw = xf32 ? O.cols : O.cols / 2;
        if (O.nxw > kChainMaxXw) {
            set_error("chain op %d reads %d words of x, more than %d (%d columns of f32, %d of bf16)", i, O.nxw,
                      kChainMaxXw, kChainMaxXw, 2 * kChainMaxXw);
            return -1;
        }
        /* addends */
        for (int m = 0; m < O.nmat; m++) {
            ChainMat & A = O.mat[m];
            A.yadd_op = 0;
            if (!A.yadd) continue;
            const uintptr_t yb = (uintptr_t) A.rows * 4;
            const int pa = producer((uintptr_t) A.yadd, yb, 1, "addend", i);
            if (pa == -2) return -1;
            if (pa >= 0) {
                const ChainOut & o = outs[pa];
                need(pf_at[o.op * kChainMats + o.mat], B[o.op].mat[o.mat].rows);
                A.yadd_op = o.op + 1;
            } else {
                ext.push_back({(uintptr_t) A.yadd, yb, i});
            }
        }
        /* this op's outputs */
        std::vector<ChainOut> mine;
        for (int m = 0; m < O.nmat; m++) {
            const ChainMat & A = O.mat[m];
            if (A.y) mine.push_back({(uintptr_t) A.y, (uintptr_t) A.rows * 4, i, m, 1});
            if (A.ybf) mine.push_back({(uintptr_t) A.ybf, (uintptr_t) A.rows * 2, i, m, 0});
        }
        if (O.act) mine.push_back({(uintptr_t) O.act, (uintptr_t) O.mat[0].rows * 2, i, -1, 0});
        if (O.xout) mine.push_back({(uintptr_t) O.xout, (uintptr_t) O.cols * 2, i, -3, 0});
        for (const ChainOut & o : mine) {
            for (const In & e : ext)
                if (overlaps(o.p, o.bytes, e.p, e.bytes)) {
                    set_error("chain op %d writes memory that op %d reads as its external input", i, e.op);
                    return -1;
                }
            for (const ChainOut & p : outs)
                if (overlaps(o.p, o.bytes, p.p, p.bytes)) {
                    set_error("chain op %d writes memory that op %d also writes", i, p.op);
                    return -1;
                }
        }
        for (const ChainOut & o : mine)
            if (o.mat != -3) outs.push_back(o);
    }
    if (c->words) { (void) hipFree(c->words); c->words = nullptr; }
    if (nwords) {
        hipError_t e = hipMalloc((void **) &c->words, nwords * 8);
        if (e != hipSuccess) return fail_hip("chain words", e);
        e = hipMemset(c->words, 0, nwords * 8);
        if (e != hipSuccess) return fail_hip("chain words", e);
    }
    for (int i = 0; i < (int) B.size(); i++) {
        ChainOp & O = B[i];
        for (int m = 0; m < O.nmat; m++) {
            const size_t f = pf_at[i * kChainMats + m], b = pb_at[i * kChainMats + m];
            O.mat[m].pf = f != (size_t) -1 ? c->words + f : nullptr;
            O.mat[m].pb = b != (size_t) -1 ? c->words + b : nullptr;
        }
        O.pact = act_at[i] != (size_t) -1 ? c->words + act_at[i] : nullptr;
    }
    /* now that the words exist: the inputs' addresses */
    for (int i = 0; i < (int) B.size(); i++) {
        ChainOp & O = B[i];
        if (O.x_op) {
            const ChainOp & Pd = B[O.x_op - 1];
            const ChainOp & Orig = c->ops[i];
            const void * x = nullptr;
            for (int m = 0; m < Pd.nmat && !x; m++) {
                if (O.xsrc == kSrcWordF32 && (const void *) Pd.mat[m].y == Orig.x) x = Pd.mat[m].pf;
                if (O.xsrc == kSrcWordBf16 && (const void *) Pd.mat[m].ybf == Orig.x) x = Pd.mat[m].pb;
            }
            if (!x && O.xsrc == kSrcWordBf16 && (const void *) Pd.act == Orig.x) x = Pd.pact;
            O.x = x;
        }
        for (int m = 0; m < O.nmat; m++) {
            ChainMat & A = O.mat[m];
            if (!A.yadd_op) continue;
            const ChainOp & Pd = B[A.yadd_op - 1];
            const void * ya = nullptr;
            for (int k = 0; k < Pd.nmat && !ya; k++)
                if ((const void *) Pd.mat[k].y == c->ops[i].mat[m].yadd) ya = Pd.mat[k].pf;
            A.yadd = ya;
        }
        if (!O.x) { set_error("chain op %d: its producer's words were not found", i); return -1; }
    }
    return 0;
}

/* Every workgroup's share of every op: a gate/up pair splits its tiles
 * evenly over all workgroups (the same rows of both matrices); other ops
 * give each matrix a run of workgroups (wg0, nwg) that split its tiles. */
static void chain_shares(const Chain * c, std::vector<ChainWg> & out) {
    const int G = c->G;
    out.assign(c->built_ops.size() * (size_t) G, ChainWg());
    for (size_t i = 0; i < c->built_ops.size(); i++) {
        const ChainOp & O = c->built_ops[i];
        for (int wg = 0; wg < G; wg++) {
            ChainWg & R = out[i * G + wg];
            memset(&R, 0, sizeof R);
            if (O.nmat == 0) continue;
            int m0 = 0, m1 = 0, t0 = 0, nt = 0, ns = 0;
            if (O.pair) {
                const int T = O.mat[0].tiles;
                t0 = (int) ((long) wg * T / G);
                nt = (int) ((long) (wg + 1) * T / G) - t0;
                ns = nt > 0 ? 2 : 0;
                m1 = 1;
            } else {
                for (int k = 0; k < O.nmat; k++) {
                    const int w0 = O.mat[k].wg0, nw = O.mat[k].nwg;
                    if (wg >= w0 && wg < w0 + nw) {
                        const int lw = wg - w0, T = O.mat[k].tiles;
                        m0 = k;
                        t0 = (int) ((long) lw * T / nw);
                        nt = (int) ((long) (lw + 1) * T / nw) - t0;
                        ns = nt > 0 ? 1 : 0;
                    }
                }
            }
            const ChainMat & A = O.mat[m0];
            const ChainMat & B = O.mat[m1];
            for (int st = 0; st < 2; st++) {
                R.strm[st] = A.st[st] + A.stream_off;
                R.strm[2 + st] = B.st[st] + B.stream_off;
                R.cb[st] = A.st[st] + 24;
                R.cb[2 + st] = B.st[st] + 24;
                R.gain[st] = A.st[st] + O.gain_off;
                R.gain[2 + st] = B.st[st] + O.gain_off;
            }
            R.y[0] = A.y;
            R.y[1] = O.pair ? B.y : nullptr;
            R.ybf = A.ybf;
            R.pf = A.pf;
            R.pb = A.pb;
            R.yadd = O.pair ? nullptr : A.yadd;
            R.yadd_op = O.pair ? 0 : A.yadd_op;
            R.ns = ns;
            R.t0 = t0;
            R.nt = nt;
            R.rows0 = A.rows;
            R.rows1 = B.rows;
        }
    }
}

static int chain_build(Chain * c) {
    if (chain_alloc(c)) return -1;
    if (chain_link(c)) return -1;
    for (auto & O : c->built_ops) {
        if (O.nmat == 0) {
            O.lgS = 0; O.C = 1; O.msc = 1;
            O.xoff = 0;
            O.roff = O.poff = (uint32_t) (264 * O.M + 16);
            continue;
        }
        if (chain_shape(c, O)) return -1;
    }
    if (c->dops) { (void) hipFree(c->dops); c->dops = nullptr; }
    if (c->dwgs) { (void) hipFree(c->dwgs); c->dwgs = nullptr; }
    if (!c->built_ops.empty()) {
        const size_t bytes = sizeof(ChainOp) * c->built_ops.size();
        hipError_t e = hipMalloc((void **) &c->dops, bytes);
        if (e != hipSuccess) return fail_hip("chain op table", e);
        e = hipMemcpy(c->dops, c->built_ops.data(), bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail_hip("chain op table", e);
        std::vector<ChainWg> wgs;
        chain_shares(c, wgs);
        e = hipMalloc((void **) &c->dwgs, sizeof(ChainWg) * wgs.size());
        if (e != hipSuccess) return fail_hip("chain share table", e);
        e = hipMemcpy(c->dwgs, wgs.data(), sizeof(ChainWg) * wgs.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail_hip("chain share table", e);
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
                  (const ChainWg *) c->dwgs, (int) c->built_ops.size(), c->flags, c->flags + c->G, c->trace);
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
    if (c->dwgs) (void) hipFree(c->dwgs);
    if (c->words) (void) hipFree(c->words);
    if (c->flags) (void) hipFree(c->flags);
    delete c;
}

int sparkmv_chain_size(void * chain) { return chain ? (int) ((Chain *) chain)->ops.size() : -1; }

int sparkmv_chain_tune(void * chain, int waves, int look, int min_units) {
    Chain * c = (Chain *) chain;
    if (!c) { set_error("chain is null"); return -1; }
    if (waves != 8 && waves != 12 && waves != 16) { set_error("a chain runs 8, 12 or 16 waves per workgroup, not %d", waves); return -1; }
    if (look != 2 && look != 4 && look != 8) { set_error("a chain keeps 2, 4 or 8 macro steps in flight per wave, not %d", look); return -1; }
    if (look == 8 && waves != 8) { set_error("8 macro steps in flight need 8 waves per workgroup, not %d", waves); return -1; }
    if (min_units < 0 || min_units > 1024) { set_error("min_units %d is outside 0..1024", min_units); return -1; }
    c->waves = waves;
    c->look = look;
    c->umin = min_units;
    c->built = 0;
    return 0;
}

int sparkmv_chain_add_vq(void * chain, const sparkmv_chain_matrix * mats, int nmat, int nstages, int dim, int nc,
                         int cols, int v3, const void * x, int x_mode, const float * norm_w, float eps,
                         uint16_t * x_out, uint16_t * act, int wait) {
    (void) wait;   /* every read of a chain output waits for exactly its words */
    Chain * c = (Chain *) chain;
    if (!c || !mats) { set_error("chain or matrix list is null"); return -1; }
    if (nmat < 1 || nmat > kChainMats) { set_error("matrix count %d is outside 1..%d", nmat, kChainMats); return -1; }
    if (nstages != 2) { set_error("a chain op takes two residual stages, not %d", nstages); return -1; }
    if (dim != 4 || !v3) { set_error("a chain op takes DQV3 dim-4 stages (dim %d, v3 %d)", dim, v3); return -1; }
    if (bits_for(nc) != 12 || nc % 2) {
        set_error("a chain op takes 12-bit indices (an even codebook of 2050..4096 entries), not nc %d", nc);
        return -1;
    }
    const int maxc = x_mode == 0 ? 2 * kChainMaxXw : kChainMaxXw;
    if (cols < 128 || cols % 128 || cols > maxc) {
        set_error("a chain op takes a multiple of 128 columns up to %d (%s x), not %d", maxc, x_mode == 0 ? "bf16" : "f32",
                  cols);
        return -1;
    }
    if (x_mode != 0 && x_mode != 1 && x_mode != 2) { set_error("unknown chain x mode %d", x_mode); return -1; }
    if (!x) { set_error("x is null"); return -1; }
    if (((uintptr_t) x & 3u)) { set_error("chain x must be 4-byte aligned"); return -1; }
    if (act && nmat != 2) { set_error("a gate/up pair has two matrices, not %d", nmat); return -1; }
    if (act && mats[0].rows != mats[1].rows) { set_error("a gate/up pair has equal row counts (%d, %d)", mats[0].rows, mats[1].rows); return -1; }
    if (act && ((uintptr_t) act & 3u)) { set_error("act must be 4-byte aligned"); return -1; }
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
        if (A.y_bf16 && ((uintptr_t) A.y_bf16 & 3u)) { set_error("matrix %d y_bf16 must be 4-byte aligned", m); return -1; }
        O.mat[m].st[0] = (const uint8_t *) A.stages[0];
        O.mat[m].st[1] = (const uint8_t *) A.stages[1];
        O.mat[m].y = A.y;
        O.mat[m].ybf = A.y_bf16;
        O.mat[m].yadd = act ? nullptr : A.y_add;
        O.mat[m].rows = A.rows;
        O.mat[m].stream_off = (uint32_t) (L0.gain_off + 2 * (size_t) A.rows);
    }
    if (L0.mrow % 4 || L0.gain_off % 4) { set_error("chain row streams are not dword aligned"); return -1; }
    if (x_out && ((uintptr_t) x_out & 3u)) { set_error("x_out must be 4-byte aligned"); return -1; }
    O.x = x;
    O.nw = norm_w;
    O.xout = x_out;
    O.act = act;
    O.eps = eps;
    O.nmat = nmat;
    O.pair = act ? 1 : 0;
    O.cols = cols;
    O.M = cols / 128;
    O.xmode = x_mode;
    O.gain_off = (uint32_t) L0.gain_off;
    O.mrow = (uint32_t) L0.mrow;
    O.cbb = ((uint32_t) nc * 8u + 1023u) & ~1023u;
    O.cbr = (uint32_t) nc * 8u;
    c->ops.push_back(O);
    c->built = 0;
    return 0;
}

int sparkmv_chain_add_norm(void * chain, const float * x, int n, const float * norm_w, float eps, uint16_t * out,
                           int wait) {
    (void) wait;
    Chain * c = (Chain *) chain;
    if (!c || !x || !out) { set_error("chain, x or out is null"); return -1; }
    if (n < 128 || n % 128 || n > kChainMaxXw) { set_error("a chain norm takes a multiple of 128 values up to %d, not %d", kChainMaxXw, n); return -1; }
    if (((uintptr_t) x & 3u) || ((uintptr_t) out & 3u)) { set_error("chain norm x and out must be 4-byte aligned"); return -1; }
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
    const int k = c->waves * 16 + c->look;
    switch (k) {
        case 8 * 16 + 2: return chain_launch_w<8, 2>(c, s);
        case 8 * 16 + 4: return chain_launch_w<8, 4>(c, s);
        case 8 * 16 + 8: return chain_launch_w<8, 8>(c, s);
        case 12 * 16 + 2: return chain_launch_w<12, 2>(c, s);
        case 12 * 16 + 4: return chain_launch_w<12, 4>(c, s);
        case 16 * 16 + 2: return chain_launch_w<16, 2>(c, s);
        default: return chain_launch_w<16, 4>(c, s);
    }
}

/* 0 when every wait of every launch so far ended in time; -1 (message set)
 * after a wait gave up, with the error word cleared so the chain can run
 * again. Synchronizes the device. */
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
    (void) hipMemset(c->flags + c->G, 0, 4);
    set_error("a chain workgroup waited too long for the others (were all %d resident?)", c->G);
    return -1;
}

/* Phase trace: with buf set (device memory of at least words uint32
 * values), every later launch records, per workgroup w and op i, at
 * buf[(w * ops + i) * 10 + k] the low 32 bits of the 100 MHz clock at the
 * op's start (k = 0), once x has arrived in every thread (1), once x is
 * staged (2), at the step loop's start (3), when wave 0's steps are done
 * (4), when every unit is done (5), when the epilogue's stores are issued
 * (6) and when x has been requested (7), then the shader clock (low 32
 * bits) at the op's start (8) and end (9), 10 words in all. NULL turns it
 * off. Returns the words a trace needs. */
int sparkmv_chain_trace(void * chain, uint32_t * buf, long words) {
    Chain * c = (Chain *) chain;
    if (!c) { set_error("chain is null"); return -1; }
    if (chain_alloc(c)) return -1;
    const long need = (long) c->G * (long) c->ops.size() * kChainStamps;
    if (buf && words < need) { set_error("a chain trace needs %ld words, not %ld", need, words); return -1; }
    c->trace = buf;
    return (int) need;
}

/* the shape the chain chose for op i: S, C, unit length */
int sparkmv_chain_op_shape(void * chain, int i, int * S, int * C, int * msc) {
    Chain * c = (Chain *) chain;
    if (!c || i < 0 || i >= (int) c->ops.size()) { set_error("no chain op %d", i); return -1; }
    if (!c->built && chain_build(c)) return -1;
    const ChainOp & O = c->built_ops[i];
    if (S) *S = 1 << O.lgS;
    if (C) *C = O.C;
    if (msc) *msc = O.msc;
    return 0;
}

}  // extern "C"
