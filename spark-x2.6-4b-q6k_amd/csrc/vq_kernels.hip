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
#include "act.h"
#include "vq.h"
#include "vq_tile.h"
#include "xrange.h"

#include <hip/hip_fp16.h>
#include <string.h>

#include <atomic>

namespace sparkmv {


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

/* Work decomposition. A tile is 16/S rows of one matrix. Row m of the MFMA A
 * operand is tile row m/S restricted to part m%S of the row's K range (the
 * row's macro steps split into S equal parts); B column n = h*NC + c holds
 * part h of activation column c (NC activation columns, S*NC <= 16). Entry
 * C[m][n] with m%S == n/NC is then row m/S's dot over part n/NC, and the
 * epilogue adds the S parts: the split of K lives in the N columns a single
 * activation column would leave idle, so short matrices still fill the chip.
 * A tile's K may further split into C chunks worked by sibling waves of the
 * workgroup, and a workgroup holds T tiles at a time (T*C waves). Partial sums
 * meet in LDS and are added in a fixed order, so results are deterministic. */

struct FastMat {
    const uint8_t * st[2];
    float * y;
    int rows;
    int tiles;   /* ceil(rows * S / 16) */
    int wg0;     /* first workgroup of this matrix */
    int nwg;     /* workgroups of this matrix */
};

struct FastArgs {
    const void * x;
    int nmat, cols, nc, ncol, ldx, ldy, accumulate;
    uint32_t gain_off;   /* 24 + nc * 8: the same for every matrix of a launch */
    uint32_t mrow, prow;
    int lgS, C, T;       /* log2 of the parts per MFMA, wave chunks per tile, tiles per workgroup pass */
    int M;               /* 32-index macro steps per row */
    int xstride;         /* LDS bytes per activation column: 264 per 128 columns, plus 8 */
    int threads;         /* the launch width, so the kernel does not wait for the hidden argument */
    int kofs;            /* first macro step of this launch in every row (a K-split launch) */
    FastMat mat[4];      /* a launch of more matrices is split into launches of 4 */
    /* XN kernels: x is the f32 residual h; the staged x is
     * bf16(rms_norm(h) * nw) with eps, and workgroup 0 also writes those
     * bf16 values to xout when it is non-null (after mat, so that the other
     * kernels' arguments keep their offsets) */
    const float * nw;
    float eps;
    uint16_t * xout;
    /* A gate/up pair (two matrices of equal rows, one column): each row's
     * y goes, tagged 1 (gate) or 2 (up), into pslot[row] by an atomic
     * exchange; the one of the two that finds the other's value there
     * writes gelu(gate) * up into pact (f32) and pact16 (bf16) when they
     * are set, and clears the slot. */
    uint64_t * pslot;
    float * pact;
    uint16_t * pact16;
    /* Shared tiles (XG, one matrix): workgroup b works the W consecutive
     * (tile, K chunk) units W*b .. W*b + W - 1 in tile-major order (W waves),
     * so every CU gets the same share even when tiles do not divide over the
     * CUs. A tile whose chunks fall to two workgroups meets in kslot[row *
     * ncol + col]: each side exchanges its sum there, and the one that finds
     * the other's adds the two (addition commutes, so the bits do not depend
     * on which comes second), writes y and clears the word. */
    int sk;
    uint64_t * kslot;
    /* Chunk-split tiles (MC == 3, several columns, one matrix): a tile's K
     * is ck * C chunks; workgroup b works chunk group g = b % ck (chunks
     * g * C .. g * C + C - 1, one wave each, added in LDS in order) of the T
     * tiles from (b / ck) * T, with x staged for that group only. A tile's
     * ck group sums meet in a binary tree of exchange words: at each level
     * the two sides of a node exchange their sums in kslot[(node_base +
     * node) * rows * ncol + row * ncol + col], and the one that finds the
     * other's adds the two (addition commutes), clears the word and carries
     * the sum to the next level; the root's carrier writes y. The tree's
     * shape is fixed by ck, so the bits do not depend on the order of
     * arrival. */
    int ck;
};

constexpr int kFastMats = 4;
/* several-column launches read x from global memory when a shape allows */
constexpr int kFastXg = 1;
/* several-column launches of one matrix split tiles by K chunk when the
 * caller gives exchange words */
constexpr int kFastCk = 1;

constexpr int kRedStride = 16 * 17;   /* floats per wave of the LDS reduction area */
/* LDS stride between the stages' codebooks for 12-bit indices (nc <= 4096) */
constexpr uint32_t kCbStride12 = 32768;

/* f32 -> bf16 bits, round to nearest even (a NaN stays a NaN) */
__device__ __forceinline__ uint32_t bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

template <int NST, int XF32, int EXT, int MSC, int MC, int XN = 0>
__global__ __launch_bounds__(MC == 1 || MC == 4 ? 1024 : 640) void vq_mfma_kernel(const FastArgs A) {
    /* MSC > 0: a unit is exactly MSC macro steps, known at compile time, so
     * the whole unit runs as straight-line code and each step waits only for
     * its own index words (a loop would make the compiler wait for all of a
     * wave's loads at its head). MSC == 0: any unit length, a ring of D steps.
     * MC: the kernel for several activation columns, with x staged in LDS
     * (1; 4: the same for a gate/up pair that also writes the activation)
     * or, XG (2), read from global memory (the L2) with each step's index
     * words, so no x is staged and any column count fits LDS; 3: chunk-split
     * tiles.
     * XN (one column, straight-line units): x is the f32 residual h and the
     * workgroup stages bf16(rms_norm(h) * nw) (model.rs:236-245: sum of
     * squares in f64, 1 / sqrt rounded once to f32, (h * inv) * w in f32),
     * so the norm needs no launch of its own. */
    static_assert(!XN || (MC == 0 && MSC > 0 && !XF32), "the fused norm stages one bf16 column");
    constexpr int XG = MC == 2 ? 1 : 0;
    constexpr int CK = MC == 3 ? 1 : 0;
    static_assert(!CK || (MSC > 0 && !XF32 && !XN), "chunk-split tiles run straight-line bf16 units");
    constexpr int D = MSC > 0 ? MSC : 8;
    /* straight-line units keep at most kLook macro steps of index words in
     * flight per wave: with every step requested up front the memory system
     * serves some CUs' words last, and those CUs then do their whole unit
     * after the stream has ended. Two measured best wherever x is in LDS
     * (one column: q+k+v+g 7.6 -> 7.4 us, down 9.7 -> 9.2 us against three;
     * one step ahead lost 0.2-0.8 us). The x-from-global kernels also carry
     * each step's x in the same loads and keep three below ten-step units
     * (N = 8 down 14.8 -> 15.8 us with two). */
    constexpr int kLook = (MSC >= 10 || !XG) ? 2 : 3;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    /* cbb: bytes of one stage's codebook; cbs: their stride in LDS, a fixed
     * 32 KB for 12-bit indices (nc <= 4096), so the second stage's gathers
     * take their offset as an immediate */
    const uint32_t cbb = (uint32_t) A.nc * 8u;
    const uint32_t cbs = EXT ? cbb : kCbStride12;
    uint8_t * lx = lds + NST * cbs;
    float * red = (float *) (lx + (XF32 ? 2 : 1) * A.ncol * A.xstride);
    /* the x range flags, after the reduction area */
    uint32_t * xr = (uint32_t *) (lds + xr_off(NST * cbs + (XF32 ? 2 : 1) * A.ncol * A.xstride +
                                               (A.threads >> 6) * kRedStride * 4));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m16 = lane & 15, q = lane >> 4;
    /* the workgroup's matrix: every record is read at once (independent
     * scalar loads) and the one owning this workgroup selected, so no load
     * waits for another before the staging loads can go out */
    FastMat M;
    M.st[0] = A.mat[0].st[0]; M.st[1] = A.mat[0].st[1]; M.y = A.mat[0].y;
    M.rows = A.mat[0].rows; M.tiles = A.mat[0].tiles; M.wg0 = A.mat[0].wg0; M.nwg = A.mat[0].nwg;
#pragma unroll
    for (int k = 1; k < kFastMats; k++) {
        const bool take = k < A.nmat && (int) blockIdx.x >= A.mat[k].wg0;
        M.st[0] = take ? A.mat[k].st[0] : M.st[0];
        M.st[1] = take ? A.mat[k].st[1] : M.st[1];
        M.y = take ? A.mat[k].y : M.y;
        M.rows = take ? A.mat[k].rows : M.rows;
        M.tiles = take ? A.mat[k].tiles : M.tiles;
        M.wg0 = take ? A.mat[k].wg0 : M.wg0;
    }
    const int rows = M.rows;
    const int S = 1 << A.lgS, C = A.C, T = A.T, ncol = A.ncol;
    const int rpt = 16 >> A.lgS;                   /* rows per tile */
    /* T consecutive tiles per workgroup (the host sized nwg = ceil(tiles / T)),
     * or, with shared tiles, this wave's one (tile, chunk) unit */
    const bool sk = XG && A.sk;
    const int W = A.threads >> 6;
    const int wb = (int) blockIdx.x - M.wg0;       /* the workgroup within its matrix */
    const int usk = wb * W + wave;
    /* chunk-split tiles: chunk group cg of the workgroup's tiles */
    const int cg = CK ? wb % A.ck : 0;
    const int t0 = sk ? usk / C : (CK ? wb / A.ck : wb) * A.T;
    const int t1 = sk ? M.tiles : min(t0 + A.T, M.tiles);
    const int j = sk ? 0 : wave / C;               /* tile slot */
    const int c = sk ? usk - t0 * C : wave - j * C;  /* K chunk (of the group with chunk-split tiles) */
    const int MP = A.M >> A.lgS;                   /* macro steps per part */
    const int MS = MSC > 0 ? MSC : MP / C;         /* macro steps per unit */
    const int r_in = m16 >> A.lgS, h = m16 & (S - 1);  /* A side: tile row, part */
    const int hp = m16 / ncol, cn = m16 - hp * ncol;   /* B side: part, activation column */
    const bool bval = hp < S;
    const int msa = h * MP + (cg * C + c) * MS;
    const int msb = (bval ? hp : 0) * MP + c * MS;
    /* x in LDS: 128 columns (one macro step) per 264 bytes, the 8-byte pad
     * putting the parts that lanes read at once on different banks. With
     * chunk-split tiles only the group's C * MS steps of each part are
     * staged, part after part. */
    const uint8_t * xb = lx + (bval ? cn : 0) * A.xstride + 264 * (CK ? ((bval ? hp : 0) * C + c) * MS : msb) + 64 * q;
    const uint8_t * xbl = xb + ncol * A.xstride;
    const int iters = sk ? 1 : (t1 - t0 + T - 1) / T;
    const uint32_t stream_off = A.gain_off + (uint32_t) rows * 2u;

    /* the matrix's stage payloads, read once (uniform) */
    const uint8_t * stp[NST];
#pragma unroll
    for (int s = 0; s < NST; s++) stp[s] = M.st[s];
    const uint8_t * rp[NST];
    const uint8_t * pp[NST];
    /* index words of D macro steps; every load is issued unconditionally
     * (steps past the unit re-read its last step), so the number of loads in
     * flight is static and each use waits only for its own words */
    Words<NST, EXT, XG> w[D];
    /* XG: the lane's x run for its B column (part hp, activation column cn;
     * lanes past the parts read part 0 of column 0 and feed no output) */
    const uint8_t * xgp = (const uint8_t *) A.x + ((size_t) (bval ? cn : 0) * A.ldx + 128 * msb + 32 * q) * 2;
    auto ld = [&](Words<NST, EXT, XG> & W, int ms) {
        load_words<NST, EXT, XG>(W, rp, pp, xgp, ms < MS ? ms : MS - 1);
    };
    auto ld_all = [&]() {
#pragma unroll
        for (int u = 0; u < D; u++) ld(w[u], u);
    };
    /* the first kLook steps of a straight-line unit (all D of a ring) */
    auto ld_head = [&]() {
#pragma unroll
        for (int u = 0; u < D; u++)
            if (MSC == 0 || u < kLook) ld(w[u], u);
    };
    auto point = [&](int tile) {
        const int row = min(tile * rpt + r_in, rows - 1);
#pragma unroll
        for (int s = 0; s < NST; s++) {
            const uint8_t * sb = stp[s] + stream_off;
            rp[s] = sb + (size_t) row * A.mrow + 48 * (A.kofs + msa) + 12 * q;
            pp[s] = sb + (size_t) rows * A.mrow + (size_t) row * A.prow + 4 * (A.kofs + msa) + q;
        }
    };
    /* gains of the rows this lane's C entries belong to, per stage */
    uint32_t gw[NST][4];
    auto ld_gains = [&](int tile) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = min(tile * rpt + ((4 * q + i) >> A.lgS), rows - 1);
#pragma unroll
            for (int s = 0; s < NST; s++) gw[s][i] = *(const uint16_t *) (stp[s] + A.gain_off + 2 * (size_t) row);
        }
    };

    /* Staging: codebooks (16-byte chunks) and activations (4-byte words)
     * go to LDS. For one activation column every thread issues all its
     * staging loads at once, then the first unit's index words and gains,
     * then the LDS stores: the prologue costs one memory latency and the
     * unit's loads are in flight when the main loop starts. Each workgroup
     * walks the codebooks from its own starting chunk, so the workgroups of
     * an XCD do not all ask the same L2 channel for the same line at once. */
    const int n16 = (int) (cbb >> 4);              /* 16-byte chunks per stage */
    const int ncb = NST * n16;
    const int rot = (int) ((blockIdx.x * 328u) % (uint32_t) ncb);
    auto rot_chunk = [&](int i) { const int r = i + rot; return r >= ncb ? r - ncb : r; };
    /* bf16 x is read as pairs: the host sends only 4-byte aligned x with an
     * even ldx here (cols is a multiple of 128) */
    const int xpr = XF32 ? A.cols : A.cols >> 1;   /* 4-byte words per activation column */
    auto cb_load = [&](int i, uint32_t * v) {
        const bool hi = NST > 1 && i >= n16;
        const uint32_t * src = (const uint32_t *) ((hi ? stp[NST - 1] : stp[0]) + 24) + 4 * (hi ? i - n16 : i);
        v[0] = src[0]; v[1] = src[1]; v[2] = src[2]; v[3] = src[3];
    };
    auto cb_store = [&](int i, const uint32_t * v) {
        const int s = NST > 1 && i >= n16 ? 1 : 0;
        uint32_t * dst = (uint32_t *) (lds + s * cbs) + 4 * (i - s * n16);
        dst[0] = v[0]; dst[1] = v[1]; dst[2] = v[2]; dst[3] = v[3];
    };
    auto x_load = [&](int n, int k) -> uint32_t {
        if (XF32) return ((const uint32_t *) A.x)[(size_t) n * A.ldx + k];
        return ((const uint32_t *) A.x)[((size_t) n * A.ldx >> 1) + k];
    };
    auto x_store = [&](int n, int k, uint32_t v) {
        if (XF32) {
            const float f = __uint_as_float(v);
            const _Float16 hi = (_Float16) f;
            const int off = 264 * (k >> 7) + 2 * (k & 127);
            *(_Float16 *) (lx + n * A.xstride + off) = hi;
            *(_Float16 *) (lx + (ncol + n) * A.xstride + off) = (_Float16) (f - (float) hi);
        } else {
            /* a pair never straddles a 128-column block: one 4-byte store */
            const int e = 2 * k;
            const int off = 264 * (e >> 7) + 2 * (e & 127);
            const _Float16 lo16 = (_Float16) __uint_as_float(v << 16), hi16 = (_Float16) __uint_as_float(v & 0xffff0000u);
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            *(h2 *) (lx + n * A.xstride + off) = h2{lo16, hi16};
        }
    };
    const int first = min(t0 + j, t1 - 1);
    /* staging chunks per thread: two 32 KB codebooks are 4096 chunks, which
     * 10 loads per thread cover from seven waves up */
    constexpr int K = 10;
    const int bd = A.threads, tid = threadIdx.x;
    float xinv = 0.0f;        /* XN: 1 / rms of h */
    uint32_t xm = 0;          /* the largest |x| this thread staged, as f32 bits */
    xr_u16x2 xm2 = {0, 0};    /* the same for bf16 x, by pairs */
    if constexpr (MC) {
        /* Several activation columns (speculative verify): codebooks and x
         * are staged in batches of unconditional 16-byte loads (indices past
         * the end re-read the last chunk), then the unit's index words are
         * requested. The host sends 16-byte aligned x with ldx % 8 == 0 and
         * at most 5 codebook chunks per thread and stage. */
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));
        constexpr int KS = 5, KXM = 8;
        {
            u4v cv[NST][KS];
#pragma unroll
            for (int s = 0; s < NST; s++)
#pragma unroll
                for (int k = 0; k < KS; k++)
                    cv[s][k] = ((const u4a *) (stp[s] + 24))[min(k * bd + tid, n16 - 1)];
#pragma unroll
            for (int s = 0; s < NST; s++)
#pragma unroll
                for (int k = 0; k < KS; k++)
                    ((u4v *) (lds + s * cbs))[min(k * bd + tid, n16 - 1)] = cv[s][k];
        }
        /* 8-column pieces of x per activation column; chunk-split tiles
         * stage the group's C * MS steps of each part, whose piece cc comes
         * from piece xsrc(cc) of the row */
        const int xq = CK ? S * C * MS * 16 : A.cols >> 3, nx = XG ? 0 : ncol * xq;
        auto xsrc = [&](int cc) {
            if constexpr (!CK) return cc;
            const int hh = cc / (C * MS * 16);
            return (hh * MP + cg * C * MS) * 16 + cc - hh * C * MS * 16;
        };
        for (int base = 0; base < nx; base += KXM * bd) {
            u4v xv[KXM];
            int ci[KXM];
#pragma unroll
            for (int k = 0; k < KXM; k++) {
                ci[k] = min(base + k * bd + tid, nx - 1);
                const int n = ci[k] / xq, cc = ci[k] - n * xq;
                /* a slot wholly past x (uniform) would only repeat the last chunk */
                if (base + k * bd < nx)
                    xv[k] = *(const u4v *) ((const uint16_t *) A.x + (size_t) n * A.ldx + 8 * xsrc(cc));
            }
#pragma unroll
            for (int k = 0; k < KXM; k++) {
                if (base + k * bd >= nx) continue;
                const int n = ci[k] / xq, e = 8 * (ci[k] - n * xq);
                uint8_t * dst = lx + n * A.xstride + 264 * (e >> 7) + 2 * (e & 127);
                xr_acc_bf16x2(xm2, xv[k].x); xr_acc_bf16x2(xm2, xv[k].y);
                xr_acc_bf16x2(xm2, xv[k].z); xr_acc_bf16x2(xm2, xv[k].w);
                h4 lo4, hi4;
                lo4[0] = (_Float16) __uint_as_float(xv[k].x << 16);
                lo4[1] = (_Float16) __uint_as_float(xv[k].x & 0xffff0000u);
                lo4[2] = (_Float16) __uint_as_float(xv[k].y << 16);
                lo4[3] = (_Float16) __uint_as_float(xv[k].y & 0xffff0000u);
                hi4[0] = (_Float16) __uint_as_float(xv[k].z << 16);
                hi4[1] = (_Float16) __uint_as_float(xv[k].z & 0xffff0000u);
                hi4[2] = (_Float16) __uint_as_float(xv[k].w << 16);
                hi4[3] = (_Float16) __uint_as_float(xv[k].w & 0xffff0000u);
                *(h4 *) dst = lo4;
                *(h4 *) (dst + 8) = hi4;
            }
        }
        point(first);
        ld_gains(first);
        ld_head();
    } else if constexpr (XN) {
        /* One column staged from the f32 residual h: bf16(rms_norm(h) * nw).
         * h and nw are requested first (as many 16-byte chunks per thread
         * as the columns need), then the codebooks; the norm (squares in
         * f64, a butterfly per wave, the waves' sums from LDS in wave order)
         * and the staging of x run while the codebooks are in flight. */
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));   /* codebooks are 4-byte aligned */
        constexpr int KXN = 2;                     /* 16-byte chunks of h and nw (4 columns) per thread, at most */
        constexpr int KS = 5;                      /* 16-byte codebook chunks per thread and stage */
        const int xq4 = A.cols >> 2;
        f4 hv[KXN], wv[KXN];
#pragma unroll
        for (int k = 0; k < KXN; k++) {
            hv[k] = f4{0.f, 0.f, 0.f, 0.f};
            wv[k] = f4{0.f, 0.f, 0.f, 0.f};
            if (k * bd < xq4) {   /* uniform: chunks past the columns are not requested */
                const int i = min(k * bd + tid, xq4 - 1);
                hv[k] = ((const f4 *) A.x)[i];
                wv[k] = ((const f4 *) A.nw)[i];
            }
        }
        u4v cv[NST][KS];
#pragma unroll
        for (int s = 0; s < NST; s++)
#pragma unroll
            for (int k = 0; k < KS; k++)
                cv[s][k] = ((const u4a *) (stp[s] + 24))[min(k * bd + tid, n16 - 1)];
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        point(first);
        ld_gains(first);
        ld_head();
        __builtin_amdgcn_sched_barrier(0);
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < KXN; k++)
            if (k * bd + tid < xq4)
#pragma unroll
                for (int j = 0; j < 4; j++) ss += (double) hv[k][j] * (double) hv[k][j];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        double * part = (double *) red;
        if (lane == 0) part[wave] = ss;
        __syncthreads();
        double tot = 0.0;
        for (int i = 0; i < (bd >> 6); i++) tot += part[i];
        xinv = (float) (1.0 / sqrt(tot / (double) A.cols + (double) A.eps));
#pragma unroll
        for (int k = 0; k < KXN; k++) {
            if (k * bd >= xq4) continue;
            /* four columns: bf16 of (h * inv) * w, staged as f16 (exact) */
            const int e = 4 * min(k * bd + tid, xq4 - 1);
            uint32_t b[4];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = bf16_rne((hv[k][j] * xinv) * wv[k][j]);
            const uint32_t p0 = b[0] | (b[1] << 16), p1 = b[2] | (b[3] << 16);
            xr_acc_bf16x2(xm2, p0);
            xr_acc_bf16x2(xm2, p1);
            h4 v4;
#pragma unroll
            for (int j = 0; j < 4; j++) v4[j] = (_Float16) __uint_as_float(b[j] << 16);
            *(h4 *) (lx + 264 * (e >> 7) + 2 * (e & 127)) = v4;
            if (A.xout && blockIdx.x == 0) {
                typedef uint32_t u2v __attribute__((ext_vector_type(2)));
                *(u2v *) (A.xout + e) = u2v{p0, p1};
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < NST; s++)
#pragma unroll
            for (int k = 0; k < KS; k++)
                ((u4v *) (lds + s * cbs))[min(k * bd + tid, n16 - 1)] = cv[s][k];
    } else if constexpr (MSC > 0 && XF32) {
        /* One 16-byte aligned f32 activation column of at most 16 * blockDim
         * columns, each value split into f16 hi + lo (hi in the column's
         * slot, lo in the next one), and an even codebook of at most KS
         * chunks per thread and stage, staged as in the bf16 form below. */
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));
        constexpr int KX = 4;                      /* 16-byte x chunks (4 columns) per thread */
        constexpr int KS = 5;
        const int xq = A.cols >> 2;
        u4v cv[NST][KS];
        u4v xv[KX];
#pragma unroll
        for (int s = 0; s < NST; s++)
#pragma unroll
            for (int k = 0; k < KS; k++)
                cv[s][k] = ((const u4a *) (stp[s] + 24))[min(k * bd + tid, n16 - 1)];
#pragma unroll
        for (int k = 0; k < KX; k++) xv[k] = ((const u4v *) A.x)[min(k * bd + tid, xq - 1)];
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        point(first);
        ld_gains(first);
        ld_head();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < NST; s++)
#pragma unroll
            for (int k = 0; k < KS; k++)
                ((u4v *) (lds + s * cbs))[min(k * bd + tid, n16 - 1)] = cv[s][k];
#pragma unroll
        for (int k = 0; k < KX; k++) {
            const int e = 4 * min(k * bd + tid, xq - 1);
            const int off = 264 * (e >> 7) + 2 * (e & 127);
            h4 hi4, lo4;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float f = __uint_as_float(xv[k][j]);
                hi4[j] = (_Float16) f;
                lo4[j] = (_Float16) (f - (float) hi4[j]);
                xm = max(xm, xr_mag_f32w(xv[k][j]));
            }
            *(h4 *) (lx + off) = hi4;
            *(h4 *) (lx + A.xstride + off) = lo4;
        }
    } else if constexpr (MSC > 0) {
        /* One 16-byte aligned activation column of at most 16 * blockDim
         * columns and an even codebook of at most KS chunks per thread and
         * stage (the host checks both). Threads past the end load and store
         * the last chunk again (one cache line per wave, the same bytes to the
         * same place), so the prologue has no branches and the compiler
         * counts every load exactly. */
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));   /* codebooks are 4-byte aligned */
        constexpr int KX = 2;                      /* 16-byte x chunks (8 columns) per thread */
        constexpr int KS = 5;                      /* 16-byte codebook chunks per thread and stage */
        const int xq = A.cols >> 3;
        u4v cv[NST][KS];
        u4v xv[KX];
#pragma unroll
        for (int s = 0; s < NST; s++)
#pragma unroll
            for (int k = 0; k < KS; k++)
                cv[s][k] = ((const u4a *) (stp[s] + 24))[min(k * bd + tid, n16 - 1)];
#pragma unroll
        for (int k = 0; k < KX; k++) xv[k] = ((const u4v *) A.x)[min(k * bd + tid, xq - 1)];
        /* every wave's staging requests enter the CU's memory pipeline
         * before any wave's index stream (which would otherwise hold them
         * up behind the unit's bulk): an execution barrier, no wait */
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        point(first);
        ld_gains(first);
        ld_head();
        /* keep the scheduler from pulling stores (and their waits) up
         * between the loads */
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < NST; s++)
#pragma unroll
            for (int k = 0; k < KS; k++)
                ((u4v *) (lds + s * cbs))[min(k * bd + tid, n16 - 1)] = cv[s][k];
#pragma unroll
        for (int k = 0; k < KX; k++) {
            const int i = k * bd + tid;
            {
                /* eight bf16 columns -> eight f16 in the padded layout */
                const int e = 8 * min(i, xq - 1);
                uint8_t * dst = lx + 264 * (e >> 7) + 2 * (e & 127);
                xr_acc_bf16x2(xm2, xv[k].x); xr_acc_bf16x2(xm2, xv[k].y);
                xr_acc_bf16x2(xm2, xv[k].z); xr_acc_bf16x2(xm2, xv[k].w);
                h4 lo4, hi4;
                lo4[0] = (_Float16) __uint_as_float(xv[k].x << 16);
                lo4[1] = (_Float16) __uint_as_float(xv[k].x & 0xffff0000u);
                lo4[2] = (_Float16) __uint_as_float(xv[k].y << 16);
                lo4[3] = (_Float16) __uint_as_float(xv[k].y & 0xffff0000u);
                hi4[0] = (_Float16) __uint_as_float(xv[k].z << 16);
                hi4[1] = (_Float16) __uint_as_float(xv[k].z & 0xffff0000u);
                hi4[2] = (_Float16) __uint_as_float(xv[k].w << 16);
                hi4[3] = (_Float16) __uint_as_float(xv[k].w & 0xffff0000u);
                *(h4 *) dst = lo4;
                *(h4 *) (dst + 8) = hi4;
            }
        }
    } else {
        for (int base = 0; base < ncb; base += K * bd) {
            uint32_t cv[K][4];
#pragma unroll
            for (int k = 0; k < K; k++)
                if (base + k * bd + tid < ncb) cb_load(rot_chunk(base + k * bd + tid), cv[k]);
#pragma unroll
            for (int k = 0; k < K; k++)
                if (base + k * bd + tid < ncb) cb_store(rot_chunk(base + k * bd + tid), cv[k]);
        }
        for (int n = 0; n < ncol; n++) {
            for (int base = 0; base < xpr; base += K * bd) {
                uint32_t xv[K];
#pragma unroll
                for (int k = 0; k < K; k++)
                    if (base + k * bd + tid < xpr) xv[k] = x_load(n, base + k * bd + tid);
#pragma unroll
                for (int k = 0; k < K; k++)
                    if (base + k * bd + tid < xpr) {
                        x_store(n, base + k * bd + tid, xv[k]);
                        if (XF32) xm = max(xm, xr_mag_f32w(xv[k]));
                        else xr_acc_bf16x2(xm2, xv[k]);
                    }
            }
        }
        point(first);
        ld_all();
        ld_gains(first);
    }
    if (MSC == 0 && (cbb & 8u) && tid < 2 * NST) {   /* an odd codebook: the last codeword of each stage */
        const int s = tid >> 1, k = tid & 1;
        ((uint32_t *) (lds + s * cbs))[4 * n16 + k] = ((const uint32_t *) ((s ? stp[NST - 1] : stp[0]) + 24))[4 * n16 + k];
    }
    if constexpr (XG == 0) xr_note(xr, XF32 ? xm : xr_bf16_max(xm2));
    __syncthreads();
    /* x outside f16's comfortable range: stage it again as x * 2^-xk (one
     * element per thread and step, the staging's layout) and scale the sums
     * back by 2^xk. XG kernels stage no x and check each unit instead. */
    int xk = 0;
    if constexpr (XG == 0) {
        if (xr_out(xr)) {
            /* staged columns per activation column (chunk-split tiles: the
             * group's steps of each part; staged column kl is row column
             * xcol(kl)) */
            const int xl = CK ? S * C * MS * 128 : A.cols;
            auto xcol = [&](int kl) {
                if constexpr (!CK) return kl;
                const int hh = kl / (C * MS * 128);
                return (hh * MP + cg * C * MS) * 128 + kl - hh * C * MS * 128;
            };
            auto xval = [&](int e) {
                const int n = e / xl, kk = xcol(e - n * xl);
                const size_t xi = (size_t) n * A.ldx + kk;
                if (XN) return __uint_as_float(bf16_rne((((const float *) A.x)[kk] * xinv) * A.nw[kk]) << 16);
                return XF32 ? ((const float *) A.x)[xi] : bf16_to_f32(((const uint16_t *) A.x)[xi]);
            };
            uint32_t fm = 0;   /* the largest finite |x| of this thread's elements */
            for (int e = tid; e < ncol * xl; e += bd) fm = max(fm, xr_fin(xr_mag(xval(e))));
            xk = xr_shift(xr, fm);
            if (xk) {
                for (int e = tid; e < ncol * xl; e += bd) {
                    const int n = e / xl, kk = e - n * xl;
                    const float f = __builtin_ldexpf(xval(e), -xk);
                    const _Float16 hi = (_Float16) f;
                    const int off = 264 * (kk >> 7) + 2 * (kk & 127);
                    *(_Float16 *) (lx + n * A.xstride + off) = hi;
                    if (XF32) *(_Float16 *) (lx + (ncol + n) * A.xstride + off) = (_Float16) (f - (float) hi);
                }
                __syncthreads();
            }
        }
    }

    /* One unit: the tile's MS macro steps, then the epilogue. The index
     * words and gains of the tile are already requested. */
    auto unit = [&](int tile) {
        const bool active = tile < t1;
        f4 acc[NST];
#pragma unroll
        for (int s = 0; s < NST; s++) acc[s] = f4{0.f, 0.f, 0.f, 0.f};
        /* XG: the largest bf16 |x| this lane converts in the unit, per half */
        u16x2 xmx = {0, 0};
        u16x2 * const xm = XG ? &xmx : nullptr;
        if (active) {
            if (MSC > 0) {
#pragma unroll
                for (int u = 0; u < D; u++) {
                    mstep<NST, XF32, EXT, XG, 0>(w[u], cbs, xb + 264 * u, xbl + 264 * u, acc, 1.0f, xm);
                    if (u + kLook < D) ld(w[u + kLook], u + kLook);
                    /* keep step u + kLook's loads here: left to itself the
                     * scheduler sinks them to just before their step, which
                     * then waits a whole memory round trip. (XG units hold
                     * 4 steps of x too: pinned, they would spill.) */
                    if constexpr (!XG) __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                for (int ms0 = 0; ms0 < MS; ms0 += D) {
#pragma unroll
                    for (int u = 0; u < D; u++) {
                        if (ms0 + u < MS)
                            mstep<NST, XF32, EXT, XG, 0>(w[u], cbs, xb + 264 * (ms0 + u), xbl + 264 * (ms0 + u), acc,
                                                      1.0f, xm);
                        if (MS > D) ld(w[u], ms0 + u + D);
                    }
                }
            }
        }
        /* the factor 2^uk that the unit's sums carry back */
        int uk = xk;
        if constexpr (XG != 0) {
            /* x read per step, converted per step, so the range is checked
             * per unit and per B column (the four lanes of lane & 15: one
             * part of one activation column), after the fact:
             *  - an |x| past f16's range shows as a non-finite sum; the
             *    column's largest finite |x| is then read again;
             *  - small x shows in the largest |x| the steps converted: a
             *    nonzero maximum below 2^-4 would leave the values below
             *    2^-14 on f16's subnormal grid.
             * A column outside [2^-4, 2^15) gets uk that brings its largest
             * finite |x| to [2^14, 2^15), and the unit runs again, one step
             * at a time, with x * 2^-uk (exact; an infinity or NaN in x stays
             * one). The sums are scaled back by 2^uk before any other
             * column's or chunk's are added to them. */
            if (active) {
                bool bad = false;
#pragma unroll
                for (int s = 0; s < NST; s++)
#pragma unroll
                    for (int i = 0; i < 4; i++) bad = bad || !__builtin_isfinite(acc[s][i]);
                /* as f32 bits; a non-finite maximum is never small */
                uint32_t m = xr_col_max((uint32_t) max(xmx[0], xmx[1]) << 16);
                const bool small = m != 0u && m < kXrLow;
                if (__builtin_amdgcn_ballot_w64(bad || small)) {
                    if (__builtin_amdgcn_ballot_w64(bad)) {
                        typedef uint32_t u4x __attribute__((ext_vector_type(4)));
                        m = 0;
#pragma unroll 1
                        for (int u = 0; u < MS; u++) {
#pragma unroll
                            for (int k = 0; k < 4; k++) {
                                const u4x v = ((const u4x *) (xgp + 256 * u))[k];
#pragma unroll
                                for (int h = 0; h < 4; h++)
                                    m = max(m, max(xr_fin((v[h] << 16) & 0x7fffffffu), xr_fin(v[h] & 0x7fff0000u)));
                            }
                        }
                        m = xr_col_max(m);   /* the column's largest finite |x| in the unit */
                    }
                    /* 2^-uk must be a normal f32: bf16 x below 2^-126 is
                     * brought up only as far as 2^126 takes it */
                    uk = max(xr_shift_of(m), -126);
                    if (__builtin_amdgcn_ballot_w64(uk != 0)) {
                        const float sc = __uint_as_float((uint32_t) (127 - uk) << 23);
#pragma unroll
                        for (int s = 0; s < NST; s++) acc[s] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
                        for (int u = 0; u < MS; u++) {
                            Words<NST, EXT, XG> W1;
                            load_words<NST, EXT, XG>(W1, rp, pp, xgp, u);
                            mstep<NST, XF32, EXT, XG, 1>(W1, cbs, xb, xbl, acc, sc);
                        }
                    }
                }
            }
        }
        /* stages combine with their row gains; entry C[4q + i][m16] of this
         * lane goes to the wave's reduction area */
        float * R = red + wave * kRedStride;
        if constexpr (MSC > 0 && !MC) {
            /* one activation column and one wave per tile: row r of the tile
             * is the sum of C[r*S + h][h] over parts h, read back by lane r.
             * A wave's LDS operations complete in order, so no barrier. */
            if (active) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float v = 0.0f;
#pragma unroll
                    for (int s = 0; s < NST; s++) v += f16_to_f32((uint16_t) gw[s][i]) * acc[s][i];
                    R[(4 * q + i) * 17 + m16] = xr_unscale(v, uk);
                }
                if (lane < rpt) {
                    float part[16];
#pragma unroll
                    for (int hh = 0; hh < 16; hh++) {
                        const int hc = hh < S ? hh : S - 1;
                        part[hh] = R[(lane * S + hc) * 17 + hc];
                    }
                    float sum = 0.0f;
#pragma unroll
                    for (int hh = 0; hh < 16; hh++) sum += hh < S ? part[hh] : 0.0f;
                    const int row = tile * rpt + lane;
                    if (row < rows) {
                        float * yp = M.y + row;
                        *yp = (A.accumulate ? *yp : 0.0f) + sum;
                        if (A.pslot) {
                            /* the pair's activation: whichever of gate and up
                             * comes second gets the other's value back from
                             * the exchange (one memory round trip, no wait) */
                            const uint32_t mi = (int) blockIdx.x >= A.mat[1].wg0 ? 1u : 0u;
                            const uint64_t mine = ((uint64_t) (1u + mi) << 32) | __float_as_uint(sum);
                            const uint64_t old =
                                __hip_atomic_exchange(A.pslot + row, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            if ((uint32_t) (old >> 32) == 2u - mi) {
                                const float o = __uint_as_float((uint32_t) old);
                                const float v = mi ? gelu_mul(o, sum) : gelu_mul(sum, o);
                                if (A.pact) A.pact[row] = v;
                                if (A.pact16) A.pact16[row] = (uint16_t) bf16_rne(v);
                                __hip_atomic_store(A.pslot + row, (uint64_t) 0, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
                            }
                        }
                    }
                }
            }
            return;
        }
        if (active) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = 0.0f;
#pragma unroll
                for (int s = 0; s < NST; s++) v += f16_to_f32((uint16_t) gw[s][i]) * acc[s][i];
                R[(4 * q + i) * 17 + m16] = xr_unscale(v, uk);
            }
        }
        /* with one wave per tile the wave only reads its own area back: its
         * LDS operations complete in order, no workgroup barrier needed */
        const int Cw = C;
        if (Cw > 1) {
            __syncthreads();
        } else {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        /* y[col][row] = sum over parts hh (and over the C chunk waves) of
         * C[r*S + hh][hh*ncol + col], added in a fixed order. With shared
         * tiles the tile's first wave in this workgroup adds the nin chunk
         * waves that follow it here; a tile split over two workgroups then
         * meets the other half's sum through kslot. */
        const int nin = sk ? min(C - c, W - wave) : Cw;
        const bool split = sk && (c != 0 || nin < C);
        if (active && (c == 0 || (sk && wave == 0))) {
            for (int e = lane; e < rpt * ncol; e += 64) {
                const int r = ncol == 1 ? e : e / ncol, col = e - r * ncol;
                const int row = tile * rpt + r;
                float sum = 0.0f;
                if (Cw == 1) {
                    /* all S reads issued together (parts past S re-read the
                     * last one and add nothing), added in part order */
                    float part[16];
#pragma unroll
                    for (int hh = 0; hh < 16; hh++) {
                        const int hc = hh < S ? hh : S - 1;
                        part[hh] = red[wave * kRedStride + (r * S + hc) * 17 + hc * ncol + col];
                    }
#pragma unroll
                    for (int hh = 0; hh < 16; hh++) sum += hh < S ? part[hh] : 0.0f;
                } else {
                    for (int hh = 0; hh < S; hh++) {
                        const float * rr = red + wave * kRedStride + (r * S + hh) * 17 + hh * ncol + col;
                        float part = rr[0];
                        for (int cw = 1; cw < nin; cw++) part += rr[cw * kRedStride];
                        sum += part;
                    }
                }
                if (row < rows) {
                    float * yp = M.y + (size_t) col * A.ldy + row;
                    bool last = true;
                    if (split) {
                        uint64_t * sl = A.kslot + (size_t) row * ncol + col;
                        const uint64_t old = __hip_atomic_exchange(sl, (1ull << 32) | __float_as_uint(sum),
                                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        last = (uint32_t) (old >> 32) == 1u;
                        if (last) {
                            sum = __uint_as_float((uint32_t) old) + sum;
                            __hip_atomic_store(sl, (uint64_t) 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    }
                    if constexpr (CK) {
                        /* the group sums' tree: idx is this sum's subtree
                         * among n at the level, whose nodes start at base;
                         * a subtree without a sibling passes up unchanged */
                        const size_t nrc = (size_t) rows * ncol, at = (size_t) row * ncol + col;
                        int idx = cg, n = A.ck, base = 0;
                        while (last && n > 1) {
                            if ((idx ^ 1) < n) {
                                uint64_t * sl = A.kslot + (size_t) (base + (idx >> 1)) * nrc + at;
                                const uint64_t old = __hip_atomic_exchange(sl, (1ull << 32) | __float_as_uint(sum),
                                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                last = (uint32_t) (old >> 32) == 1u;
                                if (last) {
                                    sum = __uint_as_float((uint32_t) old) + sum;
                                    __hip_atomic_store(sl, (uint64_t) 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                }
                            }
                            base += (n + 1) >> 1;
                            idx >>= 1;
                            n = (n + 1) >> 1;
                        }
                    }
                    if (last) *yp = (A.accumulate ? *yp : 0.0f) + sum;
                    if constexpr (MC == 4) {
                        {
                            /* a gate/up pair over several columns: the two
                             * matrices' sums of (row, col) meet in
                             * pslot[row * ncol + col] as in the one-column
                             * form, and the second to arrive writes
                             * gelu(gate) * up to act [ncol][rows] */
                            const uint32_t mi = (int) blockIdx.x >= A.mat[1].wg0 ? 1u : 0u;
                            uint64_t * sl = A.pslot + (size_t) row * ncol + col;
                            const uint64_t mine = ((uint64_t) (1u + mi) << 32) | __float_as_uint(sum);
                            const uint64_t old =
                                __hip_atomic_exchange(sl, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            if ((uint32_t) (old >> 32) == 2u - mi) {
                                const float o = __uint_as_float((uint32_t) old);
                                const float v = mi ? gelu_mul(o, sum) : gelu_mul(sum, o);
                                const size_t ai = (size_t) col * rows + row;
                                if (A.pact) A.pact[ai] = v;
                                if (A.pact16) A.pact16[ai] = (uint16_t) bf16_rne(v);
                                __hip_atomic_store(sl, (uint64_t) 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            }
                        }
                    }
                }
            }
        }
        if (Cw > 1) {
            __syncthreads();
        } else {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    };
    /* the first unit's words were requested in the prologue; later units
     * (only when a workgroup holds more tiles than waves) request their own */
    unit(t0 + j);
    for (int it = 1; it < iters; it++) {
        const int tile = t0 + it * T + j;
        point(min(tile, t1 - 1));
        ld_gains(min(tile, t1 - 1));
        ld_head();
        unit(tile);
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

/* drow, when given, holds the row in device memory (a captured graph reads
 * the token it is replayed for); rows past the matrix decode nothing. */
/* Row `row` (or drow[blockIdx.y], read on the device) into out + blockIdx.y * ldo. */
__global__ void vq_row_dequant_kernel(const uint8_t * p, const Layout L, int row, const int * drow, float * out,
                                      size_t ldo) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (drow) row = drow[blockIdx.y];
    out += blockIdx.y * ldo;
    if (i >= L.nidx_row || row < 0 || row >= L.rows) return;
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
        case 2: return (size_t) nc * dim * 2 <= (size_t) kLdsMax;
        case 3: return fast_geometry_ok(dim, nc, rows, cols, v3);
        default: return 0;
    }
}

static int aligned4(const void * p) { return ((uintptr_t) p & 3u) == 0; }

template <int NST, int XF32, int EXT, int MSC, int MC = 0, int XN = 0>
static int launch_fast_t(const FastArgs & A, int grid, int threads, size_t lds, hipStream_t s) {
    static size_t opted = 0;
    static std::atomic<int> checked{0};
    const void * fn = (const void *) vq_mfma_kernel<NST, XF32, EXT, MSC, MC, XN>;
    if (!checked.load()) {
        /* the codeword gathers address LDS from 0: no static LDS may precede
         * the dynamic array */
        hipFuncAttributes fa;
        hipError_t e = hipFuncGetAttributes(&fa, fn);
        if (e != hipSuccess) return fail_hip("VQ block kernel attributes", e);
        if (fa.sharedSizeBytes != 0) {
            set_error("the VQ block kernel has %zu bytes of static LDS; its gathers assume none", fa.sharedSizeBytes);
            return -1;
        }
        checked.store(1);
    }
    if (lds > 65536 && lds > opted) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return fail_hip("LDS opt-in for the VQ block kernel", e);
        opted = lds;
    }
    launch_kernel(vq_mfma_kernel<NST, XF32, EXT, MSC, MC, XN>, dim3(grid), dim3(threads), (uint32_t) lds, s, A);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail_hip("VQ block kernel launch", e);
    return 0;
}

/* The block kernel's launch shape for a call: parts per MFMA (S), wave chunks
 * (C) and tiles per workgroup pass (T), so that about one workgroup per CU
 * gets eight or more waves of work. */
struct FastShape {
    int S, C, T, W, nwg;
    size_t lds;
    int xg;   /* several columns with x read from global memory (no x in LDS) */
    int sk;   /* shared tiles: W (tile, chunk) units per workgroup */
    int ck;   /* chunk-split tiles: groups of C chunks per tile (0: none) */
};

/* LDS bytes per activation column: 264 bytes per 128 columns (256 of f16
 * values and 8 of pad) and 8 more between columns. */
static int fast_xstride(int cols, int S) { (void) S; return 264 * (cols / 128) + 8; }

/* LDS bytes per stage codebook in the block kernel: a fixed 32 KB for
 * 12-bit indices (nc <= 4096; a smaller codebook leaves the rest unused),
 * else nc * 8 */
static size_t fast_cbs(int nc) { return nc > 4096 ? (size_t) nc * 8 : kCbStride12; }

static size_t fast_lds(const VqCall & c, int nst, int S, int W, int xg = 0) {
    return (size_t) nst * fast_cbs(c.nc) +
           (xg ? 0 : (size_t) (c.xf32 ? 2 : 1) * c.ncol * fast_xstride(c.cols, S)) +
           (size_t) W * kRedStride * 4 + kXrBytes;
}

/* Several bf16 columns with x read from global memory: each lane loads its
 * 32 activations of a step (64 bytes, 16-byte aligned rows) with the step's
 * index words, so nothing but codebooks sits in LDS and no column count
 * splits K. Taken when x is at least 48 KB (N = 8 at 4096 and 10240
 * columns: staging it cost more than its loads, measured); smaller x is
 * staged in LDS. Straight-line units only (a ring would hold 8 steps of x
 * per lane), at most 10 waves (the registers of 4 steps in flight), and
 * enough threads to stage the codebooks in 5 chunks each. Shape: fewest
 * rounds of workgroups over the CUs, then the shortest unit. */
static int fast_shape_xg(const VqCall & c, int nst, FastShape & sh) {
    if (c.ncol < 2 || c.xf32 || c.nc % 2 || ((uintptr_t) c.x & 15u) || c.ldx % 8) return -1;
    if ((long) c.ncol * c.cols < 24576) return -1;
    const int M = c.cols / 128, G = cu_count(), n16 = c.nc * 8 / 16;
    long best = -1;
    for (int s = 1; s <= 16; s *= 2) {
        if (s * c.ncol > 16 || M % s) continue;
        const int MP = M / s;
        for (int cc = 1; cc <= 10; cc++) {
            if (MP % cc) continue;
            const int ms = MP / cc;
            if (ms != 2 && ms != 4 && ms != 5 && ms != 8 && (ms != 10 || c.nc > 4096)) continue;
            for (int tt = 1; tt * cc <= 10; tt++) {
                if (5 * 64 * tt * cc < n16) continue;
                long nwg = 0;
                for (int m = 0; m < c.nmat; m++) nwg += ((c.mats[m].rows * (long) s + 15) / 16 + tt - 1) / tt;
                const size_t lds = fast_lds(c, nst, s, tt * cc, 1);
                if (lds > (size_t) kLdsMax) continue;
                const long cost = (nwg + G - 1) / G * (8 + ms) * 64 + tt * cc;
                if (best < 0 || cost < best) {
                    best = cost;
                    sh.S = s; sh.C = cc; sh.T = tt; sh.W = tt * cc; sh.nwg = (int) nwg; sh.lds = lds; sh.xg = 1;
                    sh.sk = 0;
                }
            }
        }
    }
    if (best < 0) return -1;
    /* Shared tiles, when the caller gave the slot words and whole tiles leave
     * more than a fifth of the CUs idle (N = 8 over 2560 rows: 160 of 256
     * busy): ten waves per workgroup, each one (tile, chunk) unit, a tile's
     * chunks over at most two workgroups (W >= C), as many workgroups as
     * fit one round; then the shortest unit. Units under 4 macro steps do
     * not pay for their own staging (N = 8 over 4096 columns: 2-step units
     * measured slower than whole tiles on 160 CUs). */
    if (c.kslot && c.nmat == 1 && (long) c.mats[0].rows * c.ncol <= c.kslot_cap && 5 * sh.nwg < 4 * G) {
        const int W = 10;
        int bn = 0, bms = 0;
        for (int s = 1; s <= 16; s *= 2) {
            if (s * c.ncol > 16 || M % s) continue;
            const int MP = M / s;
            const long tiles = (c.mats[0].rows * (long) s + 15) / 16;
            for (int cc = 2; cc <= W; cc++) {
                if (MP % cc) continue;
                const int ms = MP / cc;
                if (ms != 4 && ms != 5 && ms != 8 && (ms != 10 || c.nc > 4096)) continue;
                if (5 * 64 * W < n16) continue;
                const long nwg = (tiles * cc + W - 1) / W;
                const size_t lds = fast_lds(c, nst, s, W, 1);
                if (nwg > G || lds > (size_t) kLdsMax) continue;
                if (nwg > bn || (nwg == bn && ms < bms)) {
                    bn = (int) nwg; bms = ms;
                    if (bn > sh.nwg) {
                        sh.S = s; sh.C = cc; sh.T = 1; sh.W = W; sh.nwg = bn; sh.lds = lds; sh.xg = 1; sh.sk = 1;
                    }
                }
            }
        }
    }
    return 0;
}

/* Chunk-split tiles: several bf16 columns of one matrix whose x is too large
 * to stage whole (the same 48 KB as above), when the caller gave exchange
 * words for the tree (vq_ck_words(ck) per output element). A tile's K is ck
 * groups of C chunks; each workgroup stages one group's x and runs it for T
 * tiles (T * C waves, the group's chunks added in LDS), and the ck group
 * sums of a tile meet in the tree, whose levels are memory round trips
 * (about 0.65 us each, measured). Shape: fewest rounds of workgroups over
 * the CUs, then the shortest unit plus tree, then the fewest waves. */
static int fast_shape_ck(const VqCall & c, int nst, FastShape & sh) {
    if (!kFastCk || !c.kslot || c.nmat != 1 || c.ncol < 2 || c.xf32 || c.nc % 2 || ((uintptr_t) c.x & 15u) ||
        c.ldx % 8)
        return -1;
    if ((long) c.ncol * c.cols < 24576) return -1;
    const int M = c.cols / 128, G = cu_count(), n16 = c.nc * 8 / 16;
    long best = -1;
    for (int s = 1; s <= 16; s *= 2) {
        if (s * c.ncol > 16 || M % s) continue;
        const int MP = M / s;
        const long tiles = (c.mats[0].rows * (long) s + 15) / 16;
        for (int gk = 2; gk <= kVqCkMaxGroups; gk++) {
            if ((long) c.mats[0].rows * c.ncol * vq_ck_words(gk) > c.kslot_cap) continue;
            int lv = 0;
            for (int n = gk; n > 1; n = (n + 1) >> 1) lv++;
            for (int cc = 1; cc <= 10; cc++) {
                if (MP % (gk * cc)) continue;
                const int ms = MP / (gk * cc);
                if (ms != 2 && ms != 4 && ms != 5 && ms != 8 && (ms != 10 || c.nc > 4096)) continue;
                for (int tt = 1; tt * cc <= 10; tt++) {
                    if (5 * 64 * tt * cc < n16) continue;   /* the codebooks in 5 chunks per thread */
                    const long nwg = (tiles + tt - 1) / tt * gk;
                    const size_t lds = (size_t) nst * fast_cbs(c.nc) +
                                       (size_t) c.ncol * fast_xstride(s * cc * ms * 128, s) +
                                       (size_t) tt * cc * kRedStride * 4 + kXrBytes;
                    if (lds > (size_t) kLdsMax) continue;
                    const long cost = (nwg + G - 1) / G * (8 + ms * cc + 2 * lv) * 64 + tt * cc;
                    if (best < 0 || cost < best) {
                        best = cost;
                        sh.S = s; sh.C = cc; sh.T = tt; sh.W = tt * cc; sh.nwg = (int) nwg; sh.lds = lds;
                        sh.xg = 0; sh.sk = 0; sh.ck = gk;
                    }
                }
            }
        }
    }
    return best < 0 ? -1 : 0;
}

static int fast_shape(const VqCall & c, int nst, FastShape & sh) {
    sh.ck = 0;
    if (kFastXg && fast_shape_xg(c, nst, sh) == 0) {
        /* where x from global memory would take shared tiles (whole tiles
         * leave CUs idle), chunk-split tiles instead: N = 8 down 14.7 ->
         * 13.1-13.6 us, measured; for o (whole tiles on 160 CUs) they gave
         * -0.45 and +0.2 us on two boxes, and o keeps its shape */
        FastShape ck;
        if (sh.sk && fast_shape_ck(c, nst, ck) == 0) sh = ck;
        return 0;
    }
    sh.xg = 0;
    sh.sk = 0;
    const int M = c.cols / 4 / 32;
    const int G = cu_count();
    const int want = G * 8;
    long total_rows = 0;
    for (int m = 0; m < c.nmat; m++) total_rows += c.mats[m].rows;
    auto tiles_for = [&](int S) {
        long t = 0;
        for (int m = 0; m < c.nmat; m++) t += (c.mats[m].rows * (long) S + 15) / 16;
        return t;
    };
    int S = 0;
    for (int s = 1; s <= 16; s *= 2) {
        if (s * c.ncol > 16 || M % s) continue;
        S = s;
        if (tiles_for(s) >= want) break;
    }
    if (!S) { set_error("no MFMA part split fits %d columns and %d macro steps", c.ncol, M); return -1; }
    const long tiles = tiles_for(S);
    int C = 1;
    if (tiles < want) {
        const int MP = M / S;
        for (int cc = 2; cc <= 10; cc++) {
            if (MP % cc || MP / cc < 2) continue;
            C = cc;
            if (tiles * cc >= want) break;
        }
    }
    int T = (int) ((tiles + G - 1) / G);
    if (T < 1) T = 1;
    if (T * C > 10) T = 10 / C > 0 ? 10 / C : 1;
    if (T * C > 10) { C = 10; T = 1; }
    sh.S = S; sh.C = C; sh.T = T; sh.W = T * C;
    sh.nwg = 0;
    for (int m = 0; m < c.nmat; m++) sh.nwg += (int) (((c.mats[m].rows * (long) S + 15) / 16 + T - 1) / T);
    sh.lds = fast_lds(c, nst, S, sh.W);
    (void) total_rows;
    if (c.ncol > 1) {
        /* Several columns: codebooks plus N columns of x leave room for one
         * workgroup per CU, so the shape that matters is the number of rounds
         * of workgroups over the CUs. Search parts S, K chunks C and tiles T
         * (up to 16 waves) for the fewest rounds, then the shortest unit plus
         * chunk partials, preferring unit lengths with a straight-line
         * kernel. */
        /* 16 waves only in the multi-column kernels (bf16 x, even codebook,
         * 16-byte aligned x rows, at least 5 codebook chunks' worth of threads) */
        const int mc_ok = !c.xf32 && c.nc % 2 == 0 && !((uintptr_t) c.x & 15u) && c.ldx % 8 == 0;
        const int n16 = c.nc * 8 / 16;
        long best = -1;
        for (int s = 1; s <= 16; s *= 2) {
            if (s * c.ncol > 16 || M % s) continue;
            const int MP = M / s;
            for (int cc = 1; cc <= 16; cc++) {
                if (MP % cc) continue;
                const int ms = MP / cc;
                for (int tt = 1; tt * cc <= 16; tt++) {
                    if (tt * cc > 10 && !(mc_ok && n16 <= 5 * 64 * tt * cc)) continue;
                    long nwg = 0;
                    for (int m = 0; m < c.nmat; m++) nwg += ((c.mats[m].rows * (long) s + 15) / 16 + tt - 1) / tt;
                    const size_t lds = fast_lds(c, nst, s, tt * cc);
                    if (lds > (size_t) kLdsMax) continue;
                    const long rounds = (nwg + G - 1) / G;
                    const int straight = ms == 2 || ms == 4 || ms == 5 || ms == 8 || ms == 10;
                    /* each chunk beyond the first adds an LDS partial and a
                     * barrier to the tile's epilogue (N = 8 q+k+v+g: 8-row
                     * tiles of 2 chunks, 9.15 us, against 16-row tiles of
                     * 5 shorter chunks, 9.63 us) */
                    const long cost = rounds * (8 + ms + (straight ? 0 : ms) + cc - 1) * 64 + tt * cc;
                    if (best < 0 || cost < best) {
                        best = cost;
                        sh.S = s; sh.C = cc; sh.T = tt; sh.W = tt * cc; sh.nwg = (int) nwg; sh.lds = lds;
                    }
                }
            }
        }
    }
    return 0;
}

/* Units of 1-6, 8 or 10 macro steps (the trunk's shapes give 2, 5 and 10)
 * run the straight-line kernel for bf16 x; any other length, and f32 x, the
 * ring kernel. Thirteen-bit indices hold plane bytes too, so their
 * straight-line units stop at 8 steps (10 would spill). */
/* The one-column straight-line kernels that stage rms_norm(h) themselves. */
template <int NST, int EXT, int XN>
static int launch_ms_norm(const FastArgs & A, int MS, int grid, int threads, size_t lds, hipStream_t s) {
    switch (MS) {
        case 1: return launch_fast_t<NST, 0, EXT, 1, 0, XN>(A, grid, threads, lds, s);
        case 2: return launch_fast_t<NST, 0, EXT, 2, 0, XN>(A, grid, threads, lds, s);
        case 4: return launch_fast_t<NST, 0, EXT, 4, 0, XN>(A, grid, threads, lds, s);
        case 5: return launch_fast_t<NST, 0, EXT, 5, 0, XN>(A, grid, threads, lds, s);
        case 8: return launch_fast_t<NST, 0, EXT, 8, 0, XN>(A, grid, threads, lds, s);
        case 10:
            if constexpr (!EXT) return launch_fast_t<NST, 0, EXT, 10, 0, XN>(A, grid, threads, lds, s);
            break;
        default: break;
    }
    return 1;
}

template <int NST, int XF32, int EXT>
static int launch_ms(const FastArgs & A, int MS, int mc, int grid, int threads, size_t lds, hipStream_t s) {
    if constexpr (!XF32) {
        if (mc == 4) {
            /* several columns of a gate/up pair that writes the activation */
            if constexpr (!EXT) {
                switch (MS) {
                    case 2: return launch_fast_t<NST, 0, EXT, 2, 4>(A, grid, threads, lds, s);
                    case 4: return launch_fast_t<NST, 0, EXT, 4, 4>(A, grid, threads, lds, s);
                    case 5: return launch_fast_t<NST, 0, EXT, 5, 4>(A, grid, threads, lds, s);
                    case 8: return launch_fast_t<NST, 0, EXT, 8, 4>(A, grid, threads, lds, s);
                    case 10: return launch_fast_t<NST, 0, EXT, 10, 4>(A, grid, threads, lds, s);
                    default: break;
                }
            }
            set_error("no several-column pair kernel for units of %d macro steps", MS);
            return -1;
        }
        if (mc == 3) {
            /* chunk-split tiles: the search kept to these unit lengths */
            switch (MS) {
                case 2: return launch_fast_t<NST, 0, EXT, 2, 3>(A, grid, threads, lds, s);
                case 4: return launch_fast_t<NST, 0, EXT, 4, 3>(A, grid, threads, lds, s);
                case 5: return launch_fast_t<NST, 0, EXT, 5, 3>(A, grid, threads, lds, s);
                case 8: return launch_fast_t<NST, 0, EXT, 8, 3>(A, grid, threads, lds, s);
                case 10:
                    if constexpr (!EXT) return launch_fast_t<NST, 0, EXT, 10, 3>(A, grid, threads, lds, s);
                    break;
                default: break;
            }
            set_error("no chunk-split kernel for units of %d macro steps", MS);
            return -1;
        }
        if (mc == 2) {
            /* x from global memory: the shape search kept to these unit lengths */
            switch (MS) {
                case 2: return launch_fast_t<NST, 0, EXT, 2, 2>(A, grid, threads, lds, s);
                case 4: return launch_fast_t<NST, 0, EXT, 4, 2>(A, grid, threads, lds, s);
                case 5: return launch_fast_t<NST, 0, EXT, 5, 2>(A, grid, threads, lds, s);
                case 8: return launch_fast_t<NST, 0, EXT, 8, 2>(A, grid, threads, lds, s);
                case 10:
                    if constexpr (!EXT) return launch_fast_t<NST, 0, EXT, 10, 2>(A, grid, threads, lds, s);
                    break;
                default: break;
            }
            set_error("no x-from-global kernel for units of %d macro steps", MS);
            return -1;
        }
        if (mc) {
            /* several columns: the unit lengths of the trunk's verify shapes */
            switch (MS) {
                case 2: return launch_fast_t<NST, 0, EXT, 2, 1>(A, grid, threads, lds, s);
                case 4: return launch_fast_t<NST, 0, EXT, 4, 1>(A, grid, threads, lds, s);
                case 5: return launch_fast_t<NST, 0, EXT, 5, 1>(A, grid, threads, lds, s);
                case 8: return launch_fast_t<NST, 0, EXT, 8, 1>(A, grid, threads, lds, s);
                case 10: if (!EXT) return launch_fast_t<NST, 0, EXT, EXT ? 0 : 10, 1>(A, grid, threads, lds, s); break;
                default: break;
            }
            return launch_fast_t<NST, 0, EXT, 0, 1>(A, grid, threads, lds, s);
        }
        switch (MS) {
            case 1: return launch_fast_t<NST, 0, EXT, 1>(A, grid, threads, lds, s);
            case 2: return launch_fast_t<NST, 0, EXT, 2>(A, grid, threads, lds, s);
            case 3: return launch_fast_t<NST, 0, EXT, 3>(A, grid, threads, lds, s);
            case 4: return launch_fast_t<NST, 0, EXT, 4>(A, grid, threads, lds, s);
            case 5: return launch_fast_t<NST, 0, EXT, 5>(A, grid, threads, lds, s);
            case 6: return launch_fast_t<NST, 0, EXT, 6>(A, grid, threads, lds, s);
            case 8: return launch_fast_t<NST, 0, EXT, 8>(A, grid, threads, lds, s);
            case 10: if (!EXT) return launch_fast_t<NST, 0, EXT, EXT ? 0 : 10>(A, grid, threads, lds, s); break;
            default: break;
        }
    } else if (!mc) {
        /* f32 x, one column: the trunk's unit lengths run straight-line too
         * (x as hi + lo f16 in LDS, two MFMAs per step) */
        switch (MS) {
            case 2: return launch_fast_t<NST, 1, EXT, 2>(A, grid, threads, lds, s);
            case 5: return launch_fast_t<NST, 1, EXT, 5>(A, grid, threads, lds, s);
            case 8: return launch_fast_t<NST, 1, EXT, 8>(A, grid, threads, lds, s);
            case 10: if (!EXT) return launch_fast_t<NST, 1, EXT, EXT ? 0 : 10>(A, grid, threads, lds, s); break;
            default: break;
        }
    }
    return launch_fast_t<NST, XF32, EXT, 0>(A, grid, threads, lds, s);
}

/* One launch of the block kernel over macro steps [k0, k0 + mk) of every row
 * (the whole row unless x has to be split to fit LDS). */
struct FastNorm {
    const float * w;
    float eps;
    uint16_t * xout;
};

/* nrm: stage bf16(rms_norm(x) * w) from the f32 residual x (one column, the
 * whole row in one launch, a one-column straight-line shape); returns 1
 * without launching when the call's shape has no such kernel. */
/* The unit lengths with a straight-line one-column kernel (launch_ms and
 * launch_ms_norm below). */
static int straight_ms(int MS, int ext, int norm) {
    switch (MS) {
        case 1: case 2: case 4: case 5: case 8: return 1;
        case 3: case 6: return !norm;
        case 10: return !ext;
        default: return 0;
    }
}

static int launch_fast_part(const VqCall & c, int st0, int nst, int accumulate, int k0, int mk,
                            const FastNorm * nrm = nullptr, const VqPair * pair = nullptr) {
    const Layout L0 = make_layout(c.dim, c.nc, c.mats[0].rows, c.cols, 1);
    const int ext = L0.nbit > 12;
    VqCall part = c;
    part.cols = 128 * mk;
    FastShape sh;
    if (fast_shape(part, nst, sh)) return -1;
    if (sh.lds > (size_t) kLdsMax) {
        set_error("codebooks and %d activation columns of %d need %zu bytes of LDS", c.ncol, part.cols, sh.lds);
        return -1;
    }
    FastArgs A;
    memset(&A, 0, sizeof A);
    A.x = (const uint8_t *) c.x + (size_t) 128 * k0 * (c.xf32 || nrm ? 4 : 2);
    if (nrm) {
        A.nw = nrm->w;
        A.eps = nrm->eps;
        A.xout = nrm->xout;
    }
    A.nmat = c.nmat;
    A.cols = part.cols;
    A.nc = c.nc;
    A.ncol = c.ncol;
    A.ldx = c.ldx;
    A.ldy = c.ldy;
    A.accumulate = accumulate;
    A.gain_off = (uint32_t) L0.gain_off;
    A.mrow = (uint32_t) L0.mrow;
    A.prow = (uint32_t) L0.prow;
    A.lgS = 0;
    while ((1 << A.lgS) < sh.S) A.lgS++;
    A.C = sh.C; A.T = sh.T;
    A.sk = sh.sk;
    A.ck = sh.ck;
    A.kslot = sh.sk || sh.ck ? c.kslot : nullptr;
    A.M = mk;
    A.kofs = k0;
    A.xstride = sh.xg ? 0 : sh.ck ? fast_xstride(mk * 128 / sh.ck, sh.S) : fast_xstride(part.cols, sh.S);
    int wg = 0;
    for (int m = 0; m < c.nmat; m++) {
        for (int s = 0; s < nst; s++) A.mat[m].st[s] = (const uint8_t *) c.mats[m].stages[st0 + s];
        A.mat[m].y = c.mats[m].y;
        A.mat[m].rows = c.mats[m].rows;
        A.mat[m].tiles = (int) ((c.mats[m].rows * (long) sh.S + 15) / 16);
        A.mat[m].wg0 = wg;
        A.mat[m].nwg = sh.sk   ? (A.mat[m].tiles * sh.C + sh.W - 1) / sh.W
                       : sh.ck ? (A.mat[m].tiles + sh.T - 1) / sh.T * sh.ck
                               : (A.mat[m].tiles + sh.T - 1) / sh.T;
        wg += A.mat[m].nwg;
    }
    const int threads = sh.W * 64;
    A.threads = threads;
    /* The straight-line kernels take an even codebook, and bf16 x or one
     * column of f32 x. One column is staged in one branch-free pass and
     * reduced within a wave: 16-byte aligned x of at most 16 * threads
     * values, one wave per tile, at most 5 codebook chunks per thread and
     * stage. Several bf16 columns are staged by loops before the index words
     * are requested. */
    const int n16 = c.nc * 8 / 16;
    const int one_col = sh.C == 1 && !((uintptr_t) A.x & 15u) && n16 <= 5 * threads && part.cols <= 16 * threads;
    const int multi_col = c.ncol > 1 && !((uintptr_t) A.x & 15u) && c.ldx % 8 == 0 && n16 <= 5 * threads;
    const int straight = (!c.xf32 || c.ncol == 1) && c.nc % 2 == 0 && (c.ncol > 1 ? multi_col : one_col);
    const int MS = sh.xg ? A.M / sh.S / sh.C : sh.ck ? A.M / sh.S / sh.C / sh.ck : straight ? A.M / sh.S / sh.C : 0;
    /* the multi-column kernels: x from global memory (2) or staged in LDS (1;
     * MS without its own instantiation runs their ring form); any other
     * several-column call runs the generic kernel, which the shape search
     * kept within 10 waves */
    int mc = sh.ck ? 3 : sh.xg ? 2 : c.ncol > 1 && straight;
    if (pair) {
        /* the pair's activation is written by the straight-line kernels over
         * the whole row, both stages in this launch: one column, or several
         * staged in LDS (no K split, so each tile's sum is whole in one
         * workgroup) */
        if (c.nmat != 2 || c.mats[0].rows != c.mats[1].rows || !straight || k0 != 0 || mk * 128 != c.cols ||
            accumulate || st0 != 0 || nst != c.nst || (long) c.mats[0].rows * c.ncol > pair->cap)
            return 1;
        if (c.ncol > 1 ? mc != 1 || ext || nrm || (MS != 2 && MS != 4 && MS != 5 && MS != 8 && MS != 10)
                       : mc || !straight_ms(MS, ext, nrm != nullptr))
            return 1;
        if (mc == 1) mc = 4;   /* the several-column pair's own kernel */
        A.pslot = pair->slot;
        A.pact = pair->act;
        A.pact16 = pair->act16;
    }
    if (nrm) {
        /* the staging holds 2 chunks of 4 columns per thread */
        if (c.ncol != 1 || c.xf32 || !straight || mc || k0 != 0 || mk * 128 != c.cols || ((uintptr_t) nrm->w & 15u) ||
            ((uintptr_t) nrm->xout & 7u) || c.cols > 8 * threads)
            return 1;
        if (nst == 2) return ext ? launch_ms_norm<2, 1, 1>(A, MS, wg, threads, sh.lds, c.stream)
                                 : launch_ms_norm<2, 0, 1>(A, MS, wg, threads, sh.lds, c.stream);
        return ext ? launch_ms_norm<1, 1, 1>(A, MS, wg, threads, sh.lds, c.stream)
                   : launch_ms_norm<1, 0, 1>(A, MS, wg, threads, sh.lds, c.stream);
    }
    if (nst == 2) {
        if (c.xf32) return ext ? launch_ms<2, 1, 1>(A, MS, mc, wg, threads, sh.lds, c.stream)
                               : launch_ms<2, 1, 0>(A, MS, mc, wg, threads, sh.lds, c.stream);
        return ext ? launch_ms<2, 0, 1>(A, MS, mc, wg, threads, sh.lds, c.stream)
                   : launch_ms<2, 0, 0>(A, MS, mc, wg, threads, sh.lds, c.stream);
    }
    if (c.xf32) return ext ? launch_ms<1, 1, 1>(A, MS, mc, wg, threads, sh.lds, c.stream)
                           : launch_ms<1, 1, 0>(A, MS, mc, wg, threads, sh.lds, c.stream);
    return ext ? launch_ms<1, 0, 1>(A, MS, mc, wg, threads, sh.lds, c.stream)
               : launch_ms<1, 0, 0>(A, MS, mc, wg, threads, sh.lds, c.stream);
}

/* How many consecutive K ranges the call needs so that x (all its columns)
 * fits LDS beside the codebooks: 1 for N = 1 at the trunk's shapes, 2 for
 * N = 8 over 10240 columns. 0 when no split fits. */
static int fast_splits(const VqCall & c, int nst) {
    const int M = c.cols / 128;
    for (int n = 1; n <= M; n++) {
        const int mk = (M + n - 1) / n;
        if (mk * (n - 1) >= M) continue;
        int ok = 1;
        for (int k0 = 0; k0 < M && ok; k0 += mk) {
            VqCall part = c;
            part.cols = 128 * (M - k0 < mk ? M - k0 : mk);
            FastShape sh;
            if (fast_shape(part, nst, sh) || sh.lds > (size_t) kLdsMax) ok = 0;
        }
        if (ok) return n;
    }
    return 0;
}

static int launch_fast(const VqCall & c, int st0, int nst, int accumulate) {
    const int n = fast_splits(c, nst);
    if (!n) {
        set_error("the VQ block kernel finds no split of %d columns that fits LDS", c.cols);
        return -1;
    }
    const int M = c.cols / 128, mk = (M + n - 1) / n;
    for (int k0 = 0; k0 < M; k0 += mk)
        if (launch_fast_part(c, st0, nst, accumulate || k0 > 0, k0, M - k0 < mk ? M - k0 : mk)) return -1;
    return 0;
}

static int launch_wave(const VqCall & c, int variant) {
    /* A wider request runs as more 256-thread workgroups: the width only
     * changes how many row-waves share a workgroup, never the arithmetic. */
    const int threads = c.threads && c.threads < 256 ? c.threads : 256;
    const int nw = threads / 64;
    const size_t lds = variant == 2 ? (size_t) c.nc * c.dim * 2 : 0;
    if (lds > 65536) {
        static size_t opted = 0;
        if (lds > opted) {
            hipError_t e = hipFuncSetAttribute((const void *) vq_wave_kernel<1>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
            if (e != hipSuccess) return fail_hip("LDS opt-in for the codebook wave kernel", e);
            opted = lds;
        }
    }
    for (int m = 0; m < c.nmat; m++) {
        const Layout L = make_layout(c.dim, c.nc, c.mats[m].rows, c.cols, c.v3);
        int grid = c.grid > 0 ? c.grid : (L.rows + nw - 1) / nw;
        for (int s = 0; s < c.nst; s++) {
            const int acc = s > 0 || c.accumulate;
            const uint8_t * p = (const uint8_t *) c.mats[m].stages[s];
            if (variant == 2)
                launch_kernel(vq_wave_kernel<1>, dim3(grid), dim3(threads), (uint32_t) lds, c.stream, p, L, c.x, c.ldx,
                                   c.xf32, c.ncol, c.mats[m].y, c.ldy, acc);
            else
                launch_kernel(vq_wave_kernel<0>, dim3(grid), dim3(threads), 0u, c.stream, p, L, c.x, c.ldx,
                                   c.xf32, c.ncol, c.mats[m].y, c.ldy, acc);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return fail_hip("VQ wave kernel launch", e);
        }
    }
    return 0;
}

int vq_norm_launch(const VqCall & c, const float * norm_w, float eps, uint16_t * x_out, const VqPair * pair) {
    /* the fused kernel's conditions: one f32 column, every matrix on the
     * block kernel, at most two stages and four matrices, one K range */
    if (!norm_w || c.ncol != 1 || !c.x || ((uintptr_t) c.x & 15u) || c.nst < 1 || c.nst > 2 || c.nmat < 1 ||
        c.nmat > kFastMats || c.variant || c.threads || c.grid || c.dim != 4 || c.cols % 128)
        return 1;
    if (pair && (!pair->slot || pair->cap < 1)) return 1;
    for (int m = 0; m < c.nmat; m++) {
        if (!c.mats[m].y || c.mats[m].rows <= 0) return 1;
        for (int s = 0; s < c.nst; s++)
            if (!c.mats[m].stages[s] || !aligned4(c.mats[m].stages[s])) return 1;
        if (!fast_geometry_ok(c.dim, c.nc, c.mats[m].rows, c.cols, c.v3)) return 1;
    }
    if (c.v3 && bits_for(c.nc) > 13) return 1;
    VqCall b = c;
    b.xf32 = 0;   /* what is staged: one bf16 column */
    if (fast_splits(b, c.nst) != 1) return 1;
    const FastNorm nrm{norm_w, eps, x_out};
    return launch_fast_part(b, 0, c.nst, c.accumulate, 0, c.cols / 128, &nrm, pair);
}

int vq_pair_launch(const VqCall & c, const VqPair & pair) {
    /* bf16 columns in one K range, both matrices on the block kernel */
    if (!pair.slot || pair.cap < 1 || c.ncol < 1 || c.ncol > kMaxCols || !c.x || c.xf32 || ((uintptr_t) c.x & 15u) ||
        c.nst < 1 || c.nst > 2 || c.nmat != 2 || c.variant || c.threads || c.grid || c.dim != 4 || c.cols % 128 ||
        c.accumulate)
        return 1;
    for (int m = 0; m < c.nmat; m++) {
        if (!c.mats[m].y || c.mats[m].rows <= 0) return 1;
        for (int s = 0; s < c.nst; s++)
            if (!c.mats[m].stages[s] || !aligned4(c.mats[m].stages[s])) return 1;
        if (!fast_geometry_ok(c.dim, c.nc, c.mats[m].rows, c.cols, c.v3)) return 1;
    }
    if (c.v3 && bits_for(c.nc) > 13) return 1;
    if (fast_splits(c, c.nst) != 1) return 1;
    return launch_fast_part(c, 0, c.nst, 0, 0, c.cols / 128, nullptr, &pair);
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
    /* the block kernel reads bf16 x in aligned pairs */
    if (!c.xf32 && (((uintptr_t) c.x & 3u) || (c.ncol > 1 && (c.ldx & 1)))) all_fast = 0;
    if (all_fast) {
        /* the block kernel also needs its codebooks and x resident in LDS */
        const int nst = c.nst < 2 ? c.nst : 2;
        for (int m0 = 0; m0 < c.nmat && all_fast; m0 += kFastMats) {
            VqCall part = c;
            part.mats = c.mats + m0;
            part.nmat = c.nmat - m0 < kFastMats ? c.nmat - m0 : kFastMats;
            if (!fast_splits(part, nst)) all_fast = 0;
        }
    }
    int variant = c.variant;
    if (variant == 0) variant = all_fast ? 3 : ((size_t) c.nc * c.dim * 2 <= (size_t) kLdsMax ? 2 : 1);
    if (variant == 3) {
        if (!all_fast) {
            set_error("the VQ block kernel does not take this geometry, alignment or LDS footprint");
            return -1;
        }
        for (int m0 = 0; m0 < c.nmat; m0 += kFastMats) {
            VqCall part = c;
            part.mats = c.mats + m0;
            part.nmat = c.nmat - m0 < kFastMats ? c.nmat - m0 : kFastMats;
            for (int st0 = 0; st0 < c.nst; st0 += 2) {
                const int n = c.nst - st0 < 2 ? c.nst - st0 : 2;
                if (launch_fast(part, st0, n, st0 > 0 || c.accumulate)) return -1;
            }
        }
        return 0;
    }
    if (variant == 2 && (size_t) c.nc * c.dim * 2 > (size_t) kLdsMax) {
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
                       0, s, (const uint8_t *) payload, L, row, (const int *) nullptr, out, (size_t) 0);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("row dequant launch", e);
}

int vq_row_dequant_dev_launch(const void * payload, const Layout & L, const int * drow, float * out, hipStream_t s,
                              int nrows, size_t ldo) {
    const int threads = 256;
    if (nrows < 1) { set_error("row dequant needs at least one row"); return -1; }
    hipLaunchKernelGGL(vq_row_dequant_kernel, dim3((unsigned) ((L.nidx_row + threads - 1) / threads), (unsigned) nrows),
                       dim3(threads), 0, s, (const uint8_t *) payload, L, 0, drow, out, ldo);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("row dequant launch", e);
}

int f32_gemv_launch(const float * w, const float * x, float * y, int rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL(f32_gemv_kernel, dim3((unsigned) ((rows + 3) / 4)), dim3(256), 0, s, w, x, y, rows, cols);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip("f32 gemv launch", e);
}

}  // namespace sparkmv
