/* vq_tile.h — the MFMA tile primitives of the dim-4 DQV3 GEMV kernels (device
 * code only): 12-bit field addresses, the index words of one macro step, and
 * one macro step of codeword gathers and matrix-core products.
 *
 * A macro step is 32 indices (128 columns) of a row: lane quarter q of a wave
 * reads the 12 bytes that hold indices 8q .. 8q + 7, gathers their raw f16
 * codewords from the LDS codebook straight into the A operand (two per
 * v_mfma_f32_16x16x32_f16, or one per v_mfma_f32_16x16x16_f16 when x comes
 * from global memory), and takes the matching activations as the B operand.
 * Codeword times activation is exact in f16 x f16 -> f32; only the f32
 * accumulation rounds. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sparkmv {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

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

template <int NST, int EXT, int XG = 0>
struct Words {
    uint32_t w[NST][3];
    uint32_t pb[NST];
    uint32_t xg[XG ? 16 : 1];   /* XG: the lane's 32 bf16 activations of the step */
};

/* Index words of one macro step: 12 bytes (8 indices) per lane quarter of
 * each stage's row stream, and for 13-bit indices the plane byte. With XG
 * also the lane's 64 bytes of bf16 x for the step (128 columns per step,
 * 32 per lane quarter), read straight from global memory. */
template <int NST, int EXT, int XG = 0>
__device__ __forceinline__ void load_words(Words<NST, EXT, XG> & W, const uint8_t * const * rp,
                                           const uint8_t * const * pp, const uint8_t * xp, int ms) {
#pragma unroll
    for (int s = 0; s < NST; s++) {
        const uint32_t * p = (const uint32_t *) (rp[s] + 48 * ms);
        W.w[s][0] = p[0];
        W.w[s][1] = p[1];
        W.w[s][2] = p[2];
        if (EXT) W.pb[s] = pp[s][4 * ms];
    }
    if constexpr (XG != 0) {
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        const u4v * q = (const u4v *) (xp + 256 * ms);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const u4v v = q[k];
            W.xg[4 * k] = v.x; W.xg[4 * k + 1] = v.y; W.xg[4 * k + 2] = v.z; W.xg[4 * k + 3] = v.w;
        }
    }
}

/* One macro step: 8 MFMA steps per stage. k-slot (quarter q, step t) is
 * index 8q + t of the macro step, i.e. columns 4 * that .. + 3; A (the
 * codeword) and B (the activations) use the same assignment. Every LDS read
 * of the step (8 B reads, 8 * NST codeword gathers) is issued before the
 * first MFMA, so the gathers' latency overlaps. */
template <int T, int NST, int EXT, int XG>
__device__ __forceinline__ uint32_t step_addr(const Words<NST, EXT, XG> & W, int s, uint32_t cbs) {
    uint32_t a = cw_addr<T>(W.w[s][0], W.w[s][1], W.w[s][2]);
    if (EXT) a |= (W.pb[s] << (15 - T)) & 0x8000u;
    return (uint32_t) s * cbs + a;
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

/* XG, SCX = 0: *xm (when given) keeps, per 16-bit half, the largest bf16
 * magnitude |x| of the lane's values so far (bf16 magnitudes order as
 * integers; an infinity or NaN is larger than any finite value), from which
 * the caller finds units of small x. SCX: x is multiplied by sc (a power of
 * two) before it is converted. */
/* A codeword at LDS byte address a. The codebooks sit at the start of the
 * kernel's dynamic LDS, which begins at address 0 (the kernels that call this
 * have no static LDS; their launcher checks), so the address is the gather's
 * own offset: no base is added, and a constant stage offset goes into the
 * instruction's offset field. */
__device__ __forceinline__ h4 cw_read(uint32_t a) {
    typedef const __attribute__((address_space(3))) h4 lds_h4;
    return *(lds_h4 *) (size_t) a;
}

/* cbs: LDS bytes from one stage's codebook to the next (32 KB for 12-bit
 * indices, so the second stage's offset is an immediate). Every gather goes
 * by absolute LDS address (cw_read): against a base add per gather, the
 * several-column verify step went 2087 -> 2060 us and, once two codewords
 * shared an MFMA, the one-column decode set 1534-1538 -> 1516-1520 us. */
template <int NST, int XF32, int EXT, int XG = 0, int SCX = 0>
__device__ __forceinline__ void mstep(const Words<NST, EXT, XG> & W, uint32_t cbs, const uint8_t * xb,
                                      const uint8_t * xbl, f4 * acc, float sc = 1.0f, u16x2 * xm = nullptr) {
    h4 cw[8][NST], b[8], bl[8];
    auto rd = [](uint32_t a) -> h4 { return cw_read(a); };
#pragma unroll
    for (int s = 0; s < NST; s++) {
        cw[0][s] = rd(step_addr<0, NST, EXT, XG>(W, s, cbs));
        cw[1][s] = rd(step_addr<1, NST, EXT, XG>(W, s, cbs));
        cw[2][s] = rd(step_addr<2, NST, EXT, XG>(W, s, cbs));
        cw[3][s] = rd(step_addr<3, NST, EXT, XG>(W, s, cbs));
        cw[4][s] = rd(step_addr<4, NST, EXT, XG>(W, s, cbs));
        cw[5][s] = rd(step_addr<5, NST, EXT, XG>(W, s, cbs));
        cw[6][s] = rd(step_addr<6, NST, EXT, XG>(W, s, cbs));
        cw[7][s] = rd(step_addr<7, NST, EXT, XG>(W, s, cbs));
    }
#pragma unroll
    for (int t = 0; t < 8; t++) {
        if constexpr (XG != 0) {
            /* bf16 pairs to f16 (exact from 2^-14 to 65504); SCX: times
             * the power of two sc first (the out-of-range redo) */
            const uint32_t u0 = W.xg[2 * t], u1 = W.xg[2 * t + 1];
            const float f0 = __uint_as_float(u0 << 16), f1 = __uint_as_float(u0 & 0xffff0000u);
            const float f2 = __uint_as_float(u1 << 16), f3 = __uint_as_float(u1 & 0xffff0000u);
            b[t][0] = (_Float16) (SCX ? f0 * sc : f0);
            b[t][1] = (_Float16) (SCX ? f1 * sc : f1);
            b[t][2] = (_Float16) (SCX ? f2 * sc : f2);
            b[t][3] = (_Float16) (SCX ? f3 * sc : f3);
            if (!SCX && xm) {
                *xm = __builtin_elementwise_max(*xm, __builtin_bit_cast(u16x2, u0 & 0x7fff7fffu));
                *xm = __builtin_elementwise_max(*xm, __builtin_bit_cast(u16x2, u1 & 0x7fff7fffu));
            }
        } else {
            b[t] = *(const h4 *) (xb + 8 * t);
            if (XF32) bl[t] = *(const h4 *) (xbl + 8 * t);
        }
    }
    /* With x in LDS, k-slots t and t + 1 go into one
     * v_mfma_f32_16x16x32_f16: a lane's A holds its two codewords and B the
     * matching two quads of x (the same pairing on both sides). On gfx950 it
     * issues in about the time of one 16x16x16 (31 against 30 cycles,
     * measured), so a step takes half the matrix-core time: decode set
     * 1571-1578 -> 1554-1565 us, N = 8 gate+up 16.9 -> 16.65 us. The
     * x-from-global kernels keep 16x16x16: paired, they spill at their
     * register cap and lost 0.3-0.9 us per launch. */
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    if constexpr (XG != 0) {
#pragma unroll
        for (int t = 0; t < 8; t++) {
#pragma unroll
            for (int s = 0; s < NST; s++) {
                acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(cw[t][s], b[t], acc[s], 0, 0, 0);
                if (XF32) acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(cw[t][s], bl[t], acc[s], 0, 0, 0);
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
        const h8 bp = __builtin_shufflevector(b[t], b[t + 1], 0, 1, 2, 3, 4, 5, 6, 7);
        h8 blp;
        if (XF32) blp = __builtin_shufflevector(bl[t], bl[t + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int s = 0; s < NST; s++) {
            const h8 ap = __builtin_shufflevector(cw[t][s], cw[t + 1][s], 0, 1, 2, 3, 4, 5, 6, 7);
            acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap, bp, acc[s], 0, 0, 0);
            if (XF32) acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap, blp, acc[s], 0, 0, 0);
        }
    }
}

}  // namespace sparkmv
