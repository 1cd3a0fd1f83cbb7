/* forward.hip — one decode token through the whole model on gfx950: the
 * embedding row, every layer's norm / attention / MLP around the library's
 * matvecs, the final norm and the tied-head logits.
 *
 * Semantics are the reference's CPU forward (tools/vq-runtime/src/
 * model.rs:441-591), which its GPU runtime mirrors launch by launch
 * (tools/vq/gpu/vq-model-gpu.cu:776-835):
 *
 *   h = embed[token]
 *   per layer:  xn = rms_norm(h, in_norm)                  (f64 sum of squares)
 *               [q k v] = qkv xn ; g = attn_gate xn
 *               rope over the first head_dim * partial elements of each q, k head
 *               K[pos], V[pos] = k, v
 *               per head: softmax over the layer's window of q.K/sqrt(hd), times V,
 *                         times sigmoid(g[head])
 *               h += out attn
 *               xn = rms_norm(h, post_norm)
 *               h += down (gelu(gate xn) * (up xn))        (exact erf gelu)
 *   logits = embed rms_norm(h, norm)                        (tied head)
 *
 * The matvecs are the library's own (VQ trunk, VQ or Q8_0 head). The
 * elementwise kernels here are small and latency-bound: one token is a few
 * thousand values. What matters for them is a short chain, so rope and the
 * KV store are one launch, and the norms and activations write the
 * matvecs' input in the form they read (f32, or bf16 when the model runs its
 * matvecs on bf16 activations). Activations stay f32 between kernels.
 *
 * The token and position live in device memory (two ints the chain's first
 * launch sets), and every kernel that depends on them reads them there: the
 * embedding row, rope and the KV row, the attention window. The chain's
 * launches are then the same for every token, so it is recorded once as a
 * HIP graph and replayed per token (sparkmv_model_capture / _replay); each
 * attention launch reserves LDS for its longest window.
 */
#include "act.h"
#include "kq.h"
#include "model.h"
#include "prefill.h"
#include "vq.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <vector>

#include "../../include/sparkmv.h"

namespace sparkmv {

/* f32 -> bf16, round to nearest even (NaN stays NaN) */
__device__ __forceinline__ uint16_t fw_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}

__global__ void fw_fill_kernel(float * p, int n, float v) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += blockDim.x * gridDim.x) p[i] = v;
}

/* st[0] = token, st[1] = position, and the position's rope tables for the
 * full and the sliding layers (model.rs:416-428, f32): tab[r][0][i] = cos,
 * tab[r][1][i] = sin of pos * theta_r^(-2i / pdim_r), i < pdim_r / 2 <= 128. */
__global__ void fw_set_state_kernel(int * st, int token, int pos, float theta0, int pdim0, float theta1, int pdim1,
                                    float * tab) {
    const int i = threadIdx.x;
    if (i == 0) {
        st[0] = token;
        st[1] = pos;
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const float theta = r ? theta1 : theta0;
        const int pdim = r ? pdim1 : pdim0;
        if (i < pdim / 2) {
            const float freq = 1.0f / powf(theta, (float) (2 * i) / (float) pdim);
            const float a = (float) pos * freq;
            tab[r * 256 + i] = cosf(a);
            tab[r * 256 + 128 + i] = sinf(a);
        }
    }
}

/* The embedding row of a Q8_0 tied head: row st[0], d * q exactly. */
__global__ void fw_q8_0_row_kernel(const uint8_t * blocks, int cols, const int * st, float * out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= cols) return;
    const uint8_t * b = blocks + ((size_t) st[0] * (cols >> 5) + (i >> 5)) * 34;
    _Float16 d;
    __builtin_memcpy(&d, b, 2);
    out[i] = (float) d * (float) (int8_t) b[2 + (i & 31)];
}

/* out = x * inv * w with inv = 1 / sqrt(mean(x^2) + eps), the sum of squares in
 * f64 and inv rounded once to f32 (model.rs:236-245). One workgroup. */
template <int PER>
__global__ __launch_bounds__(256) void fw_rmsnorm_kernel(const float * x, const float * w, float * out,
                                                         uint16_t * out16, int n, float eps) {
    __shared__ double part[4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    /* workgroup b normalizes column b (a verify block's tokens) */
    x += (size_t) blockIdx.x * n;
    if (out) out += (size_t) blockIdx.x * n;
    if (out16) out16 += (size_t) blockIdx.x * n;
    /* x and w of this thread's elements requested together: one memory
     * round trip before the reduction */
    float xv[PER], wv[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = t + 256 * k;
        xv[k] = i < n ? x[i] : 0.0f;
        wv[k] = i < n ? w[i] : 0.0f;
    }
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < PER; k++) s += (double) xv[k] * (double) xv[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) part[wave] = s;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = (float) (1.0 / sqrt(tot / (double) n + (double) eps));
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = t + 256 * k;
        if (i < n) {
            const float v = xv[k] * inv * wv[k];
            if (out) out[i] = v;
            if (out16) out16[i] = fw_bf16(v);
        }
    }
}

/* Rope, the KV store and attention over the layer's window of the cache,
 * positions start .. pos (model.rs:484-557; window 0: every position), split
 * by positions so that a long window keeps many CUs busy:
 *
 *   fw_attn_part_kernel: workgroup (chunk, kv head), one wave per query head
 *     of the kv head's group, kAttnChunk positions. Each lane holds VPL
 *     consecutive elements of a head. The wave rotates its query head in
 *     registers (rope over the first pdim elements with the position's f32
 *     table, model.rs:416-428, which the state kernel computes once per token
 *     for each layer type; the pair partner of element e is e +- pdim/2, in the
 *     lane pdim/2/VPL away, fetched with a lane permute). The chunk holding
 *     pos rotates the new key the same way, uses it and the new value from
 *     registers, and its first wave stores both in the cache (model.rs:
 *     498-503); other chunks read only older rows. A score is a lane-local dot
 *     and a butterfly; the wave keeps its chunk's maximum m, sum
 *     l = sum_j e^(s_j - m) and unnormalized o = sum_j e^(s_j - m) V[j].
 *   fw_attn_combine_kernel: workgroup per query head; rescales the chunks to
 *     the overall maximum M, divides by L = sum_c l_c e^(m_c - M) and applies
 *     the head's sigmoid gate. Its four waves take every fourth chunk.
 *
 * That is the CPU's softmax with the sum regrouped by chunk. Launch shapes
 * are fixed (the longest window), so a captured graph serves every position:
 * chunks past the current window do nothing. */
constexpr int kAttnChunk = 16;

template <int VPL>
__global__ __launch_bounds__(256) void fw_attn_part_kernel(const float * qkv, int qd, int kvd, float * kc, float * vc,
                                                            const int * st, int window, int heads, int kv_heads,
                                                            int pdim, const float * rtab, float scale, int nch_max,
                                                            float * part) {
    constexpr int hd = 64 * VPL, C = kAttnChunk;
    typedef float fv __attribute__((ext_vector_type(VPL)));
    const int pos = st[1];
    const int start = window > 0 && pos + 1 > window ? pos + 1 - window : 0;
    const int n = pos + 1 - start;
    const int chunk = blockIdx.x, kvh = blockIdx.y;
    const int G = heads / kv_heads;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j0 = chunk * C;
    if (j0 >= n) return;                        /* uniform: the combine reads chunks < ceil(n / chunk) */
    const int jn = min(C, n - j0);
    const int h = kvh * G + wave;               /* h * kv_heads / heads == kvh */
    const int half = pdim / 2;                  /* a multiple of VPL (the host checks) */
    /* x rotated by position pos: element e < half pairs with e + half,
     * e in [half, pdim) with e - half (apply_rope, model.rs:430-438). The
     * lane's cos and sin are read unconditionally (elements past pdim read
     * entry 0 and do not use it) and before the K and V rows: read inside
     * the per-element branch, each took a memory round trip of its own,
     * after the query's, ahead of the rows' loads. */
    const int e0 = lane * VPL;
    fv cv, sv;
#pragma unroll
    for (int v = 0; v < VPL; v++) {
        const int e = e0 + v;
        const int i = e < half ? e : (e < 2 * half ? e - half : 0);
        cv[v] = rtab[i];
        sv[v] = rtab[128 + i];
    }
    auto rope = [&](fv x) -> fv {
        const int pl = e0 < half ? lane + half / VPL : (e0 < pdim ? lane - half / VPL : lane);
        fv p, r = x;
#pragma unroll
        for (int v = 0; v < VPL; v++) p[v] = __shfl(x[v], pl, 64);
#pragma unroll
        for (int v = 0; v < VPL; v++) {
            const int e = e0 + v;
            if (e < 2 * half) r[v] = e < half ? x[v] * cv[v] - p[v] * sv[v] : x[v] * cv[v] + p[v] * sv[v];
        }
        return r;
    };
    const fv qx = *(const fv *) (qkv + (size_t) h * hd + lane * VPL);
    const float * kb = kc + (size_t) (start + j0) * kvd + (size_t) kvh * hd + lane * VPL;
    const float * vb = vc + (size_t) (start + j0) * kvd + (size_t) kvh * hd + lane * VPL;
    /* every K and V row of the chunk requested at once (rows past the
     * window re-read the last one and get weight zero), then the query
     * rotated while they are in flight */
    fv kr[C], vr[C];
#pragma unroll
    for (int j = 0; j < C; j++) kr[j] = *(const fv *) (kb + (size_t) min(j, jn - 1) * kvd);
#pragma unroll
    for (int j = 0; j < C; j++) vr[j] = *(const fv *) (vb + (size_t) min(j, jn - 1) * kvd);
    const fv q = rope(qx);
    if (j0 + jn == n) {
        /* this chunk ends at pos: the new key and value, from qkv */
        const fv kn = rope(*(const fv *) (qkv + qd + (size_t) kvh * hd + lane * VPL));
        const fv vn = *(const fv *) (qkv + qd + kvd + (size_t) kvh * hd + lane * VPL);
#pragma unroll
        for (int j = 0; j < C; j++)
            if (j == jn - 1) { kr[j] = kn; vr[j] = vn; }
        if (wave == 0) {
            *(fv *) (kc + (size_t) pos * kvd + (size_t) kvh * hd + lane * VPL) = kn;
            *(fv *) (vc + (size_t) pos * kvd + (size_t) kvh * hd + lane * VPL) = vn;
        }
    }
    float sc[C];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < C; j++) {
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < VPL; v++) s += q[v] * kr[j][v];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        sc[j] = s * scale;
        if (j < jn) m = fmaxf(m, sc[j]);
    }
    float l = 0.0f;
    fv o = (fv) 0.0f;
#pragma unroll
    for (int j = 0; j < C; j++) {
        /* rows past jn are padding that may hold anything (the row at pos
         * before its store): skipped, not weighted by zero */
        if (j < jn) {
            const float e = expf(sc[j] - m);
            l += e;
            o += e * vr[j];
        }
    }
    float * P = part + ((size_t) h * nch_max + chunk) * (hd + 2);
    *(fv *) (P + lane * VPL) = o;
    if (lane == 0) {
        P[hd] = m;
        P[hd + 1] = l;
    }
}

/* The combine of one query head from its nch chunk partials P (o, m, l per
 * chunk at stride hd + 2), four waves: M = max m_c, L = sum_c l_c e^(m_c - M)
 * (threads over chunks), wave w summing e^(m_c - M) o_c over chunks w,
 * w + 4, ... in increasing order, then out = the waves' sum / L times the
 * head's sigmoid gate gl. Each wave's first kPre chunk vectors are requested
 * before the m_c reductions, so up to 4 * kPre chunks cost one memory round
 * trip (a wave had taken one or four chunks per round trip: at context 1024
 * five of them). wts: 2 * nch floats of dynamic LDS. */
template <int VPL>
__device__ __forceinline__ void attn_combine_head(const float * P, int nch, float gl, float * out, uint16_t * out16,
                                                  float * wts) {
    constexpr int hd = 64 * VPL, kPre = 20;
    typedef float fv __attribute__((ext_vector_type(VPL)));
    __shared__ float red[8];
    __shared__ fv acc[4][64];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float * ls = wts + nch;
    float M = -INFINITY;
    for (int c = t; c < nch; c += 256) {
        const float mc = P[(size_t) c * (hd + 2) + hd], lc = P[(size_t) c * (hd + 2) + hd + 1];
        wts[c] = mc;
        ls[c] = lc;
        M = fmaxf(M, mc);
    }
    const float * Pl = P + lane * VPL;
    fv pre[kPre];
#pragma unroll
    for (int k = 0; k < kPre; k++) {
        /* chunks past nch re-read the last one (no branch between the
         * loads) and are not added. After the m_c loads on purpose: their
         * round trip then overlaps the reductions below (issued first, all
         * of them waited for together: decode token 2093 -> 2111 us) */
        const int c = min(wave + 4 * k, nch - 1);
        pre[k] = *(const fv *) (Pl + (size_t) c * (hd + 2));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float L = 0.0f;
    for (int c = t; c < nch; c += 256) {
        const float w = expf(wts[c] - M);
        wts[c] = w;
        L += w * ls[c];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
    if (lane == 0) red[4 + wave] = L;
    __syncthreads();
    fv o = (fv) 0.0f;
#pragma unroll
    for (int k = 0; k < kPre; k++)
        if (wave + 4 * k < nch) o += wts[wave + 4 * k] * pre[k];
    int c = wave + 4 * kPre;
    for (; c + 12 < nch; c += 16) {
        const fv a0 = *(const fv *) (Pl + (size_t) c * (hd + 2)), a1 = *(const fv *) (Pl + (size_t) (c + 4) * (hd + 2));
        const fv a2 = *(const fv *) (Pl + (size_t) (c + 8) * (hd + 2)), a3 = *(const fv *) (Pl + (size_t) (c + 12) * (hd + 2));
        o += wts[c] * a0;
        o += wts[c + 4] * a1;
        o += wts[c + 8] * a2;
        o += wts[c + 12] * a3;
    }
    for (; c < nch; c += 4) o += wts[c] * *(const fv *) (Pl + (size_t) c * (hd + 2));
    acc[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        const float inv = 1.0f / ((red[4] + red[5]) + (red[6] + red[7]));
        const float g = 1.0f / (1.0f + expf(-gl));
        const fv r = ((acc[0][lane] + acc[1][lane]) + (acc[2][lane] + acc[3][lane])) * inv * g;
#pragma unroll
        for (int v = 0; v < VPL; v++) {
            out[lane * VPL + v] = r[v];
            if (out16) out16[lane * VPL + v] = fw_bf16(r[v]);
        }
    }
}

template <int VPL>
__global__ __launch_bounds__(256) void fw_attn_combine_kernel(const float * part, const float * gate, const int * st,
                                                              int window, int nch_max, float * out, uint16_t * out16) {
    constexpr int hd = 64 * VPL;
    extern __shared__ float wts[];             /* per chunk: m_c, then e^(m_c - M); then l_c */
    const int pos = st[1];
    const int start = window > 0 && pos + 1 > window ? pos + 1 - window : 0;
    const int nch = (pos + 1 - start + kAttnChunk - 1) / kAttnChunk;
    const int h = blockIdx.x;
    attn_combine_head<VPL>(part + (size_t) h * nch_max * (hd + 2), nch, gate[h], out + (size_t) h * hd,
                           out16 ? out16 + (size_t) h * hd : nullptr, wts);
}

/* ---- a verify block: ntok <= 8 consecutive tokens at positions pos0 .. ----
 * (vq-model-gpu.cu:858-969 forward_batch + verify_logits). Each step of the
 * forward runs once for the whole block; token t attends causally to the
 * positions up to pos0 + t. Positions and tokens are kernel arguments: the
 * block path runs eagerly. */
struct FwTok8 {
    int t[8];
};

/* Embedding rows of a Q8_0 head for the block's tokens: column t = row tok[t]. */
__global__ void fw_q8_0_rows_kernel(const uint8_t * blocks, int cols, FwTok8 tok, float * out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (i >= cols) return;
    const uint8_t * b = blocks + ((size_t) tok.t[t] * (cols >> 5) + (i >> 5)) * 34;
    _Float16 d;
    __builtin_memcpy(&d, b, 2);
    out[(size_t) t * cols + i] = (float) d * (float) (int8_t) b[2 + (i & 31)];
}

/* Rope and the KV store for token t = blockIdx.x at position pos0 + t: pair
 * i's cos and sin computed once per token with the expressions of the decode
 * tables (model.rs:416-438, f32), then pair i of every q and k head rotated
 * in place, a rotated k pair stored to the cache too; v and the k elements
 * past pdim stored to the cache. pdim <= 256. */
__global__ __launch_bounds__(256) void fw_rope_kv_n_kernel(float * qkv, int ldq, int qd, int kvd, int heads,
                                                            int kv_heads, int hd, int pdim, float theta, int pos0,
                                                            float * kc, float * vc) {
    __shared__ float cs[2][128];
    const int half = pdim / 2, t = blockIdx.x, pos = pos0 + t, tid = threadIdx.x;
    float * row = qkv + (size_t) t * ldq;
    if (tid < half) {
        const float freq = 1.0f / powf(theta, (float) (2 * tid) / (float) pdim);
        const float a = (float) pos * freq;
        cs[0][tid] = cosf(a);
        cs[1][tid] = sinf(a);
    }
    __syncthreads();
    /* four items per thread at a time, every load issued before the stores
     * (which write the rows read) */
    constexpr int B = 4;
    const int nrot = (heads + kv_heads) * half;
    for (int j0 = tid; j0 < nrot; j0 += B * blockDim.x) {
        float x0[B], x1[B];
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int j = j0 + b * blockDim.x;
            if (j < nrot) {
                const int h = j / half, i = j - h * half;
                const float * base = h < heads ? row + (size_t) h * hd : row + qd + (size_t) (h - heads) * hd;
                x0[b] = base[i];
                x1[b] = base[i + half];
            }
        }
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int j = j0 + b * blockDim.x;
            if (j < nrot) {
                const int h = j / half, i = j - h * half;
                const float c = cs[0][i], sn = cs[1][i];
                float * base = h < heads ? row + (size_t) h * hd : row + qd + (size_t) (h - heads) * hd;
                const float r0 = x0[b] * c - x1[b] * sn, r1 = x1[b] * c + x0[b] * sn;
                base[i] = r0;
                base[i + half] = r1;
                if (h >= heads) {
                    float * k = kc + (size_t) pos * kvd + (size_t) (h - heads) * hd;
                    k[i] = r0;
                    k[i + half] = r1;
                }
            }
        }
    }
    for (int j0 = tid; j0 < kvd; j0 += B * blockDim.x) {
        float v[B], k[B];
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int j = j0 + b * blockDim.x;
            if (j < kvd) {
                v[b] = row[qd + kvd + j];
                k[b] = row[qd + j];
            }
        }
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int j = j0 + b * blockDim.x;
            if (j < kvd) {
                vc[(size_t) pos * kvd + j] = v[b];
                if (j % hd >= 2 * half) kc[(size_t) pos * kvd + j] = k[b];
            }
        }
    }
}

/* fw_rope_kv_n_kernel's work for up to kMaxCols tokens, spread over
 * N x (heads + kv_heads) workgroups: token t = blockIdx.x, head h =
 * blockIdx.y (query heads, then kv heads), thread i < pdim / 2 computing
 * pair i's cos and sin with the same expressions and rotating the head's
 * pair in place; a kv head's rotated pair, its elements past pdim and its v
 * go to the cache too. One load, rotation and store per thread: an 8-token
 * verify block 3141-3145 -> 3061 us against fw_rope_kv_n_kernel's eight
 * workgroups looping over the heads (5.8 us per launch). Long chunks keep
 * fw_rope_kv_n_kernel: this shape (or head groups looped per workgroup)
 * made a 512-token chunk 100-260 us slower. blockDim.x = 128 >= pdim / 2. */
__global__ __launch_bounds__(128) void fw_rope_kv_heads_kernel(float * qkv, int ldq, int qd, int kvd, int heads,
                                                                int hd, int pdim, float theta, int pos0, float * kc,
                                                                float * vc) {
    const int half = pdim / 2, t = blockIdx.x, h = blockIdx.y, i = threadIdx.x, pos = pos0 + t;
    float * row = qkv + (size_t) t * ldq;
    const bool kv = h >= heads;
    const int kh = h - heads;
    float * base = kv ? row + qd + (size_t) kh * hd : row + (size_t) h * hd;
    float * kr = kv ? kc + (size_t) pos * kvd + (size_t) kh * hd : nullptr;
    if (kv) {
        /* elements past pdim and v (neither is written by the rotation) */
        const float * vr = row + qd + kvd + (size_t) kh * hd;
        float * vo = vc + (size_t) pos * kvd + (size_t) kh * hd;
        for (int e = i; e < hd; e += blockDim.x) {
            vo[e] = vr[e];
            if (e >= 2 * half) kr[e] = base[e];
        }
    }
    if (i < half) {
        const float freq = 1.0f / powf(theta, (float) (2 * i) / (float) pdim);
        const float a = (float) pos * freq;
        const float c = cosf(a), sn = sinf(a);
        const float x0 = base[i], x1 = base[i + half];
        const float r0 = x0 * c - x1 * sn, r1 = x1 * c + x0 * sn;
        base[i] = r0;
        base[i + half] = r1;
        if (kv) {
            kr[i] = r0;
            kr[i + half] = r1;
        }
    }
}

/* Attention partials of token t = blockIdx.z (query rotated in qkv, every
 * key in the cache), as fw_attn_part_kernel otherwise. */
template <int VPL>
__global__ __launch_bounds__(256) void fw_attn_part_n_kernel(const float * qkv, int ldq, int kvd, const float * kc,
                                                              const float * vc, int pos0, int window, int heads,
                                                              int kv_heads, float scale, int nch_max, float * part) {
    constexpr int hd = 64 * VPL, C = kAttnChunk;
    typedef float fv __attribute__((ext_vector_type(VPL)));
    const int t = blockIdx.z, pos = pos0 + t;
    const int start = window > 0 && pos + 1 > window ? pos + 1 - window : 0;
    const int n = pos + 1 - start;
    const int chunk = blockIdx.x, kvh = blockIdx.y;
    const int G = heads / kv_heads;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j0 = chunk * C;
    if (j0 >= n) return;
    const int jn = min(C, n - j0);
    const int h = kvh * G + wave;
    const fv q = *(const fv *) (qkv + (size_t) t * ldq + (size_t) h * hd + lane * VPL);
    const float * kb = kc + (size_t) (start + j0) * kvd + (size_t) kvh * hd + lane * VPL;
    const float * vb = vc + (size_t) (start + j0) * kvd + (size_t) kvh * hd + lane * VPL;
    fv kr[C], vr[C];
#pragma unroll
    for (int j = 0; j < C; j++) kr[j] = *(const fv *) (kb + (size_t) min(j, jn - 1) * kvd);
#pragma unroll
    for (int j = 0; j < C; j++) vr[j] = *(const fv *) (vb + (size_t) min(j, jn - 1) * kvd);
    float sc[C];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < C; j++) {
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < VPL; v++) s += q[v] * kr[j][v];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        sc[j] = s * scale;
        if (j < jn) m = fmaxf(m, sc[j]);
    }
    float l = 0.0f;
    fv o = (fv) 0.0f;
#pragma unroll
    for (int j = 0; j < C; j++) {
        /* rows past jn are padding that may hold anything (the row at pos
         * before its store): skipped, not weighted by zero */
        if (j < jn) {
            const float e = expf(sc[j] - m);
            l += e;
            o += e * vr[j];
        }
    }
    float * P = part + (((size_t) t * heads + h) * nch_max + chunk) * (hd + 2);
    *(fv *) (P + lane * VPL) = o;
    if (lane == 0) {
        P[hd] = m;
        P[hd + 1] = l;
    }
}

/* The combine of token t = blockIdx.y: gates at gate + t * ldg, output row t. */
template <int VPL>
__global__ __launch_bounds__(256) void fw_attn_combine_n_kernel(const float * part, const float * gate, int ldg,
                                                                int pos0, int window, int heads, int nch_max,
                                                                float * out, uint16_t * out16) {
    constexpr int hd = 64 * VPL;
    extern __shared__ float wts[];
    const int t = blockIdx.y, pos = pos0 + t;
    const int start = window > 0 && pos + 1 > window ? pos + 1 - window : 0;
    const int nch = (pos + 1 - start + kAttnChunk - 1) / kAttnChunk;
    const int h = blockIdx.x;
    const size_t ob = (size_t) t * heads * hd + (size_t) h * hd;
    attn_combine_head<VPL>(part + ((size_t) t * heads + h) * nch_max * (hd + 2), nch, gate[(size_t) t * ldg + h],
                           out + ob, out16 ? out16 + ob : nullptr, wts);
}

/* act = gelu(g) * u with torch's exact gelu, erf in f64 as model.rs:253-258
 * calls it. */
__global__ void fw_gelu_mul_kernel(const float * g, const float * u, float * act, uint16_t * act16, int n) {
    /* four elements per thread through 16-byte loads (g, u and act 16-byte
     * aligned, act16 8-byte aligned: the callers' buffers), the tail apart;
     * act null: only act16 is written (the bf16 model reads nothing else) */
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef uint16_t u4v __attribute__((ext_vector_type(4)));
    const int n4 = n / 4;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += blockDim.x * gridDim.x) {
        const f4v a = ((const f4v *) g)[i], b = ((const f4v *) u)[i];
        f4v r;
        u4v r16;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            r[k] = gelu_mul(a[k], b[k]);
            r16[k] = fw_bf16(r[k]);
        }
        if (act) ((f4v *) act)[i] = r;
        if (act16) ((u4v *) act16)[i] = r16;
    }
    const int i = 4 * n4 + blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float r = gelu_mul(g[i], u[i]);
        if (act) act[i] = r;
        if (act16) act16[i] = fw_bf16(r);
    }
}

/* Layer-input capture: rows h[0 .. n) into slot rows pos .. pos + n - 1,
 * the position read from st[1] when st is given (a replayed graph) */
__global__ void fw_capture_kernel(const float * h, float * slot, const int * st, int pos, int n, int hidden) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (i >= hidden || t >= n) return;
    const int p = (st ? st[1] : pos) + t;
    slot[(size_t) p * hidden + i] = h[(size_t) t * hidden + i];
}

/* The index of the largest value (Model::argmax, model.rs:594-605): the
 * first of equal maxima, NaN never chosen, 0 when nothing beats -inf. One
 * workgroup of 1024 threads: each scans a stride, then a tree keeps the
 * larger value or, on a tie, the lower index. */
__global__ __launch_bounds__(1024) void fw_argmax_kernel(const float * v, int n, int * out) {
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const int t = threadIdx.x;
    float best = -INFINITY;
    int b = -1;
    for (int i = t; i < n; i += 1024) {
        const float x = v[i];
        if (x > best) { best = x; b = i; }
    }
    bv[t] = best;
    bi[t] = b;
    __syncthreads();
    for (int off = 512; off > 0; off >>= 1) {
        if (t < off) {
            const float o = bv[t + off];
            const int oi = bi[t + off];
            if (oi >= 0 && (bi[t] < 0 || o > bv[t] || (o == bv[t] && oi < bi[t]))) { bv[t] = o; bi[t] = oi; }
        }
        __syncthreads();
    }
    if (t == 0) out[0] = bi[0] < 0 ? 0 : bi[0];
}

/* ---- a prompt chunk: up to kPromptMax consecutive tokens at pos0 .. ----
 * (vq-model-gpu.cu:858-943 forward_batch). The steps are the verify
 * block's; the tokens come from device memory, and attention runs without
 * per-chunk partials (whose buffer grows with tokens x context). */
constexpr int kPromptMax = 512;

/* Embedding rows of a Q8_0 head: column t = row tok[t] (device). */
__global__ void fw_q8_0_rows_dev_kernel(const uint8_t * blocks, int cols, const int * tok, float * out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (i >= cols) return;
    const uint8_t * b = blocks + ((size_t) tok[t] * (cols >> 5) + (i >> 5)) * 34;
    _Float16 d;
    __builtin_memcpy(&d, b, 2);
    out[(size_t) t * cols + i] = (float) d * (float) (int8_t) b[2 + (i & 31)];
}

/* Attention of token t = blockIdx.y (query rotated in qkv, every key of its
 * window in the cache) for the query heads of kv head blockIdx.x, one wave
 * per query head: the window in chunks of kAttnChunk positions with a
 * running maximum m, sum l and output o (each chunk's terms scaled to the
 * new maximum, the old ones by e^(m_old - m_new)), then o / l times the
 * head's sigmoid gate. The same softmax as the CPU's (model.rs:520-557),
 * summed chunk by chunk in position order. */
template <int VPL>
__global__ __launch_bounds__(256) void fw_attn_prompt_kernel(const float * qkv, int ldq, int kvd, const float * kc,
                                                              const float * vc, const float * gate, int ldg, int pos0,
                                                              int window, int heads, int kv_heads, float scale,
                                                              float * out, uint16_t * out16) {
    constexpr int hd = 64 * VPL, C = kAttnChunk;
    typedef float fv __attribute__((ext_vector_type(VPL)));
    const int t = blockIdx.y, pos = pos0 + t;
    const int start = window > 0 && pos + 1 > window ? pos + 1 - window : 0;
    const int n = pos + 1 - start;
    const int kvh = blockIdx.x, G = heads / kv_heads;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = kvh * G + wave;
    const fv q = *(const fv *) (qkv + (size_t) t * ldq + (size_t) h * hd + lane * VPL);
    const float * kb = kc + (size_t) start * kvd + (size_t) kvh * hd + lane * VPL;
    const float * vb = vc + (size_t) start * kvd + (size_t) kvh * hd + lane * VPL;
    float m = -INFINITY, l = 0.0f;
    fv o = (fv) 0.0f;
    for (int j0 = 0; j0 < n; j0 += C) {
        const int jn = min(C, n - j0);
        fv kr[C], vr[C];
#pragma unroll
        for (int j = 0; j < C; j++) kr[j] = *(const fv *) (kb + (size_t) (j0 + min(j, jn - 1)) * kvd);
#pragma unroll
        for (int j = 0; j < C; j++) vr[j] = *(const fv *) (vb + (size_t) (j0 + min(j, jn - 1)) * kvd);
        float sc[C];
        float mc = -INFINITY;
#pragma unroll
        for (int j = 0; j < C; j++) {
            float sv = 0.0f;
#pragma unroll
            for (int v = 0; v < VPL; v++) sv += q[v] * kr[j][v];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) sv += __shfl_xor(sv, off, 64);
            sc[j] = sv * scale;
            if (j < jn) mc = fmaxf(mc, sc[j]);
        }
        const float mn = fmaxf(m, mc);
        const float a = expf(m - mn);          /* 0 on the first chunk (m = -inf) */
        l *= a;
        o *= a;
#pragma unroll
        for (int j = 0; j < C; j++) {
            /* rows past jn are padding that may hold anything (the row at pos
             * before its store): skipped, not weighted by zero */
            if (j < jn) {
                const float e = expf(sc[j] - mn);
                l += e;
                o += e * vr[j];
            }
        }
        m = mn;
    }
    const float g = 1.0f / (1.0f + expf(-gate[(size_t) t * ldg + h]));
    const fv r = o * (1.0f / l) * g;
    const size_t ob = (size_t) t * heads * hd + (size_t) h * hd + lane * VPL;
#pragma unroll
    for (int v = 0; v < VPL; v++) {
        out[ob + v] = r[v];
        if (out16) out16[ob + v] = fw_bf16(r[v]);
    }
}

/* The same prompt attention on the f32 matrix cores, for 256-element heads
 * (the reference model's): one workgroup per (query head, 16 query tokens),
 * the grid ordered so that the blocks with the longest causal range start
 * first. The block's positions are cut into tiles of 16; wave w of the 4
 * takes tiles w, w + 4, w + 8, ..., with its own running maximum, sum and
 * output, merged at the end. No wave reads another's K or V rows, so a wave
 * loads them from global memory straight into the MFMA operand layout, with
 * no LDS staging and no barrier in the loop: V of a tile is requested before
 * the tile's scores are formed and K of the next tile right after, so both
 * arrive while MFMAs run. Per tile a wave forms the 16 x 16 scores
 * S^T = K Q^T (positions x tokens) with 64 v_mfma_f32_16x16x4f32 (four
 * accumulators, so consecutive MFMAs do not wait for each other), masks
 * positions outside each token's window (causal, and the sliding window),
 * weights them by exp(score - m) for a per-token reference m, and adds
 * O^T += V^T P^T with 64 more. Unlike the kernel above, m is not the running
 * maximum itself: it moves (the sums and outputs rescaled) only when a score
 * passes it by more than kPaLag, which keeps every weight below e^8 and
 * spares most tiles the exchange between lanes and the rescale. The quotient
 * of outputs and sums does not depend on m; products and sums stay in f32,
 * and only the rounding and the order of the additions differ from the
 * kernel above.
 *
 * Operand layouts (lane l = 16 g + c): an A operand is A[l % 16][l / 16]
 * (16 x 4), a B operand B[l / 16][l % 16] (4 x 16), and the 16 x 16 result
 * sits as D[4 (l / 16) + i][l % 16], i < 4. Which head element a (k-step,
 * lane group) pair contracts over is free as long as both operands agree:
 * lane (g, c) feeds K[c][pa_k(ks, g)] and Q[c][pa_k(ks, g)] at k-step ks:
 * it reads its K row as 16 runs of 4 floats, the 4 lane groups of a row
 * together 64 contiguous bytes (a load instruction touches 16 cache lines,
 * not 64), and holds the scores of token c at positions 4 g + i. For O^T, k-step ks takes positions 4 g + ks: the B
 * value is the lane's own probability i = ks, and the A value is
 * V[4 g + ks][d], with the rows of O^T permuted (pa_d) so that d too runs in
 * groups of 4: the 16 lanes of a group read 256 contiguous bytes of a row. */
constexpr int kPaTok = 16;     /* query tokens per workgroup */
constexpr float kPaLag = 8.0f; /* how far a score may pass the reference maximum */

/* head element contracted at k-step ks by lane group g in S^T = K Q^T */
static __device__ __forceinline__ int pa_k(int ks, int g) { return 16 * (ks >> 2) + 4 * g + (ks & 3); }
/* head element of row R of O^T block b */
static __device__ __forceinline__ int pa_d(int b, int R) { return 64 * (b >> 2) + 4 * R + (b & 3); }

__global__ __launch_bounds__(256) void fw_attn_prompt_mfma_kernel(const float * qkv, int ldq, int kvd,
                                                                   const float * kc, const float * vc,
                                                                   const float * gate, int ldg, int pos0, int N,
                                                                   int window, int heads, int kv_heads, float scale,
                                                                   float * out, uint16_t * out16) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    /* the merge after the loop: outputs handed between waves, 3 x 4 blocks
     * of 64 x 4 floats per wave, and the maximum and sum per token of each;
     * before the loop the block's Q rows pass through the first part */
    __shared__ f4v lds_o[48 * 64];
    __shared__ float lds_s[4 * 32];
    const int h = blockIdx.x, t0 = ((int) gridDim.y - 1 - (int) blockIdx.y) * kPaTok;
    const int kvh = h / (heads / kv_heads);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
    /* this lane's token (column c); tokens past N compute a copy of the last
     * one and store nothing */
    const int tv = min(t0 + c, N - 1), pos_t = pos0 + tv;
    const int start_t = window > 0 && pos_t + 1 > window ? pos_t + 1 - window : 0;
    /* the block's positions: from the first token's window start to the last token */
    const int tl = min(t0 + kPaTok - 1, N - 1);
    const int pfirst = window > 0 && pos0 + t0 + 1 > window ? pos0 + t0 + 1 - window : 0;
    const int plast = pos0 + tl;
    /* the gate, requested first: it is needed at the end */
    const float gate_t = gate[(size_t) tv * ldg + h];
    /* Q^T as the B operand: Q[c][pa_k(ks, g)], ks < 64. The block's 16 Q rows
     * are read once per workgroup into LDS (rows of 65 x 4 floats, so the 16
     * rows of a lane group fall on distinct banks), in the space the merge
     * uses after the loop */
    float qv[64];
    {
        f4v * lds_q = lds_o;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = tid + 256 * k, tk = i >> 6, c4 = i & 63;
            lds_q[tk * 65 + c4] = *(const f4v *) (qkv + (size_t) min(t0 + tk, N - 1) * ldq + (size_t) h * 256 + 4 * c4);
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < 64; ks += 4) {
            const f4v q4 = lds_q[c * 65 + pa_k(ks, g) / 4];
            qv[ks] = q4[0];
            qv[ks + 1] = q4[1];
            qv[ks + 2] = q4[2];
            qv[ks + 3] = q4[3];
        }
        __syncthreads();   /* every wave holds its Q before any writes the merge */
    }
    f4v o[16];
#pragma unroll
    for (int db = 0; db < 16; db++) o[db] = f4v{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    const float * kbase = kc + (size_t) kvh * 256;
    const float * vbase = vc + (size_t) kvh * 256;
    /* K rows pw + c and V rows pw + 4 g + ks of the tile at pw; rows past
     * plast repeat it and are masked. Each is requested for the next tile as
     * soon as this tile's MFMAs have read it, so it has most of a tile's time
     * to arrive. The requests are unconditional (past the last tile they all
     * read row plast again): behind a branch, the waits for this tile's V
     * would also cover the next tile's K */
    f4v kf[16], vf[16];
    auto fetch_k = [&](int pw) {
        const float * kp = kbase + (size_t) min(pw + c, plast) * kvd;
#pragma unroll
        for (int j = 0; j < 16; j++) kf[j] = *(const f4v *) (kp + pa_k(4 * j, g));
    };
    auto fetch_v = [&](int pw) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const float * vp = vbase + (size_t) min(pw + 4 * g + ks, plast) * kvd + 4 * c;
#pragma unroll
            for (int q = 0; q < 4; q++) vf[4 * ks + q] = *(const f4v *) (vp + 64 * q);
        }
    };
    const int pbeg = (pfirst & ~15) + 16 * wave;
    /* Q, then K, then V, in the order the loop waits for them */
    __builtin_amdgcn_sched_barrier(0);
    fetch_k(pbeg);
    __builtin_amdgcn_sched_barrier(0);
    fetch_v(pbeg);
    __builtin_amdgcn_sched_barrier(0);
    for (int pw = pbeg; pw <= plast; pw += 64) {
        /* S^T = K Q^T */
        f4v s0 = f4v{0.f, 0.f, 0.f, 0.f}, s1 = s0, s2 = s0, s3 = s0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j][0], qv[4 * j], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j][1], qv[4 * j + 1], s1, 0, 0, 0);
            s2 = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j][2], qv[4 * j + 2], s2, 0, 0, 0);
            s3 = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j][3], qv[4 * j + 3], s3, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        fetch_k(pw + 64);
        __builtin_amdgcn_sched_barrier(0);
        const f4v s = (s0 + s1) + (s2 + s3);
        /* scale and mask: position pw + 4 g + i for token c */
        float e[4];
        float mc = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int pp = pw + 4 * g + i;
            const bool ok = pp >= start_t && pp <= pos_t;
            e[i] = ok ? s[i] * scale : -INFINITY;
            mc = fmaxf(mc, e[i]);
        }
        /* the weights are exp(score - m) for a reference m per token that
         * moves only when a score passes it by more than kPaLag (then to the
         * token's maximum so far, the sum and outputs rescaled): the weights
         * stay below e^kPaLag, and most tiles need neither an exchange
         * between lanes nor a rescale */
        if (__any(mc > m + kPaLag)) {   /* uniform */
            mc = fmaxf(mc, __shfl_xor(mc, 16, 64));
            mc = fmaxf(mc, __shfl_xor(mc, 32, 64));
            const float mn = fmaxf(m, mc);
            /* nothing seen yet for this token: no rescale */
            const float a = mn == -INFINITY ? 1.0f : expf(m - mn);
            l *= a;
#pragma unroll
            for (int db = 0; db < 16; db++) o[db] *= a;
            m = mn;
        }
        /* l holds this lane's share of the sum (its 4 positions), reduced
         * over the lane groups after the loop */
#pragma unroll
        for (int i = 0; i < 4; i++) {
            e[i] = e[i] == -INFINITY ? 0.0f : expf(e[i] - m);
            l += e[i];
        }
        /* O^T += V^T P^T; row c of block db is element pa_d(db, c) */
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    o[4 * q + r] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[4 * ks + q][r], e[ks], o[4 * q + r], 0, 0,
                                                                        0);
        __builtin_amdgcn_sched_barrier(0);
        fetch_v(pw + 64);
        __builtin_amdgcn_sched_barrier(0);
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    /* merge: wave w finishes head elements 64 w .. 64 w + 63 (blocks
     * 4 w .. 4 w + 3 of O^T) of the 16 tokens. The other waves hand it their
     * outputs for those blocks through LDS in their register layout, a slot
     * of 64 x 4 floats per (source wave, owner, block), owners' own blocks
     * not stored; every wave hands over its maximum and sum per token */
#pragma unroll
    for (int w = 0; w < 4; w++) {
        if (w == wave) continue;   /* uniform */
        const int k = (w - wave + 3) & 3;   /* 0 .. 2: the owner's index among the others */
#pragma unroll
        for (int b = 0; b < 4; b++) lds_o[((wave * 3 + k) * 4 + b) * 64 + lane] = o[4 * w + b];
    }
    if (g == 0) {
        lds_s[wave * 32 + c] = m;
        lds_s[wave * 32 + 16 + c] = l;
    }
    __syncthreads();
    float mw[4], aw[4];
#pragma unroll
    for (int w = 0; w < 4; w++) mw[w] = lds_s[w * 32 + c];
    const float mt = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
    float lt = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        aw[w] = mw[w] == -INFINITY ? 0.0f : expf(mw[w] - mt);
        lt += lds_s[w * 32 + 16 + c] * aw[w];
    }
    /* sum over the source waves in wave order, this wave's own blocks from
     * its registers */
    f4v v[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            f4v x;
            if (w == wave) {   /* uniform */
                x = o[4 * w + b];
            } else {
                const int k = (wave - w + 3) & 3;
                x = lds_o[((w * 3 + k) * 4 + b) * 64 + lane];
            }
            v[b] = w == 0 ? x * aw[0] : v[b] + x * aw[w];
        }
    }
    if (t0 + c >= N) return;
    const float gs = 1.0f / (1.0f + expf(-gate_t));
    const float inv = 1.0f / lt;
    /* element pa_d(4 wave + b, 4 g + i) = 64 wave + 16 g + 4 i + b: four
     * consecutive elements per i */
    const size_t ob = (size_t) tv * heads * 256 + (size_t) h * 256 + 64 * wave + 16 * g;
    /* the bf16 copy when one is asked for (the next matvec reads only it),
     * else the f32 output */
    f4v r[4];
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = f4v{v[0][i], v[1][i], v[2][i], v[3][i]} * inv * gs;
    if (out16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint2 p;
            p.x = (uint32_t) fw_bf16(r[i][0]) | ((uint32_t) fw_bf16(r[i][1]) << 16);
            p.y = (uint32_t) fw_bf16(r[i][2]) | ((uint32_t) fw_bf16(r[i][3]) << 16);
            *(uint2 *) (out16 + ob + 4 * i) = p;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) *(f4v *) (out + ob + 4 * i) = r[i];
    }
}

/* ------------------------------------------------------------------ host -- */

namespace {

struct Model {
    sparkmv_model_cfg c;
    std::vector<sparkmv_model_layer> layers;
    std::vector<int> layer_set;
    int head_kind = -1;                  /* 0 VQ container, 8 Q8_0 blocks */
    const void * head_stages[4] = {nullptr, nullptr, nullptr, nullptr};
    const void * head_blocks = nullptr;
    const float * final_norm = nullptr;
    /* device memory, one allocation */
    void * mem = nullptr;
    float * h, * xn, * qkv, * g, * attn, * mg, * mu, * act, * kv;
    uint16_t * xn16, * attn16, * act16;
    uint64_t * pslot;                    /* the gate/up launches' exchange, intermediate * kMaxCols words, kept zero */
    /* exchange words of the several-column launches over hidden rows (the
     * chunk-split tiles' tree), kept zero; the launches share them, one at
     * a time on the model's stream */
    uint64_t * kslot;
    long kslot_cap;
    /* gelu * up written by the gate/up launch (1), or by the activation
     * kernel (0: SPARKMV_SEPARATE_ACT=1 at creation; the same bits, slower) */
    int fuse_act = 1;
    int * st;                            /* token, position */
    float * part;                        /* attention partials [heads][nch_max][head_dim + 2] */
    float * rtab;                        /* rope tables [full, sliding][cos, sin][128] */
    int nch_max;
    /* the recorded chain */
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    /* cached positions (model.rs:453, :361-381) */
    int len = 0;
    /* tuned kernels per (rows, cols) of a VQ matvec: variant, threads */
    std::map<std::pair<int, int>, std::pair<int, int>> picks;
    /* device memory the model frees at destroy: weights a loader uploaded */
    std::vector<void *> owned;
    /* block buffers (verify blocks and prompt chunks), one allocation at
     * sparkmv_model_reserve or the first block: vcap columns of each
     * activation, gate rows at the qkv stride, the tokens, and attention
     * partials for verify blocks of up to 8 tokens */
    void * vmem = nullptr;
    int vcap = 0;
    float * vh, * vxn, * vqkv, * vg, * vattn, * vmg, * vmu, * vact, * vpart;
    uint16_t * vxn16, * vattn16, * vact16;
    int * vtok;
    /* layer-input capture (model.rs:322-348, vq-model-gpu.cu:632-639):
     * cap_slot[li] is layer li's slot or -1; cap is [cap_n][max_ctx][hidden] */
    std::vector<int> cap_slot;
    int cap_n = 0;
    float * cap = nullptr;
};

size_t align256(size_t b) { return (b + 255) & ~(size_t) 255; }

/* the rotated prefix of a head: (head_dim * partial) as usize, at most head_dim (model.rs:419) */
int rope_dim(int hd, double partial) {
    const int d = (int) ((float) hd * (float) partial);
    return d > hd ? hd : d;
}

int check_launch(const char * what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip(what, e);
}

int gemv(const Model & m, const void * const * st, int rows, int cols, const void * x, float * y, int acc,
         hipStream_t s, int ncol = 1, int ldy = 0) {
    VqMatDesc d;
    memset(&d, 0, sizeof d);
    for (int i = 0; i < m.c.nstages; i++) d.stages[i] = st[i];
    d.y = y;
    d.rows = rows;
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = m.c.dim; c.nc = m.c.nc; c.cols = cols; c.v3 = m.c.v3; c.nst = m.c.nstages;
    c.mats = &d; c.nmat = 1;
    c.x = x; c.ldx = cols; c.xf32 = m.c.x_dtype == SPARKMV_X_F32; c.ncol = ncol; c.ldy = ldy ? ldy : rows;
    c.accumulate = acc; c.stream = s;
    if (ncol > 1) {
        c.kslot = m.kslot;
        c.kslot_cap = m.kslot_cap;
    }
    const auto it = m.picks.find({rows, cols});
    if (it != m.picks.end()) { c.variant = it->second.first; c.threads = it->second.second; }
    return vq_launch(c);
}

int gemv2(const Model & m, const void * const * st0, int rows0, float * y0, const void * const * st1, int rows1,
          float * y1, int cols, const void * x, hipStream_t s, int ncol = 1, int ldy = 0) {
    VqMatDesc d[2];
    memset(d, 0, sizeof d);
    for (int i = 0; i < m.c.nstages; i++) { d[0].stages[i] = st0[i]; d[1].stages[i] = st1[i]; }
    d[0].y = y0; d[0].rows = rows0;
    d[1].y = y1; d[1].rows = rows1;
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = m.c.dim; c.nc = m.c.nc; c.cols = cols; c.v3 = m.c.v3; c.nst = m.c.nstages;
    c.mats = d; c.nmat = 2;
    c.x = x; c.ldx = cols; c.xf32 = m.c.x_dtype == SPARKMV_X_F32; c.ncol = ncol; c.ldy = ldy ? ldy : rows0;
    c.accumulate = 0; c.stream = s;
    /* two matrices in one launch take a tuned kernel when both are tuned alike */
    const auto a = m.picks.find({rows0, cols}), b = m.picks.find({rows1, cols});
    if (a != m.picks.end() && b != m.picks.end() && a->second == b->second) {
        c.variant = a->second.first;
        c.threads = a->second.second;
    }
    return vq_launch(c);
}

/* rms_norm(h) * w into the bf16 activations, then the two matrices over
 * them: with bf16 activations and untuned kernels, ONE launch whose
 * workgroups stage the norm of h themselves (vq_norm_launch); otherwise the
 * norm launch and gemv2. */
int rmsnorm(const Model & m, const float * x, const float * w, hipStream_t s, int ncol = 1, float * out = nullptr,
            uint16_t * out16 = nullptr);

/* gate and up over the N columns of x (bf16 or f32 [N][cols]) into mg / mu
 * [N][rows], then act / act16 = gelu(gate) * up: written by the gate/up
 * launch itself where the several-column kernel takes the shape (bf16
 * activations, no tuning profile, the activation not switched apart), else
 * by the activation kernel. */
int gate_up_act_n(const Model & m, const void * const * gate, const void * const * up, int rows, int cols,
                  const void * x, float * mg, float * mu, float * act, uint16_t * act16, hipStream_t s, int N) {
    const bool b16 = m.c.x_dtype == SPARKMV_X_BF16;
    if (b16 && m.fuse_act && m.picks.empty()) {
        VqMatDesc d[2];
        memset(d, 0, sizeof d);
        for (int i = 0; i < m.c.nstages; i++) { d[0].stages[i] = gate[i]; d[1].stages[i] = up[i]; }
        d[0].y = mg; d[0].rows = rows;
        d[1].y = mu; d[1].rows = rows;
        VqCall c;
        memset(&c, 0, sizeof c);
        c.dim = m.c.dim; c.nc = m.c.nc; c.cols = cols; c.v3 = m.c.v3; c.nst = m.c.nstages;
        c.mats = d; c.nmat = 2;
        c.x = x; c.ldx = cols; c.xf32 = 0; c.ncol = N; c.ldy = rows;
        c.accumulate = 0; c.stream = s;
        const VqPair pair{m.pslot, rows * kMaxCols, act, act16};
        const int rc = vq_pair_launch(c, pair);
        if (rc <= 0) return rc;
    }
    if (gemv2(m, gate, rows, mg, up, rows, mu, cols, x, s, N, rows)) return -1;
    hipLaunchKernelGGL(fw_gelu_mul_kernel, dim3((N * rows / 4 + 255) / 256 + 1), dim3(256), 0, s, mg, mu, act, act16,
                       N * rows);
    return check_launch("gelu launch");
}

int norm_gemv2(const Model & m, const float * h, const float * w, const void * const * st0, int rows0, float * y0,
               const void * const * st1, int rows1, float * y1, int cols, hipStream_t s, const VqPair * pair = nullptr,
               bool * act_done = nullptr) {
    const bool b16 = m.c.x_dtype == SPARKMV_X_BF16;
    if (act_done) *act_done = false;
    VqMatDesc d[2];
    memset(d, 0, sizeof d);
    for (int i = 0; i < m.c.nstages; i++) { d[0].stages[i] = st0[i]; d[1].stages[i] = st1[i]; }
    d[0].y = y0; d[0].rows = rows0;
    d[1].y = y1; d[1].rows = rows1;
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = m.c.dim; c.nc = m.c.nc; c.cols = cols; c.v3 = m.c.v3; c.nst = m.c.nstages;
    c.mats = d; c.nmat = 2;
    c.ncol = 1; c.ldy = rows0;
    c.accumulate = 0; c.stream = s;
    if (b16 && m.picks.empty()) {
        c.x = h; c.ldx = cols; c.xf32 = 1;
        if (pair) {
            /* one launch for the norm, both matrices and the activation */
            const int rc = vq_norm_launch(c, w, m.c.eps, nullptr, pair);
            if (rc <= 0) {
                if (rc == 0 && act_done) *act_done = true;
                return rc;
            }
        }
        const int rc = vq_norm_launch(c, w, m.c.eps, nullptr);
        if (rc <= 0) return rc;
    }
    if (rmsnorm(m, h, w, s, 1, nullptr, nullptr)) return -1;
    if (pair && b16 && m.picks.empty()) {
        c.x = m.xn16; c.ldx = cols; c.xf32 = 0;
        const int rc = vq_pair_launch(c, *pair);
        if (rc <= 0) {
            if (rc == 0 && act_done) *act_done = true;
            return rc;
        }
    }
    return gemv2(m, st0, rows0, y0, st1, rows1, y1, cols, b16 ? (const void *) m.xn16 : (const void *) m.xn, s);
}

int rmsnorm(const Model & m, const float * x, const float * w, hipStream_t s, int ncol, float * out,
            uint16_t * out16) {
    const bool b16 = m.c.x_dtype == SPARKMV_X_BF16;
    const int per = (m.c.hidden + 255) / 256;
    float * o = out ? out : m.xn;
    uint16_t * o16 = b16 ? (out16 ? out16 : m.xn16) : nullptr;
    const dim3 g((unsigned) ncol);
    if (per <= 4) hipLaunchKernelGGL(fw_rmsnorm_kernel<4>, g, dim3(256), 0, s, x, w, o, o16, m.c.hidden, m.c.eps);
    else if (per <= 12) hipLaunchKernelGGL(fw_rmsnorm_kernel<12>, g, dim3(256), 0, s, x, w, o, o16, m.c.hidden, m.c.eps);
    else if (per <= 32) hipLaunchKernelGGL(fw_rmsnorm_kernel<32>, g, dim3(256), 0, s, x, w, o, o16, m.c.hidden, m.c.eps);
    else { set_error("hidden %d is above 8192", m.c.hidden); return -1; }
    return check_launch("rms norm launch");
}

}  // namespace

}  // namespace sparkmv

using namespace sparkmv;

extern "C" {

void * sparkmv_model_create(const sparkmv_model_cfg * cfg) {
    if (!cfg) { set_error("model config is null"); return nullptr; }
    const sparkmv_model_cfg & c = *cfg;
    if (c.hidden <= 0 || c.layers <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.head_dim <= 0 || c.intermediate <= 0 ||
        c.vocab <= 0 || c.max_ctx <= 0 || c.sliding_window <= 0) {
        set_error("model config has a non-positive size");
        return nullptr;
    }
    if (c.heads % c.kv_heads) { set_error("heads %d is not a multiple of kv_heads %d", c.heads, c.kv_heads); return nullptr; }
    if (c.head_dim % 2) { set_error("head_dim %d is odd", c.head_dim); return nullptr; }
    if (c.x_dtype != SPARKMV_X_F32 && c.x_dtype != SPARKMV_X_BF16) { set_error("unknown x dtype %d", c.x_dtype); return nullptr; }
    if (c.nstages < 1 || c.nstages > 4) { set_error("stage count %d is outside 1..4", c.nstages); return nullptr; }
    if (!(c.eps > 0.0f)) { set_error("eps must be positive"); return nullptr; }
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) {
        set_error("head_dim %d is not 64, 128 or 256", c.head_dim);
        return nullptr;
    }
    if (c.heads / c.kv_heads > 4) { set_error("more than 4 query heads per kv head"); return nullptr; }
    for (double partial : {c.rope_full_partial, c.rope_slide_partial}) {
        const int half = rope_dim(c.head_dim, partial) / 2;
        if (half % (c.head_dim / 64)) {
            set_error("rope half-width %d is not a multiple of head_dim / 64", half);
            return nullptr;
        }
    }
    /* the combine keeps two floats per position chunk in LDS */
    const long nch_max = ((long) c.max_ctx + kAttnChunk - 1) / kAttnChunk;
    if (nch_max * 8 > 65536) { set_error("max_ctx %d is above %d", c.max_ctx, 8192 * kAttnChunk); return nullptr; }
    if (c.hidden > 8192) { set_error("hidden %d is above 8192", c.hidden); return nullptr; }
    Model * m = new Model;
    m->c = c;
    m->layers.resize(c.layers);
    m->layer_set.assign(c.layers, 0);
    m->cap_slot.assign(c.layers, -1);
    const size_t qd = (size_t) c.heads * c.head_dim, kvd = (size_t) c.kv_heads * c.head_dim;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += align256(bytes); return o; };
    const size_t o_h = take(c.hidden * 4), o_xn = take(c.hidden * 4), o_qkv = take((qd + 2 * kvd) * 4);
    const size_t o_g = take(c.heads * 4), o_attn = take(qd * 4), o_mg = take(c.intermediate * 4);
    const size_t o_mu = take(c.intermediate * 4), o_act = take(c.intermediate * 4);
    const size_t o_xn16 = take(c.hidden * 2), o_attn16 = take(qd * 2), o_act16 = take(c.intermediate * 2);
    const size_t o_kv = take((size_t) c.layers * c.max_ctx * kvd * 4 * 2);
    const size_t o_st = take(2 * sizeof(int));
    const size_t o_part = take((size_t) c.heads * nch_max * (c.head_dim + 2) * 4);
    const size_t o_rtab = take(512 * 4);
    const size_t n_pslot = (size_t) c.intermediate * kMaxCols;
    const size_t o_pslot = take(n_pslot * 8);
    const size_t n_kslot = (size_t) c.hidden * kMaxCols * vq_ck_words(kVqCkMaxGroups);
    const size_t o_kslot = take(n_kslot * 8);
    hipError_t e = hipMalloc(&m->mem, off);
    if (e != hipSuccess) {
        fail_hip("model buffers", e);
        delete m;
        return nullptr;
    }
    uint8_t * b = (uint8_t *) m->mem;
    e = hipMemset(b + o_pslot, 0, n_pslot * 8);
    if (e == hipSuccess) e = hipMemset(b + o_kslot, 0, n_kslot * 8);
    if (e != hipSuccess) {
        fail_hip("model exchange words", e);
        (void) hipFree(m->mem);
        delete m;
        return nullptr;
    }
    m->pslot = (uint64_t *) (b + o_pslot);
    m->kslot = (uint64_t *) (b + o_kslot);
    m->kslot_cap = (long) n_kslot;
    const char * sep = getenv("SPARKMV_SEPARATE_ACT");
    m->fuse_act = !(sep && sep[0] == '1');
    m->h = (float *) (b + o_h); m->xn = (float *) (b + o_xn); m->qkv = (float *) (b + o_qkv);
    m->g = (float *) (b + o_g); m->attn = (float *) (b + o_attn); m->mg = (float *) (b + o_mg);
    m->mu = (float *) (b + o_mu); m->act = (float *) (b + o_act);
    m->xn16 = (uint16_t *) (b + o_xn16); m->attn16 = (uint16_t *) (b + o_attn16); m->act16 = (uint16_t *) (b + o_act16);
    m->kv = (float *) (b + o_kv);
    m->st = (int *) (b + o_st);
    m->part = (float *) (b + o_part);
    m->rtab = (float *) (b + o_rtab);
    m->nch_max = (int) nch_max;
    return m;
}

void sparkmv_model_destroy(void * model) {
    Model * m = (Model *) model;
    if (!m) return;
    if (m->exec) (void) hipGraphExecDestroy(m->exec);
    if (m->graph) (void) hipGraphDestroy(m->graph);
    if (m->mem) (void) hipFree(m->mem);
    if (m->vmem) (void) hipFree(m->vmem);
    if (m->cap) (void) hipFree(m->cap);
    for (void * p : m->owned) (void) hipFree(p);
    delete m;
}

int sparkmv_model_set_layer(void * model, int li, const sparkmv_model_layer * L) {
    Model * m = (Model *) model;
    if (!m || !L) { set_error("model or layer is null"); return -1; }
    if (li < 0 || li >= m->c.layers) { set_error("layer %d is outside 0..%d", li, m->c.layers - 1); return -1; }
    if (!L->in_norm || !L->post_norm) { set_error("layer %d has a null norm", li); return -1; }
    const void * const * mats[6] = {L->qkv, L->attn_gate, L->out, L->gate, L->up, L->down};
    for (int k = 0; k < 6; k++)
        for (int s = 0; s < m->c.nstages; s++)
            if (!mats[k][s]) { set_error("layer %d matrix %d stage %d is null", li, k, s); return -1; }
    m->layers[li] = *L;
    m->layer_set[li] = 1;
    return 0;
}

int sparkmv_model_set_head(void * model, int kind, const void * const * stages, const void * blocks,
                           const float * final_norm) {
    Model * m = (Model *) model;
    if (!m || !final_norm) { set_error("model or final norm is null"); return -1; }
    if (kind == 0) {
        if (!stages) { set_error("VQ head without stages"); return -1; }
        for (int s = 0; s < m->c.nstages; s++) {
            if (!stages[s]) { set_error("VQ head stage %d is null", s); return -1; }
            m->head_stages[s] = stages[s];
        }
    } else if (kind == 8) {
        if (!blocks) { set_error("Q8_0 head without blocks"); return -1; }
        if (m->c.hidden % 32) { set_error("a Q8_0 head needs hidden %% 32 == 0"); return -1; }
        m->head_blocks = blocks;
    } else {
        set_error("head kind %d is neither 0 (VQ) nor 8 (Q8_0)", kind);
        return -1;
    }
    m->head_kind = kind;
    m->final_norm = final_norm;
    return 0;
}

}  // extern "C"

int sparkmv::model_adopt(void * model, void * dev_ptr) {
    Model * m = (Model *) model;
    if (!m || !dev_ptr) { set_error("model or pointer is null"); return -1; }
    m->owned.push_back(dev_ptr);
    return 0;
}

namespace {

/* Layer li's input rows into its capture slot (model.rs:466-471, before the
 * layer runs; vq-model-gpu.cu:888-895): n rows of h at pos (from st[1] when
 * st is given). */
int capture_rows(const Model & m, int li, const float * h, const int * st, int pos, int n, hipStream_t s) {
    if (!m.cap_n || m.cap_slot[(size_t) li] < 0) return 0;
    float * slot = m.cap + (size_t) m.cap_slot[(size_t) li] * m.c.max_ctx * m.c.hidden;
    hipLaunchKernelGGL(fw_capture_kernel, dim3((m.c.hidden + 255) / 256, n), dim3(256), 0, s, h, slot, st, pos, n,
                       m.c.hidden);
    return check_launch("capture launch");
}

int ready(const Model * m) {
    if (m->head_kind < 0) { set_error("the model has no head"); return -1; }
    for (int li = 0; li < m->c.layers; li++)
        if (!m->layer_set[li]) { set_error("layer %d has no weights", li); return -1; }
    return 0;
}

int check_step(const Model * m, uint32_t token, int pos) {
    if ((long) token >= m->c.vocab) { set_error("token %u is outside the vocabulary", token); return -1; }
    if (pos < 0 || pos >= m->c.max_ctx) { set_error("position %d exceeds the %d-token cache", pos, m->c.max_ctx); return -1; }
    return 0;
}

int set_state(Model * m, uint32_t token, int pos, hipStream_t s) {
    const sparkmv_model_cfg & c = m->c;
    hipLaunchKernelGGL(fw_set_state_kernel, dim3(1), dim3(128), 0, s, m->st, (int) token, pos,
                       (float) c.rope_full_theta, rope_dim(c.head_dim, c.rope_full_partial), (float) c.rope_slide_theta,
                       rope_dim(c.head_dim, c.rope_slide_partial), m->rtab);
    return check_launch("state launch");
}

/* Every launch of one token, reading token and position from m->st. */
int chain(Model * m, float * logits, hipStream_t s) {
    const sparkmv_model_cfg & c = m->c;
    const bool b16 = c.x_dtype == SPARKMV_X_BF16;
    const int qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, hd = c.head_dim;

    /* the embedding row (model.rs:462-464): the tied head's row `token` */
    if (m->head_kind == 0) {
        hipLaunchKernelGGL(fw_fill_kernel, dim3((c.hidden + 255) / 256), dim3(256), 0, s, m->h, c.hidden, 0.0f);
        if (check_launch("fill launch")) return -1;
        const Layout L = make_layout(c.dim, c.nc, c.vocab, c.hidden, c.v3);
        for (int st = 0; st < c.nstages; st++)
            if (vq_row_dequant_dev_launch(m->head_stages[st], L, m->st, m->h, s)) return -1;
    } else {
        hipLaunchKernelGGL(fw_q8_0_row_kernel, dim3((c.hidden + 255) / 256), dim3(256), 0, s,
                           (const uint8_t *) m->head_blocks, c.hidden, (const int *) m->st, m->h);
        if (check_launch("embedding launch")) return -1;
    }

    const float scale = 1.0f / sqrtf((float) hd);
    for (int li = 0; li < c.layers; li++) {
        const sparkmv_model_layer & L = m->layers[li];
        const bool full = L.full != 0;
        float * kc = m->kv + (size_t) li * 2 * c.max_ctx * kvd;
        float * vc = kc + (size_t) c.max_ctx * kvd;

        if (capture_rows(*m, li, m->h, m->st, 0, 1, s)) return -1;
        if (norm_gemv2(*m, m->h, L.in_norm, L.qkv, qd + 2 * kvd, m->qkv, L.attn_gate, c.heads, m->g, c.hidden, s))
            return -1;

        /* rope, the KV store and attention (model.rs:484-557), launched for
         * the longest window this layer can see */
        const int pdim = rope_dim(hd, full ? c.rope_full_partial : c.rope_slide_partial);
        const float * rtab = m->rtab + (full ? 0 : 256);
        const int window = full ? 0 : c.sliding_window;
        const int span = full || c.sliding_window > c.max_ctx ? c.max_ctx : c.sliding_window;
        const int nch = (span + kAttnChunk - 1) / kAttnChunk;
        const dim3 pg((unsigned) nch, (unsigned) c.kv_heads), pb((unsigned) (64 * (c.heads / c.kv_heads)));
        const uint32_t wl = (uint32_t) (nch * 8);
        uint16_t * a16 = b16 ? m->attn16 : nullptr;
#define FW_ATTN(V)                                                                                                  \
    do {                                                                                                            \
        hipLaunchKernelGGL(fw_attn_part_kernel<V>, pg, pb, 0, s, m->qkv, qd, kvd, kc, vc, (const int *) m->st,        \
                           window, c.heads, c.kv_heads, pdim, rtab, scale, m->nch_max, m->part);                    \
        hipLaunchKernelGGL(fw_attn_combine_kernel<V>, dim3(c.heads), dim3(256), wl, s, m->part, m->g,               \
                           (const int *) m->st, window, m->nch_max, m->attn, a16);                                  \
    } while (0)
        if (hd == 64) FW_ATTN(1);
        else if (hd == 128) FW_ATTN(2);
        else FW_ATTN(4);
#undef FW_ATTN
        if (check_launch("attention launch")) return -1;
        if (gemv(*m, L.out, c.hidden, qd, b16 ? (const void *) m->attn16 : (const void *) m->attn, m->h, 1, s))
            return -1;

        /* MLP (model.rs:566-581): the gate/up launch writes the activation
         * itself when its shape allows, else the activation kernel does */
        const VqPair pair{m->pslot, c.intermediate, m->act, b16 ? m->act16 : nullptr};
        bool act_done = false;
        if (norm_gemv2(*m, m->h, L.post_norm, L.gate, c.intermediate, m->mg, L.up, c.intermediate, m->mu, c.hidden, s,
                       m->fuse_act ? &pair : nullptr, &act_done))
            return -1;
        if (!act_done) {
            hipLaunchKernelGGL(fw_gelu_mul_kernel, dim3((c.intermediate / 4 + 255) / 256 + 1), dim3(256), 0, s, m->mg,
                               m->mu, m->act, b16 ? m->act16 : nullptr, c.intermediate);
            if (check_launch("gelu launch")) return -1;
        }
        if (gemv(*m, L.down, c.hidden, c.intermediate, b16 ? (const void *) m->act16 : (const void *) m->act, m->h,
                 1, s))
            return -1;
    }

    /* final norm and the tied head (model.rs:583-590) */
    if (rmsnorm(*m, m->h, m->final_norm, s)) return -1;
    const void * xin = b16 ? (const void *) m->xn16 : (const void *) m->xn;
    if (m->head_kind == 0) return gemv(*m, m->head_stages, c.vocab, c.hidden, xin, logits, 0, s);
    return kq_gemv_launch(8, m->head_blocks, c.vocab, c.hidden, xin, b16 ? 0 : 1, c.hidden, 1, logits, c.vocab, 0, s);
}

/* The block buffers for up to cap tokens (at least 8). A smaller or equal
 * reservation keeps what is there; a larger one replaces it (the caller
 * synchronizes first: work in flight may still use the old buffers). */
int alloc_block(Model * m, int cap) {
    cap = cap < 8 ? 8 : cap;
    if (m->vmem && cap <= m->vcap) return 0;
    const sparkmv_model_cfg & c = m->c;
    const size_t qd = (size_t) c.heads * c.head_dim, kvd = (size_t) c.kv_heads * c.head_dim, N = (size_t) cap;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += align256(bytes); return o; };
    const size_t o_h = take(N * c.hidden * 4), o_xn = take(N * c.hidden * 4), o_qkv = take(N * (qd + 2 * kvd) * 4);
    const size_t o_g = take(N * (qd + 2 * kvd) * 4), o_attn = take(N * qd * 4), o_mg = take(N * c.intermediate * 4);
    const size_t o_mu = take(N * c.intermediate * 4), o_act = take(N * c.intermediate * 4);
    const size_t o_xn16 = take(N * c.hidden * 2), o_attn16 = take(N * qd * 2), o_act16 = take(N * c.intermediate * 2);
    const size_t o_part = take((size_t) 8 * c.heads * (size_t) m->nch_max * (c.head_dim + 2) * 4);
    const size_t o_tok = take(N * sizeof(int));
    void * mem = nullptr;
    hipError_t e = hipMalloc(&mem, off);
    if (e != hipSuccess) return fail_hip("block buffers", e);
    if (m->vmem) (void) hipFree(m->vmem);
    m->vmem = mem;
    m->vcap = cap;
    uint8_t * b = (uint8_t *) m->vmem;
    m->vh = (float *) (b + o_h); m->vxn = (float *) (b + o_xn); m->vqkv = (float *) (b + o_qkv);
    m->vg = (float *) (b + o_g); m->vattn = (float *) (b + o_attn); m->vmg = (float *) (b + o_mg);
    m->vmu = (float *) (b + o_mu); m->vact = (float *) (b + o_act); m->vpart = (float *) (b + o_part);
    m->vxn16 = (uint16_t *) (b + o_xn16); m->vattn16 = (uint16_t *) (b + o_attn16);
    m->vact16 = (uint16_t *) (b + o_act16);
    m->vtok = (int *) (b + o_tok);
    return 0;
}

/* y[t * ldy + r] (+)= W x_t for N tokens of x ([N][cols], the model's x
 * dtype): up to kMaxCols tokens through the batched GEMV (each column the
 * decode arithmetic), more through the prefill GEMM (the reference's prompt
 * path, vq-model-gpu.cu:838-851: x enters the matrix cores as f16). */
int mat_n(const Model & m, const void * const * st, int rows, int cols, const void * x, float * y, int acc,
          hipStream_t s, int N, int ldy) {
    if (N <= kMaxCols) return gemv(m, st, rows, cols, x, y, acc, s, N, ldy);
    const Layout L = make_layout(m.c.dim, m.c.nc, rows, cols, m.c.v3);
    const int xf32 = m.c.x_dtype == SPARKMV_X_F32;
    if (m.c.nstages <= 2 && prefill_mfma_ready(L, m.c.nstages, x, xf32, cols, 0, N))
        return prefill_mfma_launch(st, m.c.nstages, L, x, xf32, cols, 0, N, y, ldy, acc, s);
    return prefill_simple_launch(st, m.c.nstages, L, x, xf32, (size_t) cols, 1, N, y, ldy, acc, s);
}

/* Rope and the KV store of N tokens at pos0 .. pos0 + N - 1 (rows of qkv at
 * stride ldq), the shape chosen by N. */
int rope_kv_launch(float * qkv, int N, int ldq, int qd, int kvd, int heads, int kv_heads, int hd, int pdim,
                          float theta, int pos0, float * kc, float * vc, hipStream_t s) {
    if (N <= kMaxCols)
        hipLaunchKernelGGL(fw_rope_kv_heads_kernel, dim3(N, heads + kv_heads), dim3(128), 0, s, qkv, ldq, qd, kvd,
                           heads, hd, pdim, theta, pos0, kc, vc);
    else
        hipLaunchKernelGGL(fw_rope_kv_n_kernel, dim3(N), dim3(256), 0, s, qkv, ldq, qd, kvd, heads, kv_heads, hd,
                           pdim, theta, pos0, kc, vc);
    return check_launch("rope launch");
}

/* A verify block: the forward of ntok consecutive tokens at pos .. pos + ntok - 1
 * with every matvec over ntok columns (weights decoded once for the block),
 * then the head over the same columns; logits are [ntok][vocab]. */
int block(Model * m, const uint32_t * tokens, int N, int pos, float * logits, hipStream_t s) {
    const sparkmv_model_cfg & c = m->c;
    const bool b16 = c.x_dtype == SPARKMV_X_BF16;
    const int qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, hd = c.head_dim, ldq = qd + 2 * kvd;
    FwTok8 tk;
    for (int t = 0; t < 8; t++) tk.t[t] = t < N ? (int) tokens[t] : 0;
    if (m->head_kind == 0) {
        hipLaunchKernelGGL(fw_fill_kernel, dim3((N * c.hidden + 255) / 256), dim3(256), 0, s, m->vh, N * c.hidden, 0.0f);
        if (check_launch("fill launch")) return -1;
        const Layout L = make_layout(c.dim, c.nc, c.vocab, c.hidden, c.v3);
        for (int t = 0; t < N; t++)
            for (int st = 0; st < c.nstages; st++)
                if (vq_row_dequant_launch(m->head_stages[st], L, (int) tokens[t], m->vh + (size_t) t * c.hidden, s))
                    return -1;
    } else {
        hipLaunchKernelGGL(fw_q8_0_rows_kernel, dim3((c.hidden + 255) / 256, N), dim3(256), 0, s,
                           (const uint8_t *) m->head_blocks, c.hidden, tk, m->vh);
        if (check_launch("embedding launch")) return -1;
    }
    const float scale = 1.0f / sqrtf((float) hd);
    const void * xin = b16 ? (const void *) m->vxn16 : (const void *) m->vxn;
    for (int li = 0; li < c.layers; li++) {
        const sparkmv_model_layer & L = m->layers[li];
        const bool full = L.full != 0;
        float * kc = m->kv + (size_t) li * 2 * c.max_ctx * kvd;
        float * vc = kc + (size_t) c.max_ctx * kvd;
        if (capture_rows(*m, li, m->vh, nullptr, pos, N, s)) return -1;
        if (rmsnorm(*m, m->vh, L.in_norm, s, N, m->vxn, m->vxn16)) return -1;
        if (gemv2(*m, L.qkv, ldq, m->vqkv, L.attn_gate, c.heads, m->vg, c.hidden, xin, s, N, ldq)) return -1;
        const double theta = full ? c.rope_full_theta : c.rope_slide_theta;
        const int pdim = rope_dim(hd, full ? c.rope_full_partial : c.rope_slide_partial);
        if (rope_kv_launch(m->vqkv, N, ldq, qd, kvd, c.heads, c.kv_heads, hd, pdim, (float) theta, pos, kc, vc, s))
            return -1;
        const int window = full ? 0 : c.sliding_window;
        const int last = pos + N - 1;
        const int span = full || c.sliding_window > last + 1 ? last + 1 : c.sliding_window;
        const int nch = (span + kAttnChunk - 1) / kAttnChunk;
        const dim3 pg((unsigned) nch, (unsigned) c.kv_heads, (unsigned) N), pb((unsigned) (64 * (c.heads / c.kv_heads)));
        uint16_t * a16 = b16 ? m->vattn16 : nullptr;
#define FW_ATTN_N(V)                                                                                                \
    do {                                                                                                            \
        hipLaunchKernelGGL(fw_attn_part_n_kernel<V>, pg, pb, 0, s, m->vqkv, ldq, kvd, kc, vc, pos, window, c.heads,   \
                           c.kv_heads, scale, m->nch_max, m->vpart);                                                \
        hipLaunchKernelGGL(fw_attn_combine_n_kernel<V>, dim3(c.heads, N), dim3(256), (uint32_t) (nch * 8), s,       \
                           m->vpart, m->vg, ldq, pos, window, c.heads, m->nch_max, m->vattn, a16);                  \
    } while (0)
        if (hd == 64) FW_ATTN_N(1);
        else if (hd == 128) FW_ATTN_N(2);
        else FW_ATTN_N(4);
#undef FW_ATTN_N
        if (check_launch("attention launch")) return -1;
        if (gemv(*m, L.out, c.hidden, qd, b16 ? (const void *) m->vattn16 : (const void *) m->vattn, m->vh, 1, s, N,
                 c.hidden))
            return -1;
        if (rmsnorm(*m, m->vh, L.post_norm, s, N, m->vxn, m->vxn16)) return -1;
        if (gate_up_act_n(*m, L.gate, L.up, c.intermediate, c.hidden, xin, m->vmg, m->vmu, m->vact,
                          b16 ? m->vact16 : nullptr, s, N))
            return -1;
        if (gemv(*m, L.down, c.hidden, c.intermediate, b16 ? (const void *) m->vact16 : (const void *) m->vact, m->vh,
                 1, s, N, c.hidden))
            return -1;
    }
    if (rmsnorm(*m, m->vh, m->final_norm, s, N, m->vxn, m->vxn16)) return -1;
    /* the head over the block's columns; the Q8_0 kernel gives each column
     * exactly its one-column result (the verify-head requirement,
     * Spark-X2.6-4B-Base-handoff.md:299-302) */
    if (m->head_kind == 0) return gemv(*m, m->head_stages, c.vocab, c.hidden, xin, logits, 0, s, N, c.vocab);
    return kq_gemv_launch(8, m->head_blocks, c.vocab, c.hidden, xin, b16 ? 0 : 1, c.hidden, N, logits, c.vocab, 0, s);
}

/* A prompt chunk (vq-model-gpu.cu:858-943 forward_batch): N tokens at
 * pos .. pos + N - 1 through every layer, the tokens already in m->vtok.
 * With logits, the final norm and the head of the last token
 * (vq-model-gpu.cu:946-953 tail_logits). */
int prompt(Model * m, int N, int pos, float * logits, hipStream_t s) {
    const sparkmv_model_cfg & c = m->c;
    const bool b16 = c.x_dtype == SPARKMV_X_BF16;
    const int qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, hd = c.head_dim, ldq = qd + 2 * kvd;
    if (m->head_kind == 0) {
        hipLaunchKernelGGL(fw_fill_kernel, dim3((N * c.hidden + 255) / 256), dim3(256), 0, s, m->vh, N * c.hidden, 0.0f);
        if (check_launch("fill launch")) return -1;
        const Layout L = make_layout(c.dim, c.nc, c.vocab, c.hidden, c.v3);
        for (int st = 0; st < c.nstages; st++)
            if (vq_row_dequant_dev_launch(m->head_stages[st], L, m->vtok, m->vh, s, N, (size_t) c.hidden)) return -1;
    } else {
        hipLaunchKernelGGL(fw_q8_0_rows_dev_kernel, dim3((c.hidden + 255) / 256, N), dim3(256), 0, s,
                           (const uint8_t *) m->head_blocks, c.hidden, (const int *) m->vtok, m->vh);
        if (check_launch("embedding launch")) return -1;
    }
    const float scale = 1.0f / sqrtf((float) hd);
    const void * xin = b16 ? (const void *) m->vxn16 : (const void *) m->vxn;
    for (int li = 0; li < c.layers; li++) {
        const sparkmv_model_layer & L = m->layers[li];
        const bool full = L.full != 0;
        float * kc = m->kv + (size_t) li * 2 * c.max_ctx * kvd;
        float * vc = kc + (size_t) c.max_ctx * kvd;
        if (capture_rows(*m, li, m->vh, nullptr, pos, N, s)) return -1;
        if (rmsnorm(*m, m->vh, L.in_norm, s, N, m->vxn, m->vxn16)) return -1;
        if (N <= kMaxCols) {
            if (gemv2(*m, L.qkv, ldq, m->vqkv, L.attn_gate, c.heads, m->vg, c.hidden, xin, s, N, ldq)) return -1;
        } else {
            if (mat_n(*m, L.qkv, ldq, c.hidden, xin, m->vqkv, 0, s, N, ldq)) return -1;
            if (mat_n(*m, L.attn_gate, c.heads, c.hidden, xin, m->vg, 0, s, N, ldq)) return -1;
        }
        const double theta = full ? c.rope_full_theta : c.rope_slide_theta;
        const int pdim = rope_dim(hd, full ? c.rope_full_partial : c.rope_slide_partial);
        if (rope_kv_launch(m->vqkv, N, ldq, qd, kvd, c.heads, c.kv_heads, hd, pdim, (float) theta, pos, kc, vc, s))
            return -1;
        const int window = full ? 0 : c.sliding_window;
        const dim3 ag((unsigned) c.kv_heads, (unsigned) N), ab((unsigned) (64 * (c.heads / c.kv_heads)));
        uint16_t * a16 = b16 ? m->vattn16 : nullptr;
        if (hd == 256) {
            hipLaunchKernelGGL(fw_attn_prompt_mfma_kernel, dim3((unsigned) c.heads, (unsigned) ((N + kPaTok - 1) / kPaTok)),
                               dim3(256), 0, s, m->vqkv, ldq, kvd, kc, vc, m->vg, ldq, pos, N, window,
                               c.heads, c.kv_heads, scale, m->vattn, a16);
        }
        else if (hd == 64)
            hipLaunchKernelGGL(fw_attn_prompt_kernel<1>, ag, ab, 0, s, m->vqkv, ldq, kvd, kc, vc, m->vg, ldq, pos,
                               window, c.heads, c.kv_heads, scale, m->vattn, a16);
        else if (hd == 128)
            hipLaunchKernelGGL(fw_attn_prompt_kernel<2>, ag, ab, 0, s, m->vqkv, ldq, kvd, kc, vc, m->vg, ldq, pos,
                               window, c.heads, c.kv_heads, scale, m->vattn, a16);
        else
            hipLaunchKernelGGL(fw_attn_prompt_kernel<4>, ag, ab, 0, s, m->vqkv, ldq, kvd, kc, vc, m->vg, ldq, pos,
                               window, c.heads, c.kv_heads, scale, m->vattn, a16);
        if (check_launch("attention launch")) return -1;
        if (mat_n(*m, L.out, c.hidden, qd, b16 ? (const void *) m->vattn16 : (const void *) m->vattn, m->vh, 1, s, N,
                  c.hidden))
            return -1;
        if (rmsnorm(*m, m->vh, L.post_norm, s, N, m->vxn, m->vxn16)) return -1;
        if (N <= kMaxCols) {
            if (gate_up_act_n(*m, L.gate, L.up, c.intermediate, c.hidden, xin, m->vmg, m->vmu, m->vact,
                              b16 ? m->vact16 : nullptr, s, N))
                return -1;
        } else {
            if (mat_n(*m, L.gate, c.intermediate, c.hidden, xin, m->vmg, 0, s, N, c.intermediate)) return -1;
            if (mat_n(*m, L.up, c.intermediate, c.hidden, xin, m->vmu, 0, s, N, c.intermediate)) return -1;
            /* bf16: down reads act16 only, so the f32 copy is not written */
            hipLaunchKernelGGL(fw_gelu_mul_kernel, dim3((N * c.intermediate / 4 + 255) / 256 + 1), dim3(256), 0, s,
                               m->vmg, m->vmu, b16 ? nullptr : m->vact, b16 ? m->vact16 : nullptr,
                               N * c.intermediate);
            if (check_launch("gelu launch")) return -1;
        }
        if (mat_n(*m, L.down, c.hidden, c.intermediate, b16 ? (const void *) m->vact16 : (const void *) m->vact, m->vh,
                  1, s, N, c.hidden))
            return -1;
    }
    if (!logits) return 0;
    /* the last token's row: final norm and the head, as one decode step's */
    if (rmsnorm(*m, m->vh + (size_t) (N - 1) * c.hidden, m->final_norm, s, 1, m->vxn, m->vxn16)) return -1;
    if (m->head_kind == 0) return gemv(*m, m->head_stages, c.vocab, c.hidden, xin, logits, 0, s);
    return kq_gemv_launch(8, m->head_blocks, c.vocab, c.hidden, xin, b16 ? 0 : 1, c.hidden, 1, logits, c.vocab, 0, s);
}

}  // namespace

extern "C" {

int sparkmv_model_forward(void * model, uint32_t token, int pos, float * logits, void * stream) {
    Model * m = (Model *) model;
    if (!m || !logits) { set_error("model or logits is null"); return -1; }
    if (check_step(m, token, pos) || ready(m)) return -1;
    hipStream_t s = (hipStream_t) stream;
    if (set_state(m, token, pos, s)) return -1;
    if (chain(m, logits, s)) return -1;
    m->len = pos + 1;
    return 0;
}

int sparkmv_model_capture(void * model, float * logits, void * stream) {
    Model * m = (Model *) model;
    if (!m || !logits) { set_error("model or logits is null"); return -1; }
    if (!stream) { set_error("capture needs a created stream, not the null stream"); return -1; }
    if (ready(m)) return -1;
    hipStream_t s = (hipStream_t) stream;
    hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail_hip("begin capture", e);
    const int rc = chain(m, logits, s);
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(s, &g);
    if (rc) { if (g) (void) hipGraphDestroy(g); return -1; }
    if (e != hipSuccess) return fail_hip("end capture", e);
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) { (void) hipGraphDestroy(g); return fail_hip("graph instantiate", e); }
    if (m->exec) (void) hipGraphExecDestroy(m->exec);
    if (m->graph) (void) hipGraphDestroy(m->graph);
    m->graph = g;
    m->exec = x;
    return 0;
}

int sparkmv_model_replay(void * model, uint32_t token, int pos, void * stream) {
    Model * m = (Model *) model;
    if (!m) { set_error("model is null"); return -1; }
    if (!m->exec) { set_error("the model has no recorded forward: call sparkmv_model_capture first"); return -1; }
    if (check_step(m, token, pos)) return -1;
    hipStream_t s = (hipStream_t) stream;
    if (set_state(m, token, pos, s)) return -1;
    hipError_t e = hipGraphLaunch(m->exec, s);
    if (e != hipSuccess) return fail_hip("graph launch", e);
    m->len = pos + 1;
    return 0;
}

int sparkmv_model_verify(void * model, const uint32_t * tokens, int ntok, int pos, float * logits, void * stream) {
    Model * m = (Model *) model;
    if (!m || !tokens || !logits) { set_error("model, tokens or logits is null"); return -1; }
    if (ntok < 1 || ntok > 8) { set_error("a verify block holds 1..8 tokens, not %d", ntok); return -1; }
    if (pos < 0 || pos + ntok > m->c.max_ctx) {
        set_error("positions %d..%d exceed the %d-token cache", pos, pos + ntok - 1, m->c.max_ctx);
        return -1;
    }
    for (int t = 0; t < ntok; t++)
        if ((long) tokens[t] >= m->c.vocab) { set_error("token %u is outside the vocabulary", tokens[t]); return -1; }
    if (ready(m)) return -1;
    if (!m->vmem && alloc_block(m, 8)) return -1;
    if (block(m, tokens, ntok, pos, logits, (hipStream_t) stream)) return -1;
    m->len = pos + ntok;
    return 0;
}

int sparkmv_model_reserve(void * model, int ntok) {
    Model * m = (Model *) model;
    if (!m) { set_error("model is null"); return -1; }
    if (ntok < 1 || ntok > kPromptMax) { set_error("a reservation covers 1..%d tokens, not %d", kPromptMax, ntok); return -1; }
    if (m->vmem && ntok > m->vcap) {
        /* the old buffers may still be in use by queued work */
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return fail_hip("synchronize before a larger reservation", e);
    }
    return alloc_block(m, ntok);
}

int sparkmv_model_forward_batch(void * model, const uint32_t * tokens, int ntok, int pos, float * logits,
                                void * stream) {
    Model * m = (Model *) model;
    if (!m || !tokens) { set_error("model or tokens is null"); return -1; }
    if (ntok < 1 || ntok > kPromptMax) { set_error("a prompt chunk holds 1..%d tokens, not %d", kPromptMax, ntok); return -1; }
    if (pos < 0 || pos + ntok > m->c.max_ctx) {
        set_error("positions %d..%d exceed the %d-token cache", pos, pos + ntok - 1, m->c.max_ctx);
        return -1;
    }
    for (int t = 0; t < ntok; t++)
        if ((long) tokens[t] >= m->c.vocab) { set_error("token %u is outside the vocabulary", tokens[t]); return -1; }
    if (ready(m)) return -1;
    if (!m->vmem || ntok > m->vcap) {
        if (m->vmem) {
            hipError_t e = hipDeviceSynchronize();
            if (e != hipSuccess) return fail_hip("synchronize before larger block buffers", e);
        }
        if (alloc_block(m, ntok)) return -1;
    }
    hipStream_t s = (hipStream_t) stream;
    /* the tokens go to device memory on the stream; the host array is read
     * before the call returns */
    static_assert(sizeof(uint32_t) == sizeof(int), "token width");
    hipError_t e = hipMemcpyAsync(m->vtok, tokens, (size_t) ntok * sizeof(int), hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return fail_hip("token upload", e);
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail_hip("token upload", e);
    if (prompt(m, ntok, pos, logits, s)) return -1;
    m->len = pos + ntok;
    return 0;
}

int sparkmv_model_rollback(void * model, int pos) {
    Model * m = (Model *) model;
    if (!m) { set_error("model is null"); return -1; }
    if (pos < 0 || pos > m->len) { set_error("rollback to %d exceeds the %d cached positions", pos, m->len); return -1; }
    m->len = pos;
    return 0;
}

int sparkmv_model_len(void * model) {
    Model * m = (Model *) model;
    return m ? m->len : -1;
}

/* Apply a trusted tuning profile to the model's VQ matvecs, per geometry,
 * as the reference's loader does (tools/vq/gpu/vq-model-gpu.cu:300-324): a
 * geometry with a runnable gemv entry takes its kernel and width; an entry
 * that is not runnable here leaves the heuristic; an untrusted profile
 * changes nothing. Returns the number of geometries tuned, or -1. Drops a
 * captured graph (capture again to replay the tuned kernels). */
int sparkmv_model_apply_profile(void * model, const void * profile, uint64_t artifact, const char * gpu) {
    Model * m = (Model *) model;
    if (!m || !profile || !gpu) { set_error("model, profile or gpu name is null"); return -1; }
    const int t = sparkmv_profile_trusted(profile, artifact, gpu);
    if (t < 0) return -1;
    if (t == 0) {
        set_error("profile: measured for another artifact or device; the heuristic stays");
        return 0;
    }
    const auto & c = m->c;
    const int qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim;
    const int geoms[][2] = {{qd + 2 * kvd, c.hidden}, {c.heads, c.hidden}, {c.hidden, qd},
                            {c.intermediate, c.hidden}, {c.hidden, c.intermediate}, {c.vocab, c.hidden}};
    int applied = 0, refused = 0;
    m->picks.clear();
    for (const auto & g : geoms) {
        if (m->picks.count({g[0], g[1]})) continue;
        int v = 0, th = 0;
        const int r = profile_gemv_pick(profile, c.dim, c.nc, g[0], g[1], c.v3, &v, &th);
        if (r < 0) refused++;
        if (r == 1) {
            m->picks[{g[0], g[1]}] = {v, th};
            applied++;
        }
    }
    if (m->exec) { (void) hipGraphExecDestroy(m->exec); m->exec = nullptr; }
    if (m->graph) { (void) hipGraphDestroy(m->graph); m->graph = nullptr; }
    set_error("profile: %d geometries take their tuned kernel, %d entries are not runnable here (heuristic kept)",
              applied, refused);
    return applied;
}

/* The kernel the model runs for a (rows, cols) VQ matvec: variant and width
 * as sparkmv_plan_op_kernel reports them (0, 0 = the heuristic). */
int sparkmv_model_matvec_kernel(void * model, int rows, int cols, int * variant, int * threads) {
    Model * m = (Model *) model;
    if (!m) { set_error("model is null"); return -1; }
    const auto it = m->picks.find({rows, cols});
    if (variant) *variant = it == m->picks.end() ? 0 : it->second.first;
    if (threads) *threads = it == m->picks.end() ? 0 : it->second.second;
    return 0;
}

/* The layer's KV cache rows (device pointers), for tests and inspection. */
int sparkmv_model_kv(void * model, int li, float ** k, float ** v) {
    Model * m = (Model *) model;
    if (!m || li < 0 || li >= m->c.layers || !k || !v) { set_error("bad model, layer or output"); return -1; }
    const size_t kvd = (size_t) m->c.kv_heads * m->c.head_dim;
    *k = m->kv + (size_t) li * 2 * m->c.max_ctx * kvd;
    *v = *k + (size_t) m->c.max_ctx * kvd;
    return 0;
}

int sparkmv_model_enable_capture(void * model, const int * layers, int n) {
    Model * m = (Model *) model;
    if (!m || (n > 0 && !layers)) { set_error("model or layer list is null"); return -1; }
    /* the runtime's limits and messages (vq-model-gpu.cu:707-736) */
    if (n <= 0 || n > 8) { set_error("capture: %d layers requested, the limit is 8", n); return -1; }
    if (m->cap) { set_error("capture: already enabled"); return -1; }
    std::vector<int> slot((size_t) m->c.layers, -1);
    for (int k = 0; k < n; k++) {
        const int li = layers[k];
        if (li < 0 || li >= m->c.layers) { set_error("capture: layer %d is outside 0..%d", li, m->c.layers); return -1; }
        if (slot[(size_t) li] >= 0) { set_error("capture: layer %d is listed twice", li); return -1; }
        slot[(size_t) li] = k;
    }
    void * mem = nullptr;
    hipError_t e = hipMalloc(&mem, (size_t) n * m->c.max_ctx * m->c.hidden * sizeof(float));
    if (e != hipSuccess) {
        set_error("capture: cannot allocate %d x %d x %d floats", n, m->c.max_ctx, m->c.hidden);
        return -1;
    }
    m->cap = (float *) mem;
    m->cap_n = n;
    m->cap_slot = slot;
    /* a recorded graph lacks the copies: record it again */
    if (m->exec) { (void) hipGraphExecDestroy(m->exec); m->exec = nullptr; }
    if (m->graph) { (void) hipGraphDestroy(m->graph); m->graph = nullptr; }
    return 0;
}

int sparkmv_model_captured(void * model, int k, float ** rows) {
    Model * m = (Model *) model;
    if (!m || !rows) { set_error("model or output is null"); return -1; }
    if (k < 0 || k >= m->cap_n) { set_error("capture slot %d is outside 0..%d", k, m->cap_n - 1); return -1; }
    *rows = m->cap + (size_t) k * m->c.max_ctx * m->c.hidden;
    return m->len;
}

int sparkmv_model_embed_row(void * model, uint32_t id, float * out, void * stream) {
    Model * m = (Model *) model;
    if (!m || !out) { set_error("model or output is null"); return -1; }
    if (m->head_kind < 0) { set_error("the model has no head"); return -1; }
    if ((long) id >= m->c.vocab) { set_error("token %u is outside the vocabulary", id); return -1; }
    const hipStream_t s = (hipStream_t) stream;
    const sparkmv_model_cfg & c = m->c;
    if (m->head_kind == 0) {
        hipLaunchKernelGGL(fw_fill_kernel, dim3((c.hidden + 255) / 256), dim3(256), 0, s, out, c.hidden, 0.0f);
        if (check_launch("fill launch")) return -1;
        const Layout L = make_layout(c.dim, c.nc, c.vocab, c.hidden, c.v3);
        for (int st = 0; st < c.nstages; st++)
            if (vq_row_dequant_launch(m->head_stages[st], L, (int) id, out, s)) return -1;
        return 0;
    }
    FwTok8 tk;
    for (int t = 0; t < 8; t++) tk.t[t] = (int) id;
    hipLaunchKernelGGL(fw_q8_0_rows_kernel, dim3((c.hidden + 255) / 256, 1), dim3(256), 0, s,
                       (const uint8_t *) m->head_blocks, c.hidden, tk, out);
    return check_launch("embedding launch");
}

int sparkmv_argmax(const float * logits, int n, int * out, void * stream) {
    if (!logits || !out) { set_error("logits or output is null"); return -1; }
    if (n < 1) { set_error("argmax needs at least one value, not %d", n); return -1; }
    hipLaunchKernelGGL(fw_argmax_kernel, dim3(1), dim3(1024), 0, (hipStream_t) stream, logits, n, out);
    return check_launch("argmax launch");
}

}  // extern "C"
