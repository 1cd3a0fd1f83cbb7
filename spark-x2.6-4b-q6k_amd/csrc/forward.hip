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
 */
#include "kq.h"
#include "vq.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

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

/* out = x * inv * w with inv = 1 / sqrt(mean(x^2) + eps), the sum of squares in
 * f64 and inv rounded once to f32 (model.rs:236-245). One workgroup. */
__global__ __launch_bounds__(256) void fw_rmsnorm_kernel(const float * x, const float * w, float * out,
                                                         uint16_t * out16, int n, float eps) {
    __shared__ double part[4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    double s = 0.0;
    for (int i = t; i < n; i += 256) {
        const double v = (double) x[i];
        s += v * v;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) part[wave] = s;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = (float) (1.0 / sqrt(tot / (double) n + (double) eps));
    for (int i = t; i < n; i += 256) {
        const float v = x[i] * inv * w[i];
        if (out) out[i] = v;
        if (out16) out16[i] = fw_bf16(v);
    }
}

/* Rope and the KV store in one launch. Items [0, (heads + kv_heads) * half)
 * rotate the pair (i, i + half) of one q or k head over its first pdim
 * elements with the f32 table of model.rs:416-428 (apply_rope, :430-438); a
 * rotated k pair also goes to the cache. Items [0, kvd) store v[item] and
 * the k elements past pdim, which rope leaves alone. */
__global__ void fw_rope_kv_kernel(float * qkv, int qd, int kvd, int heads, int kv_heads, int hd, int pdim,
                                  float theta, int pos, float * kc, float * vc) {
    const int half = pdim / 2;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < (heads + kv_heads) * half) {
        const int h = t / half, i = t - h * half;
        const float freq = 1.0f / powf(theta, (float) (2 * i) / (float) pdim);
        const float a = (float) pos * freq;
        const float c = cosf(a), s = sinf(a);
        float * base = h < heads ? qkv + (size_t) h * hd : qkv + qd + (size_t) (h - heads) * hd;
        const float x0 = base[i], x1 = base[i + half];
        const float r0 = x0 * c - x1 * s, r1 = x1 * c + x0 * s;
        base[i] = r0;
        base[i + half] = r1;
        if (h >= heads) {
            float * k = kc + (size_t) pos * kvd + (size_t) (h - heads) * hd;
            k[i] = r0;
            k[i + half] = r1;
        }
    }
    if (t < kvd) {
        vc[(size_t) pos * kvd + t] = qkv[qd + kvd + t];
        if (t % hd >= 2 * half) kc[(size_t) pos * kvd + t] = qkv[qd + t];
    }
}

/* One workgroup (4 waves) per query head over positions start .. start+n-1 of
 * the cache (model.rs:508-557). Scores: wave w takes positions w, w+4, ...,
 * its lanes split the head's elements and meet in a butterfly. Softmax with
 * the running max, then thread d sums p_j * V[j][d] in position order and
 * applies the head's sigmoid gate. The scores sit in LDS (n floats). */
__global__ __launch_bounds__(256) void fw_attn_kernel(const float * qkv, int qd, int kvd, const float * gate,
                                                      const float * kc, const float * vc, int start, int n, int heads,
                                                      int kv_heads, int hd, float scale, float * out,
                                                      uint16_t * out16) {
    extern __shared__ float sc[];
    __shared__ float red[8];
    const int h = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int kvh = h * kv_heads / heads;
    const float * q = qkv + (size_t) h * hd;
    const float * kb = kc + (size_t) start * kvd + (size_t) kvh * hd;
    for (int j = wave; j < n; j += 4) {
        const float * k = kb + (size_t) j * kvd;
        float s = 0.0f;
        for (int d = lane; d < hd; d += 64) s += q[d] * k[d];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        if (lane == 0) sc[j] = s * scale;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int j = t; j < n; j += 256) mx = fmaxf(mx, sc[j]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.0f;
    for (int j = t; j < n; j += 256) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) red[4 + wave] = sum;
    __syncthreads();
    const float inv = 1.0f / ((red[4] + red[5]) + (red[6] + red[7]));
    const float g = 1.0f / (1.0f + expf(-gate[h]));
    const float * vb = vc + (size_t) start * kvd + (size_t) kvh * hd;
    for (int d = t; d < hd; d += 256) {
        float o = 0.0f;
        for (int j = 0; j < n; j++) o += sc[j] * inv * vb[(size_t) j * kvd + d];
        const float r = o * g;
        out[(size_t) h * hd + d] = r;
        if (out16) out16[(size_t) h * hd + d] = fw_bf16(r);
    }
}

/* act = gelu(g) * u with torch's exact gelu, erf in f64 as model.rs:253-258
 * calls it. */
__global__ void fw_gelu_mul_kernel(const float * g, const float * u, float * act, uint16_t * act16, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += blockDim.x * gridDim.x) {
        const float x = g[i];
        const double e = erf((double) x * 0.70710678118654752440);
        const float r = 0.5f * x * (1.0f + (float) e) * u[i];
        act[i] = r;
        if (act16) act16[i] = fw_bf16(r);
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
};

size_t align256(size_t b) { return (b + 255) & ~(size_t) 255; }

int check_launch(const char * what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip(what, e);
}

int gemv(const Model & m, const void * const * st, int rows, int cols, const void * x, float * y, int acc,
         hipStream_t s) {
    VqMatDesc d;
    memset(&d, 0, sizeof d);
    for (int i = 0; i < m.c.nstages; i++) d.stages[i] = st[i];
    d.y = y;
    d.rows = rows;
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = m.c.dim; c.nc = m.c.nc; c.cols = cols; c.v3 = m.c.v3; c.nst = m.c.nstages;
    c.mats = &d; c.nmat = 1;
    c.x = x; c.ldx = cols; c.xf32 = m.c.x_dtype == SPARKMV_X_F32; c.ncol = 1; c.ldy = rows;
    c.accumulate = acc; c.stream = s;
    return vq_launch(c);
}

int gemv2(const Model & m, const void * const * st0, int rows0, float * y0, const void * const * st1, int rows1,
          float * y1, int cols, const void * x, hipStream_t s) {
    VqMatDesc d[2];
    memset(d, 0, sizeof d);
    for (int i = 0; i < m.c.nstages; i++) { d[0].stages[i] = st0[i]; d[1].stages[i] = st1[i]; }
    d[0].y = y0; d[0].rows = rows0;
    d[1].y = y1; d[1].rows = rows1;
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = m.c.dim; c.nc = m.c.nc; c.cols = cols; c.v3 = m.c.v3; c.nst = m.c.nstages;
    c.mats = d; c.nmat = 2;
    c.x = x; c.ldx = cols; c.xf32 = m.c.x_dtype == SPARKMV_X_F32; c.ncol = 1; c.ldy = rows0;
    c.accumulate = 0; c.stream = s;
    return vq_launch(c);
}

int rmsnorm(const Model & m, const float * x, const float * w, hipStream_t s) {
    const bool b16 = m.c.x_dtype == SPARKMV_X_BF16;
    hipLaunchKernelGGL(fw_rmsnorm_kernel, dim3(1), dim3(256), 0, s, x, w, m.xn, b16 ? m.xn16 : nullptr,
                       m.c.hidden, m.c.eps);
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
    /* the attention kernel keeps one score per position in LDS */
    const long span = (long) c.max_ctx;
    if (span * 4 > 150 * 1024) { set_error("max_ctx %d needs more than 150 KB of attention scores", c.max_ctx); return nullptr; }
    if (span * 4 > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *) fw_attn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int) (span * 4));
        if (e != hipSuccess) { fail_hip("LDS opt-in for the attention kernel", e); return nullptr; }
    }
    Model * m = new Model;
    m->c = c;
    m->layers.resize(c.layers);
    m->layer_set.assign(c.layers, 0);
    const size_t qd = (size_t) c.heads * c.head_dim, kvd = (size_t) c.kv_heads * c.head_dim;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += align256(bytes); return o; };
    const size_t o_h = take(c.hidden * 4), o_xn = take(c.hidden * 4), o_qkv = take((qd + 2 * kvd) * 4);
    const size_t o_g = take(c.heads * 4), o_attn = take(qd * 4), o_mg = take(c.intermediate * 4);
    const size_t o_mu = take(c.intermediate * 4), o_act = take(c.intermediate * 4);
    const size_t o_xn16 = take(c.hidden * 2), o_attn16 = take(qd * 2), o_act16 = take(c.intermediate * 2);
    const size_t o_kv = take((size_t) c.layers * c.max_ctx * kvd * 4 * 2);
    hipError_t e = hipMalloc(&m->mem, off);
    if (e != hipSuccess) {
        fail_hip("model buffers", e);
        delete m;
        return nullptr;
    }
    uint8_t * b = (uint8_t *) m->mem;
    m->h = (float *) (b + o_h); m->xn = (float *) (b + o_xn); m->qkv = (float *) (b + o_qkv);
    m->g = (float *) (b + o_g); m->attn = (float *) (b + o_attn); m->mg = (float *) (b + o_mg);
    m->mu = (float *) (b + o_mu); m->act = (float *) (b + o_act);
    m->xn16 = (uint16_t *) (b + o_xn16); m->attn16 = (uint16_t *) (b + o_attn16); m->act16 = (uint16_t *) (b + o_act16);
    m->kv = (float *) (b + o_kv);
    return m;
}

void sparkmv_model_destroy(void * model) {
    Model * m = (Model *) model;
    if (!m) return;
    if (m->mem) (void) hipFree(m->mem);
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

int sparkmv_model_forward(void * model, uint32_t token, int pos, float * logits, void * stream) {
    Model * m = (Model *) model;
    if (!m || !logits) { set_error("model or logits is null"); return -1; }
    const sparkmv_model_cfg & c = m->c;
    if ((long) token >= c.vocab) { set_error("token %u is outside the vocabulary", token); return -1; }
    if (pos < 0 || pos >= c.max_ctx) { set_error("position %d exceeds the %d-token cache", pos, c.max_ctx); return -1; }
    if (m->head_kind < 0) { set_error("the model has no head"); return -1; }
    for (int li = 0; li < c.layers; li++)
        if (!m->layer_set[li]) { set_error("layer %d has no weights", li); return -1; }
    hipStream_t s = (hipStream_t) stream;
    const bool b16 = c.x_dtype == SPARKMV_X_BF16;
    const int qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, hd = c.head_dim;

    /* the embedding row (model.rs:462-464): the tied head's row `token` */
    if (m->head_kind == 0) {
        hipLaunchKernelGGL(fw_fill_kernel, dim3((c.hidden + 255) / 256), dim3(256), 0, s, m->h, c.hidden, 0.0f);
        if (check_launch("fill launch")) return -1;
        const Layout L = make_layout(c.dim, c.nc, c.vocab, c.hidden, c.v3);
        for (int st = 0; st < c.nstages; st++)
            if (vq_row_dequant_launch(m->head_stages[st], L, (int) token, m->h, s)) return -1;
    } else {
        const size_t rowbytes = (size_t) (c.hidden / 32) * 34;
        if (kq_dequant_launch(8, (const uint8_t *) m->head_blocks + (size_t) token * rowbytes, 1, c.hidden, m->h, s))
            return -1;
    }

    const float scale = 1.0f / sqrtf((float) hd);
    for (int li = 0; li < c.layers; li++) {
        const sparkmv_model_layer & L = m->layers[li];
        const bool full = L.full != 0;
        float * kc = m->kv + (size_t) li * 2 * c.max_ctx * kvd;
        float * vc = kc + (size_t) c.max_ctx * kvd;

        if (rmsnorm(*m, m->h, L.in_norm, s)) return -1;
        const void * xin = b16 ? (const void *) m->xn16 : (const void *) m->xn;
        if (gemv2(*m, L.qkv, qd + 2 * kvd, m->qkv, L.attn_gate, c.heads, m->g, c.hidden, xin, s)) return -1;

        /* rope and the KV store (model.rs:484-503) */
        const double theta = full ? c.rope_full_theta : c.rope_slide_theta;
        const double partial = full ? c.rope_full_partial : c.rope_slide_partial;
        int pdim = (int) ((float) hd * (float) partial);
        if (pdim > hd) pdim = hd;
        const int items = (c.heads + c.kv_heads) * (pdim / 2) > kvd ? (c.heads + c.kv_heads) * (pdim / 2) : kvd;
        hipLaunchKernelGGL(fw_rope_kv_kernel, dim3((items + 255) / 256), dim3(256), 0, s, m->qkv, qd, kvd, c.heads,
                           c.kv_heads, hd, pdim, (float) theta, pos, kc, vc);
        if (check_launch("rope launch")) return -1;

        /* attention over the layer's window (model.rs:508-557) */
        const int start = full ? 0 : (pos + 1 > c.sliding_window ? pos + 1 - c.sliding_window : 0);
        const int n = pos + 1 - start;
        hipLaunchKernelGGL(fw_attn_kernel, dim3(c.heads), dim3(256), (uint32_t) (n * 4), s, m->qkv, qd, kvd, m->g, kc,
                           vc, start, n, c.heads, c.kv_heads, hd, scale, m->attn, b16 ? m->attn16 : nullptr);
        if (check_launch("attention launch")) return -1;
        if (gemv(*m, L.out, c.hidden, qd, b16 ? (const void *) m->attn16 : (const void *) m->attn, m->h, 1, s))
            return -1;

        /* MLP (model.rs:566-581) */
        if (rmsnorm(*m, m->h, L.post_norm, s)) return -1;
        if (gemv2(*m, L.gate, c.intermediate, m->mg, L.up, c.intermediate, m->mu, c.hidden, xin, s)) return -1;
        hipLaunchKernelGGL(fw_gelu_mul_kernel, dim3((c.intermediate + 255) / 256), dim3(256), 0, s, m->mg, m->mu,
                           m->act, b16 ? m->act16 : nullptr, c.intermediate);
        if (check_launch("gelu launch")) return -1;
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

/* The layer's KV cache rows (device pointers), for tests and inspection. */
int sparkmv_model_kv(void * model, int li, float ** k, float ** v) {
    Model * m = (Model *) model;
    if (!m || li < 0 || li >= m->c.layers || !k || !v) { set_error("bad model, layer or output"); return -1; }
    const size_t kvd = (size_t) m->c.kv_heads * m->c.head_dim;
    *k = m->kv + (size_t) li * 2 * m->c.max_ctx * kvd;
    *v = *k + (size_t) m->c.max_ctx * kvd;
    return 0;
}

}  // extern "C"
