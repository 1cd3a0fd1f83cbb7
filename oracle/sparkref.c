/* sparkref.c — the oracle (test infrastructure only; see sparkref.h).
 *
 * A CPU restatement of the reference's quantized matvec path, written from the
 * reference's Rust and C sources and cited function by function. It is built
 * with -ffp-contract=off so every `a += b * c` rounds twice, as the Rust code
 * does (the reference builds its C decoder the same way, tools/vq/build.sh:38-43).
 */
#include "sparkref.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static uint16_t rd16(const uint8_t * b, size_t o) { return (uint16_t) (b[o] | (b[o + 1] << 8)); }
static uint32_t rd32(const uint8_t * b, size_t o) {
    return (uint32_t) b[o] | ((uint32_t) b[o + 1] << 8) | ((uint32_t) b[o + 2] << 16) | ((uint32_t) b[o + 3] << 24);
}
static uint64_t rd64(const uint8_t * b, size_t o) { return (uint64_t) rd32(b, o) | ((uint64_t) rd32(b, o + 4) << 32); }

static void set_err(char * err, size_t errn, const char * msg) {
    if (err && errn) snprintf(err, errn, "%s", msg);
}

/* tools/vq-format/src/lib.rs:50-72: exact half -> single. A subnormal half is
 * normalised by shifting its significand up to the hidden bit; the exponent
 * field starts at 113 (= 127 - 15 + 1) and drops by one per shift. */
float sr_f16(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t ex = ((uint32_t) h >> 10) & 0x1fu;
    uint32_t man = (uint32_t) h & 0x3ffu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            uint32_t e = 113;
            while ((man & 0x400u) == 0) { man <<= 1; e--; }
            bits = sign | (e << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* tools/vq-runtime/src/safetensors.rs:187: bf16 is the top half of an f32. */
float sr_bf16(uint16_t h) {
    const uint32_t bits = (uint32_t) h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static int bits_for(int nc) {
    int b = 1;
    while ((1L << b) < (long) nc) b++;
    return b;
}

/* tools/vq-format/src/lib.rs:94-156 (Stage::open). */
int sr_stage_open(const uint8_t * p, size_t len, sr_stage * st, char * err, size_t errn) {
    memset(st, 0, sizeof *st);
    const int v3 = len >= 4 && memcmp(p, "DQV3", 4) == 0;
    if (len < 16 || (!v3 && memcmp(p, "DQVQ", 4) != 0)) {
        set_err(err, errn, "stage payload magic is neither DQVQ nor DQV3");
        return -1;
    }
    const size_t hdr = v3 ? 24 : 16;
    const size_t dim = rd16(p, 4), nc = rd16(p, 6), rows = rd32(p, 8), cols = rd32(p, 12);
    if (dim == 0 || nc == 0 || rows == 0 || cols == 0 || cols % dim != 0) {
        set_err(err, errn, "stage header is inconsistent");
        return -1;
    }
    const size_t cb_len = nc * dim * 2, gain_len = rows * 2;
    if (len < hdr + cb_len + gain_len) {
        set_err(err, errn, "stage payload is truncated");
        return -1;
    }
    const int nbit = bits_for((int) nc);
    if (v3 && nbit > 13) {
        char m[160];
        snprintf(m, sizeof m, "DQV3 carries 13 index bits, nc %zu needs %d; rewrite with --format v2", nc, nbit);
        set_err(err, errn, m);
        return -1;
    }
    const size_t nidx_row = cols / dim;
    size_t mrow = 0, prow = 0, idx_bytes;
    if (v3) {
        const size_t mb = nbit < 12 ? (size_t) nbit : 12;
        mrow = (nidx_row * mb + 7) / 8;
        prow = nbit > 12 ? (nidx_row + 7) / 8 : 0;
        idx_bytes = rows * (mrow + prow);
    } else {
        const size_t nidx = rows * nidx_row;
        idx_bytes = nbit == 8 ? nidx : (nidx * (size_t) nbit + 7) / 8 + 1;
    }
    if (len < hdr + cb_len + gain_len + idx_bytes) {
        set_err(err, errn, "stage index stream is truncated");
        return -1;
    }
    st->dim = (int) dim; st->nc = (int) nc; st->rows = (int) rows; st->cols = (int) cols;
    st->nbit = nbit; st->v3 = v3; st->mrow = mrow; st->prow = prow;
    st->bytes = hdr + cb_len + gain_len + idx_bytes;
    st->gains = p + hdr + cb_len;
    st->stream = p + hdr + cb_len + gain_len;
    st->stream_len = len - (hdr + cb_len + gain_len);
    st->cb32 = (float *) malloc(nc * dim * sizeof(float));
    if (!st->cb32) { set_err(err, errn, "out of memory"); return -1; }
    for (size_t i = 0; i < nc * dim; i++) st->cb32[i] = sr_f16(rd16(p + hdr, i * 2));
    return 0;
}

void sr_stage_close(sr_stage * st) {
    free(st->cb32);
    st->cb32 = NULL;
}

static uint32_t sbyte(const sr_stage * st, size_t k) { return k < st->stream_len ? st->stream[k] : 0u; }

/* tools/vq-format/src/lib.rs:162-189 (Stage::index). DQV3: row-local stream of
 * min(nbit, 12)-bit fields read through a 4-byte window whose bytes past the
 * stream read as zero, plus the plane bit as bit 12. DQVQ: one stream across
 * the whole matrix, a byte per index at 8 bits, else a 3-byte window. */
uint32_t sr_stage_index(const sr_stage * st, size_t row, size_t i) {
    if (st->v3) {
        const size_t mb = st->nbit < 12 ? (size_t) st->nbit : 12;
        const size_t bit = i * mb;
        const size_t q = row * st->mrow + (bit >> 3);
        const uint32_t w = sbyte(st, q) | sbyte(st, q + 1) << 8 | sbyte(st, q + 2) << 16 | sbyte(st, q + 3) << 24;
        uint32_t v = (w >> (bit & 7)) & ((1u << mb) - 1u);
        if (st->prow > 0) {
            const size_t pp = st->mrow * (size_t) st->rows + row * st->prow + (i >> 3);
            v |= ((sbyte(st, pp) >> (i & 7)) & 1u) << 12;
        }
        return v;
    }
    const size_t gi = row * (size_t) (st->cols / st->dim) + i;
    if (st->nbit == 8) return st->stream[gi];
    const size_t bit = gi * (size_t) st->nbit;
    const uint32_t w = (uint32_t) st->stream[bit >> 3] | (uint32_t) st->stream[(bit >> 3) + 1] << 8
                     | (uint32_t) st->stream[(bit >> 3) + 2] << 16;
    return (w >> (bit & 7)) & ((1u << st->nbit) - 1u);
}

/* tools/vq-format/src/lib.rs:192-194 */
float sr_stage_gain(const sr_stage * st, size_t row) { return sr_f16(rd16(st->gains, row * 2)); }

/* tools/vq-format/src/lib.rs:197-211: out[r][dim*i + d] += cb[v][d] * g[r]. */
void sr_stage_add_into(const sr_stage * st, float * out) {
    const size_t nidx_row = (size_t) (st->cols / st->dim), dim = (size_t) st->dim;
    for (size_t r = 0; r < (size_t) st->rows; r++) {
        const float g = sr_stage_gain(st, r);
        float * o = out + r * (size_t) st->cols;
        for (size_t i = 0; i < nidx_row; i++) {
            const size_t v = sr_stage_index(st, r, i);
            const float * cb = st->cb32 + v * dim;
            for (size_t d = 0; d < dim; d++) o[i * dim + d] += cb[d] * g;
        }
    }
}

/* tools/vq-format/src/lib.rs:215-227: one running f32 sum over the row's
 * codewords times x, then acc[r] += s * g. */
void sr_stage_dot_row(const sr_stage * st, size_t r, const float * x, float * acc) {
    const size_t nidx_row = (size_t) (st->cols / st->dim), dim = (size_t) st->dim;
    const float g = sr_stage_gain(st, r);
    float s = 0.0f;
    for (size_t i = 0; i < nidx_row; i++) {
        const size_t v = sr_stage_index(st, r, i);
        const float * cb = st->cb32 + v * dim;
        for (size_t d = 0; d < dim; d++) s += cb[d] * x[i * dim + d];
    }
    acc[r] += s * g;
}

/* tools/vq-format/src/lib.rs:240-306 (Container::open), validation only. */
int sr_container_check(const uint8_t * buf, size_t len, int * nstages, size_t * per,
                       int * rows_o, int * cols_o, int * dim_o, int * nc_o, int * v3_o,
                       char * err, size_t errn) {
    if (len < 32 || memcmp(buf, "RQVQ", 4) != 0) { set_err(err, errn, "not an RQVQ container"); return -1; }
    const size_t dim = rd16(buf, 4), nc = rd16(buf, 6), ns = rd16(buf, 8);
    const size_t rows = rd32(buf, 12), cols = rd32(buf, 16);
    const uint64_t payload = rd64(buf, 24);
    if (dim == 0 || nc == 0 || ns == 0 || rows == 0 || cols == 0) {
        set_err(err, errn, "container header is inconsistent");
        return -1;
    }
    const int nbit = bits_for((int) nc);
    const int v3 = len >= 36 && memcmp(buf + 32, "DQV3", 4) == 0;
    if (v3 && nbit > 13) {
        char m[160];
        snprintf(m, sizeof m, "DQV3 carries 13 index bits, nc %zu needs %d; rewrite with --format v2", nc, nbit);
        set_err(err, errn, m);
        return -1;
    }
    const size_t nidx_row = cols / dim;
    size_t stride;
    if (v3) {
        const size_t mb = nbit < 12 ? (size_t) nbit : 12;
        const size_t mrow = (nidx_row * mb + 7) / 8;
        const size_t prow = nbit > 12 ? (nidx_row + 7) / 8 : 0;
        stride = 24 + nc * dim * 2 + rows * 2 + rows * (mrow + prow);
    } else {
        const size_t nidx = rows * nidx_row;
        const size_t ib = nbit == 8 ? nidx : (nidx * (size_t) nbit + 7) / 8 + 1;
        stride = 16 + nc * dim * 2 + rows * 2 + ib;
    }
    if (payload != (uint64_t) (ns * stride)) {
        char m[160];
        snprintf(m, sizeof m, "payload byte count says %llu, layout implies %zu",
                 (unsigned long long) payload, ns * stride);
        set_err(err, errn, m);
        return -1;
    }
    if (len != 32 + payload) {
        char m[160];
        snprintf(m, sizeof m, "file is %zu bytes, header and payload are %llu", len,
                 (unsigned long long) (32 + payload));
        set_err(err, errn, m);
        return -1;
    }
    for (size_t s = 0; s < ns; s++) {
        sr_stage st;
        if (sr_stage_open(buf + 32 + s * stride, stride, &st, err, errn)) return -1;
        const int bad = (size_t) st.rows != rows || (size_t) st.cols != cols || (size_t) st.dim != dim || (size_t) st.nc != nc;
        sr_stage_close(&st);
        if (bad) {
            char m[96];
            snprintf(m, sizeof m, "stage %zu disagrees with the container header", s);
            set_err(err, errn, m);
            return -1;
        }
    }
    if (nstages) *nstages = (int) ns;
    if (per) *per = stride;
    if (rows_o) *rows_o = (int) rows;
    if (cols_o) *cols_o = (int) cols;
    if (dim_o) *dim_o = (int) dim;
    if (nc_o) *nc_o = (int) nc;
    if (v3_o) *v3_o = v3;
    return 0;
}

/* tools/vq-format/src/lib.rs:309-315 (Container::decode). */
int sr_container_decode(const uint8_t * buf, size_t len, float * out, char * err, size_t errn) {
    int ns, rows, cols;
    size_t per;
    if (sr_container_check(buf, len, &ns, &per, &rows, &cols, NULL, NULL, NULL, err, errn)) return -1;
    memset(out, 0, (size_t) rows * (size_t) cols * sizeof(float));
    for (int s = 0; s < ns; s++) {
        sr_stage st;
        if (sr_stage_open(buf + 32 + (size_t) s * per, per, &st, err, errn)) return -1;
        sr_stage_add_into(&st, out);
        sr_stage_close(&st);
    }
    return 0;
}

/* ---- a minimal row-split worker pool: each thread takes a contiguous range
 * of rows, which leaves each row's arithmetic exactly as in the serial code. */
typedef struct {
    void (*fn)(void * ctx, size_t r0, size_t r1);
    void * ctx;
    size_t r0, r1;
} sr_job;

static void * sr_job_run(void * a) {
    sr_job * j = (sr_job *) a;
    j->fn(j->ctx, j->r0, j->r1);
    return NULL;
}

static void sr_parallel_rows(size_t rows, int nthreads, void (*fn)(void *, size_t, size_t), void * ctx) {
    if (nthreads <= 1 || rows < 2) { fn(ctx, 0, rows); return; }
    if ((size_t) nthreads > rows) nthreads = (int) rows;
    pthread_t th[256];
    sr_job jobs[256];
    if (nthreads > 256) nthreads = 256;
    for (int t = 0; t < nthreads; t++) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].r0 = rows * (size_t) t / (size_t) nthreads;
        jobs[t].r1 = rows * (size_t) (t + 1) / (size_t) nthreads;
    }
    int started = 0;
    for (int t = 1; t < nthreads; t++) {
        if (pthread_create(&th[t], NULL, sr_job_run, &jobs[t]) != 0) break;
        started = t;
    }
    sr_job_run(&jobs[0]);
    for (int t = 1; t <= started; t++) pthread_join(th[t], NULL);
    for (int t = started + 1; t < nthreads; t++) sr_job_run(&jobs[t]);
}

typedef struct {
    const sr_stage * st;
    const float * x;
    float * y;
} fused_ctx;

static void fused_rows(void * c, size_t r0, size_t r1) {
    fused_ctx * f = (fused_ctx *) c;
    for (size_t r = r0; r < r1; r++) sr_stage_dot_row(f->st, r, f->x, f->y);
}

/* tools/dqvq/src/main.rs:131-141: the fused gather+dot, stage by stage. */
int sr_container_gemv_fused(const uint8_t * buf, size_t len, const float * x, float * y,
                            int nthreads, char * err, size_t errn) {
    int ns, rows;
    size_t per;
    if (sr_container_check(buf, len, &ns, &per, &rows, NULL, NULL, NULL, NULL, err, errn)) return -1;
    memset(y, 0, (size_t) rows * sizeof(float));
    for (int s = 0; s < ns; s++) {
        sr_stage st;
        if (sr_stage_open(buf + 32 + (size_t) s * per, per, &st, err, errn)) return -1;
        fused_ctx c = { &st, x, y };
        sr_parallel_rows((size_t) rows, nthreads, fused_rows, &c);
        sr_stage_close(&st);
    }
    return 0;
}

/* tools/vq-runtime/src/model.rs:209-226: eight strided f32 accumulators over
 * the 8-aligned prefix, combined ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)), then the
 * scalar tail added in order. */
float sr_dot(const float * a, const float * b, size_t n) {
    float acc[8] = { 0, 0, 0, 0, 0, 0, 0, 0 };
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; k++) acc[k] += a[i + k] * b[i + k];
    float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

typedef struct {
    const float * W;
    size_t cols;
    const float * x;
    float * y;
    double * y64;
} mv_ctx;

static void mv_rows(void * c, size_t r0, size_t r1) {
    mv_ctx * m = (mv_ctx *) c;
    for (size_t r = r0; r < r1; r++) m->y[r] = sr_dot(m->W + r * m->cols, m->x, m->cols);
}

/* tools/vq-runtime/src/model.rs:228-234 (rayon one task per row). */
void sr_matvec(const float * W, size_t rows, size_t cols, const float * x, float * y, int nthreads) {
    mv_ctx c = { W, cols, x, y, NULL };
    sr_parallel_rows(rows, nthreads, mv_rows, &c);
}

static void mv64_rows(void * c, size_t r0, size_t r1) {
    mv_ctx * m = (mv_ctx *) c;
    for (size_t r = r0; r < r1; r++) {
        const float * w = m->W + r * m->cols;
        double s = 0.0;
        for (size_t k = 0; k < m->cols; k++) s += (double) w[k] * (double) m->x[k];
        m->y64[r] = s;
    }
}

/* tools/vq/gpu/decode-gpu.c:469-484: the gate's host matvec, accumulated in f64. */
void sr_matvec_f64(const float * W, size_t rows, size_t cols, const float * x, double * y, int nthreads) {
    mv_ctx c = { W, cols, x, NULL, y };
    sr_parallel_rows(rows, nthreads, mv64_rows, &c);
}

/* tools/vq/decode.c:107-125 (v2_stage_bytes / v3_stage_bytes). */
size_t sr_stage_bytes(int v3, int rows, int cols, int dim, int nc) {
    const int bits = bits_for(nc);
    const size_t nidx_row = (size_t) cols / (size_t) dim;
    if (v3) {
        const int mb = bits > 12 ? 12 : bits;
        const size_t mrow = (nidx_row * (size_t) mb + 7) / 8;
        const size_t prow = bits > 12 ? (nidx_row + 7) / 8 : 0;
        return 24 + (size_t) nc * dim * 2 + (size_t) rows * 2 + (size_t) rows * (mrow + prow);
    }
    const size_t nidx = (size_t) rows * nidx_row;
    const size_t idx = bits == 8 ? nidx : (nidx * (size_t) bits + 7) / 8 + 1;
    return 16 + (size_t) nc * dim * 2 + (size_t) rows * 2 + idx;
}

static void wr16(uint8_t * p, uint16_t v) { p[0] = (uint8_t) v; p[1] = (uint8_t) (v >> 8); }
static void wr32(uint8_t * p, uint32_t v) { for (int k = 0; k < 4; k++) p[k] = (uint8_t) (v >> (8 * k)); }

static void or_bits(uint8_t * base, size_t bitpos, uint32_t v, int nbits) {
    for (int k = 0; k < nbits; k++)
        if ((v >> k) & 1u) base[(bitpos + (size_t) k) >> 3] |= (uint8_t) (1u << ((bitpos + (size_t) k) & 7));
}

/* tools/vq/gpu/build-vq-gpu.c:71-111 (v3_pack): 24-byte header with flags =
 * (bits > 12) and 4 pad bytes, f16 codebook, f16 gains, then a row-local
 * LSB-first stream of min(bits, 12)-bit fields and, above 12 bits, a plane of
 * one bit per index. */
size_t sr_v3_pack(const uint16_t * cb, const uint32_t * idx, const uint16_t * gains,
                  int rows, int cols, int dim, int nc, uint8_t * out) {
    uint8_t * p = out;
    const int bits = bits_for(nc);
    memcpy(p, "DQV3", 4);
    wr16(p + 4, (uint16_t) dim);
    wr16(p + 6, (uint16_t) nc);
    wr32(p + 8, (uint32_t) rows);
    wr32(p + 12, (uint32_t) cols);
    wr32(p + 16, bits > 12 ? 1u : 0u);
    wr32(p + 20, 0u);
    p += 24;
    for (size_t i = 0; i < (size_t) nc * dim; i++, p += 2) wr16(p, cb[i]);
    for (int r = 0; r < rows; r++, p += 2) wr16(p, gains[r]);
    const int mb = bits > 12 ? 12 : bits;
    const size_t nidx_row = (size_t) cols / (size_t) dim;
    const size_t mrow = (nidx_row * (size_t) mb + 7) / 8;
    const size_t prow = bits > 12 ? (nidx_row + 7) / 8 : 0;
    uint8_t * mainp = p;
    uint8_t * plane = p + (size_t) rows * mrow;
    memset(mainp, 0, (size_t) rows * (mrow + prow));
    for (int r = 0; r < rows; r++)
        for (size_t i = 0; i < nidx_row; i++) {
            const uint32_t v = idx[(size_t) r * nidx_row + i];
            or_bits(mainp + (size_t) r * mrow, i * (size_t) mb, v & ((1u << mb) - 1u), mb);
            if (prow) or_bits(plane + (size_t) r * prow, i, (v >> 12) & 1u, 1);
        }
    return (size_t) (plane + (size_t) rows * prow - out);
}

/* tools/vq/vendor/vq_qc.h:241-264 (vq_pack): 16-byte header, f16 codebook and
 * gains, then one LSB-first stream across the matrix (a byte per index at 8
 * bits, else ceil(bits*n/8)+1 bytes with the trailing guard byte). */
size_t sr_vq_pack(const uint16_t * cb, const uint32_t * idx, const uint16_t * gains,
                  int rows, int cols, int dim, int nc, uint8_t * out) {
    uint8_t * p = out;
    memcpy(p, "DQVQ", 4);
    wr16(p + 4, (uint16_t) dim);
    wr16(p + 6, (uint16_t) nc);
    wr32(p + 8, (uint32_t) rows);
    wr32(p + 12, (uint32_t) cols);
    p += 16;
    for (size_t i = 0; i < (size_t) nc * dim; i++, p += 2) wr16(p, cb[i]);
    for (int r = 0; r < rows; r++, p += 2) wr16(p, gains[r]);
    const size_t nidx = (size_t) rows * (size_t) cols / (size_t) dim;
    const int bits = bits_for(nc);
    if (bits == 8) {
        for (size_t i = 0; i < nidx; i++) *p++ = (uint8_t) idx[i];
        return (size_t) (p - out);
    }
    const size_t nb = (nidx * (size_t) bits + 7) / 8 + 1;
    memset(p, 0, nb);
    for (size_t i = 0; i < nidx; i++) or_bits(p, i * (size_t) bits, idx[i] & ((1u << bits) - 1u), bits);
    return (size_t) (p + nb - out);
}

/* ggml's published dequantize_row_q6_K (llama.cpp ggml-quants.c, the copy the
 * reference pins at fa3645feb5f4 and calls from tools/vq/quant_err.c:38-43;
 * absent from the reference tree). Each 128-weight half reads 64 ql bytes, 32
 * qh bytes and 8 scales: weight l (0..31) of quarter k takes the low (k = 0, 1)
 * or high (k = 2, 3) nibble of ql[l + 32*(k & 1)] and bits 2k..2k+1 of qh[l],
 * minus 32, times d * scales[l/16 + 2k]. */
void sr_q6k_dequant(const uint8_t * blocks, size_t nblocks, float * out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t * blk = blocks + b * 210;
        const float d = sr_f16(rd16(blk, 208));
        for (int half = 0; half < 2; half++) {
            const uint8_t * ql = blk + 64 * half;
            const uint8_t * qh = blk + 128 + 32 * half;
            const int8_t * sc = (const int8_t *) (blk + 192) + 8 * half;
            float * y = out + b * 256 + 128 * half;
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = (int) ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int) ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int) ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * (float) sc[is + 0] * (float) q1;
                y[l + 32] = d * (float) sc[is + 2] * (float) q2;
                y[l + 64] = d * (float) sc[is + 4] * (float) q3;
                y[l + 96] = d * (float) sc[is + 6] * (float) q4;
            }
        }
    }
}

/* ggml's published dequantize_row_q8_0: y = qs[j] * d (type 8, 34 B / 32,
 * tools/dspark/src/gguf.rs:201; call site tools/vq/quant_err.c:32-37). */
void sr_q8_0_dequant(const uint8_t * blocks, size_t nblocks, float * out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t * blk = blocks + b * 34;
        const float d = sr_f16(rd16(blk, 0));
        const int8_t * qs = (const int8_t *) (blk + 2);
        for (int j = 0; j < 32; j++) out[b * 32 + (size_t) j] = (float) qs[j] * d;
    }
}

typedef struct {
    const uint8_t * blocks;
    size_t cols;
    const float * x;
    float * y;
    int q6;
} kq_ctx;

static void kq_rows(void * c, size_t r0, size_t r1) {
    kq_ctx * k = (kq_ctx *) c;
    float * row = (float *) malloc(k->cols * sizeof(float));
    if (!row) return;
    const size_t bpr = k->q6 ? k->cols / 256 : k->cols / 32;
    const size_t bb = k->q6 ? 210 : 34;
    for (size_t r = r0; r < r1; r++) {
        if (k->q6) sr_q6k_dequant(k->blocks + r * bpr * bb, bpr, row);
        else       sr_q8_0_dequant(k->blocks + r * bpr * bb, bpr, row);
        k->y[r] = sr_dot(row, k->x, k->cols);
    }
    free(row);
}

/* Decode-to-f32 then the runtime's dot (model.rs:209-234), row by row. */
void sr_q6k_matvec(const uint8_t * blocks, size_t rows, size_t cols, const float * x, float * y, int nthreads) {
    kq_ctx c = { blocks, cols, x, y, 1 };
    sr_parallel_rows(rows, nthreads, kq_rows, &c);
}

void sr_q8_0_matvec(const uint8_t * blocks, size_t rows, size_t cols, const float * x, float * y, int nthreads) {
    kq_ctx c = { blocks, cols, x, y, 0 };
    sr_parallel_rows(rows, nthreads, kq_rows, &c);
}

int sr_hardware_threads(void) {
    const long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int) n : 1;
}
