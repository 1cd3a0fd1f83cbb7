/* abi.cpp — the extern "C" surface declared in include/sparkmv.h.
 *
 * The vqg_* functions keep the reference's C-ABI (tools/vq/gpu/decode-gpu.cu:765-1140):
 * one stage payload per call, f32 x and y, y accumulates, the default stream,
 * 0 / -1 returns with the message in vqg_decode_error(). They route to the
 * same kernels as the sparkmv_* functions, which add bf16 x, N columns, whole
 * containers, several matrices per launch and explicit streams.
 */
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/sparkmv.h"
#include "common.h"
#include "host/vq_format.hpp"
#include "kq.h"
#include "prefill.h"
#include "vq.h"

namespace sparkmv {

thread_local LaunchEvents g_launch_events;


static char g_err[512];

void set_error(const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

int fail_hip(const char * what, hipError_t e) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return -1;
}

int cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

static int width_ok(int v3, int nc) {
    if (v3 && bits_for(nc) > 13) {
        set_error("DQV3 carries 13 index bits, nc %d needs %d", nc, bits_for(nc));
        return 0;
    }
    return 1;
}

static int geometry_ok(int dim, int nc, int rows, int cols) {
    if (dim <= 0 || nc <= 0 || rows <= 0 || cols <= 0 || cols % dim) {
        set_error("geometry dim %d, nc %d, %d x %d is inconsistent", dim, nc, rows, cols);
        return 0;
    }
    return 1;
}

/* Time `iters` runs of `launch` on the default stream with events; best ms. */
template <class F>
static int timed(F launch, int iters, double * ms) {
    hipEvent_t a, b;
    hipError_t e;
    if ((e = hipEventCreate(&a)) != hipSuccess) return fail_hip("event create", e);
    if ((e = hipEventCreate(&b)) != hipSuccess) { hipEventDestroy(a); return fail_hip("event create", e); }
    float best = 1e30f;
    int rc = 0;
    for (int it = 0; it < (iters > 0 ? iters : 1); it++) {
        hipEventRecord(a, 0);
        if (launch()) { rc = -1; break; }
        hipEventRecord(b, 0);
        if ((e = hipEventSynchronize(b)) != hipSuccess) { rc = fail_hip("timed launch", e); break; }
        float t = 0;
        hipEventElapsedTime(&t, a, b);
        if (t < best) best = t;
    }
    hipEventDestroy(a);
    hipEventDestroy(b);
    if (!rc && ms) *ms = best;
    return rc;
}

/* The reference's DQV3 block-kernel preconditions (decode-gpu.cu:62-64): a
 * 12-bit main stream, whole 32-index groups, 4-byte aligned row streams. */
static int v3_blk_ok(const Layout & L) {
    return L.v3 && L.nbit >= 12 && L.nidx_row % 32 == 0 && L.mrow % 4 == 0 && L.stream_off % 4 == 0;
}

/* LDS a workgroup may hold (the variant-0 codebook kernel's bound, as the
 * reference's smem_max() bounds its shared-memory kernel) */
static const size_t kLdsLimit = 160 * 1024;

/* A reference variant number (decode-gpu.cu:788-797, :808-833, :865-906) as
 * the kernel that runs it here (VqCall's numbering: 1 the generic wave
 * kernel, 2 the wave kernel with the codebook in LDS, 3 the MFMA block
 * kernel, 0 the fastest that takes the call). `timed` is vqg_gemv_t /
 * vqg_gemv, whose variant 0 is the shared-codebook kernel; the launch forms
 * read 0 as the reference's pick (3 when the block kernel's preconditions
 * hold, else 2 for dim 4, else 1). Variant 2 is the dim-4 path (the
 * fastest dim-4 kernel that takes the geometry); 3 is the block path, which
 * here is the MFMA kernel for dim 4 and the wave kernel for other dims. */
static int map_variant(const Layout & L, int variant, int timed) {
    if (variant == 0 && timed) return 2;
    if (variant == 0) variant = v3_blk_ok(L) ? 3 : (L.dim == 4 ? 2 : 1);
    switch (variant) {
        case 1: return 1;
        case 2: return L.dim == 4 ? 0 : 1;
        case 3: return L.dim == 4 ? 0 : ((size_t) L.nc * L.dim * 2 <= kLdsLimit ? 2 : 1);
        default: return -1;
    }
}

static int one_stage_gemv(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * x,
                          float * y, int variant, int threads, int timed = 0) {
    if (!width_ok(v3, nc) || !geometry_ok(dim, nc, rows, cols)) return -1;
    if (variant < 0 || variant > 3) { set_error("unknown gemv variant %d", variant); return -1; }
    if (!payload) { set_error("payload is null"); return -1; }
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    if (variant == 3 && !v3_blk_ok(L)) { set_error("the DQV3 block kernel does not take this geometry"); return -1; }
    if (variant == 0 && timed && (size_t) nc * dim * 2 > kLdsLimit) {
        set_error("a codebook of %d x %d does not fit the shared-codebook kernel", nc, dim);
        return -1;
    }
    /* the reference takes warp multiples (32) up to 1024; a wave here is 64
     * lanes, so a width rounds up to whole waves (it only sets how many
     * row-waves share a workgroup, never the arithmetic); the shared-
     * codebook kernel runs 256 wide, as the reference's does */
    if (variant == 0 && timed) threads = 256;
    else if (threads) {
        if (threads < 32 || threads > 1024 || threads % 32) {
            set_error("gemv launch width %d is not a warp multiple up to 1024", threads);
            return -1;
        }
        threads = (threads + 63) & ~63;
    }
    variant = map_variant(L, variant, timed);
    VqMatDesc m;
    memset(&m, 0, sizeof m);
    m.stages[0] = payload;
    m.y = y;
    m.rows = rows;
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = dim; c.nc = nc; c.cols = cols; c.v3 = v3; c.nst = 1;
    c.mats = &m; c.nmat = 1;
    c.x = x; c.ldx = cols; c.xf32 = 1; c.ncol = 1; c.ldy = rows; c.accumulate = 1;
    c.stream = 0;
    c.variant = variant;
    c.threads = threads;
    return vq_launch(c);
}

}  // namespace sparkmv

using namespace sparkmv;

extern "C" {

const char * vqg_decode_error(void) { return g_err; }

int vqg_device_name(char * out, int n) {
    if (!out || n <= 0) { set_error("device name buffer is empty"); return -1; }
    hipDeviceProp_t p;
    memset(&p, 0, sizeof p);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return fail_hip("device properties", e);
    snprintf(out, (size_t) n, "%s (%s)", p.name, p.gcnArchName);
    return 0;
}

int vqg_driver_version(void) {
    int v = 0;
    if (hipDriverGetVersion(&v) != hipSuccess) return -1;
    return v;
}

/* The reference's readiness rules (decode-gpu.cu:788-797): 3 when the block
 * kernel's preconditions hold, 2 for dim 4, 1 always, 0 when the codebook
 * fits the shared-codebook kernel. A geometry the launch refuses (cols not a
 * multiple of dim, a DQV3 codebook past 13 bits, empty) is ready for no
 * variant. */
int vqg_gemv_ready(int dim, int nc, int rows, int cols, int v3, int variant) {
    if (dim <= 0 || nc <= 0 || rows <= 0 || cols <= 0 || cols % dim) return 0;
    if (v3 && bits_for(nc) > 13) return 0;
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    switch (variant) {
        case 3: return v3_blk_ok(L);
        case 2: return dim == 4;
        case 1: return 1;
        case 0: return (size_t) nc * dim * 2 <= kLdsLimit;
        default: return 0;
    }
}

}  // extern "C"

namespace sparkmv {

int profile_gemv_pick(const void * profile, int dim, int nc, int rows, int cols, int v3, int * variant, int * threads) {
    sparkmv_profile_entry e;
    memset(&e, 0, sizeof e);
    if (sparkmv_profile_find(profile, 0, dim, nc, rows, cols, v3, &e) != 0) return 0;
    if (e.variant < 0 || e.variant > 3 || !vqg_gemv_ready(dim, nc, rows, cols, v3, e.variant) || e.threads < 32 ||
        e.threads > 1024 || e.threads % 32)
        return -1;
    *variant = map_variant(make_layout(dim, nc, rows, cols, v3), e.variant, 0);
    *threads = (e.threads + 63) & ~63;
    return 1;
}

}  // namespace sparkmv

extern "C" {

int sparkmv_vq_gemv_ready(int dim, int nc, int rows, int cols, int v3, int variant) {
    return vq_variant_ready(dim, nc, rows, cols, v3, variant);
}

int vqg_gemv_t(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * x, float * y,
               int variant, int threads, int iters, double * ms) {
    if (!width_ok(v3, nc)) return -1;
    if (rows <= 0 || cols <= 0) { set_error("gemv needs a non-empty matrix"); return -1; }
    return timed([&] { return one_stage_gemv(payload, dim, nc, rows, cols, v3, x, y, variant, threads, 1); }, iters,
                 ms);
}

int vqg_gemv(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * x, float * y,
             int variant, int iters, double * ms) {
    return vqg_gemv_t(payload, dim, nc, rows, cols, v3, x, y, variant, 256, iters, ms);
}

int vqg_gemv_launch_t(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * x, float * y,
                      int variant, int threads) {
    if (!width_ok(v3, nc)) return -1;
    if (rows <= 0 || cols <= 0) { set_error("gemv needs a non-empty matrix"); return -1; }
    return one_stage_gemv(payload, dim, nc, rows, cols, v3, x, y, variant, threads);
}

int vqg_gemv_launch(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * x, float * y,
                    int variant) {
    return vqg_gemv_launch_t(payload, dim, nc, rows, cols, v3, x, y, variant, 256);
}

int vqg_dequant(const void * payload, int dim, int nc, int rows, int cols, int v3, float * out, int iters,
                double * ms) {
    if (!width_ok(v3, nc) || !geometry_ok(dim, nc, rows, cols)) return -1;
    if (!payload || !out) { set_error("null pointer passed to dequant"); return -1; }
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    return timed([&] { return vq_dequant_launch(payload, L, out, 1, 0); }, iters, ms);
}

int vqg_row_dequant(const void * payload, int dim, int nc, int rows, int cols, int v3, int row, float * out) {
    if (!width_ok(v3, nc) || !geometry_ok(dim, nc, rows, cols)) return -1;
    if (row < 0 || row >= rows) { set_error("row %d is outside %d", row, rows); return -1; }
    if (!payload || !out) { set_error("null pointer passed to row dequant"); return -1; }
    return vq_row_dequant_launch(payload, make_layout(dim, nc, rows, cols, v3), row, out, 0);
}

/* ---- prefill (reference layout: xT [cols][ntok], y [ntok][rows]) ----
 * Variants are numbered as the reference numbers them
 * (tools/vq/gpu/decode-gpu.cu:995-1004, :1017-1025): 1 and 2 are its tiled
 * f16 GEMMs (codebook through L1 / in shared memory), 3 its legacy
 * one-thread-per-output kernel, 0 picks 1 when the geometry allows it, else 3.
 * Readiness follows the reference's rules, so its runtime chooses the same
 * variant it would on CUDA (vq-model-gpu.cu:296-297). Here variants 1 and 2
 * both run the MFMA GEMM when it takes the call (dim 4, columns a multiple
 * of 128, 16-byte aligned xT with ntok a multiple of 4) and the
 * one-thread-per-output kernel otherwise; a tile (bn, bk) of the tuner's
 * table is accepted and leaves the gfx950 kernel's 128 x 128 x 64 tile as is. */

struct PreCfg { int bn, bk; };
static const PreCfg k_pre_cfg[] = { { 64, 64 }, { 128, 64 }, { 256, 64 } };
static const int k_pre_ncfg = (int) (sizeof k_pre_cfg / sizeof k_pre_cfg[0]);

/* the tiled kernels' geometry rule, decode-gpu.cu:527-530 */
static int pre_ok(const Layout & L, int bk) {
    return L.v3 && (L.dim == 4 || L.dim == 8) && L.rows > 0 && L.cols > 0 && L.nbit >= 12 && bk > 0
        && L.cols % bk == 0 && L.mrow % 4 == 0 && L.stream_off % 4 == 0;
}

int vqg_prefill_ready(int dim, int nc, int rows, int cols, int v3, int variant) {
    if (dim <= 0 || nc <= 0 || rows <= 0 || cols <= 0 || cols % dim) return 0;
    if (v3 && bits_for(nc) > 13) return 0;
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    switch (variant) {
        case 0: return 1;
        case 1: case 2: return pre_ok(L, 64);
        case 3: return L.nidx_row * 2 <= 64 * 1024;
        default: return 0;
    }
}

int vqg_prefill_cfg_count(void) { return k_pre_ncfg; }

int vqg_prefill_cfg(int idx, int * bn, int * bk) {
    if (idx < 0 || idx >= k_pre_ncfg || !bn || !bk) return -1;
    *bn = k_pre_cfg[idx].bn;
    *bk = k_pre_cfg[idx].bk;
    return 0;
}

int vqg_prefill_cfg_ready(int dim, int nc, int rows, int cols, int v3, int bn, int bk, int variant) {
    (void) bn;
    if (variant == 3) return vqg_prefill_ready(dim, nc, rows, cols, v3, 3);
    if (variant != 1 && variant != 2) return 0;
    if (!vqg_prefill_ready(dim, nc, rows, cols, v3, variant)) return 0;
    return pre_ok(make_layout(dim, nc, rows, cols, v3), bk);
}

static int prefill_ref_layout(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * xT,
                              int ntok, float * y, int variant) {
    if (!width_ok(v3, nc) || !geometry_ok(dim, nc, rows, cols)) return -1;
    if (ntok <= 0) { set_error("prefill needs at least one token"); return -1; }
    if (!payload || !xT || !y) { set_error("null pointer passed to prefill"); return -1; }
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    if (variant == 0) variant = pre_ok(L, 64) ? 1 : 3;
    if (variant < 1 || variant > 3) { set_error("unknown prefill variant %d", variant); return -1; }
    if (variant != 3 && !pre_ok(L, 64)) {
        set_error("prefill variant %d does not take this geometry", variant);
        return -1;
    }
    const void * st[1] = { payload };
    if (variant != 3 && prefill_mfma_ready(L, 1, xT, 1, ntok, 1, ntok))
        return prefill_mfma_launch(st, 1, L, xT, 1, ntok, 1, ntok, y, rows, 1, 0);
    if (variant == 3 && !vqg_prefill_ready(dim, nc, rows, cols, v3, 3)) {
        set_error("the legacy prefill kernel stages %zu bytes of indices per row, more than it holds", L.nidx_row * 2);
        return -1;
    }
    return prefill_simple_launch(st, 1, L, xT, 1, 1, (size_t) ntok, ntok, y, rows, 1, 0);
}

int vqg_prefill(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * xT, int ntok,
                float * y, int iters, double * ms, int variant) {
    return timed([&] { return prefill_ref_layout(payload, dim, nc, rows, cols, v3, xT, ntok, y, variant); }, iters, ms);
}

int vqg_prefill_tile(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * xT, int ntok,
                     float * y, int iters, double * ms, int bn, int bk, int variant) {
    if (!vqg_prefill_cfg_ready(dim, nc, rows, cols, v3, bn, bk, variant)) {
        set_error("tile %dx%d with variant %d does not fit this geometry", bn, bk, variant);
        return -1;
    }
    return vqg_prefill(payload, dim, nc, rows, cols, v3, xT, ntok, y, iters, ms, variant);
}

int vqg_prefill_launch(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * xT, int ntok,
                       float * y, int variant) {
    return prefill_ref_layout(payload, dim, nc, rows, cols, v3, xT, ntok, y, variant);
}

int vqg_prefill_launch_tile(const void * payload, int dim, int nc, int rows, int cols, int v3, const float * xT,
                            int ntok, float * y, int bn, int bk, int variant) {
    if (!vqg_prefill_cfg_ready(dim, nc, rows, cols, v3, bn, bk, variant)) {
        set_error("tile %dx%d with variant %d does not fit this geometry", bn, bk, variant);
        return -1;
    }
    return prefill_ref_layout(payload, dim, nc, rows, cols, v3, xT, ntok, y, variant);
}

int vqg_gemv_f32(const float * w, const float * x, float * y, int rows, int cols, int iters, double * ms) {
    if (!w || !x || !y || rows <= 0 || cols <= 0) { set_error("gemv f32 needs a non-empty matrix and pointers"); return -1; }
    return timed([&] { return f32_gemv_launch(w, x, y, rows, cols, 0); }, iters, ms);
}

/* ------------------------------ sparkmv_* --------------------------------- */

int sparkmv_container_open(const void * bytes, size_t len, sparkmv_container_info * info) {
    if (!bytes || !info) { set_error("null pointer passed to container open"); return -1; }
    fmt::ContainerView c;
    std::string err;
    if (!fmt::open_container((const uint8_t *) bytes, len, c, err)) {
        set_error("%s", err.c_str());
        return -1;
    }
    if (c.stages.size() > 4) { set_error("%zu stages: at most 4 are supported", c.stages.size()); return -1; }
    memset(info, 0, sizeof *info);
    info->dim = c.dim; info->nc = c.nc; info->nstages = (int) c.stages.size();
    info->rows = c.rows; info->cols = c.cols; info->v3 = c.v3; info->nbit = c.nbit;
    info->payload_bytes = c.payload;
    info->stage_bytes = c.stride;
    for (size_t s = 0; s < c.stages.size(); s++) info->stage_offset[s] = 32 + s * c.stride;
    return 0;
}

size_t sparkmv_stage_bytes(int v3, int rows, int cols, int dim, int nc) {
    if (dim <= 0 || nc <= 0 || rows <= 0 || cols <= 0 || cols % dim) return 0;
    return make_layout(dim, nc, rows, cols, v3).bytes;
}

int sparkmv_vq_gemv_multi(const sparkmv_vq_matrix * mats, int nmat, int nstages, int dim, int nc, int cols, int v3,
                          const void * x, int x_dtype, int ldx, int ncols, int ldy, int accumulate, int variant,
                          void * stream) {
    if (!mats || nmat < 1 || nmat > kMaxMats) { set_error("matrix count %d is outside 1..%d", nmat, kMaxMats); return -1; }
    if (x_dtype != SPARKMV_X_BF16 && x_dtype != SPARKMV_X_F32) { set_error("unknown x dtype %d", x_dtype); return -1; }
    if (nstages < 1 || nstages > kMaxStages) { set_error("stage count %d is outside 1..%d", nstages, kMaxStages); return -1; }
    VqMatDesc m[kMaxMats];
    memset(m, 0, sizeof m);
    for (int i = 0; i < nmat; i++) {
        for (int s = 0; s < nstages; s++) m[i].stages[s] = mats[i].stages[s];
        m[i].y = mats[i].y;
        m[i].rows = mats[i].rows;
        if (!geometry_ok(dim, nc, mats[i].rows, cols)) return -1;
    }
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = dim; c.nc = nc; c.cols = cols; c.v3 = v3; c.nst = nstages;
    c.mats = m; c.nmat = nmat;
    c.x = x; c.ldx = ldx; c.xf32 = x_dtype == SPARKMV_X_F32; c.ncol = ncols; c.ldy = ldy;
    c.accumulate = accumulate ? 1 : 0;
    c.stream = (hipStream_t) stream;
    c.variant = variant;
    return vq_launch(c);
}

int sparkmv_vq_gemv_norm(const sparkmv_vq_matrix * mats, int nmat, int nstages, int dim, int nc, int cols, int v3,
                         const float * h, const float * norm_w, float eps, uint16_t * x_out, int accumulate,
                         void * stream) {
    if (!mats || nmat < 1 || nmat > 4) { set_error("matrix count %d is outside 1..4", nmat); return -1; }
    if (nstages < 1 || nstages > 2) { set_error("the fused norm takes 1 or 2 stages, not %d", nstages); return -1; }
    if (!h || !norm_w) { set_error("h or the norm weight is null"); return -1; }
    if (!(eps > 0.0f)) { set_error("eps must be positive"); return -1; }
    VqMatDesc m[4];
    memset(m, 0, sizeof m);
    for (int i = 0; i < nmat; i++) {
        for (int s = 0; s < nstages; s++) m[i].stages[s] = mats[i].stages[s];
        m[i].y = mats[i].y;
        m[i].rows = mats[i].rows;
        if (!geometry_ok(dim, nc, mats[i].rows, cols)) return -1;
    }
    VqCall c;
    memset(&c, 0, sizeof c);
    c.dim = dim; c.nc = nc; c.cols = cols; c.v3 = v3; c.nst = nstages;
    c.mats = m; c.nmat = nmat;
    c.x = h; c.ldx = cols; c.xf32 = 1; c.ncol = 1; c.ldy = mats[0].rows;
    c.accumulate = accumulate ? 1 : 0;
    c.stream = (hipStream_t) stream;
    const int rc = vq_norm_launch(c, norm_w, eps, x_out);
    if (rc == 1) {
        set_error("the fused-norm kernel does not take this call (it needs DQV3 dim 4 with an even codebook, "
                  "columns a multiple of 128 that one workgroup stages whole, 16-byte aligned h and norm weight, "
                  "an 8-byte aligned x_out and 4-byte aligned stages): run the norm, then "
                  "sparkmv_vq_gemv_multi");
        return -1;
    }
    return rc;
}

int sparkmv_vq_gemv(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                    const void * x, int x_dtype, int ldx, int ncols, float * y, int ldy, int accumulate, int variant,
                    void * stream) {
    if (!stages) { set_error("stage pointer array is null"); return -1; }
    if (nstages < 1 || nstages > kMaxStages) { set_error("stage count %d is outside 1..%d", nstages, kMaxStages); return -1; }
    sparkmv_vq_matrix m;
    memset(&m, 0, sizeof m);
    for (int s = 0; s < nstages; s++) m.stages[s] = stages[s];
    m.y = y;
    m.rows = rows;
    return sparkmv_vq_gemv_multi(&m, 1, nstages, dim, nc, cols, v3, x, x_dtype, ldx, ncols, ldy, accumulate, variant,
                                 stream);
}

int sparkmv_vq_dequant(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                       float * out, int accumulate, void * stream) {
    if (!stages || !out) { set_error("null pointer passed to dequant"); return -1; }
    if (nstages < 1 || nstages > kMaxStages) { set_error("stage count %d is outside 1..%d", nstages, kMaxStages); return -1; }
    if (!width_ok(v3, nc) || !geometry_ok(dim, nc, rows, cols)) return -1;
    hipStream_t s = (hipStream_t) stream;
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    for (int i = 0; i < nstages; i++)
        if (!stages[i]) { set_error("stage %d payload is null", i); return -1; }
    for (int i = 0; i < nstages; i++)
        if (vq_dequant_launch(stages[i], L, out, i > 0 || accumulate, s)) return -1;
    return 0;
}

int sparkmv_q6k_gemv(const void * blocks, int rows, int cols, const void * x, int x_dtype, int ldx, int ncols,
                     float * y, int ldy, int accumulate, void * stream) {
    if (x_dtype != SPARKMV_X_BF16 && x_dtype != SPARKMV_X_F32) { set_error("unknown x dtype %d", x_dtype); return -1; }
    return kq_gemv_launch(6, blocks, rows, cols, x, x_dtype == SPARKMV_X_F32, ldx, ncols, y, ldy, accumulate ? 1 : 0,
                          (hipStream_t) stream);
}

int sparkmv_q8_0_gemv(const void * blocks, int rows, int cols, const void * x, int x_dtype, int ldx, int ncols,
                      float * y, int ldy, int accumulate, void * stream) {
    if (x_dtype != SPARKMV_X_BF16 && x_dtype != SPARKMV_X_F32) { set_error("unknown x dtype %d", x_dtype); return -1; }
    return kq_gemv_launch(8, blocks, rows, cols, x, x_dtype == SPARKMV_X_F32, ldx, ncols, y, ldy, accumulate ? 1 : 0,
                          (hipStream_t) stream);
}

int sparkmv_q6k_dequant(const void * blocks, int rows, int cols, float * out, void * stream) {
    return kq_dequant_launch(6, blocks, rows, cols, out, (hipStream_t) stream);
}

int sparkmv_q8_0_dequant(const void * blocks, int rows, int cols, float * out, void * stream) {
    return kq_dequant_launch(8, blocks, rows, cols, out, (hipStream_t) stream);
}

static int vq_prefill_impl(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                           const void * x, int x_dtype, int ldx, int ntok, float * y, int ldy, int accumulate,
                           void * stream, int noalloc) {
    if (!stages || !x || !y) { set_error("null pointer passed to prefill"); return -1; }
    if (x_dtype != SPARKMV_X_BF16 && x_dtype != SPARKMV_X_F32) { set_error("unknown x dtype %d", x_dtype); return -1; }
    if (nstages < 1 || nstages > kMaxStages) { set_error("stage count %d is outside 1..%d", nstages, kMaxStages); return -1; }
    if (ntok < 1) { set_error("prefill needs at least one token, not %d", ntok); return -1; }
    if (!width_ok(v3, nc) || !geometry_ok(dim, nc, rows, cols)) return -1;
    if (ldx < cols || ldy < rows) { set_error("ldx/ldy below the matrix extent"); return -1; }
    for (int i = 0; i < nstages; i++)
        if (!stages[i]) { set_error("stage %d payload is null", i); return -1; }
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    const int xf32 = x_dtype == SPARKMV_X_F32;
    void * ws = nullptr;
    if (noalloc && prefill_scratch(&ws)) return -1;
    if (prefill_mfma_ready(L, nstages < 2 ? nstages : 2, x, xf32, ldx, 0, ntok)) {
        /* the matrix cores, two stages per launch; later pairs accumulate */
        for (int s0 = 0; s0 < nstages; s0 += 2) {
            const int n = nstages - s0 < 2 ? nstages - s0 : 2;
            if (prefill_mfma_launch(stages + s0, n, L, x, xf32, ldx, 0, ntok, y, ldy, accumulate || s0 > 0,
                                    (hipStream_t) stream, ws))
                return -1;
        }
        return 0;
    }
    return prefill_simple_launch(stages, nstages, L, x, xf32, (size_t) ldx, 1, ntok, y, ldy, accumulate ? 1 : 0,
                                 (hipStream_t) stream);
}

int sparkmv_vq_prefill(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                       const void * x, int x_dtype, int ldx, int ntok, float * y, int ldy, int accumulate,
                       void * stream) {
    return vq_prefill_impl(stages, nstages, dim, nc, rows, cols, v3, x, x_dtype, ldx, ntok, y, ldy, accumulate,
                           stream, 0);
}

int sparkmv_vq_prefill_noalloc(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                               const void * x, int x_dtype, int ldx, int ntok, float * y, int ldy, int accumulate,
                               void * stream) {
    return vq_prefill_impl(stages, nstages, dim, nc, rows, cols, v3, x, x_dtype, ldx, ntok, y, ldy, accumulate,
                           stream, 1);
}

int sparkmv_prefill_fold(int on) {
    if (on < 0) return prefill_fold_on();
    return prefill_fold_set(on);
}

}  // extern "C"
