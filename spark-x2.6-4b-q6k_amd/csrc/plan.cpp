/* plan.cpp — a recorded chain of matvec launches (the per-token decode set)
 * that is issued eagerly or replayed as one HIP graph.
 *
 * The reference's GPU runtime issues its per-token matvecs one launch at a
 * time from the host (tools/vq/gpu/vq-model-gpu.cu:776-835, about 218 launches
 * per token). A plan records the same chain once — every VQ matvec group and
 * the tied Q8_0/Q6_K head, each with its device pointers — so a token costs
 * one graph launch. Ops run in record order on one stream; each op is a
 * single kernel launch, and no op clears memory with hipMemsetAsync (outputs
 * are written with accumulate = 0), so the chain is safe to capture.
 */
#include <hip/hip_runtime.h>
#include <string.h>

#include <utility>
#include <vector>

#include "../../include/sparkmv.h"
#include "common.h"
#include "kq.h"
#include "vq.h"

namespace sparkmv {

struct PlanOp {
    int kind;   /* 0 VQ group, 6 Q6_K, 8 Q8_0 */
    VqCall vq;
    std::vector<VqMatDesc> mats;
    const void * blocks;
    int rows, cols, xf32, ldx, ncol, ldy, accumulate;
    const void * x;
    float * y;
};

struct Plan {
    std::vector<PlanOp> ops;
    std::vector<void *> slots;   /* each several-column op's shared-tile words */
    std::vector<std::pair<void *, size_t>> unzeroed;   /* slot words not yet cleared (pointer, bytes) */
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

/* Clear the slot words added since the last run, in stream order ahead of
 * the ops that use them (outside any capture). Returns the number cleared. */
static int zero_slots(Plan * p, hipStream_t s, int * cleared) {
    *cleared = 0;
    for (auto & q : p->unzeroed) {
        hipError_t e = hipMemsetAsync(q.first, 0, q.second, s);
        if (e != hipSuccess) return fail_hip("plan shared-tile words", e);
        (*cleared)++;
    }
    p->unzeroed.clear();
    return 0;
}

static int run_op(PlanOp & op, hipStream_t s) {
    if (op.kind == 0) {
        op.vq.mats = op.mats.data();
        op.vq.stream = s;
        return vq_launch(op.vq);
    }
    return kq_gemv_launch(op.kind, op.blocks, op.rows, op.cols, op.x, op.xf32, op.ldx, op.ncol, op.y, op.ldy,
                          op.accumulate, s);
}

static void drop_graph(Plan * p) {
    if (p->exec) hipGraphExecDestroy(p->exec);
    if (p->graph) hipGraphDestroy(p->graph);
    p->exec = nullptr;
    p->graph = nullptr;
}

}  // namespace sparkmv

using namespace sparkmv;

extern "C" {

void * sparkmv_plan_create(void) { return new Plan(); }

void sparkmv_plan_destroy(void * plan) {
    Plan * p = (Plan *) plan;
    if (!p) return;
    drop_graph(p);
    for (void * q : p->slots) hipFree(q);
    delete p;
}

int sparkmv_plan_size(void * plan) { return plan ? (int) ((Plan *) plan)->ops.size() : -1; }

int sparkmv_plan_add_vq(void * plan, const sparkmv_vq_matrix * mats, int nmat, int nstages, int dim, int nc, int cols,
                        int v3, const void * x, int x_dtype, int ldx, int ncols, int ldy, int accumulate,
                        int variant) {
    Plan * p = (Plan *) plan;
    if (!p || !mats) { set_error("plan or matrix list is null"); return -1; }
    if (nmat < 1 || nmat > kMaxMats) { set_error("matrix count %d is outside 1..%d", nmat, kMaxMats); return -1; }
    if (nstages < 1 || nstages > kMaxStages) { set_error("stage count %d is outside 1..%d", nstages, kMaxStages); return -1; }
    if (x_dtype != SPARKMV_X_BF16 && x_dtype != SPARKMV_X_F32) { set_error("unknown x dtype %d", x_dtype); return -1; }
    PlanOp op;
    memset(&op.vq, 0, sizeof op.vq);
    op.kind = 0;
    for (int i = 0; i < nmat; i++) {
        VqMatDesc m;
        memset(&m, 0, sizeof m);
        for (int s = 0; s < nstages; s++) m.stages[s] = mats[i].stages[s];
        m.y = mats[i].y;
        m.rows = mats[i].rows;
        op.mats.push_back(m);
    }
    VqCall & c = op.vq;
    c.dim = dim; c.nc = nc; c.cols = cols; c.v3 = v3; c.nst = nstages;
    c.nmat = nmat; c.x = x; c.ldx = ldx; c.xf32 = x_dtype == SPARKMV_X_F32; c.ncol = ncols; c.ldy = ldy;
    c.accumulate = accumulate ? 1 : 0;
    c.variant = variant;
    if (nmat == 1 && ncols > 1 && mats[0].rows > 0) {
        /* words for workgroups that share a tile (the kernel leaves them
         * zero), enough for the deepest chunk tree: allocated here, so
         * running the plan allocates nothing, and cleared on the stream of
         * the plan's next run or capture */
        const size_t n = (size_t) mats[0].rows * ncols * (size_t) vq_ck_words(kVqCkMaxGroups);
        void * q = nullptr;
        hipError_t e = hipMalloc(&q, n * sizeof(uint64_t));
        if (e != hipSuccess) return fail_hip("plan shared-tile words", e);
        p->slots.push_back(q);
        p->unzeroed.push_back({q, n * sizeof(uint64_t)});
        c.kslot = (uint64_t *) q;
        c.kslot_cap = (long) n;
    }
    p->ops.push_back(op);
    drop_graph(p);
    return 0;
}

int sparkmv_plan_add_kquant(void * plan, int kind, const void * blocks, int rows, int cols, const void * x,
                            int x_dtype, int ldx, int ncols, float * y, int ldy, int accumulate) {
    Plan * p = (Plan *) plan;
    if (!p) { set_error("plan is null"); return -1; }
    if (kind != 6 && kind != 8) { set_error("k-quant kind %d is neither 6 (Q6_K) nor 8 (Q8_0)", kind); return -1; }
    if (x_dtype != SPARKMV_X_BF16 && x_dtype != SPARKMV_X_F32) { set_error("unknown x dtype %d", x_dtype); return -1; }
    PlanOp op;
    memset(&op.vq, 0, sizeof op.vq);
    op.kind = kind;
    op.blocks = blocks;
    op.rows = rows; op.cols = cols; op.x = x; op.xf32 = x_dtype == SPARKMV_X_F32; op.ldx = ldx; op.ncol = ncols;
    op.y = y; op.ldy = ldy; op.accumulate = accumulate ? 1 : 0;
    p->ops.push_back(op);
    drop_graph(p);
    return 0;
}

/* Issue every op in order on `stream`, no synchronization. */
int sparkmv_plan_run(void * plan, void * stream) {
    Plan * p = (Plan *) plan;
    if (!p) { set_error("plan is null"); return -1; }
    int cleared = 0;
    if (zero_slots(p, (hipStream_t) stream, &cleared)) return -1;
    for (size_t i = 0; i < p->ops.size(); i++)
        if (run_op(p->ops[i], (hipStream_t) stream)) return -1;
    return 0;
}

/* Record the chain into a HIP graph on `stream` (not the null stream). Run
 * the plan eagerly once before, so one-time launch setup happens outside. */
int sparkmv_plan_capture(void * plan, void * stream) {
    Plan * p = (Plan *) plan;
    if (!p) { set_error("plan is null"); return -1; }
    if (!stream) { set_error("a graph is captured on a created stream, not the null stream"); return -1; }
    hipStream_t s = (hipStream_t) stream;
    drop_graph(p);
    /* slot words are cleared before the capture (no memset node in the
     * graph), and waited for once, since the graph may replay on any stream */
    int cleared = 0;
    if (zero_slots(p, s, &cleared)) return -1;
    if (cleared) {
        hipError_t e0 = hipStreamSynchronize(s);
        if (e0 != hipSuccess) return fail_hip("plan shared-tile words", e0);
    }
    hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail_hip("begin capture", e);
    int rc = 0;
    for (size_t i = 0; i < p->ops.size() && !rc; i++) rc = run_op(p->ops[i], s);
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(s, &g);
    if (rc) { if (g) hipGraphDestroy(g); return -1; }
    if (e != hipSuccess) return fail_hip("end capture", e);
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) { hipGraphDestroy(g); return fail_hip("graph instantiate", e); }
    p->graph = g;
    p->exec = x;
    return 0;
}

/* Replay the captured graph, or run eagerly when none is captured. */
int sparkmv_plan_launch(void * plan, void * stream) {
    Plan * p = (Plan *) plan;
    if (!p) { set_error("plan is null"); return -1; }
    if (!p->exec) return sparkmv_plan_run(plan, stream);
    hipError_t e = hipGraphLaunch(p->exec, (hipStream_t) stream);
    return e == hipSuccess ? 0 : fail_hip("graph launch", e);
}

/* Apply a trusted tuning profile to the plan's VQ ops, as the reference's
 * runtime applies one at load (tools/vq/gpu/vq-model-gpu.cu:300-324): an op
 * takes its geometry's gemv entry when every matrix of the op has a runnable
 * entry and they agree; an entry that is not runnable here leaves the op on
 * the heuristic. An untrusted profile (another artifact or device) changes
 * nothing. Returns the number of ops changed (the message then says how many
 * entries were refused), or -1 on a null argument. */
int sparkmv_plan_apply_profile(void * plan, const void * profile, uint64_t artifact, const char * gpu) {
    Plan * p = (Plan *) plan;
    if (!p || !profile || !gpu) { set_error("plan, profile or gpu name is null"); return -1; }
    const int t = sparkmv_profile_trusted(profile, artifact, gpu);
    if (t < 0) return -1;
    if (t == 0) {
        set_error("profile: measured for another artifact or device; the heuristic stays");
        return 0;
    }
    int applied = 0, refused = 0;
    for (auto & op : p->ops) {
        if (op.kind != 0) continue;
        int v = -1, th = -1, ok = 1;
        for (const auto & m : op.mats) {
            int mv = 0, mt = 0;
            const int r = profile_gemv_pick(profile, op.vq.dim, op.vq.nc, m.rows, op.vq.cols, op.vq.v3, &mv, &mt);
            if (r < 0) refused++;
            if (r != 1 || (v >= 0 && (mv != v || mt != th))) { ok = 0; continue; }
            v = mv;
            th = mt;
        }
        if (ok && v >= 0) {
            op.vq.variant = v;
            op.vq.threads = th;
            applied++;
        }
    }
    drop_graph(p);
    set_error("profile: %d ops take their tuned kernel, %d entries are not runnable here (heuristic kept)", applied,
              refused);
    return applied;
}

/* The kernel an op runs: its variant (0 the fastest that takes the call, 1
 * the generic wave kernel, 2 the LDS-codebook wave kernel, 3 the MFMA block
 * kernel; -1 for a k-quant op) and launch width (0 = the kernel's own). */
int sparkmv_plan_op_kernel(void * plan, int i, int * variant, int * threads) {
    Plan * p = (Plan *) plan;
    if (!p || i < 0 || i >= (int) p->ops.size()) { set_error("no plan op %d", i); return -1; }
    const PlanOp & op = p->ops[(size_t) i];
    if (variant) *variant = op.kind == 0 ? op.vq.variant : -1;
    if (threads) *threads = op.kind == 0 ? op.vq.threads : 0;
    return 0;
}

/* Average device time of every op over `iters` eager runs: each op's
 * kernels carry a start and a stop event in their own dispatches, so an op's
 * time is its kernels' duration without the launch gap between ops. op_ms
 * holds plan_size entries. */
int sparkmv_plan_time_ops(void * plan, void * stream, int iters, double * op_ms) {
    Plan * p = (Plan *) plan;
    if (!p || !op_ms || iters < 1) { set_error("plan timing needs a plan, an output array and iters >= 1"); return -1; }
    hipStream_t s = (hipStream_t) stream;
    const size_t n = p->ops.size();
    std::vector<hipEvent_t> ev(2 * n);
    for (size_t i = 0; i < 2 * n; i++) {
        hipError_t e = hipEventCreate(&ev[i]);
        if (e != hipSuccess) {
            for (size_t j = 0; j < i; j++) hipEventDestroy(ev[j]);
            return fail_hip("event create", e);
        }
    }
    for (size_t i = 0; i < n; i++) op_ms[i] = 0.0;
    int cleared = 0;
    int rc = zero_slots(p, s, &cleared);
    for (int it = 0; it < iters && !rc; it++) {
        for (size_t i = 0; i < n && !rc; i++) {
            g_launch_events.start = ev[2 * i];
            g_launch_events.stop = ev[2 * i + 1];
            rc = run_op(p->ops[i], s);
            g_launch_events = LaunchEvents();
        }
        hipError_t e = n ? hipEventSynchronize(ev[2 * n - 1]) : hipSuccess;
        if (!rc && e != hipSuccess) rc = fail_hip("op timing", e);
        for (size_t i = 0; i < n && !rc; i++) {
            float t = 0;
            e = hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]);
            if (e != hipSuccess) { rc = fail_hip("op timing", e); break; }
            op_ms[i] += t / iters;
        }
    }
    for (size_t i = 0; i < 2 * n; i++) hipEventDestroy(ev[i]);
    return rc;
}

}  // extern "C"
