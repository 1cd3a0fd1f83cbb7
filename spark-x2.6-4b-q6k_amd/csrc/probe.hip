/* probe.hip — what the fixed cost of one launch is made of (gfx950).
 *
 * A decode matvec reads 8-40 MB, which at 8 TB/s is 1-5 µs of transfer; the
 * hot kernel's launches take 6.5-15 µs. These kernels split the difference,
 * each on the hot kernel's launch shape (256 workgroups of 10 waves, one
 * workgroup per CU) and timed kernel-exact (events carried by the dispatch):
 *
 *   probe_empty_kernel  nothing but its launch: dispatch of every workgroup
 *                       and the end-of-kernel drain (also run with one wave
 *                       per workgroup, to separate the dispatch's fixed part
 *                       from the waves');
 *   probe_stage_kernel  the hot kernel's prologue alone: 64 KB of codebooks
 *                       (L2-resident after the first workgroup of each XCD)
 *                       into LDS, then the barrier;
 *   probe_read_kernel   a plain read of B bytes, each workgroup one
 *                       contiguous slice, four 16-byte loads in flight per
 *                       lane (the hot kernel reads its tiles' streams the
 *                       same way);
 *   probe_touch_kernel  one dword every `stride` bytes of a buffer: with a
 *                       4 KB stride it warms address translation and almost
 *                       no data (one 64-byte line per page); with a 64-byte
 *                       stride it brings every line into the caches.
 *
 * The host entry times a read on a buffer no kernel has touched for the last
 * 640 MB of traffic (cold: beyond the 256 MB memory-side cache and every
 * XCD's L2), the same read right after a page touch of that buffer
 * (translation warm, data cold) and right after a line touch (data warm).
 * No counterpart in the reference: a measurement of this build's launches.
 */
#include "../../include/sparkmv.h"
#include "common.h"

#include <algorithm>
#include <vector>

namespace sparkmv {

constexpr int kProbeWaves = 10;
constexpr int kProbeThreads = kProbeWaves * 64;

/* no memory access at all: a wave starts and ends */
__global__ __launch_bounds__(kProbeThreads) void probe_empty_kernel(uint32_t *) {}

__global__ __launch_bounds__(kProbeThreads) void probe_stage_kernel(const uint4 * cb, uint32_t * sink) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int n = 65536 / 16;
    constexpr int per = (n + kProbeThreads - 1) / kProbeThreads;
    uint4 v[per];
#pragma unroll
    for (int k = 0; k < per; k++) v[k] = cb[min(k * kProbeThreads + (int) threadIdx.x, n - 1)];
#pragma unroll
    for (int k = 0; k < per; k++) {
        const int i = k * kProbeThreads + (int) threadIdx.x;
        if (i < n) ((uint4 *) lds)[i] = v[k];
    }
    __syncthreads();
    const uint4 w = ((const uint4 *) lds)[(threadIdx.x * 37u) % n];
    if ((w.x ^ w.y ^ w.z ^ w.w) == 0x9e3779b9u) sink[blockIdx.x] = 1u;
}

__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const uint4 * p, size_t n16, uint32_t * sink) {
    const size_t lo = n16 * blockIdx.x / gridDim.x, hi = n16 * (blockIdx.x + 1) / gridDim.x;
    uint32_t acc = 0;
    size_t i = lo + threadIdx.x;
    for (; i + 3 * kProbeThreads < hi; i += 4 * kProbeThreads) {
        const uint4 a = p[i], b = p[i + kProbeThreads], c = p[i + 2 * kProbeThreads], d = p[i + 3 * kProbeThreads];
        acc ^= a.x ^ b.y ^ c.z ^ d.w;
    }
    for (; i < hi; i += kProbeThreads) acc ^= p[i].x;
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

__global__ __launch_bounds__(kProbeThreads) void probe_touch_kernel(const uint32_t * p, size_t nwords, size_t stride,
                                                                    uint32_t * sink) {
    uint32_t acc = 0;
    for (size_t i = ((size_t) blockIdx.x * blockDim.x + threadIdx.x) * stride; i < nwords;
         i += (size_t) gridDim.x * blockDim.x * stride)
        acc ^= p[i];
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

/* A chain of K dependent "ops" over all workgroups, each op moving n words:
 * every workgroup reads all n words the previous op wrote, sums them, and
 * writes its 1/G of this op's n words. Three ways to know the words are
 * there: (0) each word carries its epoch in its upper half and a reader
 * reloads the words whose epoch is not yet current; (1) the same words, but
 * wave 0 first waits on one word of each producer; (2) plain words, each
 * producer's stores released by an agent-scope fence and counted by an
 * atomic per op, which wave 0 polls before anyone reads. Every wait is
 * bounded (past kProbeSpin polls the workgroup sets *err and waits no more).
 * out[0] is the last op's sum in workgroup 0, which the host checks. */
constexpr int kProbeMaxWords = 10;              /* words per thread */
constexpr uint32_t kProbeSpin = 1u << 18;

template <int MODE>
__global__ __launch_bounds__(512) void probe_handoff_kernel(uint64_t * buf, uint32_t * ctr, int n, int K,
                                                            uint32_t base, uint32_t * err, uint32_t * out) {
    __shared__ uint32_t red[8];
    const int tid = threadIdx.x, G = gridDim.x, wg = blockIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t s = 0;
    bool dead = false;
    for (int op = 0; op < K; op++) {
        if (op > 0) {
            const uint64_t * src = buf + (size_t) (op - 1) * n;
            const uint32_t want = base + (uint32_t) op;
            if (MODE == 1 && wave == 0 && !dead) {
                uint32_t spins = 0;
                while (true) {
                    bool ok = true;
                    for (int k = 0; k < 4; k++) {
                        const int p = lane + 64 * k;
                        const int lo = (int) ((long) p * n / G), hi = (int) ((long) (p + 1) * n / G);
                        if (p < G && hi > lo &&
                            (uint32_t) (__hip_atomic_load(src + hi - 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 32) != want)
                            ok = false;
                    }
                    if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
                    if (++spins > kProbeSpin) { if (lane == 0) atomicOr(err, 1u); dead = true; break; }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            if (MODE == 2 && wave == 0 && !dead) {
                uint32_t spins = 0;
                while (__hip_atomic_load(ctr + op - 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (uint32_t) G) {
                    if (++spins > kProbeSpin) { if (lane == 0) atomicOr(err, 1u); dead = true; break; }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            if (MODE != 0) __syncthreads();
            const int cnt = tid < n ? (n - tid + 511) / 512 : 0;
            uint64_t v[kProbeMaxWords];
#pragma unroll
            for (int k = 0; k < kProbeMaxWords; k++)
                if (k < cnt) v[k] = __hip_atomic_load(src + tid + k * 512, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            uint32_t spins = 0;
            while (!dead) {
                bool ok = true;
#pragma unroll
                for (int k = 0; k < kProbeMaxWords; k++)
                    if (k < cnt && (uint32_t) (v[k] >> 32) != want) ok = false;
                if (ok) break;
                if (++spins > kProbeSpin) { atomicOr(err, 2u); dead = true; break; }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int k = 0; k < kProbeMaxWords; k++)
                    if (k < cnt && (uint32_t) (v[k] >> 32) != want)
                        v[k] = __hip_atomic_load(src + tid + k * 512, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            uint32_t part = 0;
#pragma unroll
            for (int k = 0; k < kProbeMaxWords; k++)
                if (k < cnt) part += (uint32_t) v[k];
            for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
            if (lane == 0) red[wave] = part;
            __syncthreads();
            s = 0;
            for (int w = 0; w < 8; w++) s += red[w];
            __syncthreads();
        }
        const int lo = (int) ((long) wg * n / G), hi = (int) ((long) (wg + 1) * n / G);
        uint64_t * dst = buf + (size_t) op * n;
        const uint32_t ep = base + (uint32_t) op + 1u;
        if (lo + tid < hi)
            __hip_atomic_store(dst + lo + tid, ((uint64_t) ep << 32) | (uint32_t) (s * 31u + (uint32_t) (lo + tid)),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (MODE == 2) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __syncthreads();
            if (tid == 0) __hip_atomic_fetch_add(ctr + op, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (wg == 0 && tid == 0) out[0] = s;
}

}  // namespace sparkmv

using namespace sparkmv;

namespace {

struct Timer {
    hipEvent_t a = nullptr, b = nullptr;
    Timer() {
        (void) hipEventCreate(&a);
        (void) hipEventCreate(&b);
    }
    ~Timer() {
        if (a) (void) hipEventDestroy(a);
        if (b) (void) hipEventDestroy(b);
    }
    /* arm the next hot-path launch to carry the events */
    void arm() {
        g_launch_events.start = a;
        g_launch_events.stop = b;
    }
    double us() {
        g_launch_events = LaunchEvents();
        if (hipEventSynchronize(b) != hipSuccess) return -1.0;
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return -1.0;
        return 1000.0 * ms;
    }
};

double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    return v.empty() ? 0.0 : v[v.size() / 2];
}

}  // namespace

extern "C" {

int sparkmv_probe_startup(const size_t * sizes, int nsizes, int reps, double * out_us) {
    if (!sizes || nsizes < 1 || nsizes > 8 || reps < 3 || reps > 64 || !out_us) {
        set_error("probe: 1..8 sizes, 3..64 repetitions and an output array");
        return -1;
    }
    for (int s = 0; s < nsizes; s++)
        if (sizes[s] < 65536 || sizes[s] > ((size_t) 1 << 30) || sizes[s] % 16) {
            set_error("probe: sizes are multiples of 16 bytes from 64 KB to 1 GB, not %zu", sizes[s]);
            return -1;
        }
    const int G = cu_count();
    const size_t pool = (size_t) 640 << 20;   /* more than the memory-side cache and every L2 together */
    size_t big = 65536;
    for (int s = 0; s < nsizes; s++) big = std::max(big, sizes[s]);
    /* targets first, then a separate flush region: reading the whole region
     * leaves none of a target in any cache */
    const size_t targets = big * (size_t) reps, total = targets + pool;
    uint8_t * buf = nullptr;
    uint32_t * sink = nullptr;
    hipError_t e = hipMalloc((void **) &buf, total);
    if (e != hipSuccess) return fail_hip("probe buffer", e);
    e = hipMalloc((void **) &sink, 4 * (size_t) G);
    if (e == hipSuccess) e = hipMemset(sink, 0, 4 * (size_t) G);
    if (e == hipSuccess) e = hipMemset(buf, 1, total);
    if (e == hipSuccess) e = hipFuncSetAttribute((const void *) probe_stage_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 65536);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void) hipFree(buf);
        if (sink) (void) hipFree(sink);
        return fail_hip("probe setup", e);
    }
    hipStream_t st = nullptr;
    Timer t;
    const dim3 grid(G), block(kProbeThreads);
    int rc = 0;
    /* flush: one pass over the flush region evicts every target from the caches */
    auto flush = [&]() {
        launch_kernel(probe_read_kernel, grid, block, 0, st, (const uint4 *) (buf + targets), pool / 16, sink);
    };
    std::vector<double> v;
    /* empty launches */
    for (int r = 0; r < reps && !rc; r++) {
        t.arm();
        launch_kernel(probe_empty_kernel, grid, block, 0, st, sink);
        v.push_back(t.us());
    }
    out_us[0] = median(v);
    v.clear();
    for (int r = 0; r < reps && !rc; r++) {
        t.arm();
        launch_kernel(probe_empty_kernel, grid, dim3(64), 0, st, sink);
        v.push_back(t.us());
    }
    out_us[1] = median(v);
    /* one workgroup of one wave */
    v.clear();
    for (int r = 0; r < reps && !rc; r++) {
        t.arm();
        launch_kernel(probe_empty_kernel, dim3(1), dim3(64), 0, st, sink);
        v.push_back(t.us());
    }
    out_us[3 + 3 * nsizes] = median(v);
    /* 64 empty launches of the full shape back to back on one stream, eagerly
     * and as one captured graph: wall time per launch between two plain
     * events (no per-dispatch event) */
    {
        hipStream_t cs = nullptr;
        hipGraph_t g = nullptr;
        hipGraphExec_t gx = nullptr;
        e = hipStreamCreate(&cs);
        const int K = 64;
        auto wall = [&](bool graph) -> double {
            std::vector<double> w;
            for (int r = 0; r < 5; r++) {
                if (hipEventRecord(t.a, cs) != hipSuccess) return -1.0;
                if (graph) {
                    if (hipGraphLaunch(gx, cs) != hipSuccess) return -1.0;
                } else {
                    for (int k = 0; k < K; k++) hipLaunchKernelGGL(probe_empty_kernel, grid, block, 0, cs, sink);
                }
                if (hipEventRecord(t.b, cs) != hipSuccess || hipEventSynchronize(t.b) != hipSuccess) return -1.0;
                float ms = 0.f;
                if (hipEventElapsedTime(&ms, t.a, t.b) != hipSuccess) return -1.0;
                w.push_back(1000.0 * ms / K);
            }
            return median(w);
        };
        if (e == hipSuccess) out_us[4 + 3 * nsizes] = wall(false);
        if (e == hipSuccess) e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            for (int k = 0; k < K; k++) hipLaunchKernelGGL(probe_empty_kernel, grid, block, 0, cs, sink);
            e = hipStreamEndCapture(cs, &g);
        }
        if (e == hipSuccess) e = hipGraphInstantiate(&gx, g, nullptr, nullptr, 0);
        if (e == hipSuccess) {
            (void) hipGraphLaunch(gx, cs);   /* first replay uploads the graph */
            (void) hipStreamSynchronize(cs);
            out_us[5 + 3 * nsizes] = wall(true);
        }
        if (gx) (void) hipGraphExecDestroy(gx);
        if (g) (void) hipGraphDestroy(g);
        if (cs) (void) hipStreamDestroy(cs);
        if (e != hipSuccess) rc = fail_hip("probe back-to-back launches", e);
    }
    /* staging alone, codebooks cold in L2 each time (flushed before) */
    v.clear();
    for (int r = 0; r < reps && !rc; r++) {
        flush();
        t.arm();
        launch_kernel(probe_stage_kernel, grid, block, 65536, st, (const uint4 *) (buf + (size_t) r * 65536), sink);
        v.push_back(t.us());
    }
    out_us[2] = median(v);
    for (int s = 0; s < nsizes && !rc; s++) {
        const size_t B = sizes[s];
        std::vector<double> cold, page, line;
        for (int r = 0; r < reps; r++) {
            const uint8_t * p = buf + (size_t) r * B;
            flush();
            t.arm();
            launch_kernel(probe_read_kernel, grid, block, 0, st, (const uint4 *) p, B / 16, sink);
            cold.push_back(t.us());
            flush();
            launch_kernel(probe_touch_kernel, grid, block, 0, st, (const uint32_t *) p, B / 4, (size_t) 1024, sink);
            t.arm();
            launch_kernel(probe_read_kernel, grid, block, 0, st, (const uint4 *) p, B / 16, sink);
            page.push_back(t.us());
            flush();
            launch_kernel(probe_touch_kernel, grid, block, 0, st, (const uint32_t *) p, B / 4, (size_t) 16, sink);
            t.arm();
            launch_kernel(probe_read_kernel, grid, block, 0, st, (const uint4 *) p, B / 16, sink);
            line.push_back(t.us());
        }
        out_us[3 + 3 * s] = median(cold);
        out_us[4 + 3 * s] = median(page);
        out_us[5 + 3 * s] = median(line);
    }
    e = hipDeviceSynchronize();
    if (e != hipSuccess) rc = fail_hip("probe", e);
    (void) hipFree(buf);
    (void) hipFree(sink);
    for (int k = 0; k < 6 + 3 * nsizes; k++)
        if (out_us[k] < 0) { set_error("probe: a timing event failed"); rc = -1; }
    return rc;
}

/* Dependent handoffs over every workgroup (see probe_handoff_kernel): for
 * each mode (0 epoch-carrying words, 1 the same behind a per-producer
 * sentinel, 2 fence + counter) and each word count in nwords (up to 5120),
 * the µs per dependent op of a 400-op launch minus a 1-op launch, best of 5:
 * out_us[mode * nn + i]. The chain's result is checked against its closed
 * form; -1 on a mismatch or a wait that gave up. Needs the device to itself
 * (one workgroup per CU, all resident). */
int sparkmv_probe_handoff(const int * nwords, int nn, double * out_us) {
    if (!nwords || nn < 1 || nn > 8 || !out_us) { set_error("probe handoff: 1..8 word counts and an output array"); return -1; }
    for (int i = 0; i < nn; i++)
        if (nwords[i] < 256 || nwords[i] > 512 * kProbeMaxWords) {
            set_error("probe handoff: word counts are 256..%d, not %d", 512 * kProbeMaxWords, nwords[i]);
            return -1;
        }
    const int G = cu_count(), K = 400;
    uint64_t * buf = nullptr;
    uint32_t *ctr = nullptr, *err = nullptr, *out = nullptr;
    const size_t nbuf = (size_t) K * 512 * kProbeMaxWords;
    hipError_t e = hipMalloc((void **) &buf, nbuf * 8);
    if (e == hipSuccess) e = hipMalloc((void **) &ctr, 4 * (size_t) K);
    if (e == hipSuccess) e = hipMalloc((void **) &err, 4);
    if (e == hipSuccess) e = hipMalloc((void **) &out, 4);
    if (e == hipSuccess) e = hipMemset(buf, 0, nbuf * 8);
    if (e == hipSuccess) e = hipMemset(err, 0, 4);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    int rc = e == hipSuccess ? 0 : fail_hip("probe handoff setup", e);
    uint32_t base = 1;
    Timer t;
    auto run = [&](int mode, int n, int k) -> double {
        if (hipMemset(ctr, 0, 4 * (size_t) K) != hipSuccess) return -1.0;
        if (hipEventRecord(t.a, nullptr) != hipSuccess) return -1.0;
        const size_t lds = 96 * 1024;   /* one workgroup per CU */
        if (mode == 0) hipLaunchKernelGGL(probe_handoff_kernel<0>, dim3(G), dim3(512), lds, nullptr, buf, ctr, n, k, base, err, out);
        if (mode == 1) hipLaunchKernelGGL(probe_handoff_kernel<1>, dim3(G), dim3(512), lds, nullptr, buf, ctr, n, k, base, err, out);
        if (mode == 2) hipLaunchKernelGGL(probe_handoff_kernel<2>, dim3(G), dim3(512), lds, nullptr, buf, ctr, n, k, base, err, out);
        if (hipGetLastError() != hipSuccess || hipEventRecord(t.b, nullptr) != hipSuccess ||
            hipEventSynchronize(t.b) != hipSuccess)
            return -1.0;
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, t.a, t.b) != hipSuccess) return -1.0;
        uint32_t h[2] = {0, 0};
        if (hipMemcpy(h, out, 4, hipMemcpyDeviceToHost) != hipSuccess || hipMemcpy(h + 1, err, 4, hipMemcpyDeviceToHost) != hipSuccess)
            return -1.0;
        uint32_t want = 0;
        for (int op = 1; op < k; op++) want = (uint32_t) n * 31u * want + (uint32_t) ((uint64_t) n * (n - 1) / 2);
        base += (uint32_t) k + 1u;
        if (h[1] || h[0] != want) return -2.0;
        return 1000.0 * ms;
    };
    for (int mode = 0; mode < 3 && !rc; mode++)
        for (int i = 0; i < nn && !rc; i++) {
            const int n = nwords[i];
            double best = 1e30, best1 = 1e30;
            for (int r = 0; r < 5 && !rc; r++) {
                const double a = run(mode, n, K), b = run(mode, n, 1);
                if (a < 0 || b < 0) {
                    rc = -1;
                    set_error(a == -2.0 || b == -2.0 ? "probe handoff: a chain's result or wait failed" : "probe handoff: a launch failed");
                }
                best = std::min(best, a);
                best1 = std::min(best1, b);
            }
            out_us[mode * nn + i] = (best - best1) / (K - 1);
        }
    (void) hipFree(buf);
    (void) hipFree(ctr);
    (void) hipFree(err);
    (void) hipFree(out);
    return rc;
}

/* The floor of one launch per matvec: n plain reads (probe_read_kernel on
 * the hot kernel's launch shape) of sizes[i] bytes each, every read its own
 * region of one buffer, back to back as one captured HIP graph and eagerly
 * on a stream. out_us[0] = µs per graph replay, out_us[1] = µs per eager
 * pass (wall time between two plain events, median of reps). With the
 * decode set's byte counts (3.27 GB, beyond the 256 MB memory-side cache)
 * every replay reads cold, as a token does. */
int sparkmv_probe_read_chain(const size_t * sizes, int n, int reps, double * out_us) {
    if (!sizes || n < 1 || n > 1024 || reps < 3 || reps > 64 || !out_us) {
        set_error("probe read chain: 1..1024 sizes, 3..64 repetitions and an output array");
        return -1;
    }
    std::vector<size_t> off(n + 1, 0);
    for (int i = 0; i < n; i++) {
        if (sizes[i] < 4096 || sizes[i] > ((size_t) 1 << 30)) {
            set_error("probe read chain: sizes from 4 KB to 1 GB, not %zu", sizes[i]);
            return -1;
        }
        off[i + 1] = off[i] + ((sizes[i] + 255) & ~(size_t) 255);
    }
    if (off[n] > ((size_t) 16 << 30)) { set_error("probe read chain: more than 16 GB in all"); return -1; }
    const int G = cu_count();
    uint8_t * buf = nullptr;
    uint32_t * sink = nullptr;
    hipStream_t cs = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t gx = nullptr;
    hipError_t e = hipMalloc((void **) &buf, off[n]);
    if (e == hipSuccess) e = hipMalloc((void **) &sink, 4 * (size_t) G);
    if (e == hipSuccess) e = hipMemset(sink, 0, 4 * (size_t) G);
    if (e == hipSuccess) e = hipMemset(buf, 1, off[n]);
    if (e == hipSuccess) e = hipStreamCreate(&cs);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    const dim3 grid(G), block(kProbeThreads);
    auto pass = [&]() {
        for (int i = 0; i < n; i++)
            hipLaunchKernelGGL(probe_read_kernel, grid, block, 0, cs, (const uint4 *) (buf + off[i]), sizes[i] / 16,
                               sink);
    };
    if (e == hipSuccess) e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
        pass();
        e = hipStreamEndCapture(cs, &g);
    }
    if (e == hipSuccess) e = hipGraphInstantiate(&gx, g, nullptr, nullptr, 0);
    int rc = 0;
    if (e == hipSuccess) {
        Timer t;
        auto wall = [&](bool graph) -> double {
            std::vector<double> w;
            if (graph) (void) hipGraphLaunch(gx, cs);   /* the first replay uploads the graph */
            else pass();
            if (hipStreamSynchronize(cs) != hipSuccess) return -1.0;
            for (int r = 0; r < reps; r++) {
                if (hipEventRecord(t.a, cs) != hipSuccess) return -1.0;
                if (graph) {
                    if (hipGraphLaunch(gx, cs) != hipSuccess) return -1.0;
                } else {
                    pass();
                }
                if (hipEventRecord(t.b, cs) != hipSuccess || hipEventSynchronize(t.b) != hipSuccess) return -1.0;
                float ms = 0.f;
                if (hipEventElapsedTime(&ms, t.a, t.b) != hipSuccess) return -1.0;
                w.push_back(1000.0 * ms);
            }
            return median(w);
        };
        out_us[0] = wall(true);
        out_us[1] = wall(false);
        if (out_us[0] < 0 || out_us[1] < 0) { set_error("probe read chain: a timing event failed"); rc = -1; }
    } else {
        rc = fail_hip("probe read chain setup", e);
    }
    if (gx) (void) hipGraphExecDestroy(gx);
    if (g) (void) hipGraphDestroy(g);
    if (cs) (void) hipStreamDestroy(cs);
    e = hipDeviceSynchronize();
    if (!rc && e != hipSuccess) rc = fail_hip("probe read chain", e);
    if (buf) (void) hipFree(buf);
    if (sink) (void) hipFree(sink);
    return rc;
}

}  // extern "C"
