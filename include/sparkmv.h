/* sparkmv.h — C-ABI of the MI355X (gfx950) quantized matvec library.
 *
 * Two groups of entry points:
 *
 *  1. vqg_*: drop-in replacements for the reference's CUDA C-ABI
 *     (tools/vq/gpu/decode-gpu.cu:765-1140), same names, argument meaning,
 *     return convention and error text channel. Each declaration cites the
 *     reference function it replaces. As there:
 *       - `payload` is a device pointer to ONE stage payload (DQVQ or DQV3),
 *         not to the container;
 *       - x and y are device f32 pointers; y ACCUMULATES (y += W x), so a
 *         caller zeroes it or adds into a residual on purpose;
 *       - 0 = success, -1 = failure with a message in vqg_decode_error();
 *       - *_launch* entry points are asynchronous on the default (null)
 *         stream; timed entry points synchronize and report the best of
 *         `iters` runs in *ms;
 *       - not thread-safe (one static error buffer).
 *     Slack contract: the reference requires 8 zeroed bytes past every stage
 *     payload (decode-gpu.cu:95-102). This library never reads past a stage's
 *     index stream, so the slack is accepted but not needed.
 *
 *  2. sparkmv_*: the same operations with what the reference's ABI lacks:
 *     bf16 activations, N <= 16 activation columns decoded once
 *     (speculative verify), every stage of a container in one launch, several
 *     matrices sharing one x in one launch, Q6_K and Q8_0 GEMV, token-major
 *     prefill, and an explicit hipStream_t (passed as void *, NULL = default).
 *     Same return and error convention.
 *
 * Variant numbers. The vqg_* GEMV entry points number variants as the
 * reference does (decode-gpu.cu:788-797, :808-833, :865-906), so its
 * runtime and tuner choose what they would choose on CUDA:
 *   vqg_gemv_ready  3 when the DQV3 block preconditions hold, 2 for dim 4,
 *                   1 always, 0 when the codebook fits the shared-codebook
 *                   kernel (160 KB of LDS);
 *   vqg_gemv_t / vqg_gemv: 0 the shared-codebook kernel (256 wide), 1 the
 *                   generic wave kernel, 2 the dim-4 path (the MFMA block
 *                   kernel where it takes the geometry), 3 the block path;
 *   vqg_gemv_launch / _launch_t: 0 the reference's pick (3 when ready,
 *                   else 2 for dim 4, else 1), 1-3 as above.
 * Launch widths are warp multiples (32) up to 1024, as there; a width
 * rounds up to whole 64-lane waves, which changes only how many rows share
 * a workgroup, never a result.
 * The sparkmv_* GEMV entry points number their kernels directly: 0 the
 * fastest that takes the call, 1 the generic wave kernel, 2 the wave kernel
 * with the codebook in LDS, 3 the MFMA block kernel (sparkmv_vq_gemv_ready).
 */
#ifndef SPARKMV_H
#define SPARKMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================= reference-compatible ABI ========================= */

/* decode-gpu.cu:23 vqg_decode_error */
const char * vqg_decode_error(void);
/* decode-gpu.cu:769-775 vqg_device_name */
int vqg_device_name(char * out, int n);
/* decode-gpu.cu:779-783 vqg_driver_version (HIP's encoding) */
int vqg_driver_version(void);

/* decode-gpu.cu:788-797 vqg_gemv_ready */
int vqg_gemv_ready(int dim, int nc, int rows, int cols, int v3, int variant);
/* decode-gpu.cu:865-906 vqg_gemv_t */
int vqg_gemv_t(const void * payload, int dim, int nc, int rows, int cols, int v3,
               const float * x, float * y, int variant, int threads, int iters, double * ms);
/* decode-gpu.cu:908-911 vqg_gemv */
int vqg_gemv(const void * payload, int dim, int nc, int rows, int cols, int v3,
             const float * x, float * y, int variant, int iters, double * ms);
/* decode-gpu.cu:916-921 vqg_gemv_launch_t */
int vqg_gemv_launch_t(const void * payload, int dim, int nc, int rows, int cols, int v3,
                      const float * x, float * y, int variant, int threads);
/* decode-gpu.cu:923-928 vqg_gemv_launch */
int vqg_gemv_launch(const void * payload, int dim, int nc, int rows, int cols, int v3,
                    const float * x, float * y, int variant);
/* decode-gpu.cu:835-857 vqg_dequant: decode one stage into out (accumulates) */
int vqg_dequant(const void * payload, int dim, int nc, int rows, int cols, int v3,
                float * out, int iters, double * ms);
/* decode-gpu.cu:947-956 vqg_row_dequant: one row of one stage (accumulates) */
int vqg_row_dequant(const void * payload, int dim, int nc, int rows, int cols, int v3,
                    int row, float * out);

/* Prefill: xT is [cols][ntok], y is [ntok][rows], both device f32; y accumulates.
 * Variants: 0 auto, 1 and 2 the MFMA tile kernel (tile from the table below),
 * 3 the one-thread-per-(row, token) kernel (any geometry). */
/* decode-gpu.cu:995-1005 vqg_prefill_ready */
int vqg_prefill_ready(int dim, int nc, int rows, int cols, int v3, int variant);
/* decode-gpu.cu:1008 vqg_prefill_cfg_count */
int vqg_prefill_cfg_count(void);
/* decode-gpu.cu:1010-1015 vqg_prefill_cfg */
int vqg_prefill_cfg(int idx, int * bn, int * bk);
/* decode-gpu.cu:1020-1025 vqg_prefill_cfg_ready */
int vqg_prefill_cfg_ready(int dim, int nc, int rows, int cols, int v3, int bn, int bk, int variant);
/* decode-gpu.cu:1030-1043 vqg_prefill */
int vqg_prefill(const void * payload, int dim, int nc, int rows, int cols, int v3,
                const float * xT, int ntok, float * y, int iters, double * ms, int variant);
/* decode-gpu.cu:1046-1060 vqg_prefill_tile */
int vqg_prefill_tile(const void * payload, int dim, int nc, int rows, int cols, int v3,
                     const float * xT, int ntok, float * y, int iters, double * ms,
                     int bn, int bk, int variant);
/* decode-gpu.cu:1066-1089 vqg_prefill_launch */
int vqg_prefill_launch(const void * payload, int dim, int nc, int rows, int cols, int v3,
                       const float * xT, int ntok, float * y, int variant);
/* decode-gpu.cu:1094-1117 vqg_prefill_launch_tile */
int vqg_prefill_launch_tile(const void * payload, int dim, int nc, int rows, int cols, int v3,
                            const float * xT, int ntok, float * y, int bn, int bk, int variant);
/* decode-gpu.cu:1119-1138 vqg_gemv_f32: y[r] += dot(w row r, x), f32 */
int vqg_gemv_f32(const float * w, const float * x, float * y, int rows, int cols, int iters, double * ms);

/* ============================ sparkmv ABI ================================= */

#define SPARKMV_X_BF16 0   /* activations are bf16 bit patterns (uint16) */
#define SPARKMV_X_F32  1   /* activations are f32 */

/* Parsed RQVQ container, as tools/vq-format/src/lib.rs:240-306 validates it. */
typedef struct {
    int dim, nc, nstages, rows, cols, v3, nbit;
    uint64_t payload_bytes;
    uint64_t stage_offset[4];   /* byte offset of each stage payload in the file */
    uint64_t stage_bytes;       /* bytes per stage payload */
} sparkmv_container_info;

/* Validate a container held in HOST memory and locate its stages; refusals
 * and their messages follow Container::open (lib.rs:240-306). No counterpart
 * entry point in the reference's C-ABI: its loaders parse headers themselves
 * (tools/vq/gpu/vq-model-gpu.cu:230-328). */
int sparkmv_container_open(const void * bytes, size_t len, sparkmv_container_info * info);

/* Bytes of one stage payload for a geometry (tools/vq/decode.c:107-125). */
size_t sparkmv_stage_bytes(int v3, int rows, int cols, int dim, int nc);

/* Fused VQ GEMV over every stage of one matrix in one launch:
 *   y[n*ldy + r] (+)= sum_s g_s[r] * sum_i cb_s[idx_s(r,i)] . x[n*ldx + dim*i ..]
 * stages[s] are device pointers to the stage payloads (host array of
 * nstages <= 4 pointers); x has ncols <= 16 columns; accumulate 1 adds into y,
 * 0 overwrites it. Replaces the per-stage loop of tools/vq/gpu/vq-model-gpu.cu:651-660
 * (gemv) with the bf16 / N-column forms the reference lacks. variant as above. */
/* Whether a sparkmv_* GEMV variant (numbering above) takes this geometry. */
int sparkmv_vq_gemv_ready(int dim, int nc, int rows, int cols, int v3, int variant);
int sparkmv_vq_gemv(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                    const void * x, int x_dtype, int ldx, int ncols, float * y, int ldy,
                    int accumulate, int variant, void * stream);

/* One matrix of a multi-matrix launch. */
typedef struct {
    const void * stages[4];
    float * y;
    int rows;
} sparkmv_vq_matrix;

/* Several VQ matrices that share dim, nc, cols, format, stage count and x in
 * one launch (q/k/v/gate of a layer, or gate/up): the forward's call sites
 * tools/vq-runtime/src/model.rs:481-482 and :570-571 issue them back to back
 * on the same input. nmat <= 8. */
int sparkmv_vq_gemv_multi(const sparkmv_vq_matrix * mats, int nmat, int nstages, int dim, int nc, int cols,
                          int v3, const void * x, int x_dtype, int ldx, int ncols, int ldy,
                          int accumulate, int variant, void * stream);

/* rms_norm fused into the matvecs that read it: one column, x =
 * bf16(rms_norm(h) * norm_w) (model.rs:236-245: the sum of squares in f64,
 * 1 / sqrt(mean + eps) rounded once to f32, (h * inv) * w in f32, then
 * bf16 as the bf16 activations are stored), staged by every workgroup from
 * the f32 residual h, then y_m (+)= W_m x for the nmat <= 4 matrices. It
 * replaces the forward's norm launch followed by its matvec launch
 * (vq-model-gpu.cu:789-792, :808-813). x_out, when non-null, receives those
 * bf16 values. No counterpart in the reference ABI. Only shapes the
 * one-column block kernel stages whole (DQV3 dim 4, an even codebook, 1 or
 * 2 stages, columns a multiple of 128 up to 8 per thread of the launch,
 * 16-byte aligned h and norm_w); any other call is refused with a message
 * and launches nothing. */
int sparkmv_vq_gemv_norm(const sparkmv_vq_matrix * mats, int nmat, int nstages, int dim, int nc, int cols, int v3,
                         const float * h, const float * norm_w, float eps, uint16_t * x_out, int accumulate,
                         void * stream);

/* Bit-exact decode of every stage into out (rows x cols f32, row-major):
 * out (+)= sum_s cb_s[idx] * g_s, stage 0 first (lib.rs:197-211, :309-315). */
int sparkmv_vq_dequant(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                       float * out, int accumulate, void * stream);

/* ggml Q6_K GEMV: blocks are row-major [rows][cols/256] block_q6_K (210 B:
 * ql[128] qh[64] int8 scales[16] fp16 d). cols % 256 == 0. y as above.
 * No reference implementation exists (tools/vq/quant_err.c:38-43 calls
 * llama.cpp, absent); block size from tools/kquant/stubs.c:30,:44. */
int sparkmv_q6k_gemv(const void * blocks, int rows, int cols, const void * x, int x_dtype, int ldx, int ncols,
                     float * y, int ldy, int accumulate, void * stream);
/* ggml Q8_0 GEMV: [rows][cols/32] block_q8_0 (34 B: fp16 d, int8 qs[32]);
 * the tied head (tools/dspark/src/gguf.rs:201; tools/kquant/stubs.c:25,:39). */
int sparkmv_q8_0_gemv(const void * blocks, int rows, int cols, const void * x, int x_dtype, int ldx, int ncols,
                      float * y, int ldy, int accumulate, void * stream);
/* Exact dequant of Q6_K / Q8_0 rows into f32 (overwrites out). */
int sparkmv_q6k_dequant(const void * blocks, int rows, int cols, float * out, void * stream);
int sparkmv_q8_0_dequant(const void * blocks, int rows, int cols, float * out, void * stream);

/* Prefill GEMM over every stage, token-major: x is [ntok][ldx] (bf16 or f32),
 * y is [ntok][ldy] f32, y (+)= W x_t for each token t. Replaces the
 * transpose + vqg_prefill_launch_tile route of tools/vq/gpu/vq-model-gpu.cu:838-851, :899-900.
 * DQV3 dim-4 matrices with 16-byte aligned x rows run on the matrix cores
 * (f16 codewords from an LDS codebook, x as f16, f32 accumulation, like the
 * reference's f16 tiled kernel; two stages as sparkmv_prefill_fold says);
 * any other call runs the one-thread-per-output kernel. */
int sparkmv_vq_prefill(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                       const void * x, int x_dtype, int ldx, int ntok, float * y, int ldy,
                       int accumulate, void * stream);
/* The same prefill without any allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). A short
 * matrix's split-K partial sums go to a fixed device array of 32 MiB that the
 * library holds on every GPU it runs on until the process ends, instead of
 * the pool sparkmv_vq_prefill draws from; a call whose split slices would
 * exceed it fails with a message saying how many bytes it needs. Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams, or from different threads) race. The first call on a
 * device looks the array's address up once, under a lock. */
int sparkmv_vq_prefill_noalloc(const void * const * stages, int nstages, int dim, int nc, int rows, int cols, int v3,
                               const void * x, int x_dtype, int ldx, int ntok, float * y, int ldy,
                               int accumulate, void * stream);
/* How the matrix-core prefill treats two stages, process-wide. 1 (the
 * default): the stages fold into one f16 weight g0 c0 + g1 c1 before the
 * MFMA, one more rounding per weight (about 2e-4 relative L2 at the FFN
 * shapes, inside the prefill's 1e-3 gate). 0: each stage's exact f16
 * codewords multiply x in their own f32 accumulators and the row gains
 * apply at the end, the reference's per-stage arithmetic
 * (decode-gpu.cu:359-501, one launch per stage there), about 16 % slower on
 * the FFN pair. Matrices whose codebooks do not fit LDS (8192 entries, two
 * stages) always use decoded f16 weight tiles. Returns the previous setting;
 * on < 0 only reads it. Calls that overlap a change see either setting. */
int sparkmv_prefill_fold(int on);

/* ---- decode-set plan: a recorded chain of matvec launches ----
 * The per-token matvec chain of the forward (tools/vq/gpu/vq-model-gpu.cu:776-835
 * issues it launch by launch from the host; the Rust runtime calls matvec at
 * tools/vq-runtime/src/model.rs:481-482, :559, :570-571, :575, :585-590).
 * A plan records the chain once with its device pointers and issues it
 * eagerly (sparkmv_plan_run) or replays it as one HIP graph
 * (sparkmv_plan_capture, then sparkmv_plan_launch). Ops run in record order
 * on one stream. No op clears memory with a memset, so capture is safe. */
void * sparkmv_plan_create(void);
void sparkmv_plan_destroy(void * plan);
int sparkmv_plan_size(void * plan);
/* Append one VQ launch over nmat matrices sharing x (as sparkmv_vq_gemv_multi). */
int sparkmv_plan_add_vq(void * plan, const sparkmv_vq_matrix * mats, int nmat, int nstages, int dim, int nc, int cols,
                        int v3, const void * x, int x_dtype, int ldx, int ncols, int ldy, int accumulate,
                        int variant);
/* Append one k-quant GEMV: kind 6 = Q6_K, 8 = Q8_0 (as sparkmv_q6k_gemv / _q8_0_gemv). */
int sparkmv_plan_add_kquant(void * plan, int kind, const void * blocks, int rows, int cols, const void * x,
                            int x_dtype, int ldx, int ncols, float * y, int ldy, int accumulate);
int sparkmv_plan_run(void * plan, void * stream);
/* Capture on a created (non-null) stream; run the plan eagerly once first. */
int sparkmv_plan_capture(void * plan, void * stream);
int sparkmv_plan_launch(void * plan, void * stream);
/* Average device milliseconds of each op over `iters` eager runs on `stream`:
 * the op's kernels carry start/stop events in their own dispatches
 * (hipExtLaunchKernel), so each figure is kernel time without launch gaps;
 * op_ms receives sparkmv_plan_size(plan) values. */
int sparkmv_plan_time_ops(void * plan, void * stream, int iters, double * op_ms);
/* Apply a trusted tuning profile (VQPROF 1) to the plan's VQ ops, as
 * tools/vq/gpu/vq-model-gpu.cu:300-324 applies one at load: each op takes its
 * geometry's gemv entry (every matrix of the op tuned alike) after the entry
 * is re-checked as runnable here (vqg_gemv_ready, a warp-multiple width); a
 * stale or non-ready entry keeps the heuristic. A profile measured for another
 * artifact fingerprint or device changes nothing (returns 0). Returns the
 * number of ops changed; the error text then counts the refused entries.
 * Drops a captured graph. */
int sparkmv_plan_apply_profile(void * plan, const void * profile, uint64_t artifact, const char * gpu);
/* The kernel op i runs (sparkmv_* numbering; -1 for a k-quant op) and its
 * launch width (0 = the kernel's own). */
int sparkmv_plan_op_kernel(void * plan, int i, int * variant, int * threads);

/* ---- decode chain: the per-token matvec chain as ONE persistent launch ----
 * Replaces the launch-by-launch chain of tools/vq/gpu/vq-model-gpu.cu:776-835
 * (gemv calls :795-833; rms_norm :364-380, gelu-mul :404-414 between them)
 * with one launch of one workgroup per CU that walks the op list. Every
 * output that a later op of the chain reads (found at build time by matching
 * pointers) is also published as 8-byte words {payload, epoch}, each written
 * with one agent-scope store; the reader's load of its words is its wait (it
 * reloads the words whose epoch is not yet current, with a bounded spin). So
 * every read of chain-produced data, x or addend, waits for exactly its own
 * words, and `wait` is accepted and ignored. An input that only partly
 * overlaps an earlier op's output, or an output over an earlier op's
 * external input, is refused at build. Each op's input transform runs inside its
 * staging: x_mode 0 takes bf16 x as is, 1 rounds f32 x to bf16, 2 applies
 * rms_norm to f32 x (f64 sum of squares, tools/vq-runtime/src/model.rs:236-245;
 * norm_w may be NULL for weight 1) and rounds to bf16. Each matrix writes
 * y = y_add + W x (y_add may be NULL) in f32 and, when y_bf16 is set, a bf16
 * copy. With act set, the op is a gate/up pair: two matrices of equal rows,
 * and act[r] = bf16(gelu(y0[r]) * y1[r]) with exact-erf gelu (model.rs:253-258).
 * x_out, when set, receives the staged bf16 x (the op's actual input).
 * Geometry: DQV3, dim 4, two stages, 12-bit indices (an even nc of 2050..4096), columns a multiple
 * of 128 up to 12288 (bf16 x) or 6144 (f32 x, norm), 4-byte aligned stages. A chain needs the device to
 * itself while it runs (every workgroup resident at once); the launch is
 * asynchronous and can be captured into a HIP graph. */
typedef struct {
    const void * stages[4];   /* device stage payloads (two used) */
    float * y;                /* f32 output, rows values (may be NULL if y_bf16 is set, or for a pair) */
    uint16_t * y_bf16;        /* bf16 copy of y (may be NULL) */
    const float * y_add;      /* addend (may be NULL; ignored for a pair) */
    int rows;
} sparkmv_chain_matrix;
void * sparkmv_chain_create(void);
void sparkmv_chain_destroy(void * chain);
int sparkmv_chain_size(void * chain);
/* Waves per workgroup (8, 12 or 16), macro steps of index words each wave
 * keeps in flight (2 or 4; 8 with 8 waves), and the units per workgroup the
 * shape search aims for (0: fewest rounds of units per wave); applies at
 * the next launch. */
int sparkmv_chain_tune(void * chain, int waves, int look, int min_units);
int sparkmv_chain_add_vq(void * chain, const sparkmv_chain_matrix * mats, int nmat, int nstages, int dim, int nc,
                         int cols, int v3, const void * x, int x_mode, const float * norm_w, float eps,
                         uint16_t * x_out, uint16_t * act, int wait);
/* An op with no matrix: out = bf16(rms_norm(x)) over n values (the head's input). */
int sparkmv_chain_add_norm(void * chain, const float * x, int n, const float * norm_w, float eps, uint16_t * out,
                           int wait);
int sparkmv_chain_launch(void * chain, void * stream);
/* 0, or -1 if a wait of any launch so far gave up (the error word is then
 * cleared); synchronizes the device. */
int sparkmv_chain_status(void * chain);
/* Phase trace of later launches into buf (device memory, NULL = off): per
 * workgroup w and op i, buf[(w * ops + i) * 10 + k] holds the 100 MHz clock
 * (low 32 bits) at the op's start, x arrived, x staged, step loop entered,
 * wave 0's steps done, every unit done, epilogue issued and x requested,
 * then the shader clock at the op's start and end. Returns the words needed
 * (workgroups * ops * 10), or -1 when words is too small. No counterpart in
 * the reference: a diagnostic of this chain. */
int sparkmv_chain_trace(void * chain, uint32_t * buf, long words);
/* The shape chosen for op i: MFMA parts S, K chunks C, macro steps per unit. */
int sparkmv_chain_op_shape(void * chain, int i, int * S, int * C, int * msc);

/* ---- launch start-up measurement ----
 * No counterpart in the reference: a measurement of this build's launches,
 * for the decode set's per-launch fixed cost. On the hot kernel's launch
 * shape (one workgroup of 10 waves per CU), kernel-exact, medians of reps
 * launches: out_us[0] an empty kernel, out_us[1] the same with one wave
 * per workgroup, out_us[2] staging 64 KB of codebooks into LDS (L2 flushed
 * before), then per size s (multiples of 16 bytes, 64 KB..1 GB) a plain read
 * of sizes[s] bytes cold (out_us[3 + 3s]), after one dword per 4 KB page of
 * it was read (address translation warm, data cold; out_us[4 + 3s]) and
 * after one dword per 64-byte line was read (data warm; out_us[5 + 3s]);
 * then, with n = nsizes, out_us[3 + 3n] an empty kernel of one workgroup of
 * one wave, out_us[4 + 3n] and out_us[5 + 3n] the wall time per launch of 64
 * empty full-shape launches back to back, eagerly and as one HIP graph
 * (plain events around all 64). Allocates and frees its own buffers
 * (largest size * reps + 640 MB); synchronizes the device. */
int sparkmv_probe_startup(const size_t * sizes, int nsizes, int reps, double * out_us);
/* The cost of one dependent handoff over every workgroup (one per CU), the
 * decode chain's per-op wait, three ways: mode 0 words carrying their epoch
 * (each reader reloads the words not yet current; the chain's protocol), 1
 * the same behind one sentinel word per producer, 2 an agent-scope fence and
 * an atomic counter per op, polled before reading. For each word count
 * nwords[i] (256..5120, words an op's reader loads), out_us[mode * nn + i] =
 * µs per op of a 400-op chain minus a 1-op chain, best of 5. No counterpart
 * in the reference. Needs the device to itself; synchronizes it. */
int sparkmv_probe_handoff(const int * nwords, int nn, double * out_us);
/* The floor of one launch per matvec with no compute: n plain reads of
 * sizes[i] bytes (4 KB..1 GB each, 16 GB in all), each from its own region,
 * on the hot kernel's launch shape, back to back as one captured HIP graph
 * (out_us[0], µs per replay) and eagerly on a stream (out_us[1], µs per
 * pass), medians of reps (3..64). No counterpart in the reference.
 * Allocates and frees its own buffer; synchronizes the device. */
int sparkmv_probe_read_chain(const size_t * sizes, int n, int reps, double * out_us);

/* ---- weight artifacts (host memory) ----
 * GGUF v2/v3 (ggml's layout), the reader of tools/dspark/src/gguf.rs:95-190
 * (Gguf::open, tensor_bytes, get_u64/get_f32/get_str/get_arr), extended to
 * Q6_K: tensor bytes are handed out for F32 (type 0), F16 (1), BF16 (30),
 * Q8_0 (8, 34 B per 32) and Q6_K (14, 210 B per 256); any other type is listed
 * with nbytes 0 and refused by number. ggml dims run fastest first: a 2-D
 * weight has dims {cols, rows}, its blocks row-major, the layout the k-quant
 * GEMVs take. The file is memory-mapped; data pointers live until close. */
typedef struct {
    char name[256];
    int ndims;
    uint64_t dims[4];
    uint32_t dtype;
    uint64_t offset;   /* from the start of the data section */
    uint64_t nbytes;   /* 0 for a type this reader does not hand out */
} sparkmv_gguf_tensor;

void * sparkmv_gguf_open(const char * path);   /* NULL on refusal */
void sparkmv_gguf_close(void * gguf);
int sparkmv_gguf_version(const void * gguf);
int64_t sparkmv_gguf_tensor_count(const void * gguf);
int64_t sparkmv_gguf_find(const void * gguf, const char * name);   /* -1 if absent */
int sparkmv_gguf_tensor_info(const void * gguf, int64_t i, sparkmv_gguf_tensor * out);
const void * sparkmv_gguf_tensor_data(const void * gguf, int64_t i, uint64_t * nbytes);   /* NULL on refusal */
int64_t sparkmv_gguf_kv_count(const void * gguf);
int sparkmv_gguf_kv_key(const void * gguf, int64_t i, char * key, int cap, uint32_t * type);
int sparkmv_gguf_get_u64(const void * gguf, const char * key, uint64_t * out);
int sparkmv_gguf_get_f64(const void * gguf, const char * key, double * out);
int sparkmv_gguf_get_str(const void * gguf, const char * key, char * out, int cap);
int64_t sparkmv_gguf_get_arr_len(const void * gguf, const char * key, uint32_t * elem);   /* -1 if absent */

/* The VQ artifact directory (manifest.txt + one <name>.bin per tensor),
 * VqDir of tools/vq-runtime/src/vq_source.rs:30-104. A read validates the
 * file against its manifest line: stages 0 is an RQVF f32 sidecar
 * (RawF32::open, tools/vq-format/src/lib.rs:325-350; kind 0, data = the
 * rows x cols f32), stages >= 1 an RQVQ container (Container::open; kind 1,
 * data = the whole file). data lives until the next read or close. */
void * sparkmv_manifest_open(const char * dir);   /* NULL on refusal */
void sparkmv_manifest_close(void * manifest);
int sparkmv_manifest_count(const void * manifest);
int sparkmv_manifest_entry(const void * manifest, int i, char * name, int cap, int * rows, int * cols, int * stages);
int sparkmv_manifest_read(void * manifest, const char * name, const void ** data, size_t * nbytes, int * kind);

/* ---- the decode forward: one token through every layer on the GPU ----
 * The reference's CPU forward (tools/vq-runtime/src/model.rs:441-591) and
 * its GPU runtime's (tools/vq/gpu/vq-model-gpu.cu:776-835): embedding row,
 * per layer rms_norm (f64 sums), qkv and the per-head attention gate, rope
 * over the first head_dim * partial elements, the KV store, GQA attention
 * over the full or sliding window times sigmoid(gate), the output projection
 * added to the residual, rms_norm, exact-erf gelu(gate) * up, down added to
 * the residual; final rms_norm and the tied head. The trunk's matrices are
 * VQ containers with one geometry (dim, nc, nstages, v3); the head is VQ (the
 * reference GPU runtime's embedding) or Q8_0 (the GGUF's token_embd). x_dtype
 * is what the matvecs read: SPARKMV_X_F32 follows the f32 reference, bf16
 * halves their activation bytes. The model owns its KV cache and scratch
 * (one device allocation at create); weights stay the caller's. */
typedef struct {
    int hidden, layers, heads, kv_heads, head_dim, intermediate, vocab;
    float eps;
    int sliding_window;                          /* positions a sliding layer sees */
    double rope_full_theta, rope_full_partial;   /* config.rs:87-108 */
    double rope_slide_theta, rope_slide_partial;
    int max_ctx;                                 /* KV cache positions, at most 131072 */
    int x_dtype;
    int dim, nc, nstages, v3;                    /* the VQ geometry of every matrix */
} sparkmv_model_cfg;

typedef struct {
    const float * in_norm, * post_norm;          /* device f32 [hidden] */
    const void * qkv[4];                         /* [q_dim + 2 kv_dim] x hidden, stage pointers */
    const void * attn_gate[4];                   /* [heads] x hidden */
    const void * out[4];                         /* hidden x q_dim */
    const void * gate[4], * up[4];               /* intermediate x hidden */
    const void * down[4];                        /* hidden x intermediate */
    int full;                                    /* 1 full attention, 0 sliding (config.rs:95-100) */
} sparkmv_model_layer;

void * sparkmv_model_create(const sparkmv_model_cfg * cfg);   /* NULL on refusal */
void sparkmv_model_destroy(void * model);
int sparkmv_model_set_layer(void * model, int layer, const sparkmv_model_layer * weights);
/* kind 0: a VQ head (stages), 8: Q8_0 blocks [vocab][hidden / 32]; final_norm device f32 [hidden]. */
int sparkmv_model_set_head(void * model, int kind, const void * const * stages, const void * blocks,
                           const float * final_norm);
/* One token at pos (model.rs:441): fills the cache row pos of every layer
 * and writes vocab f32 logits. Asynchronous on stream. */
int sparkmv_model_forward(void * model, uint32_t token, int pos, float * logits, void * stream);
/* Record one token's launches as a HIP graph that writes logits, on a
 * created (non-null) stream; token and position are read from device memory
 * the replay sets. Run sparkmv_model_forward once first (first-call setup
 * stays outside the capture). No launch in the graph clears memory with a
 * memset. */
int sparkmv_model_capture(void * model, float * logits, void * stream);
/* Set token and position, then replay the recorded graph (as forward). */
int sparkmv_model_replay(void * model, uint32_t token, int pos, void * stream);
/* A speculative-verify block (vq-model-gpu.cu:955-969 verify_logits over
 * forward_batch, :858-953): ntok <= 8 consecutive tokens at positions
 * pos .. pos + ntok - 1, each attending causally to the positions up to its
 * own; every matvec runs once over the block's columns and the head gives
 * logits [ntok][vocab] (a Q8_0 head column equals its one-column result bit
 * for bit). Fills those cache rows. Without a reservation the first block
 * allocates the model's block buffers. */
int sparkmv_model_verify(void * model, const uint32_t * tokens, int ntok, int pos, float * logits, void * stream);
/* A prompt chunk (vq-model-gpu.cu:858-943 forward_batch; with logits also
 * :946-953 tail_logits): ntok <= 512 consecutive tokens at positions
 * pos .. pos + ntok - 1, each attending causally to the positions up to its
 * own; fills those cache rows. Matvecs over up to 16 tokens run the batched
 * GEMV (each column the decode arithmetic); longer chunks run the prefill
 * GEMM, whose x enters the matrix cores as f16, as in the reference's prompt
 * path. logits, when non-null, receives the last token's vocab logits; NULL
 * skips the head, as forward_batch does between chunks. The host token array
 * is read before the call returns (it waits for the stream's earlier work).
 * Refused past max_ctx or the vocabulary. A chunk longer than the
 * reservation (re)allocates the block buffers after a device
 * synchronization; split-K prefills draw their partial sums from the
 * library's stream-ordered pool (allocated on first use, kept after). */
int sparkmv_model_forward_batch(void * model, const uint32_t * tokens, int ntok, int pos, float * logits,
                                void * stream);
/* Allocate the block buffers for verify blocks and prompt chunks of up to
 * ntok tokens (1..512; at least 8 are reserved) now, so that those calls
 * allocate nothing. A larger reservation than the current one synchronizes
 * the device and replaces the buffers. */
int sparkmv_model_reserve(void * model, int ntok);
/* Keep the first pos cached positions (model.rs:361-381 rollback): refused
 * past the cached length; later steps overwrite the rows it drops. */
int sparkmv_model_rollback(void * model, int pos);
/* The cached length: one past the last position a step wrote, or as rolled back. */
int sparkmv_model_len(void * model);
/* Apply a trusted tuning profile to the model's VQ matvecs per geometry,
 * with the same checks as sparkmv_plan_apply_profile (vq-model-gpu.cu:300-324).
 * Returns the number of geometries tuned; drops a captured graph. */
int sparkmv_model_apply_profile(void * model, const void * profile, uint64_t artifact, const char * gpu);
/* The kernel the model runs for a rows x cols VQ matvec (0, 0 = heuristic). */
int sparkmv_model_matvec_kernel(void * model, int rows, int cols, int * variant, int * threads);
/* The device rows of layer's K and V cache ([max_ctx][kv_dim] f32 each). */
int sparkmv_model_kv(void * model, int layer, float ** k, float ** v);
/* Layer-input capture for a draft (model.rs:322-348 enable_capture;
 * vq-model-gpu.cu:632-639, :704-736): from now on every forward, verify
 * block and prompt chunk writes the residual entering each listed layer
 * (model.rs:466-471), position-major, into the layer's slot; slot k is the
 * k-th listed layer. At most 8 layers, each once, enabled once; the
 * refusals carry the runtime's messages. A recorded graph is dropped
 * (capture again to record the copies). */
int sparkmv_model_enable_capture(void * model, const int * layers, int n);
/* Slot k's rows (model.rs:346-348 captured): *rows = the device array
 * [max_ctx][hidden] f32; returns how many leading rows are current (the
 * cached positions; a rollback drops the rest as it drops KV rows), or -1. */
int sparkmv_model_captured(void * model, int k, float ** rows);
/* The tied embedding row of token id into out ([hidden] f32, device),
 * asynchronous on stream (model.rs:352-354 embed_row). */
int sparkmv_model_embed_row(void * model, uint32_t id, float * out, void * stream);
/* The index of the largest of n device floats into *out (device int),
 * asynchronous on stream: Model::argmax (model.rs:594-605): the first of
 * equal maxima, NaN never chosen, 0 when no value exceeds -inf. Replaces
 * the runtime's argmax_dev (vq-model-gpu.cu:471-488, :971-978), whose tree
 * keeps the lowest thread's candidate on ties instead. */
int sparkmv_argmax(const float * logits, int n, int * out, void * stream);

/* A checkpoint's config.json (tools/vq-runtime/src/config.rs:39-85,
 * Config::load): hidden_size, num_hidden_layers, num_attention_heads,
 * num_key_value_heads, head_dim, intermediate_size, vocab_size,
 * rms_norm_eps and sliding_window are required ("config.json has no numeric
 * <key>"), and so is layer_types ("config.json has no layer_types"); a
 * layer is full when its entry is "full_attention", when the entry is not a
 * string, or when the list is shorter than the layers; rope_parameters
 * gives rope_theta and partial_rotary_factor per layer type, falling back
 * to 5e6 / 0.25 (full) and 1e4 / 1.0 (sliding), both kept in f32. Fills the
 * model fields of cfg (the VQ geometry, max_ctx and x_dtype are left 0) and
 * full[i] for i < max_layers. */
int sparkmv_config_load(const char * path, sparkmv_model_cfg * cfg, int * full, int max_layers);
/* A whole model from config.json and a VQ artifact directory (model.rs:
 * 121-185 Weights::load over VqDir; vq-model-gpu.cu:230-357, :739-775
 * load_model): model.embedding.weight (the tied head), model.norm.weight,
 * and per layer input_layernorm / post_attention_layernorm and the
 * q_k_v_proj, g_proj, out_proj, gate_proj, up_proj, down_proj matrices,
 * each checked against the architecture ("<name>: is RxC, the architecture
 * needs R'xC'"); every matrix must share one VQ geometry. The weights are
 * uploaded to device memory that the model owns and frees at
 * sparkmv_model_destroy. With apply_profile, DIR/vq-tune.profile is
 * applied when it is trusted for this artifact and device; like the
 * reference's runtime (vq-model-gpu.cu:1097-1120), a profile that is absent,
 * unreadable, not version 1 or for another artifact or device never fails
 * the load: the heuristic stays, and after a successful load the message
 * channel (vqg_decode_error) says which case applied. NULL on refusal, with
 * the message set. */
void * sparkmv_model_load(const char * dir, const char * config_path, int max_ctx, int x_dtype, int apply_profile);

/* ---- the per-artifact tuning profile (VQPROF 1) ----
 * tools/vq/gpu/vq-profile.h:10-30 (format, FNV-1a fingerprint, trust rules),
 * written by tools/vq-tune/src/artifact.rs:148-171. Host only. */
typedef struct {
    int kind;                    /* 0 gemv, 1 prefill */
    int dim, nc, rows, cols, v3;
    int variant;
    int threads;                 /* gemv */
    int bn, bk;                  /* prefill */
    double rate;                 /* the measured GB/s (gemv) or tokens/s (prefill) column */
} sparkmv_profile_entry;

/* The artifact directory's fingerprint (vq-profile.h:118-146). */
int sparkmv_profile_fingerprint(const char * dir, uint64_t * out);
/* Parse a profile; NULL unless it carries version 1 (vq-profile.h:155-193). */
void * sparkmv_profile_load(const char * path);
void sparkmv_profile_close(void * profile);
/* 1 when the profile's fingerprint and device name match, 0 when not (the
 * reason in the error text), -1 on bad arguments. */
int sparkmv_profile_trusted(const void * profile, uint64_t artifact, const char * gpu);
int sparkmv_profile_count(const void * profile);
int sparkmv_profile_entry_at(const void * profile, int i, sparkmv_profile_entry * out);
/* The entry for one geometry (vq-profile.h:195-203), -1 when there is none. */
int sparkmv_profile_find(const void * profile, int kind, int dim, int nc, int rows, int cols, int v3,
                         sparkmv_profile_entry * out);
/* Write a profile in the reference's format (at most 512 entries). */
int sparkmv_profile_write(const char * path, uint64_t artifact, const char * gpu, const char * driver,
                          const sparkmv_profile_entry * entries, int n);

/* ---- synthetic workloads (host memory; no reference counterpart) ----
 * A named, seeded generator so every test and benchmark can rebuild the same
 * inputs: xoshiro256** seeded through splitmix64; normals by Box-Muller in
 * f64, rounded to nearest-even. */
size_t sparkmv_synth_container_bytes(int rows, int cols, int dim, int nc, int nstages, int v3);
/* An RQVQ container: per stage a codebook ~N(0, 0.02) in fp16, gains
 * ~U(0.5, 1.5) in fp16, indices uniform in [0, nc). */
int sparkmv_synth_vq_container(uint64_t seed, int rows, int cols, int dim, int nc, int nstages, int v3,
                               void * out, size_t len);
/* Q6_K blocks: ql, qh uniform bytes, scales uniform in [-32, 31], d ~U(1e-4, 1e-3). */
int sparkmv_synth_q6k(uint64_t seed, int rows, int cols, void * out);
/* Q8_0 blocks: qs uniform in [-128, 127], d ~U(1e-4, 1e-3). */
int sparkmv_synth_q8_0(uint64_t seed, int rows, int cols, void * out);
/* n bf16 values ~N(0, 1). */
int sparkmv_synth_bf16_normal(uint64_t seed, size_t n, uint16_t * out);

#ifdef __cplusplus
}
#endif
#endif
