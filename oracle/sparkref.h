/* sparkref.h — the oracle: a CPU restatement of the reference's quantized
 * matvec path, used ONLY as test infrastructure (tests/, the smoke check and
 * the CPU-baseline leg of bench.py). Nothing in the product library links,
 * loads or calls it.
 *
 * Each function names the reference file:line it restates. Q6_K and Q8_0 have
 * no code in the reference (its ggml copy is absent); they restate ggml's
 * published block layout and are pinned by closed-form known answers only.
 */
#ifndef SPARKREF_H
#define SPARKREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ---- */
float sr_f16(uint16_t h);   /* tools/vq-format/src/lib.rs:50-72 */
float sr_bf16(uint16_t h);  /* tools/vq-runtime/src/safetensors.rs:187 */

/* ---- one residual stage (DQVQ or DQV3) ---- */
typedef struct {
    int dim, nc, rows, cols, nbit, v3;
    size_t mrow, prow;       /* DQV3 bytes per row of main stream and plane */
    size_t bytes;            /* payload bytes this stage occupies */
    const uint8_t * gains;
    const uint8_t * stream;
    size_t stream_len;       /* bytes from `stream` to the end of the given buffer */
    float * cb32;            /* codebook widened to f32 */
} sr_stage;

/* Parse a stage payload; 0 = ok, -1 = error with a message in err.
 * tools/vq-format/src/lib.rs:94-156 */
int  sr_stage_open(const uint8_t * p, size_t len, sr_stage * st, char * err, size_t errn);
void sr_stage_close(sr_stage * st);
/* Index of group i in row; lib.rs:162-189 (reads past the stream read as 0). */
uint32_t sr_stage_index(const sr_stage * st, size_t row, size_t i);
float sr_stage_gain(const sr_stage * st, size_t row);               /* lib.rs:192-194 */
void sr_stage_add_into(const sr_stage * st, float * out);           /* lib.rs:197-211 */
void sr_stage_dot_row(const sr_stage * st, size_t r, const float * x, float * acc); /* lib.rs:215-227 */

/* Validate an RQVQ container; fills the stage count and per-stage stride.
 * lib.rs:240-306. Returns 0 or -1 with err. */
int sr_container_check(const uint8_t * buf, size_t len, int * nstages, size_t * per,
                       int * rows, int * cols, int * dim, int * nc, int * v3,
                       char * err, size_t errn);
/* Container::decode, lib.rs:309-315: stages summed into a zeroed f32 matrix. */
int sr_container_decode(const uint8_t * buf, size_t len, float * out, char * err, size_t errn);
/* Fused path of tools/dqvq/src/main.rs:131-141: y zeroed, then every stage's
 * dot_row over every row, stage 0 first. nthreads splits rows (each row's
 * arithmetic order is unchanged by the split). */
int sr_container_gemv_fused(const uint8_t * buf, size_t len, const float * x, float * y,
                            int nthreads, char * err, size_t errn);

/* ---- runtime matvec ---- */
float sr_dot(const float * a, const float * b, size_t n);     /* model.rs:209-226 */
/* model.rs:228-234: y[r] = dot(W row r, x), rows split across threads. */
void sr_matvec(const float * W, size_t rows, size_t cols, const float * x, float * y, int nthreads);
/* The reference gate's host matvec in f64 (tools/vq/gpu/decode-gpu.c:469-484). */
void sr_matvec_f64(const float * W, size_t rows, size_t cols, const float * x, double * y, int nthreads);

/* ---- DQV3 / DQVQ writers (the byte layout the readers must accept) ---- */
size_t sr_stage_bytes(int v3, int rows, int cols, int dim, int nc);   /* decode.c:107-125 */
/* tools/vq/gpu/build-vq-gpu.c:71-111, taking fp16 bits instead of f32 */
size_t sr_v3_pack(const uint16_t * cb, const uint32_t * idx, const uint16_t * gains,
                  int rows, int cols, int dim, int nc, uint8_t * out);
/* tools/vq/vendor/vq_qc.h:241-264, taking fp16 bits instead of f32 */
size_t sr_vq_pack(const uint16_t * cb, const uint32_t * idx, const uint16_t * gains,
                  int rows, int cols, int dim, int nc, uint8_t * out);

/* ---- ggml k-quant blocks (published ggml layout; parity pinned by closed form) ----
 * block_q6_K: ql[128] | qh[64] | int8 scales[16] | fp16 d    = 210 B / 256 weights
 * block_q8_0: fp16 d | int8 qs[32]                           =  34 B /  32 weights
 * Block sizes: tools/kquant/stubs.c:25,:30,:39,:44; tools/dspark/src/gguf.rs:201. */
void sr_q6k_dequant(const uint8_t * blocks, size_t nblocks, float * out);
void sr_q8_0_dequant(const uint8_t * blocks, size_t nblocks, float * out);
/* Row-major [rows][cols/blk] blocks; y[r] = sr_dot(dequant(row r), x). */
void sr_q6k_matvec(const uint8_t * blocks, size_t rows, size_t cols, const float * x, float * y, int nthreads);
void sr_q8_0_matvec(const uint8_t * blocks, size_t rows, size_t cols, const float * x, float * y, int nthreads);

int sr_hardware_threads(void);

#ifdef __cplusplus
}
#endif
#endif
