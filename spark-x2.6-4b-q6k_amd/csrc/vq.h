/* vq.h — host-side launchers of the VQ kernels (vq_kernels.hip). */
#pragma once

#include "common.h"

namespace sparkmv {

/* One matrix of a VQ launch: a device pointer per residual stage payload and
 * its output, y[n * ldy + r] for column n. */
struct VqMatDesc {
    const void * stages[kMaxStages];
    float * y;
    int rows;
};

constexpr int kMaxMats = 8;   /* matrices one launch may share an x between */

/* A fused VQ GEMV call: every matrix shares dim, nc, cols, format, stage count
 * and the activations x[n * ldx + c] (bf16 bits, or f32 when xf32), n < ncol.
 * accumulate = 1 adds into y (the reference's convention); 0 overwrites. */
struct VqCall {
    int dim, nc, cols, v3, nst;
    const VqMatDesc * mats;
    int nmat;
    const void * x;
    int ldx, xf32, ncol, ldy, accumulate;
    hipStream_t stream;
    int variant;   /* 0 auto, 1 generic, 2 LDS-codebook wave kernel, 3 MFMA block kernel */
    int threads;   /* workgroup width, a multiple of 64; 0 = the default */
    int grid;      /* workgroups; 0 = the default */
    /* Zeroed 64-bit words (kslot_cap of them) through which workgroups that
     * share a tile's K chunks meet (several columns, one matrix): two of
     * them per element with x read from global memory (rows * ncol words),
     * or chunk groups in a tree with x staged per group (rows * ncol *
     * vq_ck_words(groups)); null keeps every tile inside one workgroup. They are
     * zero again when a launch ends; launches that share them must not
     * overlap. */
    uint64_t * kslot = nullptr;
    long kslot_cap = 0;
};

/* Chunk-split tiles: at most this many chunk groups per tile, whose sums
 * meet in a binary tree of vq_ck_words(groups) exchange words per output
 * element (the nodes of each level: half the subtrees of the level below,
 * rounded up). */
constexpr int kVqCkMaxGroups = 8;
inline int vq_ck_words(int C) {
    int t = 0;
    for (int n = C; n > 1; n = (n + 1) >> 1) t += (n + 1) >> 1;
    return t;
}

/* The kernel a profile's gemv entry (tools/vq/gpu/vq-profile.h, the
 * reference's variant numbering) asks for on one geometry, re-checked for
 * runnability as tools/vq/gpu/vq-model-gpu.cu:300-324 does: 1 with *variant
 * (VqCall numbering) and *threads set; 0 when the profile has no entry; -1
 * when its entry is not runnable here (unknown or not-ready variant, or a
 * width that is not a warp multiple up to 1024), so the heuristic stays. */
int profile_gemv_pick(const void * profile, int dim, int nc, int rows, int cols, int v3, int * variant, int * threads);

/* Whether a kernel variant runs this geometry (same numbering as VqCall). */
int vq_variant_ready(int dim, int nc, int rows, int cols, int v3, int variant);
/* Validate and launch; returns 0, or -1 with the message set. */
int vq_launch(const VqCall & c);
/* A gate/up pair's activation written by the launch that computes the pair
 * (c.nmat == 2, equal rows, bf16 columns: one, or several staged in LDS):
 * besides y of both matrices, act[n * rows + r] = gelu(gate[n][r]) *
 * up[n][r] (f32, when act is set) and its bf16 (act16, when set), the bits
 * the separate activation kernel would write. slot holds cap zeroed 64-bit
 * words (cap >= rows * ncol) through which the two matrices' elements meet; they are zero again when the launch ends, and
 * launches that share them must not overlap. vq_norm_launch with a pair
 * does the same from the f32 residual. Both return 1 without launching when
 * the call's shape has no kernel that writes the activation; the caller
 * then runs its own. */
struct VqPair {
    uint64_t * slot;
    int cap;
    float * act;
    uint16_t * act16;
};
int vq_pair_launch(const VqCall & c, const VqPair & pair);

/* The same launch with x = bf16(rms_norm(h) * norm_w) staged by the kernel
 * itself from the f32 residual h = c.x (c.xf32 is ignored; x_out, when
 * non-null, receives those bf16 values). Only for calls the one-column
 * straight-line kernel takes: returns 1 without launching otherwise (the
 * caller then runs the norm and vq_launch), 0 after the launch, -1 on a
 * launch error. */
int vq_norm_launch(const VqCall & c, const float * norm_w, float eps, uint16_t * x_out, const VqPair * pair = nullptr);

/* Decode one stage into out (row-major rows x cols f32); accumulate 0 writes
 * the stage's values as if adding into zeros. */
int vq_dequant_launch(const void * payload, const Layout & L, float * out, int accumulate, hipStream_t s);
/* Decode one row of one stage into out (cols f32), accumulating. */
int vq_row_dequant_launch(const void * payload, const Layout & L, int row, float * out, hipStream_t s);
/* the same with the rows read from device memory at run time: row
 * drow[i] into out + i * ldo, for i < nrows */
int vq_row_dequant_dev_launch(const void * payload, const Layout & L, const int * drow, float * out, hipStream_t s,
                              int nrows = 1, size_t ldo = 0);
/* y[r] += dot(W row r, x): the plain f32 bandwidth yardstick. */
int f32_gemv_launch(const float * w, const float * x, float * y, int rows, int cols, hipStream_t s);

}  // namespace sparkmv
