/* common.h — shared definitions of the sparkmv library (gfx950, wave64).
 *
 * The stage layout below is the DQVQ / DQV3 payload of one residual VQ stage
 * (tools/vq-format/src/lib.rs:1-21, :94-156; writer tools/vq/gpu/build-vq-gpu.c:71-111):
 *
 *   DQVQ: 'DQVQ' u16 dim u16 nc u32 rows u32 cols            (16 B header)
 *   DQV3: 'DQV3' u16 dim u16 nc u32 rows u32 cols u32 flags u32 pad (24 B)
 *   then  f16 codebook [nc][dim], f16 gains [rows], index stream.
 *
 * DQVQ numbers nbit = ceil(log2 nc) bits across the whole matrix (a byte per
 * index at exactly 8 bits, else a bit stream plus one guard byte). DQV3
 * restarts a min(nbit, 12)-bit LSB-first stream at every row (mrow bytes per
 * row) and stores a 13th bit, when nbit is 13, in a plane of prow bytes per row
 * after all main rows.
 */
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sparkmv {

struct Layout {
    int dim, nc, rows, cols, nbit, v3, mb;  /* mb: bits per main-stream field */
    size_t cb_off, gain_off, stream_off;    /* byte offsets inside the stage payload */
    size_t nidx_row, mrow, prow, idx_bytes, bytes;
};

inline int bits_for(int nc) {
    int b = 1;
    while ((1L << b) < (long) nc) b++;
    return b;
}

/* Payload geometry of one stage; tools/vq-format/src/lib.rs:123-137 and
 * tools/vq/decode.c:107-125 compute the same byte counts. */
inline Layout make_layout(int dim, int nc, int rows, int cols, int v3) {
    Layout L;
    L.dim = dim; L.nc = nc; L.rows = rows; L.cols = cols; L.v3 = v3 ? 1 : 0;
    L.nbit = bits_for(nc);
    L.mb = L.v3 ? (L.nbit > 12 ? 12 : L.nbit) : L.nbit;
    L.nidx_row = dim > 0 ? (size_t) cols / (size_t) dim : 0;
    L.cb_off = L.v3 ? 24 : 16;
    L.gain_off = L.cb_off + (size_t) nc * (size_t) dim * 2;
    L.stream_off = L.gain_off + (size_t) rows * 2;
    if (L.v3) {
        L.mrow = (L.nidx_row * (size_t) L.mb + 7) / 8;
        L.prow = L.nbit > 12 ? (L.nidx_row + 7) / 8 : 0;
        L.idx_bytes = (size_t) rows * (L.mrow + L.prow);
    } else {
        const size_t nidx = (size_t) rows * L.nidx_row;
        L.mrow = 0; L.prow = 0;
        L.idx_bytes = L.nbit == 8 ? nidx : (nidx * (size_t) L.nbit + 7) / 8 + 1;
    }
    L.bytes = L.stream_off + L.idx_bytes;
    return L;
}

/* Error reporting shared by every entry point: a static message buffer, the
 * convention of tools/vq/gpu/decode-gpu.cu:21-28 (not thread-safe, like it). */
void set_error(const char * fmt, ...) __attribute__((format(printf, 1, 2)));
int fail_hip(const char * what, hipError_t e);

/* Device properties cached per device. */
int cu_count();

/* Kernel-exact timing. While `stop` is set (the plan's timing pass sets it
 * around one op), hot-path launches carry the events in the dispatch itself
 * (hipExtLaunchKernel): `start` is recorded as the op's first kernel begins
 * and `stop` as its last one ends, so their difference is device time with
 * no launch gap in it. */
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchEvents g_launch_events;

template <typename F, typename... Args>
inline void launch_kernel(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Args... args) {
    if (g_launch_events.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, lds, s, g_launch_events.start, g_launch_events.stop, 0, args...);
        g_launch_events.start = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
    }
}

constexpr int kMaxStages = 4;   /* residual stages one fused launch accepts */
constexpr int kMaxCols = 16;    /* activation columns one batched launch accepts (the MFMA N width) */

}  // namespace sparkmv
