/* synth.cpp — seeded synthetic weights and activations in the on-disk
 * formats, so that tests and benchmarks rebuild identical inputs anywhere.
 *
 * Generator: xoshiro256** (Blackman and Vigna) whose state is filled by
 * splitmix64 from the seed. Uniform doubles take the top 53 bits; normals
 * are Box-Muller (cosine branch) in f64. fp16 and bf16 values are rounded to
 * nearest-even. Every stage of a container draws from its own stream, seeded
 * from (seed, stage), in the order codebook, gains, indices.
 *
 * The DQV3 packing follows the writer tools/vq/gpu/build-vq-gpu.c:71-111 and
 * the DQVQ packing tools/vq/vendor/vq_qc.h:241-264 (LSB-first bit fields,
 * DQV3 rows restart on a byte boundary, 13th bit in a trailing plane, DQVQ
 * carries one guard byte).
 */
#include <math.h>
#include <string.h>

#include <vector>

#include "../../../include/sparkmv.h"
#include "../common.h"

namespace sparkmv {
namespace synth {

static uint64_t splitmix64(uint64_t & s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

struct Rng {
    uint64_t s[4];
    explicit Rng(uint64_t seed) {
        uint64_t x = seed;
        for (int i = 0; i < 4; i++) s[i] = splitmix64(x);
    }
    static uint64_t rotl(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    double u01() { return (double) (next() >> 11) * 0x1.0p-53; }
    double normal() {
        const double u1 = u01(), u2 = u01();
        return sqrt(-2.0 * log(1.0 - u1)) * cos(6.283185307179586476925 * u2);
    }
};

static uint64_t derive(uint64_t seed, uint64_t k) {
    uint64_t x = seed ^ (k * 0xd1b54a32d192ed03ull);
    return splitmix64(x);
}

/* f64 -> fp16 bits, round to nearest even, overflow to infinity. */
static uint16_t to_f16(double v) {
    const uint16_t sign = signbit(v) ? 0x8000 : 0;
    const double a = fabs(v);
    if (isnan(a)) return sign | 0x7e00;
    if (a < 0x1.0p-14) return (uint16_t) (sign | (uint16_t) nearbyint(a * 0x1.0p24));  /* 1024 lands on the min normal */
    int e;
    const double m = frexp(a, &e);            /* a = m 2^e, m in [0.5, 1) */
    double r = nearbyint(ldexp(m, 11));       /* 11 significant bits */
    int E = e - 1;
    if (r == 2048.0) { r = 1024.0; E++; }
    if (E > 15) return sign | 0x7c00;
    return (uint16_t) (sign | ((E + 15) << 10) | ((int) r - 1024));
}

/* f64 -> f32 (round to nearest even) -> bf16 bits (round to nearest even). */
static uint16_t to_bf16(double v) {
    const float f = (float) v;
    uint32_t b;
    memcpy(&b, &f, 4);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((b >> 16) | 0x40);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t) (b >> 16);
}

static void put16(uint8_t * p, uint16_t v) { p[0] = (uint8_t) v; p[1] = (uint8_t) (v >> 8); }
static void put32(uint8_t * p, uint32_t v) { for (int k = 0; k < 4; k++) p[k] = (uint8_t) (v >> (8 * k)); }

/* OR an nbits-wide value into a zeroed LSB-first bit stream at bit `pos`. */
static void put_field(uint8_t * base, size_t pos, uint32_t v, int nbits) {
    uint64_t w = (uint64_t) v << (pos & 7);
    uint8_t * q = base + (pos >> 3);
    for (int k = 0; k < ((int) (pos & 7) + nbits + 7) / 8; k++) q[k] |= (uint8_t) (w >> (8 * k));
}

/* Uniform indices in [0, nc): power-of-two nc takes floor(64 / nbit) fields
 * from each draw, low bits first; otherwise a multiply-shift of 32 bits. */
struct IndexDraw {
    Rng & r;
    int nbit, per, left = 0;
    uint32_t nc;
    bool pow2;
    uint64_t cur = 0;
    IndexDraw(Rng & rng, int nc_) : r(rng), nbit(bits_for(nc_)), per(64 / bits_for(nc_)), nc((uint32_t) nc_),
                                    pow2((nc_ & (nc_ - 1)) == 0) {}
    uint32_t next() {
        if (!pow2) return (uint32_t) (((r.next() >> 32) * (uint64_t) nc) >> 32);
        if (!left) { cur = r.next(); left = per; }
        const uint32_t v = (uint32_t) (cur & ((1ull << nbit) - 1));
        cur >>= nbit;
        left--;
        return v;
    }
};

static size_t stage_bytes(int v3, int rows, int cols, int dim, int nc) {
    return make_layout(dim, nc, rows, cols, v3).bytes;
}

static void write_stage(uint64_t seed, int rows, int cols, int dim, int nc, int v3, uint8_t * out) {
    Rng r(seed);
    const Layout L = make_layout(dim, nc, rows, cols, v3);
    memset(out, 0, L.bytes);
    memcpy(out, v3 ? "DQV3" : "DQVQ", 4);
    put16(out + 4, (uint16_t) dim);
    put16(out + 6, (uint16_t) nc);
    put32(out + 8, (uint32_t) rows);
    put32(out + 12, (uint32_t) cols);
    if (v3) put32(out + 16, L.nbit > 12 ? 1u : 0u);   /* flags; 4 pad bytes stay zero */
    uint8_t * p = out + L.cb_off;
    for (size_t i = 0; i < (size_t) nc * dim; i++) put16(p + 2 * i, to_f16(0.02 * r.normal()));
    p = out + L.gain_off;
    for (int i = 0; i < rows; i++) put16(p + 2 * (size_t) i, to_f16(0.5 + r.u01()));
    uint8_t * st = out + L.stream_off;
    IndexDraw draw(r, nc);
    if (v3) {
        uint8_t * plane = st + (size_t) rows * L.mrow;
        for (size_t row = 0; row < (size_t) rows; row++) {
            uint8_t * m = st + row * L.mrow;
            if (L.mb == 12 && L.nbit == 12) {
                size_t i = 0;
                for (; i + 1 < L.nidx_row; i += 2) {   /* two 12-bit fields fill three bytes */
                    const uint32_t a = draw.next(), b = draw.next();
                    uint8_t * q = m + (i / 2) * 3;
                    q[0] = (uint8_t) a;
                    q[1] = (uint8_t) ((a >> 8) | (b << 4));
                    q[2] = (uint8_t) (b >> 4);
                }
                for (; i < L.nidx_row; i++) put_field(m, i * 12, draw.next(), 12);
            } else {
                for (size_t i = 0; i < L.nidx_row; i++) {
                    const uint32_t v = draw.next();
                    put_field(m, i * (size_t) L.mb, v & ((1u << L.mb) - 1u), L.mb);
                    if (L.prow) put_field(plane + row * L.prow, i, (v >> 12) & 1u, 1);
                }
            }
        }
    } else {
        const size_t nidx = (size_t) rows * L.nidx_row;
        for (size_t i = 0; i < nidx; i++) {
            const uint32_t v = draw.next();
            if (L.nbit == 8) st[i] = (uint8_t) v;
            else put_field(st, i * (size_t) L.nbit, v, L.nbit);
        }
    }
}

}  // namespace synth
}  // namespace sparkmv

using namespace sparkmv;

extern "C" size_t sparkmv_synth_container_bytes(int rows, int cols, int dim, int nc, int nstages, int v3) {
    if (rows <= 0 || cols <= 0 || dim <= 0 || nc <= 0 || nstages <= 0 || cols % dim) return 0;
    return 32 + (size_t) nstages * synth::stage_bytes(v3, rows, cols, dim, nc);
}

extern "C" int sparkmv_synth_vq_container(uint64_t seed, int rows, int cols, int dim, int nc, int nstages, int v3,
                                          void * out, size_t len) {
    const size_t want = sparkmv_synth_container_bytes(rows, cols, dim, nc, nstages, v3);
    if (!want || nstages > 65535 || nc > 65535 || dim > 65535) { set_error("synthetic container geometry is invalid"); return -1; }
    if (v3 && bits_for(nc) > 13) { set_error("DQV3 carries 13 index bits, nc %d needs %d", nc, bits_for(nc)); return -1; }
    if (!out || len < want) { set_error("synthetic container needs %zu bytes, got %zu", want, len); return -1; }
    uint8_t * b = (uint8_t *) out;
    memset(b, 0, 32);
    memcpy(b, "RQVQ", 4);
    synth::put16(b + 4, (uint16_t) dim);
    synth::put16(b + 6, (uint16_t) nc);
    synth::put16(b + 8, (uint16_t) nstages);
    synth::put32(b + 12, (uint32_t) rows);
    synth::put32(b + 16, (uint32_t) cols);
    const size_t per = synth::stage_bytes(v3, rows, cols, dim, nc);
    const uint64_t payload = (uint64_t) per * (uint64_t) nstages;
    synth::put32(b + 24, (uint32_t) payload);
    synth::put32(b + 28, (uint32_t) (payload >> 32));
    for (int s = 0; s < nstages; s++)
        synth::write_stage(synth::derive(seed, (uint64_t) s + 1), rows, cols, dim, nc, v3, b + 32 + (size_t) s * per);
    return 0;
}

extern "C" int sparkmv_synth_q6k(uint64_t seed, int rows, int cols, void * out) {
    if (rows <= 0 || cols <= 0 || cols % 256 || !out) { set_error("Q6_K needs cols a multiple of 256"); return -1; }
    synth::Rng r(seed);
    uint8_t * p = (uint8_t *) out;
    const size_t nb = (size_t) rows * (cols / 256);
    for (size_t b = 0; b < nb; b++, p += 210) {
        for (int i = 0; i < 192; i += 8) {           /* ql[128] then qh[64], uniform bytes */
            const uint64_t v = r.next();
            for (int k = 0; k < 8; k++) p[i + k] = (uint8_t) (v >> (8 * k));
        }
        for (int j = 0; j < 16; j++) p[192 + j] = (uint8_t) (int8_t) ((int) (r.next() >> 58) - 32);
        synth::put16(p + 208, synth::to_f16(1e-4 + 9e-4 * r.u01()));
    }
    return 0;
}

extern "C" int sparkmv_synth_q8_0(uint64_t seed, int rows, int cols, void * out) {
    if (rows <= 0 || cols <= 0 || cols % 32 || !out) { set_error("Q8_0 needs cols a multiple of 32"); return -1; }
    synth::Rng r(seed);
    uint8_t * p = (uint8_t *) out;
    const size_t nb = (size_t) rows * (cols / 32);
    for (size_t b = 0; b < nb; b++, p += 34) {
        synth::put16(p, synth::to_f16(1e-4 + 9e-4 * r.u01()));
        for (int i = 0; i < 32; i += 8) {
            const uint64_t v = r.next();
            for (int k = 0; k < 8; k++) p[2 + i + k] = (uint8_t) (v >> (8 * k));
        }
    }
    return 0;
}

extern "C" int sparkmv_synth_bf16_normal(uint64_t seed, size_t n, uint16_t * out) {
    if (!out) { set_error("output is null"); return -1; }
    synth::Rng r(seed);
    for (size_t i = 0; i < n; i++) out[i] = synth::to_bf16(r.normal());
    return 0;
}
