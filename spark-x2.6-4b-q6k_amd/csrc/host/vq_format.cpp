/* vq_format.cpp — container and stage validation; see vq_format.hpp. */
#include "vq_format.hpp"

#include <string.h>

namespace sparkmv {
namespace fmt {

static uint16_t u16le(const uint8_t * b, size_t o) { return (uint16_t) (b[o] | (b[o + 1] << 8)); }
static uint32_t u32le(const uint8_t * b, size_t o) {
    return (uint32_t) b[o] | ((uint32_t) b[o + 1] << 8) | ((uint32_t) b[o + 2] << 16) | ((uint32_t) b[o + 3] << 24);
}
static uint64_t u64le(const uint8_t * b, size_t o) { return (uint64_t) u32le(b, o) | ((uint64_t) u32le(b, o + 4) << 32); }

static int index_bits(size_t nc) {
    int b = 1;
    while (((size_t) 1 << b) < nc) b++;
    return b;
}

float f16(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t) h >> 10) & 0x1fu;
    uint32_t m = (uint32_t) h & 0x3ffu;
    uint32_t bits;
    if (e == 0 && m == 0) {
        bits = sign;
    } else if (e == 0) {
        int shift = 0;                       /* normalise the subnormal significand */
        while (!(m & 0x400u)) { m <<= 1; shift++; }
        bits = sign | ((uint32_t) (113 - shift) << 23) | ((m & 0x3ffu) << 13);
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Index stream bytes of one stage: the row-local DQV3 stream (plus plane
 * above 12 bits) or the matrix-wide DQVQ stream with its guard byte. */
static void stream_geometry(bool v3, size_t rows, size_t cols, size_t dim, int nbit,
                            size_t & mrow, size_t & prow, size_t & idx) {
    const size_t nidx_row = cols / dim;
    if (v3) {
        const size_t mb = nbit > 12 ? 12 : (size_t) nbit;
        mrow = (nidx_row * mb + 7) / 8;
        prow = nbit > 12 ? (nidx_row + 7) / 8 : 0;
        idx = rows * (mrow + prow);
    } else {
        const size_t nidx = rows * nidx_row;
        mrow = prow = 0;
        idx = nbit == 8 ? nidx : (nidx * (size_t) nbit + 7) / 8 + 1;
    }
}

static std::string width_refusal(size_t nc, int nbit) {
    return "DQV3 carries 13 index bits, nc " + std::to_string(nc) + " needs " + std::to_string(nbit) +
           "; rewrite with --format v2";
}

bool open_stage(const uint8_t * p, size_t len, StageView & st, std::string & err) {
    const bool v3 = len >= 4 && memcmp(p, "DQV3", 4) == 0;
    if (len < 16 || (!v3 && memcmp(p, "DQVQ", 4) != 0)) {
        err = "stage payload magic is neither DQVQ nor DQV3";
        return false;
    }
    const size_t hdr = v3 ? 24 : 16;
    const size_t dim = u16le(p, 4), nc = u16le(p, 6), rows = u32le(p, 8), cols = u32le(p, 12);
    if (!dim || !nc || !rows || !cols || cols % dim) {
        err = "stage header is inconsistent";
        return false;
    }
    const size_t cb_len = nc * dim * 2, gain_len = rows * 2;
    if (len < hdr + cb_len + gain_len) {
        err = "stage payload is truncated";
        return false;
    }
    const int nbit = index_bits(nc);
    if (v3 && nbit > 13) {
        err = width_refusal(nc, nbit);
        return false;
    }
    size_t mrow, prow, idx;
    stream_geometry(v3, rows, cols, dim, nbit, mrow, prow, idx);
    if (len < hdr + cb_len + gain_len + idx) {
        err = "stage index stream is truncated";
        return false;
    }
    st.dim = (int) dim; st.nc = (int) nc; st.rows = (int) rows; st.cols = (int) cols;
    st.nbit = nbit; st.v3 = v3; st.mrow = mrow; st.prow = prow;
    st.bytes = hdr + cb_len + gain_len + idx;
    st.base = p;
    return true;
}

bool open_container(const uint8_t * buf, size_t len, ContainerView & c, std::string & err) {
    if (len < 32 || memcmp(buf, "RQVQ", 4) != 0) {
        err = "not an RQVQ container";
        return false;
    }
    const size_t dim = u16le(buf, 4), nc = u16le(buf, 6), ns = u16le(buf, 8);
    const size_t rows = u32le(buf, 12), cols = u32le(buf, 16);
    const uint64_t payload = u64le(buf, 24);
    if (!dim || !nc || !ns || !rows || !cols) {
        err = "container header is inconsistent";
        return false;
    }
    const int nbit = index_bits(nc);
    const bool v3 = len >= 36 && memcmp(buf + 32, "DQV3", 4) == 0;
    if (v3 && nbit > 13) {
        err = width_refusal(nc, nbit);
        return false;
    }
    size_t mrow, prow, idx;
    stream_geometry(v3, rows, cols, dim, nbit, mrow, prow, idx);
    const size_t per = (v3 ? 24 : 16) + nc * dim * 2 + rows * 2 + idx;
    if (payload != (uint64_t) (ns * per)) {
        err = "payload byte count says " + std::to_string(payload) + ", layout implies " + std::to_string(ns * per);
        return false;
    }
    if ((uint64_t) len != 32 + payload) {
        err = "file is " + std::to_string(len) + " bytes, header and payload are " + std::to_string(32 + payload);
        return false;
    }
    c = ContainerView();
    c.dim = (int) dim; c.nc = (int) nc; c.rows = (int) rows; c.cols = (int) cols;
    c.nbit = nbit; c.v3 = v3; c.payload = payload; c.stride = per;
    for (size_t s = 0; s < ns; s++) {
        StageView st;
        if (!open_stage(buf + 32 + s * per, per, st, err)) return false;
        if ((size_t) st.rows != rows || (size_t) st.cols != cols || (size_t) st.dim != dim || (size_t) st.nc != nc) {
            err = "stage " + std::to_string(s) + " disagrees with the container header";
            return false;
        }
        c.stages.push_back(st);
    }
    return true;
}

}  // namespace fmt
}  // namespace sparkmv
