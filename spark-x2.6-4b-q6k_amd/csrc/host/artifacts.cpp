/* artifacts.cpp — readers of the two weight artifacts the path loads.
 *
 * 1. The VQ artifact directory written by build-vq / build-vq-gpu: a
 *    manifest.txt ("name rows cols stages file_bytes relL2" per line) and one
 *    <name>.bin per tensor, an RQVQ container (stages >= 1) or an RQVF raw f32
 *    sidecar (stages 0, the norms). Restates VqDir (tools/vq-runtime/src/
 *    vq_source.rs:30-104) and RawF32::open (tools/vq-format/src/lib.rs:325-350):
 *    the manifest is the index, and a missing file or a header that disagrees
 *    with it is an error, never a silent zero tensor.
 * 2. GGUF v2/v3 files (ggml's published layout: header, typed key/value table,
 *    tensor table, data at align_up(end of table, general.alignment or 32) +
 *    each tensor's offset), as tools/dspark/src/gguf.rs:95-190 reads them.
 *    That reader refuses Q6_K; this one hands out the bytes of F32, F16, BF16,
 *    Q8_0 (34 B per 32) and Q6_K (210 B per 256) tensors, the block layouts
 *    the k-quant GEMV kernels take as they are, and refuses other types by
 *    number.
 *
 * Host only: they validate and hand out bytes; uploads and matvecs are the
 * caller's. GGUF files are memory-mapped read-only, so a tensor's bytes are a
 * pointer into the mapping, valid until the handle is closed. */
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "../../../include/sparkmv.h"
#include "../common.h"
#include "vq_format.hpp"

namespace sparkmv {
namespace art {

/* ------------------------------------------------------------------ GGUF */

constexpr uint32_t kGgufMagic = 0x46554747u;   /* "GGUF" little-endian */

enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

struct KvValue {
    uint32_t type = 0;
    bool has_u64 = false, has_f64 = false;
    uint64_t u = 0;
    double f = 0.0;
    std::string s;
    uint32_t elem = 0;     /* arrays: element type and count */
    uint64_t count = 0;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t dtype = 0;
    uint64_t offset = 0;
};

struct Gguf {
    int fd = -1;
    const uint8_t * map = nullptr;
    size_t len = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_start = 0;
    std::vector<std::pair<std::string, KvValue>> kv;
    std::map<std::string, size_t> kv_index;
    std::vector<TensorInfo> tensors;
    std::map<std::string, size_t> tensor_index;
    ~Gguf() {
        if (map) munmap((void *) map, len);
        if (fd >= 0) close(fd);
    }
};

/* A bounds-checked little-endian cursor: any read past the end fails. */
struct Cursor {
    const uint8_t * b;
    size_t n, p = 0;
    bool take(size_t k, const uint8_t ** out) {
        if (k > n - p) return false;
        *out = b + p;
        p += k;
        return true;
    }
    template <typename T>
    bool get(T & v) {
        const uint8_t * q;
        if (!take(sizeof(T), &q)) return false;
        memcpy(&v, q, sizeof(T));
        return true;
    }
    bool str(std::string & s) {
        uint64_t k;
        const uint8_t * q;
        if (!get(k) || k > n - p || !take((size_t) k, &q)) return false;
        s.assign((const char *) q, (size_t) k);
        return true;
    }
};

/* One typed value; arrays are walked element by element for their width
 * and kept as (element type, count). */
static bool read_value(Cursor & c, uint32_t type, KvValue & v, int depth, std::string & err) {
    v.type = type;
    auto num_u = [&](uint64_t x) { v.u = x; v.has_u64 = true; v.f = (double) x; v.has_f64 = true; };
    auto num_i = [&](int64_t x) {
        if (x >= 0) { v.u = (uint64_t) x; v.has_u64 = true; }
        v.f = (double) x; v.has_f64 = true;
    };
    switch (type) {
        case kU8: { uint8_t x; if (!c.get(x)) break; num_u(x); return true; }
        case kI8: { int8_t x; if (!c.get(x)) break; num_i(x); return true; }
        case kU16: { uint16_t x; if (!c.get(x)) break; num_u(x); return true; }
        case kI16: { int16_t x; if (!c.get(x)) break; num_i(x); return true; }
        case kU32: { uint32_t x; if (!c.get(x)) break; num_u(x); return true; }
        case kI32: { int32_t x; if (!c.get(x)) break; num_i(x); return true; }
        case kU64: { uint64_t x; if (!c.get(x)) break; num_u(x); return true; }
        case kI64: { int64_t x; if (!c.get(x)) break; num_i(x); return true; }
        case kF32: { float x; if (!c.get(x)) break; v.f = x; v.has_f64 = true; return true; }
        case kF64: { double x; if (!c.get(x)) break; v.f = x; v.has_f64 = true; return true; }
        case kBool: { uint8_t x; if (!c.get(x)) break; num_u(x != 0); return true; }
        case kString: if (!c.str(v.s)) break; return true;
        case kArray: {
            uint32_t elem;
            uint64_t count;
            if (!c.get(elem) || !c.get(count)) break;
            /* a count the remaining bytes cannot hold is corruption */
            if (elem != kArray && count > (uint64_t) (c.n - c.p) + 1) {
                err = "array of " + std::to_string(count) + " elements does not fit the file";
                return false;
            }
            if (depth > 4) { err = "arrays nested too deep"; return false; }
            v.elem = elem;
            v.count = count;
            for (uint64_t k = 0; k < count; k++) {
                KvValue e;
                if (!read_value(c, elem, e, depth + 1, err)) return false;
            }
            return true;
        }
        default:
            err = "metadata value type " + std::to_string(type) + " is not supported";
            return false;
    }
    err = "unexpected end of file";
    return false;
}

/* Bytes of a tensor of `ne` elements, for the types this reader hands out
 * (0 with `err` set otherwise). */
static uint64_t type_size(uint32_t dtype, uint64_t ne, std::string & err) {
    uint64_t block, bytes;
    switch (dtype) {
        case 0: block = 1; bytes = 4; break;       /* F32 */
        case 1: block = 1; bytes = 2; break;       /* F16 */
        case 30: block = 1; bytes = 2; break;      /* BF16 */
        case 8: block = 32; bytes = 34; break;     /* Q8_0 */
        case 14: block = 256; bytes = 210; break;  /* Q6_K */
        default:
            err = "ggml type " + std::to_string(dtype) + " is not supported by this reader";
            return 0;
    }
    if (ne % block) {
        err = std::to_string(ne) + " elements is not a whole number of " + std::to_string(block) + "-element blocks";
        return 0;
    }
    return ne / block * bytes;
}

static Gguf * gguf_open(const char * path, std::string & err) {
    Gguf * g = new Gguf();
    auto fail = [&](const std::string & m) { err = std::string(path) + ": " + m; delete g; return (Gguf *) nullptr; };
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) return fail(strerror(errno));
    struct stat st;
    if (fstat(g->fd, &st) != 0) return fail(strerror(errno));
    g->len = (size_t) st.st_size;
    if (g->len < 24) return fail("not a GGUF file");
    void * m = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return fail(strerror(errno));
    g->map = (const uint8_t *) m;
    Cursor c{g->map, g->len};
    uint32_t magic;
    uint64_t nt, nkv;
    if (!c.get(magic) || magic != kGgufMagic) return fail("not a GGUF file");
    if (!c.get(g->version) || g->version < 2 || g->version > 3)
        return fail("GGUF version " + std::to_string(g->version) + " is not supported");
    if (!c.get(nt) || !c.get(nkv)) return fail("unexpected end of file");
    /* every entry takes at least 12 bytes: counts beyond the file are corruption */
    if (nt > g->len / 12 || nkv > g->len / 12) return fail("tensor or key count does not fit the file");
    for (uint64_t i = 0; i < nkv; i++) {
        std::string key, e;
        uint32_t type;
        KvValue v;
        if (!c.str(key) || !c.get(type)) return fail("unexpected end of file");
        if (!read_value(c, type, v, 0, e)) return fail(e);
        g->kv_index[key] = g->kv.size();
        g->kv.emplace_back(key, v);
    }
    for (uint64_t i = 0; i < nt; i++) {
        TensorInfo t;
        uint32_t nd;
        if (!c.str(t.name) || !c.get(nd)) return fail("unexpected end of file");
        if (nd < 1 || nd > 4) return fail("tensor " + t.name + " has " + std::to_string(nd) + " dimensions");
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t x;
            if (!c.get(x)) return fail("unexpected end of file");
            t.dims.push_back(x);
        }
        if (!c.get(t.dtype) || !c.get(t.offset)) return fail("unexpected end of file");
        g->tensor_index[t.name] = g->tensors.size();
        g->tensors.push_back(t);
    }
    auto a = g->kv_index.find("general.alignment");
    if (a != g->kv_index.end() && g->kv[a->second].second.has_u64) g->alignment = g->kv[a->second].second.u;
    const uint64_t al = g->alignment > 1 ? g->alignment : 1;
    g->data_start = ((uint64_t) c.p + al - 1) / al * al;
    if (g->data_start > g->len) return fail("tensor table runs past the file");
    return g;
}

static const KvValue * gguf_kv(const Gguf * g, const char * key) {
    if (!g || !key) return nullptr;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? nullptr : &g->kv[it->second].second;
}

/* ------------------------------------------------------- manifest directory */

struct ManifestEntry {
    std::string name;
    int rows = 0, cols = 0, stages = 0;
};

struct Manifest {
    std::string dir;
    std::vector<ManifestEntry> entries;
    std::map<std::string, size_t> index;
    std::vector<uint8_t> buf;   /* the last tensor read */
};

static bool read_file(const std::string & path, std::vector<uint8_t> & out, std::string & err) {
    FILE * f = fopen(path.c_str(), "rb");
    if (!f) { err = path + ": " + strerror(errno); return false; }
    out.clear();
    uint8_t chunk[1 << 16];
    size_t k;
    while ((k = fread(chunk, 1, sizeof chunk, f)) > 0) out.insert(out.end(), chunk, chunk + k);
    const bool bad = ferror(f) != 0;
    fclose(f);
    if (bad) { err = path + ": read error"; return false; }
    return true;
}

/* a whole non-negative decimal that fits an int */
static bool parse_int(const std::string & s, int & v) {
    if (s.empty() || s.size() > 10) return false;
    long long x = 0;
    for (char ch : s) {
        if (ch < '0' || ch > '9') return false;
        x = x * 10 + (ch - '0');
    }
    if (x > 0x7fffffff) return false;
    v = (int) x;
    return true;
}

static Manifest * manifest_open(const char * dir, std::string & err) {
    const std::string path = std::string(dir) + "/manifest.txt";
    std::vector<uint8_t> text;
    if (!read_file(path, text, err)) return nullptr;
    Manifest * m = new Manifest();
    m->dir = dir;
    size_t p = 0;
    while (p < text.size()) {
        size_t q = p;
        while (q < text.size() && text[q] != '\n') q++;
        std::string line((const char *) text.data() + p, q - p);
        p = q + 1;
        /* trim, skip blanks and comments, split on whitespace */
        const size_t a = line.find_first_not_of(" \t\r");
        if (a == std::string::npos) continue;
        line = line.substr(a, line.find_last_not_of(" \t\r") - a + 1);
        if (line[0] == '#') continue;
        std::vector<std::string> f;
        size_t i = 0;
        while (i < line.size()) {
            while (i < line.size() && (line[i] == ' ' || line[i] == '\t')) i++;
            size_t j = i;
            while (j < line.size() && line[j] != ' ' && line[j] != '\t') j++;
            if (j > i) f.push_back(line.substr(i, j - i));
            i = j;
        }
        if (f.size() < 5) { err = path + ": short manifest line: " + line; delete m; return nullptr; }
        ManifestEntry e;
        e.name = f[0];
        if (!parse_int(f[1], e.rows)) { err = "bad rows in: " + line; delete m; return nullptr; }
        if (!parse_int(f[2], e.cols)) { err = "bad cols in: " + line; delete m; return nullptr; }
        if (!parse_int(f[3], e.stages)) { err = "bad stages in: " + line; delete m; return nullptr; }
        auto it = m->index.find(e.name);
        if (it != m->index.end()) {
            m->entries[it->second] = e;   /* a later line for the same name replaces it */
        } else {
            m->index[e.name] = m->entries.size();
            m->entries.push_back(e);
        }
    }
    return m;
}

/* kind 0: RQVF sidecar, data = its rows x cols f32; kind 1: RQVQ container,
 * data = the whole file. */
static bool manifest_read(Manifest * m, const char * name, const void ** data, size_t * nbytes, int * kind,
                          std::string & err) {
    auto it = m->index.find(name);
    if (it == m->index.end()) { err = std::string(name) + " is not in the manifest"; return false; }
    const ManifestEntry & e = m->entries[it->second];
    if (!read_file(m->dir + "/" + e.name + ".bin", m->buf, err)) return false;
    const uint8_t * b = m->buf.data();
    const size_t len = m->buf.size();
    if (e.stages == 0) {
        if (len < 12 || memcmp(b, "RQVF", 4) != 0) { err = e.name + ": not an RQVF sidecar"; return false; }
        uint32_t rows, cols;
        memcpy(&rows, b + 4, 4);
        memcpy(&cols, b + 8, 4);
        if (rows == 0 || cols == 0) { err = e.name + ": RQVF header is inconsistent"; return false; }
        const uint64_t n = (uint64_t) rows * cols;
        if ((uint64_t) len != 12 + n * 4) {
            err = e.name + ": RQVF file is " + std::to_string(len) + " bytes, shape needs " + std::to_string(12 + n * 4);
            return false;
        }
        if ((int) rows != e.rows || (int) cols != e.cols) {
            err = e.name + ": sidecar is " + std::to_string(rows) + "x" + std::to_string(cols) + ", manifest says " +
                  std::to_string(e.rows) + "x" + std::to_string(e.cols);
            return false;
        }
        *data = b + 12;
        *nbytes = (size_t) n * 4;
        *kind = 0;
        return true;
    }
    fmt::ContainerView c;
    std::string e2;
    if (!fmt::open_container(b, len, c, e2)) { err = e.name + ": " + e2; return false; }
    if (c.rows != e.rows || c.cols != e.cols || (int) c.stages.size() != e.stages) {
        err = e.name + ": container is " + std::to_string(c.rows) + "x" + std::to_string(c.cols) + " with " +
              std::to_string(c.stages.size()) + " stages, manifest says " + std::to_string(e.rows) + "x" +
              std::to_string(e.cols) + " with " + std::to_string(e.stages);
        return false;
    }
    *data = b;
    *nbytes = len;
    *kind = 1;
    return true;
}

static int copy_name(const std::string & s, char * out, int cap) {
    if (!out || cap <= 0 || (int) s.size() >= cap) {
        set_error("name '%s' needs %zu bytes, the buffer holds %d", s.c_str(), s.size() + 1, cap);
        return -1;
    }
    memcpy(out, s.c_str(), s.size() + 1);
    return 0;
}

}  // namespace art
}  // namespace sparkmv

using namespace sparkmv;
using namespace sparkmv::art;

extern "C" {

void * sparkmv_gguf_open(const char * path) {
    if (!path) { set_error("null GGUF path"); return nullptr; }
    std::string err;
    Gguf * g = gguf_open(path, err);
    if (!g) set_error("%s", err.c_str());
    return g;
}

void sparkmv_gguf_close(void * g) { delete (Gguf *) g; }

int sparkmv_gguf_version(const void * g) { return g ? (int) ((const Gguf *) g)->version : -1; }

int64_t sparkmv_gguf_tensor_count(const void * g) { return g ? (int64_t) ((const Gguf *) g)->tensors.size() : -1; }

int64_t sparkmv_gguf_find(const void * g, const char * name) {
    if (!g || !name) return -1;
    const Gguf * gg = (const Gguf *) g;
    auto it = gg->tensor_index.find(name);
    return it == gg->tensor_index.end() ? -1 : (int64_t) it->second;
}

int sparkmv_gguf_tensor_info(const void * g, int64_t i, sparkmv_gguf_tensor * out) {
    const Gguf * gg = (const Gguf *) g;
    if (!gg || !out || i < 0 || i >= (int64_t) gg->tensors.size()) { set_error("no GGUF tensor %lld", (long long) i); return -1; }
    const TensorInfo & t = gg->tensors[(size_t) i];
    memset(out, 0, sizeof *out);
    if (copy_name(t.name, out->name, (int) sizeof out->name)) return -1;
    out->ndims = (int) t.dims.size();
    uint64_t ne = 1;
    for (size_t d = 0; d < t.dims.size(); d++) { out->dims[d] = t.dims[d]; ne *= t.dims[d]; }
    out->dtype = t.dtype;
    out->offset = t.offset;
    std::string err;
    out->nbytes = type_size(t.dtype, ne, err);   /* 0 for a type this reader does not hand out */
    return 0;
}

const void * sparkmv_gguf_tensor_data(const void * g, int64_t i, uint64_t * nbytes) {
    const Gguf * gg = (const Gguf *) g;
    if (!gg || i < 0 || i >= (int64_t) gg->tensors.size()) { set_error("no GGUF tensor %lld", (long long) i); return nullptr; }
    const TensorInfo & t = gg->tensors[(size_t) i];
    uint64_t ne = 1;
    for (uint64_t d : t.dims) {
        if (d && ne > UINT64_MAX / d) { set_error("tensor %s: element count overflows", t.name.c_str()); return nullptr; }
        ne *= d;
    }
    std::string err;
    const uint64_t n = type_size(t.dtype, ne, err);
    if (!n && ne) { set_error("tensor %s: %s", t.name.c_str(), err.c_str()); return nullptr; }
    const uint64_t start = gg->data_start + t.offset;
    if (start < gg->data_start || n > (uint64_t) gg->len || start > (uint64_t) gg->len - n) {
        set_error("tensor %s needs bytes %llu..%llu, the file is %zu", t.name.c_str(), (unsigned long long) start,
                  (unsigned long long) (start + n), gg->len);
        return nullptr;
    }
    if (nbytes) *nbytes = n;
    return gg->map + start;
}

int64_t sparkmv_gguf_kv_count(const void * g) { return g ? (int64_t) ((const Gguf *) g)->kv.size() : -1; }

int sparkmv_gguf_kv_key(const void * g, int64_t i, char * key, int cap, uint32_t * type) {
    const Gguf * gg = (const Gguf *) g;
    if (!gg || i < 0 || i >= (int64_t) gg->kv.size()) { set_error("no GGUF key %lld", (long long) i); return -1; }
    if (type) *type = gg->kv[(size_t) i].second.type;
    return copy_name(gg->kv[(size_t) i].first, key, cap);
}

int sparkmv_gguf_get_u64(const void * g, const char * key, uint64_t * out) {
    const KvValue * v = gguf_kv((const Gguf *) g, key);
    if (!v || !v->has_u64 || !out) { set_error("GGUF key %s is absent or not a non-negative integer", key ? key : "(null)"); return -1; }
    *out = v->u;
    return 0;
}

int sparkmv_gguf_get_f64(const void * g, const char * key, double * out) {
    const KvValue * v = gguf_kv((const Gguf *) g, key);
    if (!v || !v->has_f64 || !out) { set_error("GGUF key %s is absent or not a number", key ? key : "(null)"); return -1; }
    *out = v->f;
    return 0;
}

int sparkmv_gguf_get_str(const void * g, const char * key, char * out, int cap) {
    const KvValue * v = gguf_kv((const Gguf *) g, key);
    if (!v || v->type != kString) { set_error("GGUF key %s is absent or not a string", key ? key : "(null)"); return -1; }
    return copy_name(v->s, out, cap);
}

int64_t sparkmv_gguf_get_arr_len(const void * g, const char * key, uint32_t * elem) {
    const KvValue * v = gguf_kv((const Gguf *) g, key);
    if (!v || v->type != kArray) { set_error("GGUF key %s is absent or not an array", key ? key : "(null)"); return -1; }
    if (elem) *elem = v->elem;
    return (int64_t) v->count;
}

void * sparkmv_manifest_open(const char * dir) {
    if (!dir) { set_error("null manifest directory"); return nullptr; }
    std::string err;
    Manifest * m = manifest_open(dir, err);
    if (!m) set_error("%s", err.c_str());
    return m;
}

void sparkmv_manifest_close(void * m) { delete (Manifest *) m; }

int sparkmv_manifest_count(const void * m) { return m ? (int) ((const Manifest *) m)->entries.size() : -1; }

int sparkmv_manifest_entry(const void * m, int i, char * name, int cap, int * rows, int * cols, int * stages) {
    const Manifest * mm = (const Manifest *) m;
    if (!mm || i < 0 || i >= (int) mm->entries.size()) { set_error("no manifest entry %d", i); return -1; }
    const ManifestEntry & e = mm->entries[(size_t) i];
    if (rows) *rows = e.rows;
    if (cols) *cols = e.cols;
    if (stages) *stages = e.stages;
    return copy_name(e.name, name, cap);
}

int sparkmv_manifest_read(void * m, const char * name, const void ** data, size_t * nbytes, int * kind) {
    if (!m || !name || !data || !nbytes || !kind) { set_error("manifest read needs a handle, a name and outputs"); return -1; }
    std::string err;
    if (!manifest_read((Manifest *) m, name, data, nbytes, kind, err)) {
        set_error("%s", err.c_str());
        return -1;
    }
    return 0;
}

}  // extern "C"
