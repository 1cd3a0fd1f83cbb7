/* profile.cpp — the per-artifact tuning profile (VQPROF 1): read, write and
 * trust-check the file that records which kernel, at which launch width,
 * serves each matrix geometry on one device.
 *
 * Format and fingerprint are the reference's (tools/vq/gpu/vq-profile.h:
 * 10-30, written by tools/vq-tune/src/artifact.rs:148-171):
 *
 *   VQPROF 1
 *   artifact <16 lowercase hex digits>
 *   gpu <device name, to end of line>
 *   driver <driver text, to end of line>
 *   gemv <dim> <nc> <rows> <cols> <v3> <variant> <threads> <gbs>
 *   prefill <dim> <nc> <rows> <cols> <v3> <variant> <bn> <bk> <tps>
 *
 * The fingerprint is FNV-1a 64 over manifest.txt as stored, then for every
 * matrix line (stages > 0) in file order: the name, the container's size as 8
 * little-endian bytes, its first min(4096, size) bytes and its last
 * min(4096, size) bytes. A profile is trusted only when its version, device
 * name and fingerprint all match (vq-profile.h:1-8, 24-30). Lines that are
 * not directives are skipped, as the reference's reader skips them.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../../include/sparkmv.h"
#include "../common.h"

namespace sparkmv {
namespace prof {

/* The reference's offset basis (tools/vq-tune/src/artifact.rs:14,
 * tools/vq/gpu/vq-profile.h:67): one digit short of FNV-1a's published
 * 14695981039346656037, kept because a profile must hash what its tuner
 * hashed. */
constexpr uint64_t kFnvBasis = 1469598103934665603ull;
constexpr uint64_t kFnvPrime = 1099511628211ull;

static uint64_t fnv(uint64_t h, const void * p, size_t n) {
    const unsigned char * b = (const unsigned char *) p;
    for (size_t i = 0; i < n; i++) {
        h ^= (uint64_t) b[i];
        h *= kFnvPrime;
    }
    return h;
}

static bool slurp(const std::string & path, std::string & out) {
    FILE * f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[1 << 16];
    size_t n;
    out.clear();
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    const bool ok = !ferror(f);
    fclose(f);
    return ok;
}

/* name, size, first and last min(4096, size) bytes of <dir>/<name>.bin */
static bool hash_file(uint64_t & h, const std::string & dir, const std::string & name, std::string & err) {
    const std::string path = dir + "/" + name + ".bin";
    FILE * f = fopen(path.c_str(), "rb");
    if (!f) { err = path + " cannot be opened"; return false; }
    if (fseek(f, 0, SEEK_END)) { fclose(f); err = path + " cannot be sized"; return false; }
    const long sz = ftell(f);
    if (sz < 0 || fseek(f, 0, SEEK_SET)) { fclose(f); err = path + " cannot be sized"; return false; }
    const uint64_t size = (uint64_t) sz;
    h = fnv(h, name.data(), name.size());
    unsigned char le[8];
    for (int i = 0; i < 8; i++) le[i] = (unsigned char) (size >> (8 * i));
    h = fnv(h, le, 8);
    const size_t edge = size < 4096 ? (size_t) size : 4096;
    std::vector<unsigned char> buf(edge ? edge : 1);
    bool ok = true;
    if (edge) {
        ok = fread(buf.data(), 1, edge, f) == edge;
        if (ok) h = fnv(h, buf.data(), edge);
        if (ok && size > 4096) ok = fseek(f, (long) (size - 4096), SEEK_SET) == 0 && fread(buf.data(), 1, 4096, f) == 4096;
        if (ok) h = fnv(h, buf.data(), edge);
    }
    fclose(f);
    if (!ok) err = path + " is shorter than it reported";
    return ok;
}

struct Profile {
    int version = 0;
    uint64_t artifact = 0;
    std::string gpu, driver;
    std::vector<sparkmv_profile_entry> e;
};

static std::string trim(std::string s) {
    while (!s.empty() && (s.back() == '\n' || s.back() == '\r' || s.back() == ' ')) s.pop_back();
    return s;
}

}  // namespace prof
}  // namespace sparkmv

using namespace sparkmv;
using namespace sparkmv::prof;

extern "C" {

int sparkmv_profile_fingerprint(const char * dir, uint64_t * out) {
    if (!dir || !out) { set_error("profile fingerprint: null argument"); return -1; }
    std::string man;
    if (!slurp(std::string(dir) + "/manifest.txt", man)) {
        set_error("%s/manifest.txt cannot be read", dir);
        return -1;
    }
    uint64_t h = fnv(kFnvBasis, man.data(), man.size());
    size_t p = 0;
    while (p < man.size()) {
        size_t nl = man.find('\n', p);
        const std::string line = man.substr(p, nl == std::string::npos ? std::string::npos : nl - p);
        if (!line.empty() && line[0] != '#') {
            char name[1024];
            unsigned long long rows, cols, stages, bytes;
            double rel;
            if (sscanf(line.c_str(), "%1023s %llu %llu %llu %llu %lf", name, &rows, &cols, &stages, &bytes, &rel) == 6 &&
                stages > 0) {
                std::string err;
                if (!hash_file(h, dir, name, err)) { set_error("%s", err.c_str()); return -1; }
            }
        }
        if (nl == std::string::npos) break;
        p = nl + 1;
    }
    *out = h;
    return 0;
}

void * sparkmv_profile_load(const char * path) {
    if (!path) { set_error("profile path is null"); return nullptr; }
    std::string text;
    if (!slurp(path, text)) { set_error("%s cannot be read", path); return nullptr; }
    Profile * pf = new Profile;
    size_t p = 0;
    while (p < text.size()) {
        size_t nl = text.find('\n', p);
        std::string line = trim(text.substr(p, nl == std::string::npos ? std::string::npos : nl - p));
        p = nl == std::string::npos ? text.size() : nl + 1;
        if (!line.compare(0, 7, "VQPROF ")) { pf->version = atoi(line.c_str() + 7); continue; }
        if (!line.compare(0, 9, "artifact ")) {
            unsigned long long v = 0;
            if (sscanf(line.c_str() + 9, "%llx", &v) == 1) pf->artifact = v;
            continue;
        }
        if (!line.compare(0, 4, "gpu ")) { pf->gpu = line.substr(4); continue; }
        if (!line.compare(0, 7, "driver ")) { pf->driver = line.substr(7); continue; }
        sparkmv_profile_entry e;
        memset(&e, 0, sizeof e);
        if (sscanf(line.c_str(), "gemv %d %d %d %d %d %d %d %lf", &e.dim, &e.nc, &e.rows, &e.cols, &e.v3, &e.variant,
                   &e.threads, &e.rate) >= 7) {
            e.kind = 0;
        } else if (sscanf(line.c_str(), "prefill %d %d %d %d %d %d %d %d %lf", &e.dim, &e.nc, &e.rows, &e.cols, &e.v3,
                          &e.variant, &e.bn, &e.bk, &e.rate) >= 8) {
            e.kind = 1;
        } else {
            continue;
        }
        if (pf->e.size() < 512) pf->e.push_back(e);
    }
    if (pf->version != 1) {
        set_error("%s carries profile version %d, this reader takes 1", path, pf->version);
        delete pf;
        return nullptr;
    }
    return pf;
}

void sparkmv_profile_close(void * profile) { delete (Profile *) profile; }

int sparkmv_profile_trusted(const void * profile, uint64_t artifact, const char * gpu) {
    const Profile * pf = (const Profile *) profile;
    if (!pf || !gpu) { set_error("profile or device name is null"); return -1; }
    if (pf->artifact != artifact) {
        set_error("profile fingerprint %016llx does not match the artifact's %016llx",
                  (unsigned long long) pf->artifact, (unsigned long long) artifact);
        return 0;
    }
    if (pf->gpu != gpu) {
        set_error("profile was measured on '%s', not '%s'", pf->gpu.c_str(), gpu);
        return 0;
    }
    return 1;
}

int sparkmv_profile_count(const void * profile) {
    const Profile * pf = (const Profile *) profile;
    return pf ? (int) pf->e.size() : -1;
}

int sparkmv_profile_entry_at(const void * profile, int i, sparkmv_profile_entry * out) {
    const Profile * pf = (const Profile *) profile;
    if (!pf || !out || i < 0 || i >= (int) pf->e.size()) { set_error("no profile entry %d", i); return -1; }
    *out = pf->e[i];
    return 0;
}

int sparkmv_profile_find(const void * profile, int kind, int dim, int nc, int rows, int cols, int v3,
                         sparkmv_profile_entry * out) {
    const Profile * pf = (const Profile *) profile;
    if (!pf || !out) { set_error("profile or output is null"); return -1; }
    for (const sparkmv_profile_entry & e : pf->e)
        if (e.kind == kind && e.dim == dim && e.nc == nc && e.rows == rows && e.cols == cols && e.v3 == v3) {
            *out = e;
            return 0;
        }
    set_error("no profile entry for %s %dx%d (dim %d, nc %d, v3 %d)", kind ? "prefill" : "gemv", rows, cols, dim, nc, v3);
    return -1;
}

int sparkmv_profile_write(const char * path, uint64_t artifact, const char * gpu, const char * driver,
                          const sparkmv_profile_entry * entries, int n) {
    if (!path || !gpu || !driver || (n > 0 && !entries) || n < 0 || n > 512) {
        set_error("profile write: bad arguments");
        return -1;
    }
    FILE * f = fopen(path, "w");
    if (!f) { set_error("%s cannot be written", path); return -1; }
    fprintf(f, "VQPROF 1\nartifact %016llx\ngpu %s\ndriver %s\n", (unsigned long long) artifact, gpu, driver);
    for (int i = 0; i < n; i++) {
        const sparkmv_profile_entry & e = entries[i];
        if (e.kind == 0)
            fprintf(f, "gemv %d %d %d %d %d %d %d %.2f\n", e.dim, e.nc, e.rows, e.cols, e.v3, e.variant, e.threads, e.rate);
        else
            fprintf(f, "prefill %d %d %d %d %d %d %d %d %.2f\n", e.dim, e.nc, e.rows, e.cols, e.v3, e.variant, e.bn,
                    e.bk, e.rate);
    }
    const bool ok = fclose(f) == 0;
    if (!ok) { set_error("%s could not be completed", path); return -1; }
    return 0;
}

}  // extern "C"
