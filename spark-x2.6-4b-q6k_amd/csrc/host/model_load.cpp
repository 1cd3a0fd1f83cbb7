/* model_load.cpp — a whole model from a checkpoint's config.json and a VQ
 * artifact directory.
 *
 * 1. config.json (tools/vq-runtime/src/config.rs:39-85, Config::load): the
 *    numeric sizes, rms_norm_eps, sliding_window, the per-layer
 *    layer_types ("full_attention" is full; any other entry, and any layer
 *    past the list, follows config.rs:72-77), and rope_parameters per layer
 *    type with the checkpoint's values as fallbacks (5e6 / 0.25 full,
 *    1e4 / 1.0 sliding). The JSON is parsed whole by a small recursive-
 *    descent reader, so keys are looked up in their own object.
 * 2. The weights (tools/vq-runtime/src/model.rs:121-185, Weights::load; the
 *    GPU runtime's load_model / load_mat / load_vec, tools/vq/gpu/
 *    vq-model-gpu.cu:230-357, :739-775): the tied embedding, the final norm,
 *    and per layer the two norms and the six matrices, each checked against
 *    the architecture's shape with the reference's messages. Every RQVQ
 *    container goes to the device as one buffer (the header, then its stages
 *    at their file offsets, and 64 zero bytes past the end for the kernels'
 *    aligned index windows); the norms as f32 vectors. The model owns them.
 *    Every matrix must share the first one's VQ geometry (dim, codebook,
 *    stages, payload format), which is what one sparkmv model runs.
 * 3. A tuning profile at DIR/vq-tune.profile is applied when it is trusted
 *    for this artifact and device (vq-model-gpu.cu:1100-1120 loads it from
 *    the same place), with the checks of sparkmv_model_apply_profile.
 */
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <new>
#include <string>
#include <utility>
#include <vector>

#include "../../../include/sparkmv.h"
#include "../common.h"
#include "../model.h"

namespace sparkmv {
namespace load {

/* ---------------------------------------------------------------- JSON -- */

struct Json {
    enum Type { Null, Bool, Num, Str, Arr, Obj } type = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    /* a repeated key: the last one counts, as serde_json's map keeps it */
    const Json * get(const char * key) const {
        if (type != Obj) return nullptr;
        for (size_t i = obj.size(); i-- > 0;)
            if (obj[i].first == key) return &obj[i].second;
        return nullptr;
    }
};

struct Parser {
    const char * p;
    const char * end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail(const char * what) {
        if (err.empty()) err = what;
        return false;
    }
    bool lit(const char * s) {
        const size_t n = strlen(s);
        if ((size_t) (end - p) < n || strncmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    bool hex4(unsigned & v) {
        if (end - p < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned) (c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned) (c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned) (c - 'A' + 10);
            else return false;
        }
        return true;
    }
    void utf8(std::string & out, unsigned cp) {
        if (cp < 0x80) {
            out += (char) cp;
        } else if (cp < 0x800) {
            out += (char) (0xc0 | (cp >> 6));
            out += (char) (0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += (char) (0xe0 | (cp >> 12));
            out += (char) (0x80 | ((cp >> 6) & 0x3f));
            out += (char) (0x80 | (cp & 0x3f));
        } else {
            out += (char) (0xf0 | (cp >> 18));
            out += (char) (0x80 | ((cp >> 12) & 0x3f));
            out += (char) (0x80 | ((cp >> 6) & 0x3f));
            out += (char) (0x80 | (cp & 0x3f));
        }
    }
    bool string(std::string & out) {
        if (p >= end || *p != '"') return fail("expected a string");
        p++;
        out.clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if ((unsigned char) c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p >= end) return fail("unterminated escape");
            c = *p++;
            switch (c) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    unsigned cp = 0;
                    if (!hex4(cp)) return fail("bad \\u escape");
                    if (cp >= 0xd800 && cp < 0xdc00) {
                        unsigned lo = 0;
                        if (!lit("\\u") || !hex4(lo) || lo < 0xdc00 || lo >= 0xe000) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool number(double & v) {
        const char * s = p;
        if (p < end && *p == '-') p++;
        if (p >= end || !(*p >= '0' && *p <= '9')) return fail("bad number");
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-'))
            p++;
        const std::string t(s, (size_t) (p - s));
        char * e = nullptr;
        v = strtod(t.c_str(), &e);
        if (!e || *e) return fail("bad number");
        return true;
    }
    bool value(Json & v, int depth) {
        if (depth > 64) return fail("JSON nested too deeply");
        ws();
        if (p >= end) return fail("unexpected end of JSON");
        if (*p == '{') {
            p++;
            v.type = Json::Obj;
            ws();
            if (p < end && *p == '}') { p++; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                p++;
                Json child;
                if (!value(child, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(child));
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == '}') { p++; return true; }
                return fail("expected ',' or '}'");
            }
        }
        if (*p == '[') {
            p++;
            v.type = Json::Arr;
            ws();
            if (p < end && *p == ']') { p++; return true; }
            for (;;) {
                Json child;
                if (!value(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == ']') { p++; return true; }
                return fail("expected ',' or ']'");
            }
        }
        if (*p == '"') {
            v.type = Json::Str;
            return string(v.str);
        }
        if (lit("true")) { v.type = Json::Bool; v.b = true; return true; }
        if (lit("false")) { v.type = Json::Bool; v.b = false; return true; }
        if (lit("null")) { v.type = Json::Null; return true; }
        v.type = Json::Num;
        return number(v.num);
    }
};

static bool read_text(const char * path, std::string & out, std::string & err) {
    FILE * f = fopen(path, "rb");
    if (!f) { err = std::string(path) + ": " + strerror(errno); return false; }
    out.clear();
    char chunk[1 << 16];
    size_t k;
    while ((k = fread(chunk, 1, sizeof chunk, f)) > 0) out.append(chunk, k);
    const bool bad = ferror(f) != 0;
    fclose(f);
    if (bad) { err = std::string(path) + ": read error"; return false; }
    return true;
}

constexpr int kMaxConfigLayers = 65536;

/* config.rs:39-85 */
static bool config_load(const char * path, sparkmv_model_cfg & cfg, std::vector<int> & full, std::string & err) {
    std::string text;
    if (!read_text(path, text, err)) return false;
    Parser ps{text.data(), text.data() + text.size(), std::string()};
    Json root;
    if (!ps.value(root, 0)) { err = std::string(path) + ": " + ps.err; return false; }
    ps.ws();
    if (ps.p != ps.end) { err = std::string(path) + ": trailing characters after the JSON value"; return false; }
    if (root.type != Json::Obj) { err = std::string(path) + ": not a JSON object"; return false; }
    auto num = [&](const char * k, double & v) {
        const Json * j = root.get(k);
        if (!j || j->type != Json::Num) { err = std::string("config.json has no numeric ") + k; return false; }
        v = j->num;
        return true;
    };
    double hidden, layers, heads, kvh, hd, inter, vocab, eps, window;
    if (!num("hidden_size", hidden) || !num("num_hidden_layers", layers) || !num("num_attention_heads", heads) ||
        !num("num_key_value_heads", kvh) || !num("head_dim", hd) || !num("intermediate_size", inter) ||
        !num("vocab_size", vocab) || !num("rms_norm_eps", eps) || !num("sliding_window", window))
        return false;
    const Json * lt = root.get("layer_types");
    if (!lt || lt->type != Json::Arr) { err = "config.json has no layer_types"; return false; }
    for (double v : {hidden, layers, heads, kvh, hd, inter, vocab, window})
        if (!(v >= 1.0 && v <= 2147483647.0)) { err = "config.json has a size outside 1..2^31-1"; return false; }
    /* the per-layer flags are held in memory: a layer count past any model
     * is refused here rather than allocated */
    if (layers >= (double) (kMaxConfigLayers + 1)) {
        char b[96];
        snprintf(b, sizeof b, "config.json has %.0f layers, above %d", layers, kMaxConfigLayers);
        err = b;
        return false;
    }
    memset(&cfg, 0, sizeof cfg);
    cfg.hidden = (int) hidden;
    cfg.layers = (int) layers;
    cfg.heads = (int) heads;
    cfg.kv_heads = (int) kvh;
    cfg.head_dim = (int) hd;
    cfg.intermediate = (int) inter;
    cfg.vocab = (int) vocab;
    cfg.eps = (float) eps;
    cfg.sliding_window = (int) window;
    /* a layer is full when its entry is "full_attention"; an entry that is
     * not a string counts as "full_attention", and so does a layer past the
     * list (config.rs:45-50, :72-77) */
    full.assign((size_t) cfg.layers, 1);
    for (size_t i = 0; i < lt->arr.size() && i < full.size(); i++) {
        const Json & t = lt->arr[i];
        full[i] = t.type != Json::Str || t.str == "full_attention";
    }
    /* rope_parameters per layer type, each value falling back to this
     * checkpoint's (config.rs:54-69, :79-80) */
    const Json * rp = root.get("rope_parameters");
    auto rope = [&](const char * name, double theta, double partial, double & t_out, double & p_out) {
        const Json * o = rp ? rp->get(name) : nullptr;
        const Json * t = o ? o->get("rope_theta") : nullptr;
        const Json * f = o ? o->get("partial_rotary_factor") : nullptr;
        /* the runtime keeps them in f32 (config.rs:60-67) */
        t_out = (double) (float) (t && t->type == Json::Num ? t->num : theta);
        p_out = (double) (float) (f && f->type == Json::Num ? f->num : partial);
    };
    rope("full_attention", 5000000.0, 0.25, cfg.rope_full_theta, cfg.rope_full_partial);
    rope("sliding_attention", 10000.0, 1.0, cfg.rope_slide_theta, cfg.rope_slide_partial);
    return true;
}

/* ------------------------------------------------------------- weights -- */

struct Loader {
    void * manifest = nullptr;
    void * model = nullptr;
    sparkmv_container_info geom{};   /* the first matrix's geometry */
    bool have_geom = false;
    std::vector<void *> pending;      /* device buffers not yet handed to the model */

    ~Loader() {
        for (void * p : pending) (void) hipFree(p);
        if (manifest) sparkmv_manifest_close(manifest);
    }
};

static bool upload(Loader & L, const void * host, size_t n, size_t pad, void ** out, std::string & err) {
    void * d = nullptr;
    hipError_t e = hipMalloc(&d, n + pad);
    if (e != hipSuccess) { err = std::string("device allocation: ") + hipGetErrorString(e); return false; }
    L.pending.push_back(d);
    e = hipMemcpy(d, host, n, hipMemcpyHostToDevice);
    if (e == hipSuccess && pad) e = hipMemset((uint8_t *) d + n, 0, pad);
    if (e != hipSuccess) { err = std::string("weight upload: ") + hipGetErrorString(e); return false; }
    *out = d;
    return true;
}

/* model.rs:100-108 expect() plus the upload: stage pointers into st */
static bool load_mat(Loader & L, const std::string & name, int rows, int cols, const void ** st, std::string & err) {
    const void * data = nullptr;
    size_t n = 0;
    int kind = -1;
    if (sparkmv_manifest_read(L.manifest, name.c_str(), &data, &n, &kind)) { err = vqg_decode_error(); return false; }
    if (kind != 1) { err = name + ": is a vector, the architecture needs a matrix"; return false; }
    sparkmv_container_info ci;
    if (sparkmv_container_open(data, n, &ci)) { err = name + ": " + vqg_decode_error(); return false; }
    if (ci.rows != rows || ci.cols != cols) {
        char b[256];
        snprintf(b, sizeof b, ": is %dx%d, the architecture needs %dx%d", ci.rows, ci.cols, rows, cols);
        err = name + b;
        return false;
    }
    if (!L.have_geom) {
        L.geom = ci;
        L.have_geom = true;
    } else if (ci.dim != L.geom.dim || ci.nc != L.geom.nc || ci.nstages != L.geom.nstages || ci.v3 != L.geom.v3) {
        char b[256];
        snprintf(b, sizeof b, ": dim %d, nc %d, %d stages, %s, where the first matrix has dim %d, nc %d, %d stages, %s",
                 ci.dim, ci.nc, ci.nstages, ci.v3 ? "DQV3" : "DQVQ", L.geom.dim, L.geom.nc, L.geom.nstages,
                 L.geom.v3 ? "DQV3" : "DQVQ");
        err = name + b + " (one model runs one VQ geometry)";
        return false;
    }
    void * d = nullptr;
    if (!upload(L, data, n, 64, &d, err)) return false;
    for (int s = 0; s < 4; s++) st[s] = s < ci.nstages ? (const uint8_t *) d + ci.stage_offset[s] : nullptr;
    return true;
}

/* 1 and the vector's device pointer in *out; -1 with *got set when the
 * sidecar holds another count than want; 0 with err set otherwise */
static int load_vec(Loader & L, const std::string & name, int want, const float ** out, size_t * got,
                    std::string & err) {
    const void * data = nullptr;
    size_t n = 0;
    int kind = -1;
    if (sparkmv_manifest_read(L.manifest, name.c_str(), &data, &n, &kind)) { err = vqg_decode_error(); return 0; }
    if (kind != 0) { err = name + ": is a matrix, the architecture needs a vector"; return 0; }
    if (n != (size_t) want * 4) {
        *got = n / 4;
        return -1;
    }
    void * d = nullptr;
    if (!upload(L, data, n, 0, &d, err)) return 0;
    *out = (const float *) d;
    return 1;
}

static void * model_load(const char * dir, const char * config_path, int max_ctx, int x_dtype, int apply_profile,
                         std::string & err) {
    sparkmv_model_cfg cfg;
    std::vector<int> full;
    if (!config_load(config_path, cfg, full, err)) return nullptr;
    Loader L;
    L.manifest = sparkmv_manifest_open(dir);
    if (!L.manifest) { err = vqg_decode_error(); return nullptr; }
    const long long qd64 = (long long) cfg.heads * cfg.head_dim, kvd64 = (long long) cfg.kv_heads * cfg.head_dim;
    if (qd64 + 2 * kvd64 > 2147483647LL) { err = "config.json: the attention widths overflow 32 bits"; return nullptr; }
    const int hid = cfg.hidden, qd = (int) qd64, kvd = (int) kvd64;

    /* the tied embedding decides the geometry; the model is created from it */
    const void * head[4] = {};
    if (!load_mat(L, "model.embedding.weight", cfg.vocab, hid, head, err)) return nullptr;
    const float * final_norm = nullptr;
    char b[256];
    size_t got = 0;
    int rc = load_vec(L, "model.norm.weight", hid, &final_norm, &got, err);
    if (rc < 0) {
        snprintf(b, sizeof b, "model.norm.weight: %zu values", got);   /* model.rs:126-128 */
        err = b;
    }
    if (rc != 1) return nullptr;
    cfg.max_ctx = max_ctx;
    cfg.x_dtype = x_dtype;
    cfg.dim = L.geom.dim;
    cfg.nc = L.geom.nc;
    cfg.nstages = L.geom.nstages;
    cfg.v3 = L.geom.v3;
    L.model = sparkmv_model_create(&cfg);
    if (!L.model) { err = vqg_decode_error(); return nullptr; }
    struct Drop {
        void *& m;
        ~Drop() { if (m) sparkmv_model_destroy(m); }
    } drop{L.model};
    if (sparkmv_model_set_head(L.model, 0, head, nullptr, final_norm)) { err = vqg_decode_error(); return nullptr; }

    for (int i = 0; i < cfg.layers; i++) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        sparkmv_model_layer w;
        memset(&w, 0, sizeof w);
        for (int k = 0; k < 2; k++) {
            rc = load_vec(L, p + (k ? "post_attention_layernorm.weight" : "input_layernorm.weight"), hid,
                          k ? &w.post_norm : &w.in_norm, &got, err);
            if (rc < 0) {
                snprintf(b, sizeof b, "layer %d: a norm is not %d wide", i, hid);   /* model.rs:133-135 */
                err = b;
            }
            if (rc != 1) return nullptr;
        }
        if (!load_mat(L, p + "self_attn.q_k_v_proj.weight", qd + 2 * kvd, hid, w.qkv, err)) return nullptr;
        if (!load_mat(L, p + "self_attn.g_proj.weight", cfg.heads, hid, w.attn_gate, err)) return nullptr;
        if (!load_mat(L, p + "self_attn.out_proj.weight", hid, qd, w.out, err)) return nullptr;
        if (!load_mat(L, p + "mlp.gate_proj.weight", cfg.intermediate, hid, w.gate, err)) return nullptr;
        if (!load_mat(L, p + "mlp.up_proj.weight", cfg.intermediate, hid, w.up, err)) return nullptr;
        if (!load_mat(L, p + "mlp.down_proj.weight", hid, cfg.intermediate, w.down, err)) return nullptr;
        w.full = full[(size_t) i];
        if (sparkmv_model_set_layer(L.model, i, &w)) { err = vqg_decode_error(); return nullptr; }
    }
    /* the model frees the weights from here on: each buffer leaves the
     * loader's list as soon as the model holds it, so a failure (or an
     * allocation failure thrown by the handoff) part way frees each buffer
     * exactly once, by whichever side holds it */
    while (!L.pending.empty()) {
        if (model_adopt(L.model, L.pending.back())) { err = vqg_decode_error(); return nullptr; }
        L.pending.pop_back();
    }

    /* The profile never fails a load (vq-model-gpu.cu:1097-1120): one that
     * is absent, not version 1, for another artifact or device, or that
     * cannot be checked leaves the heuristic, and the outcome is left in
     * the message channel. */
    std::string note = "profile: not requested; heuristics";
    if (apply_profile) {
        const std::string prof_path = std::string(dir) + "/vq-tune.profile";
        uint64_t fp = 0;
        char gpu[256] = {};
        void * prof = nullptr;
        if (sparkmv_profile_fingerprint(dir, &fp)) {
            note = std::string("profile: none; ") + dir + "/manifest.txt could not be fingerprinted";
        } else if (!(prof = sparkmv_profile_load(prof_path.c_str()))) {
            note = "profile: " + prof_path + " is absent or not version 1; heuristics";
        } else if (vqg_device_name(gpu, (int) sizeof gpu)) {
            note = "profile: device query failed; heuristics";
        } else {
            const int n = sparkmv_model_apply_profile(L.model, prof, fp, gpu);
            note = n < 0 ? std::string("profile: ") + vqg_decode_error() + "; heuristics" : vqg_decode_error();
        }
        if (prof) sparkmv_profile_close(prof);
    }
    set_error("%s", note.c_str());
    void * m = L.model;
    L.model = nullptr;
    return m;
}

}  // namespace load
}  // namespace sparkmv

using namespace sparkmv;

extern "C" {

int sparkmv_config_load(const char * path, sparkmv_model_cfg * cfg, int * full, int max_layers) {
    if (!path || !cfg) { set_error("config path or output is null"); return -1; }
    try {
        std::string err;
        std::vector<int> f;
        if (!load::config_load(path, *cfg, f, err)) { set_error("%s", err.c_str()); return -1; }
        if (full)
            for (int i = 0; i < max_layers && i < (int) f.size(); i++) full[i] = f[(size_t) i];
        return 0;
    } catch (const std::bad_alloc &) {
        set_error("out of host memory reading %s", path);
        return -1;
    }
}

void * sparkmv_model_load(const char * dir, const char * config_path, int max_ctx, int x_dtype, int apply_profile) {
    if (!dir || !config_path) { set_error("artifact directory or config path is null"); return nullptr; }
    try {
        std::string err;
        void * m = load::model_load(dir, config_path, max_ctx, x_dtype, apply_profile, err);
        if (!m) set_error("%s", err.c_str());
        return m;
    } catch (const std::bad_alloc &) {
        set_error("out of host memory loading %s", dir);
        return nullptr;
    }
}

}  // extern "C"
