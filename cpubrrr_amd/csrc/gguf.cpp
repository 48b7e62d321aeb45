// gguf.cpp -- GGUF v3 reader (mmap) and the MoE layer loader on top of it.
//
// Format (GGUF v3, little endian), as the reference's parser reads it
// (scripts/gguf_index.py:21-45):
//   "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x  { string key | u32 value type | value }
//   n_tensors x { string name | u32 n_dims | u64 dims[n_dims] | u32 type | u64 offset }
//   padding to general.alignment (default 32) -> data start; tensor data at
//   data start + offset.
// string = u64 length + bytes; value types 0..12 (u8, i8, u16, i16, u32, i32,
// f32, bool, string, array = {u32 type, u64 n, values}, u64, i64, f64).
// Every read is bounds-checked against the file size.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "cpb_gguf.h"
#include "cpb_internal.h"

namespace {

using cpb::fail;

enum ValType { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64 };

struct Meta {
    int type = -1;           // scalar kinds and kStr; arrays are skipped but typed kArr
    int64_t i = 0;
    double f = 0.0;
    std::string s;
};

// bytes per block and elements per block of the tensor types the reference
// uses (ggml's type traits for these ids)
bool type_size(int t, uint64_t* bytes, uint64_t* elems) {
    switch (t) {
        case CPB_GGML_F32: *bytes = 4; *elems = 1; return true;
        case CPB_GGML_F16: *bytes = 2; *elems = 1; return true;
        case CPB_GGML_BF16: *bytes = 2; *elems = 1; return true;
        case CPB_GGML_Q8_0: *bytes = 34; *elems = 32; return true;
        case CPB_GGML_Q4_K: *bytes = 144; *elems = 256; return true;
        case CPB_GGML_Q6_K: *bytes = 210; *elems = 256; return true;
        case CPB_GGML_MXFP4: *bytes = 17; *elems = 32; return true;
        default: return false;
    }
}

struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    bool ok = true;
    bool take(void* dst, size_t k) {
        if (!ok || k > n - pos) { ok = false; return false; }
        memcpy(dst, p + pos, k);
        pos += k;
        return true;
    }
    template <class T>
    T get() {
        T v{};
        take(&v, sizeof v);
        return v;
    }
    std::string str() {
        uint64_t len = get<uint64_t>();
        if (!ok || len > n - pos) { ok = false; return {}; }
        std::string s((const char*)p + pos, (size_t)len);
        pos += len;
        return s;
    }
    // one value of type t; scalars and strings land in m, arrays are skipped
    void value(int t, Meta* m, int depth = 0) {
        switch (t) {
            case kU8: m->i = get<uint8_t>(); break;
            case kI8: m->i = get<int8_t>(); break;
            case kU16: m->i = get<uint16_t>(); break;
            case kI16: m->i = get<int16_t>(); break;
            case kU32: m->i = get<uint32_t>(); break;
            case kI32: m->i = get<int32_t>(); break;
            case kF32: m->f = get<float>(); break;
            case kBool: m->i = get<uint8_t>() != 0; break;
            case kStr: m->s = str(); break;
            case kU64: m->i = (int64_t)get<uint64_t>(); break;
            case kI64: m->i = get<int64_t>(); break;
            case kF64: m->f = get<double>(); break;
            case kArr: {
                const uint32_t et = get<uint32_t>();
                const uint64_t cnt = get<uint64_t>();
                if (!ok || depth > 2 || et > kF64) { ok = false; return; }
                static const uint8_t fixed[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
                if (et != kStr && et != kArr) {
                    if (cnt > (n - pos) / fixed[et]) { ok = false; return; }
                    pos += cnt * fixed[et];
                } else {
                    Meta tmp;
                    for (uint64_t k = 0; k < cnt && ok; k++) value((int)et, &tmp, depth + 1);
                }
                break;
            }
            default: ok = false;
        }
        m->type = t;
        if (t == kF32 || t == kF64) m->i = (int64_t)m->f;
        else if (t != kStr && t != kArr) m->f = (double)m->i;
    }
};

struct TensorRec {
    std::string name;
    cpb_gguf_tensor t{};
};

}  // namespace

struct cpb_gguf {
    int fd = -1;
    const uint8_t* base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_start = 0;
    std::unordered_map<std::string, Meta> meta;
    std::vector<std::string> meta_order;     // keys in file order (a repeated key keeps its first place)
    std::vector<TensorRec> tensors;
    std::unordered_map<std::string, size_t> by_name;
};

extern "C" {

void cpb_gguf_close(cpb_gguf_t* g) {
    if (!g) return;
    if (g->base) munmap((void*)g->base, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

int cpb_gguf_open(const char* path, cpb_gguf_t** out) {
    if (!path || !out) return fail(CPB_EINVAL, "NULL argument");
    *out = nullptr;
    cpb_gguf_t* g = new cpb_gguf_t();
    auto bail = [&](int r) { cpb_gguf_close(g); return r; };
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) return bail(fail(CPB_EINVAL, "cannot open %s", path));
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 24) return bail(fail(CPB_EINVAL, "%s: not a GGUF file (too small)", path));
    g->size = (size_t)st.st_size;
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return bail(fail(CPB_ENOMEM, "mmap of %s failed", path));
    g->base = (const uint8_t*)m;
    Reader r{g->base, g->size};
    char magic[4];
    r.take(magic, 4);
    if (memcmp(magic, "GGUF", 4) != 0) return bail(fail(CPB_EINVAL, "%s: bad magic", path));
    g->version = r.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return bail(fail(CPB_EINVAL, "%s: GGUF version %u not supported", path, g->version));
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    // each KV pair and tensor info takes at least 12 / 24 bytes
    if (!r.ok || n_kv > g->size / 12 || n_tensors > g->size / 24) return bail(fail(CPB_EINVAL, "%s: corrupt header", path));
    for (uint64_t i = 0; i < n_kv && r.ok; i++) {
        std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        Meta mv;
        r.value((int)t, &mv);
        if (r.ok) {
            if (!g->meta.count(key)) g->meta_order.push_back(key);
            g->meta[key] = mv;
        }
    }
    if (!r.ok) return bail(fail(CPB_EINVAL, "%s: truncated or corrupt metadata", path));
    auto al = g->meta.find("general.alignment");
    if (al != g->meta.end() && al->second.type != kArr && al->second.type != kStr) {
        if (al->second.i <= 0 || (al->second.i & (al->second.i - 1)))
            return bail(fail(CPB_EINVAL, "%s: bad general.alignment %lld", path, (long long)al->second.i));
        g->alignment = (uint64_t)al->second.i;
    }
    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        TensorRec& tr = g->tensors[i];
        tr.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd < 1 || nd > 4) return bail(fail(CPB_EINVAL, "%s: tensor %llu has %u dims", path, (unsigned long long)i, nd));
        tr.t.n_dims = (int32_t)nd;
        uint64_t ne = 1;
        for (uint32_t k = 0; k < nd; k++) {
            tr.t.dims[k] = r.get<uint64_t>();
            if (tr.t.dims[k] && ne > UINT64_MAX / tr.t.dims[k]) r.ok = false;
            ne *= tr.t.dims[k];
        }
        for (uint32_t k = nd; k < 4; k++) tr.t.dims[k] = 1;
        tr.t.type = (int32_t)r.get<uint32_t>();
        tr.t.offset = r.get<uint64_t>();
        tr.t.n_elements = ne;
        if (!r.ok) return bail(fail(CPB_EINVAL, "%s: truncated tensor infos", path));
    }
    g->data_start = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (size_t i = 0; i < g->tensors.size(); i++) {
        TensorRec& tr = g->tensors[i];
        uint64_t bs = 0, be = 0;
        if (type_size(tr.t.type, &bs, &be)) {
            if (tr.t.dims[0] % be) return bail(fail(CPB_EINVAL, "%s: %s: row of %llu not a multiple of the block (%llu)", path,
                                                    tr.name.c_str(), (unsigned long long)tr.t.dims[0], (unsigned long long)be));
            tr.t.n_bytes = tr.t.n_elements / be * bs;
            if (tr.t.offset > g->size || g->data_start > g->size - tr.t.offset ||
                tr.t.n_bytes > g->size - g->data_start - tr.t.offset)
                return bail(fail(CPB_EINVAL, "%s: %s: data beyond the end of the file", path, tr.name.c_str()));
            tr.t.data = g->base + g->data_start + tr.t.offset;
        } else {
            tr.t.n_bytes = 0;     // a type this library does not read: listed, no data pointer
            tr.t.data = nullptr;
        }
        if (g->by_name.count(tr.name)) return bail(fail(CPB_EINVAL, "%s: duplicate tensor %s", path, tr.name.c_str()));
        g->by_name[tr.name] = i;
    }
    for (auto& tr : g->tensors) tr.t.name = tr.name.c_str();
    *out = g;
    return 0;
}

int cpb_gguf_version(const cpb_gguf_t* g, uint32_t* version, uint64_t* data_start, uint64_t* alignment) {
    if (!g) return fail(CPB_EINVAL, "NULL handle");
    if (version) *version = g->version;
    if (data_start) *data_start = g->data_start;
    if (alignment) *alignment = g->alignment;
    return 0;
}

int cpb_gguf_n_tensors(const cpb_gguf_t* g, int64_t* n) {
    if (!g || !n) return fail(CPB_EINVAL, "NULL argument");
    *n = (int64_t)g->tensors.size();
    return 0;
}

int cpb_gguf_tensor_at(const cpb_gguf_t* g, int64_t i, cpb_gguf_tensor* out) {
    if (!g || !out) return fail(CPB_EINVAL, "NULL argument");
    if (i < 0 || i >= (int64_t)g->tensors.size()) return fail(CPB_EINVAL, "tensor index %lld out of range", (long long)i);
    *out = g->tensors[(size_t)i].t;
    return 0;
}

int cpb_gguf_find(const cpb_gguf_t* g, const char* name, cpb_gguf_tensor* out) {
    if (!g || !name || !out) return fail(CPB_EINVAL, "NULL argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return fail(CPB_EINVAL, "tensor %s not in the file", name);
    *out = g->tensors[it->second].t;
    return 0;
}

static const Meta* find_meta(const cpb_gguf_t* g, const char* key) {
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

int cpb_gguf_meta_i64(const cpb_gguf_t* g, const char* key, int64_t* out) {
    if (!g || !key || !out) return fail(CPB_EINVAL, "NULL argument");
    const Meta* m = find_meta(g, key);
    if (!m || m->type == kStr || m->type == kArr) return fail(CPB_EINVAL, "no scalar metadata %s", key);
    *out = m->i;
    return 0;
}

int cpb_gguf_meta_f64(const cpb_gguf_t* g, const char* key, double* out) {
    if (!g || !key || !out) return fail(CPB_EINVAL, "NULL argument");
    const Meta* m = find_meta(g, key);
    if (!m || m->type == kStr || m->type == kArr) return fail(CPB_EINVAL, "no scalar metadata %s", key);
    *out = m->f;
    return 0;
}

int cpb_gguf_meta_str(const cpb_gguf_t* g, const char* key, const char** out) {
    if (!g || !key || !out) return fail(CPB_EINVAL, "NULL argument");
    const Meta* m = find_meta(g, key);
    if (!m || m->type != kStr) return fail(CPB_EINVAL, "no string metadata %s", key);
    *out = m->s.c_str();
    return 0;
}

// setup_model.sh:54-58 g(*suffixes): the keys in file order, the first one
// equal to "<arch>.<suffix>" or ending in ".<suffix>" (an exact key later in
// the file does not win over an earlier suffix match)
static const Meta* hp(const cpb_gguf_t* g, const std::string& arch, const char* suffix) {
    const std::string exact = arch + "." + suffix, tail = std::string(".") + suffix;
    for (const std::string& k : g->meta_order) {
        const bool ends = k.size() >= tail.size() && k.compare(k.size() - tail.size(), tail.size(), tail) == 0;
        if (k == exact || ends) return &g->meta.find(k)->second;
    }
    return nullptr;
}

int cpb_gguf_hparams_get(const cpb_gguf_t* g, cpb_gguf_hparams* out) {
    if (!g || !out) return fail(CPB_EINVAL, "NULL argument");
    cpb_gguf_hparams h;
    memset(&h, 0, sizeof h);
    const Meta* a = find_meta(g, "general.architecture");
    std::string arch = a && a->type == kStr ? a->s : "?";
    snprintf(h.arch, sizeof h.arch, "%s", arch.c_str());
    auto gi = [&](const char* s) -> int64_t {
        const Meta* m = hp(g, arch, s);
        return m && m->type != kStr && m->type != kArr ? m->i : -1;
    };
    auto gf = [&](const char* s) -> double {
        const Meta* m = hp(g, arch, s);
        return m && m->type != kStr && m->type != kArr ? m->f : 0.0;
    };
    h.n_embd = gi("embedding_length");
    h.n_layer = gi("block_count");
    h.n_head = gi("attention.head_count");
    h.n_head_kv = gi("attention.head_count_kv");
    h.head_dim = gi("attention.key_length");
    h.n_expert = gi("expert_count");
    h.n_expert_used = gi("expert_used_count");
    h.n_ff_exp = gi("expert_feed_forward_length");
    h.sliding_window = gi("attention.sliding_window");
    h.rope_freq_base = gf("rope.freq_base");
    h.rms_eps = gf("attention.layer_norm_rms_epsilon");
    h.n_vocab = gi("vocab_size");
    h.context_length = gi("context_length");
    // derived as setup_model.sh does when the key is absent
    if (h.n_vocab < 0)
        for (auto& tr : g->tensors)
            if (tr.name == "token_embd.weight" || tr.name == "output.weight") {
                uint64_t m = 0;
                for (int k = 0; k < tr.t.n_dims; k++) m = tr.t.dims[k] > m ? tr.t.dims[k] : m;
                h.n_vocab = (int64_t)m;
                break;
            }
    if (h.n_ff_exp < 0)
        for (auto& tr : g->tensors)
            if (tr.name.size() >= 20 && tr.name.compare(tr.name.size() - 20, 20, "ffn_gate_exps.weight") == 0) {
                h.n_ff_exp = (int64_t)tr.t.dims[1];
                break;
            }
    *out = h;
    return 0;
}

int cpb_gguf_write_manifest(const cpb_gguf_t* g, const char* path) {
    if (!g || !path) return fail(CPB_EINVAL, "NULL argument");
    FILE* f = fopen(path, "w");
    if (!f) return fail(CPB_EINVAL, "cannot write %s", path);
    fprintf(f, "data_start %llu\n", (unsigned long long)g->data_start);
    for (auto& tr : g->tensors)
        fprintf(f, "%s %d %llu %llu\n", tr.name.c_str(), tr.t.type, (unsigned long long)tr.t.offset,
                (unsigned long long)tr.t.n_elements);
    const bool ok = fclose(f) == 0;
    return ok ? 0 : fail(CPB_EINVAL, "write of %s failed", path);
}

int cpb_moe_load_gguf_layer(cpb_moe_t* h, const cpb_gguf_t* g, int layer) {
    if (!h || !g) return fail(CPB_EINVAL, "NULL argument");
    cpb_moe_cfg c;
    if (int r = cpb_moe_config(h, &c)) return r;
    if (layer < 0 || layer >= c.n_layer) return fail(CPB_EINVAL, "layer %d out of range", layer);
    const uint64_t d = (uint64_t)c.d, ff = (uint64_t)c.d_ff, ne = (uint64_t)c.n_expert;
    char name[256];
    auto get = [&](const char* suffix, cpb_gguf_tensor* t, bool required, bool* found = nullptr) -> int {
        snprintf(name, sizeof name, "blk.%d.%s", layer, suffix);
        auto it = g->by_name.find(name);
        if (found) *found = it != g->by_name.end();
        if (it == g->by_name.end()) {
            t->data = nullptr;
            return required ? fail(CPB_EINVAL, "tensor %s not in the file", name) : 0;
        }
        *t = g->tensors[it->second].t;
        return 0;
    };
    auto shape = [&](const cpb_gguf_tensor& t, int nd, uint64_t a, uint64_t b, uint64_t c3) -> int {
        const uint64_t want[3] = {a, b, c3};
        bool ok = t.n_dims == nd;
        for (int k = 0; k < nd && ok; k++) ok = t.dims[k] == want[k];
        if (!ok) return fail(CPB_EINVAL, "%s: dims [%llu, %llu, %llu] (%d), expected [%llu, %llu, %llu] (%d)", t.name,
                             (unsigned long long)t.dims[0], (unsigned long long)t.dims[1], (unsigned long long)t.dims[2],
                             t.n_dims, (unsigned long long)a, (unsigned long long)b, (unsigned long long)c3, nd);
        return 0;
    };
    auto f32 = [&](const cpb_gguf_tensor& t) -> int {
        // engine_gpt2.rs:601-604: f32v asserts type 0
        if (t.type != CPB_GGML_F32) return fail(CPB_EINVAL, "%s: type %d, expected F32 (0)", t.name, t.type);
        return 0;
    };
    cpb_gguf_tensor tg, tu, td, tgb, tub, tdb, trw, trb, tn;
    bool has_norm = false;
    int r;
    if ((r = get("ffn_gate_exps.weight", &tg, true)) || (r = get("ffn_up_exps.weight", &tu, true)) ||
        (r = get("ffn_down_exps.weight", &td, true)) || (r = get("ffn_gate_inp.weight", &trw, true)) ||
        (r = get("ffn_norm.weight", &tn, false, &has_norm)))
        return r;
    if ((r = shape(tg, 3, d, ff, ne)) || (r = shape(tu, 3, d, ff, ne)) || (r = shape(td, 3, ff, d, ne)) ||
        (r = shape(trw, 2, d, ne, 1)) || (r = f32(trw)))
        return r;
    // a norm weight that is present must be F32 of [d] (absent: no norm weight)
    if (has_norm && ((r = shape(tn, 1, d, 1, 1)) || (r = f32(tn)))) return r;
    const float *gb = nullptr, *ub = nullptr, *db = nullptr, *rb = nullptr;
    if (c.has_bias) {
        if ((r = get("ffn_gate_exps.bias", &tgb, true)) || (r = get("ffn_up_exps.bias", &tub, true)) ||
            (r = get("ffn_down_exps.bias", &tdb, true)) || (r = get("ffn_gate_inp.bias", &trb, true)))
            return r;
        if ((r = shape(tgb, 2, ff, ne, 1)) || (r = f32(tgb)) || (r = shape(tub, 2, ff, ne, 1)) || (r = f32(tub)) ||
            (r = shape(tdb, 2, d, ne, 1)) || (r = f32(tdb)) || (r = shape(trb, 1, ne, 1, 1)) || (r = f32(trb)))
            return r;
        gb = (const float*)tgb.data; ub = (const float*)tub.data; db = (const float*)tdb.data; rb = (const float*)trb.data;
    }
    if (!tg.data || !tu.data || !td.data)
        return fail(CPB_EINVAL, "blk.%d: expert tensor of a type this library does not read (%d/%d/%d)", layer, tg.type,
                    tu.type, td.type);
    // the load call rejects types its kernels do not take (per matrix)
    return cpb_moe_load_layer_typed(h, layer, tg.type, tu.type, td.type, tg.data, tu.data, td.data, gb, ub, db,
                                    (const float*)trw.data, rb, tn.data ? (const float*)tn.data : nullptr);
}

}  // extern "C"
