// api.hip -- host side of the C ABI in include/cpb_moe.h.
//
// Owns device memory and the stream, re-lays out expert weights at load
// time, and sequences the per-token kernels:
//   route (rmsnorm + quant + router + top-k)  ->  gate/up (+SwiGLU + Q8 of h)
//   ->  down (+bias + weighted combine into x).
// Reference caller being replaced: the MoE block of forward_worker,
// engine_gpt2.rs:845-923 (and engine_qwen2.rs:395-433).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "cpb_moe.h"
#include "cpb_internal.h"
#include "moe_kq.h"
#include "moe_mx.h"
#include "moe_grouped.h"
#include "route.h"

// Static decode scratch of the no-allocation entry point
// (cpb_moe_forward_device_noalloc): one copy per GPU, held until the process
// ends.  Host code must use the address hipGetSymbolAddress gives for the
// current device (kept per device below), never this name.
constexpr size_t kScratchBytes = 256 * 1024;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
thread_local std::string g_err;
}  // namespace

namespace cpb {
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
}  // namespace cpb

namespace {
using cpb::fail;

#define HIP_OK(expr)                                                                   \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return fail(e_ == hipErrorOutOfMemory ? CPB_ENOMEM : CPB_ENODEV, "%s: %s", \
                        #expr, hipGetErrorString(e_));                                 \
    } while (0)

// Per-call device scratch of the decode (n_tok = 1) kernels: activations,
// routing results and h.  Carved from one block, either the handle's own
// allocation or the library's static no-allocation scratch.
struct DecodeBufs {
    float* xn = nullptr;                       // [d]
    int8_t* xq = nullptr;                      // [d], then its image [2d], xsb, xsum
    uint8_t* ximg = nullptr;
    float* xsb = nullptr;
    int32_t* xsum = nullptr;
    double *lstar = nullptr, *lbound = nullptr;  // [E]
    float* logits = nullptr;                   // [E]
    int32_t* ids = nullptr;                    // [k]
    float* wts = nullptr;                      // [k]
    int32_t* fallback = nullptr;               // [1]
    int8_t* hq = nullptr;                      // [k*ff], then its image [2*k*ff], hsb
    uint8_t* himg = nullptr;
    float* hsb = nullptr;
    int32_t* hsum = nullptr;                   // [k*ff/32]
    float* hbuf = nullptr;                     // [k*ff]
};

// Lay out the decode scratch for cfg from base (null: sizing only); returns
// the bytes used.  Every piece starts on a 256-byte boundary.
size_t carve_decode(const cpb_moe_cfg& c, unsigned char* base, DecodeBufs* b) {
    const size_t d = c.d, ff = c.d_ff, k = c.top_k, ne = c.n_expert;
    size_t o = 0;
    auto take = [&](size_t bytes) -> unsigned char* {
        unsigned char* p = base ? base + o : nullptr;
        o += (bytes + 255) / 256 * 256;
        return p;
    };
    DecodeBufs t;
    t.xn = (float*)take(4 * d);
    t.xq = (int8_t*)take(3 * d + 8 * (d / 32));
    t.lstar = (double*)take(8 * ne);
    t.lbound = (double*)take(8 * ne);
    t.logits = (float*)take(4 * ne);
    t.ids = (int32_t*)take(4 * k);
    t.wts = (float*)take(4 * k);
    t.fallback = (int32_t*)take(4);
    t.hq = (int8_t*)take(3 * k * ff + 4 * (k * ff / 32));
    t.hsum = (int32_t*)take(4 * (k * ff / 32));
    t.hbuf = (float*)take(4 * k * ff);
    if (base) {
        // xq, its matrix-core image (2 bytes per element), the x scales and
        // the per-32 sums share one piece, and so do hq, its image and the hq scales
        t.ximg = (uint8_t*)(t.xq + d);
        t.xsb = (float*)(t.xq + 3 * d);
        t.xsum = (int32_t*)(t.xq + 3 * d + 4 * (d / 32));
        t.himg = (uint8_t*)(t.hq + k * ff);
        t.hsb = (float*)(t.hq + 3 * k * ff);
    }
    if (b) *b = t;
    return o;
}

struct LayerDev {
    cpb::u32x4* gu = nullptr;   // gate+up stream layout
    cpb::u32x4* up = nullptr;   // unused (kept null)
    cpb::u32x4* dn = nullptr;   // down stream
    const uint16_t* dn_d = nullptr;   // Q6_K down: its fp16 d stream (inside the dn allocation)
    float *gate_b = nullptr, *up_b = nullptr, *down_b = nullptr;
    float *router_w = nullptr, *router_b = nullptr, *norm_w = nullptr;
    int gu_type = 0, down_type = 0;   // GGUF type ids of this layer's gate/up and down tensors
    bool loaded = false;
    bool mfma_exact = false;    // MXFP4 scales all in [32, 254]: the grouped matrix-core path is exact
};

}  // namespace

struct cpb_moe {
    cpb_moe_cfg cfg{};
    int device = 0;
    hipStream_t own = nullptr, stream = nullptr;
    std::vector<LayerDev> layers;
    int nb = 0, nbf = 0, parts_gu = 0, parts_dn = 0;
    bool mx = true;
    // activations / routing (device)
    float* params = nullptr;              // per-layer router / norm / bias parameters (one arena)
    float* x = nullptr;
    unsigned char* dec_base = nullptr;    // the handle's decode scratch (one allocation)
    unsigned char* noalloc_base = nullptr;  // this device's static scratch (device address)
    DecodeBufs b;
    // trace (device, lazily allocated)
    float *t_gu = nullptr, *t_h = nullptr, *t_dn = nullptr;
    int32_t *t_gu_sums = nullptr, *t_dn_sums = nullptr;
    // staging for raw GGUF bytes at load time
    uint8_t* staging = nullptr;
    size_t staging_size = 0;
    // grouped (n_tok > 1) MXFP4 path: per-token and per-pair scratch
    bool grouped = false;
    float *g_inv = nullptr, *g_xn = nullptr, *g_xsb = nullptr, *g_logits = nullptr, *g_wts = nullptr, *g_hsb = nullptr, *g_dnout = nullptr;
    int8_t *g_xq = nullptr, *g_hq = nullptr;
    uint8_t *g_ximg = nullptr, *g_himg = nullptr;
    double *g_lstar = nullptr, *g_lbound = nullptr;
    int32_t *g_ids = nullptr, *g_fallback = nullptr, *g_sorted = nullptr, *g_ntiles = nullptr;
    int32_t *g_xsum = nullptr, *g_hsum = nullptr;   // k-quant grouped path
    float* g_hbuf = nullptr;
    int4* g_tiles = nullptr;
    unsigned* d_special = nullptr;
    // captured HIP graphs of forward_device calls, keyed by their arguments,
    // with the call counter of their last use (least recently used evicted
    // beyond kMaxGraphs)
    std::map<std::tuple<int, int, float*, int, int, hipStream_t>, std::pair<hipGraphExec_t, unsigned long long>> graphs;
    unsigned long long graph_clock = 0;
    bool use_graphs = true;
    // timing
    bool timing = false;
    std::vector<hipEvent_t> ev_pool;
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> ev_used;
    double ms[3] = {0, 0, 0};
    long nl[3] = {0, 0, 0};
};

namespace {

template <class T>
int dmalloc(T** p, size_t n) {
    if (n == 0) n = 1;
    hipError_t e = hipMalloc((void**)p, n * sizeof(T));
    if (e != hipSuccess) return fail(CPB_ENOMEM, "hipMalloc(%zu bytes): %s", n * sizeof(T), hipGetErrorString(e));
    return 0;
}

int check_cfg(const cpb_moe_cfg* c) {
    if (!c) return fail(CPB_EINVAL, "cfg is NULL");
    if (c->d <= 0 || c->d_ff <= 0 || c->n_expert <= 0 || c->n_layer <= 0 || c->max_tokens <= 0)
        return fail(CPB_EINVAL, "non-positive shape in cfg");
    if (c->top_k < 1 || c->top_k > 8 || c->top_k > c->n_expert)
        return fail(CPB_EINVAL, "top_k=%d must be in [1, min(8, n_expert)]", c->top_k);
    if (c->n_expert > 256) return fail(CPB_EINVAL, "n_expert=%d > 256 not supported", c->n_expert);
    if (c->d < 3 * c->n_expert) return fail(CPB_EINVAL, "d=%d must be >= 3*n_expert", c->d);
    bool mx = c->wtype_gate_up == CPB_GGUF_MXFP4;
    if (mx) {
        if (c->wtype_down != CPB_GGUF_MXFP4) return fail(CPB_EINVAL, "MXFP4 gate/up requires MXFP4 down");
        if (c->d % 32 || c->d_ff % 32) return fail(CPB_EINVAL, "d and d_ff must be multiples of 32");
        if (c->d % cpb::mx_down_rt(c->top_k)) return fail(CPB_EINVAL, "d must be a multiple of %d", cpb::mx_down_rt(c->top_k));
        if ((c->d / 32 + 14) / 15 > cpb::kMaxParts || (c->d_ff / 32 + 14) / 15 > cpb::kMaxParts)
            return fail(CPB_EINVAL, "d, d_ff must be <= 3840");
    } else if (c->wtype_gate_up == CPB_GGUF_Q4_K) {
        if (c->wtype_down != CPB_GGUF_Q4_K && c->wtype_down != CPB_GGUF_Q6_K)
            return fail(CPB_EINVAL, "k-quant down must be Q4_K or Q6_K");
        if (c->d % 256 || c->d_ff % 256) return fail(CPB_EINVAL, "d and d_ff must be multiples of 256");
        if (c->d > 8192 || c->d_ff > 4096) return fail(CPB_EINVAL, "k-quant path supports d <= 8192, d_ff <= 4096");
        if (c->top_k != 1 && c->top_k != 2 && c->top_k != 4 && c->top_k != 8)
            return fail(CPB_EINVAL, "k-quant path supports top_k in {1,2,4,8}, got %d", c->top_k);
    } else {
        return fail(CPB_EINVAL, "unsupported gate/up type %d", c->wtype_gate_up);
    }
    if ((size_t)c->max_tokens * c->top_k > 16384)
        return fail(CPB_EINVAL, "max_tokens * top_k = %lld exceeds 16384", (long long)c->max_tokens * c->top_k);
    if (c->router != CPB_ROUTER_TOPK_SOFTMAX && c->router != CPB_ROUTER_SOFTMAX_TOPK)
        return fail(CPB_EINVAL, "bad router %d", c->router);
    if (c->act != CPB_ACT_SWIGLU_OAI && c->act != CPB_ACT_SILU) return fail(CPB_EINVAL, "bad act %d", c->act);
    if (mx && c->act != CPB_ACT_SWIGLU_OAI) return fail(CPB_EINVAL, "MXFP4 path implements SwiGLU-OAI only");
    if (!mx && c->act != CPB_ACT_SILU) return fail(CPB_EINVAL, "k-quant path implements SiLU only");
    if (c->norm != CPB_NORM_GPTOSS && c->norm != CPB_NORM_QWEN) return fail(CPB_EINVAL, "bad norm %d", c->norm);
    if (c->norm == CPB_NORM_QWEN && (c->norm_nt < 1 || c->norm_nt > 64))
        return fail(CPB_EINVAL, "norm_nt must be in [1,64]");
    if (c->norm == CPB_NORM_QWEN && c->d < 16 * c->norm_nt)
        return fail(CPB_EINVAL, "norm_nt=%d: slices of d=%d shorter than 16 elements", c->norm_nt, c->d);
    return 0;
}

size_t row_bytes(int type, int cols) {
    if (type == CPB_GGUF_MXFP4) return (size_t)cols / 32 * 17;
    if (type == CPB_GGUF_Q4_K) return (size_t)cols / 256 * 144;
    return (size_t)cols / 256 * 210;
}

// Device address of the static scratch on the current device, looked up once
// per device (each GPU holds its own copy at its own address).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_addr[kMaxDevices] = {};
int scratch_address(int device, unsigned char** out) {
    if (device < 0 || device >= kMaxDevices) return fail(CPB_EINVAL, "device %d beyond %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[device]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return fail(CPB_ENODEV, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_addr[device] = (unsigned char*)p;
    }
    *out = g_scratch_addr[device];
    return 0;
}

int ensure_staging(cpb_moe_t* h, size_t n) {
    if (h->staging_size >= n) return 0;
    if (h->staging) (void)hipFree(h->staging);
    h->staging = nullptr;
    h->staging_size = 0;
    if (int r = dmalloc(&h->staging, n)) return r;
    h->staging_size = n;
    return 0;
}

// Copy n floats into a preassigned slot of the parameter arena (null src:
// the parameter is absent and its pointer stays null).
int upload(float** dst, float* slot, const float* src, size_t n, hipStream_t s) {
    if (!src) { *dst = nullptr; return 0; }
    *dst = slot;
    HIP_OK(hipMemcpyAsync(slot, src, n * sizeof(float), hipMemcpyHostToDevice, s));
    return 0;
}

// Per-layer small parameters (router rows and bias, norm weights, expert
// biases) of every layer live in one allocation: the route and expert kernels
// then touch a few large pages instead of one small allocation per tensor
// per layer, which keeps their address translations warm.
size_t align64(size_t n) { return (n + 63) / 64 * 64; }
struct ParamSlots {
    size_t router_w, norm_w, router_b, gate_b, up_b, down_b, per_layer;
};
ParamSlots param_slots(const cpb_moe_cfg& c) {
    const size_t ne = c.n_expert, d = c.d, ff = c.d_ff;
    ParamSlots p{};
    size_t o = 0;
    p.router_w = o; o += align64(ne * d);
    p.norm_w = o; o += align64(d);
    p.router_b = o; o += align64(ne);
    p.gate_b = o; o += align64(ne * ff);
    p.up_b = o; o += align64(ne * ff);
    p.down_b = o; o += align64(ne * d);
    p.per_layer = o;
    return p;
}

void free_layer(LayerDev& L) {
    (void)hipFree(L.gu); (void)hipFree(L.up); (void)hipFree(L.dn);
    L = LayerDev{};
}

struct Timer {
    cpb_moe_t* h;
    int cls;
    hipEvent_t a = nullptr, b = nullptr;
    Timer(cpb_moe_t* hh, int c, bool allow = true) : h(hh), cls(c) {
        if (!h->timing || !allow) return;
        if (h->ev_pool.size() < 2) {
            for (int i = 0; i < 64; i++) { hipEvent_t e; if (hipEventCreate(&e) == hipSuccess) h->ev_pool.push_back(e); }
        }
        if (h->ev_pool.size() < 2) return;
        a = h->ev_pool.back(); h->ev_pool.pop_back();
        b = h->ev_pool.back(); h->ev_pool.pop_back();
        cpb::armed_events() = cpb::LaunchEvents{a, b};   // taken by the one kernel launched in this scope
    }
    ~Timer() {
        if (!a) return;
        cpb::armed_events() = cpb::LaunchEvents{};
        h->ev_used.push_back({cls, {a, b}});
    }
};

// Trace buffers, allocated on the first traced call: all of them or none
// (a failed allocation frees the ones already made, so no later call sees a
// partial set).  Down sums are sized for two per superblock, the larger of
// Q4_K's {sumi, mint} and Q6_K's {sumi}, since the type is per layer.
void free_trace(cpb_moe_t* h) {
    void* p[] = {h->t_gu, h->t_h, h->t_dn, h->t_gu_sums, h->t_dn_sums};
    for (void* q : p) if (q) (void)hipFree(q);
    h->t_gu = h->t_h = h->t_dn = nullptr;
    h->t_gu_sums = h->t_dn_sums = nullptr;
}
int ensure_trace(cpb_moe_t* h) {
    if (h->t_gu && h->t_h && h->t_dn && h->t_gu_sums && h->t_dn_sums) return 0;
    free_trace(h);
    const auto& c = h->cfg;
    size_t k = c.top_k;
    size_t gs = h->mx ? k * 2 * c.d_ff * (c.d / 32) : k * 2 * c.d_ff * (c.d / 256) * 2;
    size_t ds = h->mx ? k * c.d * (c.d_ff / 32) : k * c.d * (c.d_ff / 256) * 2;
    int r;
    if ((r = dmalloc(&h->t_gu, k * 2 * c.d_ff)) || (r = dmalloc(&h->t_h, k * c.d_ff)) || (r = dmalloc(&h->t_dn, k * c.d)) ||
        (r = dmalloc(&h->t_gu_sums, gs)) || (r = dmalloc(&h->t_dn_sums, ds))) {
        free_trace(h);
        return r;
    }
    return 0;
}

void clear_graphs(cpb_moe_t* h) {
    for (auto& g : h->graphs) (void)hipGraphExecDestroy(g.second.first);
    h->graphs.clear();
}

// A caller that passes a new x pointer or token count on every call would
// otherwise grow the cache without bound.
constexpr size_t kMaxGraphs = 16;
void evict_lru_graph(cpb_moe_t* h) {
    auto old = h->graphs.begin();
    for (auto it = h->graphs.begin(); it != h->graphs.end(); ++it)
        if (it->second.second < old->second.second) old = it;
    // the graph may still be executing on the stream: destroying an exec
    // that is in flight is not allowed
    (void)hipStreamSynchronize(h->stream);
    (void)hipGraphExecDestroy(old->second.first);
    h->graphs.erase(old);
}

// One token through one layer, x at device address dx.
int layer_token(cpb_moe_t* h, const DecodeBufs& B, int layer, float* dx, int apply_norm, bool trace,
                bool timed = true) {
    const auto& c = h->cfg;
    LayerDev& L = h->layers[layer];
    if (!L.loaded) return fail(CPB_ESTATE, "layer %d not loaded", layer);
    cpb::RouteArgs ra{};
    ra.x = dx; ra.norm_w = L.norm_w; ra.router_w = L.router_w; ra.router_b = L.router_b;
    ra.d = c.d; ra.n_expert = c.n_expert; ra.top_k = c.top_k;
    ra.norm = c.norm; ra.norm_nt = c.norm_nt; ra.apply_norm = apply_norm; ra.eps = c.rms_eps;
    ra.qk = h->mx ? 0 : 1;
    ra.xn = B.xn; ra.xq = B.xq; ra.ximg = B.ximg; ra.xsb = B.xsb; ra.xsum = B.xsum;
    ra.lstar = B.lstar; ra.lbound = B.lbound;
    // the route launch publishes certified logits; the gate/up kernel
    // selects at its start (no cross-workgroup hand-off inside a launch)
    {
        Timer tm(h, 0, timed);
        if (cpb::launch_route(&ra, h->stream)) return fail(CPB_ENODEV, "route launch failed");
    }
    if (h->mx) {
        cpb::GateUpArgs g{};
        g.w = L.gu; g.gate_b = L.gate_b; g.up_b = L.up_b;
        g.ximg = B.ximg; g.xsb = B.xsb;
        g.ids = B.ids;
        {
            g.sel.lstar = B.lstar; g.sel.lbound = B.lbound; g.sel.router_w = L.router_w; g.sel.router_b = L.router_b;
            g.sel.xn = B.xn; g.sel.ne = c.n_expert; g.sel.k = c.top_k; g.sel.d = c.d;
            g.sel.ids = B.ids; g.sel.wts = B.wts; g.sel.logits = B.logits; g.sel.fallback = B.fallback;
        }
        g.dff = c.d_ff; g.nb = h->nb; g.nparts = h->parts_gu; g.top_k = c.top_k;
        g.alpha = c.alpha; g.limit = c.limit;
        g.hq = B.hq; g.himg = B.himg; g.hsb = B.hsb;
        g.gu = h->t_gu; g.gu_sums = h->t_gu_sums; g.h = h->t_h;
        cpb::DownArgs dn{};
        dn.w = L.dn; dn.down_b = L.down_b; dn.himg = B.himg; dn.hsb = B.hsb;
        dn.ids = B.ids; dn.wts = B.wts;
        dn.d = c.d; dn.dff = c.d_ff; dn.nbf = h->nbf; dn.nparts = h->parts_dn; dn.top_k = c.top_k;
        dn.x = dx; dn.dn = h->t_dn; dn.dn_sums = h->t_dn_sums;
        {
            Timer tm(h, 1, timed);
            if (cpb::launch_gateup_mx(g, trace, h->stream)) return fail(CPB_ENODEV, "gate/up launch failed");
        }
        {
            Timer tm(h, 2, timed);
            if (cpb::launch_down_mx(dn, trace, h->stream)) return fail(CPB_ENODEV, "down launch failed");
        }
    } else {
        cpb::KqArgs k{};
        k.gu = L.gu; k.dn = L.dn; k.dn_d = L.dn_d; k.down_type = L.down_type;
        k.xq = B.xq; k.xs = B.xsb; k.xsum = B.xsum; k.ids = B.ids; k.wts = B.wts;
        {
            k.sel.lstar = B.lstar; k.sel.lbound = B.lbound; k.sel.router_w = L.router_w; k.sel.router_b = L.router_b;
            k.sel.xn = B.xn; k.sel.ne = c.n_expert; k.sel.k = c.top_k; k.sel.d = c.d;
            k.sel.ids = B.ids; k.sel.wts = B.wts; k.sel.logits = B.logits; k.sel.fallback = B.fallback;
        }
        k.d = c.d; k.dff = c.d_ff; k.top_k = c.top_k;
        k.hbuf = B.hbuf; k.hq = B.hq; k.hs = B.hsb; k.hsum = B.hsum; k.x = dx;
        k.gu_out = h->t_gu; k.gu_sums = h->t_gu_sums; k.dn_out = h->t_dn; k.dn_sums = h->t_dn_sums;
        {
            Timer tm(h, 1, timed);
            if (cpb::launch_gateup_kq(k, trace, h->stream)) return fail(CPB_ENODEV, "k-quant gate/up launch failed");
        }
        {
            Timer tm(h, 2, timed);
            if (cpb::launch_down_kq(k, trace, h->stream)) return fail(CPB_ENODEV, "k-quant down launch failed");
        }
    }
    return 0;
}

}  // namespace

extern "C" {

const char* cpb_moe_last_error(void) { return g_err.c_str(); }

int cpb_moe_layer_bytes(const cpb_moe_cfg* c, size_t* out) {
    if (int r = check_cfg(c)) return r;
    if (!out) return fail(CPB_EINVAL, "out is NULL");
    if (c->wtype_gate_up == CPB_GGUF_MXFP4)
        *out = cpb::mx_gateup_bytes(c->n_expert, c->d_ff, c->d / 32) +
               cpb::mx_down_bytes(c->n_expert, c->d, c->d_ff / 32, c->top_k);
    else
        *out = (size_t)c->n_expert * (2 * c->d_ff * row_bytes(c->wtype_gate_up, c->d) +
                                      c->d * row_bytes(c->wtype_down, c->d_ff));
    return 0;
}

int cpb_moe_create(const cpb_moe_cfg* cfg, int device, cpb_moe_t** out) {
    if (!out) return fail(CPB_EINVAL, "out is NULL");
    *out = nullptr;
    if (int r = check_cfg(cfg)) return r;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return fail(CPB_ENODEV, "no HIP device");
    if (device < 0 || device >= ndev) return fail(CPB_EINVAL, "device %d out of range (%d devices)", device, ndev);
    HIP_OK(hipSetDevice(device));
    cpb_moe_t* h = new cpb_moe_t();
    h->cfg = *cfg;
    h->device = device;
    h->mx = cfg->wtype_gate_up == CPB_GGUF_MXFP4;
    h->nb = cfg->d / 32;
    h->nbf = cfg->d_ff / 32;
    h->parts_gu = (h->nb + cpb::kBlkPerPart - 1) / cpb::kBlkPerPart;
    h->parts_dn = (h->nbf + cpb::kBlkPerPart - 1) / cpb::kBlkPerPart;
    h->layers.resize(cfg->n_layer);
    auto bail = [&](int r) { cpb_moe_destroy(h); return r; };
    if (hipStreamCreateWithFlags(&h->own, hipStreamNonBlocking) != hipSuccess) return bail(fail(CPB_ENODEV, "stream create failed"));
    h->stream = h->own;
    const size_t d = cfg->d, ff = cfg->d_ff, k = cfg->top_k, ne = cfg->n_expert, T = cfg->max_tokens;
    int r;
    if ((r = dmalloc(&h->x, T * d)) || (r = dmalloc(&h->dec_base, carve_decode(*cfg, nullptr, nullptr))) ||
        (r = dmalloc(&h->params, param_slots(*cfg).per_layer * cfg->n_layer)))
        return bail(r);
    carve_decode(*cfg, h->dec_base, &h->b);
    if ((r = scratch_address(device, &h->noalloc_base))) return bail(r);
    if (h->mx && (r = dmalloc(&h->d_special, 1))) return bail(r);
    h->grouped = T > 1;
    if (const char* v = getenv("CPB_GROUPED")) h->grouped = h->grouped && v[0] != '0';
    if (T > 1) {
        // grouped (batched) path: per-token and per-pair buffers; MXFP4 uses
        // the fp8 images, the k-quant path the per-32 sums and fp32 h
        const size_t nb = d / 32, nbf = ff / 32, np = T * k;
        if ((r = dmalloc(&h->g_xn, T * d)) || (r = dmalloc(&h->g_inv, T)) || (r = dmalloc(&h->g_xq, T * d)) || (r = dmalloc(&h->g_xsb, T * nb)) ||
            (r = dmalloc(&h->g_lstar, T * ne)) ||
            (r = dmalloc(&h->g_lbound, T * ne)) || (r = dmalloc(&h->g_logits, T * ne)) || (r = dmalloc(&h->g_ids, np)) ||
            (r = dmalloc(&h->g_wts, np)) || (r = dmalloc(&h->g_fallback, T)) || (r = dmalloc(&h->g_sorted, np)) ||
            (r = dmalloc(&h->g_tiles, np / 32 + ne + 1)) || (r = dmalloc(&h->g_ntiles, 1)) ||
            (r = dmalloc(&h->g_hq, np * ff)) || (r = dmalloc(&h->g_hsb, np * nbf)) || (r = dmalloc(&h->g_dnout, np * d)))
            return bail(r);
        if (h->mx && ((r = dmalloc(&h->g_ximg, T * nb * 64)) || (r = dmalloc(&h->g_himg, np * nbf * 64)))) return bail(r);
        if (!h->mx && ((r = dmalloc(&h->g_xsum, T * nb)) || (r = dmalloc(&h->g_hsum, np * nbf)) || (r = dmalloc(&h->g_hbuf, np * ff))))
            return bail(r);
    }
    if (hipMemsetAsync(h->b.fallback, 0, sizeof(int32_t), h->stream) != hipSuccess ||
        hipStreamSynchronize(h->stream) != hipSuccess)
        return bail(fail(CPB_ENODEV, "init memset failed"));
    *out = h;
    return 0;
}

int cpb_moe_load_layer(cpb_moe_t* h, int layer, const void* gate, const void* up, const void* down,
                       const float* gate_b, const float* up_b, const float* down_b,
                       const float* router_w, const float* router_b, const float* norm_w) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    return cpb_moe_load_layer_typed(h, layer, h->cfg.wtype_gate_up, h->cfg.wtype_gate_up, h->cfg.wtype_down, gate, up,
                                    down, gate_b, up_b, down_b, router_w, router_b, norm_w);
}

int cpb_moe_load_layer_typed(cpb_moe_t* h, int layer, int gate_type, int up_type, int down_type, const void* gate,
                             const void* up, const void* down, const float* gate_b, const float* up_b,
                             const float* down_b, const float* router_w, const float* router_b,
                             const float* norm_w) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    const auto& c = h->cfg;
    if (layer < 0 || layer >= c.n_layer) return fail(CPB_EINVAL, "layer %d out of range", layer);
    // per-tensor type dispatch (engine_qwen2.rs:202-233 reads each matrix's
    // GGUF type): the MXFP4 kernels take type 39 only; the k-quant kernels
    // take Q4_K gate/up and a Q4_K or Q6_K down, chosen per layer
    if (h->mx) {
        if (gate_type != CPB_GGUF_MXFP4 || up_type != CPB_GGUF_MXFP4 || down_type != CPB_GGUF_MXFP4)
            return fail(CPB_EINVAL, "layer %d: MXFP4 handle needs type 39 for gate/up/down, got %d/%d/%d", layer,
                        gate_type, up_type, down_type);
    } else {
        if (gate_type != CPB_GGUF_Q4_K || up_type != CPB_GGUF_Q4_K)
            return fail(CPB_EINVAL, "layer %d: k-quant gate/up must be Q4_K (12), got %d/%d", layer, gate_type, up_type);
        if (down_type != CPB_GGUF_Q4_K && down_type != CPB_GGUF_Q6_K)
            return fail(CPB_EINVAL, "layer %d: k-quant down must be Q4_K (12) or Q6_K (14), got %d", layer, down_type);
    }
    if (!gate || !up || !down || !router_w) return fail(CPB_EINVAL, "gate/up/down/router_w must not be NULL");
    if (c.has_bias && (!gate_b || !up_b || !down_b || !router_b))
        return fail(CPB_EINVAL, "has_bias set but a bias pointer is NULL");
    HIP_OK(hipSetDevice(h->device));
    HIP_OK(hipStreamSynchronize(h->stream));
    clear_graphs(h);
    LayerDev& L = h->layers[layer];
    free_layer(L);
    const size_t ne = c.n_expert, d = c.d, ff = c.d_ff;
    const size_t gbytes = ne * ff * row_bytes(gate_type, d);
    const size_t dbytes = ne * d * row_bytes(down_type, ff);
    int r;
    if (h->mx) {
        if ((r = ensure_staging(h, 2 * gbytes > dbytes ? 2 * gbytes : dbytes))) return r;
        HIP_OK(hipMemcpyAsync(h->staging, gate, gbytes, hipMemcpyHostToDevice, h->stream));
        HIP_OK(hipMemcpyAsync(h->staging + gbytes, up, gbytes, hipMemcpyHostToDevice, h->stream));
        HIP_OK(hipMemsetAsync(h->d_special, 0, sizeof(unsigned), h->stream));
        if (cpb::launch_count_special_exps(h->staging, 2 * gbytes / 17, h->d_special, h->stream))
            return fail(CPB_ENODEV, "exponent scan launch failed");
        if ((r = dmalloc((uint8_t**)&L.gu, cpb::mx_gateup_bytes(ne, ff, d / 32)))) return r;
        if (cpb::launch_repack_gateup(h->staging, h->staging + gbytes, L.gu, ne, ff, d / 32, h->stream))
            return fail(CPB_ENODEV, "repack launch failed");
        HIP_OK(hipStreamSynchronize(h->stream));
        HIP_OK(hipMemcpyAsync(h->staging, down, dbytes, hipMemcpyHostToDevice, h->stream));
        if (cpb::launch_count_special_exps(h->staging, dbytes / 17, h->d_special, h->stream))
            return fail(CPB_ENODEV, "exponent scan launch failed");
        if ((r = dmalloc((uint8_t**)&L.dn, cpb::mx_down_bytes(ne, d, ff / 32, c.top_k)))) return r;
        if (cpb::launch_repack_down(h->staging, L.dn, ne, d, ff / 32, c.top_k, h->stream))
            return fail(CPB_ENODEV, "repack launch failed");
    } else {
        if ((r = ensure_staging(h, 2 * gbytes > dbytes ? 2 * gbytes : dbytes))) return r;
        HIP_OK(hipMemcpyAsync(h->staging, gate, gbytes, hipMemcpyHostToDevice, h->stream));
        HIP_OK(hipMemcpyAsync(h->staging + gbytes, up, gbytes, hipMemcpyHostToDevice, h->stream));
        if ((r = dmalloc((uint8_t**)&L.gu, cpb::kq_gateup_bytes(ne, ff, d)))) return r;
        if (cpb::launch_repack_kq_gateup(h->staging, h->staging + gbytes, L.gu, ne, ff, d, h->stream))
            return fail(CPB_ENODEV, "repack launch failed");
        HIP_OK(hipStreamSynchronize(h->stream));
        HIP_OK(hipMemcpyAsync(h->staging, down, dbytes, hipMemcpyHostToDevice, h->stream));
        if ((r = dmalloc((uint8_t**)&L.dn, cpb::kq_down_bytes(ne, d, ff, c.top_k, down_type)))) return r;
        if (cpb::launch_repack_kq_down(h->staging, L.dn, ne, d, ff, c.top_k, down_type, h->stream))
            return fail(CPB_ENODEV, "repack launch failed");
        L.dn_d = cpb::kq_down_dstream(L.dn, ne, d, ff, down_type);
    }
    const ParamSlots ps = param_slots(c);
    float* base = h->params + (size_t)layer * ps.per_layer;
    if (c.has_bias) {
        if ((r = upload(&L.gate_b, base + ps.gate_b, gate_b, ne * ff, h->stream)) ||
            (r = upload(&L.up_b, base + ps.up_b, up_b, ne * ff, h->stream)) ||
            (r = upload(&L.down_b, base + ps.down_b, down_b, ne * d, h->stream)) ||
            (r = upload(&L.router_b, base + ps.router_b, router_b, ne, h->stream)))
            return r;
    }
    if ((r = upload(&L.router_w, base + ps.router_w, router_w, ne * d, h->stream))) return r;
    if ((r = upload(&L.norm_w, base + ps.norm_w, norm_w, d, h->stream))) return r;
    HIP_OK(hipStreamSynchronize(h->stream));
    if (h->mx) {
        unsigned special = 0;
        HIP_OK(hipMemcpy(&special, h->d_special, sizeof special, hipMemcpyDeviceToHost));
        L.mfma_exact = special == 0;
    }
    L.gu_type = gate_type;
    L.down_type = down_type;
    L.loaded = true;
    return 0;
}

// n_tok > 1 tokens through one MXFP4 layer on the matrix cores (bit-identical
// to per-token decode); sums (test hook) receive the int32 block sums.
static int layer_grouped(cpb_moe_t* h, int layer, float* d_x, int n_tok, int apply_norm, int32_t* gu_sums,
                         int32_t* dn_sums) {
    const auto& c = h->cfg;
    const LayerDev& L = h->layers[layer];
    cpb::GroupedArgs g{};
    g.norm_w = L.norm_w; g.router_w = L.router_w; g.router_b = L.router_b;
    g.gu = L.gu; g.dn = L.dn; g.dn_d = L.dn_d; g.gate_b = L.gate_b; g.up_b = L.up_b; g.down_b = L.down_b;
    g.n_tok = n_tok; g.d = c.d; g.dff = c.d_ff; g.ne = c.n_expert; g.k = c.top_k; g.nb = h->nb; g.nbf = h->nbf;
    g.parts_gu = h->parts_gu; g.parts_dn = h->parts_dn;
    g.norm = c.norm; g.norm_nt = c.norm_nt; g.apply_norm = apply_norm;
    g.eps = c.rms_eps; g.alpha = c.alpha; g.limit = c.limit;
    g.max_tiles = n_tok * c.top_k / 32 + c.n_expert + 1;
    g.x = d_x; g.xn = h->g_xn; g.inv = h->g_inv; g.xq = h->g_xq; g.xsb = h->g_xsb; g.ximg = h->g_ximg;
    g.lstar = h->g_lstar; g.lbound = h->g_lbound; g.logits = h->g_logits; g.ids = h->g_ids; g.wts = h->g_wts;
    g.fallback = h->g_fallback; g.sorted = h->g_sorted; g.tiles = h->g_tiles; g.ntiles = h->g_ntiles;
    g.hq = h->g_hq; g.hsb = h->g_hsb; g.himg = h->g_himg; g.dnout = h->g_dnout;
    g.kq = h->mx ? 0 : 1; g.down_type = L.down_type;
    g.xsum = h->g_xsum; g.hbuf = h->g_hbuf; g.hsum = h->g_hsum;
    g.gu_sums = gu_sums; g.dn_sums = dn_sums;
    // timing mode: events around the two expert GEMMs (classes gate/up, down)
    cpb::LaunchEvents ev[2];
    Timer t1(h, 1), t2(h, 2);
    const bool timed = t1.a && t2.a;
    if (timed) {
        ev[0] = cpb::LaunchEvents{t1.a, t1.b};
        ev[1] = cpb::LaunchEvents{t2.a, t2.b};
    }
    cpb::armed_events() = cpb::LaunchEvents{};
    const int r = cpb::launch_grouped_layer(g, gu_sums != nullptr, h->stream, timed ? ev : nullptr);
    cpb::armed_events() = cpb::LaunchEvents{};
    if (r) return fail(CPB_ENODEV, "grouped layer launch failed");
    return 0;
}

static int launch_direct(cpb_moe_t* h, int layer0, int n_layers, float* d_x, int n_tok, int apply_norm) {
    const auto& c = h->cfg;
    for (int l = layer0; l < layer0 + n_layers; l++) {
        if (n_tok > 1 && h->grouped && (h->mx ? h->layers[l].mfma_exact : c.d <= 4096)) {
            if (int r = layer_grouped(h, l, d_x, n_tok, apply_norm, nullptr, nullptr)) return r;
            continue;
        }
        for (int t = 0; t < n_tok; t++)
            if (int r = layer_token(h, h->b, l, d_x + (size_t)t * c.d, apply_norm, false)) return r;
    }
    return 0;
}

int cpb_moe_forward_device(cpb_moe_t* h, int layer0, int n_layers, float* d_x, int n_tok, int apply_norm) {
    if (!h || !d_x) return fail(CPB_EINVAL, "NULL argument");
    const auto& c = h->cfg;
    if (layer0 < 0 || n_layers < 0 || layer0 + n_layers > c.n_layer) return fail(CPB_EINVAL, "layer range out of bounds");
    if (n_tok < 1 || n_tok > c.max_tokens) return fail(CPB_EINVAL, "n_tok=%d outside [1, max_tokens=%d]", n_tok, c.max_tokens);
    for (int l = layer0; l < layer0 + n_layers; l++)
        if (!h->layers[l].loaded) return fail(CPB_ESTATE, "layer %d not loaded", l);
    HIP_OK(hipSetDevice(h->device));
    // per-kernel timing needs one event pair per launch: run those directly
    if (h->timing || !h->use_graphs) return launch_direct(h, layer0, n_layers, d_x, n_tok, apply_norm);
    // a caller capturing this stream into a graph of its own gets the
    // kernels themselves in that graph
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_OK(hipStreamIsCapturing(h->stream, &cap));
    if (cap != hipStreamCaptureStatusNone) return launch_direct(h, layer0, n_layers, d_x, n_tok, apply_norm);
    // replay one captured graph per distinct call (launch overhead of ~3
    // kernels per layer paid once)
    auto key = std::make_tuple(layer0, n_layers, d_x, n_tok, apply_norm, h->stream);
    auto it = h->graphs.find(key);
    if (it == h->graphs.end()) {
        if (h->graphs.size() >= kMaxGraphs) evict_lru_graph(h);
        HIP_OK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
        int r = launch_direct(h, layer0, n_layers, d_x, n_tok, apply_norm);
        hipGraph_t g = nullptr;
        hipError_t ec = hipStreamEndCapture(h->stream, &g);
        if (r) { if (g) (void)hipGraphDestroy(g); return r; }
        if (ec != hipSuccess) return fail(CPB_ENODEV, "graph capture failed: %s", hipGetErrorString(ec));
        hipGraphExec_t ge = nullptr;
        ec = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ec != hipSuccess) return fail(CPB_ENODEV, "graph instantiate failed: %s", hipGetErrorString(ec));
        it = h->graphs.emplace(key, std::make_pair(ge, 0ull)).first;
    }
    it->second.second = ++h->graph_clock;
    HIP_OK(hipGraphLaunch(it->second.first, h->stream));
    return 0;
}

int cpb_moe_forward_device_noalloc(cpb_moe_t* h, int layer0, int n_layers, float* d_x, int n_tok, int apply_norm) {
    if (!h || !d_x) return fail(CPB_EINVAL, "NULL argument");
    const auto& c = h->cfg;
    if (layer0 < 0 || n_layers < 0 || layer0 + n_layers > c.n_layer) return fail(CPB_EINVAL, "layer range out of bounds");
    if (n_tok < 1 || n_tok > c.max_tokens) return fail(CPB_EINVAL, "n_tok=%d outside [1, max_tokens=%d]", n_tok, c.max_tokens);
    const size_t need = carve_decode(c, nullptr, nullptr);
    if (need > kScratchBytes)
        return fail(CPB_EINVAL, "this shape needs %zu bytes of decode scratch; the static scratch holds %zu", need,
                    kScratchBytes);
    for (int l = layer0; l < layer0 + n_layers; l++)
        if (!h->layers[l].loaded) return fail(CPB_ESTATE, "layer %d not loaded", l);
    if (!h->noalloc_base) return fail(CPB_ESTATE, "static scratch address not set up");
    HIP_OK(hipSetDevice(h->device));
    // the decode kernels, one token at a time, launched directly (no graph:
    // instantiating one allocates); every scratch element they read is
    // written earlier in the same call, so nothing needs clearing first
    DecodeBufs B;
    carve_decode(c, h->noalloc_base, &B);
    for (int l = layer0; l < layer0 + n_layers; l++)
        for (int t = 0; t < n_tok; t++)
            if (int r = layer_token(h, B, l, d_x + (size_t)t * c.d, apply_norm, false, false)) return r;
    return 0;
}

int cpb_moe_grouped_sums(cpb_moe_t* h, int layer, float* x, int n_tok, int apply_norm, int32_t* gu_sums,
                         int32_t* dn_sums) {
    if (!h || !x || !gu_sums || !dn_sums) return fail(CPB_EINVAL, "NULL argument");
    const auto& c = h->cfg;
    if (!h->grouped) return fail(CPB_EINVAL, "grouped path needs max_tokens > 1");
    if (layer < 0 || layer >= c.n_layer || !h->layers[layer].loaded) return fail(CPB_ESTATE, "layer %d not loaded", layer);
    if (h->mx && !h->layers[layer].mfma_exact) return fail(CPB_EINVAL, "layer %d has e8m0 scales outside [32, 254]", layer);
    if (!h->mx && c.d > 4096) return fail(CPB_EINVAL, "k-quant grouped path takes d <= 4096");
    if (n_tok < 2 || n_tok > c.max_tokens) return fail(CPB_EINVAL, "n_tok=%d outside [2, max_tokens=%d]", n_tok, c.max_tokens);
    HIP_OK(hipSetDevice(h->device));
    const size_t d = c.d, np = (size_t)n_tok * c.top_k;
    const size_t ngu = h->mx ? np * 2 * c.d_ff * h->nb : np * 2 * c.d_ff * (d / 256) * 2;
    const size_t ndn = h->mx ? np * d * h->nbf
                             : np * d * (c.d_ff / 256) * (h->layers[layer].down_type == CPB_GGUF_Q4_K ? 2 : 1);
    int32_t *dgu = nullptr, *ddn = nullptr;
    int r;
    if ((r = dmalloc(&dgu, ngu)) || (r = dmalloc(&ddn, ndn))) { (void)hipFree(dgu); return r; }
    r = 0;
    if (hipMemcpyAsync(h->x, x, n_tok * d * sizeof(float), hipMemcpyHostToDevice, h->stream) != hipSuccess) r = CPB_ENODEV;
    if (!r) r = layer_grouped(h, layer, h->x, n_tok, apply_norm, dgu, ddn);
    if (!r && (hipMemcpyAsync(x, h->x, n_tok * d * sizeof(float), hipMemcpyDeviceToHost, h->stream) != hipSuccess ||
               hipMemcpyAsync(gu_sums, dgu, ngu * 4, hipMemcpyDeviceToHost, h->stream) != hipSuccess ||
               hipMemcpyAsync(dn_sums, ddn, ndn * 4, hipMemcpyDeviceToHost, h->stream) != hipSuccess ||
               hipStreamSynchronize(h->stream) != hipSuccess))
        r = fail(CPB_ENODEV, "grouped sums copy failed");
    (void)hipFree(dgu);
    (void)hipFree(ddn);
    return r;
}

int cpb_moe_forward(cpb_moe_t* h, int layer, float* x, int n_tok, int apply_norm, cpb_moe_trace* tr) {
    if (!h || !x) return fail(CPB_EINVAL, "NULL argument");
    const auto& c = h->cfg;
    if (layer < 0 || layer >= c.n_layer) return fail(CPB_EINVAL, "layer %d out of range", layer);
    if (n_tok < 1 || n_tok > c.max_tokens) return fail(CPB_EINVAL, "n_tok=%d outside [1, max_tokens=%d]", n_tok, c.max_tokens);
    if (tr && n_tok != 1) return fail(CPB_EINVAL, "trace requires n_tok == 1");
    HIP_OK(hipSetDevice(h->device));
    const size_t d = c.d;
    HIP_OK(hipMemcpyAsync(h->x, x, n_tok * d * sizeof(float), hipMemcpyHostToDevice, h->stream));
    if (tr) {
        if (int r = ensure_trace(h)) return r;
        if (int r = layer_token(h, h->b, layer, h->x, apply_norm, true)) return r;
    } else {
        if (int r = cpb_moe_forward_device(h, layer, 1, h->x, n_tok, apply_norm)) return r;
    }
    HIP_OK(hipMemcpyAsync(x, h->x, n_tok * d * sizeof(float), hipMemcpyDeviceToHost, h->stream));
    if (tr) {
        const size_t k = c.top_k, ff = c.d_ff, ne = c.n_expert;
        const bool mx = h->mx;
        auto cp = [&](void* dst, const void* src, size_t bytes) -> int {
            if (dst && bytes) HIP_OK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, h->stream));
            return 0;
        };
        int r = 0;
        r |= cp(tr->xn, h->b.xn, d * 4);
        r |= cp(tr->xq, h->b.xq, d);
        r |= cp(tr->xsb, h->b.xsb, (mx ? d / 32 : d / 256) * 4);
        r |= cp(tr->xsum, h->b.xsum, mx ? 0 : d / 32 * 4);
        r |= cp(tr->logits, h->b.logits, ne * 4);
        r |= cp(tr->ids, h->b.ids, k * 4);
        r |= cp(tr->wts, h->b.wts, k * 4);
        r |= cp(tr->gu, h->t_gu, k * 2 * ff * 4);
        r |= cp(tr->gu_sums, h->t_gu_sums, (mx ? k * 2 * ff * (d / 32) : k * 2 * ff * (d / 256) * 2) * 4);
        r |= cp(tr->hq, h->b.hq, k * ff);
        r |= cp(tr->hsb, h->b.hsb, (mx ? k * ff / 32 : k * ff / 256) * 4);
        r |= cp(tr->hsum, h->b.hsum, mx ? 0 : k * ff / 32 * 4);
        r |= cp(tr->dn, h->t_dn, k * d * 4);
        r |= cp(tr->dn_sums, h->t_dn_sums,
                (mx ? k * d * (ff / 32) : k * d * (ff / 256) * (h->layers[layer].down_type == CPB_GGUF_Q4_K ? 2 : 1)) * 4);
        r |= cp(tr->h, mx ? h->t_h : h->b.hbuf, k * ff * 4);
        int32_t fb = 0;
        r |= cp(&fb, h->b.fallback, 4);
        HIP_OK(hipStreamSynchronize(h->stream));
        tr->exact_router_fallbacks = fb;
        if (r) return r;
    }
    HIP_OK(hipStreamSynchronize(h->stream));
    return 0;
}

int cpb_moe_config(const cpb_moe_t* h, cpb_moe_cfg* out) {
    if (!h || !out) return fail(CPB_EINVAL, "NULL argument");
    *out = h->cfg;
    return 0;
}

int cpb_moe_set_stream(cpb_moe_t* h, void* stream) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    hipStream_t ns = stream ? (hipStream_t)stream : h->own;
    if (ns == h->stream) return 0;
    HIP_OK(hipSetDevice(h->device));
    // every launch shares the handle's scratch: work on the new stream waits
    // for what is still queued on the old one (not across a graph capture,
    // where the capturing caller orders its own work)
    hipStreamCaptureStatus c0 = hipStreamCaptureStatusNone, c1 = hipStreamCaptureStatusNone;
    HIP_OK(hipStreamIsCapturing(h->stream, &c0));
    HIP_OK(hipStreamIsCapturing(ns, &c1));
    if (c0 != hipStreamCaptureStatusNone || c1 != hipStreamCaptureStatusNone) {
        h->stream = ns;
        return 0;
    }
    hipEvent_t ev = nullptr;
    HIP_OK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    hipError_t e = hipEventRecord(ev, h->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(ns, ev, 0);
    (void)hipEventDestroy(ev);
    if (e != hipSuccess) return fail(CPB_ENODEV, "stream switch: %s", hipGetErrorString(e));
    h->stream = ns;
    return 0;
}

int cpb_moe_sync(cpb_moe_t* h) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    HIP_OK(hipStreamSynchronize(h->stream));
    return 0;
}

int cpb_moe_timing(cpb_moe_t* h, int enable) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    HIP_OK(hipStreamSynchronize(h->stream));
    for (auto& u : h->ev_used) { h->ev_pool.push_back(u.second.first); h->ev_pool.push_back(u.second.second); }
    h->ev_used.clear();
    h->timing = enable != 0;
    for (int i = 0; i < 3; i++) { h->ms[i] = 0; h->nl[i] = 0; }
    return 0;
}

int cpb_moe_kernel_times(cpb_moe_t* h, double ms[3], long n[3]) {
    if (!h || !ms || !n) return fail(CPB_EINVAL, "NULL argument");
    HIP_OK(hipStreamSynchronize(h->stream));
    for (auto& u : h->ev_used) {
        float t = 0;
        HIP_OK(hipEventElapsedTime(&t, u.second.first, u.second.second));
        h->ms[u.first] += t;
        h->nl[u.first] += 1;
        h->ev_pool.push_back(u.second.first);
        h->ev_pool.push_back(u.second.second);
    }
    h->ev_used.clear();
    for (int i = 0; i < 3; i++) { ms[i] = h->ms[i]; n[i] = h->nl[i]; }
    return 0;
}

void cpb_moe_destroy(cpb_moe_t* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    clear_graphs(h);
    void* gbufs[] = {h->g_xsum, h->g_hsum, h->g_hbuf,
                     h->g_inv, h->g_xn, h->g_xsb, h->g_logits, h->g_wts, h->g_hsb, h->g_dnout, h->g_xq, h->g_hq, h->g_ximg,
                     h->g_himg, h->g_lstar, h->g_lbound, h->g_ids, h->g_fallback, h->g_sorted, h->g_ntiles, h->g_tiles,
                     h->d_special};
    for (void* p : gbufs) (void)hipFree(p);
    for (auto& L : h->layers) free_layer(L);
    void* bufs[] = {h->params, h->x, h->dec_base, h->t_gu, h->t_h,
                    h->t_dn, h->t_gu_sums, h->t_dn_sums, h->staging};
    for (void* p : bufs) if (p) (void)hipFree(p);
    for (auto& u : h->ev_used) { (void)hipEventDestroy(u.second.first); (void)hipEventDestroy(u.second.second); }
    for (auto e : h->ev_pool) (void)hipEventDestroy(e);
    if (h->own) (void)hipStreamDestroy(h->own);
    delete h;
}

}  // extern "C"
