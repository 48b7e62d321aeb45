// attn.hip -- gpt-oss attention block, decode, on gfx950.
//
// Reference (src/bin/): engine_gpt2.rs:772-843 (the layer's attention),
// rope_init / rope_yarn_slow / rope_yarn :535-590, Q8Mat :464-494, dot_q8_i8
// :169-191, qblock32 :691-699, rmsnorm_quant_par :730-738.
//
// Kernels per token and layer:
//   k_attn_norm  rmsnorm (16-lane sum of squares) + Q8 per 32 of x;
//   k_attn_qkv   q / k / v rows: the reference's Q8 dot (8 fp32 chains per
//                row, one lane each), bias, RoPE from the table, cache write;
//   k_attn_core  per q-head: scores over the window, softmax with the sink,
//                weighted sum of v, Q8 of the head's 64 outputs;
//   k_attn_oproj x[r] += wo[r] . ao + bo[r].
// The projections, RoPE and the cache rows are the reference's operations in
// its order (bit for bit given the same RoPE table, which the host computes
// once with the reference's formula); the softmax goes through expf and a
// fixed-order tree sum, so its outputs match to tolerance.
//
// Q8 weights are re-laid out at load time into tiles of 8 rows: per (tile,
// 32-block) 8 rows x 32 int8 (256 B) and 8 fp32 scales, so a wavefront (8
// rows x 8 chains) reads 512 contiguous bytes per step.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <vector>

#include "cpb_attn.h"
#include "cpb_internal.h"
#include "moe_common.h"
#include "route_dev.h"

namespace cpb {

constexpr int kAttnHd = 64;

struct AttnLayerDev {
    const int8_t *wq, *wk, *wv, *wo;    // Q8 tile streams
    const float *sq, *sk, *sv, *so;     // scales [tile][block][8]
    const float *bq, *bk, *bv, *bo, *sinks, *norm;
};

struct AttnArgs {
    int d, nh, nkv, nb, nbo, pos, start, max_seq;
    float eps;
    AttnLayerDev L;
    float* x;            // [d] residual (in place)
    float* kc;           // this layer's cache [max_seq][nkv][64]
    float* vc;
    const float* rope;   // [max_seq][32][2]
    int8_t* xq;          // [d]
    float* xsb;          // [d/32]
    float* q;            // [nh*64]
    float* ao;           // [nh*64]
    int8_t* aq;          // [nh*64]
    float* asb;          // [nh*64/32]
};

// ---- load time: Q8Mat::from_bf16 into the 8-row tile stream ----
__global__ void k_q8_tiles(const uint16_t* __restrict__ w, int rows, int cols, int8_t* __restrict__ q,
                           float* __restrict__ s) {
    const int nb = cols / 32;
    const size_t total = (size_t)rows * nb;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        const int row = (int)(idx / nb), b = (int)(idx % nb);
        float vals[32], amax = 1e-12f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            vals[i] = __uint_as_float((uint32_t)w[(size_t)row * cols + b * 32 + i] << 16);
            amax = fmaxf(amax, fabsf(vals[i]));
        }
        const float sc = amax / 127.0f;
        const size_t tb = (size_t)(row / 8) * nb + b;
        s[tb * 8 + row % 8] = sc;
        uint32_t wd[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            float r = roundf(vals[i] / sc);
            r = r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
            wd[i >> 2] |= (uint32_t)(uint8_t)(int8_t)r << (8 * (i & 3));
        }
        uint32_t* dst = (uint32_t*)(q + tb * 256 + (row % 8) * 32);
#pragma unroll
        for (int k = 0; k < 8; k++) dst[k] = wd[k];
    }
}

// dot_q8_i8 (:169-191) of tile row r (lane >> 3) against activations xl / sl
// (LDS): lane chain c = lane & 7 -> accumulator h = c >> 2 (even / odd
// blocks, an odd last block into the first), lane part j = c & 3; returns
// the row's value in every lane of its group of 8.
CPB_DEV float q8_tile_dot(const int8_t* __restrict__ w, const float* __restrict__ s, int tile, int nb,
                          const uint32_t* xl, const float* sl) {
    const int lane = threadIdx.x & 63, r = lane >> 3, h = (lane >> 2) & 1, j = lane & 3;
    const int8_t* wt = w + (size_t)tile * nb * 256 + r * 32 + 4 * j;
    const float* st = s + (size_t)tile * nb * 8 + r;
    const int nbe = nb & ~1;
    float acc = 0.0f;
#pragma unroll 4
    for (int b = h; b < nbe; b += 2) {
        const uint32_t w0 = *(const uint32_t*)(wt + (size_t)b * 256), w1 = *(const uint32_t*)(wt + (size_t)b * 256 + 16);
        const int t = sdot4(w1, xl[b * 8 + 4 + j], sdot4(w0, xl[b * 8 + j], 0));
        acc = fmaf((float)t, st[(size_t)b * 8] * sl[b], acc);
    }
    if ((nb & 1) && h == 0) {
        const int b = nb - 1;
        const uint32_t w0 = *(const uint32_t*)(wt + (size_t)b * 256), w1 = *(const uint32_t*)(wt + (size_t)b * 256 + 16);
        const int t = sdot4(w1, xl[b * 8 + 4 + j], sdot4(w0, xl[b * 8 + j], 0));
        acc = fmaf((float)t, st[(size_t)b * 8] * sl[b], acc);
    }
    const float v = acc + __shfl_xor(acc, 4);            // v_j = acc0_j + acc1_j
    const float v01 = v + __shfl_xor(v, 1);              // j = 0, 1: v0 + v1; j = 2, 3: v2 + v3
    const int g = lane & ~7;
    return __shfl(v01, g) + __shfl(v01, g + 2);
}

// activations (xq as dwords, scales) into LDS
CPB_DEV void stage_act(const int8_t* xq, const float* xsb, int nb, uint32_t* xl, float* sl) {
    for (int i = threadIdx.x; i < nb * 8; i += blockDim.x) xl[i] = ((const uint32_t*)xq)[i];
    for (int i = threadIdx.x; i < nb; i += blockDim.x) sl[i] = xsb[i];
    __syncthreads();
}

// ---- rmsnorm + Q8 of x ----
__global__ __launch_bounds__(256) void k_attn_norm(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* xs = (float*)smem;
    float* xnl = xs + a.d;
    float* scratch = xnl + a.d;
    norm_into(a.x, a.L.norm, a.d, a.eps, 0, 0, 1, xs, xnl, scratch);
    const int l = threadIdx.x & 31;
    for (int bk = threadIdx.x >> 5; bk < a.nb; bk += blockDim.x >> 5) {
        const float v = xnl[bk * 32 + l];
        float m = fabsf(v);
#pragma unroll
        for (int s2 = 16; s2 >= 1; s2 >>= 1) m = fmaxf(m, __shfl_xor(m, s2));
        const float sc = fmaxf(1e-12f, m) / 127.0f;
        a.xq[bk * 32 + l] = (int8_t)q8_round(v, sc);
        if (l == 0) a.xsb[bk] = sc;
    }
}

// ---- q / k / v rows + bias + RoPE + cache ----
// one wavefront per 8 rows {i, 32 + i} (i in [4g, 4g + 4)) of one head, so
// each RoPE pair is in the wave; grid: (nh + 2 nkv) * 8.
__global__ __launch_bounds__(64) void k_attn_qkv(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint32_t* xl = (uint32_t*)smem;
    float* sl = (float*)(xl + a.nb * 8);
    __shared__ float hv[8];
    stage_act(a.xq, a.xsb, a.nb, xl, sl);
    const int head = blockIdx.x >> 3, g = blockIdx.x & 7;
    const int lane = threadIdx.x, r = lane >> 3;                 // tile row r: head row i or 32 + i
    const int hrow = (r < 4 ? 4 * g + r : 32 + 4 * g + (r - 4));
    int kind, hh;                                                // 0 q, 1 k, 2 v
    if (head < a.nh) { kind = 0; hh = head; }
    else if (head < a.nh + a.nkv) { kind = 1; hh = head - a.nh; }
    else { kind = 2; hh = head - a.nh - a.nkv; }
    const int8_t* W = kind == 0 ? a.L.wq : kind == 1 ? a.L.wk : a.L.wv;
    const float* S = kind == 0 ? a.L.sq : kind == 1 ? a.L.sk : a.L.sv;
    const float* B = kind == 0 ? a.L.bq : kind == 1 ? a.L.bk : a.L.bv;
    const int row = hh * kAttnHd + hrow;
    // the 8 lanes of tile row r read head row `row` from its own 8-row tile
    const int tile = row >> 3, tr = row & 7;
    float v;
    {
        const int h = (lane >> 2) & 1, j = lane & 3;
        const int8_t* wt = W + (size_t)tile * a.nb * 256 + tr * 32 + 4 * j;
        const float* st = S + (size_t)tile * a.nb * 8 + tr;
        const int nb = a.nb, nbe = nb & ~1;
        float acc = 0.0f;
#pragma unroll 4
        for (int b = h; b < nbe; b += 2) {
            const uint32_t w0 = *(const uint32_t*)(wt + (size_t)b * 256), w1 = *(const uint32_t*)(wt + (size_t)b * 256 + 16);
            const int t = sdot4(w1, xl[b * 8 + 4 + j], sdot4(w0, xl[b * 8 + j], 0));
            acc = fmaf((float)t, st[(size_t)b * 8] * sl[b], acc);
        }
        if ((nb & 1) && h == 0) {
            const int b = nb - 1;
            const uint32_t w0 = *(const uint32_t*)(wt + (size_t)b * 256), w1 = *(const uint32_t*)(wt + (size_t)b * 256 + 16);
            const int t = sdot4(w1, xl[b * 8 + 4 + j], sdot4(w0, xl[b * 8 + j], 0));
            acc = fmaf((float)t, st[(size_t)b * 8] * sl[b], acc);
        }
        const float vv = acc + __shfl_xor(acc, 4);
        const float v01 = vv + __shfl_xor(vv, 1);
        const int gl = lane & ~7;
        v = __shfl(v01, gl) + __shfl(v01, gl + 2);
    }
    v = v + B[row];                                          // :786-793 dot + bias
    if ((lane & 7) == 0) hv[r] = v;
    __syncthreads();
    if (lane >= 4) return;
    // RoPE pair (i, 32 + i), i = 4g + lane (rope_yarn :578-590); v unrotated
    const int i = 4 * g + lane;
    float lo = hv[lane], hi = hv[4 + lane];
    if (kind != 2) {
        const float c = a.rope[((size_t)a.pos * 32 + i) * 2], s = a.rope[((size_t)a.pos * 32 + i) * 2 + 1];
        const float nlo = lo * c - hi * s, nhi = hi * c + lo * s;
        lo = nlo;
        hi = nhi;
    }
    if (kind == 0) {
        a.q[hh * kAttnHd + i] = lo;
        a.q[hh * kAttnHd + 32 + i] = hi;
    } else {
        float* dst = (kind == 1 ? a.kc : a.vc) + ((size_t)a.pos * a.nkv + hh) * kAttnHd;
        dst[i] = lo;
        dst[32 + i] = hi;
    }
}

// ---- per q-head: scores, softmax with the sink, weighted v, Q8 ----
__global__ __launch_bounds__(256) void k_attn_core(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* sc = (float*)smem;                                    // [n]
    __shared__ float qs[kAttnHd];
    __shared__ float red[256];
    __shared__ float part[4][kAttnHd];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int kvh = h / (a.nh / a.nkv);
    const int n = a.pos - a.start + 1;
    if (tid < kAttnHd) qs[tid] = a.q[h * kAttnHd + tid];
    __syncthreads();
    // scores (:810-820): lane-parallel fmas in 4 x 4 accumulators over steps of 16
    for (int t = tid; t < n; t += blockDim.x) {
        const float4* kp = (const float4*)(a.kc + ((size_t)(a.start + t) * a.nkv + kvh) * kAttnHd);
        float acc[4][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const float4 kv = kp[jj * 4 + m];
                const float* qv = qs + jj * 16 + 4 * m;
                acc[m][0] = fmaf(kv.x, qv[0], acc[m][0]);
                acc[m][1] = fmaf(kv.y, qv[1], acc[m][1]);
                acc[m][2] = fmaf(kv.z, qv[2], acc[m][2]);
                acc[m][3] = fmaf(kv.w, qv[3], acc[m][3]);
            }
        float s4[4];
#pragma unroll
        for (int l = 0; l < 4; l++) s4[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
        sc[t] = ((s4[0] + s4[1]) + (s4[2] + s4[3])) * 0.125f;   // 1 / sqrt(64)
    }
    __syncthreads();
    // max over the sink and the scores
    const float sink = a.L.sinks[h];
    float m = sink;
    for (int t = tid; t < n; t += blockDim.x) m = fmaxf(m, sc[t]);
    red[tid] = m;
    __syncthreads();
    for (int s2 = 128; s2 >= 1; s2 >>= 1) {
        if (tid < s2) red[tid] = fmaxf(red[tid], red[tid + s2]);
        __syncthreads();
    }
    const float mx = red[0];
    __syncthreads();
    // weights and their sum (fixed-order tree), sink term first
    float ps = 0.0f;
    for (int t = tid; t < n; t += blockDim.x) {
        const float e = expf(sc[t] - mx);
        sc[t] = e;
        ps += e;
    }
    red[tid] = ps;
    __syncthreads();
    for (int s2 = 128; s2 >= 1; s2 >>= 1) {
        if (tid < s2) red[tid] += red[tid + s2];
        __syncthreads();
    }
    const float den = expf(sink - mx) + red[0];
    // ao[u] = sum_t e_t v_t[u] / den: 4 position groups per dimension
    const int u = tid & 63, grp = tid >> 6;
    float acc = 0.0f;
    for (int t = grp; t < n; t += 4) acc = fmaf(a.vc[((size_t)(a.start + t) * a.nkv + kvh) * kAttnHd + u], sc[t], acc);
    part[grp][u] = acc;
    __syncthreads();
    if (tid >= 64) return;
    const float o = ((part[0][u] + part[1][u]) + (part[2][u] + part[3][u])) * (1.0f / den);
    a.ao[h * kAttnHd + u] = o;
    // qblock32 (:691-699) of the head's two blocks
    float mb = fabsf(o);
#pragma unroll
    for (int s2 = 16; s2 >= 1; s2 >>= 1) mb = fmaxf(mb, __shfl_xor(mb, s2));
    const float scq = fmaxf(1e-12f, mb) / 127.0f;
    a.aq[h * kAttnHd + u] = (int8_t)q8_round(o, scq);
    if ((u & 31) == 0) a.asb[h * 2 + (u >> 5)] = scq;
}

// ---- x[r] += wo[r] . ao + bo[r] (:837) ----
__global__ __launch_bounds__(64) void k_attn_oproj(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint32_t* xl = (uint32_t*)smem;
    float* sl = (float*)(xl + a.nbo * 8);
    stage_act(a.aq, a.asb, a.nbo, xl, sl);
    const int tile = blockIdx.x;
    const float v = q8_tile_dot(a.L.wo, a.L.so, tile, a.nbo, xl, sl);
    const int lane = threadIdx.x;
    if ((lane & 7) == 0) {
        const int row = tile * 8 + (lane >> 3);
        a.x[row] += v + a.L.bo[row];
    }
}

}  // namespace cpb

using cpb::fail;

struct cpb_attn {
    cpb_attn_cfg cfg{};
    int device = 0;
    hipStream_t own = nullptr, stream = nullptr;
    std::vector<cpb::AttnLayerDev> layers;
    std::vector<void*> layer_mem;
    std::vector<bool> loaded;
    float *kc = nullptr, *vc = nullptr, *rope = nullptr, *x = nullptr;
    int8_t *xq = nullptr, *aq = nullptr;
    float *xsb = nullptr, *q = nullptr, *ao = nullptr, *asb = nullptr;
};

#define HIP_OK_A(expr)                                                                  \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return fail(e_ == hipErrorOutOfMemory ? CPB_ENOMEM : CPB_ENODEV, "%s: %s", #expr, \
                        hipGetErrorString(e_));                                          \
    } while (0)

namespace {

int attn_check(const cpb_attn_cfg* c) {
    if (!c) return fail(CPB_EINVAL, "cfg is NULL");
    if (c->head_dim != 64) return fail(CPB_EINVAL, "head_dim=%d: the kernels take 64 (as the reference's)", c->head_dim);
    if (c->d <= 0 || c->d % 32 || c->d > 4096) return fail(CPB_EINVAL, "d=%d must be a multiple of 32, <= 4096", c->d);
    if (c->n_head <= 0 || c->n_head_kv <= 0 || c->n_head % c->n_head_kv)
        return fail(CPB_EINVAL, "n_head=%d must be a positive multiple of n_head_kv=%d", c->n_head, c->n_head_kv);
    if (c->n_layer <= 0 || c->max_seq <= 0 || c->max_seq > 8192) return fail(CPB_EINVAL, "bad n_layer / max_seq (<= 8192)");
    if (c->sliding_window < 1) return fail(CPB_EINVAL, "sliding_window must be >= 1");
    return 0;
}

// rope_init / rope_yarn_slow (:535-576): (cos, sin) * mscale per (pos, i),
// computed once on the host with the reference's fp32 expressions.
void rope_table(int hd, int max_seq, float base, std::vector<float>& tab) {
    const int half = hd / 2;
    tab.assign((size_t)max_seq * half * 2, 0.0f);
    const float PI = 3.14159265358979323846f;
    volatile float b32 = 32.0f, b1 = 1.0f;
    const float fd32 = (float)hd * logf(4096.0f / (b32 * 2.0f * PI)) / (2.0f * logf(base));
    const float fd1 = (float)hd * logf(4096.0f / (b1 * 2.0f * PI)) / (2.0f * logf(base));
    const float low = fmaxf(floorf(fd32), 0.0f);
    const float high = fminf(ceilf(fd1), (float)hd - 1.0f);
    const float mscale = 1.0f + 0.1f * logf(32.0f);
    for (int pos = 0; pos < max_seq; pos++)
        for (int i = 0; i < half; i++) {
            const float theta_ex = (float)pos * powf(base, -(2.0f * (float)i) / (float)hd);
            const float theta_in = theta_ex / 32.0f;
            const float y = ((float)i - low) / fmaxf(high - low, 0.001f);
            const float yc = y < 0.0f ? 0.0f : y > 1.0f ? 1.0f : y;
            const float mix = 1.0f - yc;
            const float theta = theta_in * (1.0f - mix) + theta_ex * mix;
            const float c = cosf(theta) * mscale, s = sinf(theta) * mscale;
            tab[((size_t)pos * half + i) * 2] = 1.0f * c - 0.0f * s;
            tab[((size_t)pos * half + i) * 2 + 1] = 0.0f * c + 1.0f * s;
        }
}

}  // namespace

extern "C" {

void cpb_attn_destroy(cpb_attn_t* h) {
    if (!h) return;
    hipSetDevice(h->device);
    if (h->stream) hipStreamSynchronize(h->stream);
    for (void* p : h->layer_mem)
        if (p) hipFree(p);
    void* bufs[] = {h->kc, h->vc, h->rope, h->x, h->xq, h->aq, h->xsb, h->q, h->ao, h->asb};
    for (void* p : bufs)
        if (p) hipFree(p);
    if (h->own) hipStreamDestroy(h->own);
    delete h;
}

int cpb_attn_create(const cpb_attn_cfg* cfg, int device, cpb_attn_t** out) {
    if (!out) return fail(CPB_EINVAL, "out is NULL");
    *out = nullptr;
    if (int r = attn_check(cfg)) return r;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return fail(CPB_ENODEV, "no HIP device");
    if (device < 0 || device >= ndev) return fail(CPB_EINVAL, "device %d out of range", device);
    HIP_OK_A(hipSetDevice(device));
    cpb_attn_t* h = new cpb_attn_t();
    h->cfg = *cfg;
    h->device = device;
    h->layers.resize(cfg->n_layer);
    h->layer_mem.assign(cfg->n_layer, nullptr);
    h->loaded.assign(cfg->n_layer, false);
    auto bail = [&](int r) { cpb_attn_destroy(h); return r; };
    if (hipStreamCreateWithFlags(&h->own, hipStreamNonBlocking) != hipSuccess) return bail(fail(CPB_ENODEV, "stream create failed"));
    h->stream = h->own;
    const size_t d = cfg->d, nq = (size_t)cfg->n_head * 64, nkv = (size_t)cfg->n_head_kv * 64;
    const size_t cache = (size_t)cfg->n_layer * cfg->max_seq * nkv * sizeof(float);
    auto dm = [&](void** p, size_t n) -> int {
        hipError_t e = hipMalloc(p, n ? n : 1);
        return e == hipSuccess ? 0 : fail(CPB_ENOMEM, "hipMalloc(%zu): %s", n, hipGetErrorString(e));
    };
    int r;
    if ((r = dm((void**)&h->kc, cache)) || (r = dm((void**)&h->vc, cache)) ||
        (r = dm((void**)&h->rope, (size_t)cfg->max_seq * 64 * 4)) || (r = dm((void**)&h->x, d * 4)) ||
        (r = dm((void**)&h->xq, d)) || (r = dm((void**)&h->xsb, d / 32 * 4)) || (r = dm((void**)&h->q, nq * 4)) ||
        (r = dm((void**)&h->ao, nq * 4)) || (r = dm((void**)&h->aq, nq)) || (r = dm((void**)&h->asb, nq / 32 * 4)))
        return bail(r);
    std::vector<float> tab;
    rope_table(64, cfg->max_seq, cfg->rope_base, tab);
    if (hipMemcpy(h->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemsetAsync(h->kc, 0, cache, h->stream) != hipSuccess || hipMemsetAsync(h->vc, 0, cache, h->stream) != hipSuccess ||
        hipStreamSynchronize(h->stream) != hipSuccess)
        return bail(fail(CPB_ENODEV, "attention init copies failed"));
    *out = h;
    return 0;
}

int cpb_attn_load_layer(cpb_attn_t* h, int layer, const float* attn_norm, const uint16_t* wq, const uint16_t* wk,
                        const uint16_t* wv, const uint16_t* wo, const float* bq, const float* bk, const float* bv,
                        const float* bo, const float* sinks) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    const auto& c = h->cfg;
    if (layer < 0 || layer >= c.n_layer) return fail(CPB_EINVAL, "layer %d out of range", layer);
    if (!attn_norm || !wq || !wk || !wv || !wo || !bq || !bk || !bv || !bo || !sinks)
        return fail(CPB_EINVAL, "NULL tensor");
    HIP_OK_A(hipSetDevice(h->device));
    HIP_OK_A(hipStreamSynchronize(h->stream));
    if (h->layer_mem[layer]) { hipFree(h->layer_mem[layer]); h->layer_mem[layer] = nullptr; h->loaded[layer] = false; }
    const size_t d = c.d, nq = (size_t)c.n_head * 64, nkv = (size_t)c.n_head_kv * 64;
    // one allocation: four Q8 streams + scales, then the fp32 vectors
    const size_t mats[4][2] = {{nq, d}, {nkv, d}, {nkv, d}, {d, nq}};
    size_t off[4][2], o = 0;
    for (int m = 0; m < 4; m++) {
        off[m][0] = o; o += (mats[m][0] * mats[m][1] + 255) / 256 * 256;
        off[m][1] = o; o += (mats[m][0] * (mats[m][1] / 32) * 4 + 255) / 256 * 256;
    }
    const size_t vec[6] = {d, nq, nkv, nkv, d, (size_t)c.n_head};      // norm, bq, bk, bv, bo, sinks
    size_t voff[6];
    for (int k = 0; k < 6; k++) { voff[k] = o; o += (vec[k] * 4 + 255) / 256 * 256; }
    unsigned char* base = nullptr;
    HIP_OK_A(hipMalloc((void**)&base, o));
    h->layer_mem[layer] = base;
    const uint16_t* srcs[4] = {wq, wk, wv, wo};
    uint16_t* staging = nullptr;
    hipError_t e = hipMalloc((void**)&staging, nq * d * 2 > d * nq * 2 ? nq * d * 2 : d * nq * 2);
    for (int m = 0; m < 4 && e == hipSuccess; m++) {
        const size_t n = mats[m][0] * mats[m][1];
        e = hipMemcpyAsync(staging, srcs[m], n * 2, hipMemcpyHostToDevice, h->stream);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(cpb::k_q8_tiles, dim3(4096), dim3(256), 0, h->stream, staging, (int)mats[m][0],
                               (int)mats[m][1], (int8_t*)(base + off[m][0]), (float*)(base + off[m][1]));
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    }
    if (staging) hipFree(staging);
    const float* vsrc[6] = {attn_norm, bq, bk, bv, bo, sinks};
    for (int k = 0; k < 6 && e == hipSuccess; k++) e = hipMemcpy(base + voff[k], vsrc[k], vec[k] * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(CPB_ENODEV, "attention layer load: %s", hipGetErrorString(e));
    cpb::AttnLayerDev& L = h->layers[layer];
    L.wq = (const int8_t*)(base + off[0][0]); L.sq = (const float*)(base + off[0][1]);
    L.wk = (const int8_t*)(base + off[1][0]); L.sk = (const float*)(base + off[1][1]);
    L.wv = (const int8_t*)(base + off[2][0]); L.sv = (const float*)(base + off[2][1]);
    L.wo = (const int8_t*)(base + off[3][0]); L.so = (const float*)(base + off[3][1]);
    L.norm = (const float*)(base + voff[0]); L.bq = (const float*)(base + voff[1]);
    L.bk = (const float*)(base + voff[2]); L.bv = (const float*)(base + voff[3]);
    L.bo = (const float*)(base + voff[4]); L.sinks = (const float*)(base + voff[5]);
    h->loaded[layer] = true;
    return 0;
}

static int attn_launch(cpb_attn_t* h, int layer, int pos, float* dx) {
    const auto& c = h->cfg;
    cpb::AttnArgs a{};
    a.d = c.d; a.nh = c.n_head; a.nkv = c.n_head_kv; a.nb = c.d / 32; a.nbo = c.n_head * 64 / 32;
    a.pos = pos; a.max_seq = c.max_seq; a.eps = c.rms_eps;
    // :797 sliding window on layers 0, 2, ... ((il + 1) % 2 != 0)
    a.start = ((layer + 1) % 2 != 0) ? (pos - (c.sliding_window - 1) > 0 ? pos - (c.sliding_window - 1) : 0) : 0;
    a.L = h->layers[layer];
    a.x = dx;
    const size_t lc = (size_t)c.max_seq * c.n_head_kv * 64;
    a.kc = h->kc + (size_t)layer * lc;
    a.vc = h->vc + (size_t)layer * lc;
    a.rope = h->rope;
    a.xq = h->xq; a.xsb = h->xsb; a.q = h->q; a.ao = h->ao; a.aq = h->aq; a.asb = h->asb;
    cpb::launch(cpb::k_attn_norm, dim3(1), dim3(256), sizeof(float) * (2 * c.d + 64), h->stream, a);
    cpb::launch(cpb::k_attn_qkv, dim3((c.n_head + 2 * c.n_head_kv) * 8), dim3(64), (size_t)a.nb * 36, h->stream, a);
    cpb::launch(cpb::k_attn_core, dim3(c.n_head), dim3(256), (size_t)(pos - a.start + 1) * 4, h->stream, a);
    cpb::launch(cpb::k_attn_oproj, dim3(c.d / 8), dim3(64), (size_t)a.nbo * 36, h->stream, a);
    return hipGetLastError() == hipSuccess ? 0 : fail(CPB_ENODEV, "attention launch failed");
}

int cpb_attn_forward_device(cpb_attn_t* h, int layer, int pos, float* d_x) {
    if (!h || !d_x) return fail(CPB_EINVAL, "NULL argument");
    if (layer < 0 || layer >= h->cfg.n_layer || !h->loaded[layer]) return fail(CPB_ESTATE, "layer %d not loaded", layer);
    if (pos < 0 || pos >= h->cfg.max_seq) return fail(CPB_EINVAL, "pos %d outside [0, max_seq=%d)", pos, h->cfg.max_seq);
    HIP_OK_A(hipSetDevice(h->device));
    return attn_launch(h, layer, pos, d_x);
}

int cpb_attn_forward(cpb_attn_t* h, int layer, int pos, float* x, cpb_attn_trace* tr) {
    if (!h || !x) return fail(CPB_EINVAL, "NULL argument");
    if (layer < 0 || layer >= h->cfg.n_layer || !h->loaded[layer]) return fail(CPB_ESTATE, "layer %d not loaded", layer);
    if (pos < 0 || pos >= h->cfg.max_seq) return fail(CPB_EINVAL, "pos %d outside [0, max_seq=%d)", pos, h->cfg.max_seq);
    HIP_OK_A(hipSetDevice(h->device));
    const auto& c = h->cfg;
    HIP_OK_A(hipMemcpyAsync(h->x, x, (size_t)c.d * 4, hipMemcpyHostToDevice, h->stream));
    if (int r = attn_launch(h, layer, pos, h->x)) return r;
    HIP_OK_A(hipMemcpyAsync(x, h->x, (size_t)c.d * 4, hipMemcpyDeviceToHost, h->stream));
    if (tr) {
        const size_t nq = (size_t)c.n_head * 64, nkv = (size_t)c.n_head_kv * 64;
        const size_t lc = (size_t)c.max_seq * nkv;
        auto cp = [&](void* dst, const void* src, size_t n) -> int {
            if (dst) HIP_OK_A(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, h->stream));
            return 0;
        };
        int r = 0;
        r |= cp(tr->xq, h->xq, c.d);
        r |= cp(tr->xsb, h->xsb, c.d / 32 * 4);
        r |= cp(tr->q, h->q, nq * 4);
        r |= cp(tr->k, h->kc + (size_t)layer * lc + (size_t)pos * nkv, nkv * 4);
        r |= cp(tr->v, h->vc + (size_t)layer * lc + (size_t)pos * nkv, nkv * 4);
        r |= cp(tr->ao, h->ao, nq * 4);
        r |= cp(tr->aq, h->aq, nq);
        r |= cp(tr->asb, h->asb, nq / 32 * 4);
        if (r) return r;
    }
    HIP_OK_A(hipStreamSynchronize(h->stream));
    return 0;
}

int cpb_attn_reset(cpb_attn_t* h) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    HIP_OK_A(hipSetDevice(h->device));
    const size_t cache = (size_t)h->cfg.n_layer * h->cfg.max_seq * h->cfg.n_head_kv * 64 * sizeof(float);
    HIP_OK_A(hipMemsetAsync(h->kc, 0, cache, h->stream));
    HIP_OK_A(hipMemsetAsync(h->vc, 0, cache, h->stream));
    return 0;
}

int cpb_attn_set_stream(cpb_attn_t* h, void* stream) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    hipStream_t ns = stream ? (hipStream_t)stream : h->own;
    if (ns == h->stream) return 0;
    HIP_OK_A(hipSetDevice(h->device));
    HIP_OK_A(hipStreamSynchronize(h->stream));
    h->stream = ns;
    return 0;
}

int cpb_attn_sync(cpb_attn_t* h) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    HIP_OK_A(hipStreamSynchronize(h->stream));
    return 0;
}

}  // extern "C"
