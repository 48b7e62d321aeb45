// head.hip -- two-stage LM head (Q4 screen, exact Q8 refine, greedy) on gfx950.
//
// Reference (src/bin/): head_worker engine_gpt2.rs:937-1002; Q4Mat and its
// scale search :237-300; dot4_q4_i8 :314-342; Q8Mat :464-494; dot_q8_i8
// :169-191; rmsnorm_quant_par :730-738; sample_cands (greedy) :128-134.
//
// Every float operation is the reference's, in its order, so the screen
// values, the candidate set and the Q8 logits are the reference's bit for
// bit (the integer dot products are exact; the fp32 chains are per-lane
// fmas exactly as its NEON lanes).
//
// HBM layout of the Q4 screen stream (built at load time from the bf16
// weights): rows in tiles of 64, per (tile, 32-block) 64 lanes x 16 nibble
// bytes (1 KB, one wavefront load) and 64 x bf16 scales; the Q8 rows stay
// row-major (only the few candidate rows are read).  The screen is a
// bandwidth-bound GEMV over 4.5 bits per weight (~326 MB for gpt-oss's
// 201088 x 2880 head), one lane per row.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdio>
#include <mutex>

#include "cpb_head.h"
#include "cpb_internal.h"
#include "moe_common.h"
#include "route_dev.h"

namespace cpb {

constexpr int kHeadRT = 64;          // rows per stream tile
constexpr int kHeadMaxCand = 16;

CPB_DEV float bf16f(uint32_t v) { return __uint_as_float(v << 16); }
// engine_gpt2.rs:303-307: round to nearest even into the top 16 bits
CPB_DEV uint32_t f32_to_bf16(float v) {
    const uint32_t b = __float_as_uint(v);
    return ((b + 0x7fffu + ((b >> 16) & 1u)) >> 16) & 0xffffu;
}

struct HeadDev {
    int d, nb, V, Vpad, nt, nc;
    float eps;
    const u32x4* q4;       // [Vpad/64][nb][64] nibble units
    const uint16_t* q4s;   // [Vpad/64][nb][64] bf16 scales
    const int8_t* q8;      // [V][d]
    const float* q8s;      // [V][nb]
    const float* norm_w;   // [d]
    const float* x;        // [d]
    int8_t* xq;            // [d]
    float* xsb;            // [nb]
    int32_t* xs8;          // [nb][4] sums of x over each lane part (for the -8 of the codes)
    float* screen;         // [Vpad]
    int32_t* cand_ids;     // [nt*nc]
    float* cand_screen;
    float* cand_logits;
    int32_t* chosen;       // [1]
};

// ---- load time: Q4Mat + Q8Mat rows from bf16, one thread per (row, block) ----
__global__ void k_head_quant(const uint16_t* __restrict__ w, int V, int Vpad, int d, u32x4* __restrict__ q4,
                             uint16_t* __restrict__ q4s, int8_t* __restrict__ q8, float* __restrict__ q8s) {
    const int nb = d / 32;
    const size_t total = (size_t)Vpad * nb;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        const int row = (int)(idx / nb), b = (int)(idx % nb);
        float vals[32];
#pragma unroll
        for (int i = 0; i < 32; i++) vals[i] = row < V ? bf16f(w[(size_t)row * d + b * 32 + i]) : 0.0f;
        // q4_scale_search (:274-300)
        float amax = 0.0f, vmax = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(vals[i]) > amax) { amax = fabsf(vals[i]); vmax = vals[i]; }
        uint32_t best_db = 0;
        float idq = 0.0f;
        if (amax != 0.0f) {
            float best_err = FLT_MAX;
            for (int t = 0; t < 17; t++) {
                const float nmax = 7.0f + (float)t * 0.0625f;
                const uint32_t db = f32_to_bf16(vmax / -nmax);
                const float dd = bf16f(db);
                if (dd == 0.0f) continue;
                const float id = 1.0f / dd;
                float err = 0.0f;
                for (int i = 0; i < 32; i++) {
                    int c = (int)floorf(vals[i] * id + 8.5f);
                    c = c < 0 ? 0 : c > 15 ? 15 : c;
                    const float e = vals[i] - (float)(c - 8) * dd;
                    err += e * e;
                }
                if (err < best_err) { best_err = err; best_db = db; }
            }
            const float dd = bf16f(best_db);
            idq = dd != 0.0f ? 1.0f / dd : 0.0f;
        }
        uint32_t wd[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            int lo = (int)floorf(vals[j] * idq + 8.5f), hi = (int)floorf(vals[j + 16] * idq + 8.5f);
            lo = lo < 0 ? 0 : lo > 15 ? 15 : lo;
            hi = hi < 0 ? 0 : hi > 15 ? 15 : hi;
            wd[j >> 2] |= (uint32_t)(lo | (hi << 4)) << (8 * (j & 3));
        }
        const size_t u = ((size_t)(row / kHeadRT) * nb + b) * kHeadRT + row % kHeadRT;
        q4[u] = u32x4{wd[0], wd[1], wd[2], wd[3]};
        q4s[u] = (uint16_t)best_db;
        if (row >= V) continue;
        // Q8Mat (:476-489): amax seeded 1e-12, round half away from zero
        float a8 = 1e-12f;
        for (int i = 0; i < 32; i++) a8 = fmaxf(a8, fabsf(vals[i]));
        const float sc = a8 / 127.0f;
        q8s[(size_t)row * nb + b] = sc;
        for (int i = 0; i < 32; i++) {
            float r = roundf(vals[i] / sc);
            r = r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
            q8[(size_t)row * d + b * 32 + i] = (int8_t)r;
        }
    }
}

// ---- rmsnorm (16-lane sum of squares) + Q8 per 32 of the hidden state ----
__global__ __launch_bounds__(256) void k_head_norm(HeadDev a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int d = a.d, tid = threadIdx.x;
    float* xs = (float*)smem;
    float* xnl = xs + d;
    float* scratch = xnl + d;
    norm_into(a.x, a.norm_w, d, a.eps, 0, 0, 1, xs, xnl, scratch);
    const int l = tid & 31;
    for (int bk = tid >> 5; bk < a.nb; bk += blockDim.x >> 5) {
        const float v = xnl[bk * 32 + l];
        float m = fabsf(v);
#pragma unroll
        for (int s2 = 16; s2 >= 1; s2 >>= 1) m = fmaxf(m, __shfl_xor(m, s2));
        const float sc = fmaxf(1e-12f, m) / 127.0f;
        const int q = q8_round(v, sc);
        a.xq[bk * 32 + l] = (int8_t)q;
        if (l == 0) a.xsb[bk] = sc;
        // lane part j of the screen dot = elements 4j..4j+3 and 16+4j..16+4j+3
        int s = q;
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 16);
        if (l < 16 && (l & 3) == 0) a.xs8[bk * 4 + (l >> 2)] = s;
    }
}

// ---- Q4 screen of every row (dot4_q4_i8, :314-342): one lane per row ----
__global__ __launch_bounds__(256) void k_head_screen(HeadDev a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nb = a.nb, tid = threadIdx.x, lane = tid & 63;
    uint32_t* xl = (uint32_t*)smem;                    // xq as dwords [nb][8]
    float* xsl = (float*)(xl + nb * 8);                // [nb]
    int32_t* x8 = (int32_t*)(xsl + nb);                // [nb][4]
    for (int i = tid; i < nb * 8; i += blockDim.x) xl[i] = ((const uint32_t*)a.xq)[i];
    for (int i = tid; i < nb; i += blockDim.x) xsl[i] = a.xsb[i];
    for (int i = tid; i < nb * 4; i += blockDim.x) x8[i] = a.xs8[i];
    __syncthreads();
    const int tile = blockIdx.x * (blockDim.x >> 6) + (tid >> 6);
    if (tile * kHeadRT >= a.Vpad) return;
    const u32x4* wp = a.q4 + (size_t)tile * nb * kHeadRT + lane;
    const uint16_t* sp = a.q4s + (size_t)tile * nb * kHeadRT + lane;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 6
    for (int b = 0; b < nb; b++) {
        const u32x4 w = __builtin_nontemporal_load(wp + (size_t)b * kHeadRT);
        const float sv = bf16f(sp[(size_t)b * kHeadRT]) * xsl[b];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int t = sdot4(w[j] & 0x0F0F0F0Fu, xl[b * 8 + j], 0);
            t = sdot4((w[j] >> 4) & 0x0F0F0F0Fu, xl[b * 8 + 4 + j], t);
            t -= 8 * x8[b * 4 + j];                    // codes are KVI4[c] = c - 8
            acc[j] = fmaf((float)t, sv, acc[j]);
        }
    }
    a.screen[tile * kHeadRT + lane] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// (value, index) order of the screen: larger value first, then lower index
CPB_DEV bool better(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

// ---- per worker slice: the n_cand best rows (the reference's insertion) ----
// grid: n_slices workgroups of 1024 threads.
__global__ __launch_bounds__(1024) void k_head_topk(HeadDev a) {
    __shared__ float wv[16];
    __shared__ int wi[16], wt[16];
    __shared__ int win_tid;
    const int wid = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv_id = tid >> 6;
    const long nq = a.V / 4;
    const int r0 = (int)(4 * (nq * wid / a.nt)), r1 = (int)(4 * (nq * (wid + 1) / a.nt));
    const int C = a.nc;
    float lv[kHeadMaxCand];
    int li[kHeadMaxCand];
#pragma unroll
    for (int k = 0; k < kHeadMaxCand; k++) { lv[k] = -FLT_MAX; li[k] = 0; }
    // rows visited in increasing order per thread: an equal later value stays behind
    for (int r = r0 + tid; r < r1; r += blockDim.x) {
        const float v = a.screen[r];
        if (v > lv[C - 1]) {
            lv[C - 1] = v;
            li[C - 1] = r;
#pragma unroll
            for (int p = kHeadMaxCand - 1; p > 0; p--)
                if (p < C && lv[p - 1] < lv[p]) {
                    const float tv = lv[p]; lv[p] = lv[p - 1]; lv[p - 1] = tv;
                    const int ti = li[p]; li[p] = li[p - 1]; li[p - 1] = ti;
                }
        }
    }
    // merge: C rounds of a block-wide best over each thread's next entry
    int ptr = 0;
    for (int k = 0; k < C; k++) {
        float v = -FLT_MAX;
        int i = 0x7fffffff;
#pragma unroll
        for (int p = 0; p < kHeadMaxCand; p++)
            if (p == ptr) { v = lv[p]; i = li[p]; }
        // an exhausted thread (ptr == C) offers nothing
        if (ptr >= C) { v = -FLT_MAX; i = 0x7fffffff; }
        int t = tid;
#pragma unroll
        for (int s2 = 32; s2 >= 1; s2 >>= 1) {
            const float ov = __shfl_xor(v, s2);
            const int oi = __shfl_xor(i, s2), ot = __shfl_xor(t, s2);
            if (better(ov, oi, v, i) || (ov == v && oi == i && ot < t)) { v = ov; i = oi; t = ot; }
        }
        if (lane == 0) { wv[wv_id] = v; wi[wv_id] = i; wt[wv_id] = t; }
        __syncthreads();
        if (tid == 0) {
            float bv = wv[0];
            int bi = wi[0], bt = wt[0];
            for (int q = 1; q < (int)(blockDim.x >> 6); q++)
                if (better(wv[q], wi[q], bv, bi) || (wv[q] == bv && wi[q] == bi && wt[q] < bt)) {
                    bv = wv[q]; bi = wi[q]; bt = wt[q];
                }
            // an empty slice keeps the reference's initial entries (-FLT_MAX, row 0)
            a.cand_ids[wid * C + k] = bi == 0x7fffffff ? 0 : bi;
            a.cand_screen[wid * C + k] = bv;
            win_tid = bt;
        }
        __syncthreads();
        if (tid == win_tid) ptr++;
        __syncthreads();
    }
}

// ---- exact Q8 logits of the candidates (dot_q8_i8, :169-191) + greedy ----
// 8 lanes per candidate: chain (accumulator h = even / odd blocks, lane part j)
__global__ __launch_bounds__(1024) void k_head_refine(HeadDev a) {
    __shared__ float lg[1024 / 8];
    const int tid = threadIdx.x, nc = a.nt * a.nc, nb = a.nb;
    const int c = tid >> 3, h = (tid >> 2) & 1, j = tid & 3;
    if (c < nc) {
        const int row = a.cand_ids[c];
        const int8_t* q = a.q8 + (size_t)row * a.d;
        const float* s = a.q8s + (size_t)row * nb;
        const int nbe = nb & ~1;
        float acc = 0.0f;
        auto blk = [&](int b) {
            const uint32_t w0 = *(const uint32_t*)(q + b * 32 + 4 * j), w1 = *(const uint32_t*)(q + b * 32 + 16 + 4 * j);
            const uint32_t x0 = *(const uint32_t*)(a.xq + b * 32 + 4 * j), x1 = *(const uint32_t*)(a.xq + b * 32 + 16 + 4 * j);
            const int t = sdot4(w1, x1, sdot4(w0, x0, 0));
            acc = fmaf((float)t, s[b] * a.xsb[b], acc);
        };
        for (int b = h; b < nbe; b += 2) blk(b);
        if ((nb & 1) && h == 0) blk(nb - 1);       // an odd last block goes into the first accumulator
        // v_j = acc0_j + acc1_j, then (v0 + v1) + (v2 + v3)
        const float v = acc + __shfl_xor(acc, 4);
        const float v01 = v + __shfl_xor(v, 1);     // lanes j = 0, 1 -> v0 + v1; j = 2, 3 -> v2 + v3
        const float tot = __shfl(v01, (tid & ~7)) + __shfl(v01, (tid & ~7) + 2);
        if ((tid & 7) == 0) {
            lg[c] = tot;
            a.cand_logits[c] = tot;
        }
    }
    __syncthreads();
    if (tid == 0) {
        float best = -FLT_MAX;
        int bi = 0;
        for (int k = 0; k < nc; k++)
            if (lg[k] > best) { best = lg[k]; bi = a.cand_ids[k]; }
        *a.chosen = bi;
    }
}

}  // namespace cpb

using cpb::fail;

struct cpb_head {
    cpb_head_cfg cfg{};
    int device = 0;
    hipStream_t own = nullptr, stream = nullptr;
    cpb::HeadDev a{};
    void* base[12] = {};
    bool loaded = false;
};

namespace {
int head_check(const cpb_head_cfg* c) {
    if (!c) return fail(CPB_EINVAL, "cfg is NULL");
    if (c->d <= 0 || c->d % 32 || c->d > 4096) return fail(CPB_EINVAL, "head d=%d must be a multiple of 32, <= 4096", c->d);
    if (c->n_vocab <= 0 || c->n_vocab % 4) return fail(CPB_EINVAL, "n_vocab=%d must be a positive multiple of 4", c->n_vocab);
    if (c->n_slices < 1 || c->n_slices > 32) return fail(CPB_EINVAL, "n_slices=%d outside [1, 32]", c->n_slices);
    if (c->n_cand < 1 || c->n_cand > cpb::kHeadMaxCand) return fail(CPB_EINVAL, "n_cand=%d outside [1, 16]", c->n_cand);
    if (c->n_slices * c->n_cand > 128) return fail(CPB_EINVAL, "n_slices * n_cand must be <= 128");
    return 0;
}
size_t vpad(const cpb_head_cfg* c) { return ((size_t)c->n_vocab + cpb::kHeadRT - 1) / cpb::kHeadRT * cpb::kHeadRT; }
}  // namespace

#define HIP_OK_H(expr)                                                                  \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return fail(e_ == hipErrorOutOfMemory ? CPB_ENOMEM : CPB_ENODEV, "%s: %s", #expr, \
                        hipGetErrorString(e_));                                          \
    } while (0)

extern "C" {

int cpb_head_bytes(const cpb_head_cfg* c, size_t* out) {
    if (int r = head_check(c)) return r;
    if (!out) return fail(CPB_EINVAL, "out is NULL");
    const size_t nb = c->d / 32;
    *out = vpad(c) * nb * (16 + 2) + (size_t)c->n_vocab * (c->d + nb * 4);
    return 0;
}

void cpb_head_destroy(cpb_head_t* h) {
    if (!h) return;
    hipSetDevice(h->device);
    if (h->stream) hipStreamSynchronize(h->stream);
    for (void* p : h->base)
        if (p) hipFree(p);
    if (h->own) hipStreamDestroy(h->own);
    delete h;
}

int cpb_head_create(const cpb_head_cfg* cfg, int device, cpb_head_t** out) {
    if (!out) return fail(CPB_EINVAL, "out is NULL");
    *out = nullptr;
    if (int r = head_check(cfg)) return r;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return fail(CPB_ENODEV, "no HIP device");
    if (device < 0 || device >= ndev) return fail(CPB_EINVAL, "device %d out of range", device);
    HIP_OK_H(hipSetDevice(device));
    cpb_head_t* h = new cpb_head_t();
    h->cfg = *cfg;
    h->device = device;
    auto bail = [&](int r) { cpb_head_destroy(h); return r; };
    if (hipStreamCreateWithFlags(&h->own, hipStreamNonBlocking) != hipSuccess) return bail(fail(CPB_ENODEV, "stream create failed"));
    h->stream = h->own;
    cpb::HeadDev& a = h->a;
    a.d = cfg->d; a.nb = cfg->d / 32; a.V = cfg->n_vocab; a.Vpad = (int)vpad(cfg);
    a.nt = cfg->n_slices; a.nc = cfg->n_cand; a.eps = cfg->rms_eps;
    const size_t nb = a.nb, nc = (size_t)a.nt * a.nc;
    const size_t sizes[12] = {(size_t)a.Vpad * nb * 16, (size_t)a.Vpad * nb * 2, (size_t)a.V * a.d, (size_t)a.V * nb * 4,
                              (size_t)a.d * 4, (size_t)a.d * 4, (size_t)a.d + nb * 4 + nb * 16, (size_t)a.Vpad * 4,
                              nc * 4, nc * 4, nc * 4, 4};
    for (int i = 0; i < 12; i++) {
        hipError_t e = hipMalloc(&h->base[i], sizes[i]);
        if (e != hipSuccess) return bail(fail(CPB_ENOMEM, "hipMalloc(%zu): %s", sizes[i], hipGetErrorString(e)));
    }
    a.q4 = (const cpb::u32x4*)h->base[0];
    a.q4s = (const uint16_t*)h->base[1];
    a.q8 = (const int8_t*)h->base[2];
    a.q8s = (const float*)h->base[3];
    a.norm_w = (const float*)h->base[4];
    a.x = (const float*)h->base[5];
    a.xq = (int8_t*)h->base[6];
    a.xsb = (float*)((char*)h->base[6] + a.d);
    a.xs8 = (int32_t*)((char*)h->base[6] + a.d + nb * 4);
    a.screen = (float*)h->base[7];
    a.cand_ids = (int32_t*)h->base[8];
    a.cand_screen = (float*)h->base[9];
    a.cand_logits = (float*)h->base[10];
    a.chosen = (int32_t*)h->base[11];
    *out = h;
    return 0;
}

int cpb_head_load(cpb_head_t* h, const uint16_t* out_w, const float* out_norm) {
    if (!h || !out_w || !out_norm) return fail(CPB_EINVAL, "NULL argument");
    HIP_OK_H(hipSetDevice(h->device));
    const cpb::HeadDev& a = h->a;
    const size_t wbytes = (size_t)a.V * a.d * 2;
    uint16_t* staging = nullptr;
    HIP_OK_H(hipMalloc(&staging, wbytes));
    hipError_t e = hipMemcpyAsync(staging, out_w, wbytes, hipMemcpyHostToDevice, h->stream);
    if (e == hipSuccess) e = hipMemcpyAsync((void*)a.norm_w, out_norm, (size_t)a.d * 4, hipMemcpyHostToDevice, h->stream);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(cpb::k_head_quant, dim3(8192), dim3(256), 0, h->stream, staging, a.V, a.Vpad, a.d,
                           (cpb::u32x4*)a.q4, (uint16_t*)a.q4s, (int8_t*)a.q8, (float*)a.q8s);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    hipFree(staging);
    if (e != hipSuccess) return fail(CPB_ENODEV, "head load: %s", hipGetErrorString(e));
    h->loaded = true;
    return 0;
}

static int head_launch(cpb_head_t* h) {
    const cpb::HeadDev& a = h->a;
    cpb::launch(cpb::k_head_norm, dim3(1), dim3(256), sizeof(float) * (2 * a.d + 64), h->stream, a);
    const int tiles = a.Vpad / cpb::kHeadRT;
    cpb::launch(cpb::k_head_screen, dim3((tiles + 3) / 4), dim3(256), (size_t)a.nb * (32 + 4 + 16), h->stream, a);
    cpb::launch(cpb::k_head_topk, dim3(a.nt), dim3(1024), 0, h->stream, a);
    cpb::launch(cpb::k_head_refine, dim3(1), dim3(1024), 0, h->stream, a);
    return hipGetLastError() == hipSuccess ? 0 : fail(CPB_ENODEV, "head launch failed");
}

int cpb_head_forward_device(cpb_head_t* h, const float* d_x, int32_t* d_chosen) {
    if (!h || !d_x || !d_chosen) return fail(CPB_EINVAL, "NULL argument");
    if (!h->loaded) return fail(CPB_ESTATE, "head not loaded");
    HIP_OK_H(hipSetDevice(h->device));
    HIP_OK_H(hipMemcpyAsync((void*)h->a.x, d_x, (size_t)h->a.d * 4, hipMemcpyDeviceToDevice, h->stream));
    if (int r = head_launch(h)) return r;
    HIP_OK_H(hipMemcpyAsync(d_chosen, h->a.chosen, 4, hipMemcpyDeviceToDevice, h->stream));
    return 0;
}

int cpb_head_forward(cpb_head_t* h, const float* x, int32_t* chosen, cpb_head_trace* tr) {
    if (!h || !x || !chosen) return fail(CPB_EINVAL, "NULL argument");
    if (!h->loaded) return fail(CPB_ESTATE, "head not loaded");
    HIP_OK_H(hipSetDevice(h->device));
    const cpb::HeadDev& a = h->a;
    HIP_OK_H(hipMemcpyAsync((void*)a.x, x, (size_t)a.d * 4, hipMemcpyHostToDevice, h->stream));
    if (int r = head_launch(h)) return r;
    HIP_OK_H(hipMemcpyAsync(chosen, a.chosen, 4, hipMemcpyDeviceToHost, h->stream));
    if (tr) {
        const size_t nc = (size_t)a.nt * a.nc;
        auto cp = [&](void* dst, const void* src, size_t n) -> int {
            if (dst) HIP_OK_H(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, h->stream));
            return 0;
        };
        int r = 0;
        r |= cp(tr->cand_ids, a.cand_ids, nc * 4);
        r |= cp(tr->cand_screen, a.cand_screen, nc * 4);
        r |= cp(tr->cand_logits, a.cand_logits, nc * 4);
        r |= cp(tr->xq, a.xq, a.d);
        r |= cp(tr->xsb, a.xsb, a.nb * 4);
        r |= cp(tr->screen, a.screen, (size_t)a.V * 4);
        if (r) return r;
    }
    HIP_OK_H(hipStreamSynchronize(h->stream));
    return 0;
}

int cpb_head_set_stream(cpb_head_t* h, void* stream) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    hipStream_t ns = stream ? (hipStream_t)stream : h->own;
    if (ns == h->stream) return 0;
    HIP_OK_H(hipSetDevice(h->device));
    HIP_OK_H(hipStreamSynchronize(h->stream));   // the new stream starts after the old one's work
    h->stream = ns;
    return 0;
}

int cpb_head_sync(cpb_head_t* h) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    HIP_OK_H(hipStreamSynchronize(h->stream));
    return 0;
}

}  // extern "C"
