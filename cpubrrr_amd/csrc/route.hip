// route.hip -- per-token ffn rmsnorm, activation quantisation and router
// logits with certified error bounds (gfx950).
//
// Reference: engine_gpt2.rs:846-850 (gpt-oss) and engine_qwen2.rs:395-400
// (Qwen3).  The reference router is a sequential fp32 multiply-then-add chain
// per expert (acc = bias; acc += W[j]*xn[j]).  That order cannot run in
// parallel, so workgroup e computes expert e's logit from the same fp32
// products summed exactly in fp64, together with a rigorous bound on how far
// the reference's serial fp32 sum can lie from it:
//     |serial - exact| <= u/(1-u) * (sum_k |S_k| + n*gamma_n*A),
// S_k the exact prefix sums (from a block scan), A = |b| + sum |p_j|,
// u = 2^-24, gamma_n = n*u/(1-n*u) (Higham, Accuracy and Stability of
// Numerical Algorithms, 2nd ed., sec. 4.2).  The consumer (select.h, run at
// the start of the gate/up kernel) picks the top-k and certifies it against
// these bounds, recomputing the serial chain only when an interval overlap
// could change the choice.  No cross-workgroup synchronisation here.
#include "moe_common.h"
#include "route.h"
#include "select.h"

namespace cpb {

// Per-token rmsnorm into LDS (xn) in the reference's summation order.
// gpt-oss: ssq() with 4 NEON accumulators x 4 lanes of fma over 16-wide steps
// (engine_gpt2.rs:710-726): lane q (0..15) of wave 0 runs chain q over
// x[16m + q]; Qwen: nt serial slices, then a serial sum of the partials
// (engine_qwen2.rs:457-467).
CPB_DEV void norm_into(const float* __restrict__ xg, const float* __restrict__ nw, int d, float eps,
                       int norm, int nt, int apply, float* xs, float* xn, float* scratch) {
    const int tid = threadIdx.x, nth = blockDim.x;
    for (int i = tid; i < d / 4; i += nth) ((float4*)xs)[i] = ((const float4*)xg)[i];
    __syncthreads();
    if (!apply) {
        for (int i = tid; i < d / 4; i += nth) ((float4*)xn)[i] = ((const float4*)xs)[i];
        __syncthreads();
        return;
    }
    if (norm == 0) {
        if (tid < 16) {
            float a = 0.0f;
            const int n16 = d / 16;
            int m = 0;
            for (; m + 16 <= n16; m += 16) {
                float t[16];
#pragma unroll
                for (int u = 0; u < 16; u++) t[u] = xs[(m + u) * 16 + tid];
#pragma unroll
                for (int u = 0; u < 16; u++) a = fmaf(t[u], t[u], a);
            }
            for (; m < n16; m++) { float t = xs[m * 16 + tid]; a = fmaf(t, t, a); }
            scratch[tid] = a;                  // chain q = 4v + l  ->  a[v][l]
        }
        __syncthreads();
        if (tid == 0) {
            float L[4];
            for (int l = 0; l < 4; l++) L[l] = (scratch[l] + scratch[4 + l]) + (scratch[8 + l] + scratch[12 + l]);
            float s = (L[0] + L[1]) + (L[2] + L[3]);
            for (int i = d - d % 16; i < d; i++) s += xs[i] * xs[i];
            scratch[16] = 1.0f / sqrtf(s / (float)d + eps);
        }
    } else {
        const int base = d / nt, rem = d % nt;
        if (tid < nt) {
            const int a = tid * base + (tid < rem ? tid : rem), sz = base + (tid < rem ? 1 : 0);
            float ps = 0.0f;
            int i = 0;
            for (; i + 16 <= sz; i += 16) {
                float t[16];
#pragma unroll
                for (int u = 0; u < 16; u++) t[u] = xs[a + i + u];
#pragma unroll
                for (int u = 0; u < 16; u++) ps += t[u] * t[u];
            }
            for (; i < sz; i++) { float v = xs[a + i]; ps += v * v; }
            scratch[tid] = ps;
        }
        __syncthreads();
        if (tid == 0) {
            float tot = 0.0f;
            for (int k = 0; k < nt; k++) tot += scratch[k];
            scratch[16] = 1.0f / sqrtf(tot / (float)d + eps);
        }
    }
    __syncthreads();
    const float inv = scratch[16];
    for (int i = tid; i < d; i += nth) xn[i] = xs[i] * inv * (nw ? nw[i] : 1.0f);
    __syncthreads();
}

template <typename T>
CPB_DEV T block_sum(T v, T* red) {
    // 256 threads; fixed-shape tree (deterministic)
    const int tid = threadIdx.x;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    T r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

constexpr int kChunk = 16;          // router elements per thread: d <= 4096

__global__ __launch_bounds__(256) void k_route(RouteArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* xs = (float*)smem;                 // [d]
    float* xn = xs + a.d;                     // [d]
    double* dsc = (double*)(xn + a.d + 32);   // [8]
    double* dred = dsc + 8;                   // [8]
    float* scratch = (float*)(dred + 8);      // [64]
    const int tid = threadIdx.x;
    const int e = blockIdx.x;
    const int d = a.d;

    // router row chunk of this thread, loaded before anything waits on x
    const int C = ((d + 1023) / 1024) * 4;    // multiple of 4, C*256 >= d
    const int j0 = tid * C;
    const float* W = a.router_w + (size_t)e * d;
    float4 wv[kChunk / 4];
#pragma unroll
    for (int i = 0; i < kChunk / 4; i++) {
        const int j = min(j0 + 4 * i, d - 4);
        wv[i] = *(const float4*)(W + j);
    }
    const double b = a.router_b ? (double)a.router_b[e] : 0.0;

    norm_into(a.x, a.norm_w, d, a.eps, a.norm, a.norm_nt, a.apply_norm, xs, xn, scratch);

    // quantisation, distributed over the workgroups (each also publishes the
    // xn values of its blocks)
    const int NEg = gridDim.x;
    if (a.qk == 0) {
        // Q8 per 32-block (engine_gpt2.rs:691-699): 32 lanes per block
        const int l = tid & 31;
        for (int bk = e * 8 + (tid >> 5); bk < d / 32; bk += NEg * 8) {
            const float v = xn[bk * 32 + l];
            float m = fabsf(v);
#pragma unroll
            for (int s2 = 16; s2 >= 1; s2 >>= 1) m = fmaxf(m, __shfl_xor(m, s2));
            const float sc = fmaxf(1e-12f, m) / 127.0f;
            const int qv = q8_round(v, sc);
            a.xn[bk * 32 + l] = v;
            a.xq[bk * 32 + l] = (int8_t)qv;
            a.xqn[bk * 32 + l] = (int8_t)(-qv);
            if (l == 0) a.xsb[bk] = sc;
        }
    } else {
        // Q8_K per 256 (engine_qwen2.rs:288-300): one wave per superblock
        const int l = tid & 63;
        for (int sb = e * 4 + (tid >> 6); sb < d / 256; sb += NEg * 4) {
            float v[4], m = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) { v[k] = xn[sb * 256 + 64 * k + l]; m = fmaxf(m, fabsf(v[k])); }
            const float sc = fmaxf(1e-12f, wave_max(m)) / 127.0f;
            if (l == 0) a.xsb[sb] = sc;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int qv = q8_round(v[k], sc);
                a.xn[sb * 256 + 64 * k + l] = v[k];
                a.xq[sb * 256 + 64 * k + l] = (int8_t)qv;
                a.xqn[sb * 256 + 64 * k + l] = (int8_t)(-qv);
                int s3 = qv;   // per-32 sums: group 2k + (l >= 32)
#pragma unroll
                for (int m2 = 16; m2 >= 1; m2 >>= 1) s3 += __shfl_xor(s3, m2);
                if ((l & 31) == 0) a.xsum[sb * 8 + 2 * k + (l >> 5)] = s3;
            }
        }
    }

    // ---- router logit of expert e: the reference's fp32 products, exact
    // fp64 sum and prefix sums, error bound ----
    float p[kChunk];
    double loc = 0.0, absp = 0.0;
#pragma unroll
    for (int i = 0; i < kChunk / 4; i++) {
        const int j = j0 + 4 * i;
        const int jc = min(j, d - 4);
        const float4 xv = *(const float4*)(xn + jc);
        const float4 w4 = wv[i];
        const float pr[4] = {w4.x * xv.x, w4.y * xv.y, w4.z * xv.z, w4.w * xv.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const bool in = 4 * i + k < C && j + k < d && j == jc;
            p[4 * i + k] = in ? pr[k] : 0.0f;
            loc += (double)p[4 * i + k];
            absp += fabs((double)p[4 * i + k]);
        }
    }
    // exclusive scan of the 256 chunk sums: wave scan + 4 wave totals
    const int lane = tid & 63, wv_ = tid >> 6;
    double inc = loc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double t = __shfl_up(inc, off);
        if (lane >= off) inc += t;
    }
    if (lane == 63) dsc[wv_] = inc;
    __syncthreads();
    double woff = 0.0;
    for (int w2 = 0; w2 < wv_; w2++) woff += dsc[w2];
    const double total = b + ((dsc[0] + dsc[1]) + (dsc[2] + dsc[3]));
    double run = b + woff + (inc - loc);
    double sabs = 0.0;
#pragma unroll
    for (int i = 0; i < kChunk; i++) { run += (double)p[i]; sabs += (i < C && j0 + i < d) ? fabs(run) : 0.0; }
    __syncthreads();
    const double SS = block_sum(sabs, dred);
    const double AP = block_sum(absp, dred);
    if (tid == 0) {
        const double u = 5.9604644775390625e-08;  // 2^-24
        const double n = (double)d;
        const double A = fabs(b) + AP;
        const double gam = n * u / (1.0 - n * u);
        double bound = u / (1.0 - u) * (SS + n * gam * A);
        bound = bound * 1.0001 + 1e-10 * A + 1e-30;
        a.lstar[e] = total;
        a.lbound[e] = bound;
    }
}

// One wavefront: rank, certify, softmax; publishes ids / weights / logits.
__global__ __launch_bounds__(64) void k_select(SelectArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Selection sel;
    select_experts_wave(a.lstar, a.lbound, a.n_expert, a.top_k, a.router_w, a.router_b, a.xn, a.d, (double*)smem, &sel);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int lane = threadIdx.x;
    for (int i = lane; i < a.n_expert; i += 64) a.logits[i] = (float)a.lstar[i];
    if (lane < a.top_k) {
        a.ids[lane] = sel.ids[lane];
        a.wts[lane] = sel.wts[lane];
        a.logits[sel.ids[lane]] = sel.logit[lane];   // as used (exact serial values after a fallback)
    }
    if (lane == 0) *a.fallback = sel.fallback;
}

int launch_select(const SelectArgs* a, hipStream_t s) {
    size_t lds = sizeof(double) * 4 * a->n_expert + 64;
    hipLaunchKernelGGL(k_select, dim3(1), dim3(64), lds, s, *a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_route(const RouteArgs* a, hipStream_t s) {
    if (a->n_expert > 256 || a->n_expert < a->top_k || a->top_k > 8 || a->d % 32 != 0 || a->d > 4096)
        return -22;
    size_t lds = sizeof(float) * (2 * a->d + 32) + sizeof(double) * 16 + sizeof(float) * 64;
    hipLaunchKernelGGL(k_route, dim3(a->n_expert), dim3(256), lds, s, *a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
