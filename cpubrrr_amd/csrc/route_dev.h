// route_dev.h -- device body of the per-token routing step (see route.hip).
#pragma once
#include "moe_common.h"
#include "route.h"

#ifndef CPB_DEV_HOST
#define CPB_DEV_HOST __host__ __device__
#endif

namespace cpb {

// Per-token rmsnorm into LDS (xn) in the reference's summation order.
// gpt-oss: ssq() with 4 NEON accumulators x 4 lanes of fma over 16-wide steps
// (engine_gpt2.rs:710-726): lane q (0..15) of wave 0 runs chain q over
// x[16m + q]; Qwen: nt serial slices, then a serial sum of the partials
// (engine_qwen2.rs:457-467).
CPB_DEV void norm_into(const float* __restrict__ xg, const float* __restrict__ nw, int d, float eps,
                       int norm, int nt, int apply, float* xs, float* xn, float* scratch) {
    const int tid = threadIdx.x, nth = blockDim.x;
    // x may have been written by other workgroups of the same launch:
    // coherent 16-byte loads.  Thread tid owns float4 slots tid + k*nth
    // (nth * 16 >= d for every launch: d <= 4096, nth >= 256); the norm
    // weights of the same slots are fetched alongside, before the first wait.
    u32x4 wn[4];
    {
        const __amdgpu_buffer_rsrc_t r = buf_rsrc(xg, (uint32_t)d * 4);
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(nw, nw && apply ? (uint32_t)d * 4 : 0u);
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = ld_dev16(r, (uint32_t)(tid + k * nth) * 16);
#pragma unroll
        for (int k = 0; k < 4; k++) wn[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)(tid + k * nth) * 16, 0, 0);
#pragma unroll
        for (int k = 0; k < 4; k++)
            if ((tid + k * nth) * 4 < d) ((u32x4*)xs)[tid + k * nth] = v[k];
    }
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
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i4 = tid + k * nth;
        if (i4 * 4 < d) {
            const float4 xv = ((const float4*)xs)[i4];
            float4 o;
            if (nw) {
                o.x = xv.x * inv * __uint_as_float(wn[k][0]);
                o.y = xv.y * inv * __uint_as_float(wn[k][1]);
                o.z = xv.z * inv * __uint_as_float(wn[k][2]);
                o.w = xv.w * inv * __uint_as_float(wn[k][3]);
            } else {
                o.x = xv.x * inv; o.y = xv.y * inv; o.z = xv.z * inv; o.w = xv.w * inv;
            }
            ((float4*)xn)[i4] = o;
        }
    }
    __syncthreads();
}

template <typename T>
CPB_DEV T block_sum(T v, T* red) {
    // any multiple of 64 threads (<= 1024); fixed order (deterministic)
    const int tid = threadIdx.x, nw = blockDim.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    T r = red[0];
    for (int w = 1; w < nw; w++) r += red[w];
    __syncthreads();
    return r;
}

#ifdef CPB_DECODE_STAMPS
#define RSTAMP(i) do { if (threadIdx.x == 0 && a.stamps) a.stamps[(size_t)e * 16 + (i)] = wall_clock64(); } while (0)
#else
#define RSTAMP(i) do { } while (0)
#endif

constexpr int kChunk = 16;          // router elements per thread: d <= 4096

// Logit of one router row: the reference's fp32 products w[j]*xn[j] (xn in
// LDS) summed exactly in fp64 with the bias, and a bound on how far the
// reference's serial fp32 chain (acc = b; acc += w[j]*xn[j]) can lie from it:
// u/(1-u) * (sum_k |S_k| + n*gamma_n*A) over the exact prefix sums S_k
// (Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed., 4.2).
// wv: this thread's C (<= kChunk) consecutive weights from j0.  Every thread
// of the workgroup calls it; thread 0 receives the results.
CPB_DEV void router_logit(const float4* wv, int C, int j0, const float* xn, int d, double b, double* dsc,
                          double* dred, double* out_total, double* out_bound) {
    const int tid = threadIdx.x, nth = blockDim.x;
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
    // exclusive scan of the chunk sums: wave scan + wave totals
    const int lane = tid & 63, wv_ = tid >> 6, nw = nth >> 6;
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
    double wtot = dsc[0];
    for (int w2 = 1; w2 < nw; w2++) wtot += dsc[w2];
    const double total = b + wtot;
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
        *out_total = total;
        *out_bound = bound * 1.0001 + 1e-10 * A + 1e-30;
    }
}

// LDS bytes route_expert needs
CPB_DEV_HOST inline size_t route_lds_bytes(int d) { return sizeof(float) * (2 * d + 32) + sizeof(double) * 32 + sizeof(float) * 64; }

// Workgroup-level body: expert e's logit + bound, and this workgroup's share
// (index e of NEg) of the activation quantisation.  Any multiple of 64
// threads with blockDim.x * kChunk >= d.
CPB_DEV void route_expert(const RouteArgs& a, int e, int NEg, unsigned char* smem) {
    float* xs = (float*)smem;                 // [d]
    float* xn = xs + a.d;                     // [d]
    double* dsc = (double*)(xn + a.d + 32);   // [16]
    double* dred = dsc + 16;                  // [16]
    float* scratch = (float*)(dred + 16);     // [64]
    const int tid = threadIdx.x, nth = blockDim.x;
    const int d = a.d;
    RSTAMP(0);

    // router row chunk of this thread, loaded before anything waits on x
    const int C = ((d + 4 * nth - 1) / (4 * nth)) * 4;   // multiple of 4, C*nth >= d
    const int j0 = tid * C;
    const float* W = a.router_w + (size_t)e * d;
    float4 wv[kChunk / 4];
#pragma unroll
    for (int i = 0; i < kChunk / 4; i++) {
        const int j = min(j0 + 4 * i, d - 4);
        wv[i] = *(const float4*)(W + j);
    }
    const double b = a.router_b ? (double)a.router_b[e] : 0.0;

    RSTAMP(1);
    norm_into(a.x, a.norm_w, d, a.eps, a.norm, a.norm_nt, a.apply_norm, xs, xn, scratch);
    RSTAMP(2);

    // quantisation, distributed over the workgroups (each also publishes the
    // xn values of its blocks)
    if (a.qk == 0) {
        // Q8 per 32-block (engine_gpt2.rs:691-699): 32 lanes per block
        const int l = tid & 31, g = nth >> 5;
        for (int bk = e * g + (tid >> 5); bk < d / 32; bk += NEg * g) {
            const float v = xn[bk * 32 + l];
            float m = fabsf(v);
#pragma unroll
            for (int s2 = 16; s2 >= 1; s2 >>= 1) m = fmaxf(m, __shfl_xor(m, s2));
            const float sc = fmaxf(1e-12f, m) / 127.0f;
            const int qv = q8_round(v, sc);
            st_dev(a.xn + bk * 32 + l, v);
            st_dev(a.xq + bk * 32 + l, (int8_t)qv);
            st_dev(a.xqn + bk * 32 + l, (int8_t)(-qv));
            if (l == 0) st_dev(a.xsb + bk, sc);
        }
    } else {
        // Q8_K per 256 (engine_qwen2.rs:288-300): one wave per superblock
        const int l = tid & 63, g = nth >> 6;
        for (int sb = e * g + (tid >> 6); sb < d / 256; sb += NEg * g) {
            float v[4], m = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) { v[k] = xn[sb * 256 + 64 * k + l]; m = fmaxf(m, fabsf(v[k])); }
            const float sc = fmaxf(1e-12f, wave_max(m)) / 127.0f;
            if (l == 0) st_dev(a.xsb + sb, sc);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int qv = q8_round(v[k], sc);
                st_dev(a.xn + sb * 256 + 64 * k + l, v[k]);
                st_dev(a.xq + sb * 256 + 64 * k + l, (int8_t)qv);
                st_dev(a.xqn + sb * 256 + 64 * k + l, (int8_t)(-qv));
                int s3 = qv;   // per-32 sums: group 2k + (l >= 32)
#pragma unroll
                for (int m2 = 16; m2 >= 1; m2 >>= 1) s3 += __shfl_xor(s3, m2);
                if ((l & 31) == 0) st_dev(a.xsum + sb * 8 + 2 * k + (l >> 5), s3);
            }
        }
    }

    RSTAMP(3);
    // ---- router logit of expert e ----
    double total = 0.0, bound = 0.0;
    router_logit(wv, C, j0, xn, d, b, dsc, dred, &total, &bound);
    RSTAMP(4);
    if (tid == 0) {
        st_dev(a.lstar + e, total);
        st_dev(a.lbound + e, bound);
    }
    RSTAMP(5);
}



}  // namespace cpb
