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

// ---- wavefront DPP helpers on doubles (no LDS round trips) ----
// v from the DPP source lane; lanes whose source is out of the row, or whose
// row is masked off, read 0.0
template <int CTRL, int ROWMASK>
CPB_DEV double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWMASK, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWMASK, 0xF, true);
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
// inclusive prefix sum over the 64 lanes (row_shr 1,2,4,8, then row_bcast 15, 31)
CPB_DEV double wave_scan_f64(double v) {
    v += dpp_f64<0x111, 0xF>(v);
    v += dpp_f64<0x112, 0xF>(v);
    v += dpp_f64<0x114, 0xF>(v);
    v += dpp_f64<0x118, 0xF>(v);
    v += dpp_f64<0x142, 0xA>(v);
    v += dpp_f64<0x143, 0xC>(v);
    return v;
}
// sum over the 64 lanes, valid in lane 63 (quad swaps, half-row and row
// mirrors, then row_bcast 15, 31)
CPB_DEV double wave_total63_f64(double v) {
    v += dpp_f64<0xB1, 0xF>(v);
    v += dpp_f64<0x4E, 0xF>(v);
    v += dpp_f64<0x141, 0xF>(v);
    v += dpp_f64<0x140, 0xF>(v);
    v += dpp_f64<0x142, 0xA>(v);
    v += dpp_f64<0x143, 0xC>(v);
    return v;
}
// max over each aligned group of 16 lanes (a DPP row), in every lane of it
CPB_DEV float row_max_f32(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    return v;
}
// value of the neighbouring lane (lane ^ 1)
CPB_DEV float pair_f32(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)); }
CPB_DEV int pair_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }

// 16-byte store with the cache policy of st_dev (sc1: visible across XCDs)
CPB_DEV void st_dev16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, 16);
}

constexpr int kRouteC = 16;         // consecutive elements per thread in route_expert

// LDS bytes route_expert needs (any block size; d <= 4096)
CPB_DEV_HOST inline int route_xt_stride(int d) { return (d / 16 + 63) / 64 * 64 + 4; }
CPB_DEV_HOST inline size_t route_lds_bytes(int d) {
    const size_t xt = sizeof(float) * 16 * (size_t)route_xt_stride(d);
    const size_t xr = sizeof(float) * (size_t)d;
    return (xt > xr ? xt : xr) + sizeof(double) * 64 + 64;
}

// Workgroup-level body: expert e's logit + bound, and this workgroup's share
// (blocks b with b % NEg == e) of the activation quantisation.  Any multiple
// of 64 threads with blockDim.x * 16 >= d.
//
// Thread t owns x[16t .. 16t+16): its x, norm weights and router weights
// arrive in registers from one round of loads.  The gpt-oss sum of squares
// (16 fma chains, chain q over x[16m + q], engine_gpt2.rs:710-726) runs in 16
// lanes of wave 0 over a transposed LDS copy (chain q's elements contiguous);
// the Qwen one (nt serial slices, engine_qwen2.rs:457-467) over a plain copy.
// The router logit is the exact fp64 sum of the reference's fp32 products
// with the prefix-sum error bound of router_logit, from one DPP scan.
CPB_DEV void route_expert(const RouteArgs& a, int e, int NEg, unsigned char* smem) {
    const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63, wv = tid >> 6, nw = nth >> 6;
    const int d = a.d;
    const int S = route_xt_stride(d);
    float* xl = (float*)smem;                                  // transposed (gpt-oss) or plain (Qwen) x
    double* dred = (double*)(smem + route_lds_bytes(d) - sizeof(double) * 64 - 64);   // [64]
    float* sinv = (float*)(dred + 64);
    RSTAMP(0);

    const int j0 = tid * kRouteC;
    const bool act = j0 < d;
    const uint32_t off = (uint32_t)(act ? j0 : 0) * 4;
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x, (uint32_t)d * 4);
    const __amdgpu_buffer_rsrc_t rW = buf_rsrc(a.router_w + (size_t)e * d, (uint32_t)d * 4);
    const bool use_g = a.norm_w && a.apply_norm;
    const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.norm_w, use_g ? (uint32_t)d * 4 : 0u);
    u32x4 xv[4], wq[4], gq[4];
#pragma unroll
    for (int k = 0; k < 4; k++) xv[k] = ld_dev16(rx, off + 16 * k);     // may come from this launch
#pragma unroll
    for (int k = 0; k < 4; k++) wq[k] = __builtin_amdgcn_raw_buffer_load_b128(rW, off + 16 * k, 0, 0);
#pragma unroll
    for (int k = 0; k < 4; k++) gq[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off + 16 * k, 0, 0);
    const double b = a.router_b ? (double)a.router_b[e] : 0.0;
    float xf[16];
#pragma unroll
    for (int i = 0; i < 16; i++) xf[i] = act ? __uint_as_float(xv[i >> 2][i & 3]) : 0.0f;
    RSTAMP(1);

    // ---- rmsnorm scale ----
    float inv = 1.0f;
    if (a.apply_norm) {
        if (a.norm == 0) {
            // chain q's element m = x[16m + q] lives in thread m, register q
            if (act) {
#pragma unroll
                for (int i = 0; i < 16; i++) xl[i * S + tid] = xf[i];
            }
            __syncthreads();
            if (wv == 0) {
                const int nm = d / 16;
                float acc = 0.0f;
                if (lane < 16) {
                    const float* row = xl + lane * S;
                    int m = 0;
                    for (; m + 16 <= nm; m += 16) {
                        float4 t[4];
#pragma unroll
                        for (int u = 0; u < 4; u++) t[u] = *(const float4*)(row + m + 4 * u);
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            acc = fmaf(t[u].x, t[u].x, acc);
                            acc = fmaf(t[u].y, t[u].y, acc);
                            acc = fmaf(t[u].z, t[u].z, acc);
                            acc = fmaf(t[u].w, t[u].w, acc);
                        }
                    }
                    for (; m < nm; m++) { const float t = row[m]; acc = fmaf(t, t, acc); }
                }
                // chain q = 4v + l -> acc[v][l]; L[l] = (a0 + a1) + (a2 + a3); s = (L0 + L1) + (L2 + L3)
                float c[16];
#pragma unroll
                for (int q = 0; q < 16; q++) c[q] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), q));
                float L[4];
#pragma unroll
                for (int l = 0; l < 4; l++) L[l] = (c[l] + c[4 + l]) + (c[8 + l] + c[12 + l]);
                const float s = (L[0] + L[1]) + (L[2] + L[3]);
                if (lane == 0) *sinv = 1.0f / sqrtf(s / (float)d + a.eps);
            }
        } else {
            if (act) {
#pragma unroll
                for (int k = 0; k < 4; k++) ((u32x4*)xl)[tid * 4 + k] = xv[k];
            }
            __syncthreads();
            const int nt = a.norm_nt, base = d / nt, rem = d % nt;
            float ps = 0.0f;
            if (tid < nt) {
                const int s0 = tid * base + (tid < rem ? tid : rem), sz = base + (tid < rem ? 1 : 0);
                int i = 0;
                for (; i + 16 <= sz; i += 16) {
                    float t[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) t[u] = xl[s0 + i + u];
#pragma unroll
                    for (int u = 0; u < 16; u++) ps += t[u] * t[u];
                }
                for (; i < sz; i++) { const float v = xl[s0 + i]; ps += v * v; }
            }
            // serial sum of the nt partials (nt <= 64: all in wave 0)
            if (wv == 0) {
                float tot = 0.0f;
                for (int k = 0; k < nt; k++) tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ps), k));
                if (lane == 0) *sinv = 1.0f / sqrtf(tot / (float)d + a.eps);
            }
        }
        __syncthreads();
        inv = *sinv;
    }
    RSTAMP(2);

    // ---- xn = (x * inv) * w in registers ----
    float xn[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float g = __uint_as_float(gq[i >> 2][i & 3]);
        xn[i] = !a.apply_norm ? xf[i] : use_g ? (xf[i] * inv) * g : xf[i] * inv;
    }

    // ---- activation quantisation (this workgroup's share) ----
    if (a.qk == 0) {
        // Q8 per 32-block (engine_gpt2.rs:691-699): threads 2b, 2b+1 hold block b
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(xn[i]));
        m = fmaxf(m, pair_f32(m));
        const int blk = tid >> 1;
        if (act && blk % NEg == e) {
            const float sc = fmaxf(1e-12f, m) / 127.0f;
            uint32_t qp[4] = {0, 0, 0, 0}, qn[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int qv = q8_round(xn[i], sc);
                qp[i >> 2] |= (uint32_t)(uint8_t)qv << (8 * (i & 3));
                qn[i >> 2] |= (uint32_t)(uint8_t)(-qv) << (8 * (i & 3));
            }
            const __amdgpu_buffer_rsrc_t rn = buf_rsrc(a.xn, (uint32_t)d * 4);
#pragma unroll
            for (int k = 0; k < 4; k++)
                st_dev16(rn, off + 16 * k, u32x4{__float_as_uint(xn[4 * k]), __float_as_uint(xn[4 * k + 1]),
                                                 __float_as_uint(xn[4 * k + 2]), __float_as_uint(xn[4 * k + 3])});
            st_dev16(buf_rsrc(a.xq, (uint32_t)d), (uint32_t)j0, u32x4{qp[0], qp[1], qp[2], qp[3]});
            st_dev16(buf_rsrc(a.xqn, (uint32_t)d), (uint32_t)j0, u32x4{qn[0], qn[1], qn[2], qn[3]});
            if ((tid & 1) == 0) st_dev(a.xsb + blk, sc);
        }
    } else {
        // Q8_K per 256 (engine_qwen2.rs:288-300): the 16 threads of a DPP row
        // hold one superblock; per-32 sums from thread pairs
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(xn[i]));
        m = row_max_f32(m);
        const int sb = tid >> 4;
        const float sc = fmaxf(1e-12f, m) / 127.0f;
        uint32_t qp[4] = {0, 0, 0, 0}, qn[4] = {0, 0, 0, 0};
        int s32 = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int qv = q8_round(xn[i], sc);
            s32 += qv;
            qp[i >> 2] |= (uint32_t)(uint8_t)qv << (8 * (i & 3));
            qn[i >> 2] |= (uint32_t)(uint8_t)(-qv) << (8 * (i & 3));
        }
        s32 += pair_i32(s32);
        if (act && sb % NEg == e) {
            const __amdgpu_buffer_rsrc_t rn = buf_rsrc(a.xn, (uint32_t)d * 4);
#pragma unroll
            for (int k = 0; k < 4; k++)
                st_dev16(rn, off + 16 * k, u32x4{__float_as_uint(xn[4 * k]), __float_as_uint(xn[4 * k + 1]),
                                                 __float_as_uint(xn[4 * k + 2]), __float_as_uint(xn[4 * k + 3])});
            st_dev16(buf_rsrc(a.xq, (uint32_t)d), (uint32_t)j0, u32x4{qp[0], qp[1], qp[2], qp[3]});
            st_dev16(buf_rsrc(a.xqn, (uint32_t)d), (uint32_t)j0, u32x4{qn[0], qn[1], qn[2], qn[3]});
            if ((tid & 15) == 0) st_dev(a.xsb + sb, sc);
            if ((tid & 1) == 0) st_dev(a.xsum + (tid >> 1), s32);
        }
    }
    RSTAMP(3);

    // ---- router logit of expert e: exact fp64 sum of the reference's fp32
    // products and the bound u/(1-u) * (sum_k |S_k| + n*gamma_n*A) ----
    float p[16];
    double loc = 0.0, absp = 0.0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        p[i] = act ? __fmul_rn(__uint_as_float(wq[i >> 2][i & 3]), xn[i]) : 0.0f;
        loc += (double)p[i];
        absp += fabs((double)p[i]);
    }
    const double incl = wave_scan_f64(loc);
    if (lane == 63) dred[wv] = incl;
    __syncthreads();
    double woff = 0.0, wtot = 0.0;
    for (int w2 = 0; w2 < nw; w2++) {
        const double t = dred[w2];
        if (w2 < wv) woff += t;
        wtot += t;
    }
    double run = b + woff + (incl - loc);
    double sabs = 0.0;
#pragma unroll
    for (int i = 0; i < 16; i++) { run += (double)p[i]; sabs += act ? fabs(run) : 0.0; }
    const double ws = wave_total63_f64(sabs);
    const double wa = wave_total63_f64(absp);
    if (lane == 63) { dred[16 + wv] = ws; dred[32 + wv] = wa; }
    __syncthreads();
    RSTAMP(4);
    if (tid == 0) {
        double SS = 0.0, AP = 0.0;
        for (int w2 = 0; w2 < nw; w2++) { SS += dred[16 + w2]; AP += dred[32 + w2]; }
        const double u = 5.9604644775390625e-08;  // 2^-24
        const double n = (double)d;
        const double A = fabs(b) + AP;
        const double gam = n * u / (1.0 - n * u);
        const double bound = u / (1.0 - u) * (SS + n * gam * A);
        st_dev(a.lstar + e, b + wtot);
        st_dev(a.lbound + e, bound * 1.0001 + 1e-10 * A + 1e-30);
    }
    RSTAMP(5);
}



}  // namespace cpb
