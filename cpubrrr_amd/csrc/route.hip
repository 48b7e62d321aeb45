// route.hip -- ffn rmsnorm, activation quantisation, router logits and
// top-k routing for one token (gfx950).
//
// Reference: engine_gpt2.rs:846-867 (gpt-oss) and engine_qwen2.rs:395-410
// (Qwen3).  The reference router is a sequential fp32 multiply-then-add chain
// per expert (acc = bias; acc += W[j]*xn[j]).  That order cannot be run in
// parallel, so each workgroup computes one expert's logit from the same fp32
// products summed exactly in fp64, together with a rigorous bound on how far
// the reference's serial fp32 sum can lie from it:
//     |serial - exact| <= u/(1-u) * (sum_k |S_k| + n*gamma_n*A),
// S_k the exact prefix sums (from a block scan), A = |b| + sum |p_j|,
// u = 2^-24, gamma_n = n*u/(1-n*u) (Higham, Accuracy and Stability of
// Numerical Algorithms, 2nd ed., sec. 4.2).  The last workgroup to finish
// ranks the experts and checks that the chosen top-k (ids and order) is the
// same for every value inside the bounds; if not, it recomputes all logits in
// the reference's serial order (rare: the bound is ~1e-4 against logit gaps
// of ~0.1) so the routing is always identical to the reference's.
#include "moe_common.h"
#include "route.h"

namespace cpb {

// Per-token rmsnorm into LDS (xn) in the reference's summation order.
// gpt-oss: ssq() with 4x4 fma accumulators (engine_gpt2.rs:710-726);
// Qwen: nt serial slices then a serial sum of the partials (engine_qwen2.rs:457-467).
CPB_DEV void norm_into(const float* __restrict__ xg, const float* __restrict__ nw, int d, float eps,
                       int norm, int nt, int apply, float* xs, float* xn, float* scratch) {
    const int tid = threadIdx.x, nth = blockDim.x;
    for (int i = tid; i < d; i += nth) xs[i] = xg[i];
    __syncthreads();
    if (!apply) {
        for (int i = tid; i < d; i += nth) xn[i] = xs[i];
        __syncthreads();
        return;
    }
    if (norm == 0) {
        if (tid < 16) {                 // lane tid = 4*v + l accumulates x[16i + tid]^2
            float a = 0.0f;
            for (int i = 0; i + 16 <= d; i += 16) { float t = xs[i + tid]; a = fmaf(t, t, a); }
            scratch[tid] = a;
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
        int base = d / nt, rem = d % nt;
        if (tid < nt) {
            int a = tid * base + (tid < rem ? tid : rem), sz = base + (tid < rem ? 1 : 0);
            float ps = 0.0f;
            for (int i = a; i < a + sz; i++) { float v = xs[i]; ps += v * v; }
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
    float inv = scratch[16];
    for (int i = tid; i < d; i += nth) xn[i] = xs[i] * inv * (nw ? nw[i] : 1.0f);
    __syncthreads();
}

template <typename T>
CPB_DEV T block_sum(T v, T* red) {
    // 256 threads; deterministic fixed-shape tree
    const int tid = threadIdx.x;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    T r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(256) void k_route(RouteArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* xs = (float*)smem;                 // [d]
    float* xn = xs + a.d;                     // [d]
    double* dsc = (double*)(xn + a.d + 32);   // [256] chunk sums (8-aligned: d % 32 == 0)
    double* dred = dsc + 256;                 // [8]
    float* scratch = (float*)(dred + 8);      // [64]
    const int tid = threadIdx.x;
    const int e = blockIdx.x;
    const int d = a.d;

    norm_into(a.x, a.norm_w, d, a.eps, a.norm, a.norm_nt, a.apply_norm, xs, xn, scratch);

    // workgroup 0 publishes xn and the activation quantisation
    if (e == 0) {
        for (int i = tid; i < d; i += 256) a.xn[i] = xn[i];
        if (a.qk == 0) {
            // Q8 per 32-block (engine_gpt2.rs:691-699): one thread per block
            for (int b = tid; b < d / 32; b += 256) {
                float amax = 1e-12f;
                for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xn[b * 32 + i]));
                float sc = amax / 127.0f;
                a.xsb[b] = sc;
                for (int i = 0; i < 32; i += 4) {
                    uint32_t p = 0;
                    for (int k = 0; k < 4; k++) p |= ((uint32_t)(uint8_t)q8_round(xn[b * 32 + i + k], sc)) << (8 * k);
                    ((uint32_t*)a.xq)[(b * 32 + i) / 4] = p;
                    ((uint32_t*)a.xqn)[(b * 32 + i) / 4] = neg4(p);
                }
            }
        } else {
            // Q8_K per 256 (engine_qwen2.rs:288-300): one wave per superblock
            for (int sb = tid >> 6; sb < d / 256; sb += 4) {
                int l = tid & 63;
                float m = fmaxf(fmaxf(fabsf(xn[sb * 256 + l]), fabsf(xn[sb * 256 + 64 + l])),
                                fmaxf(fabsf(xn[sb * 256 + 128 + l]), fabsf(xn[sb * 256 + 192 + l])));
                float amax = fmaxf(1e-12f, wave_max(m));
                float sc = amax / 127.0f;
                if (l == 0) a.xsb[sb] = sc;
                int qv[4];
                for (int k = 0; k < 4; k++) {
                    qv[k] = q8_round(xn[sb * 256 + 64 * k + l], sc);
                    a.xq[sb * 256 + 64 * k + l] = (int8_t)qv[k];
                    a.xqn[sb * 256 + 64 * k + l] = (int8_t)(-qv[k]);
                }
                // per-32 sums: group g = 2k + (l >= 32)
                for (int k = 0; k < 4; k++) {
                    int s = qv[k];
                    for (int m2 = 16; m2 >= 1; m2 >>= 1) s += __shfl_xor(s, m2);
                    if ((l & 31) == 0) a.xsum[sb * 8 + 2 * k + (l >> 5)] = s;
                }
            }
        }
    }

    // ---- router logit of expert e: fp32 products, exact fp64 sum + bound ----
    const int C = (d + 255) / 256;
    const int j0 = tid * C, j1 = min(d, j0 + C);
    const float* W = a.router_w + (size_t)e * d;
    const double b = a.router_b ? (double)a.router_b[e] : 0.0;
    double loc = 0.0, absp = 0.0;
    for (int j = j0; j < j1; j++) {
        float p = W[j] * xn[j];
        loc += (double)p;
        absp += fabs((double)p);
    }
    // exclusive scan of chunk sums (fixed order: serial over 256 by one thread is
    // too slow; Hillis-Steele in LDS)
    dsc[tid] = loc;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        double v = tid >= off ? dsc[tid - off] : 0.0;
        __syncthreads();
        dsc[tid] += v;
        __syncthreads();
    }
    double start = b + (tid > 0 ? dsc[tid - 1] : 0.0);
    double total = b + dsc[255];
    double sabs = 0.0, run = start;
    for (int j = j0; j < j1; j++) {
        float p = W[j] * xn[j];
        run += (double)p;
        sabs += fabs(run);
    }
    __syncthreads();
    double SS = block_sum(sabs, dred);
    double AP = block_sum(absp, dred);
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
    // ---- last workgroup: rank, certify, softmax ----
    __shared__ int is_last;
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = atomicAdd(a.counter, 1u);
        is_last = (prev == (unsigned)(gridDim.x - 1));
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();

    const int NE = gridDim.x, K = a.top_k;
    double* Ls = dsc;                  // [NE] exact logits   (NE <= 256)
    double* Bs = (double*)xs;          // [NE] bounds         (xs is free now; d >= 3*NE)
    float* lg = (float*)(Bs + NE);     // [NE] fp32 logits
    __shared__ int rank[256];
    __shared__ int slot_of[16];
    __shared__ int ok;
    for (int i = tid; i < NE; i += 256) {
        Ls[i] = __hip_atomic_load(&a.lstar[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        Bs[i] = __hip_atomic_load(&a.lbound[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0) { ok = 1; *a.counter = 0u; }
    __syncthreads();
    for (int i = tid; i < NE; i += 256) {
        int r = 0;
        double v = Ls[i];
        for (int j = 0; j < NE; j++) r += (Ls[j] > v) || (Ls[j] == v && j < i);
        rank[i] = r;
        if (r < K) slot_of[r] = i;
    }
    __syncthreads();
    for (int i = tid; i < NE; i += 256) {
        int r = rank[i];
        if (r < K) {
            double lo = Ls[i] - Bs[i];
            for (int j = 0; j < NE; j++)
                if (rank[j] > r && Ls[j] + Bs[j] >= lo) ok = 0;
        }
    }
    __syncthreads();
    if (ok) {
        for (int i = tid; i < NE; i += 256) lg[i] = (float)Ls[i];
    } else {
        // exact serial router, one thread per expert (engine_gpt2.rs:849-850)
        for (int i = tid; i < NE; i += 256) {
            float acc = a.router_b ? a.router_b[i] : 0.0f;
            const float* Wi = a.router_w + (size_t)i * d;
            for (int j = 0; j < d; j++) acc = __fadd_rn(acc, __fmul_rn(Wi[j], xn[j]));
            lg[i] = acc;
        }
        __syncthreads();
        for (int i = tid; i < NE; i += 256) {
            int r = 0;
            float v = lg[i];
            for (int j = 0; j < NE; j++) r += (lg[j] > v) || (lg[j] == v && j < i);
            if (r < K) slot_of[r] = i;
        }
    }
    __syncthreads();
    for (int i = tid; i < NE; i += 256) a.logits[i] = lg[i];
    if (tid == 0) {
        float tv[16], ex[16], wsum = 0.0f;
        for (int i = 0; i < K; i++) tv[i] = lg[slot_of[i]];
        float lmax = tv[0];
        for (int i = 0; i < K; i++) { ex[i] = expf(tv[i] - lmax); wsum += ex[i]; }
        for (int i = 0; i < K; i++) { a.ids[i] = slot_of[i]; a.wts[i] = ex[i] / wsum; }
        *a.fallback = ok ? 0 : 1;
    }
}

}  // namespace cpb

int cpb::launch_route(const cpb::RouteArgs* a, hipStream_t s) {
    if (a->n_expert > 256 || a->n_expert < a->top_k || a->top_k > 16 || a->d % 32 != 0 || a->d < 3 * a->n_expert) return -22;
    size_t lds = sizeof(float) * (2 * a->d + 32) + sizeof(double) * (256 + 8) + sizeof(float) * 64;
    hipLaunchKernelGGL(cpb::k_route, dim3(a->n_expert), dim3(256), lds, s, *a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}
