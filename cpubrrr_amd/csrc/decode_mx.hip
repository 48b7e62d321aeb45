// decode_mx.hip -- one launch decodes a token through a stack of gpt-oss MoE
// layers (gfx950).
//
// Reference: the MoE stage of forward_worker, engine_gpt2.rs:845-923, run for
// every layer (:767-930).  The reference runs it with 12 persistent CPU
// workers separated by barriers; here every workgroup of the launch is
// resident for the whole call and workgroups hand work to each other through
// phase counters in global memory:
//
//   route (first n_expert down-role workgroups; expert e's logit + bound and
//   a share of the Q8 quantisation)              -> counter R[l] == n_expert
//   select (every workgroup, one wave, LDS rank)  -- no extra hop
//   gate/up tile (T_gu workgroups) + SwiGLU + Q8  -> counter H[l] == T_gu
//   down tile (T_dn workgroups): the down weights are requested right after
//   the selection, so they stream while gate/up is still running; the
//   workgroup then waits for H[l], stages hq and finishes -> counter X[l]
//
// so HBM streams gate/up and down weights back to back and each layer pays
// only the dependency latency route -> gate/up -> down.  All waits are
// bounded: on expiry a flag is raised and the call returns an error instead
// of hanging the device.
#include "decode_mx.h"

#include <algorithm>
#include "moe_mx.h"
#include "mx_dev.h"
#include "route_dev.h"
#include "select.h"

namespace cpb {

constexpr int kThreads = 384;           // 6 waves = 6 k-parts of 15 blocks (K <= 2880)
constexpr int kWaves = kThreads / 64;
constexpr long kSpinLimit = 1L << 20;   // bounded wait (well under 1 s; a legitimate wait is < 100 us)
#ifndef CPB_SPIN_SLEEP
#define CPB_SPIN_SLEEP 2                // s_sleep units (64 cycles) between polls of a counter
#endif

// Data handed between workgroups is written with device-coherent stores
// (st_dev); each wave waits for its stores to complete, then one atomic
// publishes the workgroup's completion.
CPB_DEV void signal_done(unsigned* c) {
    drain_memory();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0 waits (bounded) for *c >= target; consumers then read the handed
// over data with device-coherent loads (ld_dev).
CPB_DEV void wait_ge(const unsigned* c, unsigned target, int32_t* err) {
    if (threadIdx.x == 0) {
        long n = 0;
        while (ld_dev(c) < target) {
            __builtin_amdgcn_s_sleep(CPB_SPIN_SLEEP);
            // a wait that expired anywhere ends every later wait at once
            if (++n > kSpinLimit || ((n & 1023) == 0 && ld_dev(err) != 0)) { st_dev(err, 1); break; }
        }
    }
    __syncthreads();
}

#ifdef CPB_DECODE_STAMPS
#define DSTAMP(i) do { if (threadIdx.x == 0 && a.stamps) a.stamps[((size_t)blockIdx.x * a.n_layers + li) * 8 + (i)] = wall_clock64(); } while (0)
#else
#define DSTAMP(i) do { } while (0)
#endif

// One workgroup = one gate/up tile (32 rows of gate and up of one expert slot,
// engine_gpt2.rs:870-906) and, for workgroups w < T_dn, one down tile (RT
// rows x K experts, :908-922).  Each lane streams a 16-deep window of 16-byte
// weight units into registers; a down-tile owner requests its down units as
// soon as its gate/up work is published, before waiting for the other tiles.
CPB_DEV void layer_tiles(const DecodeArgs& a, const LayerPtrs& Lp, const Selection& sel, int w, unsigned* H,
                         unsigned* X, unsigned char* smem, int li) {
    const int P = a.parts, K = a.k, RT = 64 / K;
    const int lane = threadIdx.x & 63;
    const int q = uniform(threadIdx.x >> 6);
    const bool active = q < P;
    const bool has_dn = w < a.T_dn;
    const int tiles = a.dff / 32;
    const int ei = w / tiles, t = w % tiles;
    const int e = sel.ids[ei];
    const int blk0 = q * kBlkPerPart;

    // ---- gate/up operands: activations (LDS image) and the weight window ----
    uint32_t* xs = (uint32_t*)smem + q * kXsDw;
    float* red = (float*)smem + kWaves * K * kXsDw;
    float* vv = red + kWaves * 64;
    {
        uint32_t xv[4];
        bool ok[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            XsSlot sl = xs_slot((const uint32_t*)a.xq, (const uint32_t*)a.xqn, a.xsb, blk0, a.nb, lane + 64 * k, active);
            xv[k] = ld_dev(sl.p);       // written by the routing workgroups of this launch
            ok[k] = sl.valid;
        }
        u32x4 wv[kUnits];
        if (active) load_part(Lp.gu + ((((size_t)e * tiles + t) * P + q) * kUnits) * 64 + lane, 64, wv);
        else for (int u = 0; u < kUnits; u++) wv[u] = u32x4{0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; k++) xs[lane + 64 * k] = ok[k] ? xv[k] : 0u;
        wave_sync_lds();

        // ---- gate/up compute ----
        const u32x4* xb4 = (const u32x4*)xs;
        const float* sb = (const float*)xs + kBlkPerPart * 16;
        const float acc = part_dot<false>(wv, xb4, sb, nullptr, blk0, a.nb);
        red[q * 64 + lane] = active ? acc : 0.0f;
        __syncthreads();
        const int row = t * 32 + (lane & 31);
        const int isup = lane >> 5;
        if (q == 0) {
            float v = 0.0f;
            for (int p = 0; p < P; p++) v += red[p * 64 + lane];
            if (isup) { if (Lp.up_b) v += Lp.up_b[(size_t)e * a.dff + row]; }
            else      { if (Lp.gate_b) v += Lp.gate_b[(size_t)e * a.dff + row]; }
            const float u = __shfl_down(v, 32);
            float h = 0.0f;
            if (!isup) {
                const float xg = fminf(v, a.limit);
                const float yu = fminf(fmaxf(u, -a.limit), a.limit);
                h = (xg / (1.0f + expf(-a.alpha * xg))) * (yu + 1.0f);
            }
            float m = isup ? 0.0f : fabsf(h);
#pragma unroll
            for (int s = 16; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s));
            const float sc = fmaxf(1e-12f, m) / 127.0f;
            if (!isup) {
                const int8_t qv = q8_round(h, sc);
                st_dev(a.hq + (size_t)ei * a.dff + row, qv);
                st_dev(a.hqn + (size_t)ei * a.dff + row, (int8_t)(-qv));
            }
            if (lane == 0) st_dev(a.hsb + (size_t)ei * (a.dff / 32) + t, sc);
        }
        signal_done(H);
        DSTAMP(5);
        if (!has_dn) return;

        // ---- down: weights requested, then wait for every gate/up tile ----
        const int dei = lane / RT, rr = lane % RT;
        int de = sel.ids[0];
#pragma unroll
        for (int i = 1; i < 4; i++) if (i < K && dei == i) de = sel.ids[i];
        if (active) load_part(Lp.dn + (((((size_t)de * (a.d / RT) + w) * P + q) * kUnits) * RT) + rr, RT, wv);
        wait_ge(H, (unsigned)a.T_gu, a.error);
        DSTAMP(6);
        uint32_t* dxs = (uint32_t*)smem + q * K * kXsDw;
        for (int k0 = 0; k0 < 4 * K; k0 += 4) {
            uint32_t hv[4];
            bool hok[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = lane + 64 * (k0 + k), ex = min(i / kXsDw, K - 1);
                XsSlot sl = xs_slot((const uint32_t*)(a.hq + (size_t)ex * a.dff),
                                    (const uint32_t*)(a.hqn + (size_t)ex * a.dff), a.hsb + (size_t)ex * a.nbf, blk0,
                                    a.nbf, i % kXsDw, active);
                hv[k] = ld_dev(sl.p);   // written by the gate/up tiles of this launch
                hok[k] = sl.valid;
            }
#pragma unroll
            for (int k = 0; k < 4; k++) dxs[lane + 64 * (k0 + k)] = hok[k] ? hv[k] : 0u;
        }
        wave_sync_lds();
        const uint32_t* mine = dxs + dei * kXsDw;
        float dacc = part_dot<false>(wv, (const u32x4*)mine, (const float*)mine + kBlkPerPart * 16, nullptr, blk0, a.nbf);
        red[q * 64 + lane] = active ? dacc : 0.0f;
        __syncthreads();
        if (q == 0) {
            const int drow = w * RT + rr;
            float v = 0.0f;
            for (int p = 0; p < P; p++) v += red[p * 64 + lane];
            if (Lp.down_b) v += Lp.down_b[(size_t)de * a.d + drow];
            vv[lane] = v;
            wave_sync_lds();
            if (lane < RT) {
                // engine_gpt2.rs:911-921: s = x[r]; s += wts[ei] * (dot + b), ei ascending
                float s = ld_dev(a.x + drow);
                for (int k = 0; k < K; k++) s += sel.wts[k] * vv[k * RT + lane];
                st_dev(a.x + drow, s);
            }
        }
        signal_done(X);
    }
}

// One layer for this workgroup.
CPB_DEV void decode_layer(const DecodeArgs& a, int li, Selection& sel,
                                                       unsigned char* smem) {
    const int w = blockIdx.x;
    // routing is done by workgroups that own no down tile (free earliest)
    const bool is_route = w >= a.T_dn && w - a.T_dn < a.ne;
    const int re = w - a.T_dn;
    const LayerPtrs Lp = a.layers[a.layer0 + li];
    unsigned* R = a.sync + 3 * li;
    unsigned* H = R + 1;
    unsigned* X = R + 2;
    DSTAMP(0);
    __shared__ unsigned last_route;
    if (is_route) {
        // warm this workgroup's router row and the norm weights into L2
        // while the previous layer finishes
        {
            const int C = ((a.d + 4 * kThreads - 1) / (4 * kThreads)) * 4, j0 = threadIdx.x * C;
            float warm = 0.0f;
            for (int j = j0; j < j0 + C && j < a.d; j += 4) warm += Lp.router_w[(size_t)re * a.d + j];
            if (Lp.norm_w && (int)threadIdx.x * 4 < a.d) warm += Lp.norm_w[threadIdx.x * 4];
            asm volatile("" :: "v"(warm));
        }
        if (li > 0) wait_ge(R - 1, (unsigned)a.T_dn, a.error);    // x of the previous layer complete
        DSTAMP(1);
        RouteArgs ra{};
        ra.x = a.x; ra.norm_w = Lp.norm_w; ra.router_w = Lp.router_w; ra.router_b = Lp.router_b;
        ra.d = a.d; ra.n_expert = a.ne; ra.top_k = a.k; ra.norm = a.norm; ra.norm_nt = a.norm_nt;
        ra.apply_norm = a.apply_norm; ra.eps = a.eps; ra.qk = 0;
        ra.xn = a.xn; ra.xq = a.xq; ra.xqn = a.xqn; ra.xsb = a.xsb; ra.xsum = nullptr;
        ra.lstar = a.lstar; ra.lbound = a.lbound;
        route_expert(ra, re, a.ne, smem);
        drain_memory();
        __syncthreads();
        if (threadIdx.x == 0)
            last_route = __hip_atomic_fetch_add(R, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)a.ne - 1;
        __syncthreads();
        DSTAMP(2);
        if (last_route) {
            // the last routing workgroup selects once for everyone and
            // publishes ids / weights, then bumps R past ne
            if (threadIdx.x < 64) {
                select_experts_wave(a.lstar, a.lbound, a.ne, a.k, Lp.router_w, Lp.router_b, a.xn, a.d, (double*)smem,
                                    &sel, a.logits);
                const int lane = threadIdx.x;
                if (lane < a.k) {
                    st_dev(a.ids + lane, sel.ids[lane]);
                    st_dev(a.wts + lane, sel.wts[lane]);
                    a.logits[sel.ids[lane]] = sel.logit[lane];
                }
                if (lane == 0) a.fallback[0] = sel.fallback;
#ifdef CPB_DECODE_STAMPS
                if (a.stamps && lane < a.k) {
                    a.stamps[(size_t)1 << 20 | (li * 16 + lane)] = (unsigned long long)sel.ids[lane];
                    a.stamps[(size_t)1 << 20 | (li * 16 + 8 + lane)] = __float_as_uint(sel.wts[lane]);
                }
#endif
            }
            signal_done(R);
        }
    }
    wait_ge(R, (unsigned)a.ne + 1, a.error);
    DSTAMP(3);
    if (threadIdx.x < 8) {
        // every workgroup reads the published selection
        const int i = threadIdx.x < a.k ? threadIdx.x : 0;
        sel.ids[threadIdx.x] = ld_dev(a.ids + i);
        sel.wts[threadIdx.x] = ld_dev(a.wts + i);
    }
    __syncthreads();
#ifdef CPB_DECODE_STAMPS
    if (a.stamps && li == 0 && threadIdx.x < a.k && w < 512)
        a.stamps[((size_t)1 << 20) + 2048 + w * 4 + threadIdx.x] = (unsigned long long)sel.ids[threadIdx.x];
#endif
    DSTAMP(4);
    layer_tiles(a, Lp, sel, w, H, X, smem, li);
    __syncthreads();
    DSTAMP(7);
}

__global__ __launch_bounds__(kThreads, 4) void k_decode_mx(const DecodeArgs* __restrict__ pa) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Selection sel;
    const int nl = pa->n_layers;
    for (int li = 0; li < nl; li++) {
        // an opaque copy of the argument pointer per layer keeps the compiler
        // from hoisting per-layer values across the loop (register pressure
        // decides how many workgroups are co-resident)
        const DecodeArgs* p = pa;
        asm volatile("" : "+s"(p));
        decode_layer(*p, li, sel, smem);
    }
    const DecodeArgs& a = *pa;
    // every workgroup is past its last wait: the last one to finish re-arms the counters
    if (threadIdx.x == 0) {
        unsigned* done = a.sync + 3 * a.n_layers;
        const unsigned prev = __hip_atomic_fetch_add(done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == gridDim.x - 1) {
            for (int i = 0; i <= 3 * a.n_layers; i++)
                __hip_atomic_store(a.sync + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

int decode_mx_grid(int d, int dff, int k) { return k * (dff / 32); }

int launch_decode_mx(const DecodeArgs& a, const DecodeArgs* dev_args, hipStream_t s) {
    // the grid is the gate/up tiles; the first T_dn of them also own a down
    // tile, and n_expert of the others do the routing
    if (a.parts > kThreads / 64 || a.d > 4096 || (a.k != 1 && a.k != 2 && a.k != 4) || a.ne > 256 ||
        a.dff % 32 || a.d % (64 / a.k) || a.T_dn > a.T_gu || a.T_gu - a.T_dn < a.ne)
        return -22;
    const int G = a.T_gu;
    size_t lds = route_lds_bytes(a.d);
    const size_t gu_lds = sizeof(uint32_t) * kWaves * kXsDw + sizeof(float) * kWaves * 64;
    const size_t dn_lds = sizeof(uint32_t) * kWaves * a.k * kXsDw + sizeof(float) * (kWaves * 64 + 64);
    const size_t sel_lds = sizeof(double) * 4 * a.ne + sizeof(float) * a.d + 64;
    lds = std::max(std::max(lds, gu_lds), std::max(dn_lds, sel_lds));
    int dev = 0, ncu = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_mx, kThreads, lds) != hipSuccess)
        return -19;
    // The occupancy query does not model how a workgroup's waves land on a
    // CU's 4 SIMDs: with kWaves = 6 the worst placement puts 2 waves of each
    // workgroup on one SIMD.  Require that many waves per SIMD for every
    // co-resident workgroup the count below relies on (register file: 512
    // VGPRs per lane per SIMD).
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, (const void*)k_decode_mx) != hipSuccess) return -19;
    const int regs = fa.numRegs > 0 ? fa.numRegs : 512;
    const int waves_per_simd = 512 / ((regs + 7) / 8 * 8);
    const int worst_per_wg = (kWaves + 3) / 4;
    const int safe_per_cu = std::min(per_cu, waves_per_simd / worst_per_wg);
    if ((long)safe_per_cu * ncu < G) return -28;
    hipLaunchKernelGGL(k_decode_mx, dim3(G), dim3(kThreads), lds, s, dev_args);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
