// moe_mx.hip -- gpt-oss MoE expert GEMVs over MXFP4 (gfx950), batch-1 decode.
//
// Reference: gate/up stage engine_gpt2.rs:870-884, SwiGLU-OAI + Q8
// :887-906, down + weighted residual :908-922, kernel dot4_mx_i8 :194-228,
// weight repack repack_mx :439-461.
//
// HBM layout ("stream layout", built at load time by k_repack_*): a matrix is
// cut into row tiles; a tile's K (= nb 32-blocks) is cut into P k-parts of 15
// blocks.  For each (tile, k-part) the data is 16 units x R lanes x 16 B:
// unit 0 holds the 15 e8m0 bytes of the k-part's blocks (+1 pad byte),
// units 1..15 hold one 32-block's 16 nibble bytes for each of the R rows.  One
// wavefront load instruction therefore reads R*16 contiguous bytes (R = 64
// for gate/up: 1 KB; R = 64/top_k for down: 16 lanes x 16 B per expert), and
// a lane's whole k-part is 16 dwordx4 loads issued back to back.
//
//   gate/up: tile = 32 rows of gate + the same 32 rows of up of one expert
//            (lanes 0-31 gate, 32-63 up) so SwiGLU and the per-32 Q8 of h
//            finish inside the workgroup.
//   down:    tile = 64/top_k rows x top_k active experts, so the weighted
//            combine over experts (ascending slot order) finishes inside the
//            workgroup and writes x directly.
//
// A workgroup has P wavefronts (one per k-part), each lane owns one row-dot
// and accumulates its 15 blocks: int32 block sum via v_perm decode + sdot4,
// one float conversion per block, fma with 2^(e-128)*xsb.  The P partial sums
// are added in fixed order (deterministic).  Batch-1 decode is HBM-bound:
// no MFMA here.
#include "moe_common.h"
#include "moe_mx.h"
#include "mx_dev.h"

#include <algorithm>

namespace cpb {

#ifdef CPB_DECODE_STAMPS
#define GSTAMP(i) do { if (threadIdx.x == 0 && a.stamps) a.stamps[((size_t)1 << 18) + blockIdx.x * 8 + (i)] = wall_clock64(); } while (0)
#else
#define GSTAMP(i) do { } while (0)
#endif

template <bool TRACE>
__global__ __launch_bounds__(64 * kMaxParts) void k_gateup_mx(GateUpArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    GSTAMP(0);
    const int P = a.nparts;
    const int lane = threadIdx.x & 63;
    const int q = uniform(threadIdx.x >> 6);
    const int tiles = a.dff / 32;
    const int ei = blockIdx.x / tiles, t = blockIdx.x % tiles;
    uint32_t* xs = (uint32_t*)smem + q * kXsDw;
    float* red = (float*)smem + P * kXsDw;                     // [P][64]
    const int blk0 = q * kBlkPerPart;

    // activations first: waiting for them must not wait for the weights
    uint32_t xv[4];
    bool ok[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        XsSlot sl = xs_slot((const uint32_t*)a.xq, (const uint32_t*)a.xqn, a.xsb, blk0, a.nb, lane + 64 * k, true);
        xv[k] = *sl.p;
        ok[k] = sl.valid;
    }
    // expert of this tile: selected here by wave 0 from the certified logits
    // (LDS scratch aliases the activation image, which is written later)
    int e;
    if (a.sel.lstar) {
        __shared__ Selection ssel;
        if (q == 0) select_topk_wave(a.sel, smem, &ssel);
        GSTAMP(1);
        __syncthreads();
        e = ssel.ids[ei];
    } else {
        e = a.ids[ei];
    }
    u32x4 wv[kUnits];
    load_part(a.w + ((((size_t)e * tiles + t) * P + q) * kUnits) * 64 + lane, 64, wv);
    // the epilogue's bias, requested now (behind the weights) instead of
    // after the reduction
    const float* bias = (lane >> 5) ? a.up_b : a.gate_b;
    float bias_pf = 0.0f;
    if (q == 0 && bias) bias_pf = bias[(size_t)e * a.dff + t * 32 + (lane & 31)];
#pragma unroll
    for (int k = 0; k < 4; k++) xs[lane + 64 * k] = ok[k] ? xv[k] : 0u;
    wave_sync_lds();
    GSTAMP(2);

    const int row = t * 32 + (lane & 31);
    const int isup = lane >> 5;                                // lanes 0-31 gate, 32-63 up
    int32_t* so = nullptr;
    if (TRACE) so = a.gu_sums + (((size_t)(ei * 2 + isup) * a.dff + row) * a.nb + blk0);
    float acc = part_dot<TRACE>(wv, (const u32x4*)xs, (const float*)xs + kBlkPerPart * 16, so, blk0, a.nb);

    red[q * 64 + lane] = acc;
    GSTAMP(3);
    __syncthreads();
    if (q != 0) return;
    float v = 0.0f;
    for (int p = 0; p < P; p++) v += red[p * 64 + lane];
    if (bias) v += bias_pf;
    if (TRACE) a.gu[(size_t)(ei * 2 + isup) * a.dff + row] = v;
    // SwiGLU-OAI (engine_gpt2.rs:887-906) in lanes 0-31: gate row r, up row r from lane r+32
    float u = __shfl_down(v, 32);
    float h = 0.0f;
    if (!isup) {
        float xg = fminf(v, a.limit);
        float yu = fminf(fmaxf(u, -a.limit), a.limit);
        h = (xg / (1.0f + expf(-a.alpha * xg))) * (yu + 1.0f);
    }
    float m = isup ? 0.0f : fabsf(h);
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s));
    float sc = fmaxf(1e-12f, m) / 127.0f;
    if (!isup) {
        int8_t qv = q8_round(h, sc);
        a.hq[(size_t)ei * a.dff + row] = qv;
        a.hqn[(size_t)ei * a.dff + row] = (int8_t)(-qv);
        if (TRACE) a.h[(size_t)ei * a.dff + row] = h;
    }
    if (lane == 0) a.hsb[(size_t)ei * (a.dff / 32) + t] = sc;
    GSTAMP(4);
}

template <bool TRACE>
__global__ __launch_bounds__(64 * kMaxParts) void k_down_mx(DownArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int P = a.nparts, K = a.top_k, RT = 64 / K;
    const int lane = threadIdx.x & 63;
    const int q = uniform(threadIdx.x >> 6);
    const int tiles = a.d / RT, t = blockIdx.x;
    const int ei = lane / RT, rr = lane % RT, row = t * RT + rr;
    // expert of this lane's slot from wave-uniform (scalar) loads of ids
    int es[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        es[k] = __builtin_amdgcn_readfirstlane(a.ids[k < K ? k : 0]);
    }
    const int e = ei == 0 ? es[0] : ei == 1 ? es[1] : ei == 2 ? es[2] : es[3];
    uint32_t* xs = (uint32_t*)smem + q * K * kXsDw;           // [K][256]
    float* red = (float*)smem + P * K * kXsDw;                 // [P][64]
    float* vv = red + P * 64;                                  // [64]
    const int blk0 = q * kBlkPerPart;

    // activations of all K expert slots (hq is [K][dff]), before the weights
    uint32_t xv[16];
    bool ok[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        int i = lane + 64 * k, ex = min(i / kXsDw, K - 1);
        XsSlot sl = xs_slot((const uint32_t*)(a.hq + (size_t)ex * a.dff), (const uint32_t*)(a.hqn + (size_t)ex * a.dff),
                            a.hsb + (size_t)ex * a.nbf, blk0, a.nbf, i % kXsDw, i < K * kXsDw);
        xv[k] = *sl.p;
        ok[k] = sl.valid;
    }
    u32x4 wv[kUnits];
    load_part(a.w + (((((size_t)e * tiles + t) * P + q) * kUnits) * RT) + rr, RT, wv);
    // the epilogue's operands (bias, residual, slot weights), requested now
    // (behind the weights) instead of after the reduction
    float dnb_pf = 0.0f, x_pf = 0.0f, w_pf[4];
    if (q == 0) {
        if (a.down_b) dnb_pf = a.down_b[(size_t)e * a.d + row];
        if (lane < RT) x_pf = a.x[row];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) w_pf[k] = a.wts[k < K ? k : 0];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        int i = lane + 64 * k;
        if (i < K * kXsDw) xs[i] = ok[k] ? xv[k] : 0u;
    }
    wave_sync_lds();

    const uint32_t* mine = xs + ei * kXsDw;
    int32_t* so = nullptr;
    if (TRACE) so = a.dn_sums + (((size_t)ei * a.d + row) * a.nbf + blk0);
    float acc = part_dot<TRACE>(wv, (const u32x4*)mine, (const float*)mine + kBlkPerPart * 16, so, blk0, a.nbf);

    red[q * 64 + lane] = acc;
    __syncthreads();
    if (q != 0) return;
    float v = 0.0f;
    for (int p = 0; p < P; p++) v += red[p * 64 + lane];
    if (a.down_b) v += dnb_pf;
    if (TRACE) a.dn[(size_t)ei * a.d + row] = v;
    vv[lane] = v;
    wave_sync_lds();
    if (lane < RT) {
        // engine_gpt2.rs:911-921: s = x[r]; s += wts[ei] * (dot + b), ei ascending
        float s = x_pf;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (k < K) s += w_pf[k] * vv[k * RT + lane];
        a.x[row] = s;
    }
}

// ---- gate/up and down in one launch (batch-1 decode) ----
// Workgroups [0, T_gu) are the gate/up tiles of k_gateup_mx; workgroups
// [T_gu, T_gu + T_dn) are the down tiles of k_down_mx.  A down tile requests
// its weights at once (the routed ids are known before the launch), so the
// down stream overlaps the gate/up stream, then waits until every gate/up
// tile has published its slice of hq (counter sync[0]) and finishes as
// k_down_mx does.  The waits are only on lower-indexed workgroups, which the
// dispatcher places first (in order per XCD) and which never wait: no
// co-residency is assumed.  The last down tile re-arms both counters.
// Arithmetic and summation order are those of the two kernels above, so x is
// bit-identical to the two-launch path.
constexpr long kLayerSpin = 1L << 22;        // bounded wait (~0.3 s): a legitimate wait is a few us

__global__ __launch_bounds__(64 * kMaxParts) void k_layer_mx(GateUpArgs g, DownArgs a, unsigned* sync, int32_t* err,
                                                   unsigned long long* stamps) {
    extern __shared__ __align__(16) unsigned char smem[];
#ifdef CPB_DECODE_STAMPS
#define LSTAMP(i) do { if (threadIdx.x == 0 && stamps) stamps[((size_t)1 << 19) + blockIdx.x * 4 + (i)] = wall_clock64(); } while (0)
#else
#define LSTAMP(i) do { (void)stamps; } while (0)
#endif
    LSTAMP(0);
    const int P = a.nparts;
    const int lane = threadIdx.x & 63;
    const int q = uniform(threadIdx.x >> 6);
    const int T_gu = g.top_k * (g.dff / 32);
    const int blk0 = q * kBlkPerPart;
    if ((int)blockIdx.x < T_gu) {
        // ---------------- gate/up tile (k_gateup_mx) ----------------
        const int tiles = g.dff / 32;
        const int ei = blockIdx.x / tiles, t = blockIdx.x % tiles;
        const int e = g.ids[ei];
        uint32_t* xs = (uint32_t*)smem + q * kXsDw;
        float* red = (float*)smem + P * kXsDw;
        uint32_t xv[4];
        bool ok[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            XsSlot sl = xs_slot((const uint32_t*)g.xq, (const uint32_t*)g.xqn, g.xsb, blk0, g.nb, lane + 64 * k, true);
            xv[k] = *sl.p;
            ok[k] = sl.valid;
        }
        u32x4 wv[kUnits];
        load_part(g.w + ((((size_t)e * tiles + t) * P + q) * kUnits) * 64 + lane, 64, wv);
        const float* bias = (lane >> 5) ? g.up_b : g.gate_b;
        float bias_pf = 0.0f;
        if (q == 0 && bias) bias_pf = bias[(size_t)e * g.dff + t * 32 + (lane & 31)];
#pragma unroll
        for (int k = 0; k < 4; k++) xs[lane + 64 * k] = ok[k] ? xv[k] : 0u;
        wave_sync_lds();
        const int row = t * 32 + (lane & 31);
        const int isup = lane >> 5;
        float acc = part_dot<false>(wv, (const u32x4*)xs, (const float*)xs + kBlkPerPart * 16, nullptr, blk0, g.nb);
        red[q * 64 + lane] = acc;
        __syncthreads();
        if (q == 0) {
            float v = 0.0f;
            for (int p = 0; p < P; p++) v += red[p * 64 + lane];
            if (bias) v += bias_pf;
            float u = __shfl_down(v, 32);
            float h = 0.0f;
            if (!isup) {
                float xg = fminf(v, g.limit);
                float yu = fminf(fmaxf(u, -g.limit), g.limit);
                h = (xg / (1.0f + expf(-g.alpha * xg))) * (yu + 1.0f);
            }
            float m = isup ? 0.0f : fabsf(h);
#pragma unroll
            for (int s = 16; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s));
            float sc = fmaxf(1e-12f, m) / 127.0f;
            if (!isup) {
                int8_t qv = q8_round(h, sc);
                st_dev(g.hq + (size_t)ei * g.dff + row, qv);
                st_dev(g.hqn + (size_t)ei * g.dff + row, (int8_t)(-qv));
            }
            if (lane == 0) st_dev(g.hsb + (size_t)ei * (g.dff / 32) + t, sc);
            drain_memory();
        }
        __syncthreads();
        LSTAMP(1);
        if (threadIdx.x == 0) __hip_atomic_fetch_add(&sync[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        LSTAMP(2);
        return;
    }
    // ---------------- down tile (k_down_mx) ----------------
    const int K = a.top_k, RT = 64 / K;
    const int tiles = a.d / RT, t = blockIdx.x - T_gu;
    const int ei = lane / RT, rr = lane % RT, row = t * RT + rr;
    int es[4];
#pragma unroll
    for (int k = 0; k < 4; k++) es[k] = __builtin_amdgcn_readfirstlane(a.ids[k < K ? k : 0]);
    const int e = ei == 0 ? es[0] : ei == 1 ? es[1] : ei == 2 ? es[2] : es[3];
    uint32_t* xs = (uint32_t*)smem + q * K * kXsDw;
    float* red = (float*)smem + P * K * kXsDw;
    float* vv = red + P * 64;
    u32x4 wv[kUnits];
    load_part(a.w + (((((size_t)e * tiles + t) * P + q) * kUnits) * RT) + rr, RT, wv);
    float dnb_pf = 0.0f, x_pf = 0.0f, w_pf[4];
    if (q == 0) {
        if (a.down_b) dnb_pf = a.down_b[(size_t)e * a.d + row];
        if (lane < RT) x_pf = a.x[row];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) w_pf[k] = a.wts[k < K ? k : 0];
    __shared__ int bad;
    if (threadIdx.x == 0) {
        long n = 0;
        int b = 0;
        while (ld_dev(&sync[0]) < (unsigned)T_gu) {
            __builtin_amdgcn_s_sleep(1);
            if (++n > kLayerSpin) { b = 1; break; }
        }
        bad = b;
    }
    __syncthreads();
    LSTAMP(1);
    // hq of all K slots, written by the gate/up tiles of this launch
    uint32_t xv[16];
    bool ok[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        int i = lane + 64 * k, ex = min(i / kXsDw, K - 1);
        XsSlot sl = xs_slot((const uint32_t*)(a.hq + (size_t)ex * a.dff), (const uint32_t*)(a.hqn + (size_t)ex * a.dff),
                            a.hsb + (size_t)ex * a.nbf, blk0, a.nbf, i % kXsDw, i < K * kXsDw);
        xv[k] = i < K * kXsDw ? ld_dev(sl.p) : 0u;
        ok[k] = sl.valid;
    }
#pragma unroll
    for (int k = 0; k < 16; k++) {
        int i = lane + 64 * k;
        if (i < K * kXsDw) xs[i] = ok[k] ? xv[k] : 0u;
    }
    wave_sync_lds();
    const uint32_t* mine = xs + ei * kXsDw;
    float acc = part_dot<false>(wv, (const u32x4*)mine, (const float*)mine + kBlkPerPart * 16, nullptr, blk0, a.nbf);
    red[q * 64 + lane] = acc;
    __syncthreads();
    if (q == 0) {
        float v = 0.0f;
        for (int p = 0; p < P; p++) v += red[p * 64 + lane];
        if (a.down_b) v += dnb_pf;
        vv[lane] = v;
        wave_sync_lds();
        if (lane < RT) {
            float s = x_pf;
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (k < K) s += w_pf[k] * vv[k * RT + lane];
            a.x[row] = s;
        }
        LSTAMP(2);
        if (lane == 0) {
            if (bad) st_dev(err, 1);
            // the last down tile re-arms the counters for the next launch
            if (__hip_atomic_fetch_add(&sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)tiles - 1) {
                st_dev(&sync[0], 0u);
                st_dev(&sync[1], 0u);
            }
        }
    }
}

// ---- load-time re-layout from native GGUF MXFP4 rows (17-byte blocks) ----
// One thread per 16-byte output unit.
__global__ void k_repack_gateup(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                u32x4* __restrict__ out, int ne, int dff, int nb, int P) {
    size_t tiles = dff / 32;
    size_t total = (size_t)ne * tiles * P * kUnits * 64;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        int lane = idx % 64;
        size_t r1 = idx / 64;
        int u = r1 % kUnits; r1 /= kUnits;
        int q = r1 % P; r1 /= P;
        int t = r1 % tiles;
        int e = (int)(r1 / tiles);
        int row = t * 32 + (lane & 31);
        const uint8_t* src = (lane < 32 ? gate : up) + ((size_t)e * dff + row) * nb * 17;
        uint8_t b[16];
        if (u > 0) {
            int blk = q * kBlkPerPart + u - 1;
            for (int i = 0; i < 16; i++) b[i] = blk < nb ? src[(size_t)blk * 17 + 1 + i] : 0;
        } else {
            for (int i = 0; i < 16; i++) {
                int blk = q * kBlkPerPart + i;
                b[i] = (i < kBlkPerPart && blk < nb) ? src[(size_t)blk * 17] : 0;
            }
        }
        u32x4 o;
        o[0] = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
        o[1] = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
        o[2] = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
        o[3] = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
        out[idx] = o;
    }
}

__global__ void k_repack_down(const uint8_t* __restrict__ down, u32x4* __restrict__ out, int ne, int d, int nbf,
                              int P, int RT) {
    size_t tiles = d / RT;
    size_t total = (size_t)ne * tiles * P * kUnits * RT;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        int rr = idx % RT;
        size_t r1 = idx / RT;
        int u = r1 % kUnits; r1 /= kUnits;
        int q = r1 % P; r1 /= P;
        int t = r1 % tiles;
        int e = (int)(r1 / tiles);
        int row = t * RT + rr;
        const uint8_t* src = down + ((size_t)e * d + row) * nbf * 17;
        uint8_t b[16];
        if (u > 0) {
            int blk = q * kBlkPerPart + u - 1;
            for (int i = 0; i < 16; i++) b[i] = blk < nbf ? src[(size_t)blk * 17 + 1 + i] : 0;
        } else {
            for (int i = 0; i < 16; i++) {
                int blk = q * kBlkPerPart + i;
                b[i] = (i < kBlkPerPart && blk < nbf) ? src[(size_t)blk * 17] : 0;
            }
        }
        u32x4 o;
        o[0] = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
        o[1] = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
        o[2] = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
        o[3] = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
        out[idx] = o;
    }
}

size_t mx_gateup_bytes(int ne, int dff, int nb) {
    int P = (nb + kBlkPerPart - 1) / kBlkPerPart;
    return (size_t)ne * (dff / 32) * P * kUnits * 64 * 16;
}
size_t mx_down_bytes(int ne, int d, int nbf, int top_k) {
    int P = (nbf + kBlkPerPart - 1) / kBlkPerPart;
    int RT = 64 / top_k;
    return (size_t)ne * (d / RT) * P * kUnits * RT * 16;
}

// Count MXFP4 blocks whose e8m0 byte the matrix-core path cannot scale exactly
// (e < 32: tbl[0] = 0 and subnormal scales; e == 255: NaN in hardware).
__global__ void k_count_special_exps(const uint8_t* __restrict__ raw, size_t nblocks, unsigned* out) {
    unsigned c = 0;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < nblocks; i += (size_t)gridDim.x * blockDim.x) {
        const uint8_t e = raw[i * 17];
        c += (e < 32 || e == 255) ? 1u : 0u;
    }
    if (c) atomicAdd(out, c);
}
int launch_count_special_exps(const uint8_t* raw, size_t nblocks, unsigned* out, hipStream_t s) {
    hipLaunchKernelGGL(k_count_special_exps, dim3(1024), dim3(256), 0, s, raw, nblocks, out);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_repack_gateup(const uint8_t* gate, const uint8_t* up, u32x4* out, int ne, int dff, int nb, hipStream_t s) {
    int P = (nb + kBlkPerPart - 1) / kBlkPerPart;
    hipLaunchKernelGGL(k_repack_gateup, dim3(4096), dim3(256), 0, s, gate, up, out, ne, dff, nb, P);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}
int launch_repack_down(const uint8_t* down, u32x4* out, int ne, int d, int nbf, int top_k, hipStream_t s) {
    int P = (nbf + kBlkPerPart - 1) / kBlkPerPart;
    hipLaunchKernelGGL(k_repack_down, dim3(4096), dim3(256), 0, s, down, out, ne, d, nbf, P, 64 / top_k);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_gateup_mx(const GateUpArgs& a, bool trace, hipStream_t s) {
    int P = a.nparts;
    if (P < 1 || P > kMaxParts || a.dff % 32 != 0) return -22;
    size_t lds = sizeof(uint32_t) * P * kXsDw + sizeof(float) * P * 64;
    if (a.sel.lstar) lds = std::max(lds, select_lds_bytes(a.sel.ne, a.sel.d));
    dim3 grid(a.top_k * (a.dff / 32)), block(64 * P);
    if (trace) launch(k_gateup_mx<true>, grid, block, lds, s, a);
    else launch(k_gateup_mx<false>, grid, block, lds, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_layer_mx(const GateUpArgs& g, const DownArgs& a, unsigned* sync, int32_t* err, unsigned long long* stamps,
                    hipStream_t s) {
    int P = a.nparts, K = a.top_k;
    if (P < 1 || P > kMaxParts || P != g.nparts || g.dff % 32 != 0 || (K != 1 && K != 2 && K != 4) || a.d % (64 / K) != 0)
        return -22;
    size_t lds_gu = sizeof(uint32_t) * P * kXsDw + sizeof(float) * P * 64;
    size_t lds_dn = sizeof(uint32_t) * P * K * kXsDw + sizeof(float) * (P * 64 + 64);
    dim3 grid(g.top_k * (g.dff / 32) + a.d / (64 / K)), block(64 * P);
    launch(k_layer_mx, grid, block, lds_gu > lds_dn ? lds_gu : lds_dn, s, g, a, sync, err, stamps);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_down_mx(const DownArgs& a, bool trace, hipStream_t s) {
    int P = a.nparts, K = a.top_k;
    if (P < 1 || P > kMaxParts || (K != 1 && K != 2 && K != 4) || a.d % (64 / K) != 0) return -22;
    size_t lds = sizeof(uint32_t) * P * K * kXsDw + sizeof(float) * (P * 64 + 64);
    dim3 grid(a.d / (64 / K)), block(64 * P);
    if (trace) launch(k_down_mx<true>, grid, block, lds, s, a);
    else launch(k_down_mx<false>, grid, block, lds, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
