// moe_kq.hip -- Qwen3 MoE expert GEMVs over Q4_K / Q6_K superblocks (gfx950),
// batch-1 decode.
//
// Reference: engine_qwen2.rs:414-418 (gate/up + SiLU*up), :423 (Q8_K of h),
// :425-432 (down + weighted accumulate, ascending slot order), superblock
// dots q4k_dot :84-114 and q6k_dot :164-200, type dispatch :202-213.
//
// Every row dot is a serial fp32 sum over superblocks of one float term per
// superblock, t_sb = ys*d*sumi - ys*dmin*mint (Q4_K) or ys*d*acc (Q6_K), the
// integer parts summed exactly.  Here one lane computes the term of one
// (row, superblock) with the same float operations, and a final lane adds
// the terms in superblock order, so the row results are the reference's bit
// for bit.
//
// HBM layout ("stream layout", k_repack_kq_*): a superblock is cut into
// 16-byte units (Q4_K: 144 B = 9 units; Q6_K: its first 208 B = 13 units,
// the fp16 d in a separate stream behind them, RT rows contiguous).
//   gate/up: tile = 16 rows of gate + the same 16 rows of up of one expert;
//            for each (expert, tile, superblock): units x 32 lanes x 16 B,
//            lanes 0-15 gate, 16-31 up.  A wave handles two superblocks
//            (lanes 0-31 and 32-63): one load instruction reads 2 x 512 B.
//   down:    tile = RT = 64/top_k rows; for each (expert, tile, superblock):
//            units x RT lanes x 16 B.  A workgroup covers RT rows of all
//            top_k active experts (lane = slot * RT + row), one wave per
//            superblock, so the weighted combine finishes in the workgroup.
// The down workgroups each re-derive the Q8_K quantisation of h (a 256-block
// spans 16 gate/up workgroups) from hbuf with the reference's operations.
#include "moe_common.h"
#include "moe_kq.h"
#include "route_dev.h"

#include <algorithm>

namespace cpb {

constexpr int kXsPad = 272;      // LDS bytes per 256-activation superblock (256 + 16: bank spread)

// Q4_K superblock term of one row (engine_qwen2.rs:84-114).  u: the 9 units
// (u[0] = d, dmin, 12 packed scale/min bytes; u[1..8] = qs[128]); xs: the 256
// int8 activations of the superblock (LDS, 16-aligned); xsum8: their 8 int32
// sums per 32; ys: their scale.  sums (TRACE): {sumi, mint}.
template <bool TRACE>
CPB_DEV float q4k_term(const u32x4 (&u)[kQ4Units], const int8_t* xs, const int32_t* xsum8, float ys, int32_t* sums) {
    const float d = half_bits(u[0][0] & 0xffffu), dmin = half_bits(u[0][0] >> 16);
    // scale bytes q[0..11] = bytes 4..15 of unit 0 (ggml get_scale_min_k4, :59-74)
    const uint32_t q03 = u[0][1], q47 = u[0][2], q811 = u[0][3];
    int sc[8], mn[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        sc[j] = (q03 >> (8 * j)) & 63;
        mn[j] = (q47 >> (8 * j)) & 63;
        const uint32_t qj4 = (q811 >> (8 * j)) & 0xff;      // q[j + 8]
        sc[4 + j] = (qj4 & 0xf) | (((q03 >> (8 * j + 6)) & 3) << 4);
        mn[4 + j] = (qj4 >> 4) | (((q47 >> (8 * j + 6)) & 3) << 4);
    }
    const u32x4* xv = (const u32x4*)xs;
    int sumi = 0;
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const u32x4 w0 = u[1 + 2 * jj], w1 = u[2 + 2 * jj];
        const uint32_t w[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
        const u32x4 a0 = xv[4 * jj + 0], a1 = xv[4 * jj + 1];   // sub-block 2jj   (32 B)
        const u32x4 b0 = xv[4 * jj + 2], b1 = xv[4 * jj + 3];   // sub-block 2jj+1 (32 B)
        const uint32_t xa[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        const uint32_t xb[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = sdot4(w[i] & 0x0F0F0F0Fu, xa[i], s0);
            s1 = sdot4((w[i] >> 4) & 0x0F0F0F0Fu, xb[i], s1);
        }
        sumi += mul24(s0, sc[2 * jj]) + mul24(s1, sc[2 * jj + 1]);
    }
    int mint = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) mint += mul24(mn[j], xsum8[j]);
    if (TRACE) { sums[0] = sumi; sums[1] = mint; }
    return ys * d * (float)sumi - ys * dmin * (float)mint;
}

// Q6_K superblock term of one row (engine_qwen2.rs:164-200).  u: 14 units in registers
// (ql[128] = u[0..7], qh[64] = u[8..11], int8 scales[16] = u[12], fp16 d in
// u[13]); xs: 256 int8 activations; xs16: their 16 int32 sums per 16.
// q - 32 is folded as dot(q, x) - 32 * sum(x) (an exact integer identity).
template <bool TRACE>
CPB_DEV float q6k_term(const u32x4 (&u)[kQ6Units], const int8_t* xs, const int32_t* xs16, float ys, int32_t* sums) {
    const float d = half_bits(u[13][0] & 0xffffu);
    const uint32_t* ql = (const uint32_t*)&u[0];
    const uint32_t* qh = (const uint32_t*)&u[8];
    const uint32_t* scw = (const uint32_t*)&u[12];
    const uint32_t* xw = (const uint32_t*)xs;
    int s[16];
#pragma unroll
    for (int g = 0; g < 16; g++) s[g] = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int l4 = 0; l4 < 8; l4++) {
            const uint32_t A = ql[h * 16 + l4], B = ql[h * 16 + 8 + l4], H = qh[h * 8 + l4];
            const uint32_t t0 = (A & 0x0F0F0F0Fu) | ((H & 0x03030303u) << 4);
            const uint32_t t1 = (B & 0x0F0F0F0Fu) | (((H >> 2) & 0x03030303u) << 4);
            const uint32_t t2 = ((A >> 4) & 0x0F0F0F0Fu) | (((H >> 4) & 0x03030303u) << 4);
            const uint32_t t3 = ((B >> 4) & 0x0F0F0F0Fu) | (((H >> 6) & 0x03030303u) << 4);
            const int hi = l4 >= 4 ? 1 : 0;          // element l = 4*l4 lies in the second 16 of its 32
            const int e0 = h * 128 + 4 * l4;         // first element of t0's 4
            s[h * 8 + 0 + hi] = sdot4(t0, xw[(e0 + 0) / 4], s[h * 8 + 0 + hi]);
            s[h * 8 + 2 + hi] = sdot4(t1, xw[(e0 + 32) / 4], s[h * 8 + 2 + hi]);
            s[h * 8 + 4 + hi] = sdot4(t2, xw[(e0 + 64) / 4], s[h * 8 + 4 + hi]);
            s[h * 8 + 6 + hi] = sdot4(t3, xw[(e0 + 96) / 4], s[h * 8 + 6 + hi]);
        }
    }
    int acc = 0;
#pragma unroll
    for (int g = 0; g < 16; g++) {
        const int sc = (int)(int8_t)(scw[g / 4] >> (8 * (g % 4)));
        acc += mul24(s[g] - 32 * xs16[g], sc);
    }
    if (TRACE) sums[0] = acc;
    return ys * d * (float)acc;
}

// ---- gate/up + SiLU * up ----
// grid: top_k * dff/16 workgroups; block: 64 * ceil(nsb/2) threads.
template <bool TRACE>
__global__ __launch_bounds__(1024) void k_gateup_kq(KqArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nsb = a.d / 256, T = a.dff / 16;
    const int lane = threadIdx.x & 63, q = uniform((int)(threadIdx.x >> 6));
    const int nth = blockDim.x;
    const int ei = blockIdx.x / T, t = blockIdx.x % T;
    int8_t* xl = (int8_t*)smem;                                  // [nsb][kXsPad]
    int32_t* xsl = (int32_t*)(smem + nsb * kXsPad);              // [nsb * 8]
    float* ysl = (float*)(xsl + nsb * 8);                        // [nsb]
    float* part = ysl + 32;                                      // [nsb][32]

    // the selection's intervals (more than 64 experts: one per thread), then
    // the activations (buffer loads; out of range reads zero)
    const bool ranked = a.sel.lstar && a.sel.ne > 64 && a.sel.ne <= (int)blockDim.x;
    SelectPre pre{0.0, 0.0};
    if (ranked) pre = select_preload_wg(a.sel);
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.xq, (uint32_t)a.d);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.xsum, (uint32_t)a.d / 8);
    const __amdgpu_buffer_rsrc_t ry = buf_rsrc(a.xs, (uint32_t)nsb * 4);
    u32x4 xv[2];
#pragma unroll
    for (int k = 0; k < 2; k++) xv[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(threadIdx.x + k * nth) * 16, 0, 0);
    const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b32(rs, threadIdx.x * 4, 0, 0);
    const uint32_t yv = __builtin_amdgcn_raw_buffer_load_b32(ry, threadIdx.x * 4, 0, 0);

    // expert of this tile: selected here by wave 0 from the certified logits
    // (its LDS scratch is used before the activations are stored)
    int e;
    __shared__ Selection ssel;
    if (a.sel.lstar) {
        // more than 64 experts: every thread ranks one expert first
        if (ranked) select_rank_wg(a.sel, smem, blockIdx.x == 0 ? a.sel.logits : nullptr, pre);
        // ids only; workgroup 0 publishes the softmax weights once its
        // weight loads are in flight
        if (q == 0) select_topk_wave(a.sel, smem, &ssel, false, nullptr, ranked, true);
        __syncthreads();
        e = uniform(ssel.ids[ei]);
    } else {
        e = uniform(a.ids[ei]);
    }

    // weights: this lane's (row, superblock); idle lanes (s >= nsb) read superblock 0
    const int s = 2 * q + (lane >> 5), r = lane & 31;
    const bool live = s < nsb;
    const size_t chunk = ((((size_t)e * T + t) * nsb + (live ? s : 0)) * kQ4Units) * 32 + r;   // in u32x4
    const u32x4* wp = a.gu + chunk;
    u32x4 u[kQ4Units];
#pragma unroll
    for (int k = 0; k < kQ4Units; k++) u[k] = __builtin_nontemporal_load(wp + k * 32);
    if (a.sel.lstar && blockIdx.x == 0 && q == 0) select_publish(a.sel, &ssel);

#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = threadIdx.x + k * nth;                     // 16-byte slot of xq
        if (i * 16 < a.d) *(u32x4*)(xl + (i / 16) * kXsPad + (i % 16) * 16) = xv[k];
    }
    if ((int)threadIdx.x < a.d / 32) xsl[threadIdx.x] = (int32_t)sv;
    if ((int)threadIdx.x < nsb) ysl[threadIdx.x] = __uint_as_float(yv);
    __syncthreads();

    const int isup = r >> 4, row = t * 16 + (r & 15);
    if (live) {
        int32_t* so = TRACE ? a.gu_sums + ((((size_t)ei * 2 + isup) * a.dff + row) * nsb + s) * 2 : nullptr;
        part[s * 32 + r] = q4k_term<TRACE>(u, xl + s * kXsPad, xsl + s * 8, ysl[s], so);
    }
    __syncthreads();
    if (threadIdx.x >= 32) return;
    float v = 0.0f;                                              // sumf, superblocks in order
    for (int k = 0; k < nsb; k++) v += part[k * 32 + r];
    if (TRACE) a.gu_out[((size_t)ei * 2 + isup) * a.dff + row] = v;
    const float up = __shfl_down(v, 16);
    if (r < 16) a.hbuf[(size_t)ei * a.dff + row] = (v / (1.0f + expf(-v))) * up;   // :416
}

// ---- Q8_K of h (into LDS) + down + weighted accumulate ----
// grid: d/RT workgroups; block: 64 * (dff/256) threads (one wave per superblock).
template <int TYPE, bool TRACE>
__global__ __launch_bounds__(1024) void k_down_kq(KqArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int U = TYPE == 12 ? kQ4Units : kQ6Units;
    const int K = a.top_k, RT = 64 / K, nsbf = a.dff / 256, T = a.d / RT;
    const int lane = threadIdx.x & 63, q = uniform((int)(threadIdx.x >> 6));
    const int ei = lane / RT, rr = lane % RT, t = blockIdx.x, row = t * RT + rr;
    const int hstride = nsbf * kXsPad;                            // LDS bytes per expert slot
    int8_t* hql = (int8_t*)smem;                                  // [K][nsbf][kXsPad]
    float* cmax = (float*)(smem + K * hstride);                   // [K*dff/32] chunk amax
    int32_t* h32 = (int32_t*)(cmax + K * a.dff / 32);             // [K*dff/32] sums per 32
    int32_t* h16 = h32 + K * a.dff / 32;                          // [K*dff/16] sums per 16
    float* hsl = (float*)(h16 + K * a.dff / 16);                  // [K*nsbf]
    float* part = hsl + K * nsbf;                                 // [nsbf][64]
    float* vv = part + nsbf * 64;                                 // [64]
    // h chunks (one-chunk case), k-major [8][K*dff/32]: consecutive threads'
    // 16-byte accesses fall on consecutive banks.  Offset from smem (not a
    // cast of the address), so that the compiler keeps it an LDS pointer: as
    // a generic one its accesses were flat, counted with the weight loads,
    // and reading them back waited for the whole weight stream.
    float4* hst = (float4*)(smem + ((((unsigned char*)(vv + 64) - smem) + 15) & ~15));

    int es[8];
#pragma unroll
    for (int k = 0; k < 8; k++) es[k] = uniform(a.ids[k < K ? k : 0]);
    int e = es[0];
#pragma unroll
    for (int k = 1; k < 8; k++) if (ei == k) e = es[k];

    // this thread's 32-value chunk of h first (K * dff / 32 chunks, at most
    // the dff / 4 threads since top_k <= 8: one chunk per thread), then the
    // weights of (slot ei, row, superblock q): the chunk lands before the
    // weight stream, so the Q8_K below runs while the weights are in flight
    // (a wave's loads complete in order).  Every access below that the Q8_K
    // makes is to LDS: a global one on any path would make the compiler wait
    // for the weights there.
    const int nch = K * a.dff / 32;
    const int c = (int)threadIdx.x;
    float4 hv[8];
    {
        const float4* src = (const float4*)(a.hbuf + (size_t)(c < nch ? c : 0) * 32);
#pragma unroll
        for (int k = 0; k < 8; k++) hv[k] = src[k];
    }
    __builtin_amdgcn_sched_barrier(0);          // the chunk's loads stay ahead of the weights'
    constexpr int SU = TYPE == 12 ? kQ4Units : kQ6StreamUnits;   // units in the stream
    const size_t sbi = ((size_t)e * T + t) * nsbf + q;           // (expert, tile, superblock)
    const u32x4* wp = a.dn + sbi * SU * RT + rr;
    u32x4 u[U];
#pragma unroll
    for (int k = 0; k < SU; k++) u[k] = __builtin_nontemporal_load(wp + k * RT);
    // Q6_K: the fp16 d from its own stream, kept as unit 13
    if constexpr (TYPE == 14) u[kQ6Units - 1] = u32x4{(uint32_t)__builtin_nontemporal_load(a.dn_d + sbi * RT + rr), 0, 0, 0};
    __builtin_amdgcn_sched_barrier(0);

    // Q8_K of hbuf (engine_qwen2.rs:288-300): chunk c = 32 values; a 256-block
    // is 8 chunks.  Pass 1: chunk amax, the chunk to LDS.
    if (c < nch) {
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = hv[k];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        cmax[c] = m;
#pragma unroll
        for (int k = 0; k < 8; k++) hst[k * nch + c] = hv[k];
    }
    __syncthreads();
    // pass 2: scale per 256 (amax seeded 1e-12), round, sums per 32 and 16
    if (c < nch) {
        const int blk = c / 8;
        float amax = 1e-12f;
#pragma unroll
        for (int k = 0; k < 8; k++) amax = fmaxf(amax, cmax[blk * 8 + k]);
        const float sc = amax / 127.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) hv[k] = hst[k * nch + c];
        const int slot = c / (a.dff / 32), cc = c % (a.dff / 32);   // expert slot, chunk within it
        int8_t* dst = hql + slot * hstride + (cc / 8) * kXsPad + (cc % 8) * 32;
        // the chunk's 32 bytes in two q8_round16 (one rarely taken branch per
        // 16 values); the per-16 sums from the packed bytes (signed dot with ones)
        float hf[32];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            hf[4 * k] = hv[k].x; hf[4 * k + 1] = hv[k].y; hf[4 * k + 2] = hv[k].z; hf[4 * k + 3] = hv[k].w;
        }
        uint32_t qp[8];
        q8_round16(hf, sc, qp);
        q8_round16(hf + 16, sc, qp + 4);
        int s16[2] = {0, 0};
#pragma unroll
        for (int k = 0; k < 8; k++) s16[k / 4] = sdot4(qp[k], 0x01010101u, s16[k / 4]);
        ((u32x4*)dst)[0] = u32x4{qp[0], qp[1], qp[2], qp[3]};
        ((u32x4*)dst)[1] = u32x4{qp[4], qp[5], qp[6], qp[7]};
        h32[c] = s16[0] + s16[1];
        h16[2 * c] = s16[0];
        h16[2 * c + 1] = s16[1];
        if (c % 8 == 0) hsl[blk] = sc;
        if (TRACE && blockIdx.x == 0) {
            for (int k = 0; k < 32; k++) a.hq[(size_t)c * 32 + k] = dst[k];
            a.hsum[c] = s16[0] + s16[1];
            if (c % 8 == 0) a.hs[blk] = sc;
        }
    }
    __syncthreads();

    // term of (slot ei, row, superblock q)
    {
        const int8_t* xs = hql + ei * hstride + q * kXsPad;
        const float ys = hsl[ei * nsbf + q];
        int32_t* so = nullptr;
        if (TRACE) so = a.dn_sums + (((size_t)ei * a.d + row) * nsbf + q) * (TYPE == 12 ? 2 : 1);
        float tv;
        if constexpr (TYPE == 12)
            tv = q4k_term<TRACE>(u, xs, h32 + (ei * nsbf + q) * 8, ys, so);
        else
            tv = q6k_term<TRACE>(u, xs, h16 + (ei * nsbf + q) * 16, ys, so);
        part[q * 64 + lane] = tv;
    }
    __syncthreads();
    if (q != 0) return;
    float v = 0.0f;
    for (int k = 0; k < nsbf; k++) v += part[k * 64 + lane];
    if (TRACE) a.dn_out[(size_t)ei * a.d + row] = v;
    vv[lane] = v;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < RT) {
        // :426-432: x[r] += wts[ei] * v, ei ascending
        float s = a.x[row];
        for (int k = 0; k < K; k++) s += a.wts[k] * vv[k * RT + lane];
        a.x[row] = s;
    }
}

// ---- load-time re-layout from native superblock rows (one thread per 16-byte unit) ----
__global__ void k_repack_kq_gateup(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                   u32x4* __restrict__ out, int ne, int dff, int nsb) {
    const size_t T = dff / 16;
    const size_t total = (size_t)ne * T * nsb * kQ4Units * 32;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        const int lane = idx % 32;
        size_t r1 = idx / 32;
        const int uu = r1 % kQ4Units; r1 /= kQ4Units;
        const int s = r1 % nsb; r1 /= nsb;
        const size_t t = r1 % T;
        const size_t e = r1 / T;
        const size_t row = e * dff + t * 16 + (lane & 15);
        const uint8_t* src = (lane < 16 ? gate : up) + (row * nsb + s) * 144 + uu * 16;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            w[k] = src[4 * k] | (src[4 * k + 1] << 8) | (src[4 * k + 2] << 16) | ((uint32_t)src[4 * k + 3] << 24);
        out[idx] = u32x4{w[0], w[1], w[2], w[3]};
    }
}

__global__ void k_repack_kq_down(const uint8_t* __restrict__ down, u32x4* __restrict__ out, int ne, int d, int nsbf,
                                 int RT, int type) {
    const int U = kq_units(type), SB = kq_sb_bytes(type);
    const size_t T = d / RT;
    const size_t total = (size_t)ne * T * nsbf * U * RT;
    uint16_t* dstream = (uint16_t*)(out + total);     // Q6_K: the fp16 d behind the units
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        const int rr = idx % RT;
        size_t r1 = idx / RT;
        const int uu = r1 % U; r1 /= U;
        const size_t sbi = r1;                        // (expert, tile, superblock)
        const int s = r1 % nsbf; r1 /= nsbf;
        const size_t t = r1 % T;
        const size_t e = r1 / T;
        const size_t row = e * d + t * RT + rr;
        const uint8_t* src = down + (row * nsbf + s) * SB;
        uint8_t b[16];
#pragma unroll
        for (int k = 0; k < 16; k++) b[k] = uu * 16 + k < SB ? src[uu * 16 + k] : 0;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            w[k] = b[4 * k] | (b[4 * k + 1] << 8) | (b[4 * k + 2] << 16) | ((uint32_t)b[4 * k + 3] << 24);
        out[idx] = u32x4{w[0], w[1], w[2], w[3]};
        if (type == 14 && uu == 0) dstream[sbi * RT + rr] = (uint16_t)(src[208] | (src[209] << 8));
    }
}

size_t kq_gateup_bytes(int ne, int dff, int d) { return (size_t)ne * 2 * dff * (d / 256) * 144; }
size_t kq_down_bytes(int ne, int d, int dff, int top_k, int down_type) {
    (void)top_k;
    return (size_t)ne * d * (dff / 256) * kq_sb_bytes(down_type);   // Q4_K 9 units; Q6_K 13 units + d
}
const uint16_t* kq_down_dstream(const u32x4* dn, int ne, int d, int dff, int down_type) {
    return down_type == 14 ? (const uint16_t*)(dn + (size_t)ne * d * (dff / 256) * kQ6StreamUnits) : nullptr;
}

int launch_repack_kq_gateup(const uint8_t* gate, const uint8_t* up, u32x4* out, int ne, int dff, int d, hipStream_t s) {
    hipLaunchKernelGGL(k_repack_kq_gateup, dim3(2048), dim3(256), 0, s, gate, up, out, ne, dff, d / 256);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}
int launch_repack_kq_down(const uint8_t* down, u32x4* out, int ne, int d, int dff, int top_k, int down_type,
                          hipStream_t s) {
    hipLaunchKernelGGL(k_repack_kq_down, dim3(2048), dim3(256), 0, s, down, out, ne, d, dff / 256, 64 / top_k, down_type);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

// Shapes (validated by the caller): d % 256 == 0, d <= 8192; dff % 256 == 0,
// dff <= 4096; top_k in {1, 2, 4, 8}; d % (64 / top_k) == 0.
int launch_gateup_kq(const KqArgs& a, bool trace, hipStream_t s) {
    const int nsb = a.d / 256;
    const int waves = (nsb + 1) / 2;
    size_t lds = (size_t)nsb * kXsPad + nsb * 8 * 4 + 32 * 4 + (size_t)nsb * 32 * 4;
    if (a.sel.lstar) lds = std::max(lds, std::max(select_lds_bytes(a.sel.ne, a.sel.d), select_ranked_bytes));
    const dim3 grid(a.top_k * (a.dff / 16)), block(64 * waves);
    if (trace) launch(k_gateup_kq<true>, grid, block, lds, s, a);
    else launch(k_gateup_kq<false>, grid, block, lds, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_down_kq(const KqArgs& a, bool trace, hipStream_t s) {
    const int K = a.top_k, nsbf = a.dff / 256, RT = 64 / K;
    if (K * a.dff / 32 > 64 * nsbf) return -22;                  // one h chunk per thread (top_k <= 8)
    const size_t lds = (size_t)K * nsbf * kXsPad + (size_t)K * a.dff / 32 * 4 * 2 + (size_t)K * a.dff / 16 * 4 +
                       (size_t)K * nsbf * 4 + (size_t)nsbf * 64 * 4 + 64 * 4 +
                       (size_t)K * a.dff / 32 * 128 + 16;
    const dim3 grid(a.d / RT), block(64 * nsbf);
    if (a.down_type == 12) {
        if (trace) launch((k_down_kq<12, true>), grid, block, lds, s, a);
        else launch((k_down_kq<12, false>), grid, block, lds, s, a);
    } else {
        if (trace) launch((k_down_kq<14, true>), grid, block, lds, s, a);
        else launch((k_down_kq<14, false>), grid, block, lds, s, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
