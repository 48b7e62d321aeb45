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
// A workgroup has 2P wavefronts, two per k-part: wave 2q + h accumulates
// blocks 0-7 (h = 0) or 8-14 (h = 1) of k-part q.  Each lane owns one row-dot
// and a block's int32 sum S becomes one fma with 2^(e-128)*xsb; the 2P partial
// sums are added in fixed order (deterministic).  Eight blocks per lane
// (rather than a whole k-part) halve the work that follows the last weight
// bytes to land, which is what bounds these single-burst kernels.  The block
// sums come from the matrix cores (mx_dev.h): exact fp8 x fp4 products of an
// fp8 image of the Q8 activations (written by the routing kernel for x, by
// the gate/up epilogue for h) with the stream's nibbles as they are.
#include "moe_common.h"
#include "moe_mx.h"
#include "mx_dev.h"
#include "route_dev.h"

#include <algorithm>

namespace cpb {

// A workgroup covers kTilesPerWG row tiles of one expert (tile pair tp:
// tiles kTilesPerWG*tp + j), every wave streaming its sub-part of each: 180
// workgroups of ~196 KB for a gpt-oss layer (no CU holds two, which a 360 x
// 98 KB split forces on 104 of 256 CUs), and one activation fetch serves both
// tiles.  Wave j then runs tile j's epilogue.
constexpr int kTilesPerWG = 2;

template <bool TRACE>
__global__ __launch_bounds__(128 * kMaxParts) __attribute__((amdgpu_waves_per_eu(3))) void k_gateup_mx(GateUpArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int P = a.nparts, W = 2 * P;
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6), q = w >> 1, hh = w & 1;
    const int ub = kSubUnits * hh;
    const int tiles = a.dff / 32, pairs = (tiles + kTilesPerWG - 1) / kTilesPerWG;
    const int ei = blockIdx.x / pairs, tp = blockIdx.x % pairs;
    // every argument the prologue needs, loaded in one batch up front (else
    // the selection's fields arrive in a second kernarg round trip)
    asm volatile("" ::"s"(a.sel.lstar), "s"(a.sel.lbound), "s"(a.sel.ne), "s"(a.sel.k), "s"(a.ximg), "s"(a.xsb),
                 "s"(a.nb), "s"(a.w));
    SelectPre pre{0.0, 0.0};
    if (a.sel.lstar && w == 0) pre = select_preload(a.sel);
    float* red = (float*)smem;                                 // [kTilesPerWG][W][64]
    const int blk0 = q * kBlkPerPart;
    // activations: the two windows' A operands and the 8 block scales (issued
    // before the weights: requests queued behind a CU's weight stream would
    // land after it)
    const __amdgpu_buffer_rsrc_t ri = buf_rsrc(a.ximg, (uint32_t)(a.nb * kImgBytes));
    WinAct xw[2];
    xw[0] = load_win_act(ri, blk0 + ub, ub, a.nb);
    xw[1] = load_win_act(ri, blk0 + ub + 4, ub + 4, a.nb);
    float xsc[kSubUnits];
    {
        const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.xsb, (uint32_t)(a.nb * 4));
#pragma unroll
        for (int i = 0; i < kSubUnits; i++) {
            const int u = ub + i;
            const bool ok = u < kBlkPerPart && blk0 + u < a.nb;
            xsc[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (uint32_t)(blk0 + u) * 4 : kOffNone, 0, 0));
        }
    }
    int e;
    __shared__ Selection ssel;
    if (a.sel.lstar) {
        // ids only; workgroup 0 publishes the softmax weights once its weight
        // loads are in flight
        if (w == 0)
            select_topk_wave(a.sel, smem, &ssel, false, &pre,
                             false, true);
        // barrier on LDS only (s_barrier without a wait for the activation loads)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // a plain LDS read: merged with the global read below into one flat
        // load it would queue behind the CU's outstanding weight loads
        e = uniform(((const __attribute__((address_space(3))) int*)ssel.ids)[ei]);
    } else {
        e = a.ids[ei];
    }
    // both tiles' sub-parts requested back to back (a missing second tile of
    // an odd tile count reads the first again; its result is dropped)
    u32x4 wv[kTilesPerWG][1 + kSubUnits];
#pragma unroll
    for (int j = 0; j < kTilesPerWG; j++) {
        const int t = min(kTilesPerWG * tp + j, tiles - 1);
        load_sub(a.w + ((((size_t)e * tiles + t) * P + q) * kUnits) * 64 + lane, 64, ub, wv[j]);
    }
    if (a.sel.lstar && blockIdx.x == 0 && w == 0) select_publish(a.sel, &ssel);
    const float* bias = (lane >> 5) ? a.up_b : a.gate_b;
    const int tw = kTilesPerWG * tp + w;                       // the tile whose epilogue wave w runs (w < kTilesPerWG)
    float bias_pf = 0.0f;
    if (w < kTilesPerWG && tw < tiles && bias)
        bias_pf = ((const __attribute__((address_space(1))) float*)bias)[(size_t)e * a.dff + tw * 32 + (lane & 31)];
    const int isup = lane >> 5;
#pragma unroll
    for (int j = 0; j < kTilesPerWG; j++) {
        const int t = kTilesPerWG * tp + j;
        int32_t* so = nullptr;
        if (TRACE && t < tiles) so = a.gu_sums + (((size_t)(ei * 2 + isup) * a.dff + t * 32 + (lane & 31)) * a.nb + blk0);
        red[(j * W + w) * 64 + lane] = part_dot_sub_mfma<TRACE>(wv[j], ub, xw, xsc, so, blk0, a.nb);
    }
    __syncthreads();
    if (w >= kTilesPerWG || tw >= tiles) return;
    const int t = tw, row = t * 32 + (lane & 31);
    float pr[2 * kMaxParts];
#pragma unroll
    for (int p = 0; p < 2 * kMaxParts; p++) pr[p] = p < W ? red[(w * W + p) * 64 + lane] : 0.0f;
    float v = 0.0f;
#pragma unroll
    for (int p = 0; p < 2 * kMaxParts; p++)
        if (p < W) v += pr[p];
    if (bias) v += bias_pf;
    if (TRACE) a.gu[(size_t)(ei * 2 + isup) * a.dff + row] = v;
    // SwiGLU-OAI (engine_gpt2.rs:887-906) in lanes 0-31: gate row r, up row r from lane r+32
    float vd = v, u = v;
    swap32f(vd, u);                      // lanes 0-31: u = v of lane + 32
    float h = 0.0f;
    if (!isup) {
        const float xg = fminf(v, a.limit);
        const float yu = fminf(fmaxf(u, -a.limit), a.limit);
        h = (xg / (1.0f + expf(-a.alpha * xg))) * (yu + 1.0f);
    }
    // block maximum over the 32 gate lanes: DPP within 16-lane rows, then the
    // partner row by a permlane swap (no LDS round trips)
    float m = row_max_f32(isup ? 0.0f : fabsf(h));
    {
        float ma = m, mb = m;
        swap16f(ma, mb);
        m = fmaxf(m, (lane & 16) ? ma : mb);
    }
    const float sc = fmaxf(1e-12f, m) / 127.0f;
    if (!isup) {
        const int8_t qv = q8_round(h, sc);
        a.hq[(size_t)ei * a.dff + row] = qv;
        // h's matrix-core image for the down kernel: element j = row % 32 of
        // block t sits at K offset 2j (j < 16) or 2(j - 16) + 1
        const int j = lane & 31, kpos = j < 16 ? 2 * j : 2 * (j - 16) + 1;
        uint8_t* im = a.himg + ((size_t)ei * (a.dff / 32) + t) * kImgBytes;
        const uint32_t qb = (uint32_t)(uint8_t)qv;
        im[kpos] = (uint8_t)img_hi(qb);
        im[32 + kpos] = (uint8_t)img_lo(qb);
        if (TRACE) a.h[(size_t)ei * a.dff + row] = h;
    }
    if (lane == 0) a.hsb[(size_t)ei * (a.dff / 32) + t] = sc;
}

// top_k in {1, 2, 4}: one tile of 64 / top_k rows x top_k slots.
template <bool TRACE>
__global__ __launch_bounds__(128 * kMaxParts) void k_down_mx(DownArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int P = a.nparts, W = 2 * P, K = a.top_k, RT = 64 / K;
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6), q = w >> 1, hh = w & 1;
    const int ub = kSubUnits * hh;
    const int tiles = a.d / RT, t = blockIdx.x;
    const int ei = lane / RT, rr = lane % RT, row = t * RT + rr;
    float* red = (float*)smem;                                 // [W][64]
    float* vv = red + W * 64;                                  // [64]
    const int blk0 = q * kBlkPerPart;
    // the routed experts (written by the gate/up launch) first: the weight
    // addresses wait on them; scalar loads, which the activation requests
    // below need not wait for
    int es[4];
#pragma unroll
    for (int k = 0; k < 4; k++) es[k] = __builtin_amdgcn_readfirstlane(a.ids[k < K ? k : 0]);
    // activations: for each window and 16-lane group (whose rows all belong
    // to expert slot 16g / RT) this lane's A fragment; the slot's scales
    const __amdgpu_buffer_rsrc_t ri = buf_rsrc(a.himg, (uint32_t)(K * a.nbf * kImgBytes));
    u32x4 xa[2][4];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            xa[h][g] = load_act_frag(ri, (uint32_t)(((16 * g) / RT) * a.nbf * kImgBytes), blk0 + ub + 4 * h, ub + 4 * h,
                                     a.nbf);
    float xsc[kSubUnits];
    {
        const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.hsb, (uint32_t)(K * a.nbf * 4));
#pragma unroll
        for (int i = 0; i < kSubUnits; i++) {
            const int u = ub + i;
            const bool ok = u < kBlkPerPart && blk0 + u < a.nbf;
            xsc[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (uint32_t)(ei * a.nbf + blk0 + u) * 4 : kOffNone, 0, 0));
        }
    }
    const int e = ei == 0 ? es[0] : ei == 1 ? es[1] : ei == 2 ? es[2] : es[3];
    u32x4 wv[1 + kSubUnits];
    load_sub(a.w + (((((size_t)e * tiles + t) * P + q) * kUnits) * RT) + rr, RT, ub, wv);
    float dnb_pf = 0.0f, x_pf = 0.0f, w_pf[4];
    if (w == 0) {
        if (a.down_b) dnb_pf = a.down_b[(size_t)e * a.d + row];
        if (lane < RT) x_pf = a.x[row];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) w_pf[k] = a.wts[k < K ? k : 0];
    int32_t* so = nullptr;
    if (TRACE) so = a.dn_sums + (((size_t)ei * a.d + row) * a.nbf + blk0);
    const float acc = part_dot_sub_mfma4<TRACE>(wv, ub, xa, xsc, so, blk0, a.nbf);
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (w != 0) return;
    float pr[2 * kMaxParts];
#pragma unroll
    for (int p = 0; p < 2 * kMaxParts; p++) pr[p] = p < W ? red[p * 64 + lane] : 0.0f;
    float v = 0.0f;
#pragma unroll
    for (int p = 0; p < 2 * kMaxParts; p++)
        if (p < W) v += pr[p];
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

// Any top_k <= 8: 16-row tiles, expert slots four at a time (one pass for
// top_k <= 4, two above), each pass a full sub-part stream and block sums as
// in k_down_mx; the combine runs over all slots in ascending order.
template <bool TRACE>
__global__ __launch_bounds__(128 * kMaxParts) void k_down_mx_slots(DownArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int P = a.nparts, W = 2 * P, K = a.top_k, RT = mx_down_rt(K);
    // slots per pass (lane groups of RT rows) and passes: one pass of K
    // slots for K in {1, 2, 4}; passes of four 16-row slots otherwise
    const int SP = 64 / RT, NP = (K + SP - 1) / SP;
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6), q = w >> 1, hh = w & 1;
    const int ub = kSubUnits * hh;
    const int tiles = a.d / RT, t = blockIdx.x;
    const int gi = lane / RT, rr = lane % RT, row = t * RT + rr;
    float* red = (float*)smem;                                 // [NP][W][64]
    float* vv = red + NP * W * 64;                             // [NP][64]
    const int blk0 = q * kBlkPerPart;
    // the routed experts (written by the gate/up launch) first: the weight
    // addresses wait on them; scalar loads, which the activation requests
    // below need not wait for
    int es[8];
#pragma unroll
    for (int k = 0; k < 8; k++) es[k] = __builtin_amdgcn_readfirstlane(a.ids[k < K ? k : 0]);
    float w_pf[8];
#pragma unroll
    for (int k = 0; k < 8; k++) w_pf[k] = a.wts[k < K ? k : 0];
    float x_pf = 0.0f;
    if (w == 0 && lane < RT) x_pf = a.x[row];
    const __amdgpu_buffer_rsrc_t ri = buf_rsrc(a.himg, (uint32_t)(K * a.nbf * kImgBytes));
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.hsb, (uint32_t)(K * a.nbf * 4));
    float dnb_pf[2] = {0.0f, 0.0f};
    for (int pass = 0; pass < NP; pass++) {
        // slot of lane group g in this pass; a slot beyond K reads zero
        // activations (its rows' results are dropped)
        const int s0 = pass * SP, slot = s0 + gi;
        // activations: for each window and 16-lane group (whose rows all
        // belong to one slot) this lane's A fragment; the slot's scales
        u32x4 xa[2][4];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int sg = s0 + (16 * g) / RT;
                xa[h][g] = sg < K ? load_act_frag(ri, (uint32_t)(sg * a.nbf * kImgBytes), blk0 + ub + 4 * h, ub + 4 * h,
                                                  a.nbf)
                                  : u32x4{0, 0, 0, 0};
            }
        float xsc[kSubUnits];
#pragma unroll
        for (int i = 0; i < kSubUnits; i++) {
            const int u = ub + i;
            const bool ok = slot < K && u < kBlkPerPart && blk0 + u < a.nbf;
            xsc[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (uint32_t)(slot * a.nbf + blk0 + u) * 4 : kOffNone, 0, 0));
        }
        int e = es[0];
#pragma unroll
        for (int k = 1; k < 8; k++)
            if (slot == k) e = es[k];
        u32x4 wv[1 + kSubUnits];
        load_sub(a.w + (((((size_t)e * tiles + t) * P + q) * kUnits) * RT) + rr, RT, ub, wv);
        if (w == 0 && a.down_b && slot < K) dnb_pf[pass] = a.down_b[(size_t)e * a.d + row];
        int32_t* so = nullptr;
        if (TRACE && slot < K) so = a.dn_sums + (((size_t)slot * a.d + row) * a.nbf + blk0);
        const float acc = part_dot_sub_mfma4<TRACE>(wv, ub, xa, xsc, so, blk0, a.nbf);
        red[(pass * W + w) * 64 + lane] = acc;
    }
    __syncthreads();
    if (w != 0) return;
    for (int pass = 0; pass < NP; pass++) {
        float pr[2 * kMaxParts];
#pragma unroll
        for (int p = 0; p < 2 * kMaxParts; p++) pr[p] = p < W ? red[(pass * W + p) * 64 + lane] : 0.0f;
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < 2 * kMaxParts; p++)
            if (p < W) v += pr[p];
        const int slot = pass * SP + gi;
        if (a.down_b) v += dnb_pf[pass];
        if (TRACE && slot < K) a.dn[(size_t)slot * a.d + row] = v;
        vv[pass * 64 + lane] = v;
    }
    wave_sync_lds();
    if (lane < RT) {
        // engine_gpt2.rs:911-921: s = x[r]; s += wts[ei] * (dot + b), ei ascending
        float s = x_pf;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (k < K) s += w_pf[k] * vv[(k / SP) * 64 + (k % SP) * RT + lane];
        a.x[row] = s;
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
    int RT = mx_down_rt(top_k);
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
    hipLaunchKernelGGL(k_repack_down, dim3(4096), dim3(256), 0, s, down, out, ne, d, nbf, P, mx_down_rt(top_k));
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_gateup_mx(const GateUpArgs& a, bool trace, hipStream_t s) {
    const int P = a.nparts;
    if (P < 1 || P > kMaxParts || a.dff % 32 != 0) return -22;
    size_t lds = sizeof(float) * kTilesPerWG * 2 * P * 64;
    if (a.sel.lstar) lds = std::max(lds, select_lds_bytes(a.sel.ne, a.sel.d));
    dim3 grid(a.top_k * ((a.dff / 32 + kTilesPerWG - 1) / kTilesPerWG)), block(128 * P);
    if (trace) launch(k_gateup_mx<true>, grid, block, lds, s, a);
    else launch(k_gateup_mx<false>, grid, block, lds, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_down_mx(const DownArgs& a, bool trace, hipStream_t s) {
    const int P = a.nparts, K = a.top_k, RT = mx_down_rt(K);
    if (P < 1 || P > kMaxParts || K < 1 || K > 8 || a.d % RT != 0) return -22;
    const int NP = (K + 64 / RT - 1) / (64 / RT);
    const size_t lds = sizeof(float) * (NP * 2 * P * 64 + NP * 64);
    dim3 grid(a.d / RT), block(128 * P);
    if (K == 1 || K == 2 || K == 4) {
        if (trace) launch(k_down_mx<true>, grid, block, lds, s, a);
        else launch(k_down_mx<false>, grid, block, lds, s, a);
    } else {
        if (trace) launch(k_down_mx_slots<true>, grid, block, lds, s, a);
        else launch(k_down_mx_slots<false>, grid, block, lds, s, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
