// attn.hip -- gpt-oss attention block, decode, on gfx950.
//
// Reference (src/bin/): engine_gpt2.rs:772-843 (the layer's attention),
// rope_init / rope_yarn_slow / rope_yarn :535-590, Q8Mat :464-494, dot_q8_i8
// :169-191, qblock32 :691-699, rmsnorm_quant_par :730-738.
//
// Kernels per token and layer:
//   k_attn_qkv   rmsnorm (16-lane sum of squares) + Q8 per 32 of x, then the
//                q / k / v rows: the reference's Q8 dot (8 fp32 chains per
//                row, one lane each), bias, RoPE from the table, cache write;
//                one workgroup per CU, 2-3 RoPE-complete 8-row tiles each;
//   k_attn_core  per (kv-head, chunk of 128 positions): scores of the group's
//                q-heads, softmax weights, weighted v; a window of 128 is one
//                chunk and finishes in the workgroup in the reference's order,
//                longer spans leave per-chunk (max, sum, weighted v) that the
//                last workgroup of the kv-head merges with the sink; then Q8
//                of the heads' outputs;
//   k_attn_oproj x[r] += wo[r] . ao + bo[r] (k_attn_oproj_wave at 64 heads:
//                one wave per 8-row tile, codes in registers).
// At the gpt-oss shapes the codes of q / k / v and of the o-projection are
// loaded straight into registers and each chain consumes them in load order.
// The projections, RoPE and the cache rows are the reference's operations in
// its order (bit for bit given the same RoPE table, which the host computes
// once with the reference's formula); the softmax goes through expf (and,
// past one chunk, a merge over chunks), so the heads' outputs match to
// tolerance.
//
// Weights: the chain-major Q8 stream described before q8c_dot, built on the
// GPU at load time from the bf16 tensors.  KV cache: [layer][kv-head]
// [position][64] fp32, so a chunk of positions of one head is one contiguous
// 32 KiB run.
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
constexpr int kAttnChunk = 128;    // cache positions per core workgroup
constexpr int kAttnMaxGroup = 8;   // q-heads per kv-head

// ---- cross-lane reductions on DPP + readlane (no LDS round trips) ----
template <int CTRL>
CPB_DEV float dppf(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false)); }
CPB_DEV float lanef(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
CPB_DEV float row_sum_f32(float v) {
    v += dppf<0xB1>(v);          // lane ^ 1
    v += dppf<0x4E>(v);          // lane ^ 2
    v += dppf<0x141>(v);         // mirror within 8
    v += dppf<0x140>(v);         // mirror within 16
    return v;
}
CPB_DEV float wave_max_f32(float v) {
    const float r = row_max_f32(v);
    return fmaxf(fmaxf(lanef(r, 0), lanef(r, 16)), fmaxf(lanef(r, 32), lanef(r, 48)));
}
CPB_DEV float wave_sum_f32(float v) {
    const float r = row_sum_f32(v);
    return (lanef(r, 0) + lanef(r, 16)) + (lanef(r, 32) + lanef(r, 48));
}
// max over each half wave (lanes 0-31, 32-63)
CPB_DEV float half_max_f32(float v) {
    const float r = row_max_f32(v);
    const float lo = fmaxf(lanef(r, 0), lanef(r, 16)), hi = fmaxf(lanef(r, 32), lanef(r, 48));
    return (threadIdx.x & 32) ? hi : lo;
}

// Chain-major Q8 stream.  dot_q8_i8 (:169-191) runs 8 fp32 chains per row:
// chain c = 4h + j accumulates, over the blocks b = h, h+2, h+4, ... in order,
// the integer dot of block b's bytes 4j..4j+3 and 16+4j..16+4j+3 times
// scale(b) * xscale(b).  Lane 8r + c of a wave runs chain c of tile row r.
// Per 8-row tile the codes are stored by pairs of chain steps: entry (tile,
// sp) is 64 lanes x 16 bytes, lane l's 16 bytes = (lo, hi) of its chain at
// steps 2sp and 2sp + 1 (step s = block 2s + h).  Scales: [tile][sp][r][h][2]
// (one float2 per lane and step pair).
// Blocks are padded to a multiple of 4 with zero codes and zero scales
// (their products are +0 and leave every chain unchanged).
CPB_DEV_HOST_INLINE int q8c_nbp(int nb) { return (nb + 3) & ~3; }
CPB_DEV_HOST_INLINE size_t q8c_code_bytes(int rows, int cols) { return (size_t)rows / 8 * q8c_nbp(cols / 32) / 4 * 1024; }
CPB_DEV_HOST_INLINE size_t q8c_scale_bytes(int rows, int cols) { return (size_t)rows / 8 * q8c_nbp(cols / 32) / 2 * 64; }

struct AttnLayerDev {
    const u32x4 *wq, *wk, *wv, *wo;     // chain-major Q8 codes
    const float *sq, *sk, *sv, *so;     // scales [tile][step][8][2]
    const float *bq, *bk, *bv, *bo, *sinks, *norm;
};

struct AttnArgs {
    int d, nh, nkv, nb, nbo, pos, start, max_seq, nsplit;
    float eps;
    AttnLayerDev L;
    float* x;            // [d] residual (in place)
    float* kc;           // this layer's cache [nkv][max_seq][64]
    float* vc;
    const float* rope;   // [max_seq][32][2]
    float* q;            // [nh*64]
    float* ao;           // [nh*64]
    int8_t* aq;          // [nh*64]
    float* asb;          // [nh*64/32]
    int8_t* xq;          // [d] (trace copy of the activations)
    float* xsb;          // [d/32]
    float* part;         // [nh][nsplit][66]: max, sum, 64 weighted values
    int* count;          // [nkv] arrivals of the core workgroups (0 between launches)
};

// ---- load time: Q8Mat::from_bf16 (:476-489) into the chain-major stream ----
// one thread per (row, block); the stream must be zeroed beforehand (padding)
// pair_tiles: within each 64-row head, tile j holds rows 4j..4j+3 (slots 0-3)
// and 32+4j..32+4j+3 (slots 4-7), so a RoPE pair (i, 32 + i) shares a tile;
// otherwise tile t holds rows 8t..8t+7.
__global__ void k_q8c_quant(const uint16_t* __restrict__ w, int rows, int cols, u32x4* __restrict__ q,
                            float* __restrict__ s, int pair_tiles) {
    const int nb = cols / 32, nbp = q8c_nbp(nb), nsp = nbp / 4, ns = nbp / 2;
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
        uint32_t wd[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            float r = roundf(vals[i] / sc);
            r = r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
            wd[i >> 2] |= (uint32_t)(uint8_t)(int8_t)r << (8 * (i & 3));
        }
        const int i64 = row & 63;
        const int tile = pair_tiles ? (row >> 6) * 8 + ((i64 & 31) >> 2) : row >> 3;
        const int r = pair_tiles ? (i64 & 3) + ((i64 >> 5) << 2) : row & 7;
        const int h = b & 1, st = b >> 1, sp = st >> 1, k = st & 1;
        s[((((size_t)tile * nsp + sp) * 8 + r) * 2 + h) * 2 + k] = sc;
        uint32_t* base = (uint32_t*)(q + ((size_t)tile * nsp + sp) * 64 + r * 8 + h * 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            base[j * 4 + k * 2] = wd[j];            // lane 8r + 4h + j: bytes 4j..4j+3
            base[j * 4 + k * 2 + 1] = wd[4 + j];    // and 16+4j..16+4j+3
        }
    }
}

// LDS writes of this wave visible to its own later reads
CPB_DEV void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// workgroup barrier ordering LDS only: unlike __syncthreads, no wait for the
// wave's outstanding global loads (the weight stream stays in flight)
CPB_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- staging of 8-row tiles into LDS ----
// A workgroup copies the codes and scales of its consecutive tiles (at most
// kMaxTiles) to LDS with every thread's 16-byte loads issued before any is
// waited for, so the whole tile stream is in flight at once; the chains then
// run from LDS.  The loads are unconditional buffer loads (an offset past the
// tiles reads zeros): with a branch around each, the compiler could not count
// them, and any use of data loaded before them (x for the norm, the
// activations) waited for nearly the whole stream.
constexpr int kMaxTiles = 3;
// 16-byte code loads and float4 scale loads per thread (x 256 threads): qkv,
// 3 tiles at d <= 4096; o-projection, 1 tile at n_head <= 128
constexpr int kQkvLoads = 24, kQkvScales = 3, kOprojLoads = 16, kOprojScales = 2;
struct TileSet {
    const u32x4* w;                   // first tile's codes (the tiles follow it)
    const float* s;                   // first tile's scales
    int nt, nsp;                      // tiles, step pairs per tile
};
template <int NL, int NS>
struct StageRegs {
    u32x4 r[NL > 0 ? NL : 1];
    float4 sc[NS];
};
template <int NL, int NS>
CPB_DEV void stage_issue(const TileSet& t, StageRegs<NL, NS>& g) {
    const int total = t.nt * t.nsp * 64, tid = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(t.w, (uint32_t)total * 16);
#pragma unroll
    for (int k = 0; k < NL; k++)
        g.r[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)(k * 256 + tid) * 16, 0, 2));
    const int stotal = t.nt * t.nsp * 8;                  // float4: ns * 16 / 4 per tile
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(t.s, (uint32_t)stotal * 16);
#pragma unroll
    for (int k = 0; k < NS; k++)
        g.sc[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(k * 256 + tid) * 16, 0, 0));
}
template <int NL, int NS>
CPB_DEV void stage_commit(const TileSet& t, const StageRegs<NL, NS>& g, u32x4* lw, float* ls) {
    const int total = t.nt * t.nsp * 64, tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NL; k++) {
        const int i = k * 256 + tid;
        if (i < total) lw[i] = g.r[k];
    }
    const int stotal = t.nt * t.nsp * 8;
#pragma unroll
    for (int k = 0; k < NS; k++) {
        const int i = k * 256 + tid;
        if (i < stotal) ((float4*)ls)[i] = g.sc[k];
    }
}

// Activations in LDS in the chains' order too: dword i of the Q8 row (block
// b = i / 8, word w = i % 8: bytes 4j..4j+3 of the block for w = j, 16+4j..
// for w = 4 + j) goes to entry (sp = b / 4, h = b % 2, j) component 2t + w / 4
// (t = (b / 2) % 2), so a lane reads its step pair's four dwords at once;
// the block scales as float2 per (sp, h): blocks 4sp + h and 4sp + 2 + h.
CPB_DEV_HOST_INLINE int xc_index(int i) {
    const int b = i >> 3, w = i & 7;
    return ((((b >> 2) * 2 + (b & 1)) * 4 + (w & 3)) * 4) + ((b >> 1) & 1) * 2 + (w >> 2);
}
CPB_DEV_HOST_INLINE int xs_index(int b) { return ((b >> 2) * 2 + (b & 1)) * 2 + ((b >> 1) & 1); }

// The chain of this lane over one 8-row tile staged in LDS (codes lw, scales
// ls), activations in LDS (xl: dwords in xc_index order; sl: scales in
// xs_index order; both padded to q8c_nbp blocks with zeros).  Returns the
// row's dot_q8_i8 in lane 0 of the row's group of 8.  NSP > 0: the step-pair
// count is NSP (== nbp / 4) and the chain is unrolled whole, so the LDS reads
// are scheduled ahead of the fmas that wait for them; NSP == 0: any count.
struct Q8cOps {
    u32x4 w, xa;
    float2 ws, xs;
};
CPB_DEV Q8cOps q8c_load(const u32x4* lw, const float2* wsc, const u32x4* xc, const float2* xsc, int sp, int lane) {
    return Q8cOps{lw[sp * 64 + lane], xc[sp * 8], wsc[sp * 16], xsc[sp * 2]};
}
CPB_DEV void q8c_fma(const Q8cOps& o, float& acc) {
    // steps 2sp (block 4sp + h) and 2sp + 1 (block 4sp + 2 + h)
    const int d0 = sdot4(o.w[1], o.xa[1], sdot4(o.w[0], o.xa[0], 0));
    acc = fmaf((float)d0, o.ws.x * o.xs.x, acc);
    const int d1 = sdot4(o.w[3], o.xa[3], sdot4(o.w[2], o.xa[2], 0));
    acc = fmaf((float)d1, o.ws.y * o.xs.y, acc);
}
// The same chain with this lane's codes in registers (wreg[sp]: its 16 bytes
// of step pair sp, loaded in step order): step pair sp waits for its own load
// only, so the chain runs while the later codes are still arriving.  An empty
// volatile asm passes acc and step sp's codes through, so step sp's dots come
// after step sp - 1's fma: as plain code the compiler hoisted later steps'
// dots, whose operands are the later loads, and the chain waited for the
// whole stream.
template <int NSP>
CPB_DEV float q8c_dot_regs(const u32x4 (&wreg)[NSP], const float* ls, const uint32_t* xl, const float* sl) {
    const int lane = threadIdx.x & 63, r = lane >> 3, h = (lane >> 2) & 1, j = lane & 3;
    const float2* wsc = (const float2*)ls + r * 2 + h;
    const u32x4* xc = (const u32x4*)xl + h * 4 + j;
    const float2* xsc = (const float2*)sl + h;
    float acc = 0.0f;
#pragma unroll
    for (int sp = 0; sp < NSP; sp++) {
        u32x4 w = wreg[sp];
        asm volatile("" : "+v"(acc), "+v"(w));
        const u32x4 xa = xc[sp * 8];
        const float2 ws = wsc[sp * 16], xs = xsc[sp * 2];
        // steps 2sp (block 4sp + h) and 2sp + 1 (block 4sp + 2 + h)
        const int d0 = sdot4(w[1], xa[1], sdot4(w[0], xa[0], 0));
        acc = fmaf((float)d0, ws.x * xs.x, acc);
        const int d1 = sdot4(w[3], xa[3], sdot4(w[2], xa[2], 0));
        acc = fmaf((float)d1, ws.y * xs.y, acc);
    }
    const float v = acc + dppf<0x12C>(acc);
    const float v01 = v + dppf<0xB1>(v);
    return v01 + dppf<0x4E>(v01);
}

CPB_DEV float q8c_dot(const u32x4* lw, const float* ls, int nbp, const uint32_t* xl, const float* sl) {
    const int lane = threadIdx.x & 63, r = lane >> 3, h = (lane >> 2) & 1, j = lane & 3;
    const float2* wsc = (const float2*)ls + r * 2 + h;           // [sp][8][2] float2
    const u32x4* xc = (const u32x4*)xl + h * 4 + j;              // [sp][2][4] u32x4
    const float2* xsc = (const float2*)sl + h;                   // [sp][2] float2
    float acc = 0.0f;
    const int nsp = nbp / 4;
#pragma unroll 4
    for (int sp = 0; sp < nsp; sp++) q8c_fma(q8c_load(lw, wsc, xc, xsc, sp, lane), acc);
    // lanes 0-3 of each group of 8: v_j = acc0_j + acc1_j (lane + 4: row_ror by 12)
    const float v = acc + dppf<0x12C>(acc);
    const float v01 = v + dppf<0xB1>(v);                 // lane 0: v0 + v1, lane 2: v2 + v3
    return v01 + dppf<0x4E>(v01);                        // lane 0 of the group: (v0 + v1) + (v2 + v3)
}

// rmsnorm of x (gpt-oss: 16 fp32 chains, chain q over x[16m + q],
// :710-726) and Q8 per 32 (qblock32 :691-699) into LDS (xl dwords / sl
// scales, padded with zeros to nbp blocks).  xr / wr: this thread's float4
// slots tid + 256k of x and of the norm weights, in registers.  xt: LDS for a
// transposed copy (chain q's elements contiguous, row stride attn_xt_stride,
// zero padded so that whole 32-value groups can be read; the chain's one-group
// look-ahead past the last row lands in red); red: 64 floats.
CPB_DEV_HOST_INLINE int attn_xt_stride(int d) { return (d / 16 + 32 + 63) / 64 * 64 + 4; }   // = 4 (mod 64): distinct banks
template <int KS>
CPB_DEV void attn_norm_q8(const float4 (&xr)[KS], const float4 (&wr)[KS], int d, int nb, int nbp, float eps, float* xt,
                          float* red, uint32_t* xl, float* sl, int8_t* gxq, float* gxsb) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int n16 = d / 16, S = attn_xt_stride(d);
#pragma unroll
    for (int k = 0; k < KS; k++) {
        const int i = tid + k * 256;
        if (i * 4 < d) {
            const float xv[4] = {xr[k].x, xr[k].y, xr[k].z, xr[k].w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int e = 4 * i + c;
                xt[(e & 15) * S + (e >> 4)] = xv[c];
            }
        }
    }
    // zero padding past d / 16: fma(0, 0, acc) leaves acc (>= 0) unchanged
    for (int e = tid; e < 16 * (S - n16); e += 256) xt[(e & 15) * S + n16 + (e >> 4)] = 0.0f;
    lds_barrier();
    if (tid < 64) {
        // lane q (mod 16) streams row q: the next group's reads are issued
        // before the current group's fmas
        float acc = 0.0f;
        uint32_t ra = lds_addr(xt + (lane & 15) * S);
        f32x4 ga[8], gb[8];                           // ping-pong groups of 32 values
        lds_read8(ga, ra);
        for (int m = 0;; m += 64) {
            lds_read8(gb, ra + 128);
            lds_wait_older8(ga);
            acc = sumsq_chain(ga, acc);
            if (m + 32 >= n16) break;
            lds_read8(ga, ra + 256);
            lds_wait_older8(gb);
            acc = sumsq_chain(gb, acc);
            if (m + 64 >= n16) break;
            ra += 256;
        }
        lds_wait_all();
        // chain q = 4v + l -> acc[v][l]; L[l] = (a0 + a1) + (a2 + a3); s = (L0 + L1) + (L2 + L3)
        float c16[16];
#pragma unroll
        for (int q = 0; q < 16; q++) c16[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), q));
        float L[4];
#pragma unroll
        for (int l = 0; l < 4; l++) L[l] = (c16[l] + c16[4 + l]) + (c16[8 + l] + c16[12 + l]);
        const float sq = (L[0] + L[1]) + (L[2] + L[3]);
        if (lane == 0) red[16] = 1.0f / sqrtf(sq / (float)d + eps);
    }
    lds_barrier();
    const float inv = red[16];
    // Q8 from registers: slot i = 4 elements, a 32-block = 8 consecutive slots
    // (lanes).  The KS slots of a thread are computed side by side (a slot
    // past d holds x[0..3]: computed, not stored; d % 32 == 0 keeps a block's
    // eight slots all inside or all past d), one rarely taken branch for the
    // exact rounding path.
    float v[KS][4], sc[KS], rs[KS], r[KS][4];
    bool near = false;
#pragma unroll
    for (int k = 0; k < KS; k++) {
        v[k][0] = xr[k].x * inv * wr[k].x;
        v[k][1] = xr[k].y * inv * wr[k].y;
        v[k][2] = xr[k].z * inv * wr[k].z;
        v[k][3] = xr[k].w * inv * wr[k].w;
        float m = fmaxf(fmaxf(fabsf(v[k][0]), fabsf(v[k][1])), fmaxf(fabsf(v[k][2]), fabsf(v[k][3])));
        m = fmaxf(m, dppf<0xB1>(m));
        m = fmaxf(m, dppf<0x4E>(m));
        m = fmaxf(m, dppf<0x141>(m));                // the other quad of the 8
        sc[k] = fmaxf(1e-12f, m) / 127.0f;
        rs[k] = __builtin_amdgcn_rcpf(sc[k]);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float y = v[k][u] * rs[k];
            r[k][u] = __builtin_rintf(y);
            near = near || q8_near_half(y);
        }
    }
    if (near) {
        // the exact quotients of all 16 side by side (no branch per value)
#pragma unroll
        for (int k = 0; k < KS; k++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float ex = roundf(v[k][u] / sc[k]);
                r[k][u] = q8_near_half(v[k][u] * rs[k]) ? ex : r[k][u];
            }
    }
#pragma unroll
    for (int k = 0; k < KS; k++) {
        const int i = tid + k * 256;
        uint32_t wd = 0u;
#pragma unroll
        for (int u = 0; u < 4; u++) wd |= (uint32_t)(uint8_t)q8_clamp(r[k][u]) << (8 * u);
        if (i * 4 < d) {
            xl[xc_index(i)] = wd;
            if ((i & 7) == 0) sl[xs_index(i >> 3)] = sc[k];
            if (gxq) {
                ((uint32_t*)gxq)[i] = wd;
                if ((i & 7) == 0) gxsb[i >> 3] = sc[k];
            }
        }
    }
    for (int i = d / 4 + tid; i < nbp * 8; i += 256) xl[xc_index(i)] = 0u;
    for (int bk = nb + tid; bk < nbp; bk += 256) sl[xs_index(bk)] = 0.0f;
}

// ---- rmsnorm + Q8 of x, q / k / v rows + bias + RoPE + cache ----
// The q, k and v streams are one sequence of T = (nh + 2 nkv) * 8 tiles
// (q heads, then k heads, then v heads; tile j of a head holds rows 4j..4j+3
// and 32+4j..32+4j+3, so each RoPE pair (i, 32 + i) is in one tile).
// Workgroup g of G takes tiles [g T / G, (g + 1) T / G) (at most kMaxTiles),
// with G = min(256, T) where that allows: one workgroup per CU, none of them
// streaming twice the bytes of another.  256 threads; wave w runs tile w's
// chains.  Every workgroup normalises x itself (the reference's order,
// rmsnorm_quant_par :730-738) while its weight loads are in flight.
CPB_DEV_HOST_INLINE size_t qkv_lds_bytes(int d) {
    const int nbp = q8c_nbp(d / 32);
    // tiles' codes and scales, transposed x, red, activation dwords and scales
    return (size_t)kMaxTiles * ((nbp / 4) * 1024 + (nbp / 2) * 64) + sizeof(float) * (16 * attn_xt_stride(d) + 64) + (size_t)nbp * 36;
}
CPB_DEV_HOST_INLINE int qkv_groups(int tiles) {
    const int g = tiles < 256 ? tiles : 256;
    return g * kMaxTiles >= tiles ? g : (tiles + kMaxTiles - 1) / kMaxTiles;
}
template <int NSP>
__global__ __launch_bounds__(256) void k_attn_qkv(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nbp = q8c_nbp(a.nb), nsp = nbp / 4, ns = nbp / 2;
    u32x4* lw = (u32x4*)smem;                         // [kMaxTiles][nsp * 64]
    float* ls = (float*)(lw + kMaxTiles * nsp * 64);  // [kMaxTiles][ns * 16]
    float* xt = ls + kMaxTiles * ns * 16;             // [16][attn_xt_stride(d)] transposed x
    float* red = xt + 16 * attn_xt_stride(a.d);       // [64]
    uint32_t* xl = (uint32_t*)(red + 64);             // [nbp * 8]
    float* sl = (float*)(xl + nbp * 8);               // [nbp]
    __shared__ float hv[kMaxTiles][8];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // x and the norm weights first: the norm waits for them, not for the tiles
    // x in float4 slots tid + 256k: 3 per thread cover d <= 3072 (every
    // register-streamed shape: nbp = 92 blocks at most), 4 cover d <= 4096
    constexpr int KS = NSP > 0 ? 3 : 4;
    float4 xr[KS], wr[KS];
#pragma unroll
    for (int k = 0; k < KS; k++) {
        const int i4 = (tid + k * 256) * 4 < a.d ? tid + k * 256 : 0;
        xr[k] = ((const float4*)a.x)[i4];
        wr[k] = ((const float4*)a.L.norm)[i4];
    }
    const int T = (a.nh + 2 * a.nkv) * 8, G = gridDim.x;
    const int t0 = (int)((long long)blockIdx.x * T / G), nt = (int)((long long)(blockIdx.x + 1) * T / G) - t0;
    // this wave's tile: head, kind (0 q, 1 k, 2 v), the row of this lane's
    // slot r = lane / 8, its bias, and (lanes 0-3) the RoPE entries of pair
    // i = 4j + lane, all requested up front
    const int tw = t0 + (wave < nt ? wave : 0), head = tw >> 3, j = tw & 7;
    int kind, hh;
    if (head < a.nh) { kind = 0; hh = head; }
    else if (head < a.nh + a.nkv) { kind = 1; hh = head - a.nh; }
    else { kind = 2; hh = head - a.nh - a.nkv; }
    const float* B = kind == 0 ? a.L.bq : kind == 1 ? a.L.bk : a.L.bv;
    const int r = lane >> 3, rrow = (r < 4 ? 4 * j + r : 32 + 4 * j + r - 4);
    const float bias = B[hh * kAttnHd + rrow];
    const int ri = 4 * j + (lane & 3);
    const float rc = a.rope[((size_t)a.pos * 32 + ri) * 2], rs = a.rope[((size_t)a.pos * 32 + ri) * 2 + 1];
    TileSet ts;
    ts.w = a.L.wq + (size_t)t0 * nsp * 64;
    ts.s = a.L.sq + (size_t)t0 * ns * 16;
    ts.nt = nt;
    ts.nsp = nsp;
    // every wave's x requests go out before any wave's weight requests (an
    // execution barrier, no memory wait): x then lands ahead of the stream
    __builtin_amdgcn_s_barrier();
    u32x4 wreg[NSP > 0 ? NSP : 1];
    if constexpr (NSP > 0) {
        // the scales through LDS (requested first), each wave's own tile's
        // codes straight into its registers: unconditional loads (a wave past
        // the workgroup's tiles reads zeros from an empty range), so every
        // wait below is counted exactly
        StageRegs<0, kQkvScales> g;
        stage_issue(ts, g);
        const __amdgpu_buffer_rsrc_t rw =
            buf_rsrc(a.L.wq + (size_t)(t0 + (wave < nt ? wave : 0)) * NSP * 64, wave < nt ? (uint32_t)NSP * 64 * 16 : 0u);
        // half the codes before the norm, the rest after it (all of them up
        // front, or the rest as soon as x has landed, delays x and the norm
        // behind the other workgroups' streams: both measured slower)
        constexpr int kEarly = NSP / 2;
#pragma unroll
        for (int sp = 0; sp < kEarly; sp++)
            wreg[sp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)(sp * 64 + lane) * 16, 0, 2));
        attn_norm_q8(xr, wr, a.d, a.nb, nbp, a.eps, xt, red, xl, sl, blockIdx.x == 0 ? a.xq : nullptr, a.xsb);
#pragma unroll
        for (int sp = kEarly; sp < NSP; sp++)
            wreg[sp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)(sp * 64 + lane) * 16, 0, 2));
        stage_commit(ts, g, lw, ls);
    } else {
        StageRegs<kQkvLoads, kQkvScales> g;
        stage_issue(ts, g);
        attn_norm_q8(xr, wr, a.d, a.nb, nbp, a.eps, xt, red, xl, sl, blockIdx.x == 0 ? a.xq : nullptr, a.xsb);
        stage_commit(ts, g, lw, ls);
    }
    lds_barrier();
    if (wave >= nt) return;
    float v;
    if constexpr (NSP > 0) v = q8c_dot_regs<NSP>(wreg, ls + wave * ns * 16, xl, sl);
    else v = q8c_dot(lw + wave * nsp * 64, ls + wave * ns * 16, nbp, xl, sl);
    if ((lane & 7) == 0) hv[wave][r] = v + bias;      // :786-793 dot + bias (row)
    wave_sync_lds();
    if (lane >= 4) return;
    // RoPE pair (i, 32 + i), i = 4j + lane (rope_yarn :578-590); v unrotated
    const int i = 4 * j + lane;
    float lo = hv[wave][lane], hi = hv[wave][lane + 4];
    if (kind != 2) {
        const float nlo = lo * rc - hi * rs, nhi = hi * rc + lo * rs;
        lo = nlo;
        hi = nhi;
    }
    if (kind == 0) {
        a.q[hh * kAttnHd + i] = lo;
        a.q[hh * kAttnHd + 32 + i] = hi;
    } else {
        float* dst = (kind == 1 ? a.kc : a.vc) + ((size_t)hh * a.max_seq + a.pos) * kAttnHd;
        dst[i] = lo;
        dst[32 + i] = hi;
    }
}

// ---- attention of one kv-head's q-heads over one chunk of positions ----
// grid (nkv, nsplit), chunks of 128 positions (a window of 128 is one
// chunk); 512 threads, wave w runs q-head w of the group (two waves per SIMD
// hide each other's latencies), lane l positions l and l + 64.  With several chunks each workgroup leaves (max, sum, weighted
// v) per head and the last to arrive for its kv-head merges them with the
// sink; then the heads' outputs are quantised (qblock32 :691-699).
__device__ __forceinline__ float score64(const float* kr, const float4 (&qv)[16]) {
    // :810-820: 4 x 4 fma accumulators over steps of 16, then the fixed tree
    float4 kk[16];
#pragma unroll
    for (int i = 0; i < 16; i++) kk[i] = *(const float4*)&kr[4 * i];
    float acc[4][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int jj = 0; jj < 4; jj++)
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float4 kv = kk[jj * 4 + m];
            const float4 q4 = qv[jj * 4 + m];
            acc[m][0] = fmaf(kv.x, q4.x, acc[m][0]);
            acc[m][1] = fmaf(kv.y, q4.y, acc[m][1]);
            acc[m][2] = fmaf(kv.z, q4.z, acc[m][2]);
            acc[m][3] = fmaf(kv.w, q4.w, acc[m][3]);
        }
    float s4[4];
#pragma unroll
    for (int l = 0; l < 4; l++) s4[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    return ((s4[0] + s4[1]) + (s4[2] + s4[3])) * 0.125f;     // 1 / sqrt(64)
}


__global__ __launch_bounds__(512) void k_attn_core(AttnArgs a) {
    __shared__ __align__(16) float ks[kAttnChunk][68];
    __shared__ __align__(16) float vs[kAttnHd][kAttnChunk + 4];    // transposed: [dimension][position]
    __shared__ __align__(16) float es[kAttnMaxGroup][kAttnChunk];
    __shared__ int last;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvh = blockIdx.x, split = blockIdx.y, R = a.nh / a.nkv;
    const int p0 = a.start + split * kAttnChunk;
    const int cnt = min(kAttnChunk, a.pos + 1 - p0);
    const float* kb = a.kc + ((size_t)kvh * a.max_seq + p0) * kAttnHd;
    const float* vb = a.vc + ((size_t)kvh * a.max_seq + p0) * kAttnHd;
    constexpr int kIt = kAttnChunk * 16 / 512;
    static_assert(kIt * 512 == kAttnChunk * 16, "every LDS row of the chunk is written");
    const bool live = wave < R;                       // wave w runs q-head w of the group
    const int h = kvh * R + (live ? wave : 0);
    const float sink = a.L.sinks[h];
    {
        float4 kr[kIt], vr[kIt];
#pragma unroll
        for (int it = 0; it < kIt; it++) {
            const int e = it * 512 + tid, p = e >> 4, c = e & 15;
            // rows past the chunk take row 0 (stored, never read): no branch
            // around the stores, so the loads are not sunk into one each
            const int pc = p < cnt ? p : 0;
            kr[it] = *(const float4*)(kb + pc * kAttnHd + c * 4);
            vr[it] = *(const float4*)(vb + pc * kAttnHd + c * 4);
        }
#pragma unroll
        for (int it = 0; it < kIt; it++) {
            const int e = it * 512 + tid, p = e >> 4, c = e & 15;
            *(float4*)&ks[p][c * 4] = kr[it];
            vs[c * 4][p] = vr[it].x;
            vs[c * 4 + 1][p] = vr[it].y;
            vs[c * 4 + 2][p] = vr[it].z;
            vs[c * 4 + 3][p] = vr[it].w;
        }
    }
    __syncthreads();
    float mv = 0.0f, sv = 0.0f, ov = 0.0f, den = 1.0f;
    if (live) {
        // scores of positions lane and lane + 64, softmax weights
        // the head's q is uniform over the wave: scalar loads (constant
        // address space: q is not written during this launch), used as the
        // scalar operand of the score fmas, so the LDS serves only the K rows
        typedef __attribute__((address_space(4))) const float cfloat;
        cfloat* qc = (cfloat*)(a.q + (size_t)uniform(h) * kAttnHd);
        float4 qv[16];
#pragma unroll
        for (int i = 0; i < 16; i++) qv[i] = make_float4(qc[4 * i], qc[4 * i + 1], qc[4 * i + 2], qc[4 * i + 3]);
        const float s0 = lane < cnt ? score64(ks[lane], qv) : -INFINITY;
        const float s1 = lane + 64 < cnt ? score64(ks[lane + 64], qv) : -INFINITY;
        float m = wave_max_f32(fmaxf(s0, s1));
        if (a.nsplit == 1) m = fmaxf(m, sink);            // one chunk: the sink joins the max here
        const float e0 = lane < cnt ? expf(s0 - m) : 0.0f;
        const float e1 = lane + 64 < cnt ? expf(s1 - m) : 0.0f;
        if (a.nsplit > 1) sv = wave_sum_f32(e0 + e1);
        mv = m;
        es[wave][lane] = e0;
        es[wave][lane + 64] = e1;
        wave_sync_lds();
        const float* vrow = vs[lane];
        const float* er = es[wave];
        if (a.nsplit == 1) {
            // the reference's order (:823-831): den = exp(sink - mx), then += e in
            // position order; per dimension one fma chain over the positions; ao
            // = acc * (1 / den)
            float acc = 0.0f, d0 = expf(sink - m);
            int p = 0;
            if (cnt == kAttnChunk) {
                // a whole chunk: groups of 16 positions, the next group's LDS
                // reads issued before this group's chain steps
                float4 vv[2][4], ee[2][4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    vv[0][u] = *(const float4*)&vrow[4 * u];
                    ee[0][u] = *(const float4*)&er[4 * u];
                }
#pragma unroll
                for (int g = 0; g < kAttnChunk / 16; g++) {
                    const int b = g & 1;
                    if (g + 1 < kAttnChunk / 16) {
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            vv[b ^ 1][u] = *(const float4*)&vrow[16 * (g + 1) + 4 * u];
                            ee[b ^ 1][u] = *(const float4*)&er[16 * (g + 1) + 4 * u];
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const float4 v4 = vv[b][u], e4 = ee[b][u];
                        acc = fmaf(v4.x, e4.x, acc); acc = fmaf(v4.y, e4.y, acc);
                        acc = fmaf(v4.z, e4.z, acc); acc = fmaf(v4.w, e4.w, acc);
                        d0 += e4.x; d0 += e4.y; d0 += e4.z; d0 += e4.w;
                    }
                }
                p = kAttnChunk;
            }
#pragma unroll 4
            for (; p + 4 <= cnt; p += 4) {
                const float4 vv = *(const float4*)&vrow[p];
                const float4 e4 = *(const float4*)&er[p];
                acc = fmaf(vv.x, e4.x, acc); acc = fmaf(vv.y, e4.y, acc);
                acc = fmaf(vv.z, e4.z, acc); acc = fmaf(vv.w, e4.w, acc);
                d0 += e4.x; d0 += e4.y; d0 += e4.z; d0 += e4.w;
            }
            for (; p < cnt; p++) {
                acc = fmaf(vrow[p], er[p], acc);
                d0 += er[p];
            }
            ov = acc;
            den = d0;
        } else {
            // one chunk of several: 4 position chains, merged below with the sink
            float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            int p = 0;
            if (cnt == kAttnChunk) {
                float4 vv[2][4], ee[2][4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    vv[0][u] = *(const float4*)&vrow[4 * u];
                    ee[0][u] = *(const float4*)&er[4 * u];
                }
#pragma unroll
                for (int g = 0; g < kAttnChunk / 16; g++) {
                    const int b = g & 1;
                    if (g + 1 < kAttnChunk / 16) {
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            vv[b ^ 1][u] = *(const float4*)&vrow[16 * (g + 1) + 4 * u];
                            ee[b ^ 1][u] = *(const float4*)&er[16 * (g + 1) + 4 * u];
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const float4 v4 = vv[b][u], e4 = ee[b][u];
                        o[0] = fmaf(v4.x, e4.x, o[0]); o[1] = fmaf(v4.y, e4.y, o[1]);
                        o[2] = fmaf(v4.z, e4.z, o[2]); o[3] = fmaf(v4.w, e4.w, o[3]);
                    }
                }
                p = kAttnChunk;
            }
#pragma unroll 4
            for (; p + 4 <= cnt; p += 4) {
                const float4 vv = *(const float4*)&vrow[p];
                const float4 e4 = *(const float4*)&er[p];
                o[0] = fmaf(vv.x, e4.x, o[0]); o[1] = fmaf(vv.y, e4.y, o[1]);
                o[2] = fmaf(vv.z, e4.z, o[2]); o[3] = fmaf(vv.w, e4.w, o[3]);
            }
            for (; p < cnt; p++) o[0] = fmaf(vrow[p], er[p], o[0]);
            ov = (o[0] + o[1]) + (o[2] + o[3]);
        }
        if (a.nsplit == 1) {
            // softmax with the sink in the denominator, then Q8 of the head
            const float val = ov * (1.0f / den);
            a.ao[h * kAttnHd + lane] = val;
            const float mb = half_max_f32(fabsf(val));
            const float scq = fmaxf(1e-12f, mb) / 127.0f;
            a.aq[h * kAttnHd + lane] = (int8_t)q8_round(val, scq);
            if ((lane & 31) == 0) a.asb[h * 2 + (lane >> 5)] = scq;
        } else {
            // coherent (write-through) stores: read by another workgroup of this launch
            float* pp = a.part + ((size_t)h * a.nsplit + split) * 66;
            st_dev(pp + 2 + lane, ov);
            if (lane == 0) {
                st_dev(pp, mv);
                st_dev(pp + 1, sv);
            }
        }
    }
    if (a.nsplit == 1) return;
    // arrival: the last workgroup of this kv-head merges.  Each wave waits for
    // its stores to complete before the barrier; the counter is then bumped.
    drain_memory();
    __syncthreads();
    if (tid == 0) {
        const int prev = __hip_atomic_fetch_add(a.count + kvh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == a.nsplit - 1;
        if (last) __hip_atomic_store(a.count + kvh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last || !live) return;
    // the chunks' partials of this wave's head: coherent loads (they bypass
    // this CU's and this XCD's caches, which may hold older values), the first
    // kMergeRegs chunks all requested before any is used (one round trip;
    // nsplit <= max_seq / 128 <= 64)
    constexpr int kMergeRegs = 16;
    const float* pp = a.part + (size_t)h * a.nsplit * 66;
    const bool ok = lane < a.nsplit;
    const float mi = ok ? ld_dev(pp + lane * 66) : -INFINITY;
    const float lsum = ok ? ld_dev(pp + lane * 66 + 1) : 0.0f;
    float ovc[kMergeRegs];
#pragma unroll
    for (int c = 0; c < kMergeRegs; c++) ovc[c] = c < a.nsplit ? ld_dev(pp + c * 66 + 2 + lane) : 0.0f;
    const float M = wave_max_f32(fmaxf(mi, sink));
    const float f = ok ? expf(mi - M) : 0.0f;
    const float dsum = wave_sum_f32(ok ? lsum * f : 0.0f) + expf(sink - M);
    es[wave][lane] = f;
    wave_sync_lds();
    // weighted merge of the chunks' values, dimension lane
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < kMergeRegs; c++) o[c & 3] = fmaf(ovc[c], es[wave][c], o[c & 3]);
    for (int c = kMergeRegs; c < a.nsplit; c++) o[c & 3] = fmaf(ld_dev(pp + c * 66 + 2 + lane), es[wave][c], o[c & 3]);
    const float acc = (o[0] + o[1]) + (o[2] + o[3]);
    const float val = acc * (1.0f / dsum);
    a.ao[h * kAttnHd + lane] = val;
    const float mb = half_max_f32(fabsf(val));
    const float scq = fmaxf(1e-12f, mb) / 127.0f;
    a.aq[h * kAttnHd + lane] = (int8_t)q8_round(val, scq);
    if ((lane & 31) == 0) a.asb[h * 2 + (lane >> 5)] = scq;
}

// ---- x[r] += wo[r] . ao + bo[r] (:837), one 8-row tile per workgroup ----
__global__ __launch_bounds__(256) void k_attn_oproj(AttnArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nbp = q8c_nbp(a.nbo), nsp = nbp / 4, ns = nbp / 2;
    u32x4* lw = (u32x4*)smem;                         // [nsp * 64]
    float* ls = (float*)(lw + nsp * 64);              // [ns * 16]
    uint32_t* xl = (uint32_t*)(ls + ns * 16);         // [nbp * 8]
    float* sl = (float*)(xl + nbp * 8);               // [nbp]
    const int tile = blockIdx.x, tid = threadIdx.x;
    // activations, bias and the residual rows first (nbo <= 256: 8 dwords a thread)
    uint32_t ar[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = tid + k * 256;
        ar[k] = i < a.nbo * 8 ? ((const uint32_t*)a.aq)[i] : 0u;
    }
    const float as = tid < a.nbo ? a.asb[tid] : 0.0f;
    const int row = tile * 8 + ((tid >> 3) & 7);
    const float bo = a.L.bo[row], xo = a.x[row];
    TileSet ts;
    ts.w = a.L.wo + (size_t)tile * nsp * 64;
    ts.s = a.L.so + (size_t)tile * ns * 16;
    ts.nt = 1;
    ts.nsp = nsp;
    {
        StageRegs<kOprojLoads, kOprojScales> g;
        stage_issue(ts, g);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = tid + k * 256;
            if (i < nbp * 8) xl[xc_index(i)] = ar[k];
        }
        if (tid < nbp) sl[xs_index(tid)] = as;
        stage_commit(ts, g, lw, ls);
    }
    __syncthreads();
    if (tid >= 64) return;
    const float v = q8c_dot(lw, ls, nbp, xl, sl);
    if ((tid & 7) == 0) a.x[row] = xo + (v + bo);
}

// The o-projection at 64 heads (32 step pairs): one wave per 8-row tile,
// its codes loaded straight into registers in step order and the chain
// consuming each step pair as it lands.  Activations and the tile's scales
// go through LDS (the wave's own; no barrier).
__global__ __launch_bounds__(64) void k_attn_oproj_wave(AttnArgs a) {
    constexpr int NSP = 32, NBP = 4 * NSP, NS = 2 * NSP;
    __shared__ __align__(16) uint32_t xl[NBP * 8];
    __shared__ __align__(16) float sl[NBP];
    __shared__ __align__(16) float ls[NS * 16];
    const int tile = blockIdx.x, lane = threadIdx.x;
    // activations (nbo = NBP blocks: 16 dwords a lane), their scales, the tile's
    // scales, then the codes; bias and residual rows last
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a.aq, (uint32_t)NBP * 32);
    const __amdgpu_buffer_rsrc_t rsb = buf_rsrc(a.asb, (uint32_t)NBP * 4);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.L.so + (size_t)tile * NS * 16, (uint32_t)NS * 64);
    uint32_t ar[16];
#pragma unroll
    for (int k = 0; k < 16; k++) ar[k] = __builtin_amdgcn_raw_buffer_load_b32(ra, (uint32_t)(lane + k * 64) * 4, 0, 0);
    float as[2];
#pragma unroll
    for (int k = 0; k < 2; k++) as[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsb, (uint32_t)(lane + k * 64) * 4, 0, 0));
    u32x4 sc[4];
#pragma unroll
    for (int k = 0; k < 4; k++) sc[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(lane + k * 64) * 16, 0, 0));
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(a.L.wo + (size_t)tile * NSP * 64, (uint32_t)NSP * 64 * 16);
    u32x4 wreg[NSP];
#pragma unroll
    for (int sp = 0; sp < NSP; sp++)
        wreg[sp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)(sp * 64 + lane) * 16, 0, 2));
    const int row = tile * 8 + (lane >> 3);
    const float bo = a.L.bo[row], xo = a.x[row];
#pragma unroll
    for (int k = 0; k < 16; k++) xl[xc_index(lane + k * 64)] = ar[k];
#pragma unroll
    for (int k = 0; k < 2; k++) sl[xs_index(lane + k * 64)] = as[k];
#pragma unroll
    for (int k = 0; k < 4; k++) ((u32x4*)ls)[lane + k * 64] = sc[k];
    wave_sync_lds();
    const float v = q8c_dot_regs<NSP>(wreg, ls, xl, sl);
    if ((lane & 7) == 0) a.x[row] = xo + (v + bo);
}

// Step-pair counts with a register-streamed instantiation: q / k / v at
// d = 2880 (90 blocks padded to 92) and the o-projection at 64 heads (128
// blocks, k_attn_oproj_wave); other shapes take the LDS-staged kernels.
constexpr int kQkvNsp = 23, kOprojNsp = 32;
typedef void (*AttnKernel)(AttnArgs);
inline AttnKernel qkv_kernel(int nsp) { return nsp == kQkvNsp ? k_attn_qkv<kQkvNsp> : k_attn_qkv<0>; }

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
    float* part = nullptr;
    int* count = nullptr;
    int max_split = 1;
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
    if (c->n_head / c->n_head_kv > cpb::kAttnMaxGroup)
        return fail(CPB_EINVAL, "n_head / n_head_kv = %d: at most %d q-heads per kv-head", c->n_head / c->n_head_kv,
                    cpb::kAttnMaxGroup);
    if (c->n_head > 128) return fail(CPB_EINVAL, "n_head=%d: at most 128", c->n_head);
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
    // teardown: errors here have no caller to report to
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    for (void* p : h->layer_mem)
        if (p) (void)hipFree(p);
    void* bufs[] = {h->kc, h->vc, h->rope, h->x, h->xq, h->aq, h->xsb, h->q, h->ao, h->asb, h->part, h->count};
    for (void* p : bufs)
        if (p) (void)hipFree(p);
    if (h->own) (void)hipStreamDestroy(h->own);
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
    h->max_split = (cfg->max_seq + cpb::kAttnChunk - 1) / cpb::kAttnChunk;
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
        (r = dm((void**)&h->ao, nq * 4)) || (r = dm((void**)&h->aq, nq)) || (r = dm((void**)&h->asb, nq / 32 * 4)) ||
        (r = dm((void**)&h->part, (size_t)cfg->n_head * h->max_split * 66 * 4)) ||
        (r = dm((void**)&h->count, (size_t)cfg->n_head_kv * 4)))
        return bail(r);
    // LDS beyond 64 KiB per workgroup (d = 4096: 136 KiB for k_attn_qkv) is opted into
    {
        const int nbp = cpb::q8c_nbp(cfg->d / 32), nbpo = cpb::q8c_nbp(cfg->n_head * 2);
        const int lq = (int)cpb::qkv_lds_bytes(cfg->d);
        const int lo = (nbpo / 4) * 1024 + (nbpo / 2) * 64 + nbpo * 36;
        if (hipFuncSetAttribute((const void*)cpb::qkv_kernel(nbp / 4), hipFuncAttributeMaxDynamicSharedMemorySize, lq) != hipSuccess ||
            hipFuncSetAttribute((const void*)cpb::k_attn_oproj, hipFuncAttributeMaxDynamicSharedMemorySize, lo) != hipSuccess)
            return bail(fail(CPB_ENODEV, "LDS attribute (%d / %d bytes) refused", lq, lo));
        // static + dynamic LDS of every kernel the forward launches within the
        // device's per-workgroup limit (160 KiB on gfx950)
        int lim = 0;
        if (hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, device) != hipSuccess || lim <= 0)
            return bail(fail(CPB_ENODEV, "LDS limit query failed"));
        const struct { const void* f; size_t dyn; const char* name; } ks[] = {
            {(const void*)cpb::qkv_kernel(nbp / 4), (size_t)lq, "k_attn_qkv"},
            {(const void*)cpb::k_attn_core, 0, "k_attn_core"},
            {(const void*)cpb::k_attn_oproj, (size_t)lo, "k_attn_oproj"},
            {(const void*)cpb::k_attn_oproj_wave, 0, "k_attn_oproj_wave"}};
        for (const auto& k : ks) {
            hipFuncAttributes fa{};
            if (hipFuncGetAttributes(&fa, k.f) != hipSuccess) return bail(fail(CPB_ENODEV, "attributes of %s", k.name));
            if (fa.sharedSizeBytes + k.dyn > (size_t)lim)
                return bail(fail(CPB_EINVAL, "%s needs %zu + %zu bytes of LDS, above the device's %d", k.name,
                                 (size_t)fa.sharedSizeBytes, k.dyn, lim));
        }
    }
    std::vector<float> tab;
    rope_table(64, cfg->max_seq, cfg->rope_base, tab);
    if (hipMemcpy(h->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemsetAsync(h->kc, 0, cache, h->stream) != hipSuccess || hipMemsetAsync(h->vc, 0, cache, h->stream) != hipSuccess ||
        hipMemsetAsync(h->count, 0, (size_t)cfg->n_head_kv * 4, h->stream) != hipSuccess ||
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
    if (h->layer_mem[layer]) { (void)hipFree(h->layer_mem[layer]); h->layer_mem[layer] = nullptr; h->loaded[layer] = false; }
    const size_t d = c.d, nq = (size_t)c.n_head * 64, nkv = (size_t)c.n_head_kv * 64;
    // one allocation: the four Q8 code streams back to back (q, k, v form one
    // sequence of tiles for k_attn_qkv), then their scales, then the fp32 vectors
    const size_t mats[4][2] = {{nq, d}, {nkv, d}, {nkv, d}, {d, nq}};
    size_t off[4][2], o = 0;
    for (int m = 0; m < 4; m++) { off[m][0] = o; o += cpb::q8c_code_bytes((int)mats[m][0], (int)mats[m][1]); }
    o = (o + 255) / 256 * 256;
    for (int m = 0; m < 4; m++) { off[m][1] = o; o += cpb::q8c_scale_bytes((int)mats[m][0], (int)mats[m][1]); }
    o = (o + 255) / 256 * 256;
    const size_t wbytes = o;
    const size_t vec[6] = {d, nq, nkv, nkv, d, (size_t)c.n_head};      // norm, bq, bk, bv, bo, sinks
    size_t voff[6];
    for (int k = 0; k < 6; k++) { voff[k] = o; o += (vec[k] * 4 + 255) / 256 * 256; }
    unsigned char* base = nullptr;
    HIP_OK_A(hipMalloc((void**)&base, o));
    h->layer_mem[layer] = base;
    const uint16_t* srcs[4] = {wq, wk, wv, wo};
    uint16_t* staging = nullptr;
    hipError_t e = hipMalloc((void**)&staging, nq * d * 2);
    if (e == hipSuccess) e = hipMemsetAsync(base, 0, wbytes, h->stream);     // block padding
    for (int m = 0; m < 4 && e == hipSuccess; m++) {
        const size_t n = mats[m][0] * mats[m][1];
        e = hipMemcpyAsync(staging, srcs[m], n * 2, hipMemcpyHostToDevice, h->stream);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(cpb::k_q8c_quant, dim3(4096), dim3(256), 0, h->stream, staging, (int)mats[m][0],
                               (int)mats[m][1], (cpb::u32x4*)(base + off[m][0]), (float*)(base + off[m][1]), m < 3 ? 1 : 0);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    }
    if (staging) (void)hipFree(staging);
    const float* vsrc[6] = {attn_norm, bq, bk, bv, bo, sinks};
    for (int k = 0; k < 6 && e == hipSuccess; k++) e = hipMemcpy(base + voff[k], vsrc[k], vec[k] * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(CPB_ENODEV, "attention layer load: %s", hipGetErrorString(e));
    cpb::AttnLayerDev& L = h->layers[layer];
    L.wq = (const cpb::u32x4*)(base + off[0][0]); L.sq = (const float*)(base + off[0][1]);
    L.wk = (const cpb::u32x4*)(base + off[1][0]); L.sk = (const float*)(base + off[1][1]);
    L.wv = (const cpb::u32x4*)(base + off[2][0]); L.sv = (const float*)(base + off[2][1]);
    L.wo = (const cpb::u32x4*)(base + off[3][0]); L.so = (const float*)(base + off[3][1]);
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
    a.nsplit = (pos - a.start + 1 + cpb::kAttnChunk - 1) / cpb::kAttnChunk;
    a.L = h->layers[layer];
    a.x = dx;
    const size_t lc = (size_t)c.max_seq * c.n_head_kv * 64;
    a.kc = h->kc + (size_t)layer * lc;
    a.vc = h->vc + (size_t)layer * lc;
    a.rope = h->rope;
    a.xq = h->xq; a.xsb = h->xsb; a.q = h->q; a.ao = h->ao; a.aq = h->aq; a.asb = h->asb;
    a.part = h->part; a.count = h->count;
    const int nbpo = cpb::q8c_nbp(a.nbo);
    const size_t lds_o = (size_t)(nbpo / 4) * 1024 + (size_t)(nbpo / 2) * 64 + (size_t)nbpo * 36;
    cpb::launch(cpb::qkv_kernel(cpb::q8c_nbp(a.nb) / 4), dim3(cpb::qkv_groups((c.n_head + 2 * c.n_head_kv) * 8)), dim3(256), cpb::qkv_lds_bytes(c.d),
                h->stream, a);
    cpb::launch(cpb::k_attn_core, dim3(c.n_head_kv, a.nsplit), dim3(512), 0, h->stream, a);
    if (nbpo / 4 == cpb::kOprojNsp) cpb::launch(cpb::k_attn_oproj_wave, dim3(c.d / 8), dim3(64), 0, h->stream, a);
    else cpb::launch(cpb::k_attn_oproj, dim3(c.d / 8), dim3(256), lds_o, h->stream, a);
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
        // cache rows of pos: one 256-byte row per kv-head ([nkv][max_seq][64])
        if (tr->k) HIP_OK_A(hipMemcpy2DAsync(tr->k, 256, h->kc + (size_t)layer * lc + (size_t)pos * 64,
                                             (size_t)c.max_seq * 256, 256, c.n_head_kv, hipMemcpyDeviceToHost, h->stream));
        if (tr->v) HIP_OK_A(hipMemcpy2DAsync(tr->v, 256, h->vc + (size_t)layer * lc + (size_t)pos * 64,
                                             (size_t)c.max_seq * 256, 256, c.n_head_kv, hipMemcpyDeviceToHost, h->stream));
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
