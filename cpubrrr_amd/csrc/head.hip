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
// bytes (1 KB, one wavefront load) and 64 x bf16 scales; the Q2 stream (the
// reference's CPBRR_HEAD2 option) the same with 8 code bytes per lane (two
// blocks per 16-byte lane unit measured slower: fewer loads in flight); the Q8 rows stay
// row-major (only the few candidate rows are read).  The screen is a
// bandwidth-bound GEMV over 4.5 bits per weight (~326 MB for gpt-oss's
// 201088 x 2880 head), one lane per row.
//
// Kernels per token: k_head_norm (rmsnorm + Q8 of the hidden state);
// k_head_screen (every row's screen value; each 256-row workgroup also leaves
// its best n_cand rows in every worker slice it meets); k_head_refine (one
// workgroup per worker slice: the slice's best n_cand from those lists, their
// exact Q8 logits; the last workgroup to finish takes the greedy choice).
// A slice's best n_cand by the reference's insertion (strict comparisons) are
// its n_cand largest values, equal values in row order; every selection here
// ranks by that order.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdio>
#include <mutex>
#include <vector>

#include "cpb_head.h"
#include "cpb_internal.h"
#include "moe_common.h"
#include "route_dev.h"

namespace cpb {

constexpr int kHeadRT = 64;          // rows per stream tile
constexpr int kHeadMaxCand = 16;
constexpr int kHeadMaxSlices = 32;
constexpr int kHeadGroupRows = 4 * 64;    // rows of one screen workgroup (4 tiles)

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
    const uint64_t* q2;    // [Vpad/64][nb][64] Q2 bytes (8 per row and block)
    const uint16_t* q2s;   // [Vpad/64][nb][64] bf16 scales
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
    // per worker slice: the rows' tiles and where their candidates go
    const int32_t* wtab;   // [nt][2]: first screen workgroup (256 rows), base offset into candv / candi
    float* candv;          // per (worker, workgroup): its best n_cand screen values in the slice
    int32_t* candi;        //   and their rows (INT32_MAX: none)
    int32_t* count;        // [1] arrivals of the refine workgroups (0 between launches)
};

// rows of worker slice w: quads [nq su(w) / tu, nq su(w + 1) / tu), the
// reference's sl() (engine_gpt2.rs:636-642) with its unit weights (wunits,
// total_units :29-38): 5 units for workers 0-11, 2 for workers 12 and above,
// tu = su(nt)
CPB_DEV_HOST_INLINE long head_units(int w) { return w < 12 ? 5L * w : 60L + 2L * (w - 12); }
CPB_DEV_HOST_INLINE int slice_r0(long nq, int nt, int w) { return (int)(4 * (nq * head_units(w) / head_units(nt))); }

// ---- cross-lane helpers on DPP + readlane ----
template <int CTRL>
CPB_DEV float dpp_fh(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false)); }
template <int CTRL>
CPB_DEV int dpp_ih(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }

// (value, index) order of the screen: larger value first, then lower index
CPB_DEV bool better(float v, int i, float w, int j) { return v > w || (v == w && i < j); }
template <int CTRL>
CPB_DEV void best_step(float& v, int& i) {
    const float ov = dpp_fh<CTRL>(v);
    const int oi = dpp_ih<CTRL>(i);
    if (better(ov, oi, v, i)) { v = ov; i = oi; }
}
// the best (value, index) of the wave, in every lane
CPB_DEV void wave_best(float& v, int& i) {
    best_step<0xB1>(v, i);       // lane ^ 1
    best_step<0x4E>(v, i);       // lane ^ 2
    best_step<0x141>(v, i);      // mirror within 8
    best_step<0x140>(v, i);      // mirror within 16
    float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), r));
        const int ri = __builtin_amdgcn_readlane(i, r);
        if (better(rv, ri, bv, bi)) { bv = rv; bi = ri; }
    }
    v = bv;
    i = bi;
}

// 64-bit key ordered as better(): the value's bits made monotonic (-0 as +0,
// as the float comparisons treat them), then the complement of the index
CPB_DEV uint64_t rank_key(float v, int i) {
    uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}
// rank of this lane's (value, index) among the wave's 64 (the number of
// better entries; sentinels (-inf, INT32_MAX) are below every entry).  sk:
// this wave's 64-entry LDS scratch.
CPB_DEV int wave_rank(float v, int i, uint64_t* sk) {
    const int lane = threadIdx.x & 63;
    const uint64_t k = rank_key(v, i);
    sk[lane] = k;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int r[4] = {0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < 32; q++) {
        const ulonglong2 o = ((const ulonglong2*)sk)[q];
        r[q & 3] += (o.x > k) + (o.y > k);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return (r[0] + r[1]) + (r[2] + r[3]);
}

// ---- load time: Q4Mat, Q2Mat and Q8Mat rows from bf16, one thread per (row, block) ----
__global__ void k_head_quant(const uint16_t* __restrict__ w, int V, int Vpad, int d, u32x4* __restrict__ q4,
                             uint16_t* __restrict__ q4s, uint64_t* __restrict__ q2, uint16_t* __restrict__ q2s,
                             int8_t* __restrict__ q8, float* __restrict__ q8s) {
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
        // Q2Mat (:366-399): scale bf16(vmax / -2), code clamp(floor(v / scale
        // + 2.5), 0, 3); byte j holds elements j, j + 8, j + 16, j + 24
        {
            const uint32_t db2 = f32_to_bf16(vmax / -2.0f);
            const float dq2 = bf16f(db2);
            const float idq2 = dq2 != 0.0f ? 1.0f / dq2 : 0.0f;
            uint64_t bytes = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint32_t byte = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    int c = (int)floorf(vals[j + 8 * k] * idq2 + 2.5f);
                    c = c < 0 ? 0 : c > 3 ? 3 : c;
                    byte |= (uint32_t)c << (2 * k);
                }
                bytes |= (uint64_t)byte << (8 * j);
            }
            q2[u] = bytes;
            q2s[u] = (uint16_t)db2;
        }
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
    // 4 lanes per block, 8 consecutive values each (lane q: elements 8q .. 8q + 7)
    for (int e = tid; e < a.nb * 4; e += blockDim.x) {
        const int bk = e >> 2, q = e & 3;
        float v[8];
        float m = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            v[u] = xnl[bk * 32 + 8 * q + u];
            m = fmaxf(m, fabsf(v[u]));
        }
        m = fmaxf(m, dpp_fh<0xB1>(m));
        m = fmaxf(m, dpp_fh<0x4E>(m));
        const float sc = fmaxf(1e-12f, m) / 127.0f;
        // q8_round of the 8 values, the exact division only near a tie
        float r[8];
        {
            const float rs = __builtin_amdgcn_rcpf(sc);
            bool near = false;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float y = v[u] * rs;
                r[u] = __builtin_rintf(y);
                near = near || q8_near_half(y);
            }
            if (near) {
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (q8_near_half(v[u] * rs)) r[u] = roundf(v[u] / sc);
            }
        }
        uint32_t wd[2] = {0u, 0u};
        int slo = 0, shi = 0;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int qv = q8_clamp(r[u]);
            wd[u >> 2] |= (uint32_t)(uint8_t)qv << (8 * (u & 3));
            if (u < 4) slo += qv; else shi += qv;
        }
        ((uint2*)a.xq)[bk * 4 + q] = make_uint2(wd[0], wd[1]);
        if (q == 0) a.xsb[bk] = sc;
        // lane part j of the screen dot = elements 4j..4j+3 and 16+4j..16+4j+3:
        // j = 0, 1 from lanes 0 and 2 (low / high four), j = 2, 3 from lanes 1 and 3
        const int plo = slo + dpp_ih<0x4E>(slo), phi = shi + dpp_ih<0x4E>(shi);
        if (q < 2) {
            a.xs8[bk * 4 + 2 * q] = plo;
            a.xs8[bk * 4 + 2 * q + 1] = phi;
        }
    }
}

// ---- screen of every row: one lane per row.  Q4 (dot4_q4_i8, :314-342) or
// Q2 (dot4_q2_i8, :403-428; head2_on() at :953-957 selects it), the same
// lane order: lane part j = elements 4j..4j+3 and 16+4j..16+4j+3, an int
// dot per block, acc_j = fma(t_j, bf16 scale * xsb, acc_j) ----
constexpr int kScreenRing = 6;
template <bool Q2>
__global__ __launch_bounds__(256) void k_head_screen(HeadDev a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nb = a.nb, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t* xl = (uint32_t*)smem;                    // xq as dwords [nb][8]
    float* xsl = (float*)(xl + nb * 8);                // [nb]
    int32_t* x8 = (int32_t*)(xsl + nb);                // [nb][4]
    __shared__ __align__(16) uint64_t rsk[4][64];
    __shared__ float lv[kHeadMaxSlices][4][kHeadMaxCand];
    __shared__ int li[kHeadMaxSlices][4][kHeadMaxCand];
    const int tile = blockIdx.x * 4 + wave;
    const bool live = tile * kHeadRT < a.Vpad;
    float val = -INFINITY;
    const int row = tile * kHeadRT + lane;
    // Each lane streams its row's blocks through a ring of kScreenRing
    // loads: block b's codes and scale are requested kScreenRing blocks
    // before they are used, so the loads in flight never drain between
    // groups.  Buffer loads over the tile's streams: requests past the last
    // block fall outside the resource and fetch nothing; a wave past the last
    // tile gets empty resources.  The ring's first loads go out before x is
    // staged in LDS (they do not need it).
    {
        const size_t tb = live ? (size_t)tile * nb * kHeadRT : 0;
        const uint32_t nr = live ? (uint32_t)(nb * kHeadRT) : 0u;
        const __amdgpu_buffer_rsrc_t rw = Q2 ? buf_rsrc(a.q2 + tb, nr * 8) : buf_rsrc(a.q4 + tb, nr * 16);
        const __amdgpu_buffer_rsrc_t rsc = buf_rsrc((Q2 ? a.q2s : a.q4s) + tb, nr * 2);
        constexpr uint32_t ub = Q2 ? 8 : 16;                 // code bytes per lane and block
        const uint32_t wo = (uint32_t)lane * ub, so = (uint32_t)lane * 2;
        auto ldw = [&](int b) -> u32x4 {
            if constexpr (Q2) {
                const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, wo, b * kHeadRT * (int)ub, 2));
                return u32x4{v.x, v.y, 0u, 0u};
            } else {
                return __builtin_amdgcn_raw_buffer_load_b128(rw, wo, b * kHeadRT * (int)ub, 2);
            }
        };
        // lane offsets in fixed registers, the block's offset in a scalar one
        // (scales held as 32-bit values: 16-bit ones were packed in pairs
        // across the loop, which waited for both loads)
        auto lds = [&](int b) -> uint32_t { return __builtin_amdgcn_raw_buffer_load_b16(rsc, so, b * kHeadRT * 2, 2); };
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        u32x4 wq[kScreenRing];
        uint32_t sq[kScreenRing];
#pragma unroll
        for (int k = 0; k < kScreenRing; k++) {
            wq[k] = ldw(k);
            sq[k] = lds(k);
            __builtin_amdgcn_sched_barrier(0);          // the loop's order, for exact waits
        }
        for (int i = tid; i < nb * 8; i += blockDim.x) xl[i] = ((const uint32_t*)a.xq)[i];
        for (int i = tid; i < nb; i += blockDim.x) xsl[i] = a.xsb[i];
        for (int i = tid; i < nb * 4; i += blockDim.x) x8[i] = a.xs8[i];
        __syncthreads();
        auto block = [&](int b, const u32x4& w, float sv) {
            if constexpr (Q2) {
                const uint32_t w0 = w[0], w1 = w[1];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    // elements 4j..4j+3: bytes 4 (j & 1) .. +3, bits 2 (j >> 1);
                    // elements 16+4j..: the same bytes, bits 4 + 2 (j >> 1)
                    const uint32_t src = (j & 1) ? w1 : w0;
                    const int sh = 2 * (j >> 1);
                    int t = sdot4((src >> sh) & 0x03030303u, xl[b * 8 + j], 0);
                    t = sdot4((src >> (sh + 4)) & 0x03030303u, xl[b * 8 + 4 + j], t);
                    t -= 2 * x8[b * 4 + j];                    // codes are KVI2[c] = c - 2
                    acc[j] = fmaf((float)t, sv, acc[j]);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int t = sdot4(w[j] & 0x0F0F0F0Fu, xl[b * 8 + j], 0);
                    t = sdot4((w[j] >> 4) & 0x0F0F0F0Fu, xl[b * 8 + 4 + j], t);
                    t -= 8 * x8[b * 4 + j];                    // codes are KVI4[c] = c - 8
                    acc[j] = fmaf((float)t, sv, acc[j]);
                }
            }
        };
        // whole groups with no branch inside (a branch there made the
        // compiler wait for every load in flight at each block), then the
        // last nb % kScreenRing blocks from the ring
        const int nfull = nb - nb % kScreenRing;
        for (int b0 = 0; b0 < nfull; b0 += kScreenRing) {
#pragma unroll
            for (int k = 0; k < kScreenRing; k++) {
                const int b = b0 + k;
                block(b, wq[k], bf16f(sq[k]) * xsl[b]);
                // the refill after the block's last use of its registers, so
                // that it lands in the same ones (a refill issued before the
                // use left the loop rotating copies that waited for every
                // load), and kept there
                __builtin_amdgcn_sched_barrier(0);
                wq[k] = ldw(b + kScreenRing);
                sq[k] = lds(b + kScreenRing);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int k = 0; k < kScreenRing - 1; k++)
            if (nfull + k < nb) block(nfull + k, wq[k], bf16f(sq[k]) * xsl[nfull + k]);
        if (live) {
            val = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            a.screen[row] = val;
        }
    }
    // the workgroup's best n_cand rows in each worker slice it meets (a slice's
    // best n_cand are among its row groups' best n_cand): per tile by rank,
    // then the four tiles' lists by rank again
    const long nq = a.V / 4;
    const int C = a.nc;
    const int glo = blockIdx.x * 4 * kHeadRT, ghi = min(glo + 4 * kHeadRT, a.V) - 1;
    int wa = (int)((long)(glo / 4) * a.nt / nq);
    while (wa > 0 && slice_r0(nq, a.nt, wa) > glo) wa--;
    while (wa + 1 < a.nt && slice_r0(nq, a.nt, wa + 1) <= glo) wa++;
    int wb = wa;
    while (wb + 1 < a.nt && slice_r0(nq, a.nt, wb + 1) <= ghi) wb++;
    for (int w = wa; w <= wb; w++) {
        const int r0 = slice_r0(nq, a.nt, w), r1 = slice_r0(nq, a.nt, w + 1);
        // head_worker inserts only values above its initial -FLT_MAX
        const bool in = live && row >= r0 && row < r1 && row < a.V && val > -FLT_MAX;
        const float v = in ? val : -INFINITY;
        const int i = in ? row : INT32_MAX;
        const int rank = wave_rank(v, i, rsk[wave]);
        if (in && rank < C) { lv[w - wa][wave][rank] = v; li[w - wa][wave][rank] = i; }
        const int n_in = __builtin_popcountll(__ballot(in));
        if (lane >= n_in && lane < C) { lv[w - wa][wave][lane] = -INFINITY; li[w - wa][wave][lane] = INT32_MAX; }
    }
    __syncthreads();
    for (int w = wa + wave; w <= wb; w += 4) {
        const int r0 = slice_r0(nq, a.nt, w), r1 = slice_r0(nq, a.nt, w + 1);
        if (r0 == r1) continue;
        const bool has = lane < 4 * C;
        const float v = has ? lv[w - wa][lane / C][lane % C] : -INFINITY;
        const int i = has ? li[w - wa][lane / C][lane % C] : INT32_MAX;
        const int rank = wave_rank(v, i, rsk[wave]);
        const size_t slot = (size_t)a.wtab[2 * w + 1] + (size_t)(blockIdx.x - a.wtab[2 * w]) * C;
        const bool real = i != INT32_MAX;
        if (real && rank < C) { a.candv[slot + rank] = v; a.candi[slot + rank] = i; }
        const int n_real = __builtin_popcountll(__ballot(real));
        if (lane >= n_real && lane < C) { a.candv[slot + lane] = -INFINITY; a.candi[slot + lane] = INT32_MAX; }
    }
}

// ---- per worker slice: merge the tiles' candidates into the n_cand best
// (the reference's insertion keeps the n_cand largest values, equal values in
// row order), their exact Q8 logits (dot_q8_i8, :169-191), then the greedy
// choice over all workers' candidates in worker / rank order (:128-134) by the
// last workgroup to finish.  grid: n_slices workgroups of 1024 threads.
constexpr int kRefineWaves = 16;
__global__ __launch_bounds__(1024) void k_head_refine(HeadDev a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int C = a.nc, nb = a.nb, d = a.d;
    u32x4* rows = (u32x4*)smem;                        // [C][d / 16] candidate rows' Q8 codes
    float* rs = (float*)(rows + (size_t)C * (d / 16)); // [C][nb] their scales
    uint32_t* xl = (uint32_t*)(rs + C * nb);           // xq as dwords [nb][8]
    float* xsl = (float*)(xl + nb * 8);                // [nb]
    __shared__ float wv[kRefineWaves][kHeadMaxCand];
    __shared__ int wi[kRefineWaves][kHeadMaxCand];
    __shared__ float wv2[4][kHeadMaxCand];
    __shared__ int wi2[4][kHeadMaxCand];
    __shared__ __align__(16) float rsv[kRefineWaves][64];
    __shared__ __align__(16) int rsi[kRefineWaves][64];
    __shared__ __align__(16) uint64_t rsk[kRefineWaves][64];
    __shared__ int cid[kHeadMaxCand];
    __shared__ float lgs[128];
    __shared__ int ids_s[128];
    __shared__ int last;
    const int w = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < nb * 8; i += 1024) xl[i] = ((const uint32_t*)a.xq)[i];
    for (int i = tid; i < nb; i += 1024) xsl[i] = a.xsb[i];
    const long nq = a.V / 4;
    const int r0 = slice_r0(nq, a.nt, w), r1 = slice_r0(nq, a.nt, w + 1);
    const int M = r0 == r1 ? 0 : ((r1 - 1) / kHeadGroupRows - a.wtab[2 * w] + 1) * C;
    const float* cv = a.candv + a.wtab[2 * w + 1];
    const int* ci = a.candi + a.wtab[2 * w + 1];
    // each wave: chunks of 64 entries by rank, folded into a running best n_cand
    {
        const int nchunk = (M + 63) / 64;
        float runv = -INFINITY;
        int runi = INT32_MAX;                 // lane k < C: the wave's k-th best so far
        for (int ch = wave; ch < nchunk; ch += kRefineWaves) {
            const int e = ch * 64 + lane;
            const float v = e < M ? cv[e] : -INFINITY;
            const int i = e < M ? ci[e] : INT32_MAX;
            const int rank = wave_rank(v, i, rsk[wave]);
            // lanes C .. 2C - 1: this chunk's best n_cand, then rank the 2C
            float mv = lane < C ? runv : -INFINITY;
            int mi = lane < C ? runi : INT32_MAX;
            rsv[wave][lane] = -INFINITY;
            rsi[wave][lane] = INT32_MAX;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (i != INT32_MAX && rank < C) { rsv[wave][C + rank] = v; rsi[wave][C + rank] = i; }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (lane >= C && lane < 2 * C) { mv = rsv[wave][lane]; mi = rsi[wave][lane]; }
            const int r2 = wave_rank(mv, mi, rsk[wave]);
            rsv[wave][lane] = -INFINITY;
            rsi[wave][lane] = INT32_MAX;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (mi != INT32_MAX && r2 < C) { rsv[wave][r2] = mv; rsi[wave][r2] = mi; }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            runv = rsv[wave][lane];
            runi = rsi[wave][lane];
        }
        if (lane < C) { wv[wave][lane] = runv; wi[wave][lane] = runi; }
    }
    __syncthreads();
    // waves 0-3: the n_cand best of four waves' lists each
    if (wave < 4) {
        const float v = lane < 4 * C ? wv[4 * wave + lane / C][lane % C] : -INFINITY;
        const int i = lane < 4 * C ? wi[4 * wave + lane / C][lane % C] : INT32_MAX;
        const int rank = wave_rank(v, i, rsk[wave]);
        if (i != INT32_MAX && rank < C) { wv2[wave][rank] = v; wi2[wave][rank] = i; }
        const int n_real = __builtin_popcountll(__ballot(i != INT32_MAX));
        if (lane >= n_real && lane < C) { wv2[wave][lane] = -INFINITY; wi2[wave][lane] = INT32_MAX; }
    }
    __syncthreads();
    // wave 0: the n_cand best of those four
    if (wave == 0) {
        const float v = lane < 4 * C ? wv2[lane / C][lane % C] : -INFINITY;
        const int i = lane < 4 * C ? wi2[lane / C][lane % C] : INT32_MAX;
        const int rank = wave_rank(v, i, rsk[0]);
        const bool real = i != INT32_MAX;
        if (real && rank < C) {
            cid[rank] = i;
            st_dev(a.cand_ids + w * C + rank, i);
            st_dev(a.cand_screen + w * C + rank, v);
        }
        const int n_real = __builtin_popcountll(__ballot(real));
        // fewer than n_cand rows: the reference's initial entries (-FLT_MAX, row 0)
        if (lane >= n_real && lane < C) {
            cid[lane] = 0;
            st_dev(a.cand_ids + w * C + lane, 0);
            st_dev(a.cand_screen + w * C + lane, -FLT_MAX);
        }
    }
    __syncthreads();
    // the candidates' Q8 rows and scales into LDS, every load in flight at once
    {
        const int per = d / 16;
        for (int e = tid; e < C * per; e += 1024) {
            const int c = e / per, o = e - c * per;
            rows[e] = *((const u32x4*)(a.q8 + (size_t)cid[c] * d) + o);
        }
        for (int e = tid; e < C * nb; e += 1024) {
            const int c = e / nb, o = e - c * nb;
            rs[e] = a.q8s[(size_t)cid[c] * nb + o];
        }
    }
    __syncthreads();
    // exact Q8 logits: 8 lanes per candidate, lane (h, j) runs the reference's
    // chain j of the even (h = 0) or odd (h = 1) blocks
    if (tid < C * 8) {
        const int c = tid >> 3, h = (tid >> 2) & 1, j = tid & 3;
        const uint32_t* q = (const uint32_t*)(rows + (size_t)c * (d / 16));
        const float* sc = rs + c * nb;
        const int nbe = nb & ~1;
        float acc = 0.0f;
        auto blk = [&](int b) {
            const int t = sdot4(q[b * 8 + 4 + j], xl[b * 8 + 4 + j], sdot4(q[b * 8 + j], xl[b * 8 + j], 0));
            acc = fmaf((float)t, sc[b] * xsl[b], acc);
        };
#pragma unroll 4
        for (int b = h; b < nbe; b += 2) blk(b);
        if ((nb & 1) && h == 0) blk(nb - 1);       // an odd last block goes into the first accumulator
        // lanes 0-3 of each group of 8: v_j = acc0_j + acc1_j (lane + 4: row_ror by 12),
        // then lane 0: (v0 + v1) + (v2 + v3)
        const float v = acc + dpp_fh<0x12C>(acc);
        const float v01 = v + dpp_fh<0xB1>(v);
        const float tot = v01 + dpp_fh<0x4E>(v01);
        if ((tid & 7) == 0) st_dev(a.cand_logits + w * C + c, tot);
    }
    // arrival: the last workgroup takes the greedy choice
    drain_memory();
    __syncthreads();
    if (tid == 0) {
        const int prev = __hip_atomic_fetch_add(a.count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == a.nt - 1;
        if (last) __hip_atomic_store(a.count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    const int nc = a.nt * C;
    if (tid < nc) {
        lgs[tid] = ld_dev(a.cand_logits + tid);
        ids_s[tid] = ld_dev(a.cand_ids + tid);
    }
    __syncthreads();
    if (tid == 0) {
        float best = -FLT_MAX;
        int bi = 0;
        for (int k = 0; k < nc; k++)
            if (lgs[k] > best) { best = lgs[k]; bi = ids_s[k]; }
        *a.chosen = bi;
    }
}

// LDS of k_head_refine: candidate rows and scales, activations
inline size_t head_refine_lds(int d, int nc) { return (size_t)nc * d + (size_t)nc * (d / 32) * 4 + (size_t)(d / 32) * 36; }

}  // namespace cpb

using cpb::fail;

constexpr int kHeadBufs = 18;

struct cpb_head {
    cpb_head_cfg cfg{};
    int device = 0;
    hipStream_t own = nullptr, stream = nullptr;
    cpb::HeadDev a{};
    void* base[kHeadBufs] = {};
    bool loaded = false;
    bool q2 = false;          // screen with the Q2 rows (cpb_head_set_screen)
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
    *out = vpad(c) * nb * (16 + 2 + 8 + 2) + (size_t)c->n_vocab * (c->d + nb * 4);
    return 0;
}

void cpb_head_destroy(cpb_head_t* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    for (void* p : h->base)
        if (p) (void)hipFree(p);
    if (h->own) (void)hipStreamDestroy(h->own);
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
    // worker slices: first tile and candidate offset of each
    std::vector<int32_t> wtab(2 * a.nt);
    size_t ncand = 0;
    {
        const long nq = a.V / 4;
        for (int w = 0; w < a.nt; w++) {
            const int r0 = cpb::slice_r0(nq, a.nt, w), r1 = cpb::slice_r0(nq, a.nt, w + 1);
            wtab[2 * w] = r0 / cpb::kHeadGroupRows;
            wtab[2 * w + 1] = (int32_t)ncand;
            if (r1 > r0) ncand += (size_t)((r1 - 1) / cpb::kHeadGroupRows - r0 / cpb::kHeadGroupRows + 1) * a.nc;
        }
    }
    const size_t sizes[kHeadBufs] = {(size_t)a.Vpad * nb * 16, (size_t)a.Vpad * nb * 2, (size_t)a.V * a.d,
                                     (size_t)a.V * nb * 4, (size_t)a.d * 4, (size_t)a.d * 4,
                                     (size_t)a.d + nb * 4 + nb * 16, (size_t)a.Vpad * 4, nc * 4, nc * 4, nc * 4, 4,
                                     wtab.size() * 4, ncand * 4, ncand * 4, 4, (size_t)a.Vpad * nb * 8,
                                     (size_t)a.Vpad * nb * 2};
    for (int i = 0; i < kHeadBufs; i++) {
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
    a.wtab = (const int32_t*)h->base[12];
    a.candv = (float*)h->base[13];
    a.candi = (int32_t*)h->base[14];
    a.count = (int32_t*)h->base[15];
    a.q2 = (const uint64_t*)h->base[16];
    a.q2s = (const uint16_t*)h->base[17];
    if (hipFuncSetAttribute((const void*)cpb::k_head_refine, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)cpb::head_refine_lds(a.d, a.nc)) != hipSuccess)
        return bail(fail(CPB_ENODEV, "LDS attribute refused"));
    if (hipMemcpy(h->base[12], wtab.data(), wtab.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(a.count, 0, 4) != hipSuccess)
        return bail(fail(CPB_ENODEV, "head init copies failed"));
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
                           (cpb::u32x4*)a.q4, (uint16_t*)a.q4s, (uint64_t*)a.q2, (uint16_t*)a.q2s, (int8_t*)a.q8,
                           (float*)a.q8s);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    (void)hipFree(staging);
    if (e != hipSuccess) return fail(CPB_ENODEV, "head load: %s", hipGetErrorString(e));
    h->loaded = true;
    return 0;
}

// x: the hidden state (device), chosen: where the token goes (device)
static int head_launch(cpb_head_t* h, const float* x, int32_t* chosen) {
    cpb::HeadDev a = h->a;
    a.x = x;
    a.chosen = chosen;
    cpb::launch(cpb::k_head_norm, dim3(1), dim3(256), sizeof(float) * (2 * a.d + 64), h->stream, a);
    const int tiles = a.Vpad / cpb::kHeadRT;
    if (h->q2) cpb::launch(cpb::k_head_screen<true>, dim3((tiles + 3) / 4), dim3(256), (size_t)a.nb * (32 + 4 + 16), h->stream, a);
    else cpb::launch(cpb::k_head_screen<false>, dim3((tiles + 3) / 4), dim3(256), (size_t)a.nb * (32 + 4 + 16), h->stream, a);
    cpb::launch(cpb::k_head_refine, dim3(a.nt), dim3(1024), cpb::head_refine_lds(a.d, a.nc), h->stream, a);
    return hipGetLastError() == hipSuccess ? 0 : fail(CPB_ENODEV, "head launch failed");
}

int cpb_head_forward_device(cpb_head_t* h, const float* d_x, int32_t* d_chosen) {
    if (!h || !d_x || !d_chosen) return fail(CPB_EINVAL, "NULL argument");
    if (!h->loaded) return fail(CPB_ESTATE, "head not loaded");
    HIP_OK_H(hipSetDevice(h->device));
    return head_launch(h, d_x, d_chosen);
}

int cpb_head_forward(cpb_head_t* h, const float* x, int32_t* chosen, cpb_head_trace* tr) {
    if (!h || !x || !chosen) return fail(CPB_EINVAL, "NULL argument");
    if (!h->loaded) return fail(CPB_ESTATE, "head not loaded");
    HIP_OK_H(hipSetDevice(h->device));
    const cpb::HeadDev& a = h->a;
    HIP_OK_H(hipMemcpyAsync((void*)a.x, x, (size_t)a.d * 4, hipMemcpyHostToDevice, h->stream));
    if (int r = head_launch(h, a.x, a.chosen)) return r;
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

int cpb_head_set_screen(cpb_head_t* h, int bits) {
    if (!h) return fail(CPB_EINVAL, "handle is NULL");
    if (bits != 4 && bits != 2) return fail(CPB_EINVAL, "screen bits %d: 4 (Q4, default) or 2 (Q2)", bits);
    h->q2 = bits == 2;
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
