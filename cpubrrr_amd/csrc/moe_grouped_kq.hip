// moe_grouped_kq.hip -- batched / prefill Qwen3 MoE layer on the int8 matrix
// cores (gfx950): Q4_K gate/up, Q4_K or Q6_K down.
//
// Reference: the k-wide superblock dot q4k_dot_k (engine_qwen2.rs:115-163:
// "read each weight row ONCE, dot against k activation vectors"), whose
// results are q4k_dot's per token; the layer is engine_qwen2.rs:395-433.
// Tokens' (token, slot) pairs are grouped by expert (moe_grouped.hip) and each
// expert's products run as v_mfma_i32_32x32x32_i8 over 32 weight rows x 32
// tokens x one 32-element scale group:
//   Q4_K: A = the group's 4-bit quants (0..15, exact int8), B = Q8_K
//         activations: D = the reference's per-32 integer dot;
//   Q6_K: A = q - 32 (in [-32, 31], exact int8) of two 16-element groups in
//         the two K halves, B = the activations of one group with the other
//         half zero (two instructions per 32 elements): D = the per-16 dot of
//         (q - 32) and x, i.e. s_g - 32 * sum_g(x) of q6k_dot (an integer
//         identity).
// The integer superblock sums (sumi = sum_j sc_j * D_j, mint = sum_j mn_j *
// xsum_j; acc = sum_g sc_g * D_g) are exact, and every float operation after
// them is the decode kernels' (moe_kq.hip) in the same order, so outputs are
// per-token decode's bit for bit.
//
// Operand layouts (gfx950, checked on the device): A lane l = row l%32, bytes
// b <-> K 16*(l/32) + b; B lane l = token l%32, the same K mapping; D lane l
// register i = (row 8*(i/4) + 4*(l/32) + i%4, token l%32).  Here K offset k
// of a 32-element group is its element k.
//
// Weights are read in the decode kernels' stream layouts (one copy in HBM):
// gate/up per (expert, 16-row tile, superblock) 9 units x 32 lanes (lanes
// 0-15 gate, 16-31 up); down per (expert, RT-row tile, superblock) U units x
// RT lanes (RT = 64 / top_k), and for Q6_K the fp16 d of those RT rows in the
// d stream.
#include "moe_common.h"
#include "moe_grouped.h"
#include "moe_kq.h"
#include "route_dev.h"

#include <algorithm>

namespace cpb {

typedef int v4i_k __attribute__((ext_vector_type(4)));
typedef int v16i_k __attribute__((ext_vector_type(16)));

CPB_DEV v16i_k mfma_i8(const u32x4& a, const u32x4& b) {
    const v4i_k A = {(int)a[0], (int)a[1], (int)a[2], (int)a[3]};
    const v4i_k B = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
    const v16i_k Z = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, Z, 0, 0, 0);
}
// 32 x 32 x 16 int8 product: lanes 0-31 hold K 0-7 of their row / column,
// lanes 32-63 K 8-15
CPB_DEV v16i_k mfma_i8_k16(uint2 a, uint2 b) {
    const long A = (long)(((uint64_t)a.y << 32) | a.x), B = (long)(((uint64_t)b.y << 32) | b.x);
    const v16i_k Z = {};
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B, Z, 0, 0, 0);
}
// Two 16-element groups held one per lane half (lanes 0-31 group G0 as
// dwords 0-3, lanes 32-63 group G1) into the 32 x 32 x 16 operand layout:
// dwords 0-1 become G0 (lanes 0-31 its elements 0-7, lanes 32-63 its 8-15),
// dwords 2-3 G1 likewise (v_permlane32_swap of dwords 0/2 and 1/3)
CPB_DEV void groups_to_k16(u32x4& v) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    v[0] = s0[0]; v[2] = s0[1]; v[1] = s1[0]; v[3] = s1[1];
}
CPB_DEV u32x4 and4(const u32x4& v, uint32_t m) { return u32x4{v[0] & m, v[1] & m, v[2] & m, v[3] & m}; }
CPB_DEV u32x4 shr4(const u32x4& v, int s) { return u32x4{v[0] >> s, v[1] >> s, v[2] >> s, v[3] >> s}; }
// row of D register i for lane half hb
CPB_DEV int d_row(int i, int hb) { return 8 * (i >> 2) + 4 * hb + (i & 3); }

// Q4_K scale / min bytes of one superblock header (unit 0: d, dmin, 12
// packed bytes; engine_qwen2.rs:57-74 get_scale_min_k4)
CPB_DEV u32x4 unpack_q4k(const u32x4& u0) {
    // sc[0..7] in words 0-1, mn[0..7] in words 2-3: bytes j < 4 are the low
    // six bits of bytes j of q[0..3] / q[4..7]; bytes 4 + j take the low /
    // high nibble of q[8 + j] and, as bits 4-5, the top two bits of byte j
    const uint32_t q03 = u0[1], q47 = u0[2], q811 = u0[3];
    return u32x4{q03 & 0x3F3F3F3Fu, (q811 & 0x0F0F0F0Fu) | ((q03 >> 2) & 0x30303030u), q47 & 0x3F3F3F3Fu,
                 ((q811 >> 4) & 0x0F0F0F0Fu) | ((q47 >> 2) & 0x30303030u)};
}

// ---- per token: rmsnorm + Q8_K per 256 (engine_qwen2.rs:287-300, the
// decode route kernel's operations) ----
__global__ __launch_bounds__(256) void k_prep_batch_kq(GroupedArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int t = blockIdx.x, d = a.d, tid = threadIdx.x, lane = tid & 63;
    float* xs = (float*)smem;
    float* xnl = xs + d;
    float* scratch = xnl + d;
    norm_into(a.x + (size_t)t * d, a.norm_w, d, a.eps, a.norm, a.norm_nt, a.apply_norm, xs, xnl, scratch);
    if (tid == 0) a.inv[t] = a.apply_norm ? scratch[16] : 1.0f;
    // 8 consecutive elements per thread, 32 threads per superblock
    for (int e0 = tid * 8; e0 < d; e0 += 256 * 8) {
        float v[8];
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            v[k] = xnl[e0 + k];
            m = fmaxf(m, fabsf(v[k]));
        }
#pragma unroll
        for (int s2 = 16; s2 >= 1; s2 >>= 1) m = fmaxf(m, __shfl_xor(m, s2));
        const float sc = fmaxf(1e-12f, m) / 127.0f;
        int q[8], s = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            q[k] = q8_round(v[k], sc);
            s += q[k];
        }
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);                           // 4 threads = 32 elements
        const uint32_t lo = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
                            ((uint32_t)(uint8_t)q[3] << 24);
        const uint32_t hi = (uint32_t)(uint8_t)q[4] | ((uint32_t)(uint8_t)q[5] << 8) | ((uint32_t)(uint8_t)q[6] << 16) |
                            ((uint32_t)(uint8_t)q[7] << 24);
        *(uint2*)(a.xq + (size_t)t * d + e0) = uint2{lo, hi};
        *(float4*)(a.xn + (size_t)t * d + e0) = float4{v[0], v[1], v[2], v[3]};
        *(float4*)(a.xn + (size_t)t * d + e0 + 4) = float4{v[4], v[5], v[6], v[7]};
        if ((lane & 3) == 0) a.xsum[(size_t)t * (d / 32) + e0 / 32] = s;
        if ((lane & 31) == 0) a.xsb[(size_t)t * (d / 256) + e0 / 256] = sc;
    }
}

// ---- a token tile's activations in LDS ----
// For K-element rows (gate/up: the tokens' Q8_K x, K = d; down: the pairs'
// Q8_K h, K = d_ff): slot ti's bytes at ti * kq_row_stride(K) (whole 1 KB
// pieces plus 16 bytes, which spreads the 32 slots' reads over the banks),
// then the per-32 sums at stride kq_sum_stride(K) ints, then the per-256
// scales (K / 256 per slot).  Written once per workgroup by direct
// global-to-LDS loads (no staging registers); padding slots read zeros.
CPB_DEV_HOST_INLINE int kq_row_stride(int K) { return (K + 1023) / 1024 * 1024 + 16; }
CPB_DEV_HOST_INLINE int kq_sum_stride(int K) { return (K / 32 > 64 ? (K / 32 + 63) / 64 * 64 : 64) + 4; }
CPB_DEV_HOST_INLINE size_t kq_stage_bytes(int K) {
    return (size_t)32 * kq_row_stride(K) + (size_t)32 * kq_sum_stride(K) * 4 + (size_t)32 * (K / 256) * 4;
}
// staged when two workgroups' LDS still fit a CU
CPB_DEV_HOST_INLINE bool kq_staged(int K) { return kq_stage_bytes(K) <= 76 * 1024; }
typedef __attribute__((address_space(3))) void lds_void_k;
// row of slot ti = src[ti] / div (-1: padding); rows_total bounds the buffers
CPB_DEV void stage_tile_acts(const int8_t* q, const int32_t* sums, const float* scales, int K, int div,
                             size_t rows_total, const int* src, unsigned char* st) {
    const int nsb = K / 256, lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int RS = kq_row_stride(K), XS = kq_sum_stride(K);
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(q, (uint32_t)(rows_total * K));
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(sums, (uint32_t)(rows_total * (K / 32) * 4));
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(scales, (uint32_t)(rows_total * nsb * 4));
    // bytes: 1 KB pieces, lanes past the row's end read zeros into the pad
    const int per = (K + 1023) / 1024;
    for (int i = w; i < 32 * per; i += nw) {
        const int ti = i / per, h = i % per, pr = src[ti], c = h * 1024 + lane * 16;
        const uint32_t off = pr >= 0 && c < K ? (uint32_t)((size_t)(pr / div) * K + c) : kOffNone;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_k*)(st + (size_t)ti * RS + h * 1024), 16, off, 0, 0, 0);
    }
    // per-32 sums: 64 ints per load
    unsigned char* xsl = st + (size_t)32 * RS;
    const int sper = (K / 32 + 63) / 64;
    for (int i = w; i < 32 * sper; i += nw) {
        const int ti = i / sper, h = i % sper, pr = src[ti], j = h * 64 + lane;
        const uint32_t off = pr >= 0 && j < K / 32 ? (uint32_t)(((size_t)(pr / div) * (K / 32) + j) * 4) : kOffNone;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_k*)(xsl + ((size_t)ti * XS + h * 64) * 4), 4, off, 0, 0, 0);
    }
    // per-256 scales: slot ti's nsb values contiguous
    unsigned char* xbl = xsl + (size_t)32 * XS * 4;
    for (int i = w; i < (32 * nsb + 63) / 64; i += nw) {
        const int g = i * 64 + lane, ti = g / nsb, sb = g % nsb;
        const int pr = g < 32 * nsb ? src[ti] : -1;
        const uint32_t off = pr >= 0 ? (uint32_t)(((size_t)(pr / div) * nsb + sb) * 4) : kOffNone;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_k*)(xbl + (size_t)i * 256), 4, off, 0, 0, 0);
    }
}

// ---- gate/up (+ SiLU * up) ----
// one workgroup per (token tile, pair of 32-row tiles) (grouped_item); wave w
// = row tile w / 2, gate (w even) or up (w odd).
// STAGED: the tile's activations are read from LDS (stage_tile_acts), else
// from global memory per superblock.
template <bool TRACE, bool STAGED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gateup_kq_grouped(GroupedArgs a) {
    extern __shared__ __align__(16) unsigned char kst[];
    __shared__ int src[32];
    __shared__ __align__(16) uint8_t s_sm[4][32][16];          // per wave and row: sc[8], mn[8]
    __shared__ float s_dm[4][32][2];             // d, dmin
    __shared__ float xch_s[STAGED ? 1 : 2 * 16 * 64];
    // up results to the gate waves (the staging area once the products are done)
    float (*xch)[16][64] = (float (*)[16][64])(STAGED ? (float*)kst : xch_s);
    const int T32 = a.dff / 32, T16 = a.dff / 16, nsb = a.d / 256;
    int tile, grp;
    if (!grouped_item(uniform(*a.ntiles), (T32 + 1) / 2, &tile, &grp)) return;
    const int4 tl = a.tiles[tile];
    const int e = uniform(tl.x), start = uniform(tl.y), cnt = uniform(tl.z);
    const int lane = threadIdx.x & 63, w = uniform((int)(threadIdx.x >> 6));
    const int rt = grp * 2 + (w >> 1), isup = w & 1;
    const bool live = rt < T32;
    if (threadIdx.x < 32) src[threadIdx.x] = (int)threadIdx.x < cnt ? a.sorted[start + threadIdx.x] : -1;
    __syncthreads();
    if constexpr (STAGED) stage_tile_acts(a.xq, a.xsum, a.xsb, a.d, a.k, (size_t)a.n_tok, src, kst);
    const int r = lane & 31, hb = lane >> 5;
    const int pair = src[r], tok = pair >= 0 ? pair / a.k : -1;        // B column / D column of this lane
    // this lane's A row: stream tile 2 rt + r / 16, lane r % 16 (+16 for up)
    const u32x4* wrow = a.gu + (((size_t)e * T16 + (live ? 2 * rt + (r >> 4) : 0)) * nsb) * kQ4Units * 32 +
                        isup * 16 + (r & 15);
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.xq, (uint32_t)((size_t)a.n_tok * a.d));
    float sumf[16];
#pragma unroll
    for (int i = 0; i < 16; i++) sumf[i] = 0.0f;
    // the next superblock's weight units are requested before this one's
    // products (software pipelined; one superblock of lead)
    u32x4 nu0, nwq[4];
    {
        nu0 = wrow[0];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) nwq[jj] = wrow[(1 + 2 * jj + hb) * 32];
    }
    const unsigned char* xl = kst + (size_t)r * kq_row_stride(a.d) + 16 * hb;
    const int* xsl = (const int*)(kst + (size_t)32 * kq_row_stride(a.d)) + r * kq_sum_stride(a.d);
    const float* xbl = (const float*)(kst + (size_t)32 * kq_row_stride(a.d) + (size_t)32 * kq_sum_stride(a.d) * 4) + r * nsb;
    if constexpr (STAGED) __syncthreads();       // the tile's activations landed (the barrier waits for every load)
    for (int sb = 0; sb < nsb; sb++) {
        const u32x4 u0 = nu0;
        u32x4 wq[4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) wq[jj] = nwq[jj];
        if (sb + 1 < nsb) {
            const u32x4* wp = wrow + (size_t)(sb + 1) * kQ4Units * 32;
            nu0 = wp[0];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) nwq[jj] = wp[(1 + 2 * jj + hb) * 32];
        }
        u32x4 xb[8];
        int xs8[8];
        float ys = 0.0f;
        if constexpr (STAGED) {
#pragma unroll
            for (int j = 0; j < 8; j++) xb[j] = *(const u32x4*)(xl + sb * 256 + 32 * j);
#pragma unroll
            for (int j = 0; j < 8; j++) xs8[j] = xsl[sb * 8 + j];
            ys = xbl[sb];
        } else {
#pragma unroll
        for (int j = 0; j < 8; j++)
            xb[j] = __builtin_amdgcn_raw_buffer_load_b128(
                rx, tok >= 0 ? (uint32_t)((size_t)tok * a.d + sb * 256 + 32 * j + 16 * hb) : kOffNone, 0, 0);
        if (tok >= 0) {
#pragma unroll
            for (int j = 0; j < 8; j++) xs8[j] = a.xsum[(size_t)tok * (a.d / 32) + sb * 8 + j];
            ys = a.xsb[(size_t)tok * nsb + sb];
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) xs8[j] = 0;
        }
        }
        if (hb == 0) {
            *(u32x4*)&s_sm[w][r][0] = unpack_q4k(u0);
            s_dm[w][r][0] = half_bits(u0[0] & 0xffffu);
            s_dm[w][r][1] = half_bits(u0[0] >> 16);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        int sumi[16];
#pragma unroll
        for (int i = 0; i < 16; i++) sumi[i] = 0;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const v16i_k D0 = mfma_i8(and4(wq[jj], 0x0F0F0F0Fu), xb[2 * jj]);
            const v16i_k D1 = mfma_i8(and4(shr4(wq[jj], 4), 0x0F0F0F0Fu), xb[2 * jj + 1]);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = d_row(i, hb);
                sumi[i] += mul24(D0[i], (int)s_sm[w][row][2 * jj]) + mul24(D1[i], (int)s_sm[w][row][2 * jj + 1]);
            }
        }
        // mint = sum_j mn[row][j] * xs8[tok][j] on the matrix cores: xs8 =
        // 64 bh + bl with bl in [0, 63] and bh in [-64, 63] (|xs8| < 2^12) both
        // int8; lanes 0-31 carry (mn, bl) in K 0-7 of the first product and
        // lanes 32-63 (mn, bh) in K 8-15 of the second (the other half's A
        // zero), so mint = M1 + 64 M2 exactly
        v16i_k M1, M2;
        {
            const uint2 mn = *(const uint2*)&s_sm[w][r][8];
            uint32_t bw[2] = {0u, 0u};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint32_t v = (uint32_t)(hb ? (xs8[j] >> 6) : (xs8[j] & 63)) & 0xffu;
                bw[j >> 2] |= v << (8 * (j & 3));
            }
            const uint2 zero = {0u, 0u}, B = {bw[0], bw[1]};
            M1 = mfma_i8_k16(hb ? zero : mn, B);
            M2 = mfma_i8_k16(hb ? mn : zero, B);
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int row = d_row(i, hb);
            const int mint = M1[i] + 64 * M2[i];
            const float dd = s_dm[w][row][0], dmin = s_dm[w][row][1];
            sumf[i] += ys * dd * (float)sumi[i] - ys * dmin * (float)mint;      // engine_qwen2.rs:110
            if (TRACE && pair >= 0 && live) {
                int32_t* o = a.gu_sums + ((((size_t)pair * 2 + isup) * a.dff + rt * 32 + row) * nsb + sb) * 2;
                o[0] = sumi[i];
                o[1] = mint;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if constexpr (STAGED) __syncthreads();       // every wave is done with the staged activations
    if (isup) {
#pragma unroll
        for (int i = 0; i < 16; i++) xch[w >> 1][i][lane] = sumf[i];
    }
    __syncthreads();
    if (isup || !live || pair < 0) return;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float v = sumf[i], up = xch[w >> 1][i][lane];
        a.hbuf[(size_t)pair * a.dff + rt * 32 + d_row(i, hb)] = (v / (1.0f + expf(-v))) * up;   // :416
    }
}

// ---- Q8_K of h per pair (engine_qwen2.rs:288-300, as the decode down
// kernel derives it): one wavefront per (pair, superblock) ----
__global__ __launch_bounds__(256) void k_quant_h_batch(GroupedArgs a) {
    const int nsbf = a.dff / 256, np = a.n_tok * a.k;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (item >= np * nsbf) return;
    const int pair = item / nsbf, sb = item % nsbf;
    const float4 v = *(const float4*)(a.hbuf + (size_t)pair * a.dff + sb * 256 + 4 * lane);
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int s2 = 32; s2 >= 1; s2 >>= 1) m = fmaxf(m, __shfl_xor(m, s2));
    const float sc = fmaxf(1e-12f, m) / 127.0f;
    const int q0 = q8_round(v.x, sc), q1 = q8_round(v.y, sc), q2 = q8_round(v.z, sc), q3 = q8_round(v.w, sc);
    int s = q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);                               // 8 lanes = 32 elements
    *(uint32_t*)(a.hq + (size_t)pair * a.dff + sb * 256 + 4 * lane) =
        (uint32_t)(uint8_t)q0 | ((uint32_t)(uint8_t)q1 << 8) | ((uint32_t)(uint8_t)q2 << 16) | ((uint32_t)(uint8_t)q3 << 24);
    if ((lane & 7) == 0) a.hsum[(size_t)pair * (a.dff / 32) + sb * 8 + lane / 8] = s;
    if (lane == 0) a.hsb[(size_t)pair * nsbf + sb] = sc;
}

// q - 32 of four packed 6-bit values (0..63) as int8 bytes
CPB_DEV uint32_t q6_minus32(uint32_t v) {
    const uint32_t t = v ^ 0x20202020u, m = t & 0x20202020u;
    return t | (m << 1) | (m << 2);
}

// ---- down (Q4_K or Q6_K) into dnout ----
// one workgroup per (token tile, group of 4 row tiles of 32 rows); wave w =
// row tile w.
// STAGED: the tile's Q8_K h is read from LDS (stage_tile_acts), else from
// global memory per superblock.
template <int TYPE, bool TRACE, bool STAGED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_down_kq_grouped(GroupedArgs a) {
    constexpr int U = TYPE == 12 ? kQ4Units : kQ6StreamUnits;   // units per superblock in the stream
    extern __shared__ __align__(16) unsigned char kst[];
    __shared__ int src[32];
    __shared__ __align__(16) uint8_t s_sm[4][32][16];          // Q4_K: sc[8], mn[8]; Q6_K: int8 scales[16]
    __shared__ float s_dm[4][32][2];
    const int nsbf = a.dff / 256, RT = 64 / a.k, Td = a.d / RT, T32 = a.d / 32;
    int tile, grp;
    if (!grouped_item(uniform(*a.ntiles), (T32 + 3) / 4, &tile, &grp)) return;
    const int4 tl = a.tiles[tile];
    const int e = uniform(tl.x), start = uniform(tl.y), cnt = uniform(tl.z);
    const int lane = threadIdx.x & 63, w = uniform((int)(threadIdx.x >> 6));
    const int rt = grp * 4 + w;
    const bool live = rt < T32;
    if (threadIdx.x < 32) src[threadIdx.x] = (int)threadIdx.x < cnt ? a.sorted[start + threadIdx.x] : -1;
    __syncthreads();
    if constexpr (STAGED)
        stage_tile_acts(a.hq, a.hsum, a.hsb, a.dff, 1, (size_t)a.n_tok * a.k, src, kst);
    const int r = lane & 31, hb = lane >> 5;
    const int pair = src[r];
    const int R = (live ? rt : 0) * 32 + r;                   // this lane's A row
    const u32x4* wrow = a.dn + (((size_t)e * Td + R / RT) * nsbf) * U * RT + R % RT;
    const uint16_t* drow = TYPE == 14 ? a.dn_d + ((size_t)e * Td + R / RT) * nsbf * RT + R % RT : nullptr;
    const __amdgpu_buffer_rsrc_t rh = buf_rsrc(a.hq, (uint32_t)((size_t)a.n_tok * a.k * a.dff));
    float sumf[16];
#pragma unroll
    for (int i = 0; i < 16; i++) sumf[i] = 0.0f;
    // this lane's weight units of a superblock: Q4_K d/dmin/scales + 4 quant
    // units; Q6_K 4 ql + 2 qh units, the int8 scales, the fp16 d.  The next
    // superblock's are requested before the current products (one
    // superblock of lead).
    auto wload = [&](int sb, u32x4 (&wu)[7], uint32_t& du) {
        const u32x4* wp = wrow + (size_t)sb * U * RT;
        if constexpr (TYPE == 12) {
            wu[0] = wp[0];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) wu[1 + jj] = wp[(1 + 2 * jj + hb) * RT];
            du = 0;
        } else {
#pragma unroll
            for (int h6 = 0; h6 < 2; h6++) {
#pragma unroll
                for (int pp = 0; pp < 2; pp++) wu[h6 * 2 + pp] = wp[(h6 * 4 + pp * 2 + hb) * RT];
                wu[4 + h6] = wp[(8 + h6 * 2 + hb) * RT];
            }
            wu[6] = wp[12 * RT];
            du = drow[(size_t)sb * RT];
        }
    };
    u32x4 nwu[7];
    uint32_t ndu;
    wload(0, nwu, ndu);
    const unsigned char* hl = kst + (size_t)r * kq_row_stride(a.dff) + 16 * hb;
    const int* hsl = (const int*)(kst + (size_t)32 * kq_row_stride(a.dff)) + r * kq_sum_stride(a.dff);
    const float* hbl =
        (const float*)(kst + (size_t)32 * kq_row_stride(a.dff) + (size_t)32 * kq_sum_stride(a.dff) * 4) + r * nsbf;
    if constexpr (STAGED) __syncthreads();       // the tile's h landed (the barrier waits for every load)
    for (int sb = 0; sb < nsbf; sb++) {
        u32x4 wu[7];
#pragma unroll
        for (int k = 0; k < 7; k++) wu[k] = nwu[k];
        const uint32_t du = ndu;
        if (sb + 1 < nsbf) wload(sb + 1, nwu, ndu);
        const float ys = STAGED ? hbl[sb] : pair >= 0 ? a.hsb[(size_t)pair * nsbf + sb] : 0.0f;
        int acc[16], mint[16];
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = mint[i] = 0;
        if constexpr (TYPE == 12) {
            const u32x4 u0 = wu[0];
            u32x4 wq[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) wq[jj] = wu[1 + jj];
            u32x4 xb[8];
            int xs8[8];
            if constexpr (STAGED) {
#pragma unroll
                for (int j = 0; j < 8; j++) xb[j] = *(const u32x4*)(hl + sb * 256 + 32 * j);
#pragma unroll
                for (int j = 0; j < 8; j++) xs8[j] = hsl[sb * 8 + j];
            } else {
#pragma unroll
            for (int j = 0; j < 8; j++)
                xb[j] = __builtin_amdgcn_raw_buffer_load_b128(
                    rh, pair >= 0 ? (uint32_t)((size_t)pair * a.dff + sb * 256 + 32 * j + 16 * hb) : kOffNone, 0, 0);
#pragma unroll
            for (int j = 0; j < 8; j++) xs8[j] = pair >= 0 ? a.hsum[(size_t)pair * (a.dff / 32) + sb * 8 + j] : 0;
            }
            if (hb == 0) {
                *(u32x4*)&s_sm[w][r][0] = unpack_q4k(u0);
                s_dm[w][r][0] = half_bits(u0[0] & 0xffffu);
                s_dm[w][r][1] = half_bits(u0[0] >> 16);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const v16i_k D0 = mfma_i8(and4(wq[jj], 0x0F0F0F0Fu), xb[2 * jj]);
                const v16i_k D1 = mfma_i8(and4(shr4(wq[jj], 4), 0x0F0F0F0Fu), xb[2 * jj + 1]);
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int row = d_row(i, hb);
                    acc[i] += mul24(D0[i], (int)s_sm[w][row][2 * jj]) + mul24(D1[i], (int)s_sm[w][row][2 * jj + 1]);
                }
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = d_row(i, hb);
#pragma unroll
                for (int j = 0; j < 8; j++) mint[i] += mul24((int)s_sm[w][row][8 + j], xs8[j]);
            }
        } else {
            // ql[128] = units 0-7, qh[64] = units 8-11, int8 scales = unit 12, d from the d stream
            const u32x4 ql[4] = {wu[0], wu[1], wu[2], wu[3]}, qh[2] = {wu[4], wu[5]};
            const u32x4 scu = wu[6];
            if (hb == 0) {
                *(u32x4*)&s_sm[w][r][0] = scu;
                s_dm[w][r][0] = half_bits(du & 0xffffu);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // the superblock's activations, all eight requests in flight at once
            u32x4 xvs[8];
#pragma unroll
            for (int m = 0; m < 8; m++)
                xvs[m] = STAGED ? *(const u32x4*)(hl + sb * 256 + 32 * m)
                                : __builtin_amdgcn_raw_buffer_load_b128(
                                      rh, pair >= 0 ? (uint32_t)((size_t)pair * a.dff + sb * 256 + 32 * m + 16 * hb) : kOffNone, 0, 0);
#pragma unroll
            for (int m = 0; m < 8; m++) {
                // elements 32 m .. 32 m + 31 (engine_qwen2.rs:171-190): 128-half h6, quarter p
                const int h6 = m >> 2, p = m & 3;
                const u32x4 lq = (p >> 1) ? shr4(ql[h6 * 2 + (p & 1)], 4) : ql[h6 * 2 + (p & 1)];
                const u32x4 hq2 = shr4(qh[h6], 2 * p);
                u32x4 A;
#pragma unroll
                for (int c = 0; c < 4; c++) A[c] = q6_minus32((lq[c] & 0x0F0F0F0Fu) | ((hq2[c] & 0x03030303u) << 4));
                u32x4 xv = xvs[m];
                // lane half hb holds group 2m + hb (weights and activations):
                // one 32 x 32 x 16 product per group
                groups_to_k16(A);
                groups_to_k16(xv);
                const v16i_k D0 = mfma_i8_k16(uint2{A[0], A[1]}, uint2{xv[0], xv[1]});
                const v16i_k D1 = mfma_i8_k16(uint2{A[2], A[3]}, uint2{xv[2], xv[3]});
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int row = d_row(i, hb);
                    acc[i] += mul24(D0[i], (int)(int8_t)s_sm[w][row][2 * m]) + mul24(D1[i], (int)(int8_t)s_sm[w][row][2 * m + 1]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int row = d_row(i, hb);
            const float dd = s_dm[w][row][0];
            if constexpr (TYPE == 12)
                sumf[i] += ys * dd * (float)acc[i] - ys * s_dm[w][row][1] * (float)mint[i];
            else
                sumf[i] += ys * dd * (float)acc[i];                               // engine_qwen2.rs:196
            if (TRACE && pair >= 0 && live) {
                int32_t* o = a.dn_sums + (((size_t)pair * a.d + rt * 32 + row) * nsbf + sb) * (TYPE == 12 ? 2 : 1);
                o[0] = acc[i];
                if (TYPE == 12) o[1] = mint[i];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (!live || pair < 0) return;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int row = rt * 32 + d_row(i, hb);
        a.dnout[(size_t)pair * a.d + row] = sumf[i] + (a.down_b ? a.down_b[(size_t)e * a.d + row] : 0.0f);
    }
}

int launch_prep_kq(const GroupedArgs& a, hipStream_t s) {
    launch(k_prep_batch_kq, dim3(a.n_tok), dim3(256), sizeof(float) * (2 * a.d + 64), s, a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_kq_gemms(const GroupedArgs& a, bool trace, hipStream_t s, const LaunchEvents* ev) {
    const int ngu = a.max_tiles * ((a.dff / 32 + 1) / 2), ndn = a.max_tiles * ((a.d / 32 + 3) / 4);
    const dim3 ggu((ngu + 7) / 8 * 8), gdn((ndn + 7) / 8 * 8);
    const int np = a.n_tok * a.k, nq = np * (a.dff / 256);
    if (ev) armed_events() = ev[0];
    if (trace) launch(k_gateup_kq_grouped<true, false>, ggu, dim3(256), 0, s, a);
    else if (kq_staged(a.d)) launch(k_gateup_kq_grouped<false, true>, ggu, dim3(256), kq_stage_bytes(a.d), s, a);
    else launch(k_gateup_kq_grouped<false, false>, ggu, dim3(256), 0, s, a);
    launch(k_quant_h_batch, dim3((nq + 3) / 4), dim3(256), 0, s, a);
    if (ev) armed_events() = ev[1];
    const bool sd = kq_staged(a.dff);
    const size_t ldn = sd ? kq_stage_bytes(a.dff) : 0;
    if (a.down_type == 12) {
        if (trace) launch(k_down_kq_grouped<12, true, false>, gdn, dim3(256), 0, s, a);
        else if (sd) launch(k_down_kq_grouped<12, false, true>, gdn, dim3(256), ldn, s, a);
        else launch(k_down_kq_grouped<12, false, false>, gdn, dim3(256), 0, s, a);
    } else {
        if (trace) launch(k_down_kq_grouped<14, true, false>, gdn, dim3(256), 0, s, a);
        else if (sd) launch(k_down_kq_grouped<14, false, true>, gdn, dim3(256), ldn, s, a);
        else launch(k_down_kq_grouped<14, false, false>, gdn, dim3(256), 0, s, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
