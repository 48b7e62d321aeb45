// mx_dev.h -- device building blocks of the MXFP4 expert GEMVs (moe_mx.hip;
// the grouped path shares the sub-part split and the image encoding).  Stream
// layout and lane mapping: see moe_mx.hip.
#pragma once
#include "moe_common.h"

namespace cpb {

// A k-part is processed by two wavefronts: sub-part h covers blocks
// 8h .. 8h + 7 of it (the last slot of sub-part 1 is empty).
constexpr int kSubUnits = 8;

// Issue the sub-part's loads in stream order: the e8m0 unit, then units
// 1 + ub .. 1 + ub + 7 (stride: 16-byte units between consecutive units);
// unit 16 (beyond the k-part) is not read.
CPB_DEV void load_sub(const u32x4* p, size_t stride, int ub, u32x4* wv) {
    wv[0] = __builtin_nontemporal_load(p);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kSubUnits; i++) {
        wv[i + 1] = ub + i < kBlkPerPart ? __builtin_nontemporal_load(p + (size_t)(1 + ub + i) * stride) : u32x4{0, 0, 0, 0};
        __builtin_amdgcn_sched_barrier(0);
    }
}

CPB_DEV void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}


// ---- matrix-core block sums of one sub-part ----
//
// v_mfma_scale_f32_16x16x128_f8f6f4 with A = activations (fp8 e4m3, 16 x 128)
// and B = weights (fp4 e2m1, 128 x 16): a "window" is 4 consecutive blocks
// (128 K) of 16 weight rows.  An int8 activation x is split exactly as
// x = 16*h + l (h = x >> 4 in [-8, 7], l in [0, 15]) and A row m = 2*bo + p
// holds 32*h (p = 0) or 2*l (p = 1) of window block bo at that block's K and
// zeros elsewhere (rows 8-15 are zero).  Both are exact in e4m3, every product
// with an e2m1 weight and every partial sum is an integer below 2^16, so
//     D[2*bo][n] + D[2*bo + 1][n] = sum_i 2*E2M1(w_ni) * x_i = S
// exactly: the reference's int32 block sum (engine_gpt2.rs:194-228, KVI =
// 2*E2M1 at :152) as a float, bit for bit.
//
// Operand layouts (gfx950): A lane (m = l%16, g = l/16) holds K 16g..16g+15 in
// bytes 0-15 and K 64+16g.. in bytes 16-31; B lane (n = l%16, g) holds K
// 32g..32g+31 as nibbles, low nibble first (= block g's 16 GGUF bytes as they
// are); D lane l holds column l%16, rows 4*(l/16)..+3.  A GGUF block's byte i
// holds elements i (low nibble) and i + 16, so K offset k inside a block is
// element k/2 + 16*(k%2): the activation image (below) is stored in K order.
//
// The stream layout gives lane r row r of a 64-row tile and one block per
// register; B needs rows 16t..16t+15 x the window's 4 blocks in one register.
// That is a 4 x 4 transpose of (16-lane group, register), two rounds of
// permlane swaps per dword; the four row groups' sums come back to lane = row
// the same way.
//
// Activation image: per 32-block 64 bytes, [32*h of the 32 elements in K
// order | 2*l in K order], fp8 e4m3 (written by the routing kernel).
constexpr int kImgBytes = 64;

typedef int v8i_mx __attribute__((ext_vector_type(8)));
typedef float v4f_mx __attribute__((ext_vector_type(4)));
typedef uint32_t u2_mx __attribute__((ext_vector_type(2)));

// a.upper 32 lanes <-> b.lower 32 lanes
CPB_DEV void swap32(uint32_t& a, uint32_t& b) {
    const u2_mx r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
// a's 16-lane groups 1, 3 <-> b's groups 0, 2
CPB_DEV void swap16(uint32_t& a, uint32_t& b) {
    const u2_mx r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
CPB_DEV void swap32f(float& a, float& b) {
    uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
    swap32(x, y);
    a = __uint_as_float(x);
    b = __uint_as_float(y);
}
CPB_DEV void swap16f(float& a, float& b) {
    uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
    swap16(x, y);
    a = __uint_as_float(x);
    b = __uint_as_float(y);
}

// Window activations of this lane: 16 bytes for its low and high K halves.
struct WinAct {
    u32x4 lo, hi;
};
// Issue the loads of a window's A operand: blocks wb .. wb+3 (absolute block
// indices), u0 = index of block wb inside its k-part; blocks beyond the k-part
// or the row (nb) read as zero (out-of-range buffer offset).
CPB_DEV WinAct load_win_act(__amdgpu_buffer_rsrc_t img, int wb, int u0, int nb) {
    const int lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4, bo = m >> 1, p = m & 1;
    const int bl = g >> 1, bh = 2 + (g >> 1);
    const uint32_t sub = (uint32_t)(p * 32 + (g & 1) * 16);
    const bool lo_ok = m < 8 && bo == bl && u0 + bl < kBlkPerPart && wb + bl < nb;
    const bool hi_ok = m < 8 && bo == bh && u0 + bh < kBlkPerPart && wb + bh < nb;
    WinAct r;
    r.lo = __builtin_amdgcn_raw_buffer_load_b128(img, lo_ok ? (uint32_t)(wb + bl) * kImgBytes + sub : kOffNone, 0, 0);
    r.hi = __builtin_amdgcn_raw_buffer_load_b128(img, hi_ok ? (uint32_t)(wb + bh) * kImgBytes + sub : kOffNone, 0, 0);
    return r;
}

// One 16-byte A fragment per lane: lane (m, g) with m < 8 holds part p = m%2
// of window block bo = m/2 at K half (g%2) of that block, i.e. the low half
// of A when bo = g/2 (m < 4) or the high half when bo = 2 + g/2 (4 <= m < 8);
// every other fragment is zero.  img: the image of one activation vector;
// blocks beyond the k-part or the row (nb) read as zero (out-of-range offset).
CPB_DEV u32x4 load_act_frag(__amdgpu_buffer_rsrc_t img, uint32_t base, int wb, int u0, int nb) {
    const int lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int bi = (m < 4 ? 0 : 2) + (g >> 1);   // block of the window this lane could hold
    const bool ok = m < 8 && (m >> 1) == bi && u0 + bi < kBlkPerPart && wb + bi < nb;
    const uint32_t off = base + (uint32_t)(wb + bi) * kImgBytes + (uint32_t)((m & 1) * 32 + (g & 1) * 16);
    return __builtin_amdgcn_raw_buffer_load_b128(img, ok ? off : kOffNone, 0, 0);
}
CPB_DEV v8i_mx act_operand(const u32x4& x) {
    const bool lo = (threadIdx.x & 15) < 4;
    const u32x4 z = {0, 0, 0, 0};
    const u32x4 l = lo ? x : z, h = lo ? z : x;
    return v8i_mx{(int)l[0], (int)l[1], (int)l[2], (int)l[3], (int)h[0], (int)h[1], (int)h[2], (int)h[3]};
}

// Block sums of one window: r[0..3] = the lane's row, blocks 0-3 of the
// window (transposed in place); a(t) = the A operand for rows 16t..16t+15
// (lane group t); S[0..3] = the row's four block sums.
template <typename AFn>
CPB_DEV void window_sums(u32x4* r, AFn a, float* S) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        uint32_t a0 = r[0][c], a1 = r[1][c], a2 = r[2][c], a3 = r[3][c];
        swap32(a0, a2);
        swap32(a1, a3);
        swap16(a0, a1);
        swap16(a2, a3);
        r[0][c] = a0; r[1][c] = a1; r[2][c] = a2; r[3][c] = a3;
    }
    float sa[4], sb[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const v8i_mx B = {(int)r[t][0], (int)r[t][1], (int)r[t][2], (int)r[t][3], 0, 0, 0, 0};
        const v4f_mx D = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a(t), B, v4f_mx{0, 0, 0, 0}, 0, 4, 0, 127, 0, 127);
        // lanes 0-15: blocks 0, 1 of row 16t + n; lanes 16-31: blocks 2, 3
        sa[t] = D[0] + D[1];
        sb[t] = D[2] + D[3];
    }
    swap32f(sa[0], sa[2]);
    swap32f(sa[1], sa[3]);
    swap16f(sa[0], sa[1]);
    swap32f(sb[0], sb[2]);
    swap32f(sb[1], sb[3]);
    swap16f(sb[0], sb[1]);
    S[0] = sa[0];
    S[1] = sb[0];
    S[2] = sa[1];
    S[3] = sb[1];
}

// A sub-part's fma chain over block sums S[0..7] of blocks ub .. ub+7: one
// fma with 2^(e-128) * xsb per block, in block order.
template <bool TRACE>
CPB_DEV float sub_chain(const u32x4& ew4, int ub, const float* S, const float* sc, int32_t* sums_out, int blk0, int nb) {
    const uint32_t ew[4] = {ew4[0], ew4[1], ew4[2], ew4[3]};
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kSubUnits; i++) {
        const int u = ub + i;
        const uint32_t e = (ew[u >> 2] >> (8 * (u & 3))) & 0xffu;
        acc = fmaf(S[i], e8m0_scale(e, sc[i]), acc);
        if (TRACE && sums_out && u < kBlkPerPart && blk0 + u < nb) sums_out[u] = (int32_t)S[i];
    }
    return acc;
}

// One lane's sub-part on the matrix cores, one activation vector for all 64
// rows (gate/up): wv as from load_sub, x[0..1] the windows' activations,
// sc[0..7] the blocks' activation scales.
template <bool TRACE>
CPB_DEV float part_dot_sub_mfma(u32x4* wv, int ub, const WinAct* x, const float* sc, int32_t* sums_out, int blk0,
                                int nb) {
    float S[kSubUnits];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const v8i_mx A = {(int)x[h].lo[0], (int)x[h].lo[1], (int)x[h].lo[2], (int)x[h].lo[3],
                          (int)x[h].hi[0], (int)x[h].hi[1], (int)x[h].hi[2], (int)x[h].hi[3]};
        window_sums(wv + 1 + 4 * h, [&](int) { return A; }, S + 4 * h);
    }
    return sub_chain<TRACE>(wv[0], ub, S, sc, sums_out, blk0, nb);
}

// The same with a different activation vector per 16-row lane group
// (down: xa[h][t] = window h's fragment of the vector of lane group t).
template <bool TRACE>
CPB_DEV float part_dot_sub_mfma4(u32x4* wv, int ub, const u32x4 (*xa)[4], const float* sc, int32_t* sums_out,
                                 int blk0, int nb) {
    float S[kSubUnits];
#pragma unroll
    for (int h = 0; h < 2; h++) window_sums(wv + 1 + 4 * h, [&](int t) { return act_operand(xa[h][t]); }, S + 4 * h);
    return sub_chain<TRACE>(wv[0], ub, S, sc, sums_out, blk0, nb);
}

}  // namespace cpb
