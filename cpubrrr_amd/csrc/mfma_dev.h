// mfma_dev.h -- MXFP4 expert GEMV on the gfx950 matrix cores, exact.
//
// v_mfma_scale_f32_16x16x128_f8f6f4 multiplies a 16x128 fp8 (e4m3) matrix A
// by a 128x16 fp4 (e2m1) matrix B into 16x16 fp32.  Here B is 16 weight rows
// x one 4-block (128-element) window of the raw MXFP4 codes, so the weights
// go into the matrix cores undecoded, and A carries the Q8 activations of
// that window.  An int8 activation x is split exactly as x = 16*h + l with
// h = x >> 4 in [-8, 7] and l in [0, 15]; 16*h and l are exact in e4m3, every
// product with an e2m1 weight is exact in fp32 and so is every partial sum
// (|sum| < 2^15 on a half-integer grid).  A row m = 2*bo + p holds part p
// (p = 0: 16*h, p = 1: l) of block bo of the window and zeros elsewhere, so
//     D[2*bo][n] + D[2*bo + 1][n] = sum_i E2M1(w_ni) * x_i = S_b / 2
// is the exact int32 block sum S_b = sum KVI[c]*xq of the reference's
// dot4_mx_i8 (engine_gpt2.rs:194-228; KVI = 2*E2M1, :152), recovered as a
// float.  Each block then contributes one fma: acc += (S_b/2) * 2^(e-127)*xsb,
// i.e. S_b * tbl[e] * xsb with tbl[e] = 2^(e-128) (:436-438).
//
// Operand layouts (measured on gfx950): A lane (m = l%16, g = l/16) holds K
// 16g..16g+15 in bytes 0-15 and K 64+16g.. in bytes 16-31; B lane
// (n = l%16, g) holds K 32g..32g+31 as nibbles (low nibble first); D lane q
// holds column q%16, rows 4*(q/16)..+3.  An MXFP4 block's byte i holds
// elements i (low nibble) and i+16 (high), so K offset k within a block is
// element k/2 + 16*(k%2); the activation image below is stored in that order.
//
// Stream layout of one expert matrix ("rowgroup" = 16 rows, "group" = 16
// blocks = 4 windows):  for each rowgroup, for each group: an e8m0 unit of
// 256 B (row n's 16 exponents at n*16) followed by the group's windows, a
// window of nw blocks being nw*256 B with (row n, block gq) at gq*256 + n*16.
// One 64-lane load of 16 B per lane reads a whole window (1 KB).
#pragma once
#include "moe_common.h"

namespace cpb {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// bytes of one rowgroup (16 rows) of a matrix with nb 32-blocks per row
CPB_DEV_HOST_INLINE size_t mf_rowgroup_bytes(int nb) {
    const int groups = (nb + 15) / 16;
    return (size_t)groups * 256 + (size_t)nb * 256;
}
// byte offset of group gi's e8m0 unit inside a rowgroup
CPB_DEV_HOST_INLINE size_t mf_group_offset(int gi) { return (size_t)gi * (256 + 16 * 256); }

// Activation image (LDS or global): per block b, 64 bytes =
// [16*h parts in K order (32 B) | l parts in K order (32 B)], all fp8 e4m3.
constexpr int kImgBlock = 64;

// exact e4m3 encodings used by the split: 16*h (h in [-8,7]) and l in [0,15]
CPB_DEV uint8_t e4m3_of_small(int v) {
    // v is 0, an integer in [1, 15], or 16*h: every such |v| has <= 4 significant bits
    if (v == 0) return 0;
    const uint32_t s = v < 0 ? 0x80u : 0u;
    const uint32_t a = (uint32_t)(v < 0 ? -v : v);
    const int E = 31 - __builtin_clz(a);
    const uint32_t m = E >= 3 ? (a >> (E - 3)) & 7u : (a << (3 - E)) & 7u;
    return (uint8_t)(s | ((uint32_t)(E + 7) << 3) | m);
}
// K offset inside a block of element e (0..31)
CPB_DEV int k_of_elem(int e) { return e < 16 ? 2 * e : 2 * (e - 16) + 1; }

// Write the image bytes of int8 activation q (element e of block b).
CPB_DEV void put_image(uint8_t* img, int b, int e, int q) {
    const int h = q >> 4;               // arithmetic shift: floor(q / 16)
    const int l = q - 16 * h;
    const int k = k_of_elem(e);
    st_dev(img + b * kImgBlock + k, e4m3_of_small(16 * h));
    st_dev(img + b * kImgBlock + 32 + k, e4m3_of_small(l));
}

// One wave: 16 rows (n = lane%16) x groups [gi0, gi1) (at most kMaxGroups)
// of one matrix rowgroup; weights come from mf_issue.
// img/sb: activation image and block scales (LDS); zero16: 16 zero bytes in
// LDS.  Returns the partial sum of row n over the range in lanes 0-15 (lanes
// 16-63 return 0).  TRACE writes the int32 block sums of row n to
// sums[n * nb + b].
constexpr int kMaxGroups = 3;

// Weight registers of one wave's range: exponent units and windows of up to
// kMaxGroups groups.  mf_issue starts every load; mf_rows consumes them, so a
// caller can issue the weight stream before it stages the activations.
struct MfRegs {
    u32x4 ev[kMaxGroups];
    u32x4 wv[kMaxGroups][4];
};

// s * 2^(e - 127) for an e8m0 exponent byte e, 0 for e == 0 (the reference's
// tbl[0] = 0); equal to ldexpf(s, e - 127) bit for bit, without a branch: the
// power of two is built from its bit pattern (e = 255 as 2^127 * 2).
CPB_DEV float e8m0_times(float s, uint32_t e) {
    const float r = s * __uint_as_float(min(e, 254u) << 23);
    return e == 255u ? r * 2.0f : r;
}

// Start the weight loads of groups [gi0, gi1) of rowgroup rg (nontemporal).
CPB_DEV void mf_issue(MfRegs& r, const uint8_t* __restrict__ rg, int nb, int gi0, int gi1) {
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g = lane >> 4;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(rg, (uint32_t)mf_rowgroup_bytes(nb));
    gi0 = uniform(gi0); gi1 = uniform(gi1); nb = uniform(nb);
#pragma unroll
    for (int j = 0; j < kMaxGroups; j++) {
        const int gi = gi0 + j;
        const int gb = gi < gi1 ? min(16, nb - 16 * gi) : 0;
        const uint32_t go = (uint32_t)mf_group_offset(gi);
        r.ev[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, gb > 0 ? go + n * 16 : kOffNone, 0, 2);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const bool has = g < gb - 4 * w;
            r.wv[j][w] = __builtin_amdgcn_raw_buffer_load_b128(
                rs, has ? go + 256 + w * 1024 + g * 256 + n * 16 : kOffNone, 0, 2);
        }
    }
}

template <bool TRACE>
CPB_DEV float mf_rows(const MfRegs& r, int nb, int gi0, int gi1, const uint8_t* img,
                      const float* sb, const uint8_t* zero16, int32_t* sums) {
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g = lane >> 4;
    // A operand geometry: row m = lane%16 -> (bo, p), live for m < 8; the low
    // 16 bytes carry block g/2 of the window, the high 16 bytes block 2 + g/2,
    // K half (g & 1)
    const int m = lane & 15, bo = m >> 1, p = m & 1;
    const bool lo_half = m < 8 && (g >> 1) == bo;
    const bool hi_half = m < 8 && 2 + (g >> 1) == bo;
    const int abyte = p * 32 + (g & 1) * 16;
    const u32x4 (&ev)[kMaxGroups] = r.ev;
    const u32x4 (&wv)[kMaxGroups][4] = r.wv;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxGroups; j++) {
        const int gi = gi0 + j;
        const bool gin = gi < gi1;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // every window is computed (straight-line code); windows and blocks
            // outside the range get zero activations and a zero scale
            const int b0 = 16 * gi + 4 * w;               // first block of the window
            const bool ain = gin && b0 + bo < nb;
            const uint8_t* alo = lo_half && ain ? img + (b0 + bo) * kImgBlock + abyte : zero16;
            const uint8_t* ahi = hi_half && ain ? img + (b0 + bo) * kImgBlock + abyte : zero16;
            const u32x4 a0 = *(const u32x4*)alo;
            const u32x4 a1 = *(const u32x4*)ahi;
            const v8i A = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
            const v8i B = {(int)wv[j][w][0], (int)wv[j][w][1], (int)wv[j][w][2], (int)wv[j][w][3], 0, 0, 0, 0};
            v4f D = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, v4f{0, 0, 0, 0}, 0, 4, 0, 127, 0, 127);
            // pin the MFMA to its window (an unpinned MFMA is sunk past later
            // windows, which then hold all their operands live at once)
            asm volatile("" : "+v"(D));
            // lanes 0-15 (g = 0): blocks b0, b0+1; lanes 16-31 (g = 1): b0+2, b0+3.
            // The epilogue is branch-free: a use of D under a lane condition
            // lets the compiler sink the MFMA into the branch, where it would
            // run with half the wave masked off (and read half of B as zero).
            const bool live = g < 2;
            const float t0 = D[0] + D[1];                 // S/2 of block bb (exact)
            const float t1 = D[2] + D[3];                 // S/2 of block bb + 1
            const int bi = 4 * w + 2 * (g & 1);           // block index inside the group
            const uint32_t ew = ev[j][w];
            const int bb = 16 * gi + bi;
            const bool ok0 = live && gin && bb < nb, ok1 = live && gin && bb + 1 < nb;
            // a block outside the range gets exponent 0, i.e. scale 0
            const uint32_t e0 = ok0 ? (ew >> (16 * (g & 1))) & 0xffu : 0u;
            const uint32_t e1 = ok1 ? (ew >> (16 * (g & 1) + 8)) & 0xffu : 0u;
            const float s0 = sb[ok0 ? bb : 0];
            const float s1 = sb[ok1 ? bb + 1 : 0];
            acc = fmaf(t0, e8m0_times(s0, e0), acc);
            acc = fmaf(t1, e8m0_times(s1, e1), acc);
            if (TRACE) {
                if (ok0) sums[n * nb + bb] = (int32_t)(2.0f * t0);
                if (ok1) sums[n * nb + bb + 1] = (int32_t)(2.0f * t1);
            }
            // keep each window's activation reads next to its MFMA: hoisting
            // them all would hold every window's A operand (8 VGPRs each) at once
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // combine the two block-pair halves of row n into lanes 0-15
    acc += __shfl_down(acc, 16);
    return lane < 16 ? acc : 0.0f;
}

}  // namespace cpb
