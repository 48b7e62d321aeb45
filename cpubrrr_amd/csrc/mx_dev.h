// mx_dev.h -- device building blocks of the MXFP4 expert GEMVs (moe_mx.hip,
// and the activation staging of the grouped path).  Stream layout and lane
// mapping: see moe_mx.hip.
#pragma once
#include "moe_common.h"

namespace cpb {

// LDS image of one expert's activations for one k-part: 15 blocks x
// [xq 8 dwords | -xq 8 dwords], then 15 block scales (+1 pad): 256 dwords.
constexpr int kXsDw = 256;

// Fill one 256-dword activation image from global xq / -xq / scales.
// `slot` runs over the image's dwords; returns the value for that slot.
struct XsSlot {
    const uint32_t* p;
    bool valid;
};
CPB_DEV XsSlot xs_slot(const uint32_t* __restrict__ q, const uint32_t* __restrict__ qn,
                       const float* __restrict__ sc, int blk0, int nb, int slot, bool use) {
    // one clamped address per slot; the validity select is applied when the
    // value is stored to LDS, after the weight loads have been issued.  A
    // consumer whose data was written earlier in the same launch must load
    // through ld_dev (another XCD's L2 may hold a stale copy).
    const bool isx = slot < kBlkPerPart * 16;
    const int u = isx ? slot / 16 : slot - kBlkPerPart * 16;
    const int j = slot & 15;
    const int blk = blk0 + u;
    const int bc = min(blk, nb - 1);
    const uint32_t* base = isx ? (j < 8 ? q : qn) : (const uint32_t*)sc;
    return XsSlot{base + (isx ? bc * 8 + (j & 7) : bc), use && blk < nb && (isx || u < kBlkPerPart)};
}

// A k-part is processed by two wavefronts: sub-part h covers blocks
// 8h .. 8h + 7 of it (the last slot of sub-part 1 is empty).
constexpr int kSubUnits = 8;

// One lane's sub-part: wv[0] = the 15 e8m0 bytes, wv[1 .. 8] = the nibble
// blocks ub .. ub + 7 of the k-part.  Block 15 (the second sub-part's eighth
// slot) does not exist: its weights load as zero and its pad exponent byte is
// zero, so it adds exactly nothing.
template <bool TRACE>
CPB_DEV float part_dot_sub(const u32x4* wv, int ub, const u32x4* xs, const float* sb, int32_t* sums_out, int blk0,
                           int nb) {
    const MxConsts k = mx_consts();
    const uint32_t ew[4] = {wv[0][0], wv[0][1], wv[0][2], wv[0][3]};
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kSubUnits; i++) {
        const int u = ub + i;
        const u32x4* xb = xs + u * 4;
        int S = mx_block_sum(wv[i + 1], xb[0], xb[1], xb[2], xb[3], k);
        const uint32_t e = (ew[u >> 2] >> (8 * (u & 3))) & 0xffu;
        acc = fmaf((float)S, e8m0_scale(e, sb[u]), acc);
        if (TRACE && u < kBlkPerPart && blk0 + u < nb) sums_out[u] = S;
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
}

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

}  // namespace cpb
