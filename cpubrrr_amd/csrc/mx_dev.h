// mx_dev.h -- device building blocks of the MXFP4 expert GEMVs, shared by
// the per-phase kernels (moe_mx.hip) and the persistent decode kernel
// (decode_mx.hip).  Stream layout and lane mapping: see moe_mx.hip.
#pragma once
#include "moe_common.h"

namespace cpb {

// One lane's k-part: wv[0] = the 15 e8m0 bytes, wv[1..15] = nibble blocks.
// xs: LDS activations of these 15 blocks as [15][xp 2 x u32x4][xn 2 x u32x4],
// sb: their 15 scales.
template <bool TRACE>
CPB_DEV float part_dot(const u32x4* wv, const u32x4* xs, const float* sb, int32_t* sums_out, int blk0, int nb) {
    const MxConsts k = mx_consts();
    const uint32_t ew[4] = {wv[0][0], wv[0][1], wv[0][2], wv[0][3]};
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < kBlkPerPart; u++) {
        const u32x4* xb = xs + u * 4;
#ifdef CPB_PROBE_NO_DECODE
        // probe builds only: same loads and epilogue, no decode arithmetic
        int S = (int)(wv[u + 1][0] ^ xb[0][0]) & 7;
#else
        int S = mx_block_sum(wv[u + 1], xb[0], xb[1], xb[2], xb[3], k);
#endif
        uint32_t e = (ew[u >> 2] >> (8 * (u & 3))) & 0xffu;
        acc = fmaf((float)S, e8m0_scale(e, sb[u]), acc);
        if (TRACE && blk0 + u < nb) sums_out[u] = S;
        // keep each block's LDS operand reads next to their use: with the
        // weights already resident the scheduler would otherwise hoist all
        // 15 blocks' reads (240 VGPRs)
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
}

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

// Issue the lane's 16 weight loads in stream order (e8m0 unit first) so the
// compiler's in-order vmcnt waits release each block as soon as it lands.
CPB_DEV void load_part(const u32x4* p, size_t stride, u32x4* wv) {
#pragma unroll
    for (int u = 0; u < kUnits; u++) {
        wv[u] = __builtin_nontemporal_load(p + (size_t)u * stride);
        __builtin_amdgcn_sched_barrier(0);
    }
}

CPB_DEV void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace cpb
