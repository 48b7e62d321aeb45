// moe_grouped.h -- batched / prefill gpt-oss MoE: tokens grouped by expert,
// expert GEMMs on the gfx950 matrix cores (exact), bit-identical to the
// per-token decode kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "moe_common.h"

namespace cpb {

struct GroupedArgs {
    // layer
    const float* norm_w;
    const float* router_w;
    const float* router_b;
    const u32x4* gu;           // decode stream layouts (moe_mx.hip), read as MFMA operands
    const u32x4* dn;
    const uint16_t* dn_d;      // Q6_K down: the fp16 d stream (kq_down_dstream)
    const float* gate_b;
    const float* up_b;
    const float* down_b;
    // shapes / semantics
    int n_tok, d, dff, ne, k, nb, nbf, parts_gu, parts_dn;
    int norm, norm_nt, apply_norm;
    float eps, alpha, limit;
    int max_tiles;             // grid bound of the expert GEMMs: n_tok*k/32 + ne
    // activations (device)
    float* x;                  // [n_tok][d] residual, updated in place
    float* xn;                 // [n_tok][d]
    float* inv;                // [n_tok] rmsnorm scale (1 without the norm)
    int8_t* xq;                // [n_tok][d]
    float* xsb;                // [n_tok][nb]
    uint8_t* ximg;             // [n_tok][nb][64] fp8 image of xq (MFMA operand)
    double* lstar;             // [n_tok][ne]
    double* lbound;            // [n_tok][ne]
    float* logits;             // [n_tok][ne]
    int32_t* ids;              // [n_tok][k]
    float* wts;                // [n_tok][k]
    int32_t* fallback;         // [n_tok]
    int32_t* sorted;           // [n_tok*k] pair ids (t*k + slot), grouped by expert (any order within one)
    int4* tiles;               // [max_tiles] {expert, first sorted index, count, 0}
    int32_t* ntiles;           // [1]
    int8_t* hq;                // [n_tok*k][dff]
    float* hsb;                // [n_tok*k][nbf]
    uint8_t* himg;             // [n_tok*k][nbf][64]
    float* dnout;              // [n_tok*k][d] down rows + bias
    // k-quant (Qwen3) layers: Q8_K activations and h, weights of down_type
    int kq;                    // 1: Q4_K gate/up, Q4_K / Q6_K down (int8 matrix cores)
    int down_type;             // 12 or 14
    int32_t* xsum;             // [n_tok][d/32] sums of xq per 32 (xsb: per-256 scales)
    float* hbuf;               // [n_tok*k][dff] SiLU(gate) * up
    int32_t* hsum;             // [n_tok*k][dff/32] (hsb: per-256 scales of hq)
    // trace (optional, small shapes): int32 block sums, pair-major
    int32_t* gu_sums;          // MXFP4 [n_tok*k][2][dff][nb]; Q4_K [n_tok*k][2][dff][d/256][2]
    int32_t* dn_sums;          // MXFP4 [n_tok*k][d][nbf]; Q4_K [..][d][dff/256][2]; Q6_K [..][d][dff/256]
};

// XCD-aware work order of the grouped GEMMs.  Work item w = (row group
// w / ntiles, token tile w % ntiles); the workgroups of a launch are dealt to
// the 8 XCDs round robin (workgroup L runs on XCD L % 8, in order of L), so
// XCD x takes the contiguous range of items [x * per, (x + 1) * per): the
// token tiles of one expert and row group then run back to back on one XCD
// and re-read that weight slice from its L2 instead of HBM.  Returns false for
// workgroups past the last item.
CPB_DEV bool grouped_item(int ntiles, int ngroups, int* tile, int* group) {
    const int L = blockIdx.x, total = ntiles * ngroups;
    const int per = (total + 7) / 8;
    const int slot = L >> 3, w = (L & 7) * per + slot;
    if (slot >= per || w >= total) return false;
    *group = w / ntiles;
    *tile = w % ntiles;
    return true;
}

// All stages of one layer on stream s.  Shapes validated by the caller
// (MXFP4: d and dff multiples of 32; k-quants: multiples of 256).
// ev (optional): event pairs armed for the gate/up GEMM (ev[0]) and the down
// GEMM (ev[1]) launches (timing mode).
int launch_grouped_layer(const GroupedArgs& a, bool trace, hipStream_t s, const LaunchEvents* ev = nullptr);

// k-quant stages (moe_grouped_kq.hip): per-token rmsnorm + Q8_K, and the
// expert GEMMs on int8 matrix cores (gate/up + SiLU * up, Q8_K of h, down)
int launch_prep_kq(const GroupedArgs& a, hipStream_t s);
int launch_kq_gemms(const GroupedArgs& a, bool trace, hipStream_t s, const LaunchEvents* ev = nullptr);

}  // namespace cpb
