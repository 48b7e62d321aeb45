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
    int32_t* sorted;           // [n_tok*k] pair ids (t*k + slot), grouped by expert, stable
    int4* tiles;               // [max_tiles] {expert, first sorted index, count, 0}
    int32_t* ntiles;           // [1]
    int8_t* hq;                // [n_tok*k][dff]
    float* hsb;                // [n_tok*k][nbf]
    uint8_t* himg;             // [n_tok*k][nbf][64]
    float* dnout;              // [n_tok*k][d] down rows + bias
    // trace (optional, small shapes): int32 block sums, pair-major
    int32_t* gu_sums;          // [n_tok*k][2][dff][nb]
    int32_t* dn_sums;          // [n_tok*k][d][nbf]
};

// All stages of one layer on stream s.  Shapes validated by the caller
// (MXFP4, top_k in {1,2,4}, d and dff multiples of 32).
int launch_grouped_layer(const GroupedArgs& a, bool trace, hipStream_t s);

}  // namespace cpb
