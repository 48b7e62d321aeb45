// decode_mx.h -- persistent single-launch decode of a stack of gpt-oss MoE
// layers (MXFP4 experts) for one token.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "moe_common.h"

namespace cpb {

struct LayerPtrs {
    const u32x4* gu;         // gate+up stream layout
    const u32x4* dn;         // down stream layout
    const float* gate_b;
    const float* up_b;
    const float* down_b;
    const float* router_w;
    const float* router_b;
    const float* norm_w;
};

struct DecodeArgs {
    const LayerPtrs* layers; // device array, indexed by absolute layer
    int layer0, n_layers;
    float* x;                // [d] residual, updated in place
    int apply_norm;
    int d, dff, ne, k, nb, nbf, parts;
    float alpha, limit, eps;
    int norm, norm_nt;
    int T_gu, T_dn;          // workgroup roles: [0, T_gu) gate/up tiles, then T_dn down tiles
    // activations / routing scratch
    float* xn;
    int8_t* xq;
    int8_t* xqn;
    float* xsb;
    double* lstar;
    double* lbound;
    int32_t* ids;
    float* wts;
    float* logits;
    int32_t* fallback;
    int8_t* hq;
    int8_t* hqn;
    float* hsb;
    // phase counters [3 * n_layers + 1], zero at launch, zeroed again on exit
    unsigned* sync;
    int32_t* error;          // set when a bounded wait expires
    unsigned long long* stamps;  // probe builds (CPB_DECODE_STAMPS) only: [G][n_layers][8]
};

// 0 on success; -22 when the shapes are unsupported, -28 when the grid cannot
// be co-resident on this device (the caller then uses the per-phase kernels).
// `a` is validated on the host; `dev_args` is a device copy of it.
int launch_decode_mx(const DecodeArgs& a, const DecodeArgs* dev_args, hipStream_t s);
int decode_mx_grid(int d, int dff, int k);

}  // namespace cpb
