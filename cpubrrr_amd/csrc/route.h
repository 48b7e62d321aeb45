// route.h -- launch arguments of the per-token routing kernel.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cpb {

struct RouteArgs {
    const float* x;          // [d] residual input
    const float* norm_w;     // [d] or null (ones)
    const float* router_w;   // [ne][d]
    const float* router_b;   // [ne] or null
    int d, n_expert, top_k;
    int norm, norm_nt, apply_norm;
    float eps;
    int qk;                  // 0: Q8 per 32 (MXFP4 experts), 1: Q8_K per 256 (k-quant experts)
    float* xn;               // [d]
    int8_t* xq;              // [d]
    uint8_t* ximg;           // [d/32][64] fp8 activation image of xq (qk == 0; layout in mx_dev.h)
    float* xsb;              // [d/32] or [d/256]
    int32_t* xsum;           // [d/32] (qk == 1)
    double* lstar;           // [ne] fp64 logit (route_dev.h)
    double* lbound;          // [ne] bound on |reference serial fp32 logit - lstar|
};

// Routing: expert e's certified logit (lstar / lbound) and the activation
// quantisation, one workgroup per expert.
int launch_route(const RouteArgs* a, hipStream_t s);

}  // namespace cpb
