// moe_mx.h -- launch arguments of the MXFP4 expert GEMV kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "moe_common.h"
#include "select.h"

namespace cpb {

struct GateUpArgs {
    const u32x4* w;          // stream layout of gate+up, all experts
    const float* gate_b;     // [ne][dff] or null
    const float* up_b;       // [ne][dff] or null
    const uint8_t* ximg;     // [d/32][64] fp8 activation image (mx_dev.h)
    const float* xsb;        // [d/32]
    const int32_t* ids;      // [top_k] selected experts, when sel.lstar is null
    SelectIn sel;            // otherwise every workgroup selects at its start (workgroup 0 publishes ids / wts)
    int dff, nb, nparts, top_k;
    float alpha, limit;
    int8_t* hq;              // [top_k][dff]
    uint8_t* himg;           // [top_k][dff/32][64] fp8 image of hq (mx_dev.h)
    float* hsb;              // [top_k][dff/32]
    // trace (TRACE instantiation only)
    float* gu;               // [top_k][2][dff]
    int32_t* gu_sums;        // [top_k][2][dff][nb]
    float* h;                // [top_k][dff]
};

struct DownArgs {
    const u32x4* w;          // stream layout of down, all experts
    const float* down_b;     // [ne][d] or null
    const uint8_t* himg;     // [top_k][dff/32][64]
    const float* hsb;        // [top_k][dff/32]
    const int32_t* ids;
    const float* wts;
    int d, dff, nbf, nparts, top_k;
    float* x;                // [d] residual, updated in place
    float* dn;               // trace [top_k][d]
    int32_t* dn_sums;        // trace [top_k][d][nbf]
};

// Rows per down row tile of the stream layout: 64 / top_k lanes of one
// expert slot per 16-lane group for top_k in {1, 2, 4}; otherwise 16 rows,
// with the slots run four at a time (a 5th..8th slot in a second pass).
CPB_DEV_HOST_INLINE int mx_down_rt(int top_k) { return (top_k == 1 || top_k == 2) ? 64 / top_k : 16; }

size_t mx_gateup_bytes(int ne, int dff, int nb);
size_t mx_down_bytes(int ne, int d, int nbf, int top_k);
int launch_count_special_exps(const uint8_t* raw, size_t nblocks, unsigned* out, hipStream_t s);
int launch_repack_gateup(const uint8_t* gate, const uint8_t* up, u32x4* out, int ne, int dff, int nb, hipStream_t s);
int launch_repack_down(const uint8_t* down, u32x4* out, int ne, int d, int nbf, int top_k, hipStream_t s);
int launch_gateup_mx(const GateUpArgs& a, bool trace, hipStream_t s);
int launch_down_mx(const DownArgs& a, bool trace, hipStream_t s);

}  // namespace cpb
