// moe_kq.h -- launch arguments of the Q4_K / Q6_K (Qwen3) expert kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cpb {

struct KqArgs {
    const uint8_t* gate;     // [ne][dff] Q4_K rows (native superblock layout)
    const uint8_t* up;       // [ne][dff] Q4_K rows
    const uint8_t* down;     // [ne][d] Q6_K or Q4_K rows
    int gate_type, down_type;
    const int8_t* xq;        // [d]
    const float* xs;         // [d/256]
    const int32_t* xsum;     // [d/32]
    const int32_t* ids;      // [top_k]
    const float* wts;        // [top_k]
    int d, dff, top_k;
    float* hbuf;             // [top_k][dff]
    int8_t* hq;              // [top_k][dff]
    float* hs;               // [top_k][dff/256]
    int32_t* hsum;           // [top_k][dff/32]
    float* x;                // [d] residual, updated in place
    // trace
    float* gu;               // [top_k][2][dff]
    int32_t* gu_sums;        // [top_k][2][dff][d/256][2]
    float* dn;               // [top_k][d]
    int32_t* dn_sums;        // [top_k][d][dff/256]
};

int launch_gateup_kq(const KqArgs& a, bool trace, hipStream_t s);
int launch_down_kq(const KqArgs& a, bool trace, hipStream_t s);

}  // namespace cpb
