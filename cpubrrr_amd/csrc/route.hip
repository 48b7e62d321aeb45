// route.hip -- per-token ffn rmsnorm, activation quantisation and router
// logits with certified error bounds (gfx950).
//
// Reference: engine_gpt2.rs:846-850 (gpt-oss) and engine_qwen2.rs:395-400
// (Qwen3).  The reference router is a sequential fp32 multiply-then-add chain
// per expert (acc = bias; acc += W[j]*xn[j]).  That order cannot run in
// parallel, so workgroup e computes expert e's logit in fp64 together with a
// rigorous bound on how far the reference's serial fp32 result can lie from
// it (route_dev.h).  The consumer kernel (the expert gate/up GEMV) selects the
// top-k from these intervals at its start (select.h), recomputing the serial
// chain only when an interval overlap could change the choice.
#include "moe_common.h"
#include "route.h"
#include "route_dev.h"

namespace cpb {

// Workgroup e: expert e's certified logit and its share of the activation
// quantisation.
__global__ __launch_bounds__(320) void k_route(RouteArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    route_expert(a, blockIdx.x, gridDim.x, smem);
}

int launch_route(const RouteArgs* a, hipStream_t s) {
    if (a->n_expert > 256 || a->n_expert < a->top_k || a->top_k > 8 || a->d % 32 != 0 || a->d > 4096)
        return -22;
    launch(k_route, dim3(a->n_expert), dim3(route_threads(a->d)), route_lds_bytes(a->d, route_slices(*a)), s, *a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
