// route.hip -- per-token ffn rmsnorm, activation quantisation and router
// logits with certified error bounds (gfx950).
//
// Reference: engine_gpt2.rs:846-850 (gpt-oss) and engine_qwen2.rs:395-400
// (Qwen3).  The reference router is a sequential fp32 multiply-then-add chain
// per expert (acc = bias; acc += W[j]*xn[j]).  That order cannot run in
// parallel, so workgroup e computes expert e's logit from the same fp32
// products summed exactly in fp64, together with a rigorous bound on how far
// the reference's serial fp32 sum can lie from it:
//     |serial - exact| <= u/(1-u) * (sum_k |S_k| + n*gamma_n*A),
// S_k the exact prefix sums (from a block scan), A = |b| + sum |p_j|,
// u = 2^-24, gamma_n = n*u/(1-n*u) (Higham, Accuracy and Stability of
// Numerical Algorithms, 2nd ed., sec. 4.2).  The selection (select.h), run by
// the last workgroup of the same launch, picks the top-k and certifies it
// against these bounds, recomputing the serial chain only when an interval
// overlap could change the choice.
#include "moe_common.h"
#include "route.h"
#include "route_dev.h"
#include "select.h"

namespace cpb {

// Selection by one wavefront: rank, certify, softmax; publishes ids /
// weights / logits.
CPB_DEV void select_publish(const SelectArgs& a, unsigned char* smem, unsigned long long* stamps = nullptr) {
    __shared__ Selection sel;
    select_experts_wave(a.lstar, a.lbound, a.n_expert, a.top_k, a.router_w, a.router_b, a.xn, a.d, (double*)smem, &sel,
                        a.logits, stamps);
    const int lane = threadIdx.x;
    if (lane < a.top_k) {
        a.ids[lane] = sel.ids[lane];
        a.wts[lane] = sel.wts[lane];
        a.logits[sel.ids[lane]] = sel.logit[lane];   // as used (exact serial values after a fallback)
    }
    if (lane == 0) *a.fallback = sel.fallback;
}

// Workgroup e: expert e's certified logit and its share of the activation
// quantisation.  The last workgroup to finish (arrival counter) then runs the
// selection in its first wavefront and re-arms the counter for the next launch.
__global__ __launch_bounds__(256) void k_route(RouteArgs a, SelectArgs s, unsigned* arrive) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ unsigned last;
    route_expert(a, blockIdx.x, gridDim.x, smem);
    if (!arrive) return;            // the consumer kernel selects (kernel boundary orders the results)
    drain_memory();                 // this workgroup's results are visible device-wide
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (!last || threadIdx.x >= 64) return;
    if (threadIdx.x == 0) st_dev(arrive, 0u);
    const int e = blockIdx.x;
    select_publish(s, smem, a.stamps ? a.stamps + (size_t)e * 16 + 8 : nullptr);
}

// Standalone selection (one wavefront), for callers that route elsewhere.
__global__ __launch_bounds__(64) void k_select(SelectArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    select_publish(a, smem);
}

int launch_select(const SelectArgs* a, hipStream_t s) {
    size_t lds = sizeof(double) * 4 * a->n_expert + sizeof(float) * a->d + 64;
    launch(k_select, dim3(1), dim3(64), lds, s, *a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

int launch_route(const RouteArgs* a, const SelectArgs* sa, unsigned* arrive, hipStream_t s) {
    if (a->n_expert > 256 || a->n_expert < a->top_k || a->top_k > 8 || a->d % 32 != 0 || a->d > 4096)
        return -22;
    size_t lds = route_lds_bytes(a->d);
    const size_t lds_sel = sizeof(double) * 4 * a->n_expert + sizeof(float) * a->d + 64;
    if (lds_sel > lds) lds = lds_sel;
    launch(k_route, dim3(a->n_expert), dim3(256), lds, s, *a, *sa, arrive);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
