/* cpb_moe.h -- C ABI of the MI355X (gfx950) MoE expert-FFN decode path.
 *
 * Drop-in boundary for the MoE block of arizqi/cpubrrr's engines.  The
 * reference has no library, plugin or FFI layer: the path is inline code in
 * each engine's worker loop.  Each entry point below names the reference code
 * it replaces (paths relative to the reference's src/bin/).
 *
 * Conventions
 *  - Plain C types only.  Every call returns 0 on success or a negative
 *    CPB_E* code; cpb_moe_last_error() gives the message of the last failure
 *    on the calling thread.  (The reference panics instead: missing tensors,
 *    type mismatches and config asserts, engine_gpt2.rs:73-74, 603-615.)
 *  - Host pointers are copied in; all device memory is owned by the handle.
 *  - A handle serves one HIP stream and is not re-entrant; separate handles
 *    may be used from separate threads.
 *  - Weights are passed in their native GGUF layouts (MXFP4 type 39: 17-byte
 *    blocks [e8m0][16 nibble bytes]; Q4_K type 12; Q6_K type 14), exactly the
 *    bytes the reference mmaps from the model blob.
 */
#ifndef CPB_MOE_H
#define CPB_MOE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CPB_OK          0
#define CPB_EINVAL     -22   /* bad argument / shape the kernels do not support */
#define CPB_ENOMEM     -12   /* device or host allocation failed                */
#define CPB_ENODEV     -19   /* no HIP device / HIP runtime error               */
#define CPB_ESTATE     -71   /* call out of order (e.g. layer not loaded)       */

/* router: how logits become (ids, weights) */
#define CPB_ROUTER_TOPK_SOFTMAX 0  /* gpt-oss: top-k on logits, softmax over k (engine_gpt2.rs:852-867) */
#define CPB_ROUTER_SOFTMAX_TOPK 1  /* Qwen3: softmax over all, top-k, renormalise == top-k then softmax
                                      over k (engine_qwen2.rs:403-410; engine_qwen.rs:374-381)      */
/* activation */
#define CPB_ACT_SWIGLU_OAI 0       /* min(g,lim), clamp(u,+-lim), g*sigmoid(alpha*g)*(u+1) (engine_gpt2.rs:887-906) */
#define CPB_ACT_SILU       1       /* silu(g)*u (engine_qwen2.rs:414-418) */
/* rmsnorm summation order of the engine being replaced */
#define CPB_NORM_GPTOSS 0          /* 16-lane fma accumulators (engine_gpt2.rs:710-749)        */
#define CPB_NORM_QWEN   1          /* nt static slices, then serial (engine_qwen2.rs:457-467) */
/* GGUF tensor type ids */
#define CPB_GGUF_MXFP4 39
#define CPB_GGUF_Q4_K  12
#define CPB_GGUF_Q6_K  14

/* Model shape + semantics.  Mirrors the reference's config.txt keys
 * (n_embd, n_expert, n_expert_used, n_ff_exp, n_layer, rms_eps;
 * engine_gpt2.rs:64-80, engine_qwen2.rs:25-38). */
typedef struct cpb_moe_cfg {
    int   d;              /* n_embd                                     */
    int   n_expert;       /* n_expert                                   */
    int   top_k;          /* n_expert_used (1..8)                       */
    int   d_ff;           /* n_ff_exp                                   */
    int   n_layer;        /* n_layer                                    */
    int   router;         /* CPB_ROUTER_*                               */
    int   act;            /* CPB_ACT_*                                  */
    int   norm;           /* CPB_NORM_*                                 */
    int   norm_nt;        /* CPB_NORM_QWEN: number of slices (reference NT = 12), 1..64, d >= 16 * norm_nt */
    float alpha, limit;   /* SwiGLU-OAI constants (1.702, 7.0)          */
    float rms_eps;
    int   wtype_gate_up;  /* CPB_GGUF_MXFP4 or CPB_GGUF_Q4_K            */
    int   wtype_down;     /* CPB_GGUF_MXFP4, CPB_GGUF_Q4_K or CPB_GGUF_Q6_K */
    int   has_bias;       /* gpt-oss: expert biases and router bias     */
    int   max_tokens;     /* largest n_tok a forward call will pass (>=1) */
} cpb_moe_cfg;

typedef struct cpb_moe cpb_moe_t;

/* Optional per-layer intermediates, all host buffers, any may be NULL.
 * Shapes for one token (n_tok = 1); nb = d/32, nbf = d_ff/32, k = top_k.
 * MXFP4: block sums S = sum over a 32-block of KVI[code]*xq (int32).
 * Q4_K/Q6_K: per 256-superblock {sumi, mint} / {sumi}.                     */
typedef struct cpb_moe_trace {
    float*   xn;        /* [d]   normed input fed to router and quant      */
    int8_t*  xq;        /* [d]                                             */
    float*   xsb;       /* [nb] (MXFP4) or [d/256] (Q8_K)                  */
    int32_t* xsum;      /* [d/32] Q8_K only                                */
    float*   logits;    /* [n_expert]                                      */
    int32_t* ids;       /* [k]                                             */
    float*   wts;       /* [k]                                             */
    float*   gu;        /* [k][2][d_ff] gate/up outputs (+bias)            */
    int32_t* gu_sums;   /* MXFP4 [k][2][d_ff][nb]; Q4_K [k][2][d_ff][d/256][2] */
    float*   h;         /* [k][d_ff] SwiGLU-OAI / SiLU*up output before Q8  */
    int8_t*  hq;        /* [k][d_ff]                                       */
    float*   hsb;       /* [k][nbf] (MXFP4) or [k][d_ff/256] (Q8_K)        */
    int32_t* hsum;      /* [k][nbf] Q8_K only                              */
    float*   dn;        /* [k][d] down outputs (+bias)                     */
    int32_t* dn_sums;   /* MXFP4 [k][d][nbf]; Q6_K [k][d][d_ff/256]; Q4_K [k][d][d_ff/256][2] */
    int32_t  exact_router_fallbacks; /* out: 1 if this call needed the exact serial router */
} cpb_moe_trace;

/* Create a handle on HIP device `device`.  Replaces engine setup
 * (load_cfg + buffer allocation, engine_gpt2.rs:64-80, 1326-1352). */
int cpb_moe_create(const cpb_moe_cfg* cfg, int device, cpb_moe_t** out);

/* Upload one layer and re-lay out its expert weights for the GPU.
 * Replaces Layer construction + repack_mx (engine_gpt2.rs:439-461,
 * 1290-1310; engine_qwen2.rs KMat setup :220-233).
 *   gate, up : [n_expert][d_ff] rows of native GGUF bytes
 *   down     : [n_expert][d]    rows of native GGUF bytes
 *   gate_b, up_b [n_expert][d_ff], down_b [n_expert][d], router_b [n_expert]:
 *              fp32, required iff cfg.has_bias
 *   router_w : fp32 [n_expert][d] (ffn_gate_inp)
 *   norm_w   : fp32 [d] (ffn_norm), may be NULL (treated as all ones)   */
int cpb_moe_load_layer(cpb_moe_t* h, int layer,
                       const void* gate, const void* up, const void* down,
                       const float* gate_b, const float* up_b, const float* down_b,
                       const float* router_w, const float* router_b, const float* norm_w);

/* The same with each tensor's GGUF type id given explicitly, as a GGUF file
 * records it per tensor (engine_qwen2.rs:202-233 dispatches every matrix on
 * its own type; Q4_K_M Qwen3 files mix Q4_K and Q6_K ffn_down across layers).
 * MXFP4 handles take 39 for all three; k-quant handles take Q4_K (12) gate/up
 * and a Q4_K (12) or Q6_K (14) down, per layer.  Other types: CPB_EINVAL.
 * cpb_moe_load_layer is this call with cfg.wtype_gate_up / wtype_down.   */
int cpb_moe_load_layer_typed(cpb_moe_t* h, int layer, int gate_type, int up_type, int down_type,
                             const void* gate, const void* up, const void* down,
                             const float* gate_b, const float* up_b, const float* down_b,
                             const float* router_w, const float* router_b, const float* norm_w);

/* One MoE block on host memory: x[n_tok][d] <- x + MoE(norm(x)).
 * Replaces engine_gpt2.rs:845-923 (n_tok == 1), :1120-1239 (n_tok > 1),
 * engine_qwen2.rs:395-433.  apply_norm = 0 feeds x itself to the router and
 * the quantiser (input already normalised).  trace (n_tok == 1 only) may be NULL.
 * Synchronous: returns after x has been copied back.                       */
int cpb_moe_forward(cpb_moe_t* h, int layer, float* x, int n_tok, int apply_norm,
                    cpb_moe_trace* trace);

/* Same on device memory, asynchronous on the handle's stream, over layers
 * [layer0, layer0 + n_layers).  d_x is a device pointer [n_tok][d].  The
 * layer loop of forward_worker (engine_gpt2.rs:767-930, MoE part only).
 * Each distinct (layer0, n_layers, d_x, n_tok, apply_norm, stream) is
 * captured once into a HIP graph and replayed (at most 16 kept, least
 * recently used evicted).  If the stream is already being captured by the
 * caller, the kernels are launched into the caller's capture instead.      */
int cpb_moe_forward_device(cpb_moe_t* h, int layer0, int n_layers, float* d_x, int n_tok,
                           int apply_norm);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): cpb_moe_forward_device with no allocation of any kind.
 * The per-call scratch (activations, routing, h) lives in a static 256 KiB
 * device array per GPU instead of the handle's buffers; shapes whose scratch
 * exceeds it get CPB_EINVAL.  Kernels are launched directly on the handle's
 * stream (no graph is captured; per-kernel timing is not recorded).  All
 * calls on one GPU share that array: calls that overlap on one GPU (from any
 * handle or thread) race.  Each token goes through the per-token decode
 * kernels, so results equal cpb_moe_forward_device's bit for bit for n_tok = 1,
 * and those of n_tok such calls, one token each, for n_tok > 1 (where
 * cpb_moe_forward_device batches the tokens through the grouped path). */
int cpb_moe_forward_device_noalloc(cpb_moe_t* h, int layer0, int n_layers, float* d_x, int n_tok,
                                   int apply_norm);

/* Use `stream` (a hipStream_t) for all further work of this handle; NULL
 * restores the handle's own stream.  Ordered: work issued on the new stream
 * waits for everything already queued on the old one. */
int cpb_moe_set_stream(cpb_moe_t* h, void* stream);
int cpb_moe_sync(cpb_moe_t* h);
void cpb_moe_destroy(cpb_moe_t* h);
const char* cpb_moe_last_error(void);

/* The configuration the handle was created with. */
int cpb_moe_config(const cpb_moe_t* h, cpb_moe_cfg* out);

/* Device bytes held for one layer's re-laid-out expert weights (for sizing). */
int cpb_moe_layer_bytes(const cpb_moe_cfg* cfg, size_t* out);

/* Kernel timing: when enabled, forward_device records HIP events around each
 * launch on the handle's stream; cpb_moe_kernel_times returns the summed
 * milliseconds and launch counts per kernel class since the last reset:
 *   ms[0]/n[0] route, ms[1]/n[1] gate/up, ms[2]/n[2] down.                   */
int cpb_moe_timing(cpb_moe_t* h, int enable);
int cpb_moe_kernel_times(cpb_moe_t* h, double ms[3], long n[3]);

/* Test hook of the grouped (n_tok > 1) path, no counterpart in the
 * reference: one layer on host x[n_tok][d] like cpb_moe_forward, also
 * returning every integer block sum of the matrix-core products, pair-major
 * (pair = token * top_k + slot), in the per-token trace's layouts:
 *   MXFP4:  gu_sums [pairs][2][d_ff][d/32], dn_sums [pairs][d][d_ff/32];
 *   Q4_K gate/up: gu_sums [pairs][2][d_ff][d/256][2] {sumi, mint};
 *   down: Q6_K [pairs][d][d_ff/256] {acc}, Q4_K [pairs][d][d_ff/256][2].
 * Lets tests check them bit for bit against the per-token trace.           */
int cpb_moe_grouped_sums(cpb_moe_t* h, int layer, float* x, int n_tok, int apply_norm,
                         int32_t* gu_sums, int32_t* dn_sums);

#ifdef __cplusplus
}
#endif
#endif
