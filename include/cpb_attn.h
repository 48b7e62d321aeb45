/* cpb_attn.h -- C ABI of the gpt-oss attention block on MI355X (gfx950),
 * decode (one token at a time, KV cache on the GPU).
 *
 * Replaces the attention part of the gpt-oss engine's layer loop (paths
 * relative to the reference's src/bin/): engine_gpt2.rs:772-843 -- rmsnorm +
 * Q8 of x with attn_norm, the q/k/v Q8 projections + biases, YaRN RoPE from a
 * table computed once (rope_init / rope_yarn_slow :535-576), the KV cache
 * write, per-head attention with the head's sink in the softmax denominator
 * and a sliding window of sliding_window positions on every other layer
 * (layers 0, 2, ...), Q8 of the heads' outputs and x += wo . ao + bo -- and
 * the load-time Q8Mat::from_bf16 of the four weight matrices (:464-494).
 * Error codes and cpb_moe_last_error() are those of cpb_moe.h.
 */
#ifndef CPB_ATTN_H
#define CPB_ATTN_H
#include <stddef.h>
#include <stdint.h>
#include "cpb_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cpb_attn_cfg {
    int   d;               /* n_embd (multiple of 32, <= 4096)                 */
    int   n_head;          /* q heads                                          */
    int   n_head_kv;       /* k / v heads (n_head a multiple of it)            */
    int   head_dim;        /* 64 (the reference's kernels assume it)          */
    int   n_layer;
    int   max_seq;         /* cache positions (reference MAXSEQ = 4096)        */
    int   sliding_window;  /* window of the even layers (gpt-oss: 128)         */
    float rope_base;       /* rope.freq_base (gpt-oss: 150000)                 */
    float rms_eps;
} cpb_attn_cfg;

typedef struct cpb_attn cpb_attn_t;

/* Optional intermediates of one forward (host buffers, any may be NULL). */
typedef struct cpb_attn_trace {
    int8_t* xq;    /* [d]              */
    float*  xsb;   /* [d/32]           */
    float*  q;     /* [n_head*hd] after bias and RoPE */
    float*  k;     /* [n_head_kv*hd] after bias and RoPE (the cache row) */
    float*  v;     /* [n_head_kv*hd]   */
    float*  ao;    /* [n_head*hd] heads' outputs */
    int8_t* aq;    /* [n_head*hd]      */
    float*  asb;   /* [n_head*hd/32]   */
} cpb_attn_trace;

int  cpb_attn_create(const cpb_attn_cfg* cfg, int device, cpb_attn_t** out);
/* bf16 weights (host, GGUF type 30): wq [n_head*hd][d], wk / wv
 * [n_head_kv*hd][d], wo [d][n_head*hd]; fp32 attn_norm [d], bq, bk, bv, bo,
 * sinks [n_head] (blk.{layer}.attn_q/k/v/out.weight/.bias, attn_sinks,
 * attn_norm.weight). */
int  cpb_attn_load_layer(cpb_attn_t* h, int layer, const float* attn_norm, const uint16_t* wq, const uint16_t* wk,
                         const uint16_t* wv, const uint16_t* wo, const float* bq, const float* bk, const float* bv,
                         const float* bo, const float* sinks);
/* x [d] (host) <- x + attention(x) for the token at position pos (< max_seq)
 * of layer `layer`; the cache rows of pos are written.  Synchronous.      */
int  cpb_attn_forward(cpb_attn_t* h, int layer, int pos, float* x, cpb_attn_trace* trace);
/* The same on device x [d], asynchronous on the handle's stream. */
int  cpb_attn_forward_device(cpb_attn_t* h, int layer, int pos, float* d_x);
/* Forget every cached position (a new sequence). */
int  cpb_attn_reset(cpb_attn_t* h);
/* Calls on one handle run in order on its stream (set_stream waits for the
 * old stream's work).  Two calls that overlap -- the same handle driven from
 * two streams at once -- race on its scratch, the cache and the arrival
 * counters.  Launches of cpb_attn_forward_device may be captured into a
 * caller's graph (they record no memset); the position is part of what is
 * captured. */
int  cpb_attn_set_stream(cpb_attn_t* h, void* stream);
int  cpb_attn_sync(cpb_attn_t* h);
void cpb_attn_destroy(cpb_attn_t* h);

#ifdef __cplusplus
}
#endif
#endif
