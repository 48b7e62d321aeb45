/* cpb_head.h -- C ABI of the two-stage LM head on MI355X (gfx950).
 *
 * Replaces the gpt-oss engine's head (paths relative to the reference's
 * src/bin/): head_worker (engine_gpt2.rs:937-1002) -- rmsnorm + Q8 of the
 * final hidden state with output_norm (rmsnorm_quant_par :730-738), a Q4
 * (or Q2) screen of every vocabulary row (dot4_q4_i8 :314-342, dot4_q2_i8
 * :403-428) in which each of n_slices workers keeps the n_cand best rows of
 * its contiguous slice of row quads (NT = 12, CAND = 8, :21-38), the exact Q8 logits of those rows
 * (dot_q8_i8 :169-191) and the greedy choice among them (sample_cands with
 * temperature 0, :128-134) -- and the load-time quantisation of the bf16
 * output.weight into Q8Mat (:464-494), Q4Mat (:237-300) and Q2Mat (:356-399) form.
 * Error codes and cpb_moe_last_error() are those of cpb_moe.h.
 */
#ifndef CPB_HEAD_H
#define CPB_HEAD_H
#include <stddef.h>
#include <stdint.h>
#include "cpb_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cpb_head_cfg {
    int   d;          /* n_embd (multiple of 32, <= 4096)                         */
    int   n_vocab;    /* rows of output.weight (multiple of 4)                    */
    int   n_slices;   /* screening workers NT (reference default 12; 1..32)       */
    int   n_cand;     /* rows kept per worker CAND (reference 8; 1..16)           */
    float rms_eps;
} cpb_head_cfg;

typedef struct cpb_head cpb_head_t;

/* Optional outputs of one forward (host buffers, any may be NULL). */
typedef struct cpb_head_trace {
    int32_t* cand_ids;     /* [n_slices * n_cand] in worker / rank order     */
    float*   cand_screen;  /* [n_slices * n_cand] their Q4 screen values     */
    float*   cand_logits;  /* [n_slices * n_cand] their exact Q8 logits      */
    int8_t*  xq;           /* [d]    Q8 of the normed hidden state           */
    float*   xsb;          /* [d/32]                                         */
    float*   screen;       /* [n_vocab] every row's Q4 screen value          */
} cpb_head_trace;

int  cpb_head_create(const cpb_head_cfg* cfg, int device, cpb_head_t** out);
/* out_w: bf16 output.weight [n_vocab][d] (GGUF type 30, host); out_norm: fp32
 * output_norm [d].  Quantised on the GPU to the reference's Q4, Q2 and Q8 forms. */
int  cpb_head_load(cpb_head_t* h, const uint16_t* out_w, const float* out_norm);
/* x: host [d] final hidden state; *chosen: the greedy token.  Synchronous. */
int  cpb_head_forward(cpb_head_t* h, const float* x, int32_t* chosen, cpb_head_trace* trace);
/* Device x [d] and device *chosen, asynchronous on the handle's stream. */
int  cpb_head_forward_device(cpb_head_t* h, const float* d_x, int32_t* d_chosen);
/* The screen's row format: 4 (Q4Mat, the reference's default) or 2 (Q2Mat,
 * the reference's CPBRR_HEAD2 option: head2_on(), engine_gpt2.rs:953-957;
 * Q2Mat :356-399, dot4_q2_i8 :403-428).  Both forms are built at load;
 * the choice applies from the next forward on.  The refine stays Q8. */
int  cpb_head_set_screen(cpb_head_t* h, int bits);
/* Calls on one handle run in order on its stream (set_stream waits for the
 * old stream's work).  Two calls that overlap -- the same handle driven from
 * two streams at once -- race on its scratch and its arrival counter. */
int  cpb_head_set_stream(cpb_head_t* h, void* stream);
int  cpb_head_sync(cpb_head_t* h);
void cpb_head_destroy(cpb_head_t* h);
/* Device bytes of the quantised head (Q4 and Q2 screen streams + Q8 rows). */
int  cpb_head_bytes(const cpb_head_cfg* cfg, size_t* out);

#ifdef __cplusplus
}
#endif
#endif
