/* oracle.h -- CPU restatement of the cpubrrr MoE expert-FFN decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product path (cpubrrr_amd/) and the "port" CPU baseline timed by bench.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product never links, imports or calls anything here.
 *
 * Every function restates the reference (arizqi/cpubrrr, Rust + NEON) in
 * plain C, keeping the reference's floating-point operation order so that
 * results are bit-identical wherever the reference's arithmetic is
 * deterministic IEEE-754 (everything except libm expf, see oracle.c).
 * Compiled with -ffp-contract=off: an fma appears only where the reference
 * has one (NEON vfmaq), written as fmaf().
 *
 * Layouts are the reference's native GGUF layouts:
 *   MXFP4 (type 39): row = nb blocks of 17 bytes [e8m0][16 nibble bytes];
 *     element j<16 = low nibble of byte j, element 16+j = high nibble.
 *   Q4_K (type 12): 144-byte superblocks of 256; Q6_K (type 14): 210 bytes.
 */
#ifndef CPB_ORACLE_H
#define CPB_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
float orc_e8m0_half(uint8_t e);                 /* engine_gpt2.rs:436-438 */
float orc_half_to_f32(uint16_t h);              /* engine_qwen2.rs:40-51  */
void  orc_unpack_k4(const uint8_t* scales12, uint8_t sc[8], uint8_t mn[8]); /* engine_qwen2.rs:59-74 */

/* ---- norms and activation quantisation ---------------------------------- */
float orc_ssq_gptoss(const float* x, int d);                                   /* engine_gpt2.rs:710-726 */
void  orc_rmsnorm_gptoss(const float* x, const float* w, int d, float eps, float* out); /* :742-749 */
void  orc_rmsnorm_qwen(const float* x, const float* w, int d, float eps, int nt, float* out); /* engine_qwen2.rs:457-467 */
void  orc_qblock32(const float* src, int n, int8_t* xq, float* xsb);           /* engine_gpt2.rs:691-699 */
void  orc_qblock_k(const float* src, int n, int8_t* xq, float* ys, int32_t* xsum); /* engine_qwen2.rs:288-300 */

/* ---- router ------------------------------------------------------------- */
/* logits[e] = b[e] (or 0 when b == NULL) + sequential sum of W[e][j]*xn[j]   */
void  orc_router(const float* W, const float* b, const float* xn, int ne, int d, float* logits);
void  orc_topk_gptoss(const float* logits, int ne, int k, int32_t* ids, float* wts); /* engine_gpt2.rs:852-867 */
void  orc_topk_qwen(const float* logits, int ne, int k, int32_t* ids, float* wts);   /* engine_qwen2.rs:403-410 */

/* ---- expert dots -------------------------------------------------------- */
/* MXFP4 row dot, reference lane order (dot4_mx_i8, engine_gpt2.rs:194-228).
 * If sums != NULL, writes the nb int32 block sums S_b = sum KVI[c]*xq.       */
float orc_mx_row_dot(const uint8_t* row, const int8_t* xq, const float* xsb, int nb, int32_t* sums);
/* Q4_K / Q6_K int-accumulation dots (engine_qwen2.rs:84-114, 164-200).
 * If sums != NULL: Q4_K writes per superblock {sumi, mint}; Q6_K writes sumi. */
float orc_q4k_dot(const uint8_t* row, const int8_t* xq, const float* ys, const int32_t* xsum, int cols, int32_t* sums);
float orc_q6k_dot(const uint8_t* row, const int8_t* xq, const float* ys, int cols, int32_t* sums);

/* ---- one MoE layer ------------------------------------------------------- */
typedef struct orc_trace {
    float*   xn;        /* [d]                                   */
    int8_t*  xq;        /* [d]                                   */
    float*   xsb;       /* [d/32]  gpt-oss; [d/256] qwen (ys)     */
    int32_t* xsum;      /* [d/32]  qwen only                      */
    float*   logits;    /* [ne]                                  */
    int32_t* ids;       /* [k]                                   */
    float*   wts;       /* [k]                                   */
    float*   gu;        /* [k][2][dff]  gate/up dot (+bias)       */
    int32_t* gu_sums;   /* gpt-oss [k][2][dff][d/32]; qwen [k][2][dff][d/256][2] */
    float*   h;         /* [k][dff]  activation before quant      */
    int8_t*  hq;        /* [k][dff]                              */
    float*   hsb;       /* [k][dff/32] gpt-oss; [k][dff/256] qwen */
    int32_t* hsum;      /* [k][dff/32] qwen only                  */
    float*   dn;        /* [k][d]  down dot (+bias)               */
    int32_t* dn_sums;   /* gpt-oss [k][d][dff/32]; qwen [k][d][dff/256] */
} orc_trace;

typedef struct orc_gptoss_layer {
    int d, dff, ne, k;
    float alpha, limit, eps;
    const uint8_t* gate;   /* [ne][dff][d/32*17]   */
    const uint8_t* up;     /* [ne][dff][d/32*17]   */
    const uint8_t* down;   /* [ne][d][dff/32*17]   */
    const float* gate_b;   /* [ne][dff] */
    const float* up_b;     /* [ne][dff] */
    const float* down_b;   /* [ne][d]   */
    const float* router_w; /* [ne][d]   */
    const float* router_b; /* [ne]      */
    const float* norm_w;   /* [d] (used when apply_norm) */
} orc_gptoss_layer;

/* engine_gpt2.rs:845-923: x <- x + sum_ei w_ei * (down_e(hq_ei) + down_b_e).
 * apply_norm=0 feeds x itself as xn (config 0 of the bench: input already normed). */
void orc_gptoss_moe(const orc_gptoss_layer* L, float* x, int apply_norm, orc_trace* tr);
/* scripts/ffn_reference.py's float64 dequant algorithm (scale 2^(e-128)):
 * the CPU baseline's second mode.  x <- x + the layer's MoE output. */
void orc_gptoss_moe_f64(const orc_gptoss_layer* L, float* x, int apply_norm);

typedef struct orc_qwen_layer {
    int d, dff, ne, k, nt;
    float eps;
    int gate_type, up_type, down_type;  /* GGUF ids 12 (Q4_K) / 14 (Q6_K) */
    const uint8_t* gate;   /* [ne][dff] rows of d/256 superblocks */
    const uint8_t* up;
    const uint8_t* down;   /* [ne][d] rows of dff/256 superblocks */
    const float* router_w; /* [ne][d] */
    const float* norm_w;   /* [d] */
} orc_qwen_layer;

/* engine_qwen2.rs:395-433 */
void orc_qwen_moe(const orc_qwen_layer* L, float* x, int apply_norm, orc_trace* tr);

/* ---- two-stage LM head (head.c; engine_gpt2.rs:237-342, 464-494, 937-1002) -- */
uint16_t orc_f32_to_bf16(float v);
float    orc_bf16_to_f32(uint16_t v);
uint16_t orc_q4_scale_search(const float* vals, float* idq);
void  orc_q4_quant_row(const uint16_t* w, int cols, uint8_t* nib, uint16_t* sc);
void  orc_q8_quant_row(const uint16_t* w, int cols, int8_t* q, float* s);
float orc_q4_row_dot(const uint8_t* nib, const uint16_t* sc, const int8_t* xq, const float* xsb, int nb);
float orc_q8_row_dot(const int8_t* q, const float* s, const int8_t* xq, const float* xsb, int cols);
long  orc_head_slice_start(long n, int nt, int wid);
void  orc_q2_quant_row(const uint16_t* w, int cols, uint8_t* nib, uint16_t* sc);
float orc_q2_row_dot(const uint8_t* nib, const uint16_t* sc, const int8_t* xq, const float* xsb, int nb);
void  orc_head_q2(const uint16_t* w, int V, int d, const float* x, const float* norm_w, float eps, int nt, int cand,
                  int32_t* cand_ids, float* cand_screen, float* cand_logits, int8_t* xq_out, float* xsb_out,
                  int32_t* chosen);
void  orc_head(const uint16_t* w, int V, int d, const float* x, const float* norm_w, float eps, int nt, int cand,
               int32_t* cand_ids, float* cand_screen, float* cand_logits, int8_t* xq_out, float* xsb_out,
               int32_t* chosen);
void  orc_q4_quant_rows(const uint16_t* w, int V, int d, uint8_t* nib, uint16_t* sc);
void  orc_head_pre(const uint16_t* w, const uint8_t* nib, const uint16_t* sc, int V, int d, const float* x,
                   const float* norm_w, float eps, int nt, int cand, int32_t* cand_ids, float* cand_screen,
                   float* cand_logits, int8_t* xq_out, float* xsb_out, int32_t* chosen);

/* ---- attention block, decode (attn.c; engine_gpt2.rs:535-590, 772-843) ---- */
typedef struct orc_attn_layer_t {
    int d, nh, nkv, hd, swa;
    float eps;
    const float* attn_norm;                       /* [d] */
    const int8_t* wq; const float* sq;            /* Q8 rows [nh*hd][d], scales [nh*hd][d/32] */
    const int8_t* wk; const float* sk;            /* [nkv*hd][d] */
    const int8_t* wv; const float* sv;            /* [nkv*hd][d] */
    const int8_t* wo; const float* so;            /* [d][nh*hd] */
    const float *bq, *bk, *bv, *bo, *sinks;       /* [nh*hd] [nkv*hd] [nkv*hd] [d] [nh] */
} orc_attn_layer_t;
typedef struct orc_attn_trace {
    int8_t* xq; float* xsb; float* q; float* k; float* v; float* ao; int8_t* aq; float* asb;
} orc_attn_trace;
void orc_rope_table(int hd, int max_seq, float base, float* tab);
/* x [d] updated in place; kc / vc: this layer's cache [max_seq][nkv][hd] */
void orc_attn_layer(const orc_attn_layer_t* L, int il, int pos, float* x, float* kc, float* vc, const float* rope_tab,
                    orc_attn_trace* tr);

/* ---- configuration --------------------------------------------------------*/
void orc_set_threads(int n);   /* OpenMP threads for the row loops (0 = default) */
int  orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
