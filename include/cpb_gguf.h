/* cpb_gguf.h -- GGUF v3 reader feeding the MoE library (C ABI).
 *
 * Replaces the reference's model-loading chain for the MoE tensors:
 *   scripts/gguf_index.py:21-45   header, key/value metadata, tensor infos,
 *                                 data start aligned to general.alignment (32)
 *   scripts/setup_model.sh:45-86  manifest.txt ("data_start N", then
 *                                 "name type offset n_elements" per tensor)
 *                                 and the arch-prefix-free hparam config
 *   engine_gpt2.rs:1276-1285      mmap of the blob + manifest index
 *   engine_gpt2.rs:600-617        typed accessors that assert the GGUF type
 *                                 (0 = F32, 30 = BF16, 39 = MXFP4)
 *   engine_qwen2.rs:202-233       per-matrix Q4_K / Q6_K dispatch
 * The file is memory-mapped read-only; tensor data pointers stay valid until
 * cpb_gguf_close.  Errors are the CPB_E* codes of cpb_moe.h, with the message
 * in cpb_moe_last_error(); the reference panics on the same conditions.
 */
#ifndef CPB_GGUF_H
#define CPB_GGUF_H
#include <stddef.h>
#include <stdint.h>
#include "cpb_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids used by the reference's models */
#define CPB_GGML_F32    0
#define CPB_GGML_F16    1
#define CPB_GGML_Q8_0   8
#define CPB_GGML_Q4_K  12
#define CPB_GGML_Q6_K  14
#define CPB_GGML_BF16  30
#define CPB_GGML_MXFP4 39

typedef struct cpb_gguf cpb_gguf_t;

typedef struct cpb_gguf_tensor {
    const char*    name;        /* NUL-terminated, owned by the handle       */
    int32_t        type;        /* GGUF type id                              */
    int32_t        n_dims;      /* 1..4                                      */
    uint64_t       dims[4];     /* ggml order: dims[0] varies fastest        */
    uint64_t       n_elements;  /* product of dims (manifest's 4th column)   */
    uint64_t       offset;      /* from the data start (manifest's 3rd column) */
    uint64_t       n_bytes;     /* size of the data in the file              */
    const void*    data;        /* mmapped bytes                             */
} cpb_gguf_tensor;

/* Hyperparameters with the architecture prefix stripped, as setup_model.sh
 * writes config.txt; -1 / 0 where the file has no such key. */
typedef struct cpb_gguf_hparams {
    char    arch[32];
    int64_t n_embd, n_layer, n_head, n_head_kv, head_dim;
    int64_t n_expert, n_expert_used, n_ff_exp, sliding_window, n_vocab, context_length;
    double  rope_freq_base, rms_eps;
} cpb_gguf_hparams;

int  cpb_gguf_open(const char* path, cpb_gguf_t** out);
void cpb_gguf_close(cpb_gguf_t* g);
int  cpb_gguf_version(const cpb_gguf_t* g, uint32_t* version, uint64_t* data_start, uint64_t* alignment);
int  cpb_gguf_n_tensors(const cpb_gguf_t* g, int64_t* n);
int  cpb_gguf_tensor_at(const cpb_gguf_t* g, int64_t i, cpb_gguf_tensor* out);
/* CPB_EINVAL if absent */
int  cpb_gguf_find(const cpb_gguf_t* g, const char* name, cpb_gguf_tensor* out);
/* Scalar metadata by exact key (integers, floats and bools; strings via
 * cpb_gguf_meta_str).  CPB_EINVAL if absent or of another kind.           */
int  cpb_gguf_meta_i64(const cpb_gguf_t* g, const char* key, int64_t* out);
int  cpb_gguf_meta_f64(const cpb_gguf_t* g, const char* key, double* out);
int  cpb_gguf_meta_str(const cpb_gguf_t* g, const char* key, const char** out);
int  cpb_gguf_hparams_get(const cpb_gguf_t* g, cpb_gguf_hparams* out);
/* setup_model.sh's manifest.txt */
int  cpb_gguf_write_manifest(const cpb_gguf_t* g, const char* path);

/* Load MoE layer `layer` of a handle from the file's tensors
 * blk.{layer}.ffn_{gate,up,down}_exps.weight (+ .bias when cfg.has_bias),
 * blk.{layer}.ffn_gate_inp.weight (+ .bias), blk.{layer}.ffn_norm.weight,
 * checking every tensor's type and shape against the handle's config
 * (gate/up dims [d, d_ff, n_expert], down [d_ff, d, n_expert], router
 * [d, n_expert], F32 vectors) and dispatching each matrix on its own type. */
int  cpb_moe_load_gguf_layer(cpb_moe_t* h, const cpb_gguf_t* g, int layer);

#ifdef __cplusplus
}
#endif
#endif
