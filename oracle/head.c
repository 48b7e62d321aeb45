/* head.c -- CPU restatement of cpubrrr's two-stage LM head (gpt-oss engine).
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker of the HIP head); built into
 * liboracle.so with oracle.c.  Citations are relative to the reference's
 * src/bin/.  Every operation is the reference's fp32 operation in its order
 * (NEON vfmaq written as fmaf; no contraction elsewhere).
 *
 * The head (engine_gpt2.rs:937-1002): rmsnorm + Q8 of the final hidden state
 * (rmsnorm_quant_par :730-738), a Q4 screen of every vocabulary row
 * (dot4_q4_i8 :314-342 over Q4Mat :237-272) in which each of NT workers keeps
 * the top CAND rows of its contiguous slice of row quads (sl(), NT = 12 by
 * default, up to 32, weighted 5 units for workers 0-11 and 2 above; CAND =
 * 8, :21-38, :636-642), then the exact Q8 logits of those NT * CAND rows
 * (dot_q8_i8 :169-191 over Q8Mat :464-494) and greedy selection over them
 * (sample_cands with temperature 0, :128-134).
 */
#include "oracle.h"
#include <math.h>
#include <float.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* engine_gpt2.rs:302-310 */
uint16_t orc_f32_to_bf16(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return (uint16_t)(((b + 0x7fffu + ((b >> 16) & 1u)) >> 16) & 0xffffu);
}
float orc_bf16_to_f32(uint16_t v) {
    uint32_t b = (uint32_t)v << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* engine_gpt2.rs:274-300 q4_scale_search: the bf16 block scale among 17
 * candidates (vmax / -nmax, nmax = 7 + t/16) with the least squared error.
 * Returns the stored scale; *idq = 1 / dequantised scale (0 if zero). */
uint16_t orc_q4_scale_search(const float* vals, float* idq) {
    float amax = 0.0f, vmax = 0.0f;
    for (int i = 0; i < 32; i++)
        if (fabsf(vals[i]) > amax) { amax = fabsf(vals[i]); vmax = vals[i]; }
    if (amax == 0.0f) { *idq = 0.0f; return 0; }
    float best_err = FLT_MAX;
    uint16_t best_db = 0;
    for (int t = 0; t < 17; t++) {
        float nmax = 7.0f + (float)t * 0.0625f;
        uint16_t db = orc_f32_to_bf16(vmax / -nmax);
        float d = orc_bf16_to_f32(db);
        if (d == 0.0f) continue;
        float id = 1.0f / d;
        float err = 0.0f;
        for (int i = 0; i < 32; i++) {
            int c = (int)floorf(vals[i] * id + 8.5f);
            c = c < 0 ? 0 : c > 15 ? 15 : c;
            float e = vals[i] - (float)(c - 8) * d;
            err += e * e;
        }
        if (err < best_err) { best_err = err; best_db = db; }
    }
    float d = orc_bf16_to_f32(best_db);
    *idq = d != 0.0f ? 1.0f / d : 0.0f;
    return best_db;
}

/* engine_gpt2.rs:240-272 Q4Mat::from_bf16, one row (natural layout: per
 * 32-block 16 bytes, byte j = code(j) | code(j + 16) << 4; one bf16 scale) */
void orc_q4_quant_row(const uint16_t* w, int cols, uint8_t* nib, uint16_t* sc) {
    for (int b = 0; b < cols / 32; b++) {
        float vals[32];
        for (int i = 0; i < 32; i++) vals[i] = orc_bf16_to_f32(w[b * 32 + i]);
        float idq;
        sc[b] = orc_q4_scale_search(vals, &idq);
        for (int j = 0; j < 16; j++) {
            int lo = (int)floorf(vals[j] * idq + 8.5f);
            int hi = (int)floorf(vals[j + 16] * idq + 8.5f);
            lo = lo < 0 ? 0 : lo > 15 ? 15 : lo;
            hi = hi < 0 ? 0 : hi > 15 ? 15 : hi;
            nib[b * 16 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* engine_gpt2.rs:356-399 Q2Mat::from_bf16, one row (natural layout: per
 * 32-block 8 bytes, byte j = code(j) | code(j + 8) << 2 | code(j + 16) << 4 |
 * code(j + 24) << 6; one bf16 scale bf16(vmax / -2), vmax the first value
 * of largest magnitude; code = clamp(floor(v / scale + 2.5), 0, 3), value
 * KVI2[code] = code - 2) */
void orc_q2_quant_row(const uint16_t* w, int cols, uint8_t* nib, uint16_t* sc) {
    for (int b = 0; b < cols / 32; b++) {
        float vals[32], vmax = 0.0f, amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            vals[i] = orc_bf16_to_f32(w[b * 32 + i]);
            if (fabsf(vals[i]) > amax) { amax = fabsf(vals[i]); vmax = vals[i]; }
        }
        uint16_t db = orc_f32_to_bf16(vmax / -2.0f);
        float dq = orc_bf16_to_f32(db);
        float idq = dq != 0.0f ? 1.0f / dq : 0.0f;
        sc[b] = db;
        for (int j = 0; j < 8; j++) {
            uint8_t byte = 0;
            for (int k = 0; k < 4; k++) {
                int c = (int)floorf(vals[j + k * 8] * idq + 2.5f);
                c = c < 0 ? 0 : c > 3 ? 3 : c;
                byte |= (uint8_t)(c << (2 * k));
            }
            nib[b * 8 + j] = byte;
        }
    }
}

/* engine_gpt2.rs:403-428 dot4_q2_i8, one row: as dot4_q4_i8, lane j takes
 * elements 4j..4j+3 and 16+4j..16+4j+3 (code of element e: bits 2 (e / 8) of
 * byte e % 8), KVI2[c] = c - 2 */
float orc_q2_row_dot(const uint8_t* nib, const uint16_t* sc, const int8_t* xq, const float* xsb, int nb) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nb; b++) {
        float sv = orc_bf16_to_f32(sc[b]) * xsb[b];
        for (int j = 0; j < 4; j++) {
            int t = 0;
            for (int i = 0; i < 4; i++) {
                int e0 = 4 * j + i, e1 = 16 + 4 * j + i;
                int c0 = (nib[b * 8 + e0 % 8] >> (2 * (e0 / 8))) & 3;
                int c1 = (nib[b * 8 + e1 % 8] >> (2 * (e1 / 8))) & 3;
                t += (c0 - 2) * xq[b * 32 + e0];
                t += (c1 - 2) * xq[b * 32 + e1];
            }
            a[j] = fmaf((float)t, sv, a[j]);
        }
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

/* engine_gpt2.rs:466-494 Q8Mat::from_bf16, one row */
void orc_q8_quant_row(const uint16_t* w, int cols, int8_t* q, float* s) {
    for (int b = 0; b < cols / 32; b++) {
        float vals[32], amax = 1e-12f;
        for (int i = 0; i < 32; i++) {
            vals[i] = orc_bf16_to_f32(w[b * 32 + i]);
            amax = fmaxf(amax, fabsf(vals[i]));
        }
        float sc = amax / 127.0f;
        s[b] = sc;
        for (int i = 0; i < 32; i++) {
            float r = roundf(vals[i] / sc);
            r = r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
            q[b * 32 + i] = (int8_t)r;
        }
    }
}

/* engine_gpt2.rs:314-342 dot4_q4_i8, one row: lane j (elements 4j..4j+3 and
 * 16+4j..16+4j+3) keeps acc_j = fma(t_j, scale * xsb, acc_j) over the blocks
 * in order (KVI4[c] = c - 8); the result is the pairwise lane sum. */
float orc_q4_row_dot(const uint8_t* nib, const uint16_t* sc, const int8_t* xq, const float* xsb, int nb) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nb; b++) {
        float sv = orc_bf16_to_f32(sc[b]) * xsb[b];
        for (int j = 0; j < 4; j++) {
            int t = 0;
            for (int i = 0; i < 4; i++) {
                int e = 4 * j + i;
                t += ((nib[b * 16 + e] & 15) - 8) * xq[b * 32 + e];
                t += ((nib[b * 16 + e] >> 4) - 8) * xq[b * 32 + 16 + e];
            }
            a[j] = fmaf((float)t, sv, a[j]);
        }
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

/* engine_gpt2.rs:169-191 dot_q8_i8: two accumulators (even / odd blocks, an
 * odd last block into the first), lane j as above; vaddvq_f32(acc0 + acc1) */
float orc_q8_row_dot(const int8_t* q, const float* s, const int8_t* xq, const float* xsb, int cols) {
    float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
    int nb = cols / 32, b = 0;
    for (; b + 2 <= nb; b += 2) {
        for (int h = 0; h < 2; h++) {
            int bb = b + h;
            float sv = s[bb] * xsb[bb];
            for (int j = 0; j < 4; j++) {
                int t = 0;
                for (int i = 0; i < 4; i++) {
                    t += q[bb * 32 + 4 * j + i] * xq[bb * 32 + 4 * j + i];
                    t += q[bb * 32 + 16 + 4 * j + i] * xq[bb * 32 + 16 + 4 * j + i];
                }
                if (h == 0) a0[j] = fmaf((float)t, sv, a0[j]);
                else a1[j] = fmaf((float)t, sv, a1[j]);
            }
        }
    }
    if (b < nb) {
        float sv = s[b] * xsb[b];
        for (int j = 0; j < 4; j++) {
            int t = 0;
            for (int i = 0; i < 4; i++) {
                t += q[b * 32 + 4 * j + i] * xq[b * 32 + 4 * j + i];
                t += q[b * 32 + 16 + 4 * j + i] * xq[b * 32 + 16 + 4 * j + i];
            }
            a0[j] = fmaf((float)t, sv, a0[j]);
        }
    }
    float v[4];
    for (int j = 0; j < 4; j++) v[j] = a0[j] + a1[j];
    return (v[0] + v[1]) + (v[2] + v[3]);
}

/* engine_gpt2.rs:937-1002 head_worker (greedy).  w: bf16 output.weight
 * [V][d] (V % 4 == 0), norm_w: output_norm [d].  Outputs (any may be NULL
 * except chosen): the nt * cand candidate ids in worker / rank order, their
 * Q4 screen values and exact Q8 logits; xq / xsb: the quantised activations.
 * The Q4 rows are quantised here (OpenMP over rows), the Q8 rows only for the
 * candidates. */
/* Q4Mat of every row (OpenMP over rows): nib [V][d/2], sc [V][d/32] -- the
 * reference's load-time quantisation (:237-300), for orc_head_pre. */
void orc_q4_quant_rows(const uint16_t* w, int V, int d, uint8_t* nib, uint16_t* sc) {
    int nth = orc_get_threads();
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int r = 0; r < V; r++)
        orc_q4_quant_row(w + (size_t)r * d, d, nib + (size_t)r * (d / 2), sc + (size_t)r * (d / 32));
}

/* sl() (engine_gpt2.rs:636-642) over n items, with wunits / total_units
 * (:29-38): workers 0..11 weigh 5 units, workers 12.. weigh EW = 2 (:21-22);
 * worker wid's slice starts at n * su(wid) / tu (integer division). */
static long head_units(int w) { return w < 12 ? 5L * w : 60L + 2L * (w - 12); }
long orc_head_slice_start(long n, int nt, int wid) {
    return (long)((unsigned long long)n * (unsigned long long)head_units(wid) / (unsigned long long)head_units(nt));
}

static void head_impl(const uint16_t* w, const uint8_t* pre_nib, const uint16_t* pre_sc, int V, int d,
                      const float* x, const float* norm_w, float eps, int nt, int cand, int32_t* cand_ids,
                      float* cand_screen, float* cand_logits, int8_t* xq_out, float* xsb_out, int32_t* chosen, int q2);

void orc_head(const uint16_t* w, int V, int d, const float* x, const float* norm_w, float eps, int nt, int cand,
              int32_t* cand_ids, float* cand_screen, float* cand_logits, int8_t* xq_out, float* xsb_out,
              int32_t* chosen) {
    head_impl(w, NULL, NULL, V, d, x, norm_w, eps, nt, cand, cand_ids, cand_screen, cand_logits, xq_out, xsb_out,
              chosen, 0);
}

/* the head with the Q2 screen (head2_on(), engine_gpt2.rs:953-957) */
void orc_head_q2(const uint16_t* w, int V, int d, const float* x, const float* norm_w, float eps, int nt, int cand,
                 int32_t* cand_ids, float* cand_screen, float* cand_logits, int8_t* xq_out, float* xsb_out,
                 int32_t* chosen) {
    head_impl(w, NULL, NULL, V, d, x, norm_w, eps, nt, cand, cand_ids, cand_screen, cand_logits, xq_out, xsb_out,
              chosen, 1);
}

/* orc_head with the Q4 rows already quantised (orc_q4_quant_rows): the
 * per-token work of the reference's head. */
void orc_head_pre(const uint16_t* w, const uint8_t* nib, const uint16_t* sc, int V, int d, const float* x,
                  const float* norm_w, float eps, int nt, int cand, int32_t* cand_ids, float* cand_screen,
                  float* cand_logits, int8_t* xq_out, float* xsb_out, int32_t* chosen) {
    head_impl(w, nib, sc, V, d, x, norm_w, eps, nt, cand, cand_ids, cand_screen, cand_logits, xq_out, xsb_out,
              chosen, 0);
}

static void head_impl(const uint16_t* w, const uint8_t* pre_nib, const uint16_t* pre_sc, int V, int d,
                      const float* x, const float* norm_w, float eps, int nt, int cand, int32_t* cand_ids,
                      float* cand_screen, float* cand_logits, int8_t* xq_out, float* xsb_out, int32_t* chosen, int q2) {
    int nb = d / 32, nq = V / 4;
    float* xn = (float*)malloc(sizeof(float) * d);
    int8_t* xq = (int8_t*)malloc(d);
    float* xsb = (float*)malloc(sizeof(float) * nb);
    float* screen = (float*)malloc(sizeof(float) * V);
    /* rmsnorm_quant_par :730-738 (ssq in the 16-lane order, then qblock32) */
    orc_rmsnorm_gptoss(x, norm_w, d, eps, xn);
    orc_qblock32(xn, d, xq, xsb);
    int nth = orc_get_threads();
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int r = 0; r < V; r++) {
        if (q2) {
            uint8_t nib[2048];
            uint16_t sc[256];
            orc_q2_quant_row(w + (size_t)r * d, d, nib, sc);
            screen[r] = orc_q2_row_dot(nib, sc, xq, xsb, nb);
        } else if (pre_nib) {
            screen[r] = orc_q4_row_dot(pre_nib + (size_t)r * (d / 2), pre_sc + (size_t)r * nb, xq, xsb, nb);
        } else {
            uint8_t nib[4096];
            uint16_t sc[256];
            orc_q4_quant_row(w + (size_t)r * d, d, nib, sc);
            screen[r] = orc_q4_row_dot(nib, sc, xq, xsb, nb);
        }
    }
    /* per worker: top-cand of its quads sl(wid, nq) (:944), insertion with
     * strict comparisons (an equal later value goes behind) */
    int nc = nt * cand;
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * nc);
    float* lv = (float*)malloc(sizeof(float) * nc);
    for (int wid = 0; wid < nt; wid++) {
        float* l = lv + wid * cand;
        int32_t* li = ids + wid * cand;
        for (int k = 0; k < cand; k++) { l[k] = -FLT_MAX; li[k] = 0; }
        long qa = orc_head_slice_start(nq, nt, wid), qb = orc_head_slice_start(nq, nt, wid + 1);
        for (long q = qa; q < qb; q++)
            for (int i = 0; i < 4; i++) {
                float val = screen[q * 4 + i];
                if (val > l[cand - 1]) {
                    int p = cand - 1;
                    while (p > 0 && l[p - 1] < val) { l[p] = l[p - 1]; li[p] = li[p - 1]; p--; }
                    l[p] = val;
                    li[p] = (int32_t)(q * 4 + i);
                }
            }
    }
    /* exact Q8 logits of the candidates, greedy over them in order (:971-986,
     * sample_cands :130-133; the slices are disjoint, so no id repeats) */
    float best = -FLT_MAX;
    int32_t bi = 0;
    for (int k = 0; k < nc; k++) {
        int8_t q8[8192];
        float s8[256];
        orc_q8_quant_row(w + (size_t)ids[k] * d, d, q8, s8);
        float lg = orc_q8_row_dot(q8, s8, xq, xsb, d);
        if (cand_ids) cand_ids[k] = ids[k];
        if (cand_screen) cand_screen[k] = lv[k];
        if (cand_logits) cand_logits[k] = lg;
        if (lg > best) { best = lg; bi = ids[k]; }
    }
    *chosen = bi;
    if (xq_out) memcpy(xq_out, xq, d);
    if (xsb_out) memcpy(xsb_out, xsb, sizeof(float) * nb);
    free(xn); free(xq); free(xsb); free(screen); free(ids); free(lv);
}
