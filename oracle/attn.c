/* attn.c -- CPU restatement of the gpt-oss engine's attention block (decode).
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker of the HIP attention); built
 * into liboracle.so.  Citations are relative to the reference's src/bin/.
 *
 * One token at position pos through one layer (engine_gpt2.rs:772-843):
 *   rmsnorm + Q8 of x with attn_norm (rmsnorm_quant_par :730-738);
 *   q/k/v = Q8 rows (Q8Mat :464-494, dot_q8_i8 :169-191) + bias, YaRN RoPE of
 *   q and k from a table computed once (rope_init / rope_yarn_slow :535-576,
 *   rope_yarn :578-590), k and v into the cache at pos;
 *   per q-head: scores = dot(k_t, q) * 1/sqrt(hd) for t in the window (every
 *   other layer a sliding window of swa positions, :797), softmax with the
 *   head's sink in the denominator, weighted sum of v_t, Q8 per 32;
 *   x += wo . ao + bo (:837).
 * Operations follow the reference's fp32 order (NEON lanes as fmaf chains).
 * The reference's exp, ln, powf, cos and sin are its platform's libm (Apple);
 * this file calls the host libm, so the RoPE table and the softmax are
 * within ulps of the reference's, and everything after them to tolerance.
 */
#include "oracle.h"
#include <math.h>
#include <float.h>
#include <stdlib.h>
#include <string.h>

/* rope_yarn_slow (:556-576) on the basis (1, 0): the table (cos, sin) * mscale
 * per (pos, i), i < hd / 2. */
void orc_rope_table(int hd, int max_seq, float base, float* tab) {
    int half = hd / 2;
    const float PI = 3.14159265358979323846f;
    float f32 = 32.0f, f1 = 1.0f;
    float fd32 = (float)hd * logf(4096.0f / (f32 * 2.0f * PI)) / (2.0f * logf(base));
    float fd1 = (float)hd * logf(4096.0f / (f1 * 2.0f * PI)) / (2.0f * logf(base));
    float low = fmaxf(floorf(fd32), 0.0f);
    float high = fminf(ceilf(fd1), (float)hd - 1.0f);
    float mscale = 1.0f + 0.1f * logf(32.0f);
    for (int pos = 0; pos < max_seq; pos++)
        for (int i = 0; i < half; i++) {
            float theta_ex = (float)pos * powf(base, -(2.0f * (float)i) / (float)hd);
            float theta_in = theta_ex / 32.0f;
            float y = ((float)i - low) / fmaxf(high - low, 0.001f);
            float yc = y < 0.0f ? 0.0f : y > 1.0f ? 1.0f : y;
            float mix = 1.0f - yc;
            float theta = theta_in * (1.0f - mix) + theta_ex * mix;
            float c = cosf(theta) * mscale, s = sinf(theta) * mscale;
            /* v = (1, 0) rotated: a*c - b*s, b*c + a*s with a = 1, b = 0 */
            tab[((size_t)pos * half + i) * 2] = 1.0f * c - 0.0f * s;
            tab[((size_t)pos * half + i) * 2 + 1] = 0.0f * c + 1.0f * s;
        }
}

/* rope_yarn (:578-590) */
static void rope(float* v, int hd, const float* tab_pos) {
    int half = hd / 2;
    for (int i = 0; i < half; i++) {
        float c = tab_pos[i * 2], s = tab_pos[i * 2 + 1];
        float a = v[i], b = v[half + i];
        v[i] = a * c - b * s;
        v[half + i] = b * c + a * s;
    }
}

void orc_attn_layer(const orc_attn_layer_t* L, int il, int pos, float* x, float* kc, float* vc, const float* rope_tab,
                    orc_attn_trace* tr) {
    int d = L->d, nh = L->nh, nkv = L->nkv, hd = L->hd, nb = d / 32;
    float* xn = (float*)malloc(sizeof(float) * d);
    int8_t* xq = (int8_t*)malloc(d);
    float* xsb = (float*)malloc(sizeof(float) * nb);
    float* q = (float*)malloc(sizeof(float) * nh * hd);
    float* k = (float*)malloc(sizeof(float) * nkv * hd);
    float* v = (float*)malloc(sizeof(float) * nkv * hd);
    float* ao = (float*)malloc(sizeof(float) * nh * hd);
    int8_t* aq = (int8_t*)malloc(nh * hd);
    float* asb = (float*)malloc(sizeof(float) * nh * hd / 32);
    float* sc = (float*)malloc(sizeof(float) * (pos + 1));
    /* :775 rmsnorm_quant_par */
    orc_rmsnorm_gptoss(x, L->attn_norm, d, L->eps, xn);
    orc_qblock32(xn, d, xq, xsb);
    const float* tp = rope_tab + (size_t)pos * (hd / 2) * 2;
    /* :782-803 q heads, then k / v heads */
    for (int r = 0; r < nh * hd; r++)
        q[r] = orc_q8_row_dot(L->wq + (size_t)r * d, L->sq + (size_t)r * nb, xq, xsb, d) + L->bq[r];
    for (int h = 0; h < nh; h++) rope(q + h * hd, hd, tp);
    for (int r = 0; r < nkv * hd; r++) {
        k[r] = orc_q8_row_dot(L->wk + (size_t)r * d, L->sk + (size_t)r * nb, xq, xsb, d) + L->bk[r];
        v[r] = orc_q8_row_dot(L->wv + (size_t)r * d, L->sv + (size_t)r * nb, xq, xsb, d) + L->bv[r];
    }
    for (int h = 0; h < nkv; h++) rope(k + h * hd, hd, tp);
    memcpy(kc + (size_t)pos * nkv * hd, k, sizeof(float) * nkv * hd);
    memcpy(vc + (size_t)pos * nkv * hd, v, sizeof(float) * nkv * hd);
    /* :806-834 attention per q-head */
    float scale = 1.0f / sqrtf((float)hd);
    int start = ((il + 1) % 2 != 0) ? (pos - (L->swa - 1) > 0 ? pos - (L->swa - 1) : 0) : 0;
    for (int h = 0; h < nh; h++) {
        int kvh = h / (nh / nkv);
        const float* qh = q + h * hd;
        for (int t = start; t <= pos; t++) {
            const float* kp = kc + ((size_t)t * nkv + kvh) * hd;
            float a[4][4] = {{0}};
            for (int j = 0; j < hd; j += 16)
                for (int m = 0; m < 4; m++)
                    for (int l = 0; l < 4; l++) a[m][l] = fmaf(kp[j + 4 * m + l], qh[j + 4 * m + l], a[m][l]);
            float s4[4];
            for (int l = 0; l < 4; l++) s4[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
            sc[t - start] = ((s4[0] + s4[1]) + (s4[2] + s4[3])) * scale;
        }
        int n = pos - start + 1;
        float mx = L->sinks[h];
        for (int t = 0; t < n; t++) if (sc[t] > mx) mx = sc[t];
        float den = expf(L->sinks[h] - mx);
        for (int t = 0; t < n; t++) { float e = expf(sc[t] - mx); sc[t] = e; den += e; }
        float acc[64];
        for (int u = 0; u < hd; u++) acc[u] = 0.0f;
        for (int ti = 0; ti < n; ti++) {
            const float* vp = vc + ((size_t)(start + ti) * nkv + kvh) * hd;
            for (int u = 0; u < hd; u++) acc[u] = fmaf(vp[u], sc[ti], acc[u]);
        }
        float inv = 1.0f / den;
        for (int u = 0; u < hd; u++) ao[h * hd + u] = acc[u] * inv;
    }
    orc_qblock32(ao, nh * hd, aq, asb);
    /* :837 o-proj + bias + residual */
    for (int r = 0; r < d; r++) {
        float o = orc_q8_row_dot(L->wo + (size_t)r * nh * hd, L->so + (size_t)r * (nh * hd / 32), aq, asb, nh * hd);
        x[r] += o + L->bo[r];
    }
    if (tr) {
        if (tr->xq) memcpy(tr->xq, xq, d);
        if (tr->xsb) memcpy(tr->xsb, xsb, sizeof(float) * nb);
        if (tr->q) memcpy(tr->q, q, sizeof(float) * nh * hd);
        if (tr->k) memcpy(tr->k, k, sizeof(float) * nkv * hd);
        if (tr->v) memcpy(tr->v, v, sizeof(float) * nkv * hd);
        if (tr->ao) memcpy(tr->ao, ao, sizeof(float) * nh * hd);
        if (tr->aq) memcpy(tr->aq, aq, nh * hd);
        if (tr->asb) memcpy(tr->asb, asb, sizeof(float) * nh * hd / 32);
    }
    free(xn); free(xq); free(xsb); free(q); free(k); free(v); free(ao); free(aq); free(asb); free(sc);
}
