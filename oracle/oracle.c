/* oracle.c -- CPU restatement of the cpubrrr MoE expert-FFN decode path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + "port" CPU baseline); the HIP
 * product path never links or calls it.  Reference = arizqi/cpubrrr;
 * file:line citations are relative to its src/bin/ directory.
 *
 * Bit-exactness: every operation below is the reference's IEEE-754 fp32
 * operation in the reference's order (Rust never contracts a*b+c into an fma;
 * NEON vfmaq is an fma and is written as fmaf here).  The one thing no
 * restatement can reproduce is the ulp behaviour of the reference platform's
 * libm expf (Apple, aarch64): this file calls the host libm expf, which is
 * within 1 ulp of it.  Values that pass through expf (router softmax weights,
 * the SwiGLU activation and therefore hq/hsb) are compared to tolerance;
 * everything upstream of expf is compared bit-for-bit.
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* doubled E2M1: engine_gpt2.rs:152 (KVI) */
static const int8_t KVI[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static int g_threads = 0;
void orc_set_threads(int n) { g_threads = n; }
int orc_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

/* engine_gpt2.rs:436-438: tbl[e] = 2f32.powi(e - 128).  Rust's powi for a
 * negative exponent computes 1 / (2^|n|) by repeated squaring, so for e = 0
 * the intermediate 2^128 overflows to +inf and the table entry is 0, not
 * 2^-128.  Every other entry is the exact power of two (e = 1 gives the
 * subnormal 2^-127). */
float orc_e8m0_half(uint8_t e) {
    int n = (int)e - 128;
    int recip = n < 0;
    unsigned p = (unsigned)(recip ? -n : n);
    float a = 2.0f, mul = 1.0f;
    for (;;) {
        if (p & 1u) mul *= a;
        p >>= 1;
        if (p == 0) break;
        a *= a;
    }
    return recip ? 1.0f / mul : mul;
}

/* engine_qwen2.rs:40-51 */
float orc_half_to_f32(uint16_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) bits = s << 31;
        else {
            int ex = -1; uint32_t mm = m;
            do { ex += 1; mm <<= 1; } while (!(mm & 0x400u));
            bits = (s << 31) | ((uint32_t)(112 - ex) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 0x1f) bits = (s << 31) | (0xffu << 23) | (m << 13);
    else bits = (s << 31) | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &bits, 4); return f;
}

/* engine_qwen2.rs:59-74 (ggml get_scale_min_k4, all 8 at once) */
void orc_unpack_k4(const uint8_t* q, uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 8; j++) {
        if (j < 4) { sc[j] = q[j] & 63; mn[j] = q[j + 4] & 63; }
        else {
            sc[j] = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
            mn[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
        }
    }
}

/* engine_gpt2.rs:710-726: 4 NEON accumulators x 4 lanes over 16-wide steps
 * (fma), vaddvq(vaddq(vaddq(a0,a1), vaddq(a2,a3))), then a scalar tail. */
float orc_ssq_gptoss(const float* x, int d) {
    float a[4][4] = {{0}};
    int i = 0;
    for (; i + 16 <= d; i += 16)
        for (int v = 0; v < 4; v++)
            for (int l = 0; l < 4; l++) {
                float t = x[i + 4 * v + l];
                a[v][l] = fmaf(t, t, a[v][l]);
            }
    float L[4];
    for (int l = 0; l < 4; l++) L[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    float s = (L[0] + L[1]) + (L[2] + L[3]);      /* vaddvq_f32: pairwise */
    for (; i < d; i++) s += x[i] * x[i];
    return s;
}

/* engine_gpt2.rs:742-749 */
void orc_rmsnorm_gptoss(const float* x, const float* w, int d, float eps, float* out) {
    float inv = 1.0f / sqrtf(orc_ssq_gptoss(x, d) / (float)d + eps);
    for (int i = 0; i < d; i++) out[i] = x[i] * inv * w[i];
}

/* engine_qwen2.rs:457-467 with the static slices of sl() (:243-250):
 * worker partial sums (mul then add), then a sequential sum of the nt partials. */
void orc_rmsnorm_qwen(const float* x, const float* w, int d, float eps, int nt, float* out) {
    if (nt <= 0) nt = 12;
    float tot = 0.0f;
    int base = d / nt, rem = d % nt;
    for (int wid = 0; wid < nt; wid++) {
        int a = wid * base + (wid < rem ? wid : rem);
        int sz = base + (wid < rem ? 1 : 0);
        float ps = 0.0f;
        for (int i = a; i < a + sz; i++) { float v = x[i]; ps += v * v; }
        tot += ps;
    }
    float inv = 1.0f / sqrtf(tot / (float)d + eps);
    for (int i = 0; i < d; i++) out[i] = x[i] * inv * w[i];
}

static inline int8_t q8_round(float v, float sc) {
    float r = roundf(v / sc);               /* Rust f32::round: ties away from zero */
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

/* engine_gpt2.rs:691-699 (per 32-block, amax seeded at 1e-12) */
void orc_qblock32(const float* src, int n, int8_t* xq, float* xsb) {
    for (int b = 0; b < n / 32; b++) {
        float amax = 1e-12f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(src[b * 32 + i]));
        float sc = amax / 127.0f;
        xsb[b] = sc;
        for (int i = 0; i < 32; i++) xq[b * 32 + i] = q8_round(src[b * 32 + i], sc);
    }
}

/* engine_qwen2.rs:288-300 (Q8_K-style: one scale per 256, int32 sums per 32) */
void orc_qblock_k(const float* src, int n, int8_t* xq, float* ys, int32_t* xsum) {
    for (int sb = 0; sb < n / 256; sb++) {
        float amax = 1e-12f;
        for (int i = 0; i < 256; i++) amax = fmaxf(amax, fabsf(src[sb * 256 + i]));
        float sc = amax / 127.0f;
        ys[sb] = sc;
        for (int j = 0; j < 8; j++) {
            int32_t acc = 0;
            for (int i = 0; i < 32; i++) {
                int8_t q = q8_round(src[sb * 256 + j * 32 + i], sc);
                xq[sb * 256 + j * 32 + i] = q;
                acc += q;
            }
            xsum[sb * 8 + j] = acc;
        }
    }
}

/* engine_gpt2.rs:849-850 (gpt-oss, acc seeded with the bias) and
 * engine_qwen2.rs:400 (Qwen, acc seeded with 0.0): a sequential fp32
 * multiply-then-add chain. */
void orc_router(const float* W, const float* b, const float* xn, int ne, int d, float* logits) {
    for (int e = 0; e < ne; e++) {
        float acc = b ? b[e] : 0.0f;
        const float* w = W + (size_t)e * d;
        for (int j = 0; j < d; j++) acc += w[j] * xn[j];
        logits[e] = acc;
    }
}

/* engine_gpt2.rs:852-867: descending insertion (strict comparisons: the
 * lowest expert index wins a tie), softmax over the k selected. */
void orc_topk_gptoss(const float* logits, int ne, int k, int32_t* ids, float* wts) {
    int top[8] = {0}; float tv[8];
    for (int i = 0; i < 8; i++) tv[i] = -FLT_MAX;
    for (int e = 0; e < ne; e++) {
        float v = logits[e];
        if (v > tv[k - 1]) {
            int p = k - 1;
            while (p > 0 && tv[p - 1] < v) { tv[p] = tv[p - 1]; top[p] = top[p - 1]; p--; }
            tv[p] = v; top[p] = e;
        }
    }
    float lmax = tv[0], wsum = 0.0f, ex[8];
    for (int i = 0; i < k; i++) { ex[i] = expf(tv[i] - lmax); wsum += ex[i]; }
    for (int i = 0; i < k; i++) { ids[i] = top[i]; wts[i] = ex[i] / wsum; }
}

/* engine_qwen2.rs:403-410: stable descending sort, top-k, softmax over the k
 * (lmax = max of the k).  Equivalent in ids to the definition "softmax over
 * all experts, top-k, renormalise" (engine_qwen.rs:374-381). */
void orc_topk_qwen(const float* logits, int ne, int k, int32_t* ids, float* wts) {
    int order[512];
    for (int i = 0; i < ne; i++) order[i] = i;
    /* stable insertion sort, descending */
    for (int i = 1; i < ne; i++) {
        int o = order[i]; int p = i;
        while (p > 0 && logits[order[p - 1]] < logits[o]) { order[p] = order[p - 1]; p--; }
        order[p] = o;
    }
    float lmax = -FLT_MAX;
    for (int i = 0; i < k; i++) lmax = fmaxf(lmax, logits[order[i]]);
    float wsum = 0.0f, ex[16];
    for (int i = 0; i < k; i++) { ex[i] = expf(logits[order[i]] - lmax); wsum += ex[i]; }
    for (int i = 0; i < k; i++) { ids[i] = order[i]; wts[i] = ex[i] / wsum; }
}

/* engine_gpt2.rs:194-228 for one row.  Per 32-block b: four sdot lanes
 * t_j (lane j covers elements 4j..4j+3 and 16+4j..16+4j+3), converted once,
 * fma'd with sv = tbl[e]*xsb[b] into four lane accumulators; vaddvq at the end. */
float orc_mx_row_dot(const uint8_t* row, const int8_t* xq, const float* xsb, int nb, int32_t* sums) {
    float a[4] = {0, 0, 0, 0};
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = row + (size_t)b * 17;
        const uint8_t* qs = blk + 1;
        const int8_t* x0 = xq + b * 32;
        const int8_t* x1 = x0 + 16;
        float sv = orc_e8m0_half(blk[0]) * xsb[b];
        int32_t S = 0;
        for (int j = 0; j < 4; j++) {
            int32_t t = 0;
            for (int i = 0; i < 4; i++) {
                uint8_t c = qs[4 * j + i];
                t += (int32_t)KVI[c & 0xF] * x0[4 * j + i];
            }
            for (int i = 0; i < 4; i++) {
                uint8_t c = qs[4 * j + i];
                t += (int32_t)KVI[c >> 4] * x1[4 * j + i];
            }
            a[j] = fmaf((float)t, sv, a[j]);
            S += t;
        }
        if (sums) sums[b] = S;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

/* engine_qwen2.rs:84-114 */
float orc_q4k_dot(const uint8_t* row, const int8_t* xq, const float* ys, const int32_t* xsum, int cols, int32_t* sums) {
    float sumf = 0.0f;
    for (int sb = 0; sb < cols / 256; sb++) {
        const uint8_t* b = row + (size_t)sb * 144;
        float d = orc_half_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        float dmin = orc_half_to_f32((uint16_t)(b[2] | (b[3] << 8)));
        uint8_t sc[8], mn[8];
        orc_unpack_k4(b + 4, sc, mn);
        const uint8_t* qs = b + 16;
        int32_t sumi = 0;
        for (int jj = 0; jj < 4; jj++) {
            int j0 = 2 * jj, j1 = 2 * jj + 1;
            const int8_t* x0 = xq + sb * 256 + j0 * 32;
            const int8_t* x1 = xq + sb * 256 + j1 * 32;
            int32_t s0 = 0, s1 = 0;
            for (int i = 0; i < 32; i++) {
                s0 += (int32_t)(qs[jj * 32 + i] & 0xF) * x0[i];
                s1 += (int32_t)(qs[jj * 32 + i] >> 4) * x1[i];
            }
            sumi += s0 * sc[j0] + s1 * sc[j1];
        }
        int32_t mint = 0;
        for (int j = 0; j < 8; j++) mint += (int32_t)mn[j] * xsum[sb * 8 + j];
        float ysb = ys[sb];
        if (sums) { sums[2 * sb] = sumi; sums[2 * sb + 1] = mint; }
        sumf += ysb * d * (float)sumi - ysb * dmin * (float)mint;
    }
    return sumf;
}

/* engine_qwen2.rs:164-200 */
float orc_q6k_dot(const uint8_t* row, const int8_t* xq, const float* ys, int cols, int32_t* sums) {
    float sumf = 0.0f;
    for (int sb = 0; sb < cols / 256; sb++) {
        const uint8_t* b = row + (size_t)sb * 210;
        const uint8_t* ql = b; const uint8_t* qh = b + 128; const int8_t* scp = (const int8_t*)(b + 192);
        float d = orc_half_to_f32((uint16_t)(b[208] | (b[209] << 8)));
        int8_t t[256];
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                uint8_t qla = ql[h * 64 + l], qlb = ql[h * 64 + 32 + l], qhv = qh[h * 32 + l];
                t[h * 128 + l]      = (int8_t)(((qla & 0xF) | ((qhv & 3) << 4)) - 32);
                t[h * 128 + 32 + l] = (int8_t)(((qlb & 0xF) | (((qhv >> 2) & 3) << 4)) - 32);
                t[h * 128 + 64 + l] = (int8_t)(((qla >> 4) | (((qhv >> 4) & 3) << 4)) - 32);
                t[h * 128 + 96 + l] = (int8_t)(((qlb >> 4) | ((qhv >> 6) << 4)) - 32);
            }
        int32_t acc = 0;
        for (int g = 0; g < 16; g++) {
            int32_t s = 0;
            for (int i = 0; i < 16; i++) s += (int32_t)t[g * 16 + i] * xq[sb * 256 + g * 16 + i];
            acc += s * (int32_t)scp[g];
        }
        if (sums) sums[sb] = acc;
        sumf += ys[sb] * d * (float)acc;
    }
    return sumf;
}

/* engine_gpt2.rs:887-906 for one 32-block: clamped SwiGLU-OAI, then Q8. */
static void swiglu_oai_q8_block(const float* g, const float* u, float alpha, float lim,
                                float* hout, int8_t* hq, float* hsb) {
    float h[32]; float amax = 1e-12f;
    for (int k = 0; k < 32; k++) {
        float xg = fminf(g[k], lim);
        float yu = fminf(fmaxf(u[k], -lim), lim);
        float v = (xg / (1.0f + expf(-alpha * xg))) * (yu + 1.0f);
        h[k] = v;
        amax = fmaxf(amax, fabsf(v));
    }
    float sc = amax / 127.0f;
    *hsb = sc;
    for (int k = 0; k < 32; k++) { hq[k] = q8_round(h[k], sc); if (hout) hout[k] = h[k]; }
}

void orc_gptoss_moe(const orc_gptoss_layer* L, float* x, int apply_norm, orc_trace* tr) {
    const int d = L->d, dff = L->dff, ne = L->ne, k = L->k;
    const int nb = d / 32, nbf = dff / 32;
    const size_t rowb = (size_t)nb * 17, rowbf = (size_t)nbf * 17;
    int nth = orc_get_threads();
    (void)nth;
    float* xn = (float*)malloc(sizeof(float) * d);
    int8_t* xq = (int8_t*)malloc(d);
    float* xsb = (float*)malloc(sizeof(float) * nb);
    float logits[512]; int32_t ids[8]; float wts[8];
    float* gu = (float*)malloc(sizeof(float) * (size_t)k * 2 * dff);
    int8_t* hq = (int8_t*)malloc((size_t)k * dff);
    float* hsb = (float*)malloc(sizeof(float) * (size_t)k * nbf);

    /* :846 rmsnorm (or the given normed input), :847 qblock32, :849-850 router */
    if (apply_norm) orc_rmsnorm_gptoss(x, L->norm_w, d, L->eps, xn);
    else memcpy(xn, x, sizeof(float) * d);
    orc_qblock32(xn, d, xq, xsb);
    orc_router(L->router_w, L->router_b, xn, ne, d, logits);
    orc_topk_gptoss(logits, ne, k, ids, wts);                       /* :852-867 */

    /* :870-884 gate/up (+bias) */
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int it = 0; it < k * 2 * dff; it++) {
        int ei = it / (2 * dff), rem = it % (2 * dff), isup = rem >= dff, r = rem % dff;
        int e = ids[ei];
        const uint8_t* W = isup ? L->up : L->gate;
        const float* B = isup ? L->up_b : L->gate_b;
        int32_t* sums = tr && tr->gu_sums ? tr->gu_sums + (size_t)it * nb : NULL;
        float acc = orc_mx_row_dot(W + ((size_t)e * dff + r) * rowb, xq, xsb, nb, sums);
        gu[it] = acc + B[(size_t)e * dff + r];
    }
    /* :887-906 SwiGLU-OAI + Q8 per 32-block */
    for (int it = 0; it < k * nbf; it++) {
        int ei = it / nbf, blk = it % nbf;
        const float* g = gu + (size_t)ei * 2 * dff + blk * 32;
        const float* u = g + dff;
        swiglu_oai_q8_block(g, u, L->alpha, L->limit,
                            tr && tr->h ? tr->h + (size_t)ei * dff + blk * 32 : NULL,
                            hq + (size_t)ei * dff + blk * 32, hsb + (size_t)ei * nbf + blk);
    }
    /* :908-922 down + bias + weighted residual, ei ascending per element */
    float* dn = tr && tr->dn ? tr->dn : NULL;
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int r = 0; r < d; r++) {
        float s = x[r];
        for (int ei = 0; ei < k; ei++) {
            int e = ids[ei];
            int32_t* sums = tr && tr->dn_sums ? tr->dn_sums + ((size_t)ei * d + r) * nbf : NULL;
            float acc = orc_mx_row_dot(L->down + ((size_t)e * d + r) * rowbf,
                                       hq + (size_t)ei * dff, hsb + (size_t)ei * nbf, nbf, sums);
            float v = acc + L->down_b[(size_t)e * d + r];
            if (dn) dn[(size_t)ei * d + r] = v;
            s += wts[ei] * v;
        }
        x[r] = s;
    }
    if (tr) {
        if (tr->xn) memcpy(tr->xn, xn, sizeof(float) * d);
        if (tr->xq) memcpy(tr->xq, xq, d);
        if (tr->xsb) memcpy(tr->xsb, xsb, sizeof(float) * nb);
        if (tr->logits) memcpy(tr->logits, logits, sizeof(float) * ne);
        if (tr->ids) memcpy(tr->ids, ids, sizeof(int32_t) * k);
        if (tr->wts) memcpy(tr->wts, wts, sizeof(float) * k);
        if (tr->gu) memcpy(tr->gu, gu, sizeof(float) * (size_t)k * 2 * dff);
        if (tr->hq) memcpy(tr->hq, hq, (size_t)k * dff);
        if (tr->hsb) memcpy(tr->hsb, hsb, sizeof(float) * (size_t)k * nbf);
    }
    free(xn); free(xq); free(xsb); free(gu); free(hq); free(hsb);
}

static float kdot(int type, const uint8_t* row, const int8_t* xq, const float* ys, const int32_t* xsum,
                  int cols, int32_t* sums) {
    /* KMat::dot type dispatch, engine_qwen2.rs:202-213 */
    if (type == 12) return orc_q4k_dot(row, xq, ys, xsum, cols, sums);
    if (type == 14) return orc_q6k_dot(row, xq, ys, cols, sums);
    return 0.0f;
}
static size_t kbpr(int type, int cols) { return type == 12 ? (size_t)cols / 256 * 144 : (size_t)cols / 256 * 210; }

void orc_qwen_moe(const orc_qwen_layer* L, float* x, int apply_norm, orc_trace* tr) {
    const int d = L->d, ff = L->dff, ne = L->ne, k = L->k;
    const int nsb = d / 256, nsbf = ff / 256;
    int nth = orc_get_threads();
    float* xn = (float*)malloc(sizeof(float) * d);
    int8_t* xq = (int8_t*)malloc(d);
    float ys[64]; int32_t xsum[512];
    float logits[512]; int32_t ids[16]; float wts[16];
    float* hbuf = (float*)malloc(sizeof(float) * (size_t)k * ff);
    int8_t* hq = (int8_t*)malloc((size_t)k * ff);
    float* hs = (float*)malloc(sizeof(float) * (size_t)k * ff / 256);
    int32_t* hm = (int32_t*)malloc(sizeof(int32_t) * (size_t)k * ff / 32);
    size_t gb = kbpr(L->gate_type, d), ub = kbpr(L->up_type, d), db = kbpr(L->down_type, ff);

    if (apply_norm) orc_rmsnorm_qwen(x, L->norm_w, d, L->eps, L->nt, xn);   /* :396 */
    else memcpy(xn, x, sizeof(float) * d);
    orc_qblock_k(xn, d, xq, ys, xsum);                                     /* :397 */
    orc_router(L->router_w, NULL, xn, ne, d, logits);                      /* :400 */
    orc_topk_qwen(logits, ne, k, ids, wts);                                /* :403-410 */

    /* :414-418 gate/up + SiLU*up over topk*ff rows */
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int it = 0; it < k * ff; it++) {
        int ei = it / ff, r = it % ff;
        size_t gr = (size_t)ids[ei] * ff + r;
        int32_t* sg = tr && tr->gu_sums ? tr->gu_sums + ((size_t)(ei * 2) * ff + r) * nsb * 2 : NULL;
        int32_t* su = tr && tr->gu_sums ? tr->gu_sums + ((size_t)(ei * 2 + 1) * ff + r) * nsb * 2 : NULL;
        float g = kdot(L->gate_type, L->gate + gr * gb, xq, ys, xsum, d, sg);
        float u = kdot(L->up_type, L->up + gr * ub, xq, ys, xsum, d, su);
        if (tr && tr->gu) { tr->gu[(size_t)ei * 2 * ff + r] = g; tr->gu[(size_t)ei * 2 * ff + ff + r] = u; }
        hbuf[it] = (g / (1.0f + expf(-g))) * u;
    }
    orc_qblock_k(hbuf, k * ff, hq, hs, hm);                                /* :423 */
    /* :426-432 down + weighted accumulate, ei ascending per element */
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int r = 0; r < d; r++) {
        for (int ei = 0; ei < k; ei++) {
            int32_t* sums = tr && tr->dn_sums ? tr->dn_sums + ((size_t)ei * d + r) * nsbf * (L->down_type == 12 ? 2 : 1) : NULL;
            float v = kdot(L->down_type, L->down + ((size_t)ids[ei] * d + r) * db,
                           hq + (size_t)ei * ff, hs + (size_t)ei * nsbf, hm + (size_t)ei * (ff / 32), ff, sums);
            if (tr && tr->dn) tr->dn[(size_t)ei * d + r] = v;
            x[r] += wts[ei] * v;
        }
    }
    if (tr) {
        if (tr->xn) memcpy(tr->xn, xn, sizeof(float) * d);
        if (tr->xq) memcpy(tr->xq, xq, d);
        if (tr->xsb) memcpy(tr->xsb, ys, sizeof(float) * nsb);
        if (tr->xsum) memcpy(tr->xsum, xsum, sizeof(int32_t) * d / 32);
        if (tr->logits) memcpy(tr->logits, logits, sizeof(float) * ne);
        if (tr->ids) memcpy(tr->ids, ids, sizeof(int32_t) * k);
        if (tr->wts) memcpy(tr->wts, wts, sizeof(float) * k);
        if (tr->h) memcpy(tr->h, hbuf, sizeof(float) * (size_t)k * ff);
        if (tr->hq) memcpy(tr->hq, hq, (size_t)k * ff);
        if (tr->hsb) memcpy(tr->hsb, hs, sizeof(float) * (size_t)k * ff / 256);
        if (tr->hsum) memcpy(tr->hsum, hm, sizeof(int32_t) * (size_t)k * ff / 32);
    }
    free(xn); free(xq); free(hbuf); free(hq); free(hs); free(hm);
}


/* ---- f64 dequant reference of one gpt-oss MoE layer ----
 * scripts/ffn_reference.py:23-62 (the spec its header recovers from
 * llama.cpp: router logits = W x + b, top-4, softmax over the four;
 * g = gate_e x + gate_b, u = up_e x + up_b, SwiGLU-OAI, out += w_e (down_e h
 * + down_b)) in float64 with every weight dequantised, KV[c] * 2^(e - 128)
 * (the script's line 28 writes 2^(e - 127) with the doubled table KV, i.e.
 * twice the MXFP4 value; the reference engines use 2^(e - 128),
 * engine_gpt2.rs:437).  apply_norm: an f64 rmsnorm (x / sqrt(mean x^2 +
 * eps) * w) first, as the stacks feed it.  Ties in the top-k keep the lower
 * index (a stable descending order).  Weights are decoded row by row on the
 * fly (the script dequantised whole matrices at load). */
static double mx_row_f64(const uint8_t* row, const double* v, int cols) {
    double acc = 0.0;
    for (int b = 0; b < cols / 32; b++) {
        const uint8_t* blk = row + (size_t)b * 17;
        const double sc = ldexp(1.0, (int)blk[0] - 128);
        double s = 0.0;
        for (int j = 0; j < 16; j++) {
            s += (double)KVI[blk[1 + j] & 0xF] * v[b * 32 + j];
            s += (double)KVI[blk[1 + j] >> 4] * v[b * 32 + 16 + j];
        }
        acc += s * sc;
    }
    return acc;
}

void orc_gptoss_moe_f64(const orc_gptoss_layer* L, float* x, int apply_norm) {
    const int d = L->d, dff = L->dff, ne = L->ne, k = L->k;
    const size_t rowb = (size_t)(d / 32) * 17, rowbf = (size_t)(dff / 32) * 17;
    int nth = orc_get_threads();
    (void)nth;
    double* xn = (double*)malloc(sizeof(double) * d);
    double* h = (double*)malloc(sizeof(double) * dff);
    double* out = (double*)calloc((size_t)d, sizeof(double));
    double logit[512];
    if (apply_norm) {
        double ss = 0.0;
        for (int i = 0; i < d; i++) ss += (double)x[i] * (double)x[i];
        const double inv = 1.0 / sqrt(ss / d + (double)L->eps);
        for (int i = 0; i < d; i++) xn[i] = (double)x[i] * inv * (L->norm_w ? (double)L->norm_w[i] : 1.0);
    } else {
        for (int i = 0; i < d; i++) xn[i] = x[i];
    }
    for (int e = 0; e < ne; e++) {
        double a = L->router_b ? (double)L->router_b[e] : 0.0;
        for (int j = 0; j < d; j++) a += (double)L->router_w[(size_t)e * d + j] * xn[j];
        logit[e] = a;
    }
    int top[8];
    for (int i = 0; i < k; i++) {
        int best = -1;
        for (int e = 0; e < ne; e++) {
            int used = 0;
            for (int t = 0; t < i; t++) used |= top[t] == e;
            if (!used && (best < 0 || logit[e] > logit[best])) best = e;
        }
        top[i] = best;
    }
    double w[8], wmax = logit[top[0]], wsum = 0.0;
    for (int i = 0; i < k; i++) { w[i] = exp(logit[top[i]] - wmax); wsum += w[i]; }
    for (int i = 0; i < k; i++) w[i] /= wsum;
    const double alpha = L->alpha, lim = L->limit;
    for (int i = 0; i < k; i++) {
        const int e = top[i];
        #pragma omp parallel for schedule(static) num_threads(nth)
        for (int r = 0; r < dff; r++) {
            const size_t row = (size_t)e * dff + r;
            const double g = mx_row_f64(L->gate + row * rowb, xn, d) + (L->gate_b ? (double)L->gate_b[row] : 0.0);
            const double u = mx_row_f64(L->up + row * rowb, xn, d) + (L->up_b ? (double)L->up_b[row] : 0.0);
            const double xg = fmin(g, lim), yu = fmin(fmax(u, -lim), lim);
            h[r] = (xg / (1.0 + exp(-alpha * xg))) * (yu + 1.0);
        }
        #pragma omp parallel for schedule(static) num_threads(nth)
        for (int r = 0; r < d; r++) {
            const size_t row = (size_t)e * d + r;
            out[r] += w[i] * (mx_row_f64(L->down + row * rowbf, h, dff) + (L->down_b ? (double)L->down_b[row] : 0.0));
        }
    }
    for (int i = 0; i < d; i++) x[i] = (float)((double)x[i] + out[i]);
    free(xn); free(h); free(out);
}
