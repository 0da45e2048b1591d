/*
 * oracle.c - CPU restatement of qwen3.c's fmt=6 int4 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the CPU baseline); the product library
 * never links or calls this file.  Each function follows the cited lines of
 * zhaohb/qwen3.c c/qwen.c statement for statement where the floating-point order
 * matters, so that the compiled result is bit-identical to the reference's own
 * code built with the same flags (checked in tests/test_oracle_golden.py against
 * vectors written by the compiled reference).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* c/qwen.c:172-173 */
float orc_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }
float orc_silu(float x) { return x / (1.f + expf(-x)); }

/* c/qwen.c:211-229.  Per group: awn = sum x*nib, ax = sum x (sequential fp32, no FMA),
 * acc += scale * (awn - zero * ax). */
void orc_matmul_q4g_asym(float *y, const float *x, const uint8_t *q, const float *sz,
                         int I, int O, int gs) {
    const int rb = (I + 1) / 2, ng = (I + gs - 1) / gs;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q + (int64_t)o * rb;
        const float *sr = sz + (int64_t)o * ng * 2;
        float acc = 0.f;
        for (int g = 0; g < ng; g++) {
            const int i0 = g * gs;
            const int i1 = i0 + gs < I ? i0 + gs : I;
            const float scale = sr[2 * g], zero = sr[2 * g + 1];
            float awn = 0.f, ax = 0.f;
            for (int i = i0; i < i1; i++) {
                const int nib = (i & 1) ? (w[i >> 1] >> 4) : (w[i >> 1] & 0xF);
                awn += x[i] * (float)nib;
                ax += x[i];
            }
            acc += scale * (awn - zero * ax);
        }
        y[o] = acc;
    }
}

/* c/qwen.c:178-189: o outer, s inner, sequential fp32 dot. */
void orc_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int o = 0; o < O; o++) {
        const float *w = W + (int64_t)o * I;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float acc = 0.f;
            for (int i = 0; i < I; i++) acc += xs[i] * w[i];
            y[(int64_t)s * O + o] = acc;
        }
    }
}

/* c/qwen.c:230-238 */
void orc_matmul_q8(float *y, const float *x, const uint8_t *q, const float *scale, int I, int O) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int o = 0; o < O; o++) {
        const int8_t *w = (const int8_t *)q + (int64_t)o * I;
        float acc = 0.f;
        for (int i = 0; i < I; i++) acc += x[i] * (float)w[i];
        y[o] = acc * scale[o];
    }
}

static int clamp_i(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* c/qwen.c:242-292 (fmt 6 branch :246-265, fmt 1 branch :268-276).  RTN with a
 * real-valued zero point: scale = max((max-min)/15, 1e-8), zero = -min/scale,
 * q = clamp(lrint(w/scale + zero), 0, 15); odd tail nibble is 0. */
void orc_quant_rows(const float *W, int I, int O, int fmt, int gs, uint8_t *q, float *s) {
    for (int o = 0; o < O; o++) {
        const float *w = W + (int64_t)o * I;
        if (fmt == 6) {
            const int ng = (I + gs - 1) / gs;
            uint8_t *row = q + (int64_t)o * ((I + 1) / 2);
            float *sr = s + (int64_t)o * ng * 2;
            for (int g = 0; g < ng; g++) {
                const int i0 = g * gs;
                const int i1 = i0 + gs < I ? i0 + gs : I;
                float lo = 1e30f, hi = -1e30f;
                for (int i = i0; i < i1; i++) {
                    if (w[i] < lo) lo = w[i];
                    if (w[i] > hi) hi = w[i];
                }
                float scale = (hi - lo) / 15.f;
                if (scale < 1e-8f) scale = 1e-8f;
                const float zero = -lo / scale;
                sr[2 * g] = scale;
                sr[2 * g + 1] = zero;
                for (int i = i0; i < i1; i += 2) {
                    const int q0 = clamp_i((int)lrintf(w[i] / scale + zero), 0, 15);
                    const int q1 = i + 1 < i1 ? clamp_i((int)lrintf(w[i + 1] / scale + zero), 0, 15) : 0;
                    row[i / 2] = (uint8_t)(q0 | (q1 << 4));
                }
            }
        } else if (fmt == 1) {
            float amax = 0.f;
            for (int i = 0; i < I; i++) {
                const float a = fabsf(w[i]);
                if (a > amax) amax = a;
            }
            const float sc = amax > 0 ? amax / 127.f : 1.f;
            int8_t *row = (int8_t *)q + (int64_t)o * I;
            for (int i = 0; i < I; i++) row[i] = (int8_t)clamp_i((int)lrintf(w[i] / sc), -127, 127);
            s[o] = sc;
        }
    }
}

/* c/qwen.c:326-330 */
void orc_rmsnorm_zc(float *out, const float *x, const float *w, int D, float eps) {
    double ms = 0;
    for (int i = 0; i < D; i++) ms += (double)x[i] * x[i];
    const float r = 1.f / sqrtf((float)(ms / D) + eps);
    for (int i = 0; i < D; i++) out[i] = x[i] * r * (1.f + w[i]);
}

/* c/qwen.c:332-336 */
void orc_softmax_row(float *x, int n) {
    float m = -1e30f;
    for (int i = 0; i < n; i++)
        if (x[i] > m) m = x[i];
    float s = 0;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        s += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= s;
}

/* c/qwen.c:806-817 (identical loop at :1057-1072) */
void orc_route_topk(float *pr, int E, int K, int *idx, float *val) {
    orc_softmax_row(pr, E);
    for (int k = 0; k < K; k++) {
        int best = -1;
        float bv = -1.f;
        for (int e = 0; e < E; e++) {
            int taken = 0;
            for (int j = 0; j < k; j++)
                if (idx[j] == e) { taken = 1; break; }
            if (!taken && pr[e] > bv) { bv = pr[e]; best = e; }
        }
        idx[k] = best;
        val[k] = bv;
    }
    float sm = 0;
    for (int k = 0; k < K; k++) sm += val[k];
    for (int k = 0; k < K; k++) val[k] /= sm;
}

/* c/qwen.c:780-786 (fmt 6 branch) */
void orc_expert_mlp_fmt6(const OrcExpert *e, const float *x, int D, int I, int gs, float *y) {
    float *g = malloc((size_t)I * sizeof(float)), *u = malloc((size_t)I * sizeof(float));
    orc_matmul_q4g_asym(g, x, e->g, e->gs, D, I, gs);
    orc_matmul_q4g_asym(u, x, e->u, e->us, D, I, gs);
    for (int i = 0; i < I; i++) g[i] = orc_silu(g[i]) * u[i];
    orc_matmul_q4g_asym(y, g, e->d, e->ds, I, D, gs);
    free(g);
    free(u);
}

/* The shared expert through mm_dense2/mm_dense's quantized fallback (c/qwen.c:300-305,
 * :311-322, :911-918): gate over all rows, then up over all rows, SiLU*up, down. */
static void shared_expert_rows(const OrcExpert *sh, const float *xs, int S, int D, int I, int gs,
                               float *ysh) {
    float *g = malloc((size_t)S * I * sizeof(float)), *u = malloc((size_t)S * I * sizeof(float));
    for (int s = 0; s < S; s++) orc_matmul_q4g_asym(g + (int64_t)s * I, xs + (int64_t)s * D, sh->g, sh->gs, D, I, gs);
    for (int s = 0; s < S; s++) orc_matmul_q4g_asym(u + (int64_t)s * I, xs + (int64_t)s * D, sh->u, sh->us, D, I, gs);
    for (int64_t i = 0; i < (int64_t)S * I; i++) g[i] = orc_silu(g[i]) * u[i];
    for (int s = 0; s < S; s++) orc_matmul_q4g_asym(ysh + (int64_t)s * D, g + (int64_t)s * I, sh->d, sh->ds, I, D, gs);
    free(g);
    free(u);
}

/* c/qwen.c:833-834 (and :1159-1161): sequential dot then sigmoid. */
static float shared_gate(const float *sh_gate, const float *x, int D) {
    float t = 0;
    for (int d = 0; d < D; d++) t += sh_gate[d] * x[d];
    return orc_sigmoid(t);
}

/* c/qwen.c:922-928 + :804-920, pure-CPU branch. */
void orc_moe_decode(const float *x, const float *router, const OrcExpert *experts,
                    const OrcExpert *shared, const float *sh_gate,
                    int D, int I, int E, int K, int gs,
                    float *out, int *idx_out, float *val_out, float *shgt_out, float *logits_out) {
    float *pr = malloc((size_t)E * sizeof(float));
    orc_matmul_f32(pr, x, router, 1, D, E);
    if (logits_out) memcpy(logits_out, pr, (size_t)E * sizeof(float));
    int idx[64];
    float val[64];
    orc_route_topk(pr, E, K, idx, val);
    for (int d = 0; d < D; d++) out[d] = 0;
    const float shgt = shared_gate(sh_gate, x, D);
    float *hh = malloc((size_t)D * sizeof(float));
    for (int k = 0; k < K; k++) {
        orc_expert_mlp_fmt6(&experts[idx[k]], x, D, I, gs, hh);
        for (int d = 0; d < D; d++) out[d] += val[k] * hh[d];
    }
    shared_expert_rows(shared, x, 1, D, I, gs, hh);
    for (int d = 0; d < D; d++) out[d] += shgt * hh[d];
    if (idx_out) memcpy(idx_out, idx, (size_t)K * sizeof(int));
    if (val_out) memcpy(val_out, val, (size_t)K * sizeof(float));
    if (shgt_out) *shgt_out = shgt;
    free(hh);
    free(pr);
}

/* c/qwen.c:1185-1190 + :1050-1183, pure-CPU branch. */
void orc_moe_prefill(const float *xs, int S, const float *router, const OrcExpert *experts,
                     const OrcExpert *shared, const float *sh_gate,
                     int D, int I, int E, int K, int gs,
                     float *out, int *tidx_out, float *tval_out) {
    float *pr = malloc((size_t)S * E * sizeof(float));
    orc_matmul_f32(pr, xs, router, S, D, E);
    int *tidx = malloc((size_t)S * K * sizeof(int));
    float *tval = malloc((size_t)S * K * sizeof(float));
    for (int s = 0; s < S; s++) orc_route_topk(pr + (int64_t)s * E, E, K, tidx + (int64_t)s * K, tval + (int64_t)s * K);
    memset(out, 0, (size_t)S * D * sizeof(float));

    /* counting sort of the (token, slot) pairs by expert (c/qwen.c:1076-1083) */
    int *ecnt = calloc((size_t)E + 1, sizeof(int)), *ecur = calloc((size_t)E, sizeof(int));
    int *epair = malloc((size_t)S * K * sizeof(int));
    for (int64_t i = 0; i < (int64_t)S * K; i++) ecnt[tidx[i]]++;
    int acc = 0;
    for (int e = 0; e < E; e++) {
        const int n = ecnt[e];
        ecnt[e] = acc;
        acc += n;
    }
    ecnt[E] = acc;
    for (int64_t i = 0; i < (int64_t)S * K; i++) {
        const int e = tidx[i];
        epair[ecnt[e] + ecur[e]++] = (int)i;
    }

    /* ascending expert id, pair order within an expert (c/qwen.c:1032-1041, :1144) */
    float *hh = malloc((size_t)D * sizeof(float));
    for (int e = 0; e < E; e++) {
        for (int r = ecnt[e]; r < ecnt[e + 1]; r++) {
            const int i = epair[r], tok = i / K;
            const float w = tval[i];
            orc_expert_mlp_fmt6(&experts[e], xs + (int64_t)tok * D, D, I, gs, hh);
            float *o = out + (int64_t)tok * D;
            for (int d = 0; d < D; d++) o[d] += w * hh[d];
        }
    }
    free(hh);

    /* shared expert over all S rows (c/qwen.c:1170-1181) */
    float *ysh = malloc((size_t)S * D * sizeof(float));
    shared_expert_rows(shared, xs, S, D, I, gs, ysh);
    for (int s = 0; s < S; s++) {
        const float gt = shared_gate(sh_gate, xs + (int64_t)s * D, D);
        float *o = out + (int64_t)s * D;
        const float *y = ysh + (int64_t)s * D;
        for (int d = 0; d < D; d++) o[d] += gt * y[d];
    }
    if (tidx_out) memcpy(tidx_out, tidx, (size_t)S * K * sizeof(int));
    if (tval_out) memcpy(tval_out, tval, (size_t)S * K * sizeof(float));
    free(ysh);
    free(ecnt);
    free(ecur);
    free(epair);
    free(tidx);
    free(tval);
    free(pr);
}

/* ---------------- layer blocks ---------------- */
/* c/qwen.c:296-309: quantized host copy first (fmt 6), else the f32 original. */
void orc_proj(const OrcMat *m, const float *x, float *y) {
    if (m->fmt == 6)
        orc_matmul_q4g_asym(y, x, (const uint8_t *)m->w, m->sz, m->I, m->O, m->gs);
    else
        orc_matmul_f32(y, x, (const float *)m->w, 1, m->I, m->O);
}

/* c/qwen.c:570-579 */
void orc_rope_partial(float *x, int pos, int rot, float theta) {
    const int hr = rot / 2;
    for (int j = 0; j < hr; j++) {
        const float inv = powf(theta, -2.0f * j / rot);
        const float ang = (float)pos * inv, cs = cosf(ang), sn = sinf(ang);
        const float lo = x[j], hi = x[j + hr];
        x[j] = lo * cs - hi * sn;
        x[j + hr] = hi * cs + lo * sn;
    }
}

/* c/qwen.c:581-667 with S = 1 (CPU branch). */
void orc_gqa_decode(const OrcGqa *L, float *Kc, float *Vc, int max_t, int pos, const float *x, float *out) {
    const int H = L->H, KH = L->KH, hd = L->hd, qo = H * hd * 2, ko = KH * hd;
    float *qg = malloc((size_t)qo * sizeof(float)), *k = malloc((size_t)ko * sizeof(float));
    float *v = malloc((size_t)ko * sizeof(float)), *ctx = malloc((size_t)H * hd * sizeof(float));
    float *sc = malloc((size_t)(pos + 1) * sizeof(float));
    orc_proj(&L->q, x, qg);
    orc_proj(&L->k, x, k);
    orc_proj(&L->v, x, v);
    for (int h = 0; h < H; h++) {            /* :598-604 per-head q norm, then RoPE */
        float *qh = qg + (int64_t)h * 2 * hd;
        orc_rmsnorm_zc(qh, qh, L->qn, hd, L->eps);
        orc_rope_partial(qh, pos, L->rot, L->theta);
    }
    for (int h = 0; h < KH; h++) {           /* :605-614 k norm + RoPE, cache rows */
        float *kh = k + (int64_t)h * hd;
        orc_rmsnorm_zc(kh, kh, L->kn, hd, L->eps);
        orc_rope_partial(kh, pos, L->rot, L->theta);
        memcpy(Kc + ((int64_t)h * max_t + pos) * hd, kh, (size_t)hd * sizeof(float));
        memcpy(Vc + ((int64_t)h * max_t + pos) * hd, v + (int64_t)h * hd, (size_t)hd * sizeof(float));
    }
    const float scale = 1.f / sqrtf((float)hd);
    const int gq = H / KH;
    for (int h = 0; h < H; h++) {            /* :638-665 */
        const int kvh = h / gq;
        const float *qv = qg + (int64_t)h * 2 * hd;
        for (int t = 0; t <= pos; t++) {
            const float *kv = Kc + ((int64_t)kvh * max_t + t) * hd;
            float acc = 0;
            for (int d = 0; d < hd; d++) acc += qv[d] * kv[d];
            sc[t] = acc * scale;
        }
        orc_softmax_row(sc, pos + 1);
        float *cx = ctx + (int64_t)h * hd;
        for (int d = 0; d < hd; d++) cx[d] = 0;
        for (int t = 0; t <= pos; t++) {
            const float *vr = Vc + ((int64_t)kvh * max_t + t) * hd;
            const float a = sc[t];
            for (int d = 0; d < hd; d++) cx[d] += a * vr[d];
        }
        const float *gate = qv + hd;
        for (int d = 0; d < hd; d++) cx[d] *= orc_sigmoid(gate[d]);
    }
    orc_proj(&L->o, ctx, out);
    free(qg);
    free(k);
    free(v);
    free(ctx);
    free(sc);
}

/* c/qwen.c:175 softplus (torch default beta 1, threshold 20) */
static float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }

/* c/qwen.c:669-776 (CPU branch). */
void orc_gdn_step(const OrcGdn *L, float *st, float *S, const float *x, float *out) {
    const int KH = L->KH, KD = L->KD, VH = L->VH, VD = L->VD, K = L->K;
    const int key_dim = KH * KD, value_dim = VH * VD, CD = 2 * key_dim + value_dim;
    float *qkv = malloc((size_t)CD * sizeof(float)), *cv = malloc((size_t)CD * sizeof(float));
    float *z = malloc((size_t)value_dim * sizeof(float)), *y = malloc((size_t)value_dim * sizeof(float));
    float *qn = malloc((size_t)key_dim * sizeof(float)), *kn = malloc((size_t)key_dim * sizeof(float));
    float *a = malloc((size_t)VH * sizeof(float)), *b = malloc((size_t)VH * sizeof(float));
    float *dec = malloc((size_t)VH * sizeof(float)), *bet = malloc((size_t)VH * sizeof(float));
    float *kvm = malloc((size_t)VD * sizeof(float)), *del = malloc((size_t)VD * sizeof(float));
    orc_proj(&L->qkv, x, qkv);
    orc_proj(&L->z, x, z);
    /* :697-707 ring shift, append, conv + SiLU */
    memmove(st, st + CD, (size_t)(K - 1) * CD * sizeof(float));
    memcpy(st + (size_t)(K - 1) * CD, qkv, (size_t)CD * sizeof(float));
    for (int ch = 0; ch < CD; ch++) {
        const float *w = L->conv + (int64_t)ch * K;
        float acc = 0;
        for (int j = 0; j < K; j++) acc += w[j] * st[(size_t)j * CD + ch];
        cv[ch] = orc_silu(acc);
    }
    orc_proj(&L->b, x, b);                  /* :710-711 */
    orc_proj(&L->a, x, a);
    for (int h = 0; h < KH; h++) {           /* :713-721 */
        const float *qs = cv + h * KD, *ks = cv + key_dim + h * KD;
        float sq = 0, sk = 0;
        for (int d = 0; d < KD; d++) {
            sq += qs[d] * qs[d];
            sk += ks[d] * ks[d];
        }
        const float rq = 1.f / sqrtf(sq + L->eps) / sqrtf((float)KD), rk = 1.f / sqrtf(sk + L->eps);
        for (int d = 0; d < KD; d++) {
            qn[h * KD + d] = qs[d] * rq;
            kn[h * KD + d] = ks[d] * rk;
        }
    }
    for (int h = 0; h < VH; h++) {           /* :722-728 */
        bet[h] = orc_sigmoid(b[h]);
        dec[h] = expf(-expf(L->alog[h]) * softplus(a[h] + L->dtb[h]));
    }
    for (int h = 0; h < VH; h++) {           /* :749-773 delta rule + gated RMSNorm */
        const int src = h / (VH / KH);
        const float *qh = qn + src * KD, *kh = kn + src * KD, *vh = cv + 2 * key_dim + h * VD;
        float *Sh = S + (size_t)h * KD * VD;
        for (int d = 0; d < VD; d++) kvm[d] = 0;
        for (int i = 0; i < KD; i++) {
            float *row = Sh + (size_t)i * VD;
            const float kk = kh[i];
            for (int d = 0; d < VD; d++) {
                row[d] *= dec[h];
                kvm[d] += row[d] * kk;
            }
        }
        for (int d = 0; d < VD; d++) del[d] = (vh[d] - kvm[d]) * bet[h];
        float *yh = y + (size_t)h * VD;
        for (int d = 0; d < VD; d++) yh[d] = 0;
        for (int i = 0; i < KD; i++) {
            float *row = Sh + (size_t)i * VD;
            const float kk = kh[i], qq = qh[i];
            for (int d = 0; d < VD; d++) {
                row[d] += kk * del[d];
                yh[d] += row[d] * qq;
            }
        }
        const float *zh = z + (size_t)h * VD;
        double ms = 0;
        for (int d = 0; d < VD; d++) ms += (double)yh[d] * yh[d];
        const float r = 1.f / sqrtf((float)(ms / VD) + L->eps);
        for (int d = 0; d < VD; d++) yh[d] = yh[d] * r * L->gnorm[d] * orc_silu(zh[d]);
    }
    orc_proj(&L->out, y, out);
    free(qkv); free(cv); free(z); free(y); free(qn); free(kn);
    free(a); free(b); free(dec); free(bet); free(kvm); free(del);
}

/* c/qwen.c:1471-1472 */
int orc_argmax(const float *v, int n) {
    int best = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

void orc_topk_logits(const float *v, int n, int k, int *idx, float *val) {
    unsigned char *taken = calloc((size_t)n, 1);
    for (int r = 0; r < k; r++) {
        int best = -1;
        float bv = -INFINITY;
        for (int i = 0; i < n; i++)
            if (!taken[i] && (best < 0 || v[i] > bv)) { bv = v[i]; best = i; }
        taken[best] = 1;
        idx[r] = best;
        val[r] = bv;
    }
    free(taken);
}

/* ---------------- synthetic data ---------------- */
uint64_t orc_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t orc_hash(uint64_t seed, uint64_t i) { return orc_mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL); }

uint64_t orc_stream(uint64_t base, uint64_t tag) { return orc_mix64(base ^ orc_mix64(tag + 1)); }

static double u01(uint64_t seed, uint64_t i) { return ((double)(orc_hash(seed, i) >> 11) + 0.5) * 0x1p-53; }

double orc_normal(uint64_t seed, uint64_t i) {
    const double u1 = u01(seed, 2 * i), u2 = u01(seed, 2 * i + 1);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

float orc_f16_round(double v) {
    if (v == 0.0 || v != v) return (float)v;
    const double a = fabs(v);
    int e;
    (void)frexp(a, &e);            /* a = m * 2^e, m in [0.5, 1) */
    int ulp = e - 11;              /* binary16 keeps 11 significant bits */
    if (ulp < -24) ulp = -24;      /* subnormal spacing 2^-24 */
    double r = ldexp(nearbyint(ldexp(a, -ulp)), ulp);
    if (r > 65504.0) r = INFINITY;
    return (float)(v < 0 ? -r : r);
}

void orc_gen_bytes(uint8_t *dst, size_t n, uint64_t seed) {
    for (size_t j = 0; j < n; j++) dst[j] = (uint8_t)(orc_hash(seed, j >> 3) >> (8 * (j & 7)));
}

void orc_gen_sz(float *sz, size_t ngroups, uint64_t seed, double sigma) {
    const uint64_t zseed = seed ^ 0x5A5A5A5A5A5A5A5AULL;
    for (size_t g = 0; g < ngroups; g++) {
        sz[2 * g] = orc_f16_round(fabs(sigma * orc_normal(seed, g)));
        sz[2 * g + 1] = (float)(orc_hash(zseed, g) >> 60);
    }
}

void orc_gen_normal(float *dst, size_t n, uint64_t seed, double sigma) {
    for (size_t i = 0; i < n; i++) dst[i] = (float)(sigma * orc_normal(seed, i));
}
