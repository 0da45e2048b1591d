/*
 * ref_harness.c - exposes the reference's own CPU kernels from zhaohb/qwen3.c
 * (c/qwen.c, compiled unmodified from /root/reference by inclusion) so the oracle
 * can be checked bit for bit against them and the CPU baseline can time them.
 *
 * TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile (target `ref`) into
 * oracle/_ref/libqwenref.so, which is git-ignored; nothing here is shipped.
 * The reference's static functions are reachable because this translation unit
 * includes c/qwen.c; its main() is renamed so the result can be a shared library.
 * The reference's stock build is `gcc -O2 -std=c11` (c/Makefile:22-30); the recipe
 * adds `-D_GNU_SOURCE -include sys/resource.h` because c/qwen.c:167 uses struct
 * rusage without including <sys/resource.h>.
 */
#define main qwen_reference_main
#include "qwen.c"
#undef main

#include <stdint.h>

void ref_matmul_q4g_asym(float *y, const float *x, const uint8_t *q, const float *sz,
                         int I, int O, int gs) {
    matmul_q4g_asym(y, x, q, sz, I, O, gs);
}

void ref_matmul(float *y, const float *x, const float *W, int S, int I, int O) {
    matmul(y, x, W, S, I, O);
}

void ref_matmul_q8(float *y, const float *x, const uint8_t *q, const float *scale, int I, int O) {
    matmul_q8(y, x, q, scale, I, O);
}

void ref_quant_rows(const float *W, int I, int O, int fmt, int gs, uint8_t *q, float *s) {
    quant_rows(W, I, O, fmt, gs, q, s);
}

void ref_rmsnorm_zc(float *out, const float *x, const float *w, int D, float eps) {
    rmsnorm_zc(out, x, w, D, eps);
}

void ref_softmax_row(float *x, int n) { softmax_row(x, n); }

/* One fmt=6 expert as the engine's Slot (c/qwen.c:117-122). */
typedef struct {
    const uint8_t *g, *u, *d;
    const float *gs, *us, *ds;
} RefExpert;

static void fill_slot(Slot *s, const RefExpert *e, int eid) {
    memset(s, 0, sizeof(*s));
    s->eid = eid;
    s->g = (uint8_t *)e->g; s->u = (uint8_t *)e->u; s->d = (uint8_t *)e->d;
    s->gs = (float *)e->gs; s->us = (float *)e->us; s->ds = (float *)e->ds;
}

void ref_expert_mlp_fmt6(const RefExpert *e, const float *x, int D, int I, int gs, float *y) {
    Cfg c;
    memset(&c, 0, sizeof(c));
    c.expert_fmt = 6; c.group_size = gs; c.expert_bits = 4;
    Slot s;
    fill_slot(&s, e, 0);
    float *g = falloc(I), *u = falloc(I);
    expert_mlp_cpu(&c, &s, x, g, u, y, D, I);
    free(g); free(u);
}

/* A one-layer Model whose expert LRU already holds every expert, so expert_get()
 * always hits and never reads a container (c/qwen.c:538-554). */
typedef struct { Model m; Layer l; LCache lc; } RefMoe;

static void ref_moe_setup(RefMoe *r, const float *router, const RefExpert *experts,
                          const RefExpert *shared, const float *sh_gate,
                          int D, int I, int E, int K, int gs) {
    memset(r, 0, sizeof(*r));
    Cfg *c = &r->m.c;
    c->hidden = D; c->n_experts = E; c->topk = K; c->inter = I; c->sh_inter = I;
    c->expert_bits = 4; c->expert_fmt = 6; c->group_size = gs; c->n_layers = 1;
    r->lc.slots = calloc((size_t)E, sizeof(Slot));
    r->lc.n = r->lc.cap = E;
    for (int e = 0; e < E; e++) fill_slot(&r->lc.slots[e], &experts[e], e);
    r->m.cache = &r->lc;
    r->m.eusage = calloc((size_t)E, sizeof(uint32_t));
    r->m.L = &r->l;
    r->l.router = (float *)router;          /* grouter.q == NULL -> f32 matmul router */
    r->l.sh_gate = (float *)sh_gate;
    VkDense *sd[3] = {&r->l.gsg, &r->l.gsu, &r->l.gsd};
    const uint8_t *sq[3] = {shared->g, shared->u, shared->d};
    const float *ss[3] = {shared->gs, shared->us, shared->ds};
    for (int j = 0; j < 3; j++) {          /* quantized host copy -> mm_dense fmt 6 path */
        sd[j]->q = (uint8_t *)sq[j]; sd[j]->s = (float *)ss[j]; sd[j]->fmt = 6; sd[j]->gs = gs;
    }
}

static void ref_moe_free(RefMoe *r) { free(r->lc.slots); free(r->m.eusage); }

/* c/qwen.c:922-928 moe_token. usage[E] (optional) receives the expert-use counts. */
void ref_moe_token(const float *x, const float *router, const RefExpert *experts,
                   const RefExpert *shared, const float *sh_gate,
                   int D, int I, int E, int K, int gs, float *out, uint32_t *usage) {
    RefMoe r;
    ref_moe_setup(&r, router, experts, shared, sh_gate, D, I, E, K, gs);
    moe_token(&r.m, &r.l, 0, x, out);
    if (usage) memcpy(usage, r.m.eusage, (size_t)E * sizeof(uint32_t));
    ref_moe_free(&r);
}

/* c/qwen.c:1185-1190 moe_batch. */
void ref_moe_batch(const float *xs, int S, const float *router, const RefExpert *experts,
                   const RefExpert *shared, const float *sh_gate,
                   int D, int I, int E, int K, int gs, float *out, uint32_t *usage) {
    RefMoe r;
    ref_moe_setup(&r, router, experts, shared, sh_gate, D, I, E, K, gs);
    moe_batch(&r.m, &r.l, 0, xs, S, out);
    if (usage) memcpy(usage, r.m.eusage, (size_t)E * sizeof(uint32_t));
    ref_moe_free(&r);
}

/* ---- layer blocks: c/qwen.c:581-667 attention and :669-776 gdn_step, CPU branch ----
 * Projections arrive as fmt 6 quantized host copies (VkDense.q, the mm_dense fallback
 * c/qwen.c:300-305); GDN a/b are f32 [VH, D] as the CPU branch reads them. */
typedef struct {
    const uint8_t *q;
    const float *s;
} RefQ6;

static void set_dense(VkDense *d, const RefQ6 *w, int gs) {
    memset(d, 0, sizeof(*d));
    d->q = (uint8_t *)w->q;
    d->s = (float *)w->s;
    d->fmt = 6;
    d->gs = gs;
}

/* One token at position pos through attention(); Kc/Vc [KH][max_t][hd] are updated. */
void ref_attention(const RefQ6 *q, const RefQ6 *k, const RefQ6 *v, const RefQ6 *o, const float *qn,
                   const float *kn, int D, int H, int KH, int hd, int rot, float theta, float eps, int gs,
                   float *Kc, float *Vc, int max_t, int pos, const float *x, float *out) {
    Model m;
    Layer l;
    memset(&m, 0, sizeof(m));
    memset(&l, 0, sizeof(l));
    Cfg *c = &m.c;
    c->hidden = D; c->n_heads = H; c->n_kv_heads = KH; c->head_dim = hd; c->rot = rot;
    c->theta = theta; c->eps = eps;
    m.K = &Kc; m.V = &Vc; m.max_t = max_t;
    set_dense(&l.gq, q, gs); set_dense(&l.gk, k, gs); set_dense(&l.gv, v, gs); set_dense(&l.go, o, gs);
    l.qn = (float *)qn; l.kn = (float *)kn;
    attention(&m, &l, 0, x, 1, pos, out);
}

/* One token through gdn_step(); convst [K][CD] and S [VH][KD][VD] are updated. */
void ref_gdn_step(const RefQ6 *qkv, const RefQ6 *z, const RefQ6 *outp, const float *a, const float *b,
                  const float *conv, const float *alog, const float *dtb, const float *gnorm, int D, int KH,
                  int KD, int VH, int VD, int K, float eps, int gs, float *convst, float *S, const float *x,
                  float *out) {
    Model m;
    Layer l;
    memset(&m, 0, sizeof(m));
    memset(&l, 0, sizeof(l));
    Cfg *c = &m.c;
    c->hidden = D; c->eps = eps;
    c->gdn_kh = KH; c->gdn_kd = KD; c->gdn_vh = VH; c->gdn_vd = VD; c->conv_k = K;
    c->key_dim = KH * KD; c->value_dim = VH * VD; c->conv_dim = 2 * c->key_dim + c->value_dim;
    m.gdnS = &S; m.convst = &convst;
    set_dense(&l.gqkv, qkv, gs); set_dense(&l.gz, z, gs); set_dense(&l.gout, outp, gs);
    l.a = (float *)a; l.b = (float *)b; l.conv = (float *)conv;
    l.alog = (float *)alog; l.dtb = (float *)dtb; l.gnorm = (float *)gnorm;
    gdn_step(&m, &l, 0, x, out);
}
