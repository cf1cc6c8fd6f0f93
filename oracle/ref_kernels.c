/* ref_kernels.c -- thin extern wrappers over the reference's own header-only
 * MoE kernels, compiled from the reference sources where they lie
 * (-I <reference>/c; see oracle/Makefile) into oracle/_ref/.
 *
 * TEST INFRASTRUCTURE ONLY: the compiled reference is the checker for the
 * oracle restatement (tests/test_oracle_ref.py), the generator of the golden
 * vectors (tests/golden/make_golden.py) and the "reference" CPU baseline of
 * bench.py.  No reference source is copied here; these functions only forward
 * to the reference's static functions and wire its moe_block() to hooks. */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include "moe_arch.h"
#include "moe_block.h"
#include "moe_math.h"
#include "moe_matmul.h"
#include "moe_quant.h"
#include "quant.h"

void ref_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O, int exact) { matmul_f32(y, x, W, S, I, O, exact); }
void ref_matmul_bf16(float *y, const float *x, const uint16_t *W, int S, int I, int O, int round_x, int exact) { matmul_bf16_k(y, x, W, S, I, O, round_x, exact); }
void ref_matmul_q8(float *y, const float *x, const int8_t *q, const float *s, int I, int O, int mode) { matmul_q8_k(y, x, q, s, I, O, mode, 0); }
void ref_matmul_q4_kb(float *y, const float *x, const uint8_t *p, const float *s, int S, int I, int O, int mode, int exact) { matmul_q4_kb(y, x, p, s, S, I, O, mode, exact); }
void ref_matmul_i4_grouped(float *y, const float *x, const uint8_t *p, const float *s, int S, int I, int O, int gs) { matmul_i4_grouped(y, x, p, s, S, I, O, gs); }
void ref_softmax_row(float *x, int n) { softmax_row(x, n); }
void ref_moe_topk(const float *score, const float *bias, int use_bias, int E, int K, int *sel) { moe_topk(score, bias, use_bias, E, K, sel); }
float ref_siluf(float x) { return siluf(x); }
float ref_softplusf(float x) { return softplusf(x); }
float ref_expf(float x) { return expf(x); }
float ref_log1pf(float x) { return log1pf(x); }
void ref_rmsnorm_row(float *out, const float *x, const float *w, int D, float eps) { rmsnorm_row(out, x, w, D, eps); }
void ref_omp_autotune(void) { moe_omp_autotune(); }
int ref_physical_cores(void) { return moe_physical_cores(); }

/* ---- moe_block() over host weights, hooks in the shape of laguna's
 * (router matmul, block-concatenated int4 gate_up -> SiLU-GLU -> down, bf16
 * shared expert).  gs > 0 uses matmul_i4_grouped (the reference's only
 * group-scale kernel), gs == 0 matmul_q4_k at `mode` (F32/IDOT) or exact. ---- */
typedef struct {
    int D, I, Is, E, gs, router_bf16, mode, exact;
    const void *router; const float *logit_bias;
    const uint8_t *gu_q, *dn_q; const float *gu_s, *dn_s;
    const uint16_t *sg, *su, *sd;
    float *gu, *glu, *t1, *t2;
} RefCtx;

static void hk_router(void *cx, const float *x, float *lg) {
    RefCtx *c = cx;
    if (c->router_bf16) matmul_bf16_k(lg, x, (const uint16_t *)c->router, 1, c->D, c->E, 0, c->exact);
    else matmul_f32(lg, x, (const float *)c->router, 1, c->D, c->E, c->exact);
    if (c->logit_bias) for (int e = 0; e < c->E; e++) lg[e] += c->logit_bias[e];
}
static void q4(RefCtx *c, float *y, const float *x, const uint8_t *p, const float *s, int I, int O) {
    if (c->gs > 0) matmul_i4_grouped(y, x, p, s, 1, I, O, c->gs);
    else matmul_q4_k(y, x, p, s, I, O, c->mode, c->exact);
}
static void hk_expert(void *cx, int e, const float *x, float *out) {
    RefCtx *c = cx; int D = c->D, I = c->I, gs = c->gs;
    int ngD = gs > 0 ? (D + gs - 1) / gs : 1, ngI = gs > 0 ? (I + gs - 1) / gs : 1;
    q4(c, c->gu, x, c->gu_q + (int64_t)e * 2 * I * (D / 2), c->gu_s + (int64_t)e * 2 * I * ngD, D, 2 * I);
    for (int i = 0; i < I; i++) c->glu[i] = siluf(c->gu[i]) * c->gu[I + i];
    q4(c, out, c->glu, c->dn_q + (int64_t)e * D * (I / 2), c->dn_s + (int64_t)e * D * ngI, I, D);
}
static void hk_shared(void *cx, const float *x, float *out) {
    RefCtx *c = cx; int D = c->D, SI = c->Is;
    matmul_bf16_k(c->t1, x, c->sg, 1, D, SI, 0, c->exact);
    matmul_bf16_k(c->t2, x, c->su, 1, D, SI, 0, c->exact);
    for (int i = 0; i < SI; i++) c->t1[i] = siluf(c->t1[i]) * c->t2[i];
    matmul_bf16_k(out, c->t1, c->sd, 1, SI, D, 0, c->exact);
}

/* out[s] += moe_block(x[s]) for S rows; route_act 0 sigmoid / 1 softmax */
int ref_moe_block_rows(int E, int K, int route_act, int use_corr_bias, int norm_topk, float route_scale,
                       int shared_mode, int D, int I, int Is, int gs, int router_bf16,
                       const void *router, const float *corr_bias, const float *logit_bias,
                       const uint8_t *gu_q, const float *gu_s, const uint8_t *dn_q, const float *dn_s,
                       const uint16_t *sg, const uint16_t *su, const uint16_t *sd,
                       const float *x, float *out, int S, int mode, int exact) {
    if (route_act != MOE_ROUTE_SIGMOID && route_act != MOE_ROUTE_SOFTMAX) return -1;
    RefCtx c = { D, I, Is, E, gs, router_bf16, mode, exact, router, logit_bias, gu_q, dn_q, gu_s, dn_s,
                 sg, su, sd, falloc(2 * I), falloc(I), falloc(Is > 0 ? Is : 1), falloc(Is > 0 ? Is : 1) };
    MoeDesc desc = { E, K, (MoeRouteAct)route_act, use_corr_bias, norm_topk, route_scale, (MoeSharedMode)shared_mode };
    MoeHooks hooks = { &c, hk_router, corr_bias, hk_expert, shared_mode ? hk_shared : NULL, NULL };
    for (int s = 0; s < S; s++) moe_block(&desc, &hooks, x + (int64_t)s * D, out + (int64_t)s * D, D);
    free(c.gu); free(c.glu); free(c.t1); free(c.t2);
    return 0;
}
