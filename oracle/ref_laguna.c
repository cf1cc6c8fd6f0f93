/* ref_laguna.c -- runs the reference Laguna engine's own MoE entry point,
 * lag_moe_rows (c/laguna.c:805-824: per-token moe_block for S == 1, chunked
 * lag_moe_group for S > 1), on host weights, by compiling c/laguna.c where it
 * lies with main() renamed (the reference tests include engine sources the
 * same way, e.g. c/tests/test_i4_grouped.c:20-22).  Laguna's container is
 * per-row int4 (gs = 0), an f32 router with e_score_correction_bias, sigmoid
 * routing, norm_topk, route_scale and a bf16 shared expert.
 *
 * TEST INFRASTRUCTURE ONLY (oracle/_ref): pins the oracle's sw_moe_block_rows
 * and sw_moe_group_rows, at gs = 0, to the engine's real code path. */
#define main laguna_main_unused
#include "laguna.c"
#undef main

/* h[S,D] += MoE(x[S,D]) through lag_moe_rows.  exact -> g_exact (double
 * kernels); group -> LAG_NOGROUP off/on (grouped vs per-token for S > 1). */
int ref_laguna_moe_rows(int E, int K, int norm_topk, float route_scale, int D, int I, int Is,
                        const float *router, const float *ebias,
                        const uint8_t *gu_q, const float *gu_s, const uint8_t *dn_q, const float *dn_s,
                        const uint16_t *sg, const uint16_t *su, const uint16_t *sd,
                        const float *x, float *h, int S, int exact, int group) {
    static Model m;
    static Layer L;
    memset(&m, 0, sizeof m); memset(&L, 0, sizeof L);
    m.c.hidden = D; m.c.n_experts = E; m.c.topk = K; m.c.moe_inter = I; m.c.shared_inter = Is;
    m.c.norm_topk = norm_topk; m.c.route_scale = route_scale;
    m.xq = 1; m.res_dt = 1;
    L.router = (float *)router; L.ebias = (float *)ebias;
    L.gu_q = (uint8_t *)gu_q; L.gu_s = (float *)gu_s; L.dn_q = (uint8_t *)dn_q; L.dn_s = (float *)dn_s;
    L.sg = (void *)sg; L.su = (void *)su; L.sd = (void *)sd;
    g_res_dt = 1; g_exact = exact; g_group = group;
    lag_moe_rows(&m, &L, x, h, S);
    g_exact = 0; g_group = 1;
    return 0;
}

#ifdef COLI_CUDA
/* The same engine entry with the layer resident on the device, as the engine's
 * loader leaves it (c/laguna.c:420-433): built with -DCOLI_CUDA and linked
 * against libsabrewing_loader.so, lag_moe_rows then calls lag_cuda_moe_experts
 * (S == 1, through moe_block's expert_batch hook), lag_cuda_moe_group (S > 1,
 * after its own host counting sort, chunked at 128 rows) and
 * lag_cuda_matmul_bf16 (the shared expert).  The host pointers are whatever
 * the caller passes: a test passes poisoned copies, so that a silent fallback
 * to the engine's CPU path shows up as a wrong result. */
int ref_laguna_moe_rows_dev(int E, int K, int norm_topk, float route_scale, int D, int I, int Is,
                            const float *router, const float *ebias,
                            const uint8_t *gu_q, const float *gu_s, const uint8_t *dn_q, const float *dn_s,
                            const uint16_t *sg, const uint16_t *su, const uint16_t *sd,
                            void *d_gu_q, float *d_gu_s, void *d_dn_q, float *d_dn_s,
                            void *d_sg, void *d_su, void *d_sd,
                            const float *x, float *h, int S, int group) {
    static int inited = 0;
    if (!inited) { if (lag_cuda_init(0) != 0) return -1; inited = 1; }
    static Model m;
    static Layer L;
    memset(&m, 0, sizeof m); memset(&L, 0, sizeof L);
    m.c.hidden = D; m.c.n_experts = E; m.c.topk = K; m.c.moe_inter = I; m.c.shared_inter = Is;
    m.c.norm_topk = norm_topk; m.c.route_scale = route_scale;
    m.xq = 1; m.res_dt = 1;
    L.router = (float *)router; L.ebias = (float *)ebias;
    L.gu_q = (uint8_t *)gu_q; L.gu_s = (float *)gu_s; L.dn_q = (uint8_t *)dn_q; L.dn_s = (float *)dn_s;
    L.sg = (void *)sg; L.su = (void *)su; L.sd = (void *)sd;
    L.d_gu_q = d_gu_q; L.d_gu_s = d_gu_s; L.d_dn_q = d_dn_q; L.d_dn_s = d_dn_s;
    L.d_sg = d_sg; L.d_su = d_su; L.d_sd = d_sd;
    g_res_dt = 1; g_exact = 0; g_group = group;
    lag_moe_rows(&m, &L, x, h, S);
    g_group = 1;
    return 0;
}
#endif
