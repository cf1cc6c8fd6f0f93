/* ref_qwen35.c -- runs the reference qwen35 engine's own MoE forward,
 * moe_forward_rows (c/qwen35.c:595-700): the router on the host, its own
 * moe_route and host counting sort, lag_cuda_moe_group for the routed experts
 * (c/qwen35.c:637-642) and resmm -> lag_cuda_matmul_bf16 for the shared expert
 * and its sigmoid gate, by compiling c/qwen35.c where it lies with main()
 * renamed (as ref_laguna.c does for c/laguna.c), built with -DCOLI_CUDA and
 * linked against libsabrewing_loader.so (oracle/Makefile).  With null device
 * pointers the same entry runs the engine's CPU path (matmul_q4_kb, the
 * rank-order combine, matmul_bf16_k).
 *
 * TEST INFRASTRUCTURE ONLY (oracle/_ref): the engine's second caller of
 * lag_cuda_moe_group, unmodified, against this backend. */
#define main qwen35_main_unused
#include "qwen35.c"
#undef main

/* out[S,D] = MoE(x[S,D]) (routed + gated shared expert) through moe_forward_rows.
 * Per-row int4 experts (the engine's MOE_Q4_F32 container), an f32 router [E,D],
 * the shared gate sgate [D] and a bf16 shared expert.  d_*: the device copies
 * (all null: the CPU path).  0 = ok. */
int ref_qwen35_moe_rows(int E, int K, int D, int I, int Is, const float *router, const float *sgate,
                        const uint8_t *gu_q, const float *gu_s, const uint8_t *dn_q, const float *dn_s,
                        const uint16_t *sg, const uint16_t *su, const uint16_t *sd,
                        void *d_gu_q, float *d_gu_s, void *d_dn_q, float *d_dn_s,
                        void *d_sg, void *d_su, void *d_sd, const float *x, float *out, int S) {
    static int inited = 0;
    if (d_gu_q && !inited) { if (lag_cuda_init(0) != 0) return -1; inited = 1; }
    static Model m;
    static Layer L;
    memset(&m, 0, sizeof m); memset(&L, 0, sizeof L);
    m.c.D = D; m.c.E = E; m.c.K = K; m.c.moe_I = I; m.c.shared_I = Is;
    m.xq = 1; m.res_dt = 1;
    L.router = (float *)router; L.sgate = (float *)sgate;
    L.gu_q = (uint8_t *)gu_q; L.gu_s = (float *)gu_s; L.dn_q = (uint8_t *)dn_q; L.dn_s = (float *)dn_s;
    L.sg = (void *)sg; L.su = (void *)su; L.sd = (void *)sd;
    L.d_gu_q = d_gu_q; L.d_gu_s = d_gu_s; L.d_dn_q = d_dn_q; L.d_dn_s = d_dn_s;
    L.d_sg = d_sg; L.d_su = d_su; L.d_sd = d_sd;
    g_exact = 0;
    moe_forward_rows(&m, &L, x, S, out);
    return 0;
}
