/* sw_oracle.h -- CPU restatement of the sabrewing MoE-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (sabrewing_amd/, include/)
 * links, loads or calls this code.  It is the checker for the HIP path: the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg are its only
 * users.  Every function restates one reference function and cites the
 * reference file:line it follows (paths relative to the reference repo root).
 *
 * Pinning (see the header of sw_oracle.c and tests/test_oracle_*.py):
 *   - bit-exact against the compiled reference (oracle/_ref) on seeded inputs,
 *   - bit-exact against committed golden vectors made from the compiled
 *     reference (tests/golden/),
 *   - against closed forms / brute force for what neither fixes.
 */
#ifndef SW_ORACLE_H
#define SW_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- seeded synthetic data ----------------
 * SplitMix64 counter stream -> Box-Muller in double.  The transcendental steps
 * use this file's own fixed-sequence ln/sin/cos so that the HIP generator can
 * reproduce the same bits (tests compare tensor hashes). */
uint64_t sw_mix64(uint64_t z);
uint64_t sw_u64(uint64_t seed, uint64_t i);
double   sw_normal(uint64_t seed, uint64_t i);
uint64_t sw_tensor_seed(uint64_t base, int layer, int tensor_id);
void     sw_fill_normal_f32(float *out, int64_t n, uint64_t seed, uint64_t offset, double sigma);
float    sw_round_bf16(float x);                 /* f32 -> bf16 (RNE) -> f32 */
uint16_t sw_f32_to_bf16(float x);
float    sw_bf16_to_f32(uint16_t b);
void     sw_round_bf16_inplace(float *x, int64_t n);
void     sw_f32_to_bf16_array(uint16_t *out, const float *x, int64_t n);
uint64_t sw_fnv1a64(const void *p, size_t n, uint64_t h);

/* tensor ids for sw_tensor_seed */
enum { SW_T_ROUTER = 1, SW_T_GATE_UP = 2, SW_T_DOWN = 3, SW_T_SH_GATE = 4, SW_T_SH_UP = 5,
       SW_T_SH_DOWN = 6, SW_T_X = 7, SW_T_CORR_BIAS = 8, SW_T_NORM = 9, SW_T_HEAD = 10 };

/* ---------------- int4 container quantisers ----------------
 * nibble = q + 8, low nibble = even column; per-row (gs=0) or per-group (gs>0)
 * f32 scale s = max(amax/7, 1e-8).  gs>0 scale layout: scale[o*ng + g]. */
void sw_quant_i4(uint8_t *packed, float *scale, const float *w, int O, int I, int gs);
/* generate rows [row0, row0+nrows) of a seeded N(0,sigma) [O,I] tensor and
 * quantise them straight into the container (no full f32 copy) */
void sw_gen_q4(uint8_t *packed, float *scale, uint64_t seed, double sigma,
               int64_t row0, int64_t nrows, int I, int gs);

/* ---------------- kernels (reference contracts) ---------------- */
void sw_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O, int exact);
void sw_glm_logits(const float *x, const float *W, const float *bias, int D, int E, float *logit, float *choice);
void sw_glm_matmul(float *y, const float *x, const float *W, int S, int I, int O);
void sw_matmul_bf16(float *y, const float *x, const uint16_t *W, int S, int I, int O, int exact);
/* bf16 weights against bf16-rounded activations (inkling's matmul_h contract) */
void sw_matmul_bf16_rx(float *y, const float *x, const uint16_t *W, int S, int I, int O);
uint16_t sw_f32_to_bf16_ne(float f);
enum { SW_Q4_F32 = 0, SW_Q4_IDOT = 1 };
/* int8 weights + f32 row scales (mode SW_Q4_F32 / SW_Q4_IDOT: the same two contracts) */
void sw_matmul_q8(float *y, const float *x, const int8_t *q, const float *scale, int S, int I, int O, int mode);
void sw_matmul_q4(float *y, const float *x, const uint8_t *packed, const float *scale,
                  int S, int I, int O, int mode, int exact);
void sw_matmul_i4_grouped(float *y, const float *x, const uint8_t *q4, const float *scale,
                          int S, int I, int O, int gs);
void  sw_expf_array(float *y, const float *x, int64_t n);
void  sw_log1pf_array(float *y, const float *x, int64_t n);
float sw_siluf(float x);
float sw_softplusf(float x);
float sw_sigmoidf(float x);
void  sw_softmax_row(float *x, int n);
void  sw_softmax_row_olmoe(float *x, int n);
void  sw_moe_route_qwen(const float *logit, int E, int K, int *sel, float *w);
void  sw_moe_topk(const float *score, const float *corr_bias, int use_bias, int E, int K, int *sel);
void  sw_rmsnorm_row(float *out, const float *x, const float *w, int D, float eps);
int   sw_argmax(const float *v, int n);

/* ---------------- MoE block ---------------- */
/* SW_ROUTE_INKLING: the Inkling engine's moe() routing (c/inkling.c:1027-1043):
 * logits over E routed + n_shared shared rows; selection by moe_topk on the
 * routed sigmoids plus the correction bias; weights the sigmoids of the K
 * picks' and the n_shared shared logits, their float sum (ranks, then the
 * shared) s, each times route_scale / s (route_scale = the engine's
 * route_scale * gate.global_scale, formed by the caller in float).
 * SW_SHARED_GATED: the n_shared shared experts take those weights, after the
 * routed ranks, with no further scale (c/inkling.c:1166-1183); their matmuls
 * are inkling's matmul_h (bf16 weights, bf16-rounded activations). */
enum { SW_ROUTE_SIGMOID = 0, SW_ROUTE_SOFTMAX = 1, SW_ROUTE_SOFTPLUS = 2, SW_ROUTE_SOFTMAX_OLMOE = 3,
       SW_ROUTE_SOFTMAX_QWEN = 4, SW_ROUTE_SQRT_SOFTPLUS = 5, SW_ROUTE_INKLING = 6 };
enum { SW_SHARED_NONE = 0, SW_SHARED_UNSCALED = 1, SW_SHARED_GATED = 3 };

typedef struct {
    int   n_experts, topk, route_act, use_corr_bias, norm_topk;
    float route_scale;
    int   shared_mode;
    int   n_shared;            /* SW_ROUTE_INKLING: shared logit rows / SW_SHARED_GATED experts */
} SwMoeDesc;

/* Host weights of one MoE layer, in the reference container layout
 * (docs/laguna.md:34-44; c/laguna.c:586-588):
 *   gu_q [E*2I, D/2] (gate rows then up rows per expert), gu_s [E*2I*ngD]
 *   dn_q [E*D, I/2], dn_s [E*D*ngI]   (ng = 1 when gs == 0)
 *   router: f32 [E,D] or bf16 [E,D] (router_bf16)
 *   shared: bf16 [Is,D],[Is,D],[D,Is] (or f32 when shared_f32); GATED:
 *           n_shared experts stacked, [ns*Is,D],[ns*Is,D],[ns,D,Is]
 *   SW_ROUTE_INKLING: router [E + n_shared, D]                          */
typedef struct {
    int D, I, Is, E, gs;
    int router_bf16, shared_f32;
    const void *router;
    const float *corr_bias;     /* [E] or NULL */
    const float *logit_bias;    /* [E] or NULL: router-hook wrapper adding b_e to logits */
    const uint8_t *gu_q, *dn_q;
    const float *gu_s, *dn_s;
    const void *sg, *su, *sd;
} SwMoeLayer;

enum { SW_MODE_F32 = 0, SW_MODE_IDOT = 1, SW_MODE_EXACT = 2 };

/* routing for S rows: logits (optional out), sel [S*K], w [S*K] */
/* gate + top-k of S rows of given logits [S,E] (no corr_bias) */
void sw_route_logits(const SwMoeDesc *d, const float *logits, int S, int *sel, float *w);
void sw_moe_route(const SwMoeDesc *d, const SwMoeLayer *L, const float *x, int S,
                  int mode, float *logits, int *sel, float *w);
/* per-token moe_block for each of S rows: out[s] += MoE(x[s]) */
void sw_moe_block_rows(const SwMoeDesc *d, const SwMoeLayer *L, const float *x, float *out,
                       int S, int mode);
/* grouped batched path (lag_moe_group): bit-identical to sw_moe_block_rows */
void sw_moe_group_rows(const SwMoeDesc *d, const SwMoeLayer *L, const float *x, float *out,
                       int S, int mode);
/* the counting sort of lag_moe_group; returns G */
int sw_bucket(const int *sel, int S, int K, int E, int *gexp, int *gbeg, int *gcnt,
              int *grow, int *rowof);

#ifdef __cplusplus
}
#endif
#endif
