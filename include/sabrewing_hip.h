/* sabrewing_hip.h -- C ABI of the MI355X (gfx950) MoE-block backend,
 * libsabrewing_hip.so.  Plain pointers and sizes only.
 *
 * Three layers of entry points:
 *   1. lag_hip_*            the Laguna backend ABI, entry for entry: same
 *                           arguments, same 0 = ok / -1 = failure convention,
 *                           host activations, device weights from
 *                           lag_hip_upload (c/backend_cuda_laguna.h:25-75).
 *                           The Linux loader (libsabrewing_loader.so,
 *                           include/sabrewing_loader.h) exports them under the
 *                           reference's lag_cuda_* names for unmodified engines.
 *   2. lag_hip_*_g          the same entries for group-scaled int4 (one f32
 *                           scale per gs inputs, the fmt=4 layout of
 *                           c/quant.h:168-203); the reference's lag family is
 *                           per-row only.
 *   3. lag_hip_moe_forward  the whole MoE block with routing on the device
 *                           (router GEMV -> gate -> top-k -> group-by-expert
 *                           -> SwiGLU experts -> combine -> shared expert ->
 *                           residual), device activations, the descriptor of
 *                           c/moe_arch.h:33-41.
 *
 * Like the reference backend: one device and one stream per process (a second
 * lag_hip_init naming another device fails), results
 * valid on return for the host-pointer entries, not thread-safe.
 * COLI_GPU_FAIL_AFTER=N makes every compute entry fail after N successful
 * calls (the reference's fault-injection hook, c/backend_cuda.cu:684-693). */
#ifndef SABREWING_HIP_H
#define SABREWING_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- 1. Laguna backend ABI (replaces c/backend_cuda_laguna.h) ---------------- */
/* lag_cuda_init (c/backend_cuda_laguna.h:25): select device, create the stream. 0 = ok */
int    lag_hip_init(int dev);
/* lag_cuda_free_bytes / lag_cuda_total_bytes (:26-27) */
size_t lag_hip_free_bytes(void);
size_t lag_hip_total_bytes(void);
/* lag_cuda_upload / lag_cuda_free (:28-29): plain byte copy, NULL = error */
void  *lag_hip_upload(const void *h, size_t n);
void   lag_hip_free(void *d);
/* lag_cuda_matmul_bf16 (:32): y[S,O] = x[S,I] @ W^T, W device bf16 [O,I], x/y host f32 */
int    lag_hip_matmul_bf16(float *y, const float *x, const void *W, int S, int I, int O);
/* lag_cuda_matmul_q4 (:39): per-row int4 [O,I/2] + f32 scale [O], nibble-8 */
int    lag_hip_matmul_q4(float *y, const float *x, const void *packed, const void *scale, int S, int I, int O);
/* lag_cuda_expert_q4 (:44): out[D] = W2 @ silu_glu(W13 @ x), gate_up block-concatenated */
int    lag_hip_expert_q4(float *out, const float *x, const void *p13, const void *s13,
                         const void *p2, const void *s2, int I, int D);
/* lag_cuda_moe_experts (:51): out[D] = sum_k w[k] * expert(sel[k], x), layer blobs */
int    lag_hip_moe_experts(float *out, const float *x, const void *gu_q, const float *gu_s,
                           const void *dn_q, const float *dn_s, const int *sel, const float *w,
                           int K, int I, int D);
/* lag_cuda_moe_group (:70): acc[S,D] = rank-order sum over the packed groups */
int    lag_hip_moe_group(float *acc, const float *x, const void *gu_q, const float *gu_s,
                         const void *dn_q, const float *dn_s, const int *gexp, const int *gbeg,
                         const int *gcnt, int G, const int *grow, const int *rowof, const float *w,
                         int S, int K, int I, int D);

/* lag_cuda_matmul_q8 (:36): int8 weights [O,I] followed in the same buffer by
 * their f32 row scales [O] (c/backend_cuda_laguna.cu:125-126) */
int    lag_hip_matmul_q8(float *y, const float *x, const void *W, int S, int I, int O);
/* ink_cuda_matmul_q8 (c/backend_cuda_ink.h:27-28): the same with the scales in
 * their own buffer */
int    lag_hip_matmul_q8_s(float *y, const float *x, const void *q8, const void *scale, int S, int I, int O);
/* ink_cuda_matmul_bf16 (c/backend_cuda_ink.h:17-18): activations rounded to bf16
 * (c/backend_cuda_ink.cu:63-64), in the lane order of the CPU's matmul_h
 * (c/moe_matmul.h:66-89, vdpbf16ps); I % 32 != 0 takes the f32-activation
 * contract, as the CPU does */
int    lag_hip_matmul_bf16_rx(float *y, const float *x, const void *W, int S, int I, int O);
/* Numerics of the host-activation matmuls: every call, whatever its row count,
 * reproduces the reference CPU's SIMD contracts bit for bit -- matmul_bf16 the
 * 16 f32-activation lanes of c/moe_matmul.h:92-110, matmul_q4 (per-row scales)
 * matmul_q4_k's F32 lanes (c/moe_quant.h:85-109), matmul_q8 matmul_q8_k's F32
 * lanes (c/moe_quant.h:378-391), matmul_bf16_rx the vdpbf16ps lanes -- so a
 * token's result does not depend on how many rows share its call. */

/* ---------------- 2. group-scaled int4 forms (scale[o*ng + g], ng = I/gs) ---------------- */
int    lag_hip_matmul_q4_g(float *y, const float *x, const void *packed, const void *scale,
                           int S, int I, int O, int gs);
int    lag_hip_expert_q4_g(float *out, const float *x, const void *p13, const void *s13,
                           const void *p2, const void *s2, int I, int D, int gs);
int    lag_hip_moe_experts_g(float *out, const float *x, const void *gu_q, const float *gu_s,
                             const void *dn_q, const float *dn_s, const int *sel, const float *w,
                             int K, int I, int D, int gs);
int    lag_hip_moe_group_g(float *acc, const float *x, const void *gu_q, const float *gu_s,
                           const void *dn_q, const float *dn_s, const int *gexp, const int *gbeg,
                           const int *gcnt, int G, const int *grow, const int *rowof, const float *w,
                           int S, int K, int I, int D, int gs);

/* ---------------- 3. device-resident MoE block ---------------- */
enum { LAG_HIP_ROUTE_SIGMOID = 0, LAG_HIP_ROUTE_SOFTMAX = 1, LAG_HIP_ROUTE_SOFTPLUS = 2,
       LAG_HIP_ROUTE_SOFTMAX_OLMOE = 3, LAG_HIP_ROUTE_SOFTMAX_QWEN = 4, LAG_HIP_ROUTE_SQRT_SOFTPLUS = 5,
       LAG_HIP_ROUTE_INKLING = 6 };
enum { LAG_HIP_SHARED_NONE = 0, LAG_HIP_SHARED_UNSCALED = 1, LAG_HIP_SHARED_GATED = 3 };

/* MoeDesc (c/moe_arch.h:33-41) plus the layer shape.  route_act: SIGMOID and
 * SOFTMAX are moe_block's (c/moe_block.h:24-26); the others are extensions:
 * SOFTPLUS x > 20 ? x : log1pf(expf(x)) (c/moe_math.h:54); SOFTMAX_OLMOE the
 * OLMoE engine's routing (float-sum softmax, each probability divided by the
 * sum, c/olmoe.c:212-216, 607-632; norm_topk as moe_block's); SOFTMAX_QWEN
 * qwen35's moe_route (double-sum softmax, (float)(p / sum) in double, the
 * picks always renormalised in double, c/qwen35.c:558-589; norm_topk and the
 * correction bias unused); SQRT_SOFTPLUS sqrtf(softplusf(x)), DeepSeek-V4's
 * router score (c/deepseek.c:854), selected and weighted as moe_block's
 * sigmoid scores; INKLING the Inkling engine's moe() routing (c/inkling.c:
 * 1027-1043): a router of n_experts + n_shared rows, the routed sigmoids
 * selected by moe_topk with the correction bias, weights the sigmoids of the
 * K picks and of the n_shared shared gates, each * route_scale / (their float
 * sum), route_scale being the engine's route_scale * gate.global_scale formed
 * in float (norm_topk unused; the routed sum is not scaled again).  The
 * reference wires shared NONE and UNSCALED; GATED (moe_arch.h's
 * MOE_SHARED_GATED, with INKLING only) adds n_shared shared experts after the
 * routed ranks, each output times its gate's weight (c/inkling.c:1166-1183),
 * their matmuls in inkling's matmul_h contract (bf16 weights, bf16-rounded
 * activations): sg and su [n_shared*Is, D], sd [n_shared*D, Is]. */
typedef struct {
    int   n_experts, topk, route_act, use_corr_bias, norm_topk;
    float route_scale;
    int   shared_mode;
    int   hidden, moe_inter, shared_inter, gs;   /* D, I, Is; gs = 0: per-row int4 scale */
    int   router_bf16;                           /* router element type: 1 bf16, 0 f32 */
    int   n_shared;                              /* INKLING: shared gate rows / GATED experts (else 0) */
} LagHipMoeDesc;

/* Device pointers of one layer.  Experts in the reference container layout
 * (c/laguna.c:586-588; docs/laguna.md:34-44); router from lag_hip_router_upload. */
typedef struct {
    const void  *router;
    const float *corr_bias;     /* [E] e_score_correction_bias (selection only) or NULL */
    const float *logit_bias;    /* [E] added to the router logits (a router-hook wrapper) or NULL */
    const void  *gu_q;
    const float *gu_s;
    const void  *dn_q;
    const float *dn_s;
    const void  *sg, *su, *sd;  /* bf16 shared expert [Is,D],[Is,D],[D,Is] or NULL */
} LagHipMoeWeights;

/* Upload a router [E,D] (bf16 or f32, host) into the order the routing
 * kernel streams, in its own element type: experts in groups of 4
 * (E4 = 4*ceil(E/4), the padding experts zero), each group a run of 1 KB
 * slices, slice q holding the next P elements (P = 8 bf16 or 4 f32) of each
 * of its 64 chains c = 16*(e%4) + i%16 (chain element m = i/16):
 * element (e, i) at ((e/4 * D/(16P) + m/P) * 64 + c) * P + m%P.
 * NULL = error.  Free with lag_hip_free. */
void  *lag_hip_router_upload(const void *W, int E, int D, int w_bf16);
/* the same transform from a device router W [E,D] into device Wc
 * (E4*D elements) (0 = ok) */
int    lag_hip_router_chain(const void *W, void *Wc, int E, int D, int w_bf16);
/* out[S,D] += MoE(x[S,D]) for S tokens (device pointers), queued on the
 * backend stream; S == 1 runs the per-token path, S > 1 the grouped path
 * (bit-identical per token).  0 = ok. */
int    lag_hip_moe_forward(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out, int S);
/* lag_hip_moe_forward without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The scratch of the forward lives in a static device array of
 * LAG_HIP_NOALLOC_SCRATCH_BYTES on each device (held from library load until
 * the process ends) instead of the growing arena; the call makes no
 * hipMalloc/hipFree and no other allocation.  A shape whose scratch does not
 * fit returns -1 before any launch (lag_hip_last_error gives the bytes it
 * needed): the C2 layer (D=4096, E=256, K=10, I=Is=1024) fits up to S = 78
 * (up to S = 66 with lag_hip_set_q4_mode(1) on per-row scales, which also
 * keeps int8 activations and an f32 h).
 * Same results, bit for bit, as lag_hip_moe_forward.  Every call on a device
 * shares that device's array, so calls that overlap on one device race. */
#define LAG_HIP_NOALLOC_SCRATCH_BYTES ((size_t)24 << 20)
int    lag_hip_moe_forward_noalloc(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out, int S);
/* The device scratch bytes lag_hip_moe_forward(_noalloc) needs for S tokens of
 * this layer in the current q4 mode (0 = unsupported descriptor or shape).
 * Host arithmetic only: callable before lag_hip_init and without a device, so a
 * caller can size its batches to the fixed region above. */
size_t lag_hip_moe_forward_scratch_bytes(const LagHipMoeDesc *d, const LagHipMoeWeights *w, int S);
/* the same with host x/out; synchronous */
int    lag_hip_moe_block(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out, int S);
/* routing only (device pointers): logits [S,E] (may be NULL), sel [S,K], w [S,K];
 * INKLING: logits [S, E + n_shared], w [S, K + n_shared] (the picks' weights,
 * then the shared gates') */
int    lag_hip_route(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, int S,
                     float *logits, int *sel, float *wts);
/* last routing's expert groups (device pointers of the backend's scratch;
 * valid until the next forward): G (host out), gexp/gbeg/gcnt [G] host copies */
int    lag_hip_last_groups(int *G, int *gexp, int *gbeg, int *gcnt, int cap);

/* ---------------- stack glue (device pointers, queued on the backend stream) ----------------
 * A layer of a stack is h += MoE(rmsnorm(h, w_l)) (lag_hip_rmsnorm, then
 * lag_hip_moe_forward with x = the normed rows and out = h); a step ends in
 * rmsnorm, the head and a greedy pick. */
/* out[s] = x[s] / sqrt(mean(x[s]^2) + eps) * w, the squares summed in double
 * (rmsnorm_row, c/moe_math.h:58-62); out may be x.  0 = ok */
int    lag_hip_rmsnorm(const float *x, const float *w, float *out, int S, int D, float eps);
/* One stack layer in one call: xn = rmsnorm(h, norm_w, eps) as lag_hip_rmsnorm (the
 * same bits), then h += MoE(xn) as lag_hip_moe_forward.  No counterpart in the
 * reference (c/laguna.c:1156-1160 calls rmsnorm_row and the block separately); for
 * stack callers: without a shared expert and below 512 tokens the routing launch
 * applies the norm as it stages the rows, one launch fewer per layer.  0 = ok */
int    lag_hip_moe_forward_rmsnorm(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *norm_w, float eps,
                                   float *xn, float *h, int S);
/* logits[S,V] = x[S,D] . head^T under the 16-lane contract of the head's
 * resmm -> matmul_bf16 (c/laguna.c:1156-1158; Wc from lag_hip_router_upload
 * of the [V,D] head), and with tok non-null tok[s] = the greedy pick of
 * argmax_logits (strict ascending scan: ties to the lowest index,
 * c/laguna.c:1159).  0 = ok */
int    lag_hip_head_argmax(const void *Wc, int w_bf16, const float *x, int S, int D, int V, float *logits, int *tok);
/* tok[s] = argmax_logits' pick over logits[s, 0..V) alone (c/laguna.c:1159).  0 = ok */
int    lag_hip_argmax(const float *logits, int S, int V, int *tok);

/* ---------------- memory, stream, timing ---------------- */
void  *lag_hip_alloc(size_t n);
int    lag_hip_h2d(void *dst, const void *src, size_t n);
int    lag_hip_d2h(void *dst, const void *src, size_t n);
int    lag_hip_d2d(void *dst, const void *src, size_t n);   /* async on the backend stream */
int    lag_hip_memset(void *dst, int v, size_t n);
int    lag_hip_sync(void);
void  *lag_hip_event_create(void);
int    lag_hip_event_record(void *ev);
float  lag_hip_event_elapsed_ms(void *start, void *end);
void   lag_hip_event_destroy(void *ev);

/* ---------------- graphs ----------------
 * Record the device-pointer entries (lag_hip_moe_forward, lag_hip_route,
 * lag_hip_d2d) issued between begin and end into one graph, replayed with a
 * single submission by lag_hip_graph_launch (async on the backend stream).
 * Pointers and shapes are fixed at recording; scratch must already be large
 * enough (issue the same shapes once first), else the entry fails.  A
 * finished recording owns the backend scratch it was recorded over until
 * lag_hip_graph_destroy (which waits for the stream, then frees it); later
 * calls of any size allocate their own, so they never disturb a live graph.
 * A recording begun right after another one gets fresh scratch of the same
 * capacity, so same-shaped graphs can be recorded back to back.  A destroy
 * issued while a recording is open takes effect when that recording ends.
 * No counterpart in the reference (its decode loop launches per layer): this
 * is the launch-overhead-free way to drive a decode step. */
int    lag_hip_graph_begin(void);
void  *lag_hip_graph_end(void);          /* NULL on failure */
int    lag_hip_graph_launch(void *g);
void   lag_hip_graph_destroy(void *g);

/* Kernel choice for the grouped expert GEMMs of lag_hip_moe_forward with
 * S > 1: 0 auto (the f16 MFMA when the batch's groups average >= 6.5 tokens,
 * else dot8), 1 dot8, 2 f16 MFMA.  Both give the same bits.  Returns the
 * previous mode, -1 for a bad one.  No counterpart in the reference (one
 * grouped kernel there, c/backend_cuda.cu:618-700): a tuning switch. */
int    lag_hip_set_grouped_kernel(int mode);

/* The int4 activation contract of lag_hip_moe_forward / lag_hip_moe_block for
 * per-row scales (gs == 0): 0 (default) this build's exact-integer digits,
 * 1 the reference's IDOT contract -- activations to int8 per 32-block
 * (amax/127, lrintf), exact int8 x int4 block dots, acc = fma(s_b, dot_b, acc)
 * in block order, x row scale (c/moe_quant.h:48-82, 141-182) -- which gives
 * the bits of the CPU tier under LAG_IDOT=1 (c/laguna.c:204-207).  Returns
 * the previous mode, -1 for a bad one; descriptors with gs > 0 ignore it (the
 * reference's grouped kernel has no IDOT form, c/quant.h:168-203). */
int    lag_hip_set_q4_mode(int mode);

/* per-kernel timing with events on the backend stream (the analogue of the
 * reference's COLI_CUDA_PROFILE=1, c/backend_cuda.cu:822-940) */
int    lag_hip_profile(int enable);
int    lag_hip_profile_count(void);
int    lag_hip_profile_read(int idx, char *name, int cap, double *total_ms, long long *launches);
void   lag_hip_profile_reset(void);

/* ---------------- synthetic data (bit-identical to the host generator) ---------------- */
int    lag_hip_gen_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, double sigma, int to_bf16);
int    lag_hip_gen_bf16(uint16_t *out, int64_t n, uint64_t seed, uint64_t offset, double sigma);
int    lag_hip_gen_q4(uint8_t *q, float *s, uint64_t seed, double sigma, int64_t row0, int64_t nrows, int K, int gs);

/* ---------------- diagnostics ---------------- */
/* MFMA lane-layout probes (f16, bf16, int8) + libm evaluation on n host
 * inputs; out_host gets 768 + 3n floats (layout in k_route.hip).  0 = ran */
int    lag_hip_selftest(float *out_host, const float *xin_host, int n);
const char *lag_hip_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
