/* sabrewing_loader.h -- the Linux runtime seam between an unmodified
 * sabrewing engine and the gfx950 backend.
 *
 * libsabrewing_loader.so exports the reference's Laguna backend ABI under its
 * own names (the declarations of c/backend_cuda_laguna.h:25-95, same
 * signatures and 0 / -1 returns), and the GLM engine's coli_cuda_* table
 * below.  Each wrapper forwards through a function table resolved from libsabrewing_hip.so at first use, with the semantics of
 * the reference's Windows DLL loader (c/backend_loader.c:99-253): the library
 * is opened by absolute path only (next to the loader, or $SABREWING_HIP_LIB),
 * every table slot must resolve or the library is unloaded again, and while
 * the backend is unavailable every wrapper returns the "not initialised"
 * value (-1 / NULL / 0), so the engine keeps its CPU path.  Entries with no
 * MI355X counterpart (the fp4 experts) always return -1.  The Inkling
 * engine's ink_cuda_* table (c/backend_cuda_ink.h:14-34) is exported too, with
 * its own all-or-nothing resolution.
 * An engine links this object in place of backend_cuda_laguna.o (or
 * backend_cuda_ink.o). */
#ifndef SABREWING_LOADER_H
#define SABREWING_LOADER_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

int    lag_cuda_init(int dev);
size_t lag_cuda_free_bytes(void);
size_t lag_cuda_total_bytes(void);
void  *lag_cuda_upload(const void *h, size_t n);
void   lag_cuda_free(void *d);
int    lag_cuda_matmul_bf16(float *y, const float *x, const void *W, int S, int I, int O);
int    lag_cuda_matmul_q8(float *y, const float *x, const void *W, int S, int I, int O);
int    lag_cuda_matmul_q4(float *y, const float *x, const void *packed, const void *scale, int S, int I, int O);
int    lag_cuda_expert_q4(float *out, const float *x, const void *p13, const void *s13,
                          const void *p2, const void *s2, int I, int D);
int    lag_cuda_moe_experts(float *out, const float *x, const void *gu_q, const float *gu_s,
                            const void *dn_q, const float *dn_s, const int *sel, const float *w, int K, int I, int D);
int    lag_cuda_moe_group(float *acc, const float *x, const void *gu_q, const float *gu_s,
                          const void *dn_q, const float *dn_s, const int *gexp, const int *gbeg, const int *gcnt,
                          int G, const int *grow, const int *rowof, const float *w, int S, int K, int I, int D);
int    lag_cuda_matmul_fp4(float *y, const float *x, const void *packed, const void *es, int S, int I, int O);
int    lag_cuda_moe_experts_fp4(float *out, const float *x, const void *gu_q, const void *gu_es,
                                const void *dn_q, const void *dn_es, const int *sel, const float *w, int K,
                                int I, int D, float limit);

/* The Inkling engine's table (c/backend_cuda_ink.h:14-34, 0 ok / -1 fail), each
 * slot forwarded to its lag_hip_* entry: init, memory and upload as the lag
 * family's; matmul_bf16 rounds the activations to bf16 (c/backend_cuda_ink.cu:63-64)
 * -- lag_hip_matmul_bf16_rx, the CPU's matmul_h lane order; matmul_q4 and
 * expert_q4 the lag family's per-row int4; matmul_q8 int8 weights with their
 * row scales in a separate buffer (lag_hip_matmul_q8_s). */
int    ink_cuda_init(int dev);
size_t ink_cuda_free_bytes(void);
size_t ink_cuda_total_bytes(void);
void  *ink_cuda_upload(const void *h, size_t n);
int    ink_cuda_matmul_bf16(float *y, const float *x, const void *W, int S, int I, int O);
int    ink_cuda_matmul_q4(float *y, const float *x, const void *packed, const void *scale, int S, int I, int O);
int    ink_cuda_matmul_q8(float *y, const float *x, const void *q8, const void *scale, int S, int I, int O);
int    ink_cuda_expert_q4(float *out, const float *x, const void *p13, const void *s13,
                          const void *p2, const void *s2, int I, int D);

/* The GLM engine's table (c/backend_cuda.h:28-169, 1 ok / 0 fail), the slots of
 * the reference's Windows loader (c/backend_loader.c:99-150), each forwarded to
 * its coli_hip_* entry (include/sabrewing_coli.h).  Its own all-or-nothing
 * resolution: while unavailable every wrapper returns 0 / NULL / -1 or nothing. */
typedef struct ColiCudaTensor ColiCudaTensor;
int coli_cuda_init(const int *devices, int count);
void coli_cuda_shutdown(void);
int coli_cuda_device_count(void);
int coli_cuda_device_at(int index);
int coli_cuda_mem_info(int device, size_t *free_bytes, size_t *total_bytes);
void coli_cuda_stats(int device, size_t *tensor_count, size_t *tensor_bytes);
void coli_cuda_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows, double *h2d_ms, double *kernel_ms, double *d2h_ms);
int coli_cuda_tensor_upload_g(ColiCudaTensor **tensor, const void *weights, const float *scales, int fmt, int I, int O, int device, int gs);
int coli_cuda_tensor_upload(ColiCudaTensor **tensor, const void *weights, const float *scales, int fmt, int I, int O, int device);
int coli_cuda_matmul(ColiCudaTensor **tensor, float *y, const float *x, const void *weights, const float *scales, int fmt, int S, int I, int O, int device, int gs);
int coli_cuda_expert_mlp(ColiCudaTensor *gate, ColiCudaTensor *up, ColiCudaTensor *down, float *y, const float *x, int S);
int coli_cuda_shared_mlp_w4a16(ColiCudaTensor *gate, ColiCudaTensor *up, ColiCudaTensor *down, float *y, const float *x, int S);
int coli_cuda_expert_group_issue(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups, ColiCudaTensor *const *downs, const int *rows, int count, const float *x);
const float *coli_cuda_expert_group_take(int device);
int coli_cuda_expert_group(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups, ColiCudaTensor *const *downs, const int *rows, int count, float *y, const float *x);
int coli_cuda_attention_absorb(ColiCudaTensor *kv_b, float *ctx, const float *q, const float *latent, const float *rope, int H, int Q, int R, int V, int K, int T, float attention_scale);
int coli_cuda_attention_absorb_batch(ColiCudaTensor *kv_b, float *ctx, const float *q, const float *latent, const float *rope, int S, int H, int Q, int R, int V, int K, int T, float attention_scale);
int coli_cuda_attention_project_batch(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out, const float *q, const float *latent, const float *rope, int S, int H, int Q, int R, int V, int K, int T, float attention_scale);
int coli_cuda_attention_project_ragged(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out, const float *q, const void *const *keys, const float *const *latent, const float *const *rope, const int *lengths, int S, int H, int Q, int R, int V, int K, int max_t, float attention_scale);
int coli_cuda_attention_project_batch_dev(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out, const float *q_dev, const float *latent_dev, const float *rope_dev, int S, int H, int Q, int R, int V, int K, int T, float scale);
int coli_cuda_attention_absorb_batch_dev(ColiCudaTensor *kv_b_shard, float *ctx_dev, const float *q_dev, const float *latent_dev, const float *rope_dev, int S, int H, int Q, int R, int V, int K, int T, float scale);
int coli_cuda_attention_absorb_kvdev(ColiCudaTensor *kv_b, float *ctx, const float *q, const float *latent_dev, const float *rope_dev, int H, int Q, int R, int V, int K, int T, float scale);
int coli_cuda_attention_project_batch_dev_out(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out_dev, const float *q_dev, const float *latent_dev, const float *rope_dev, int S, int H, int Q, int R, int V, int K, int T, float scale);
void coli_cuda_tensor_free(ColiCudaTensor *tensor);
size_t coli_cuda_tensor_bytes(const ColiCudaTensor *tensor);
int coli_cuda_tensor_device(const ColiCudaTensor *tensor);
int coli_cuda_tensor_update(ColiCudaTensor *tensor, const void *weights, const float *scales);
float *coli_cuda_pipe_scratch(int device, int slot, size_t bytes);
void *coli_cuda_pipe_alloc(int device, size_t bytes);
void coli_cuda_pipe_free(int device, void *p);
int coli_cuda_pipe_upload(int device, void *dst, const void *src, size_t bytes);
int coli_cuda_pipe_download(int device, const void *src, void *dst, size_t bytes);
int coli_cuda_pipe_rmsnorm(int device, float *y_dev, const float *x_dev, const float *w_dev, int S, int D, float eps);
int coli_cuda_pipe_rope(int device, float *v_dev, const int *pos_dev, int rows, int stride, int offset, int R, int heads, float theta);
int coli_cuda_pipe_silu_mul(int device, float *gate_dev, const float *up_dev, size_t n);
int coli_cuda_pipe_add(int device, float *x_dev, const float *t_dev, size_t n);
int coli_cuda_pipe_rows_add(int device, float *x_dev, const float *partial_dev, const int *rows_dev, int nrows, int D);
int coli_cuda_pipe_gemm(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S);
int coli_cuda_pipe_rmsnorm_s(int device, float *y_dev, const float *x_dev, const float *w_dev, int S, int D, float eps, int xstride, int ystride);
int coli_cuda_pipe_rope_base(int device, float *v_dev, int pos_base, int rows, int stride, int offset, int R, int heads, float theta);
int coli_cuda_pipe_copy2d(int device, float *dst, int dpitch, const float *src, int spitch, int width, int height);
int coli_cuda_pipe_peer_copy(int dst_dev, float *dst, int src_dev, const float *src, size_t bytes);
int coli_cuda_pipe_sync(int device);
int coli_cuda_expert_group_resident_issue(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups, ColiCudaTensor *const *downs, const float *weights, int count, int home_device, const float *x_src_dev, float *partial_slot_dev);
int coli_cuda_expert_group_resident_take(int home_device, const int *devices, int n_issued, float *slots_dev, float *acc_dev, int D);
int coli_cuda_pipe_router(int device, const float *x_dev, const void *rw_dev, const void *rb_dev, int D, int E, int Ksel, float topp, int norm_topk, float routed_scale, int *idx_host, float *w_host, int *keff_host);

/* 1 when the backend library loaded and every lag slot resolved (loads on first call) */
int    sabrewing_loader_available(void);
/* the same for the coli slots */
int    sabrewing_loader_coli_available(void);
/* the same for the ink slots */
int    sabrewing_loader_ink_available(void);
/* the absolute path tried (or "" before the first attempt) */
const char *sabrewing_loader_path(void);

#ifdef __cplusplus
}
#endif
#endif
