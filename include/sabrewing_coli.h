/* sabrewing_coli.h -- the GLM engine's coli_cuda_* table on gfx950 (libsabrewing_hip.so).
 *
 * One entry per slot of c/backend_cuda.h:28-169, same arguments, same return
 * convention: 1 ok / 0 fail (NULL / -1 / nothing for the slots that return
 * pointers, ids or void).  A 0 is the reference's "unavailable" answer: the
 * engine keeps that call on the CPU (c/colibri.c:3586-3600).  The loader
 * (include/sabrewing_loader.h) exports these under their coli_cuda_* names.
 *
 * MoE slots are implemented: device contexts, int4 tensors (fmt 2 per-row,
 * fmt 4 group-scaled), matmul / pipe_gemm, the fused expert MLPs, the expert
 * group (sync, issue/take, resident issue/take), the device router, and the
 * pipe data plane (scratch, alloc, copies, add, rows_add, silu_mul).  Slots of
 * the engine's attention and norm/RoPE stages (outside the MoE block) resolve
 * and return 0, as the reference allows for a backend without them.
 *
 * Numerics: the int4 projections are the exact-integer dot8 contract of the
 * lag family (sabrewing_hip.h), so a coli expert's output equals the same
 * expert's lag_hip_expert_q4 output bit for bit.  The router reproduces the
 * CPU engine's routing (c/colibri.c:2871-2999 with c/quant.h:98-102) bit for
 * bit: a sequential fma chain per expert, glibc-exact expf, strict-greater
 * selection with the CPU's non-finite fallback.
 *
 * Threads: entries on different devices may run concurrently (as the engine's
 * per-device omp loop does, c/colibri.c:3577); entries on one device are
 * serialised by that device's mutex.
 */
#ifndef SABREWING_COLI_H
#define SABREWING_COLI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define COLI_HIP_MAX_DEVICES 16

/* opaque resident tensor (ColiCudaTensor, c/backend_cuda.h:25) */
typedef struct ColiHipTensor ColiHipTensor;

/* c/backend_cuda.h:28-35: contexts for the listed device ordinals (distinct, in
 * range); 1 ok.  mem_info/stats/group_stats as the reference. */
int coli_hip_init(const int *devices, int count);
void coli_hip_shutdown(void);
int coli_hip_device_count(void);
int coli_hip_device_at(int index);
int coli_hip_mem_info(int device, size_t *free_bytes, size_t *total_bytes);
void coli_hip_stats(int device, size_t *tensor_count, size_t *tensor_bytes);
void coli_hip_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows,
                          double *h2d_ms, double *kernel_ms, double *d2h_ms);

/* c/backend_cuda.h:38-43 (c/backend_cuda.cu:607-663): upload W[O][I] and its
 * scales.  fmt 2: packed int4 (low nibble = even input, offset 8), scales[O];
 * fmt 4: the same bytes with scales[O][I/gs].  The bytes stay as stored.
 * Returns 0 for the other formats and for shapes the gfx950 kernels do not
 * take (I a multiple of 32, I <= 8192; gs a power of two >= 32 dividing I),
 * so the engine keeps such a tensor on the CPU from the start.  A non-NULL
 * *tensor is a cached copy: 1 when its (fmt, I, O, device, gs) match. */
int coli_hip_tensor_upload_g(ColiHipTensor **tensor, const void *weights, const float *scales,
                             int fmt, int I, int O, int device, int gs);
int coli_hip_tensor_upload(ColiHipTensor **tensor, const void *weights, const float *scales,
                           int fmt, int I, int O, int device);

/* c/backend_cuda.h:45-55: y[S,O] = x[S,I] . W^T (host x, y), uploading W on
 * first use.  fmt 4 needs gs > 0. */
int coli_hip_matmul(ColiHipTensor **tensor, float *y, const float *x, const void *weights,
                    const float *scales, int fmt, int S, int I, int O, int device, int gs);

/* c/backend_cuda.h:57-60: y = down(silu(gate . x) * up . x) for S host rows */
int coli_hip_expert_mlp(ColiHipTensor *gate, ColiHipTensor *up, ColiHipTensor *down,
                        float *y, const float *x, int S);
/* c/backend_cuda.h:62-68: the shared-expert MLP (fmt 2 tensors only, as the
 * reference's W4A16 entry); the same kernels and numerics as expert_mlp */
int coli_hip_shared_mlp_w4a16(ColiHipTensor *gate, ColiHipTensor *up, ColiHipTensor *down,
                              float *y, const float *x, int S);

/* c/backend_cuda.h:70-86: count <= 64 experts of one device, rows[c] >= 1 host
 * rows each, concatenated in call order in x [sum rows][D] and y [sum rows][D].
 * issue/take: the same computation, launched and returned at once (sum rows
 * <= 8, one outstanding issue per device); take waits and returns the rows in
 * a pinned buffer valid until the next issue on that device, or NULL. */
int coli_hip_expert_group_issue(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                ColiHipTensor *const *downs, const int *rows, int count, const float *x);
const float *coli_hip_expert_group_take(int device);
int coli_hip_expert_group(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                          ColiHipTensor *const *downs, const int *rows, int count, float *y, const float *x);

/* c/backend_cuda.h:88-111, 147-162: MLA attention -- not on this backend (0) */
int coli_hip_attention_absorb(ColiHipTensor *kv_b, float *ctx, const float *q, const float *latent,
                              const float *rope, int H, int Q, int R, int V, int K, int T, float attention_scale);
int coli_hip_attention_absorb_batch(ColiHipTensor *kv_b, float *ctx, const float *q, const float *latent,
                                    const float *rope, int S, int H, int Q, int R, int V, int K, int T,
                                    float attention_scale);
int coli_hip_attention_project_batch(ColiHipTensor *kv_b, ColiHipTensor *o_proj, float *out, const float *q,
                                     const float *latent, const float *rope, int S, int H, int Q, int R, int V,
                                     int K, int T, float attention_scale);
int coli_hip_attention_project_ragged(ColiHipTensor *kv_b, ColiHipTensor *o_proj, float *out, const float *q,
                                      const void *const *keys, const float *const *latent,
                                      const float *const *rope, const int *lengths, int S, int H, int Q, int R,
                                      int V, int K, int max_t, float attention_scale);
int coli_hip_attention_project_batch_dev(ColiHipTensor *kv_b, ColiHipTensor *o_proj, float *out,
                                         const float *q_dev, const float *latent_dev, const float *rope_dev,
                                         int S, int H, int Q, int R, int V, int K, int T, float scale);
int coli_hip_attention_absorb_batch_dev(ColiHipTensor *kv_b_shard, float *ctx_dev, const float *q_dev,
                                        const float *latent_dev, const float *rope_dev, int S, int H, int Q,
                                        int R, int V, int K, int T, float scale);
int coli_hip_attention_absorb_kvdev(ColiHipTensor *kv_b, float *ctx, const float *q, const float *latent_dev,
                                    const float *rope_dev, int H, int Q, int R, int V, int K, int T, float scale);
int coli_hip_attention_project_batch_dev_out(ColiHipTensor *kv_b, ColiHipTensor *o_proj, float *out_dev,
                                             const float *q_dev, const float *latent_dev, const float *rope_dev,
                                             int S, int H, int Q, int R, int V, int K, int T, float scale);

/* c/backend_cuda.h:113-120 */
void coli_hip_tensor_free(ColiHipTensor *tensor);
size_t coli_hip_tensor_bytes(const ColiHipTensor *tensor);
int coli_hip_tensor_device(const ColiHipTensor *tensor);
int coli_hip_tensor_update(ColiHipTensor *tensor, const void *weights, const float *scales);

/* c/backend_cuda.h:122-146, 163-164: device-pointer data plane.  Every pipe
 * entry of a device is ordered on that device's stream; upload, download and
 * peer_copy return when the copy is done.  pipe_scratch: slot 0..26, grow-only
 * (a grown slot's earlier pointer is gone).  rmsnorm and RoPE (attention
 * stages) return 0. */
float *coli_hip_pipe_scratch(int device, int slot, size_t bytes);
void *coli_hip_pipe_alloc(int device, size_t bytes);
void coli_hip_pipe_free(int device, void *p);
int coli_hip_pipe_upload(int device, void *dst, const void *src, size_t bytes);
int coli_hip_pipe_download(int device, const void *src, void *dst, size_t bytes);
int coli_hip_pipe_rmsnorm(int device, float *y_dev, const float *x_dev, const float *w_dev, int S, int D, float eps);
int coli_hip_pipe_rope(int device, float *v_dev, const int *pos_dev, int rows, int stride, int offset, int R,
                       int heads, float theta);
int coli_hip_pipe_silu_mul(int device, float *gate_dev, const float *up_dev, size_t n);
int coli_hip_pipe_add(int device, float *x_dev, const float *t_dev, size_t n);
int coli_hip_pipe_rows_add(int device, float *x_dev, const float *partial_dev, const int *rows_dev, int nrows, int D);
int coli_hip_pipe_gemm(ColiHipTensor *t, float *y_dev, const float *x_dev, int S);
int coli_hip_pipe_rmsnorm_s(int device, float *y_dev, const float *x_dev, const float *w_dev, int S, int D, float eps,
                            int xstride, int ystride);
int coli_hip_pipe_rope_base(int device, float *v_dev, int pos_base, int rows, int stride, int offset, int R,
                            int heads, float theta);
int coli_hip_pipe_copy2d(int device, float *dst, int dpitch, const float *src, int spitch, int width, int height);
int coli_hip_pipe_peer_copy(int dst_dev, float *dst, int src_dev, const float *src, size_t bytes);
int coli_hip_pipe_sync(int device);

/* c/backend_cuda.h:150-152 (c/backend_cuda.cu:1401-1479): count <= 64 experts of
 * one row x_src_dev (on home_device); partial_slot_dev[D] (on home_device) <-
 * sum_c weights[c] * expert_c(x) in c order, one fma per expert.  Per-row int4
 * (fmt 2) only, as the reference.  take: acc_dev[D] = sum of the n_issued slots
 * in issue order, after every issuing device's work. */
int coli_hip_expert_group_resident_issue(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                         ColiHipTensor *const *downs, const float *weights, int count,
                                         int home_device, const float *x_src_dev, float *partial_slot_dev);
int coli_hip_expert_group_resident_take(int home_device, const int *devices, int n_issued, float *slots_dev,
                                        float *acc_dev, int D);

/* c/backend_cuda.h:153-156 (c/backend_cuda.cu:1350-1378): one decode row's
 * routing on the device.  x_dev[D], rw_dev f32 [E][D], rb_dev f32 [E];
 * logit = sigmoid(x . w_e), selection by logit + bias (Ksel passes, strict >,
 * lowest id), top-p truncation (0 < topp < 1), norm_topk, routed_scale.
 * idx_host[Ksel], w_host[Ksel], *keff_host: the kept count.  E <= 4096,
 * Ksel <= 64. */
int coli_hip_pipe_router(int device, const float *x_dev, const void *rw_dev, const void *rb_dev, int D, int E,
                         int Ksel, float topp, int norm_topk, float routed_scale, int *idx_host, float *w_host,
                         int *keff_host);

#ifdef __cplusplus
}
#endif
#endif
