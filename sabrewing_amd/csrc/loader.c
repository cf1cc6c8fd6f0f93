/* loader.c -- Linux dlopen loader: the reference's lag_cuda_* and coli_cuda_* ABIs
 * forwarded to libsabrewing_hip.so's lag_hip_* and coli_hip_* entries
 * (include/sabrewing_loader.h).
 *
 * Same rules as the reference's Windows loader (c/backend_loader.c): one load
 * attempt, absolute path only (no search path, no current directory), all
 * symbols or none, and "not initialised" sentinels while unavailable. */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "../../include/sabrewing_loader.h"
#include "../../include/sabrewing_coli.h"

typedef int (*fn_init)(int);
typedef size_t (*fn_bytes)(void);
typedef void *(*fn_upload)(const void *, size_t);
typedef void (*fn_free)(void *);
typedef int (*fn_mm_bf16)(float *, const float *, const void *, int, int, int);
typedef int (*fn_mm_q4)(float *, const float *, const void *, const void *, int, int, int);
typedef int (*fn_expert)(float *, const float *, const void *, const void *, const void *, const void *, int, int);
typedef int (*fn_experts)(float *, const float *, const void *, const float *, const void *, const float *,
                          const int *, const float *, int, int, int);
typedef int (*fn_group)(float *, const float *, const void *, const float *, const void *, const float *,
                        const int *, const int *, const int *, int, const int *, const int *, const float *,
                        int, int, int, int);

static struct {
    int loaded, available;
    void *lib;
    char path[4096];
    fn_init init;
    fn_bytes free_bytes, total_bytes;
    fn_upload upload;
    fn_free free_;
    fn_mm_bf16 matmul_bf16;
    fn_mm_q4 matmul_q4;
    fn_mm_bf16 matmul_q8;
    fn_expert expert_q4;
    fn_experts moe_experts;
    fn_group moe_group;
} T;

static void resolve_path(void) {
    const char *env = getenv("SABREWING_HIP_LIB");
    if (env && env[0] == '/') { snprintf(T.path, sizeof T.path, "%s", env); return; }
    Dl_info info;
    if (dladdr((void *)&resolve_path, &info) && info.dli_fname && info.dli_fname[0] == '/') {
        snprintf(T.path, sizeof T.path, "%s", info.dli_fname);
        char *slash = strrchr(T.path, '/');
        if (slash) { slash[1] = 0; strncat(T.path, "libsabrewing_hip.so", sizeof T.path - strlen(T.path) - 1); return; }
    }
    T.path[0] = 0;
}

#define RESOLVE(field, name)                                       \
    do {                                                           \
        *(void **)(&T.field) = dlsym(T.lib, name);                 \
        if (!T.field) { missing = name; goto unload; }             \
    } while (0)

static void load_once(void) {
    if (T.loaded) return;
    T.loaded = 1;
    resolve_path();
    if (!T.path[0]) return;
    T.lib = dlopen(T.path, RTLD_NOW | RTLD_LOCAL);
    if (!T.lib) return;
    {
        const char *missing = NULL;
        RESOLVE(init, "lag_hip_init");
        RESOLVE(free_bytes, "lag_hip_free_bytes");
        RESOLVE(total_bytes, "lag_hip_total_bytes");
        RESOLVE(upload, "lag_hip_upload");
        RESOLVE(free_, "lag_hip_free");
        RESOLVE(matmul_bf16, "lag_hip_matmul_bf16");
        RESOLVE(matmul_q4, "lag_hip_matmul_q4");
        RESOLVE(matmul_q8, "lag_hip_matmul_q8");
        RESOLVE(expert_q4, "lag_hip_expert_q4");
        RESOLVE(moe_experts, "lag_hip_moe_experts");
        RESOLVE(moe_group, "lag_hip_moe_group");
        T.available = 1;
        return;
    unload:
        fprintf(stderr, "[sabrewing-loader] %s: missing symbol %s; backend unavailable\n", T.path, missing);
        dlclose(T.lib);
        memset(&T.init, 0, sizeof T - ((char *)&T.init - (char *)&T));
        T.lib = NULL;
    }
}

int sabrewing_loader_available(void) { load_once(); return T.available; }
const char *sabrewing_loader_path(void) { return T.path; }

int lag_cuda_init(int dev) { load_once(); return T.available ? T.init(dev) : -1; }
size_t lag_cuda_free_bytes(void) { load_once(); return T.available ? T.free_bytes() : 0; }
size_t lag_cuda_total_bytes(void) { load_once(); return T.available ? T.total_bytes() : 0; }
void *lag_cuda_upload(const void *h, size_t n) { load_once(); return T.available ? T.upload(h, n) : NULL; }
void lag_cuda_free(void *d) { load_once(); if (T.available) T.free_(d); }
int lag_cuda_matmul_bf16(float *y, const float *x, const void *W, int S, int I, int O) {
    load_once(); return T.available ? T.matmul_bf16(y, x, W, S, I, O) : -1;
}
int lag_cuda_matmul_q8(float *y, const float *x, const void *W, int S, int I, int O) {
    load_once(); return T.available ? T.matmul_q8(y, x, W, S, I, O) : -1;
}
int lag_cuda_matmul_q4(float *y, const float *x, const void *packed, const void *scale, int S, int I, int O) {
    load_once(); return T.available ? T.matmul_q4(y, x, packed, scale, S, I, O) : -1;
}
int lag_cuda_expert_q4(float *out, const float *x, const void *p13, const void *s13, const void *p2, const void *s2, int I, int D) {
    load_once(); return T.available ? T.expert_q4(out, x, p13, s13, p2, s2, I, D) : -1;
}
int lag_cuda_moe_experts(float *out, const float *x, const void *gu_q, const float *gu_s, const void *dn_q,
                         const float *dn_s, const int *sel, const float *w, int K, int I, int D) {
    load_once(); return T.available ? T.moe_experts(out, x, gu_q, gu_s, dn_q, dn_s, sel, w, K, I, D) : -1;
}
int lag_cuda_moe_group(float *acc, const float *x, const void *gu_q, const float *gu_s, const void *dn_q,
                       const float *dn_s, const int *gexp, const int *gbeg, const int *gcnt, int G, const int *grow,
                       const int *rowof, const float *w, int S, int K, int I, int D) {
    load_once();
    return T.available ? T.moe_group(acc, x, gu_q, gu_s, dn_q, dn_s, gexp, gbeg, gcnt, G, grow, rowof, w, S, K, I, D) : -1;
}
int lag_cuda_matmul_fp4(float *y, const float *x, const void *packed, const void *es, int S, int I, int O) {
    (void)y; (void)x; (void)packed; (void)es; (void)S; (void)I; (void)O; return -1;   /* fp4: CPU path */
}
int lag_cuda_moe_experts_fp4(float *out, const float *x, const void *gu_q, const void *gu_es, const void *dn_q,
                             const void *dn_es, const int *sel, const float *w, int K, int I, int D, float limit) {
    (void)out; (void)x; (void)gu_q; (void)gu_es; (void)dn_q; (void)dn_es; (void)sel; (void)w; (void)K; (void)I;
    (void)D; (void)limit; return -1;
}

/* ---- the Inkling family (c/backend_cuda_ink.h:14-34): its own table over the
 * same library, all of its eight slots or none; -1 / NULL / 0 while unavailable.
 * The same device and stream as the lag family (one backend per process). ---- */
typedef int (*fn_mm_q8s)(float *, const float *, const void *, const void *, int, int, int);
static struct {
    int loaded, available;
    void *lib;
    fn_init init;
    fn_bytes free_bytes, total_bytes;
    fn_upload upload;
    fn_mm_bf16 matmul_bf16_rx;
    fn_mm_q4 matmul_q4;
    fn_mm_q8s matmul_q8_s;
    fn_expert expert_q4;
} K;

#define RESOLVE_K(field, name)                                     \
    do {                                                           \
        *(void **)(&K.field) = dlsym(K.lib, name);                 \
        if (!K.field) { missing = name; goto unload; }             \
    } while (0)

static void ink_load_once(void) {
    if (K.loaded) return;
    K.loaded = 1;
    if (!T.path[0]) resolve_path();
    if (!T.path[0]) return;
    K.lib = dlopen(T.path, RTLD_NOW | RTLD_LOCAL);
    if (!K.lib) return;
    {
        const char *missing = NULL;
        RESOLVE_K(init, "lag_hip_init");
        RESOLVE_K(free_bytes, "lag_hip_free_bytes");
        RESOLVE_K(total_bytes, "lag_hip_total_bytes");
        RESOLVE_K(upload, "lag_hip_upload");
        RESOLVE_K(matmul_bf16_rx, "lag_hip_matmul_bf16_rx");
        RESOLVE_K(matmul_q4, "lag_hip_matmul_q4");
        RESOLVE_K(matmul_q8_s, "lag_hip_matmul_q8_s");
        RESOLVE_K(expert_q4, "lag_hip_expert_q4");
        K.available = 1;
        return;
    unload:
        fprintf(stderr, "[sabrewing-loader] %s: missing symbol %s; inkling backend unavailable\n", T.path, missing);
        dlclose(K.lib);
        memset(&K.init, 0, sizeof K - ((char *)&K.init - (char *)&K));
        K.lib = NULL;
    }
}

int sabrewing_loader_ink_available(void) { ink_load_once(); return K.available; }
int ink_cuda_init(int dev) { ink_load_once(); return K.available ? K.init(dev) : -1; }
size_t ink_cuda_free_bytes(void) { ink_load_once(); return K.available ? K.free_bytes() : 0; }
size_t ink_cuda_total_bytes(void) { ink_load_once(); return K.available ? K.total_bytes() : 0; }
void *ink_cuda_upload(const void *h, size_t n) { ink_load_once(); return K.available ? K.upload(h, n) : NULL; }
/* bf16 weights against bf16-rounded activations (c/backend_cuda_ink.cu:63-64; the CPU's matmul_h) */
int ink_cuda_matmul_bf16(float *y, const float *x, const void *W, int S, int I, int O) {
    ink_load_once(); return K.available ? K.matmul_bf16_rx(y, x, W, S, I, O) : -1;
}
int ink_cuda_matmul_q4(float *y, const float *x, const void *packed, const void *scale, int S, int I, int O) {
    ink_load_once(); return K.available ? K.matmul_q4(y, x, packed, scale, S, I, O) : -1;
}
int ink_cuda_matmul_q8(float *y, const float *x, const void *q8, const void *scale, int S, int I, int O) {
    ink_load_once(); return K.available ? K.matmul_q8_s(y, x, q8, scale, S, I, O) : -1;
}
int ink_cuda_expert_q4(float *out, const float *x, const void *p13, const void *s13, const void *p2, const void *s2,
                       int I, int D) {
    ink_load_once(); return K.available ? K.expert_q4(out, x, p13, s13, p2, s2, I, D) : -1;
}

/* ---- the coli family (c/backend_loader.c:99-512): its own table over the same
 * library, every one of its slots resolved or none; 0 / NULL / -1 while
 * unavailable ---- */
static struct {
    int loaded, available;
    void *lib;
    __typeof__(coli_hip_init) *init;
    __typeof__(coli_hip_shutdown) *shutdown;
    __typeof__(coli_hip_device_count) *device_count;
    __typeof__(coli_hip_device_at) *device_at;
    __typeof__(coli_hip_mem_info) *mem_info;
    __typeof__(coli_hip_stats) *stats;
    __typeof__(coli_hip_group_stats) *group_stats;
    __typeof__(coli_hip_tensor_upload_g) *tensor_upload_g;
    __typeof__(coli_hip_tensor_upload) *tensor_upload;
    __typeof__(coli_hip_matmul) *matmul;
    __typeof__(coli_hip_expert_mlp) *expert_mlp;
    __typeof__(coli_hip_shared_mlp_w4a16) *shared_mlp_w4a16;
    __typeof__(coli_hip_expert_group_issue) *expert_group_issue;
    __typeof__(coli_hip_expert_group_take) *expert_group_take;
    __typeof__(coli_hip_expert_group) *expert_group;
    __typeof__(coli_hip_attention_absorb) *attention_absorb;
    __typeof__(coli_hip_attention_absorb_batch) *attention_absorb_batch;
    __typeof__(coli_hip_attention_project_batch) *attention_project_batch;
    __typeof__(coli_hip_attention_project_ragged) *attention_project_ragged;
    __typeof__(coli_hip_attention_project_batch_dev) *attention_project_batch_dev;
    __typeof__(coli_hip_attention_absorb_batch_dev) *attention_absorb_batch_dev;
    __typeof__(coli_hip_attention_absorb_kvdev) *attention_absorb_kvdev;
    __typeof__(coli_hip_attention_project_batch_dev_out) *attention_project_batch_dev_out;
    __typeof__(coli_hip_tensor_free) *tensor_free;
    __typeof__(coli_hip_tensor_bytes) *tensor_bytes;
    __typeof__(coli_hip_tensor_device) *tensor_device;
    __typeof__(coli_hip_tensor_update) *tensor_update;
    __typeof__(coli_hip_pipe_scratch) *pipe_scratch;
    __typeof__(coli_hip_pipe_alloc) *pipe_alloc;
    __typeof__(coli_hip_pipe_free) *pipe_free;
    __typeof__(coli_hip_pipe_upload) *pipe_upload;
    __typeof__(coli_hip_pipe_download) *pipe_download;
    __typeof__(coli_hip_pipe_rmsnorm) *pipe_rmsnorm;
    __typeof__(coli_hip_pipe_rope) *pipe_rope;
    __typeof__(coli_hip_pipe_silu_mul) *pipe_silu_mul;
    __typeof__(coli_hip_pipe_add) *pipe_add;
    __typeof__(coli_hip_pipe_rows_add) *pipe_rows_add;
    __typeof__(coli_hip_pipe_gemm) *pipe_gemm;
    __typeof__(coli_hip_pipe_rmsnorm_s) *pipe_rmsnorm_s;
    __typeof__(coli_hip_pipe_rope_base) *pipe_rope_base;
    __typeof__(coli_hip_pipe_copy2d) *pipe_copy2d;
    __typeof__(coli_hip_pipe_peer_copy) *pipe_peer_copy;
    __typeof__(coli_hip_pipe_sync) *pipe_sync;
    __typeof__(coli_hip_expert_group_resident_issue) *expert_group_resident_issue;
    __typeof__(coli_hip_expert_group_resident_take) *expert_group_resident_take;
    __typeof__(coli_hip_pipe_router) *pipe_router;
} C;

#define RESOLVE_C(field)                                                 \
    do {                                                                 \
        *(void **)(&C.field) = dlsym(C.lib, "coli_hip_" #field);         \
        if (!C.field) { missing = "coli_hip_" #field; goto unload; }    \
    } while (0)

static void coli_load_once(void) {
    if (C.loaded) return;
    C.loaded = 1;
    if (!T.path[0]) resolve_path();
    if (!T.path[0]) return;
    C.lib = dlopen(T.path, RTLD_NOW | RTLD_LOCAL);
    if (!C.lib) return;
    {
        const char *missing = NULL;
        RESOLVE_C(init);
        RESOLVE_C(shutdown);
        RESOLVE_C(device_count);
        RESOLVE_C(device_at);
        RESOLVE_C(mem_info);
        RESOLVE_C(stats);
        RESOLVE_C(group_stats);
        RESOLVE_C(tensor_upload_g);
        RESOLVE_C(tensor_upload);
        RESOLVE_C(matmul);
        RESOLVE_C(expert_mlp);
        RESOLVE_C(shared_mlp_w4a16);
        RESOLVE_C(expert_group_issue);
        RESOLVE_C(expert_group_take);
        RESOLVE_C(expert_group);
        RESOLVE_C(attention_absorb);
        RESOLVE_C(attention_absorb_batch);
        RESOLVE_C(attention_project_batch);
        RESOLVE_C(attention_project_ragged);
        RESOLVE_C(attention_project_batch_dev);
        RESOLVE_C(attention_absorb_batch_dev);
        RESOLVE_C(attention_absorb_kvdev);
        RESOLVE_C(attention_project_batch_dev_out);
        RESOLVE_C(tensor_free);
        RESOLVE_C(tensor_bytes);
        RESOLVE_C(tensor_device);
        RESOLVE_C(tensor_update);
        RESOLVE_C(pipe_scratch);
        RESOLVE_C(pipe_alloc);
        RESOLVE_C(pipe_free);
        RESOLVE_C(pipe_upload);
        RESOLVE_C(pipe_download);
        RESOLVE_C(pipe_rmsnorm);
        RESOLVE_C(pipe_rope);
        RESOLVE_C(pipe_silu_mul);
        RESOLVE_C(pipe_add);
        RESOLVE_C(pipe_rows_add);
        RESOLVE_C(pipe_gemm);
        RESOLVE_C(pipe_rmsnorm_s);
        RESOLVE_C(pipe_rope_base);
        RESOLVE_C(pipe_copy2d);
        RESOLVE_C(pipe_peer_copy);
        RESOLVE_C(pipe_sync);
        RESOLVE_C(expert_group_resident_issue);
        RESOLVE_C(expert_group_resident_take);
        RESOLVE_C(pipe_router);
        C.available = 1;
        return;
    unload:
        fprintf(stderr, "[sabrewing-loader] %s: missing symbol %s; coli backend unavailable\n", T.path, missing);
        dlclose(C.lib);
        memset(&C, 0, sizeof C);
        C.loaded = 1;
    }
}

int sabrewing_loader_coli_available(void) { coli_load_once(); return C.available; }

int coli_cuda_init(const int *devices, int count) {
    coli_load_once();
    return C.available ? C.init(devices, count) : 0;
}
void coli_cuda_shutdown(void) {
    coli_load_once();
    if (C.available) C.shutdown();
}
int coli_cuda_device_count(void) {
    coli_load_once();
    return C.available ? C.device_count() : 0;
}
int coli_cuda_device_at(int index) {
    coli_load_once();
    return C.available ? C.device_at(index) : -1;
}
int coli_cuda_mem_info(int device, size_t *free_bytes, size_t *total_bytes) {
    coli_load_once();
    return C.available ? C.mem_info(device, free_bytes, total_bytes) : 0;
}
void coli_cuda_stats(int device, size_t *tensor_count, size_t *tensor_bytes) {
    coli_load_once();
    if (C.available) C.stats(device, tensor_count, tensor_bytes);
}
void coli_cuda_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows, double *h2d_ms, double *kernel_ms, double *d2h_ms) {
    coli_load_once();
    if (C.available) C.group_stats(calls, experts, rows, h2d_ms, kernel_ms, d2h_ms);
}
int coli_cuda_tensor_upload_g(ColiCudaTensor **tensor, const void *weights, const float *scales, int fmt, int I, int O, int device, int gs) {
    coli_load_once();
    return C.available ? C.tensor_upload_g((ColiHipTensor **)tensor, weights, scales, fmt, I, O, device, gs) : 0;
}
int coli_cuda_tensor_upload(ColiCudaTensor **tensor, const void *weights, const float *scales, int fmt, int I, int O, int device) {
    coli_load_once();
    return C.available ? C.tensor_upload((ColiHipTensor **)tensor, weights, scales, fmt, I, O, device) : 0;
}
int coli_cuda_matmul(ColiCudaTensor **tensor, float *y, const float *x, const void *weights, const float *scales, int fmt, int S, int I, int O, int device, int gs) {
    coli_load_once();
    return C.available ? C.matmul((ColiHipTensor **)tensor, y, x, weights, scales, fmt, S, I, O, device, gs) : 0;
}
int coli_cuda_expert_mlp(ColiCudaTensor *gate, ColiCudaTensor *up, ColiCudaTensor *down, float *y, const float *x, int S) {
    coli_load_once();
    return C.available ? C.expert_mlp((ColiHipTensor *)gate, (ColiHipTensor *)up, (ColiHipTensor *)down, y, x, S) : 0;
}
int coli_cuda_shared_mlp_w4a16(ColiCudaTensor *gate, ColiCudaTensor *up, ColiCudaTensor *down, float *y, const float *x, int S) {
    coli_load_once();
    return C.available ? C.shared_mlp_w4a16((ColiHipTensor *)gate, (ColiHipTensor *)up, (ColiHipTensor *)down, y, x, S) : 0;
}
int coli_cuda_expert_group_issue(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups, ColiCudaTensor *const *downs, const int *rows, int count, const float *x) {
    coli_load_once();
    return C.available ? C.expert_group_issue((ColiHipTensor *const *)gates, (ColiHipTensor *const *)ups, (ColiHipTensor *const *)downs, rows, count, x) : 0;
}
const float *coli_cuda_expert_group_take(int device) {
    coli_load_once();
    return C.available ? C.expert_group_take(device) : NULL;
}
int coli_cuda_expert_group(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups, ColiCudaTensor *const *downs, const int *rows, int count, float *y, const float *x) {
    coli_load_once();
    return C.available ? C.expert_group((ColiHipTensor *const *)gates, (ColiHipTensor *const *)ups, (ColiHipTensor *const *)downs, rows, count, y, x) : 0;
}
int coli_cuda_attention_absorb(ColiCudaTensor *kv_b, float *ctx, const float *q, const float *latent, const float *rope, int H, int Q, int R, int V, int K, int T, float attention_scale) {
    coli_load_once();
    return C.available ? C.attention_absorb((ColiHipTensor *)kv_b, ctx, q, latent, rope, H, Q, R, V, K, T, attention_scale) : 0;
}
int coli_cuda_attention_absorb_batch(ColiCudaTensor *kv_b, float *ctx, const float *q, const float *latent, const float *rope, int S, int H, int Q, int R, int V, int K, int T, float attention_scale) {
    coli_load_once();
    return C.available ? C.attention_absorb_batch((ColiHipTensor *)kv_b, ctx, q, latent, rope, S, H, Q, R, V, K, T, attention_scale) : 0;
}
int coli_cuda_attention_project_batch(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out, const float *q, const float *latent, const float *rope, int S, int H, int Q, int R, int V, int K, int T, float attention_scale) {
    coli_load_once();
    return C.available ? C.attention_project_batch((ColiHipTensor *)kv_b, (ColiHipTensor *)o_proj, out, q, latent, rope, S, H, Q, R, V, K, T, attention_scale) : 0;
}
int coli_cuda_attention_project_ragged(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out, const float *q, const void *const *keys, const float *const *latent, const float *const *rope, const int *lengths, int S, int H, int Q, int R, int V, int K, int max_t, float attention_scale) {
    coli_load_once();
    return C.available ? C.attention_project_ragged((ColiHipTensor *)kv_b, (ColiHipTensor *)o_proj, out, q, keys, latent, rope, lengths, S, H, Q, R, V, K, max_t, attention_scale) : 0;
}
int coli_cuda_attention_project_batch_dev(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out, const float *q_dev, const float *latent_dev, const float *rope_dev, int S, int H, int Q, int R, int V, int K, int T, float scale) {
    coli_load_once();
    return C.available ? C.attention_project_batch_dev((ColiHipTensor *)kv_b, (ColiHipTensor *)o_proj, out, q_dev, latent_dev, rope_dev, S, H, Q, R, V, K, T, scale) : 0;
}
int coli_cuda_attention_absorb_batch_dev(ColiCudaTensor *kv_b_shard, float *ctx_dev, const float *q_dev, const float *latent_dev, const float *rope_dev, int S, int H, int Q, int R, int V, int K, int T, float scale) {
    coli_load_once();
    return C.available ? C.attention_absorb_batch_dev((ColiHipTensor *)kv_b_shard, ctx_dev, q_dev, latent_dev, rope_dev, S, H, Q, R, V, K, T, scale) : 0;
}
int coli_cuda_attention_absorb_kvdev(ColiCudaTensor *kv_b, float *ctx, const float *q, const float *latent_dev, const float *rope_dev, int H, int Q, int R, int V, int K, int T, float scale) {
    coli_load_once();
    return C.available ? C.attention_absorb_kvdev((ColiHipTensor *)kv_b, ctx, q, latent_dev, rope_dev, H, Q, R, V, K, T, scale) : 0;
}
int coli_cuda_attention_project_batch_dev_out(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj, float *out_dev, const float *q_dev, const float *latent_dev, const float *rope_dev, int S, int H, int Q, int R, int V, int K, int T, float scale) {
    coli_load_once();
    return C.available ? C.attention_project_batch_dev_out((ColiHipTensor *)kv_b, (ColiHipTensor *)o_proj, out_dev, q_dev, latent_dev, rope_dev, S, H, Q, R, V, K, T, scale) : 0;
}
void coli_cuda_tensor_free(ColiCudaTensor *tensor) {
    coli_load_once();
    if (C.available) C.tensor_free((ColiHipTensor *)tensor);
}
size_t coli_cuda_tensor_bytes(const ColiCudaTensor *tensor) {
    coli_load_once();
    return C.available ? C.tensor_bytes((const ColiHipTensor *)tensor) : 0;
}
int coli_cuda_tensor_device(const ColiCudaTensor *tensor) {
    coli_load_once();
    return C.available ? C.tensor_device((const ColiHipTensor *)tensor) : -1;
}
int coli_cuda_tensor_update(ColiCudaTensor *tensor, const void *weights, const float *scales) {
    coli_load_once();
    return C.available ? C.tensor_update((ColiHipTensor *)tensor, weights, scales) : 0;
}
float *coli_cuda_pipe_scratch(int device, int slot, size_t bytes) {
    coli_load_once();
    return C.available ? C.pipe_scratch(device, slot, bytes) : NULL;
}
void *coli_cuda_pipe_alloc(int device, size_t bytes) {
    coli_load_once();
    return C.available ? C.pipe_alloc(device, bytes) : NULL;
}
void coli_cuda_pipe_free(int device, void *p) {
    coli_load_once();
    if (C.available) C.pipe_free(device, p);
}
int coli_cuda_pipe_upload(int device, void *dst, const void *src, size_t bytes) {
    coli_load_once();
    return C.available ? C.pipe_upload(device, dst, src, bytes) : 0;
}
int coli_cuda_pipe_download(int device, const void *src, void *dst, size_t bytes) {
    coli_load_once();
    return C.available ? C.pipe_download(device, src, dst, bytes) : 0;
}
int coli_cuda_pipe_rmsnorm(int device, float *y_dev, const float *x_dev, const float *w_dev, int S, int D, float eps) {
    coli_load_once();
    return C.available ? C.pipe_rmsnorm(device, y_dev, x_dev, w_dev, S, D, eps) : 0;
}
int coli_cuda_pipe_rope(int device, float *v_dev, const int *pos_dev, int rows, int stride, int offset, int R, int heads, float theta) {
    coli_load_once();
    return C.available ? C.pipe_rope(device, v_dev, pos_dev, rows, stride, offset, R, heads, theta) : 0;
}
int coli_cuda_pipe_silu_mul(int device, float *gate_dev, const float *up_dev, size_t n) {
    coli_load_once();
    return C.available ? C.pipe_silu_mul(device, gate_dev, up_dev, n) : 0;
}
int coli_cuda_pipe_add(int device, float *x_dev, const float *t_dev, size_t n) {
    coli_load_once();
    return C.available ? C.pipe_add(device, x_dev, t_dev, n) : 0;
}
int coli_cuda_pipe_rows_add(int device, float *x_dev, const float *partial_dev, const int *rows_dev, int nrows, int D) {
    coli_load_once();
    return C.available ? C.pipe_rows_add(device, x_dev, partial_dev, rows_dev, nrows, D) : 0;
}
int coli_cuda_pipe_gemm(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    coli_load_once();
    return C.available ? C.pipe_gemm((ColiHipTensor *)t, y_dev, x_dev, S) : 0;
}
int coli_cuda_pipe_rmsnorm_s(int device, float *y_dev, const float *x_dev, const float *w_dev, int S, int D, float eps, int xstride, int ystride) {
    coli_load_once();
    return C.available ? C.pipe_rmsnorm_s(device, y_dev, x_dev, w_dev, S, D, eps, xstride, ystride) : 0;
}
int coli_cuda_pipe_rope_base(int device, float *v_dev, int pos_base, int rows, int stride, int offset, int R, int heads, float theta) {
    coli_load_once();
    return C.available ? C.pipe_rope_base(device, v_dev, pos_base, rows, stride, offset, R, heads, theta) : 0;
}
int coli_cuda_pipe_copy2d(int device, float *dst, int dpitch, const float *src, int spitch, int width, int height) {
    coli_load_once();
    return C.available ? C.pipe_copy2d(device, dst, dpitch, src, spitch, width, height) : 0;
}
int coli_cuda_pipe_peer_copy(int dst_dev, float *dst, int src_dev, const float *src, size_t bytes) {
    coli_load_once();
    return C.available ? C.pipe_peer_copy(dst_dev, dst, src_dev, src, bytes) : 0;
}
int coli_cuda_pipe_sync(int device) {
    coli_load_once();
    return C.available ? C.pipe_sync(device) : 0;
}
int coli_cuda_expert_group_resident_issue(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups, ColiCudaTensor *const *downs, const float *weights, int count, int home_device, const float *x_src_dev, float *partial_slot_dev) {
    coli_load_once();
    return C.available ? C.expert_group_resident_issue((ColiHipTensor *const *)gates, (ColiHipTensor *const *)ups, (ColiHipTensor *const *)downs, weights, count, home_device, x_src_dev, partial_slot_dev) : 0;
}
int coli_cuda_expert_group_resident_take(int home_device, const int *devices, int n_issued, float *slots_dev, float *acc_dev, int D) {
    coli_load_once();
    return C.available ? C.expert_group_resident_take(home_device, devices, n_issued, slots_dev, acc_dev, D) : 0;
}
int coli_cuda_pipe_router(int device, const float *x_dev, const void *rw_dev, const void *rb_dev, int D, int E, int Ksel, float topp, int norm_topk, float routed_scale, int *idx_host, float *w_host, int *keff_host) {
    coli_load_once();
    return C.available ? C.pipe_router(device, x_dev, rw_dev, rb_dev, D, E, Ksel, topp, norm_topk, routed_scale, idx_host, w_host, keff_host) : 0;
}
