/* loader.c -- Linux dlopen loader: the reference's lag_cuda_* ABI forwarded to
 * libsabrewing_hip.so's lag_hip_* entries (include/sabrewing_loader.h).
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
    (void)y; (void)x; (void)W; (void)S; (void)I; (void)O; return -1;          /* int8 residents: CPU path */
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
