/* sabrewing_loader.h -- the Linux runtime seam between an unmodified
 * sabrewing engine and the gfx950 backend.
 *
 * libsabrewing_loader.so exports the reference's Laguna backend ABI under its
 * own names (the declarations of c/backend_cuda_laguna.h:25-95, same
 * signatures and 0 / -1 returns).  Each wrapper forwards through a function
 * table resolved from libsabrewing_hip.so at first use, with the semantics of
 * the reference's Windows DLL loader (c/backend_loader.c:99-253): the library
 * is opened by absolute path only (next to the loader, or $SABREWING_HIP_LIB),
 * every table slot must resolve or the library is unloaded again, and while
 * the backend is unavailable every wrapper returns the "not initialised"
 * value (-1 / NULL / 0), so the engine keeps its CPU path.  Entries with no
 * MI355X counterpart (int8 residents, fp4 experts) always return -1.
 * An engine links this object in place of backend_cuda_laguna.o. */
#ifndef SABREWING_LOADER_H
#define SABREWING_LOADER_H
#include <stddef.h>
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

/* 1 when the backend library loaded and every slot resolved (loads on first call) */
int    sabrewing_loader_available(void);
/* the absolute path tried (or "" before the first attempt) */
const char *sabrewing_loader_path(void);

#ifdef __cplusplus
}
#endif
#endif
