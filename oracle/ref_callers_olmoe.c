/* ref_callers_olmoe.c -- the OLMoE engine's routing (c/olmoe.c:607-632),
 * from its own softmax_row (c/olmoe.c:212-216), compiled where it lies with
 * main() renamed.  Its top-k is the inline scan of c/olmoe.c:609-630, the
 * selection rule of moe_topk (c/moe_arch.h:64-89: strict > from -1e30, ties
 * to the lowest id, the lowest unselected expert when nothing is valid),
 * which this file calls; the weights are the picks' probabilities,
 * renormalised in float when norm (c/olmoe.c:632).
 *
 * TEST INFRASTRUCTURE ONLY (oracle/_ref): pins the oracle's OLMoE routing. */
#define main olmoe_main_unused
#include "olmoe.c"
#undef main
#include "moe_arch.h"

void ref_olmoe_route(const float *logits, int E, int K, int norm, int *sel, float *w) {
    float *pr = (float *)malloc((size_t)E * sizeof(float));
    memcpy(pr, logits, (size_t)E * sizeof(float));
    softmax_row(pr, E);
    moe_topk(pr, NULL, 0, E, K, sel);
    for (int k = 0; k < K; k++) w[k] = pr[sel[k]];
    if (norm) { float sm = 0; for (int k = 0; k < K; k++) sm += w[k]; for (int k = 0; k < K; k++) w[k] /= sm; }
    free(pr);
}
void ref_olmoe_softmax_row(float *x, int n) { softmax_row(x, n); }
