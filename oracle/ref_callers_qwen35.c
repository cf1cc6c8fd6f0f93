/* ref_callers_qwen35.c -- qwen35's routing, its own moe_route
 * (c/qwen35.c:558-589), compiled where it lies with main() renamed.
 *
 * TEST INFRASTRUCTURE ONLY (oracle/_ref): pins the oracle's qwen35 routing. */
#define main qwen35_main_unused
#include "qwen35.c"
#undef main

void ref_qwen35_route(const float *logit, int E, int K, int *sel, float *w) { moe_route(logit, E, K, sel, w); }
