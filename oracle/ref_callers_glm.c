/* ref_callers_glm.c -- the GLM engine's router GEMV: c/quant.h's f32 matmul
 * (c/quant.h:98-102, called by c/colibri.c:2871), compiled where it lies.
 *
 * TEST INFRASTRUCTURE ONLY (oracle/_ref): pins the oracle's GLM router logits. */
#include "quant.h"

void ref_glm_matmul(float *y, const float *x, const float *W, int S, int I, int O) { matmul(y, x, W, S, I, O); }
