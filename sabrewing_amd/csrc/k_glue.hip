// k_glue.hip -- the stack glue around the MoE block (a layer is
// h += MoE(rmsnorm(h)), the step ends in rmsnorm, the head and a greedy
// pick): RMSNorm of the residual rows and the argmax of the head's logits.
// The head's logits come from the router kernel: the reference computes them
// with resmm -> matmul_bf16 (c/laguna.c:1156-1158), the same 16-lane bf16
// contract as the router, so they are bit-exact and the greedy pick is the
// reference's.
#include "sw_hip.h"
#include "sw_gate.h"

// out[r] = x[r] / rms(x[r]) * w (c/moe_math.h:58-62): the factor by rms_inv_block
// (sw_gate.h), then out = x * inv * w left to right.
__global__ __launch_bounds__(RN_NT) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w,
                                                   float *__restrict__ out, int D, float eps) {
    __shared__ double part[RN_NT / 64];
    const int tid = threadIdx.x;
    const float *xr = x + (int64_t)blockIdx.x * D;
    float v[RN_CH];
    const float inv = rms_inv_block(xr, D, eps, part, v);
    float *orow = out + (int64_t)blockIdx.x * D;
    if (D <= RN_NT * RN_CH) {                          // the row is in registers
#pragma unroll
        for (int k = 0; k < RN_CH; k++) {
            const int i = tid + k * RN_NT;
            if (i < D) orow[i] = v[k] * inv * w[i];
        }
    } else {
        for (int i = tid; i < D; i += RN_NT) orow[i] = xr[i] * inv * w[i];
    }
}

// tok[r] = the index a strict ascending scan `if (v[i] > v[best]) best = i`
// from best = 0 ends on (c/laguna.c:1159): 0 when v[0] is NaN (nothing
// compares greater than it), else the lowest index of the largest non-NaN
// value (-0.0 and +0.0 equal).  Each thread takes the largest word (order
// bits of v + 0.0, ~index) of its values; the block takes the largest word
// (a maximum: the same word whatever order the values are taken in).  Rows
// of a multiple of 4 values that start 16-byte aligned are read as float4,
// AM_U loads per thread in flight before any is used.
#define AM_NT 1024
#define AM_U 8
__global__ __launch_bounds__(AM_NT) void k_argmax(const float *__restrict__ logits, int V, int *__restrict__ tok) {
    __shared__ unsigned long long part[AM_NT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *v = logits + (int64_t)blockIdx.x * V;
    unsigned long long best = 0ull;
    auto take = [&](float f, int i) {
        if (f == f) {
            const unsigned long long k = ((unsigned long long)ord_f32(f + 0.0f) << 32) | (0xFFFFFFFFu - (uint32_t)i);
            best = k > best ? k : best;
        }
    };
    if ((V & 3) == 0 && ((uintptr_t)v & 15) == 0) {
        const sw_f32x4 *v4 = (const sw_f32x4 *)v;
        const int n4 = V / 4;
        for (int i0 = tid; i0 < n4; i0 += AM_NT * AM_U) {
            sw_f32x4 r[AM_U];
#pragma unroll
            for (int u = 0; u < AM_U; u++) r[u] = v4[min(i0 + u * AM_NT, n4 - 1)];
#pragma unroll
            for (int u = 0; u < AM_U; u++) {
                const int i = i0 + u * AM_NT;
                if (i < n4) {
#pragma unroll
                    for (int c = 0; c < 4; c++) take(r[u][c], 4 * i + c);
                }
            }
        }
    } else {
        for (int i = tid; i < V; i += AM_NT) take(v[i], i);
    }
    for (int o = 32; o; o >>= 1) {
        const unsigned long long t = __shfl_xor(best, o);
        best = t > best ? t : best;
    }
    if (lane == 0) part[wave] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long m = part[0];
        for (int q = 1; q < AM_NT / 64; q++) m = part[q] > m ? part[q] : m;
        const float f0 = v[0];
        tok[blockIdx.x] = (f0 != f0) ? 0 : (int)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull));
    }
}

int sw_launch_rmsnorm(hipStream_t st, const float *x, const float *w, float *out, int S, int D, float eps) {
    if (S <= 0 || D <= 0) return -1;
    SW_LAUNCH(k_rmsnorm, dim3((unsigned)S), dim3(RN_NT), 0, st, x, w, out, D, eps);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_argmax(hipStream_t st, const float *logits, int S, int V, int *tok) {
    if (S <= 0 || V <= 0) return -1;
    SW_LAUNCH(k_argmax, dim3((unsigned)S), dim3(AM_NT), 0, st, logits, V, tok);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
