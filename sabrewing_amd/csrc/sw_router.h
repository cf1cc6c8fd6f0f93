// sw_router.h -- the router GEMV block (exact 16-lane FMA-chain contract),
// usable alone or as part of a fused stage kernel.
#ifndef SW_ROUTER_H
#define SW_ROUTER_H
#include "sw_hip.h"
#include "sw_libm.h"
#include "sw_gate.h"

// logits[s,e] = sum_i x[s,i] W[e,i] under the contract of the reference's
// AVX-512 router (c/moe_matmul.h:25-43; bf16 weights c/moe_matmul.h:92-110):
// 16 FMA chains, chain j over i = j mod 16 ascending, then GCC's
// _mm512_reduce_add_ps tree (j,j+8) -> (j,j+4) -> (0+2, 1+3) -> final.
// One wave per expert: the expert's chain-major block (16 chains of M = D/16
// elements) comes in with coalesced 16-byte loads into a wave-private LDS
// region (chain stride padded by 16 bytes), x is staged transposed once per
// block, and lanes 0..15 then run the 16 chains from LDS; the tree is four
// shuffles.  Chains are staged in runs of at most RT_MC elements so any D
// fits.  Block = nw experts of one token.
#define RT_MC 256
#define RT_XB 16          // x float4 loads in flight per thread
struct RouterArgs {
    const void *Wc;            // chain-major router
    const float *x;            // [S, D]
    int D, E;
    const float *lbias;        // logit bias or null
    float *logits;             // [S, E]
    int act;
    float *scores;             // [S, E] sigmoid / softplus scores (act != 1) or null
    sw_u32x4 *xl;              // dot8 limbs of x, or null
    float *xs;
};
// block bx (of nbx per token) of token s; nw = blockDim.x / 64 experts per block;
// smem: the dynamic LDS (router_lds bytes)
template <int BF16>
__device__ __forceinline__ void router_block(const RouterArgs &R, int bx, int s, int nbx, float *smem) {
    __shared__ uint64_t tab[32];                     // expf table for the sigmoid / softplus scores
    constexpr int ESZ = BF16 ? 2 : 4;
    const void *__restrict__ Wc = R.Wc;
    const float *__restrict__ x = R.x;
    const int D = R.D, E = R.E, act = R.act;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int M = D / 16, ML = M + 4;
    const int MC = M < RT_MC ? M : RT_MC;            // chain elements per run
    const int runb = MC * ESZ, runs = runb + 16;      // run bytes, padded LDS stride
    float *xt = smem;                                 // [16][ML]
    char *wl = (char *)(smem + 16 * ML) + wave * 16 * runs;
    const int e = bx * nw + wave;
    const bool valid = e < E;
    const char *wsrc = (const char *)Wc + (int64_t)(valid ? e : 0) * 16 * M * ESZ;
    const int nseg = runb;                            // 16-byte segments per run (16 chains x runb bytes)
    // first run of this wave's expert: loads in flight while x is staged
    sw_u32x4 wv[8];
    auto wload = [&](int s0, int m0) {
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const int seg = min(s0 + 64 * l + lane, nseg - 1);
            const int o = 16 * seg, j = o / runb, w = o - j * runb;
            wv[l] = *(const sw_u32x4 *)(wsrc + (int64_t)j * M * ESZ + (int64_t)m0 * ESZ + w);
        }
    };
    auto wstore = [&](int s0) {
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const int seg = s0 + 64 * l + lane;
            if (seg < nseg) {
                const int o = 16 * seg, j = o / runb, w = o - j * runb;
                *(sw_u32x4 *)(wl + j * runs + w) = wv[l];
            }
        }
    };
    wload(0, 0);
    if (tid < 32) tab[tid] = sw_exp2f_tab[tid];
    if (R.xl) {                                       // the token's dot8 limbs, half a wave per group
        const int G = D / SW_RG;
        for (int g = bx * 2 * nw + (tid >> 5); g < G; g += nbx * 2 * nw)
            limbs_group(x[(int64_t)s * D + g * SW_RG + (tid & 31)], tid & 31, R.xl + ((int64_t)s * G + g) * SW_NL,
                        R.xs + (int64_t)s * G + g);
    }
    {
        const float *xr = x + (int64_t)s * D;
        const int nx4 = D / 4;
        for (int i0 = 0; i0 < nx4; i0 += RT_XB * (int)blockDim.x) {
            sw_f32x4 xv[RT_XB];
#pragma unroll
            for (int u = 0; u < RT_XB; u++) xv[u] = *(const sw_f32x4 *)(xr + 4 * min(i0 + u * (int)blockDim.x + tid, nx4 - 1));
#pragma unroll
            for (int u = 0; u < RT_XB; u++) {
                const int i4 = i0 + u * (int)blockDim.x + tid;
                if (i4 < nx4) {
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const int k = 4 * i4 + c;
                        xt[(k & 15) * ML + (k >> 4)] = xv[u][c];
                    }
                }
            }
        }
    }
    float acc = 0.f;
    for (int m0 = 0; m0 < M; m0 += MC) {
        if (m0 > 0) {
            __builtin_amdgcn_wave_barrier();          // every lane done with the previous run
            wload(0, m0);
        }
        wstore(0);
        for (int s0 = 8 * 64; s0 < nseg; s0 += 8 * 64) {
            wload(s0, m0);
            wstore(s0);
        }
        if (m0 == 0) __syncthreads();                 // x^T staged by the whole block
        __builtin_amdgcn_wave_barrier();
        if (valid && lane < 16) {
            const int j = lane;
            const float *xj = xt + j * ML + m0;
            const char *wj = wl + j * runs;
            if (BF16) {
#pragma unroll 4
                for (int m = 0; m < MC; m += 8) {
                    const sw_u32x4 wd = *(const sw_u32x4 *)(wj + 2 * m);
                    const sw_f32x4 xa = *(const sw_f32x4 *)(xj + m), xb = *(const sw_f32x4 *)(xj + m + 4);
                    const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const uint32_t bits = (u & 1) ? (wd[u >> 1] & 0xFFFF0000u) : (wd[u >> 1] << 16);
                        acc = __builtin_fmaf(xv[u], __builtin_bit_cast(float, bits), acc);
                    }
                }
            } else {
#pragma unroll 4
                for (int m = 0; m < MC; m += 4) {
                    const sw_u32x4 wd = *(const sw_u32x4 *)(wj + 4 * m);
                    const sw_f32x4 xa = *(const sw_f32x4 *)(xj + m);
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        // element copied to a scalar first: clang lowers a bit_cast of a
                        // vector-element lvalue to a read of element 0
                        const uint32_t wu = wd[u];
                        acc = __builtin_fmaf(xa[u], __builtin_bit_cast(float, wu), acc);
                    }
                }
            }
        }
    }
    float v = acc;
    v = v + __shfl_down(v, 8, 16);
    v = v + __shfl_down(v, 4, 16);
    v = v + __shfl_down(v, 2, 16);
    v = v + __shfl_down(v, 1, 16);
    if (lane == 0 && valid) {
        if (R.lbias) v = v + R.lbias[e];
        R.logits[(int64_t)s * E + e] = v;
        if (act != 1 && R.scores)
            R.scores[(int64_t)s * E + e] = (act == 2) ? sw_softplus_ref_t(v, tab) : sw_sigmoid_ref_t(v, tab);
    }
}
__host__ inline size_t router_lds(int D, int w_bf16, int nw) {
    const int M = D / 16, MC = M < RT_MC ? M : RT_MC;
    return (size_t)16 * (M + 4) * 4 + (size_t)nw * 16 * (MC * (w_bf16 ? 2 : 4) + 16);
}


#endif
