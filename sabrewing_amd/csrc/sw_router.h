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
// Lane l = 16 q + j of wave w runs chain j of expert 4 * (block's first wave
// + w) + q.  The router comes in the order of k_chain_major (k_route.hip), in
// its own element type: experts in groups of 4, each group a run of 1 KB
// slices, slice q holding the next P elements (8 bf16 or 4 f32) of each of
// its 64 chains, so one 16-byte load per lane reads one slice, contiguous,
// and gives each lane the next P elements of its own chain; RT_PF slices are
// in flight (half of a D = 4096 bf16 chain, issued before the block's other
// traffic); a bf16 weight widens exactly to f32; x is
// staged transposed in LDS once per block, so chain j reads x[16m + j] as
// xt[j][m]; the tree is four shuffles within each 16-lane row.  The chain is
// M = D/16 dependent fmas per lane, the critical path of the routing.
#define RT_PF 16
#define RT_XB 8           // x float4 loads in flight per thread
struct RouterArgs {
    const void *Wc;            // router in the streaming order (k_chain_major)
    const float *x;            // [S, D]
    int D, E;
    const float *lbias;        // logit bias or null
    float *logits;             // [S, E]
    int act;
    float *scores;             // [S, E] sigmoid / softplus scores (act != 1) or null
    sw_u32x4 *xl;              // dot8 limbs of x, or null
    float *xs;
};
// experts per block of nt threads
__host__ __device__ inline int router_epb(int nt) { return 4 * (nt / 64); }
// block bx (of nbx per token) of token s; smem: the dynamic LDS (router_lds bytes)
template <int BF16>
__device__ __forceinline__ void router_block(const RouterArgs &R, int bx, int s, int nbx, float *smem) {
    constexpr int P = BF16 ? 8 : 4;
    __shared__ uint64_t tab[32];                     // expf table for the sigmoid / softplus scores
    const float *__restrict__ x = R.x;
    const int D = R.D, E = R.E, act = R.act;
    const int nt = blockDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    const int M = D / 16, ML = M + 4, NQ = M / P;
    const int j = lane & 15;
    const int eg = bx * nw + wave, e = eg * 4 + (lane >> 4);
    const bool valid = e < E;
    // slice q of this lane: byte voff + 1024 q of the router (groups past the last: clamp)
    const int ng4 = (E + 3) / 4;
    const int egc = eg < ng4 ? eg : ng4 - 1;
    const sw_rsrc rw = sw_make_rsrc(R.Wc, (uint32_t)ng4 * 4u * (uint32_t)D * (BF16 ? 2u : 4u));
    const uint32_t voff = ((uint32_t)egc * NQ * 64 + lane) * 16;
    auto slice = [&](int q) { return sw_ld16(rw, voff, (uint32_t)min(q, NQ - 1) * 1024u); };
    float *xt = smem;                                 // [16][ML]
    sw_u32x4 ring[RT_PF];
#pragma unroll
    for (int u = 0; u < RT_PF; u++) ring[u] = slice(u);
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
        for (int i0 = 0; i0 < nx4; i0 += RT_XB * nt) {
            sw_f32x4 xv[RT_XB];
#pragma unroll
            for (int u = 0; u < RT_XB; u++) xv[u] = *(const sw_f32x4 *)(xr + 4 * min(i0 + u * nt + tid, nx4 - 1));
#pragma unroll
            for (int u = 0; u < RT_XB; u++) {
                const int i4 = i0 + u * nt + tid;
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
    __syncthreads();
    const float *xj = xt + j * ML;
    float acc = 0.f;
    auto chain4 = [&](int q, const sw_u32x4 &w) {
        if constexpr (BF16) {
            const sw_f32x4 xa = *(const sw_f32x4 *)(xj + 8 * q), xb = *(const sw_f32x4 *)(xj + 8 * q + 4);
            acc = __builtin_fmaf(xa.x, __builtin_bit_cast(float, w.x << 16), acc);
            acc = __builtin_fmaf(xa.y, __builtin_bit_cast(float, w.x & 0xFFFF0000u), acc);
            acc = __builtin_fmaf(xa.z, __builtin_bit_cast(float, w.y << 16), acc);
            acc = __builtin_fmaf(xa.w, __builtin_bit_cast(float, w.y & 0xFFFF0000u), acc);
            acc = __builtin_fmaf(xb.x, __builtin_bit_cast(float, w.z << 16), acc);
            acc = __builtin_fmaf(xb.y, __builtin_bit_cast(float, w.z & 0xFFFF0000u), acc);
            acc = __builtin_fmaf(xb.z, __builtin_bit_cast(float, w.w << 16), acc);
            acc = __builtin_fmaf(xb.w, __builtin_bit_cast(float, w.w & 0xFFFF0000u), acc);
        } else {
            // the whole vector is cast: clang lowers a bit_cast of a vector-element
            // lvalue to a read of element 0
            const sw_f32x4 xa = *(const sw_f32x4 *)(xj + 4 * q), wf = __builtin_bit_cast(sw_f32x4, w);
            acc = __builtin_fmaf(xa.x, wf.x, acc);
            acc = __builtin_fmaf(xa.y, wf.y, acc);
            acc = __builtin_fmaf(xa.z, wf.z, acc);
            acc = __builtin_fmaf(xa.w, wf.w, acc);
        }
    };
    // full rounds with unconditional refills (a refill past the end re-reads the last slice),
    // then the last round without: no ring rotation, loads stay in flight across rounds
    int q0 = 0;
    for (; q0 + RT_PF < NQ; q0 += RT_PF) {
#pragma unroll
        for (int u = 0; u < RT_PF; u++) {          // the slot is consumed before its refill
            chain4(q0 + u, ring[u]);
            ring[u] = slice(q0 + u + RT_PF);
            __builtin_amdgcn_sched_barrier(0);        // keep the refill here, not sunk to the round's end
        }
    }
#pragma unroll
    for (int u = 0; u < RT_PF; u++)
        if (q0 + u < NQ) chain4(q0 + u, ring[u]);
    float v = acc;
    v = v + __shfl_down(v, 8, 16);
    v = v + __shfl_down(v, 4, 16);
    v = v + __shfl_down(v, 2, 16);
    v = v + __shfl_down(v, 1, 16);
    if (j == 0 && valid) {
        if (R.lbias) v = v + R.lbias[e];
        R.logits[(int64_t)s * E + e] = v;
        if (act != 1 && R.scores)
            R.scores[(int64_t)s * E + e] = (act == 2) ? sw_softplus_ref_t(v, tab) : sw_sigmoid_ref_t(v, tab);
    }
}
__host__ inline size_t router_lds(int D) { return (size_t)16 * (D / 16 + 4) * 4; }


#endif
