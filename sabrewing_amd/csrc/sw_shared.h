// sw_shared.h -- the shared expert (bf16 weights) as block jobs on the VALU,
// usable alone or as extra blocks of the routed-expert kernels.
//
// Per output row and token, every group of 32 consecutive inputs gives one
// term: a chain of 32 f32 fmas in input order from 0 (the bf16 weight is
// exact in f32); the row is the sum of its group terms in the fixed order of
// the int4 kernels (runs of 16 groups left to right, the runs left to right).
// Tokens are independent, so a token's result does not depend on the batch.
#ifndef SW_SHARED_H
#define SW_SHARED_H
#include "sw_hip.h"

#define SH_RG 32               // inputs per group
#define SH_CHG 16              // groups per run of the row sum

__device__ __forceinline__ float bf16lo(uint32_t u) { return __builtin_bit_cast(float, u << 16); }
__device__ __forceinline__ float bf16hi(uint32_t u) { return __builtin_bit_cast(float, u & 0xFFFF0000u); }

// 32 bf16 weights (4 x 16 bytes) against 32 f32 inputs, in input order
__device__ __forceinline__ float bf16_group_chain(const sw_u32x4 *w, const float *x) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const sw_u32x4 v = w[q];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t u = v[j];
            t = __builtin_fmaf(bf16lo(u), x[8 * q + 2 * j], t);
            t = __builtin_fmaf(bf16hi(u), x[8 * q + 2 * j + 1], t);
        }
    }
    return t;
}

// fixed-order sum of the G group terms p[0..G)
__device__ __forceinline__ float sh_row_sum(const float *p, int G) {
    const int CH = G < SH_CHG ? G : SH_CHG, NC = G / CH;
    float y = 0.f;
    for (int c = 0; c < NC; c++) {
        float run = p[c * CH];
        for (int j = 1; j < CH; j++) run = run + p[c * CH + j];
        y = c == 0 ? run : y + run;
    }
    return y;
}

// Rows job: NR rows (the K bf16 inputs of local row lr at rowp(lr)) against
// the tokens tok0..tok0+nt-1 (nt <= TT) of x [*, K] f32; the row results go
// out through emit(lr, t, y).  Block of 256 threads: thread (ro, g) with
// G = K/32 groups and RPS = 256/G rows per step, SH_PF steps of loads in
// flight.  LDS: red[NR * TT * (G + 1)] floats.
#define SH_PF 4
template <int NR, int TT, class RowPtr, class Emit>
__device__ __forceinline__ void sh_rows_job(RowPtr rowp, int K, const float *__restrict__ x, int tok0, int nt, Emit emit,
                                            float *red) {
    const int G = K / SH_RG, Gp = G + 1;
    const int tid = threadIdx.x;
    const int RPS = 256 / G, NS = (NR + RPS - 1) / RPS;
    const int ro = tid / G, g = tid - ro * G;
    const bool worker = ro < RPS;
    auto wld = [&](int s, sw_u32x4 *w) {
        int lr = s * RPS + (worker ? ro : 0);
        lr = lr < NR ? lr : NR - 1;
        const sw_u32x4 *wp = (const sw_u32x4 *)(rowp(lr) + g * SH_RG);
#pragma unroll
        for (int q = 0; q < 4; q++) w[q] = wp[q];
    };
    sw_u32x4 ring[SH_PF][4];
#pragma unroll
    for (int u = 0; u < SH_PF; u++) wld(u, ring[u]);
    float xv[TT][SH_RG];
#pragma unroll
    for (int t = 0; t < TT; t++) {
        const int tk = tok0 + (t < nt ? t : 0);
        const sw_f32x4 *xp = (const sw_f32x4 *)(x + (int64_t)tk * K + g * SH_RG);
#pragma unroll
        for (int q = 0; q < SH_RG / 4; q++) {
            const sw_f32x4 v = xp[q];
            xv[t][4 * q] = v.x; xv[t][4 * q + 1] = v.y; xv[t][4 * q + 2] = v.z; xv[t][4 * q + 3] = v.w;
        }
    }
    auto step = [&](int s, int u, bool refill) {
        sw_u32x4 w[4];
#pragma unroll
        for (int q = 0; q < 4; q++) w[q] = ring[u][q];
        if (refill) { wld(s + SH_PF, ring[u]); __builtin_amdgcn_sched_barrier(0); }
        const int lr = s * RPS + ro;
        const bool live = worker && lr < NR && s < NS;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float p = bf16_group_chain(w, xv[t]);
            if (live) red[(lr * TT + t) * Gp + g] = p;
        }
    };
    int s0 = 0;
    for (; s0 + SH_PF < NS; s0 += SH_PF) {
#pragma unroll
        for (int u = 0; u < SH_PF; u++) step(s0 + u, u, true);
    }
#pragma unroll
    for (int u = 0; u < SH_PF; u++) step(s0 + u, u, false);
    __syncthreads();
    for (int it = tid; it < NR * TT; it += 256) {
        const int lr = it / TT, t = it - lr * TT;
        if (t < nt) emit(lr, t, sh_row_sum(red + it * Gp, G));
    }
    __syncthreads();
}

// shared expert gate_up: SH_GLU_O outputs i per block; local rows 0..O-1 are
// gate rows i0.., rows O..2O-1 the up rows; h[tok][i] = silu(gate) * up (f32)
#define SH_GLU_O 8
template <int TT>
__device__ __forceinline__ void sh_glu_block(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu,
                                             const float *__restrict__ x, int S, int D, int Is, float *__restrict__ h,
                                             int bid, float *red) {
    const int nrs = Is / SH_GLU_O;
    const int rs = bid % nrs, tt = bid / nrs;
    const int i0 = rs * SH_GLU_O, tok0 = tt * TT;
    const int nt = min(TT, S - tok0);
    float *ys = red + 2 * SH_GLU_O * TT * (D / SH_RG + 1);   // [2*SH_GLU_O][TT] row results
    sh_rows_job<2 * SH_GLU_O, TT>(
        [&](int lr) { return (lr < SH_GLU_O ? Wg : Wu) + (int64_t)(i0 + (lr & (SH_GLU_O - 1))) * D; }, D, x, tok0, nt,
        [&](int lr, int t, float y) { ys[lr * TT + t] = y; }, red);
    const int tid = threadIdx.x;
    if (tid < SH_GLU_O * TT) {
        const int lr = tid / TT, t = tid - lr * TT;
        if (t < nt) {
            const float yg = ys[lr * TT + t], yu = ys[(SH_GLU_O + lr) * TT + t];
            h[(int64_t)(tok0 + t) * Is + i0 + lr] = (yg / (1.0f + expf(-yg))) * yu;
        }
    }
    __syncthreads();
}
template <int TT>
__host__ __device__ constexpr size_t sh_glu_lds(int D) {
    return ((size_t)2 * SH_GLU_O * TT * (D / SH_RG + 1) + (size_t)2 * SH_GLU_O * TT) * 4;
}
__host__ __device__ inline int sh_glu_blocks(int S, int Is, int TT) { return (Is / SH_GLU_O) * ((S + TT - 1) / TT); }

// shared expert down: SH_DN_O output rows d per block, out[tok][d] (f32)
#define SH_DN_O 16
template <int TT>
__device__ __forceinline__ void sh_down_block(const uint16_t *__restrict__ Wd, const float *__restrict__ h, int S, int Is,
                                              int D, float *__restrict__ out, int bid, float *red) {
    const int nrs = D / SH_DN_O;
    const int rs = bid % nrs, tt = bid / nrs;
    const int d0 = rs * SH_DN_O, tok0 = tt * TT;
    const int nt = min(TT, S - tok0);
    sh_rows_job<SH_DN_O, TT>([&](int lr) { return Wd + (int64_t)(d0 + lr) * Is; }, Is, h, tok0, nt,
                             [&](int lr, int t, float y) { out[(int64_t)(tok0 + t) * D + d0 + lr] = y; }, red);
}
template <int TT>
__host__ __device__ constexpr size_t sh_down_lds(int Is) { return (size_t)SH_DN_O * TT * (Is / SH_RG + 1) * 4; }
__host__ __device__ inline int sh_down_blocks(int S, int D, int TT) { return (D / SH_DN_O) * ((S + TT - 1) / TT); }

#endif
