// sw_shared.h -- the shared expert (bf16 weights) as block jobs on the VALU,
// usable alone or as extra blocks of the routed-expert kernels.
//
// Per output row and token, every group of 32 consecutive inputs gives one
// term: a chain of 32 f32 fmas in input order from 0 (the bf16 weight is
// exact in f32); the row is the sum of its group terms in the fixed order of
// the int4 kernels (run_sum in sw_gate.h).  Tokens are independent, so a
// token's result does not depend on the batch.
#ifndef SW_SHARED_H
#define SW_SHARED_H
#include "sw_hip.h"
#include "sw_gate.h"

#define SH_RG 32               // inputs per group
#define SH_CHG 16              // groups per run of the row sum
#define SH_TT 2                // tokens per weight pass of a batch

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

// K inputs in G = K/32 groups, G <= 256
__host__ __device__ inline bool sh_shape_ok(int K) { return K > 0 && K % SH_RG == 0 && K / SH_RG <= 256; }

// Rows job: NR rows (the K bf16 inputs of local row lr at rowp(lr)) against
// the tokens tok0..tok0+nt-1 (nt <= TT) of x [*, K] f32; the row results go
// out through emit(lr, t, y).  Block of NT threads: thread (row slot ro,
// group g) with G = K/32 groups, Gq = run_lanes(G) lanes per row (lanes
// g >= G add zero terms) and RPS row slots (a power of two); slot ro takes
// NS = NR/RPS consecutive rows, one per step, SH_PF steps of loads in flight,
// the group's inputs of every token of the tile in registers.  LDS:
// runs[NR * TT * NC] floats, NC = Gq / min(Gq, 16).
#ifndef SH_PF
#define SH_PF 2
#endif
__host__ __device__ inline int sh_rps(int Gq, int NR, int NT) {
    int r = 1;
    while (r * 2 * Gq <= NT && r < NR) r *= 2;
    return r;
}
template <int NR, int TT, int NT, class RowPtr, class Emit>
__device__ __forceinline__ void sh_rows_job(RowPtr rowp, int K, const float *__restrict__ x, int tok0, int nt, Emit emit,
                                            float *runs) {
    const int G = K / SH_RG, Gq = run_lanes(G);
    const int CH = Gq < SH_CHG ? Gq : SH_CHG, NC = Gq / CH;
    const bool c16 = G % SH_CHG == 0;              // no padding lanes (else they add zero terms)
    const int tid = threadIdx.x;
    const int RPS = sh_rps(Gq, NR, NT), NS = NR / RPS;
    const int ro = tid / Gq, gq = tid - ro * Gq, c = gq / CH;
    const bool worker = ro < RPS, lead = worker && (gq & (CH - 1)) == 0, gv = gq < G;
    const int g = gv ? gq : G - 1;                   // padding lanes load group G-1 and add 0
    const int roc = worker ? ro : 0;
    auto wld = [&](int s, sw_u32x4 *w) {
        const sw_u32x4 *wp = (const sw_u32x4 *)(rowp(roc * NS + s) + g * SH_RG);
#pragma unroll
        for (int q = 0; q < 4; q++) w[q] = wp[q];
    };
    sw_u32x4 ring[SH_PF][4];
#pragma unroll
    for (int u = 0; u < SH_PF; u++) wld(u < NS ? u : NS - 1, ring[u]);
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
        const int lr = roc * NS + s;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            if (t < nt) {                              // uniform over the block
                const float q = bf16_group_chain(w, xv[t]);
                const float p = c16 ? run_sum16(q) : run_sum(gv ? q : 0.f, CH);
                if (lead && s < NS) runs[(lr * TT + t) * NC + c] = p;
            }
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
    for (int it = tid; it < NR * TT; it += NT) {
        const int lr = it / TT, t = it - lr * TT;
        if (t < nt) {
            const float *rr = runs + it * NC;
            float y = rr[0];
            for (int cc = 1; cc < NC; cc++) y = y + rr[cc];
            emit(lr, t, y);
        }
    }
    __syncthreads();
}

__host__ __device__ inline int sh_nc(int K) { return K / SH_RG < SH_CHG ? 1 : run_lanes(K / SH_RG) / SH_CHG; }

// shared expert gate_up: SH_GLU_O outputs i per block; local rows 0..O-1 are
// gate rows i0.., rows O..2O-1 the up rows; h[tok][i] = silu(gate) * up (f32)
#define SH_NT 512              // threads per block of the shared-expert jobs
#ifndef SH_GLU_O
#define SH_GLU_O 8
#endif
template <int TT>
__device__ __forceinline__ void sh_glu_block(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu,
                                             const float *__restrict__ x, int S, int D, int Is, float *__restrict__ h,
                                             int bid, float *red) {
    const int nrs = Is / SH_GLU_O;
    const int rs = bid % nrs, tt = bid / nrs;
    const int i0 = rs * SH_GLU_O, tok0 = tt * TT;
    const int nt = min(TT, S - tok0);
    float *ys = red + 2 * SH_GLU_O * TT * sh_nc(D);   // [2*SH_GLU_O][TT] row results
    sh_rows_job<2 * SH_GLU_O, TT, SH_NT>(
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
__host__ __device__ inline size_t sh_glu_lds(int D) {
    return ((size_t)2 * SH_GLU_O * TT * sh_nc(D) + (size_t)2 * SH_GLU_O * TT) * 4;
}
__host__ __device__ inline int sh_glu_blocks(int S, int Is, int TT) { return (Is / SH_GLU_O) * ((S + TT - 1) / TT); }

// shared expert down: SH_DN_O output rows d per block, out[tok][d] (f32)
#ifndef SH_DN_O
#define SH_DN_O 32
#endif
template <int TT>
__device__ __forceinline__ void sh_down_block(const uint16_t *__restrict__ Wd, const float *__restrict__ h, int S, int Is,
                                              int D, float *__restrict__ out, int bid, float *red) {
    const int nrs = D / SH_DN_O;
    const int rs = bid % nrs, tt = bid / nrs;
    const int d0 = rs * SH_DN_O, tok0 = tt * TT;
    const int nt = min(TT, S - tok0);
    sh_rows_job<SH_DN_O, TT, SH_NT>([&](int lr) { return Wd + (int64_t)(d0 + lr) * Is; }, Is, h, tok0, nt,
                             [&](int lr, int t, float y) { out[(int64_t)(tok0 + t) * D + d0 + lr] = y; }, red);
}
template <int TT>
__host__ __device__ inline size_t sh_down_lds(int Is) { return (size_t)SH_DN_O * TT * sh_nc(Is) * 4; }
__host__ __device__ inline int sh_down_blocks(int S, int D, int TT) { return (D / SH_DN_O) * ((S + TT - 1) / TT); }

// ---- batches (S > 1): token tiles staged in LDS ----
// The same per-(row, token) arithmetic as sh_rows_job (bf16_group_chain over
// each group of 32 inputs, then run_sum, then the runs left to right), for a
// tile of up to SHT_T tokens whose inputs are staged once in LDS and read by
// every row of the block, so a weight row is read once per tile instead of
// once per token pair.  Block of SHT_NT threads: thread (row slot ro, group g)
// with Gq = run_lanes(G) lanes per row and RPS = SHT_NT / Gq row slots; slot
// ro takes rows ro*NS .. ro*NS+NS-1 (NS = ceil(NR / RPS)), in batches of SHT_R
// rows.  LDS: the tile xt[t][g][8 chunks of 16 bytes],
// chunk c of group g stored at chunk c ^ (g & 7) (the lanes of a wave read
// consecutive groups), then runs[NR][SHT_T][NC].
#define SHT_T 8
#ifndef SH_TILE_MARK
#define SH_TILE_MARK(i)
#endif
#define SHT_NT 512
#define SHT_R 4               // rows per batch (one LDS read of a token's inputs serves all)
#define SHT_XB 8              // tile chunks per thread in flight while staging
__host__ __device__ inline size_t sh_tile_lds(int K, int NR) {
    const int G = K / SH_RG, NC = G < SH_CHG ? 1 : run_lanes(G) / SH_CHG;
    return ((size_t)SHT_T * G * SH_RG + (size_t)NR * SHT_T * NC) * 4;
}
template <class RowPtr, class Emit>
__device__ __forceinline__ void sh_tile_job(RowPtr rowp, int NR, int K, const float *__restrict__ x, int tok0, int nt,
                                            Emit emit, float *lds) {
    const int G = K / SH_RG, Gq = run_lanes(G);
    const int CH = Gq < SH_CHG ? Gq : SH_CHG, NC = Gq / CH;
    const bool c16 = G % SH_CHG == 0;              // no padding lanes (else they add zero terms)
    const int tid = threadIdx.x;
    const int RPS = SHT_NT / Gq, NS = (NR + RPS - 1) / RPS;
    const int ro = tid / Gq, gq = tid - ro * Gq, c = gq / CH;
    const bool worker = ro < RPS, lead = worker && (gq & (CH - 1)) == 0, gv = gq < G;
    const int g = gv ? gq : G - 1;
    const int roc = worker ? ro : 0;
    float *xt = lds, *runs = lds + (size_t)SHT_T * G * SH_RG;
    auto row_of = [&](int s) { const int lr = roc * NS + s; return lr < NR ? lr : NR - 1; };
    auto wld = [&](int s, sw_u32x4 *w) {
        const sw_u32x4 *wp = (const sw_u32x4 *)(rowp(row_of(s)) + g * SH_RG);
#pragma unroll
        for (int q = 0; q < 4; q++) w[q] = wp[q];
    };
    // rows in batches of SHT_R: every 16-byte chunk of a token's inputs read from LDS
    // feeds the chains of SHT_R rows (each chain still in input order)
    const int NB = (NS + SHT_R - 1) / SHT_R;
    sw_u32x4 w[SHT_R][4];
#pragma unroll
    for (int r = 0; r < SHT_R; r++) wld(r < NS ? r : NS - 1, w[r]);
    // the tile: nt tokens x G groups x 8 chunks of 16 bytes; per token row, chunk r
    // by thread r mod SHT_NT, SHT_XB chunks per thread in flight (rows past the tile
    // load the tile's last row and are not stored)
    const int rch = G * 8;
    for (int t0 = 0; t0 < nt; t0 += SHT_XB) {
        for (int r = tid; r < rch; r += SHT_NT) {
            const int gg = r >> 3, cc = r & 7;
            sw_f32x4 v[SHT_XB];
#pragma unroll
            for (int u = 0; u < SHT_XB; u++)
                v[u] = *(const sw_f32x4 *)(x + (int64_t)(tok0 + min(t0 + u, nt - 1)) * K + gg * SH_RG + 4 * cc);
#pragma unroll
            for (int u = 0; u < SHT_XB; u++)
                if (t0 + u < nt) *(sw_f32x4 *)(xt + (((t0 + u) * G + gg) * 8 + (cc ^ (gg & 7))) * 4) = v[u];
        }
    }
    __syncthreads();
    SH_TILE_MARK(1);
    const float *xg = xt + (size_t)g * 8 * 4;
    const int sw = g & 7;
    for (int b = 0; b < NB; b++) {
        // this batch's weights widened once for the tile's tokens; the next batch's in flight
        float wf[SHT_R][SH_RG];
#pragma unroll
        for (int r = 0; r < SHT_R; r++)
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                const sw_u32x4 v = w[r][qq];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    wf[r][8 * qq + 2 * j] = bf16lo(v[j]);
                    wf[r][8 * qq + 2 * j + 1] = bf16hi(v[j]);
                }
            }
        if (b + 1 < NB) {
#pragma unroll
            for (int r = 0; r < SHT_R; r++) wld(min((b + 1) * SHT_R + r, NS - 1), w[r]);
        }
        for (int t = 0; t < nt; t++) {                 // uniform over the block
            const float *xr = xg + (size_t)t * G * 8 * 4;
            float q[SHT_R];
#pragma unroll
            for (int r = 0; r < SHT_R; r++) q[r] = 0.f;
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {           // bf16_group_chain, inputs from the tile
                const sw_f32x4 xa = *(const sw_f32x4 *)(xr + ((2 * qq) ^ sw) * 4);
                const sw_f32x4 xb = *(const sw_f32x4 *)(xr + ((2 * qq + 1) ^ sw) * 4);
#pragma unroll
                for (int r = 0; r < SHT_R; r++) {
                    const float *wr = wf[r] + 8 * qq;
                    q[r] = __builtin_fmaf(wr[0], xa.x, q[r]);
                    q[r] = __builtin_fmaf(wr[1], xa.y, q[r]);
                    q[r] = __builtin_fmaf(wr[2], xa.z, q[r]);
                    q[r] = __builtin_fmaf(wr[3], xa.w, q[r]);
                    q[r] = __builtin_fmaf(wr[4], xb.x, q[r]);
                    q[r] = __builtin_fmaf(wr[5], xb.y, q[r]);
                    q[r] = __builtin_fmaf(wr[6], xb.z, q[r]);
                    q[r] = __builtin_fmaf(wr[7], xb.w, q[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < SHT_R; r++) {
                const int s = b * SHT_R + r, lr = roc * NS + s;
                const float p = c16 ? run_sum16(q[r]) : run_sum(gv ? q[r] : 0.f, CH);
                if (lead && s < NS && lr < NR) runs[(lr * SHT_T + t) * NC + c] = p;
            }
        }
        SH_TILE_MARK(2 + (b < 3 ? b : 3));
    }
    __syncthreads();
    for (int it = tid; it < NR * nt; it += SHT_NT) {
        const int lr = it / nt, t = it - lr * nt;
        const float *rr = runs + (lr * SHT_T + t) * NC;
        float y = rr[0];
        for (int cc = 1; cc < NC; cc++) y = y + rr[cc];
        emit(lr, t, y);
    }
}
// gate_up: SHT_GLU_O outputs i per block (gate rows, then up rows), a tile of tokens
#define SHT_GLU_O 16
// down: SHT_DN_O output rows per block
#define SHT_DN_O 64

#endif
