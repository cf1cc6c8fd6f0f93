// sw_router.h -- the router GEMV block (exact 16-lane FMA-chain contract),
// usable alone or as part of a fused stage kernel.
#ifndef SW_ROUTER_H
#define SW_ROUTER_H
#include "sw_hip.h"
#include "sw_libm.h"
#include "sw_gate.h"
#include "sw_shared.h"

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
// in flight in a single token's blocks (all of a D = 4096 bf16 chain, issued
// before the block's other traffic), RT_PF_B in a batch's; a bf16 weight widens
// exactly to f32; x is
// staged transposed in LDS once per block, so chain j reads x[16m + j] as
// xt[j][m]; the tree is four shuffles within each 16-lane row.  The chain is
// M = D/16 dependent fmas per lane, the critical path of the routing.
#define RT_PF 32
// the slices in flight of a batch's router blocks (not ONE): 16 keeps their kernels within
// 120-138 VGPRs, 3-4 waves per SIMD instead of 2 (B=64's routing launch with the shared
// expert's blocks 41.5 -> 33.1 us, B=128 78.8 -> 58.2; B=2 unchanged)
#define RT_PF_B 16
#define RT_XB 8           // x float4 loads per thread: D <= 4 * RT_XB * threads
struct RouterArgs {
    const void *Wc;            // router in the streaming order (k_chain_major)
    const float *x;            // [S, D]
    int D, E;
    const float *lbias;        // logit bias or null
    float *logits;             // [S, E]
    int act;
    float *scores;             // [S, E] sigmoid / softplus scores (act 0, 2) or null
    sw_u32x4 *xl;              // dot8 limbs of x, or null
    float *xs;
    uint16_t *xp;              // the bf16 parts of x for the shared expert's MFMA (sw_shared.h), or null
    const float *nw;           // RMSNorm weight [D]: x is a raw row, normalised as it is staged
    float eps;                 //   (rms_inv_block, then x * inv * w); null: x is used as given
    float *xn;                 // with nw: the normalised rows [S, D], written by each token's first block
};
// experts per router block of nt threads: 4 (ONE: wave 0 runs the chains,
// the other waves stage x -- the router spread over as many CUs as there are
// groups of 4 experts) or 4 per wave
__host__ __device__ inline int router_epb(int one, int nt) { return one ? 4 : 4 * (nt / 64); }
// ONE while the blocks of S tokens stay within 256
__host__ inline int router_one(int S, int E) { return (int64_t)S * ((E + 3) / 4) <= 256; }

// block bx (of nbx per token) of token s; smem: the dynamic LDS (router_lds
// bytes)
// NORM: x is a raw row, normalised as it is staged (R.nw, R.eps; R.xn written)
template <int BF16, int ONE, int NORM = 0>
__device__ __forceinline__ void router_block(const RouterArgs &R, int bx, int s, int nbx, float *smem) {
    constexpr int P = BF16 ? 8 : 4;
    __shared__ uint64_t tab[32];                     // expf table for the sigmoid / softplus scores
    const float *__restrict__ x = R.x;
    const int D = R.D, E = R.E, act = R.act;
    const int nt = blockDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    const int M = D / 16, ML = M + 4, NQ = M / P;
    const int j = lane & 15;
    const bool chain = ONE ? wave == 0 : true;        // uniform per wave
    const int eg = ONE ? bx : bx * nw + wave, e = eg * 4 + (lane >> 4);
    const bool valid = chain && e < E;
    // slice q of this lane: byte voff + 1024 q of the router (groups past the last: clamp)
    const int ng4 = (E + 3) / 4;
    const int egc = eg < ng4 ? eg : ng4 - 1;
    const sw_rsrc rw = sw_make_rsrc(R.Wc, (uint32_t)ng4 * 4u * (uint32_t)D * (BF16 ? 2u : 4u));
    const uint32_t voff = ((uint32_t)egc * NQ * 64 + lane) * 16;
    auto slice = [&](int q) { return sw_ld16(rw, voff, (uint32_t)min(q, NQ - 1) * 1024u); };
    float *xt = smem;                                 // [16][ML]
    const float *xr = x + (int64_t)s * D;
    const int nx4 = D / 4;
    // x staged transposed into LDS, xt[k % 16][k / 16], by xs threads from thread x0: one pass
    // of unconditional loads (clamped; D <= 4 * RT_XB * xs), so no loop or branch join at
    // which the wait counts would drain slices in flight
    const int xs = ONE ? nt - 64 : nt, x0 = ONE ? 64 : 0, xt_id = tid - x0;
    // (NORM: the norm weights come with x, the staged value is x * inv * w, and the first
    // block of the token also writes it to R.xn)
    const float *__restrict__ nwr = R.nw;
    auto stage_x_load = [&](sw_f32x4 *xv, sw_f32x4 *wv) {
#pragma unroll
        for (int u = 0; u < RT_XB; u++) xv[u] = *(const sw_f32x4 *)(xr + 4 * min(u * xs + xt_id, nx4 - 1));
        if constexpr (NORM) {
#pragma unroll
            for (int u = 0; u < RT_XB; u++) wv[u] = *(const sw_f32x4 *)(nwr + 4 * min(u * xs + xt_id, nx4 - 1));
        }
    };
    auto stage_x_store = [&](sw_f32x4 *xv, const sw_f32x4 *wv, float inv) {
        float *xnr = NORM && R.xn && bx == 0 ? R.xn + (int64_t)s * D : nullptr;
#pragma unroll
        for (int u = 0; u < RT_XB; u++) {
            const int i4 = u * xs + xt_id;
            if (i4 < nx4) {
                if constexpr (NORM) {
#pragma unroll
                    for (int c = 0; c < 4; c++) xv[u][c] = xv[u][c] * inv * wv[u][c];
                    if (xnr) *(sw_f32x4 *)(xnr + 4 * i4) = xv[u];
                }
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int k = 4 * i4 + c;
                    xt[(k & 15) * ML + (k >> 4)] = xv[u][c];
                }
            }
        }
    };
    __shared__ double rn_part[RN_NT / 64];
    // the token's RMSNorm factor (every thread calls: the function holds a block barrier)
    auto norm_inv = [&]() {
        if constexpr (NORM) {
            float v[RN_CH];
            return rms_inv_block(xr, D, R.eps, rn_part, v);
        } else {
            return 1.f;
        }
    };
    const uint64_t tabv = sw_exp2f_tab[lane & 31];  // stored after the chain, where the scores need it
    constexpr int PFR = ONE ? RT_PF : RT_PF_B;       // slices in flight per lane
    sw_u32x4 ring[PFR];
    if constexpr (ONE && NORM) {
        sw_f32x4 xv[RT_XB], wv[RT_XB];
        if (wave == 0) {
#pragma unroll
            for (int u = 0; u < PFR; u++) ring[u] = slice(u);
        } else {
            stage_x_load(xv, wv);
        }
        const float inv = norm_inv();
        if (wave != 0) stage_x_store(xv, wv, inv);
    } else if constexpr (ONE) {
        if (wave == 0) {
#pragma unroll
            for (int u = 0; u < PFR; u++) ring[u] = slice(u);
        } else {
            sw_f32x4 xv[RT_XB], wv[RT_XB];
            stage_x_load(xv, wv);
            stage_x_store(xv, wv, 1.f);
        }
    } else {
        sw_f32x4 xv[RT_XB], wv[RT_XB];
        stage_x_load(xv, wv);                         // x first, then every slice of the ring
#pragma unroll
        for (int u = 0; u < PFR; u++) ring[u] = slice(u);
        const float inv = norm_inv();
        stage_x_store(xv, wv, inv);
    }
    __syncthreads();
    const float *xj = xt + j * ML;
    float acc = 0.f;
    // x of the slices two ahead is read from LDS while this slice's fmas run (the chain
    // would otherwise wait out an LDS latency per slice): xn[0] holds slice q + 1's P
    // values, xn[1] slice q + 2's
    constexpr int XV = BF16 ? 2 : 1;                  // float4 of x per slice
    sw_f32x4 xn[2][XV];
    auto xload = [&](int q, sw_f32x4 *dst) {
        const int qc = min(q, NQ - 1);
#pragma unroll
        for (int v = 0; v < XV; v++) dst[v] = *(const sw_f32x4 *)(xj + P * qc + 4 * v);
    };
    auto chain4 = [&](int q, const sw_u32x4 &w) {
        sw_f32x4 xc[XV];
#pragma unroll
        for (int v = 0; v < XV; v++) { xc[v] = xn[0][v]; xn[0][v] = xn[1][v]; }
        xload(q + 2, xn[1]);
        if constexpr (BF16) {
            const sw_f32x4 xa = xc[0], xb = xc[XV - 1];
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
            const sw_f32x4 xa = xc[0], wf = __builtin_bit_cast(sw_f32x4, w);
            acc = __builtin_fmaf(xa.x, wf.x, acc);
            acc = __builtin_fmaf(xa.y, wf.y, acc);
            acc = __builtin_fmaf(xa.z, wf.z, acc);
            acc = __builtin_fmaf(xa.w, wf.w, acc);
        }
    };
    if (ONE && !chain && R.xl) {                      // the limbs by the staging waves while wave 0 chains
        const int G = D / SW_RG, hw = (tid - 64) >> 5, nhw = 2 * (nw - 1);
        for (int g = bx * nhw + hw; g < G; g += nbx * nhw) {
            const int k = g * SW_RG + (tid & 31);
            limbs_group(xt[(k & 15) * ML + (k >> 4)], tid & 31, R.xl + ((int64_t)s * G + g) * SW_NL, R.xs + (int64_t)s * G + g);
        }
    }
    if (chain) {
        sw_f32x4 x0[XV];
        xload(0, x0);
        xload(1, xn[1]);
#pragma unroll
        for (int v = 0; v < XV; v++) xn[0][v] = x0[v];
        // full rounds with unconditional refills (a refill past the end re-reads the last
        // slice), then the last round without: no ring rotation, loads stay in flight
        int q0 = 0;
        for (; q0 + PFR < NQ; q0 += PFR) {
#pragma unroll
            for (int u = 0; u < PFR; u++) {         // the slot is consumed before its refill
                chain4(q0 + u, ring[u]);
                ring[u] = slice(q0 + u + PFR);
                __builtin_amdgcn_sched_barrier(0);    // keep the refill here, not sunk to the round's end
            }
        }
#pragma unroll
        for (int u = 0; u < PFR; u++)
            if (q0 + u < NQ) chain4(q0 + u, ring[u]);
    }
    tab[lane & 31] = tabv;                            // every wave writes the whole table (equal values)
    wave_sync();
    float v = row_reduce16(acc);
    if (j == 0 && valid) {
        if (R.lbias) v = v + R.lbias[e];
        R.logits[(int64_t)s * E + e] = v;
        if (!sw_act_softmax(act) && R.scores)
            R.scores[(int64_t)s * E + e] = act == 2   ? sw_softplus_ref_t(v, tab)
                                           : act == 5 ? sw_sqrt_rn(sw_softplus_ref_t(v, tab))   // c/deepseek.c:854
                                                      : sw_sigmoid_ref_t(v, tab);
    }
    if (R.xp && bx == 0) {                            // the token's bf16 parts, by its first block
        for (int c = tid; c < D / 8; c += nt) {
            const sw_f32x4 *xv = (const sw_f32x4 *)(xr + 8 * c);
            sw_u32x4 p0, p1, p2;
            sh_split8(xv[0], xv[1], p0, p1, p2);
            uint16_t *dst = R.xp + (int64_t)s * D * 3 + (c >> 2) * 3 * SH_RG + (c & 3) * 8;
            *(sw_u32x4 *)dst = p0;
            *(sw_u32x4 *)(dst + SH_RG) = p1;
            *(sw_u32x4 *)(dst + 2 * SH_RG) = p2;
        }
    }
    if (!ONE && R.xl) {                               // the token's dot8 limbs, half a wave per group, from xt
        const int G = D / SW_RG;
        for (int g = bx * 2 * nw + (tid >> 5); g < G; g += nbx * 2 * nw) {
            const int k = g * SW_RG + (tid & 31);
            limbs_group(xt[(k & 15) * ML + (k >> 4)], tid & 31, R.xl + ((int64_t)s * G + g) * SW_NL, R.xs + (int64_t)s * G + g);
        }
    }
}
__host__ inline size_t router_lds(int D) { return (size_t)16 * (D / 16 + 4) * 4; }

// The same logits and scores for a tile of TT tokens per pass over the
// weights: wave w of block (bx, by) runs the 16 chains of each of the 4 GPW
// experts of groups GPW (bx NW + w) .. + GPW - 1, for tokens TT by .. TT by +
// TT - 1 (lane 16 q + j keeps chain j of expert q of each of its groups, one
// accumulator per group and token), so a router slice is loaded once per TT
// tokens instead of once per token, and each x value read from LDS feeds
// the chains of GPW experts (LDS reads are the limit: TT x values of 4 bytes
// per weight element and group).  x goes through LDS in chunks of 256 inputs
// (16 elements of every chain), staged transposed, xt[t][j][m] = x[t][256 c +
// 16 m + j] (rows of 20 floats: the 16 lanes of a row read 16 bytes each from
// distinct banks); the next chunk's x is loaded into registers while this one
// is used, and the slices of RT_TCH chunks of each lane's chains are in
// flight.  Every chain is the same fma sequence as router_block's, so the
// results are the same bits.
#define RT_CK 256
#define RT_XS 20
#define RT_TCH 3           // chunks of router slices in flight
template <int BF16, int TT, int NW, int GPW>
__device__ __forceinline__ void router_tile_block(const RouterArgs &R, int S, int bx, int by) {
    constexpr int P = BF16 ? 8 : 4, SPC = 16 / P, NTH = 64 * NW;
    constexpr int XR4 = TT * RT_CK / 4 / NTH;          // float4 of x per thread per chunk
    static_assert(XR4 >= 1 && XR4 * 4 * NTH == TT * RT_CK, "x chunk splits evenly over the block");
    __shared__ __align__(16) float xt[TT * 16 * RT_XS];
    __shared__ uint64_t tab[32];
    const int D = R.D, E = R.E, act = R.act;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15;
    const int eg0 = (bx * NW + wave) * GPW;            // the wave's first group of 4 experts
    const int ng4 = (E + 3) / 4;
    const int s0 = by * TT, nt = min(TT, S - s0);
    const int M = D / 16, NQ = M / P, NCH = D / RT_CK;
    const sw_rsrc rw = sw_make_rsrc(R.Wc, (uint32_t)ng4 * 4u * (uint32_t)D * (BF16 ? 2u : 4u));
    uint32_t voff[GPW];                                // groups past the last clamp to it
#pragma unroll
    for (int g = 0; g < GPW; g++) voff[g] = ((uint32_t)min(eg0 + g, ng4 - 1) * NQ * 64 + lane) * 16;
    auto slice = [&](int g, int q) { return sw_ld16(rw, voff[g], (uint32_t)min(q, NQ - 1) * 1024u); };
    // x float4 f of a chunk: token f / 64, inputs 4 (f % 64) .. +3 of the chunk
    auto xload = [&](int c, sw_f32x4 *xr) {
#pragma unroll
        for (int u = 0; u < XR4; u++) {
            const int f = u * NTH + tid, t = f >> 6, k4 = f & 63;
            const int tok = s0 + (t < nt ? t : nt - 1);
            xr[u] = *(const sw_f32x4 *)(R.x + (int64_t)tok * D + c * RT_CK + 4 * k4);
        }
    };
    auto xstore = [&](const sw_f32x4 *xr) {
#pragma unroll
        for (int u = 0; u < XR4; u++) {
            const int f = u * NTH + tid, t = f >> 6, k4 = f & 63;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int k = 4 * k4 + i;
                xt[(t * 16 + (k & 15)) * RT_XS + (k >> 4)] = xr[u][i];
            }
        }
    };
    float acc[GPW][TT];
#pragma unroll
    for (int g = 0; g < GPW; g++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[g][t] = 0.f;
    // the slices of chunks c .. c + RT_TCH - 1 in flight (RT_TCH chunks ahead of their use)
    sw_u32x4 wc[RT_TCH][GPW][SPC];
#pragma unroll
    for (int u = 0; u < RT_TCH; u++)
#pragma unroll
        for (int g = 0; g < GPW; g++)
#pragma unroll
            for (int sl = 0; sl < SPC; sl++) wc[u][g][sl] = slice(g, u * SPC + sl);
    sw_f32x4 xr[XR4];
    xload(0, xr);
    // element p of slice sl of the chunk against the tile's tokens: the slices widened once,
    // then each token's x read from LDS once for the chains of every group (four tokens at a
    // time, so the reads in flight stay few)
    auto use = [&](int sl, const sw_u32x4 (&w)[GPW]) {
        const float *xj = xt + j * RT_XS + sl * P;
        float wf[GPW][P];
#pragma unroll
        for (int g = 0; g < GPW; g++) {
            if constexpr (BF16) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    wf[g][2 * q] = __builtin_bit_cast(float, w[g][q] << 16);
                    wf[g][2 * q + 1] = __builtin_bit_cast(float, w[g][q] & 0xFFFF0000u);
                }
            } else {
                // the whole vector is cast (a bit_cast of one element lvalue reads element 0)
                const sw_f32x4 wv = __builtin_bit_cast(sw_f32x4, w[g]);
#pragma unroll
                for (int q = 0; q < 4; q++) wf[g][q] = wv[q];
            }
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float *xp = xj + t * 16 * RT_XS;
#pragma unroll
            for (int h = 0; h < P / 4; h++) {
                const sw_f32x4 xa = *(const sw_f32x4 *)(xp + 4 * h);
#pragma unroll
                for (int g = 0; g < GPW; g++) {
                    acc[g][t] = __builtin_fmaf(xa.x, wf[g][4 * h], acc[g][t]);
                    acc[g][t] = __builtin_fmaf(xa.y, wf[g][4 * h + 1], acc[g][t]);
                    acc[g][t] = __builtin_fmaf(xa.z, wf[g][4 * h + 2], acc[g][t]);
                    acc[g][t] = __builtin_fmaf(xa.w, wf[g][4 * h + 3], acc[g][t]);
                }
            }
            if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
    };
    for (int c = 0; c < NCH; c++) {
        __syncthreads();                              // the previous chunk's reads are done
        xstore(xr);
        xload(min(c + 1, NCH - 1), xr);
        __syncthreads();
#pragma unroll
        for (int sl = 0; sl < SPC; sl++) {
            sw_u32x4 w[GPW];
#pragma unroll
            for (int g = 0; g < GPW; g++) w[g] = wc[0][g][sl];
            use(sl, w);
        }
#pragma unroll
        for (int u = 0; u + 1 < RT_TCH; u++)
#pragma unroll
            for (int g = 0; g < GPW; g++)
#pragma unroll
                for (int sl = 0; sl < SPC; sl++) wc[u][g][sl] = wc[u + 1][g][sl];
#pragma unroll
        for (int g = 0; g < GPW; g++)
#pragma unroll
            for (int sl = 0; sl < SPC; sl++) wc[RT_TCH - 1][g][sl] = slice(g, (c + RT_TCH) * SPC + sl);
    }
    tab[lane & 31] = sw_exp2f_tab[lane & 31];         // every wave writes the whole table (equal values)
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GPW; g++) {
        const int e = (eg0 + g) * 4 + (lane >> 4);
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float v = row_reduce16(acc[g][t]);
            if (j == 0 && e < E && t < nt) {
                const int64_t s = s0 + t;
                if (R.lbias) v = v + R.lbias[e];
                R.logits[s * E + e] = v;
                if (!sw_act_softmax(act) && R.scores)
                    R.scores[s * E + e] = act == 2   ? sw_softplus_ref_t(v, tab)
                                          : act == 5 ? sw_sqrt_rn(sw_softplus_ref_t(v, tab))
                                                     : sw_sigmoid_ref_t(v, tab);
            }
        }
    }
}


#endif
