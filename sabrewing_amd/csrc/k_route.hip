// k_route.hip -- routing side of the MoE block on gfx950: activation planes,
// the router GEMV under the reference's exact FMA-chain contract, gate +
// top-k, the counting sort into expert groups, and the rank-order combine.
#include "sw_hip.h"
#include "sw_libm.h"

static int launch_err(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

// ------------------------------------------------------------ router ----
// Chain-major router copy: Wc[(e*16 + j)*M + m] = W[e*D + 16m + j], M = D/16,
// so lane j of expert e reads its FMA chain contiguously.
__global__ void k_chain_major(const void *__restrict__ W, int w_bf16, int E, int D, void *__restrict__ Wc) {
    const int M = D / 16;
    const int64_t n = (int64_t)E * D;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = i / D, k = i % D, m = k / 16, j = k % 16;
        const int64_t o = (e * 16 + j) * M + m;
        if (w_bf16) ((uint16_t *)Wc)[o] = ((const uint16_t *)W)[i];
        else ((float *)Wc)[o] = ((const float *)W)[i];
    }
}

int sw_launch_chain_major(hipStream_t st, const void *W, int w_bf16, int E, int D, void *Wc) {
    if (D % 128 || E <= 0) return -1;
    const int64_t n = (int64_t)E * D;
    hipLaunchKernelGGL(k_chain_major, dim3((unsigned)sw_imin64((n + 255) / 256, 8192)), dim3(256), 0, st, W, w_bf16, E, D, Wc);
    return launch_err();
}

// ------------------------------------------------------------ gate + top-k ----
// One wave finishes the routing of one token.  Gate with the reference's
// host expressions and glibc-exact expf/log1pf (c/moe_block.h:26;
// c/moe_math.h:54,68-72) -- sigmoid/softplus scores come from the logits
// kernel, softmax is done here -- then moe_topk (c/moe_arch.h:64-89): K passes
// of "largest score+bias among the unselected, valid only if > -1e30, ties to
// the lowest id", the all-invalid fallback to the lowest unselected id,
// weight = unbiased score, optional renormalisation summed in rank order
// (c/moe_block.h:121-122).  Block = one wave = one token.
//
// A pass is one wave-wide max over 64-bit keys (order-preserving bits of
// key + 0.0 above ~id, so a larger key wins and equal keys go to the lower
// id; invalid or taken experts are key 0), reduced with DPP row operations.
#define TK_MAXE 1024

template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    const uint32_t lo2 = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWMASK, 0xF, false);
    const uint32_t hi2 = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWMASK, 0xF, false);
    return ((uint64_t)hi2 << 32) | lo2;
}
__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// max over the 64 lanes, returned uniform
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max64(v, dpp64<0xB1, 0xF>(v));    // quad_perm [1,0,3,2]
    v = max64(v, dpp64<0x4E, 0xF>(v));    // quad_perm [2,3,0,1]
    v = max64(v, dpp64<0x141, 0xF>(v));   // row_half_mirror
    v = max64(v, dpp64<0x140, 0xF>(v));   // row_mirror
    v = max64(v, dpp64<0x142, 0xA>(v));   // row_bcast:15 into rows 1, 3
    v = max64(v, dpp64<0x143, 0xC>(v));   // row_bcast:31 into rows 2, 3
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t ord_f32(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f + 0.0f);   // -0 -> +0: equal keys tie on the id
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int TK_NPER>   // expert slots per lane: E <= 64 * TK_NPER
__global__ __launch_bounds__(64) void k_gate_topk(const float *__restrict__ logits, const float *__restrict__ scores,
                                                  int E, int K, int act, const float *__restrict__ bias, int use_bias,
                                                  int norm, int *__restrict__ sel_all, float *__restrict__ w_all) {
    __shared__ float sc[TK_MAXE];
    __shared__ float wk[64];
    __shared__ int sk[64];
    __shared__ uint64_t tab[32];
    __shared__ float inv;
    const int lane = threadIdx.x, s = blockIdx.x;
    const float *src = (act == 1 ? logits : scores) + (int64_t)s * E;
    float v[TK_NPER], b[TK_NPER];
    // every load of the token issued before any is used (clamped indices)
    if (act == 1 && lane < 32) tab[lane] = sw_exp2f_tab[lane];
    const bool hasb = use_bias && bias;
#pragma unroll
    for (int i = 0; i < TK_NPER; i++) {
        const int e = min(lane + 64 * i, E - 1);
        v[i] = src[e];
        b[i] = hasb ? bias[e] : 0.f;
    }
    if (act == 1) {                                   // softmax
        __syncthreads();
        float mx = -__builtin_inff();
        bool any = false;
#pragma unroll
        for (int i = 0; i < TK_NPER; i++) {
            const int e = lane + 64 * i;
            if (e < E && v[i] == v[i]) { mx = any ? fmaxf(mx, v[i]) : v[i]; any = true; }
        }
        for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float r0 = __shfl(v[0], 0);
        if (r0 != r0) mx = r0;                        // a NaN in slot 0 propagates, as in the scan
#pragma unroll
        for (int i = 0; i < TK_NPER; i++) {
            const int e = lane + 64 * i;
            if (e < E) sc[e] = sw_expf_t(v[i] - mx, tab);
        }
        __syncthreads();
        if (lane == 0) {
            double sum = 0.0;
            for (int e = 0; e < E; e++) sum += (double)sc[e];
            inv = (float)(1.0 / sum);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TK_NPER; i++) {
            const int e = lane + 64 * i;
            if (e < E) { v[i] = sc[e] * inv; sc[e] = v[i]; }
        }
    } else {
#pragma unroll
        for (int i = 0; i < TK_NPER; i++) {
            const int e = lane + 64 * i;
            if (e < E) sc[e] = v[i];
        }
    }
    __syncthreads();
    uint64_t kk[TK_NPER];
    bool fr[TK_NPER];
#pragma unroll
    for (int i = 0; i < TK_NPER; i++) {
        const int e = lane + 64 * i;
        const float key = v[i] + b[i];
        fr[i] = e < E;
        kk[i] = (e < E && key > -1e30f) ? (((uint64_t)ord_f32(key) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e)) : 0ull;
    }
    for (int a = 0; a < K; a++) {
        uint64_t m = kk[0];
#pragma unroll
        for (int i = 1; i < TK_NPER; i++) m = max64(m, kk[i]);
        m = wave_max_u64(m);
        int bi;
        if (m != 0ull) {
            bi = (int)(0xFFFFFFFFu - (uint32_t)m);
        } else {                                      // nothing valid left: the lowest unselected id
            bi = 0x7fffffff;
#pragma unroll
            for (int i = TK_NPER - 1; i >= 0; i--) {
                const unsigned long long bal = __ballot(fr[i]);
                if (bal) bi = 64 * i + __builtin_ctzll(bal);
            }
            if (bi >= E) bi = 0;
        }
        if ((bi & 63) == lane) {
#pragma unroll
            for (int i = 0; i < TK_NPER; i++)
                if (i == (bi >> 6)) { kk[i] = 0ull; fr[i] = false; }
        }
        if (lane == 0) { sk[a] = bi; wk[a] = sc[bi]; }
    }
    __syncthreads();
    if (lane == 0 && norm) {
        float sm = 0.f;
        for (int a = 0; a < K; a++) sm += wk[a];
        for (int a = 0; a < K; a++) wk[a] = wk[a] / sm;
    }
    __syncthreads();
    if (lane < K) { sel_all[(int64_t)s * K + lane] = sk[lane]; w_all[(int64_t)s * K + lane] = wk[lane]; }
}

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
template <int BF16>
__global__ __launch_bounds__(256) void k_router_logits(const void *__restrict__ Wc, const float *__restrict__ x, int D, int E,
                                                       const float *__restrict__ lbias, float *__restrict__ logits,
                                                       int act, float *__restrict__ scores) {
    extern __shared__ __align__(16) float smem[];
    __shared__ uint64_t tab[32];                     // expf table for the sigmoid / softplus scores
    constexpr int ESZ = BF16 ? 2 : 4;
    const int s = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int M = D / 16, ML = M + 4;
    const int MC = M < RT_MC ? M : RT_MC;            // chain elements per run
    const int runb = MC * ESZ, runs = runb + 16;      // run bytes, padded LDS stride
    float *xt = smem;                                 // [16][ML]
    char *wl = (char *)(smem + 16 * ML) + wave * 16 * runs;
    const int e = blockIdx.x * nw + wave;
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
        if (lbias) v = v + lbias[e];
        logits[(int64_t)s * E + e] = v;
        if (act != 1 && scores)
            scores[(int64_t)s * E + e] = (act == 2) ? sw_softplus_ref_t(v, tab) : sw_sigmoid_ref_t(v, tab);
    }
}

int sw_launch_router_topk(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                          const float *logit_bias, float *logits, float *scores, int K, int route_act,
                          const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w) {
    if (D % 128 || D > 16384 || E <= 0 || E > TK_MAXE || S <= 0 || K <= 0 || K > 64 || K > E) return -1;
    if (route_act < 0 || route_act > 2 || (sel && route_act != 1 && !scores)) return -1;
    const int M = D / 16, MC = M < RT_MC ? M : RT_MC;
    const size_t xb = (size_t)16 * (M + 4) * 4, wb = (size_t)16 * (MC * (w_bf16 ? 2 : 4) + 16);
    // one expert per wave; several per block once there are enough tokens to fill the chip
    int nw = S >= 4 ? 4 : 1;
    while (nw > 1 && xb + nw * wb > 65536) nw >>= 1;
    if (xb + nw * wb > 65536) return -1;
    dim3 grid((unsigned)((E + nw - 1) / nw), (unsigned)S);
    const size_t lds = xb + nw * wb;
    if (w_bf16)
        hipLaunchKernelGGL(k_router_logits<1>, grid, dim3(64 * nw), lds, st, Wc, x, D, E, logit_bias, logits, route_act, scores);
    else
        hipLaunchKernelGGL(k_router_logits<0>, grid, dim3(64 * nw), lds, st, Wc, x, D, E, logit_bias, logits, route_act, scores);
    if (launch_err()) return -1;
    if (!sel) return 0;                              // logits only
    const int nper = (E + 63) / 64;
#define SW_GATE(NP) hipLaunchKernelGGL(k_gate_topk<NP>, dim3((unsigned)S), dim3(64), 0, st, logits, scores, E, K, route_act, \
                                       corr_bias, use_corr_bias, norm_topk, sel, w)
    if (nper <= 1) SW_GATE(1);
    else if (nper <= 2) SW_GATE(2);
    else if (nper <= 4) SW_GATE(4);
    else if (nper <= 8) SW_GATE(8);
    else SW_GATE(16);
#undef SW_GATE
    return launch_err();
}

// ------------------------------------------------------------ bucketing ----
// The counting sort of lag_moe_group (c/laguna.c:708-727) on the device:
// groups in ascending expert id, packed rows stable in (token, rank) order.
// One block of 1024 threads; pairs are taken 1024 at a time in order, and a
// pair's rank among earlier pairs of its expert comes from per-wave ballot
// match masks plus per-wave counts of the earlier waves.
#define BK_THREADS 1024
#define BK_MAXE 512
__global__ __launch_bounds__(BK_THREADS) void k_bucket(const int *__restrict__ sel, int T, int K, int E,
                                                       int *__restrict__ gexp, int *__restrict__ gbeg,
                                                       int *__restrict__ gcnt, int *__restrict__ Gout,
                                                       int *__restrict__ grow, int *__restrict__ rowof) {
    __shared__ int cnt[BK_MAXE], run[BK_MAXE], sa[BK_MAXE], sb[BK_MAXE];
    __shared__ int wcnt[BK_THREADS / 64][BK_MAXE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < E; i += BK_THREADS) {
        cnt[i] = 0;
        for (int w = 0; w < BK_THREADS / 64; w++) wcnt[w][i] = 0;
    }
    __syncthreads();
    for (int p = tid; p < T; p += BK_THREADS) atomicAdd(&cnt[sel[p]], 1);
    __syncthreads();
    // exclusive scans of cnt (packed offsets) and of cnt > 0 (group index)
    for (int i = tid; i < E; i += BK_THREADS) { sa[i] = cnt[i]; sb[i] = cnt[i] > 0; }
    __syncthreads();
    for (int off = 1; off < E; off <<= 1) {
        int va = 0, vb = 0;
        if (tid < E && tid >= off) { va = sa[tid - off]; vb = sb[tid - off]; }
        __syncthreads();
        if (tid < E && tid >= off) { sa[tid] += va; sb[tid] += vb; }
        __syncthreads();
    }
    if (tid < E) {
        const int c = cnt[tid];
        const int offx = sa[tid] - c, gi = sb[tid] - (c > 0);
        run[tid] = offx;
        if (c > 0) { gexp[gi] = tid; gbeg[gi] = offx; gcnt[gi] = c; }
        if (tid == E - 1) *Gout = sb[tid];
    }
    __syncthreads();
    int nbits = 0;
    while ((1 << nbits) < E) nbits++;
    const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < T; base += BK_THREADS) {
        const int p = base + tid;
        const bool act = p < T;
        const int e = act ? sel[p] : 0;
        unsigned long long peers = __ballot(act);
        for (int b = 0; b < nbits; b++) {
            const unsigned long long m = __ballot(act && ((e >> b) & 1));
            peers &= ((e >> b) & 1) ? m : ~m;
        }
        const int rank = __popcll(peers & lt);
        if (act && rank == 0) wcnt[wave][e] = __popcll(peers);
        __syncthreads();
        if (act) {
            int pre = 0;
            for (int w = 0; w < wave; w++) pre += wcnt[w][e];
            const int slot = run[e] + pre + rank;
            grow[slot] = p / K;
            rowof[p] = slot;
        }
        __syncthreads();
        for (int i = tid; i < E; i += BK_THREADS) {
            int tot = 0;
            for (int w = 0; w < BK_THREADS / 64; w++) { tot += wcnt[w][i]; wcnt[w][i] = 0; }
            run[i] += tot;
        }
        __syncthreads();
    }
}

int sw_launch_bucket(hipStream_t st, const int *sel, int S, int K, int E, int *gexp, int *gbeg,
                     int *gcnt, int *G, int *grow, int *rowof) {
    if (E <= 0 || E > BK_MAXE || S <= 0 || K <= 0) return -1;
    hipLaunchKernelGGL(k_bucket, dim3(1), dim3(BK_THREADS), 0, st, sel, S * K, K, E, gexp, gbeg, gcnt, G, grow, rowof);
    return launch_err();
}

// ------------------------------------------------------------ combine ----
// out[s,d] (+)= (sum_a w[s,a] * slots[rowof[s,a], d]) * route_scale (+ shared[s,d])
// The sum runs in rank order from 0 with one fused multiply-add per rank,
// the operation sequence of moe_block's `acc[i] += w[a] * scr[i]` as the
// reference build compiles it (c/moe_block.h:124-142; c/laguna.c:761-782).
__global__ void k_combine(const float *__restrict__ slots, const int *__restrict__ rowof, const float *__restrict__ w,
                          int S, int K, int D, float route_scale, const float *__restrict__ shared,
                          float *__restrict__ out, int accumulate) {
    const int64_t n4 = (int64_t)S * (D / 4);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t s = i / (D / 4), d = (i % (D / 4)) * 4;
        sw_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int a0 = 0; a0 < K; a0 += 8) {
            sw_f32x4 v[8];
            float wa[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (a0 + u < K) {
                    wa[u] = w[s * K + a0 + u];
                    v[u] = *(const sw_f32x4 *)(slots + (int64_t)rowof[s * K + a0 + u] * D + d);
                }
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (a0 + u < K)
#pragma unroll
                    for (int c = 0; c < 4; c++) acc[c] = __builtin_fmaf(wa[u], v[u][c], acc[c]);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] = acc[c] * route_scale;
        if (shared) {
            const sw_f32x4 sh = *(const sw_f32x4 *)(shared + s * D + d);
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = acc[c] + sh[c];
        }
        sw_f32x4 *o = (sw_f32x4 *)(out + s * D + d);
        if (accumulate) {
            sw_f32x4 cur = *o;
#pragma unroll
            for (int c = 0; c < 4; c++) cur[c] = cur[c] + acc[c];
            *o = cur;
        } else {
            *o = acc;
        }
    }
}

int sw_launch_combine(hipStream_t st, const float *slots, const int *rowof, const float *w, int S, int K, int D,
                      float route_scale, const float *shared, float *out, int accumulate) {
    if (D % 4 || S <= 0) return -1;
    const int64_t n4 = (int64_t)S * (D / 4);
    hipLaunchKernelGGL(k_combine, dim3((unsigned)sw_imin64((n4 + 255) / 256, 4096)), dim3(256), 0, st, slots, rowof, w,
                       S, K, D, route_scale, shared, out, accumulate);
    return launch_err();
}

// ------------------------------------------------------------ self test ----
// MFMA lane-layout probe: A[i][k] = 32 i + k, B[k][j] = (k == j), so
// C[i][j] = 32 i + j under the layout in sw_hip.h; plus glibc-exact libm on
// host-chosen inputs.  out: [0,256) f16 MFMA C per lane (4 each), [256,512)
// bf16 MFMA, [512, 512+n) sw_expf(xin), [512+n, 512+2n) sw_log1pf(xin).
__global__ void k_selftest_mfma(float *out) {
    const int l = threadIdx.x;
    sw_half8 a, b;
    sw_bf16x8 ab, bb;
    for (int h = 0; h < 8; h++) {
        const int k = 8 * (l >> 4) + h;
        const int i = l & 15;
        a[h] = (_Float16)(float)(32 * i + k);
        b[h] = (_Float16)(k == (l & 15) ? 1.0f : 0.0f);
        ab[h] = (__bf16)(float)(i * 2 + (k & 1));
        bb[h] = (__bf16)(k == (l & 15) ? 1.0f : 0.0f);
    }
    sw_f32x4 c = {0.f, 0.f, 0.f, 0.f}, c2 = {0.f, 0.f, 0.f, 0.f};
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, bb, c2, 0, 0, 0);
    for (int j = 0; j < 4; j++) { out[l * 4 + j] = c[j]; out[256 + l * 4 + j] = c2[j]; }
}

__global__ void k_selftest_libm(float *out, const float *xin, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        out[512 + i] = sw_expf(xin[i]);
        out[512 + n + i] = sw_log1pf(xin[i]);
    }
}

int sw_launch_selftest(hipStream_t st, float *out, const float *xin, int n) {
    hipLaunchKernelGGL(k_selftest_mfma, dim3(1), dim3(64), 0, st, out);
    if (n > 0) hipLaunchKernelGGL(k_selftest_libm, dim3((unsigned)sw_imin64((n + 255) / 256, 4096)), dim3(256), 0, st, out, xin, n);
    return launch_err();
}
