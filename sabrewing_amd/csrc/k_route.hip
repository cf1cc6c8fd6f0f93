// k_route.hip -- routing side of the MoE block on gfx950: activation planes,
// the router GEMV under the reference's exact FMA-chain contract, gate +
// top-k, the counting sort into expert groups, and the rank-order combine.
#include "sw_hip.h"
#include "sw_libm.h"

static int launch_err(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

// ------------------------------------------------------------ activations ----
// x f32 [S,D] -> f16 planes [2S,D]: row 2s = RN(x), row 2s+1 = RN(x - RN(x)),
// 8-blocks permuted 0,4,1,5,2,6,3,7 (the int4 MFMA B-fragment order).
__global__ void k_prep_f16(const float *__restrict__ x, int S, int D, _Float16 *__restrict__ p) {
    const int64_t nb = (int64_t)S * (D / 8);
    for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const int64_t s = b / (D / 8), k0 = (b % (D / 8)) * 8;
        const sw_f32x4 v0 = *(const sw_f32x4 *)(x + s * D + k0);
        const sw_f32x4 v1 = *(const sw_f32x4 *)(x + s * D + k0 + 4);
        const float v[8] = {v0.x, v1.x, v0.y, v1.y, v0.z, v1.z, v0.w, v1.w};   // 0,4,1,5,2,6,3,7
        sw_half8 hi, lo;
#pragma unroll
        for (int h = 0; h < 8; h++) {
            const _Float16 a = (_Float16)v[h];
            hi[h] = a;
            lo[h] = (_Float16)(v[h] - (float)a);
        }
        *(sw_half8 *)(p + (2 * s) * D + k0) = hi;
        *(sw_half8 *)(p + (2 * s + 1) * D + k0) = lo;
    }
}

__device__ __forceinline__ uint16_t bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// x f32 [S,D] -> bf16 planes [2S,D] (natural order)
__global__ void k_prep_bf16(const float *__restrict__ x, int S, int D, uint16_t *__restrict__ p) {
    const int64_t n = (int64_t)S * D;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t s = i / D, k = i % D;
        const float v = x[i];
        const uint16_t hi = bf16_rne(v);
        const uint16_t lo = bf16_rne(v - __builtin_bit_cast(float, (uint32_t)hi << 16));
        p[(2 * s) * D + k] = hi;
        p[(2 * s + 1) * D + k] = lo;
    }
}

int sw_launch_prep_f16(hipStream_t st, const float *x, int S, int D, _Float16 *planes) {
    if (D % 8 || S <= 0) return -1;
    const int64_t nb = (int64_t)S * (D / 8);
    const unsigned grid = (unsigned)sw_imin64((nb + 255) / 256, 4096);
    hipLaunchKernelGGL(k_prep_f16, dim3(grid), dim3(256), 0, st, x, S, D, planes);
    return launch_err();
}

int sw_launch_prep_bf16(hipStream_t st, const float *x, int S, int D, uint16_t *planes) {
    if (S <= 0) return -1;
    const int64_t n = (int64_t)S * D;
    const unsigned grid = (unsigned)sw_imin64((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_prep_bf16, dim3(grid), dim3(256), 0, st, x, S, D, planes);
    return launch_err();
}

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

// logits[s,e] = sum_i x[s,i] W[e,i] under the contract of the reference's
// AVX-512 router (c/moe_matmul.h:25-43; bf16 weights c/moe_matmul.h:92-110):
// 16 FMA chains, chain j over i = j mod 16 ascending, then GCC's
// _mm512_reduce_add_ps tree (j,j+8) -> (j,j+4) -> (0+2, 1+3) -> final.
// Lane j of a 16-lane group runs chain j; the tree is three shuffles.
// One wave = 4 experts; one block per (4 experts, token).
template <int BF16>
__global__ __launch_bounds__(64) void k_router(const void *__restrict__ Wc, const float *__restrict__ x, int D, int E,
                                               const float *__restrict__ lbias, float *__restrict__ logits) {
    extern __shared__ float xs[];
    const int s = blockIdx.y;
    const int tid = threadIdx.x;
    const float *xr = x + (int64_t)s * D;
    for (int i = tid * 4; i < D; i += 256) *(sw_f32x4 *)(xs + i) = *(const sw_f32x4 *)(xr + i);
    __syncthreads();
    const int e = blockIdx.x * 4 + (tid >> 4), j = tid & 15;
    const int M = D / 16;
    float acc = 0.f;
    if (e < E) {
        if (BF16) {
            const uint16_t *ch = (const uint16_t *)Wc + (int64_t)(e * 16 + j) * M;
            for (int m0 = 0; m0 < M; m0 += 8) {
                const sw_u32x4 wv = *(const sw_u32x4 *)(ch + m0);
                const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t bits = (u & 1) ? (wd[u >> 1] & 0xFFFF0000u) : (wd[u >> 1] << 16);
                    acc = __builtin_fmaf(xs[16 * (m0 + u) + j], __builtin_bit_cast(float, bits), acc);
                }
            }
        } else {
            const float *ch = (const float *)Wc + (int64_t)(e * 16 + j) * M;
            for (int m0 = 0; m0 < M; m0 += 4) {
                const sw_f32x4 wv = *(const sw_f32x4 *)(ch + m0);
#pragma unroll
                for (int u = 0; u < 4; u++) acc = __builtin_fmaf(xs[16 * (m0 + u) + j], wv[u], acc);
            }
        }
    }
    float v = acc;
    v = v + __shfl_down(v, 8, 16);
    v = v + __shfl_down(v, 4, 16);
    v = v + __shfl_down(v, 2, 16);
    v = v + __shfl_down(v, 1, 16);
    if (j == 0 && e < E) {
        if (lbias) v = v + lbias[e];
        logits[(int64_t)s * E + e] = v;
    }
}

int sw_launch_router(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                     const float *logit_bias, float *logits) {
    if (D % 128 || D > 16384 || E <= 0 || S <= 0) return -1;
    dim3 grid((unsigned)((E + 3) / 4), (unsigned)S);
    const size_t lds = (size_t)D * sizeof(float);
    if (w_bf16) hipLaunchKernelGGL(k_router<1>, grid, dim3(64), lds, st, Wc, x, D, E, logit_bias, logits);
    else hipLaunchKernelGGL(k_router<0>, grid, dim3(64), lds, st, Wc, x, D, E, logit_bias, logits);
    return launch_err();
}

// ------------------------------------------------------------ gate + top-k ----
// One wave per token.  Activation with the reference's host expressions and
// glibc-exact expf/log1pf (c/moe_block.h:26; c/moe_math.h:54,68-72), then
// moe_topk (c/moe_arch.h:64-89): K passes of "largest score+bias among the
// unselected, valid only if > -1e30, ties to the lowest id", the all-invalid
// fallback to the lowest unselected id, weight = unbiased score, optional
// renormalisation summed in rank order (c/moe_block.h:121-122).
#define TK_MAXE 1024
__global__ __launch_bounds__(64) void k_gate_topk(const float *__restrict__ logits, int E, int K, int act,
                                                  const float *__restrict__ bias, int use_bias, int norm,
                                                  int *__restrict__ sel, float *__restrict__ wout) {
    __shared__ float sc[TK_MAXE];
    __shared__ float wk[64];
    __shared__ int sk[64];
    __shared__ float bc;
    const int s = blockIdx.x, lane = threadIdx.x;
    const float *rl = logits + (int64_t)s * E;
    if (act == 1) {                                   // softmax (laguna contract)
        float mx = -__builtin_inff();
        bool any = false;
        for (int e = lane; e < E; e += 64) {
            const float v = rl[e];
            if (v == v) { mx = any ? fmaxf(mx, v) : v; any = true; }
        }
        for (int o = 32; o; o >>= 1) {
            const float t = __shfl_xor(mx, o);
            mx = fmaxf(mx, t);
        }
        if (rl[0] != rl[0]) mx = rl[0];               // a NaN in slot 0 propagates, as in the scan
        for (int e = lane; e < E; e += 64) sc[e] = sw_expf(rl[e] - mx);
        __syncthreads();
        if (lane == 0) {
            double sum = 0.0;
            for (int e = 0; e < E; e++) sum += (double)sc[e];
            bc = (float)(1.0 / sum);
        }
        __syncthreads();
        const float inv = bc;
        for (int e = lane; e < E; e += 64) sc[e] = sc[e] * inv;
    } else {
        for (int e = lane; e < E; e += 64) {
            const float v = rl[e];
            sc[e] = (act == 2) ? sw_softplus_ref(v) : sw_sigmoid_ref(v);
        }
    }
    __syncthreads();
    uint32_t taken = 0;                               // bit i: expert lane + 64 i selected
    const int nper = (E + 63) / 64;
    for (int a = 0; a < K; a++) {
        float bv = 0.f;
        int bi = -1, lowfree = 0x7fffffff;
        for (int i = 0; i < nper; i++) {
            const int e = lane + 64 * i;
            if (e >= E || ((taken >> i) & 1u)) continue;
            if (e < lowfree) lowfree = e;
            const float v = sc[e] + ((use_bias && bias) ? bias[e] : 0.f);
            if (v > -1e30f && (bi < 0 || v > bv)) { bv = v; bi = e; }
        }
        for (int o = 32; o; o >>= 1) {
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bi, o);
            const int ol = __shfl_xor(lowfree, o);
            bool take;
            if (oi < 0) take = false;
            else if (bi < 0) take = true;
            else if (ov > bv) take = true;
            else if (bv > ov) take = false;
            else take = oi < bi;
            if (take) { bv = ov; bi = oi; }
            lowfree = min(lowfree, ol);
        }
        if (bi < 0) bi = (lowfree < E) ? lowfree : 0;
        if ((bi & 63) == lane && bi < E) taken |= 1u << (bi >> 6);
        if (lane == 0) { sk[a] = bi; wk[a] = sc[bi]; }
    }
    __syncthreads();
    if (lane == 0) {
        if (norm) {
            float sm = 0.f;
            for (int a = 0; a < K; a++) sm += wk[a];
            for (int a = 0; a < K; a++) wk[a] = wk[a] / sm;
        }
        for (int a = 0; a < K; a++) {
            sel[(int64_t)s * K + a] = sk[a];
            wout[(int64_t)s * K + a] = wk[a];
        }
    }
}

int sw_launch_gate_topk(hipStream_t st, const float *logits, int S, int E, int K, int route_act,
                        const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w) {
    if (E <= 0 || E > TK_MAXE || K <= 0 || K > 64 || K > E || S <= 0 || route_act < 0 || route_act > 2) return -1;
    hipLaunchKernelGGL(k_gate_topk, dim3((unsigned)S), dim3(64), 0, st, logits, E, K, route_act, corr_bias,
                       use_corr_bias, norm_topk, sel, w);
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
        for (int a = 0; a < K; a++) {
            const float wa = w[s * K + a];
            const sw_f32x4 v = *(const sw_f32x4 *)(slots + (int64_t)rowof[s * K + a] * D + d);
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = __builtin_fmaf(wa, v[c], acc[c]);
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
