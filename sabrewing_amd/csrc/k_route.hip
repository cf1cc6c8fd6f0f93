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
// One wave finishes the routing of one token.  Activation with the reference's
// host expressions and glibc-exact expf/log1pf (c/moe_block.h:26;
// c/moe_math.h:54,68-72), then moe_topk (c/moe_arch.h:64-89): K passes of
// "largest score+bias among the unselected, valid only if > -1e30, ties to
// the lowest id", the all-invalid fallback to the lowest unselected id,
// weight = unbiased score, optional renormalisation summed in rank order
// (c/moe_block.h:121-122).  All four waves of the block call this (barriers);
// only wave 0 works.
#define TK_MAXE 1024
#define TK_NPER (TK_MAXE / 64)
struct TopkShared {
    float sc[TK_MAXE];
    float wk[64];
    int sk[64];
    float inv;
};

__device__ __forceinline__ float load_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ void gate_topk_token(const float *rl, int E, int K, int act, const float *__restrict__ bias, int use_bias,
                                int norm, int *sel, float *wout, TopkShared &sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nper = (E + 63) / 64;
    float v[TK_NPER], key[TK_NPER];
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < TK_NPER; i++) {
            const int e = lane + 64 * i;
            v[i] = (i < nper && e < E) ? load_agent(rl + e) : 0.f;
        }
    }
    if (act == 1) {                                   // softmax (the laguna contract)
        if (wave == 0) {
            float mx = -__builtin_inff();
            bool any = false;
#pragma unroll
            for (int i = 0; i < TK_NPER; i++) {
                const int e = lane + 64 * i;
                if (i < nper && e < E && v[i] == v[i]) { mx = any ? fmaxf(mx, v[i]) : v[i]; any = true; }
            }
            for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            const float r0 = __shfl(v[0], 0);
            if (r0 != r0) mx = r0;                    // a NaN in slot 0 propagates, as in the scan
#pragma unroll
            for (int i = 0; i < TK_NPER; i++) {
                const int e = lane + 64 * i;
                if (i < nper && e < E) sh.sc[e] = sw_expf(v[i] - mx);
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            double sum = 0.0;
            for (int e = 0; e < E; e++) sum += (double)sh.sc[e];
            sh.inv = (float)(1.0 / sum);
        }
        __syncthreads();
        if (wave == 0) {
            const float inv = sh.inv;
#pragma unroll
            for (int i = 0; i < TK_NPER; i++) {
                const int e = lane + 64 * i;
                if (i < nper && e < E) { v[i] = sh.sc[e] * inv; sh.sc[e] = v[i]; }
            }
        }
    } else if (wave == 0) {
#pragma unroll
        for (int i = 0; i < TK_NPER; i++) {
            const int e = lane + 64 * i;
            if (i < nper && e < E) {
                v[i] = (act == 2) ? sw_softplus_ref(v[i]) : sw_sigmoid_ref(v[i]);
                sh.sc[e] = v[i];
            }
        }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < TK_NPER; i++) {
            const int e = lane + 64 * i;
            key[i] = (i < nper && e < E) ? v[i] + ((use_bias && bias) ? bias[e] : 0.f) : 0.f;
        }
        uint32_t taken = 0;
        for (int a = 0; a < K; a++) {
            float bv = 0.f;
            int bi = -1, lowfree = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < TK_NPER; i++) {
                const int e = lane + 64 * i;
                if (i < nper && e < E && !((taken >> i) & 1u)) {
                    if (e < lowfree) lowfree = e;
                    if (key[i] > -1e30f && (bi < 0 || key[i] > bv)) { bv = key[i]; bi = e; }
                }
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
            if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
            if (lane == 0) { sh.sk[a] = bi; sh.wk[a] = sh.sc[bi]; }
        }
        if (lane == 0) {
            if (norm) {
                float sm = 0.f;
                for (int a = 0; a < K; a++) sm += sh.wk[a];
                for (int a = 0; a < K; a++) sh.wk[a] = sh.wk[a] / sm;
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (lane < K) { sel[lane] = sh.sk[lane]; wout[lane] = sh.wk[lane]; }
    }
}

// logits[s,e] = sum_i x[s,i] W[e,i] under the contract of the reference's
// AVX-512 router (c/moe_matmul.h:25-43; bf16 weights c/moe_matmul.h:92-110):
// 16 FMA chains, chain j over i = j mod 16 ascending, then GCC's
// _mm512_reduce_add_ps tree (j,j+8) -> (j,j+4) -> (0+2, 1+3) -> final.
// Lane j of a 16-lane group runs chain j (weights chain-major, all loads in
// flight before the chain starts; x transposed in LDS so a lane reads its
// chain's inputs contiguously); the tree is four shuffles.  Block = 16
// experts of one token; the block that finishes a token's last logits (a
// per-token arrival counter, reset by that block) runs gate + top-k.
#define RT_MAXLD 32
template <int BF16>
__global__ __launch_bounds__(256) void k_router_topk(const void *__restrict__ Wc, const float *__restrict__ x, int D, int E,
                                                     const float *__restrict__ lbias, float *__restrict__ logits,
                                                     int *__restrict__ counters, int K, int act,
                                                     const float *__restrict__ cbias, int use_bias, int norm,
                                                     int *__restrict__ sel, float *__restrict__ wout) {
    extern __shared__ __align__(16) float xt[];      // [16][M + 4]
    __shared__ TopkShared sh;
    __shared__ int last;
    const int s = blockIdx.y, tid = threadIdx.x;
    const int M = D / 16, ML = M + 4;
    const int e = blockIdx.x * 16 + (tid >> 4), j = tid & 15;
    const bool valid = e < E;
    const int per = BF16 ? 8 : 4;                     // chain elements per 16-byte load
    float acc = 0.f;
    for (int m0 = 0; m0 < M; m0 += RT_MAXLD * per) {
        const int nld = min(RT_MAXLD, (M - m0) / per);
        sw_u32x4 wr[RT_MAXLD];
        const char *ch = (const char *)Wc + ((int64_t)(valid ? e : 0) * 16 + j) * M * (BF16 ? 2 : 4) + (int64_t)m0 * (BF16 ? 2 : 4);
#pragma unroll
        for (int l = 0; l < RT_MAXLD; l++)
            if (l < nld && valid) wr[l] = *(const sw_u32x4 *)(ch + 16 * l);
        if (m0 == 0) {
            const float *xr = x + (int64_t)s * D;
            for (int i = tid * 4; i < D; i += 1024) {
                const sw_f32x4 v = *(const sw_f32x4 *)(xr + i);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int k = i + c;
                    xt[(k & 15) * ML + (k >> 4)] = v[c];
                }
            }
            __syncthreads();
        }
        if (valid) {
            const float *xj = xt + j * ML + m0;
#pragma unroll
            for (int l = 0; l < RT_MAXLD; l++) {
                if (l < nld) {
                    const uint32_t wd[4] = {wr[l].x, wr[l].y, wr[l].z, wr[l].w};
                    if (BF16) {
                        const sw_f32x4 xa = *(const sw_f32x4 *)(xj + 8 * l), xb = *(const sw_f32x4 *)(xj + 8 * l + 4);
                        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                        for (int u = 0; u < 8; u++) {
                            const uint32_t bits = (u & 1) ? (wd[u >> 1] & 0xFFFF0000u) : (wd[u >> 1] << 16);
                            acc = __builtin_fmaf(xv[u], __builtin_bit_cast(float, bits), acc);
                        }
                    } else {
                        const sw_f32x4 xa = *(const sw_f32x4 *)(xj + 4 * l);
#pragma unroll
                        for (int u = 0; u < 4; u++) acc = __builtin_fmaf(xa[u], __builtin_bit_cast(float, wd[u]), acc);
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
    if (j == 0 && valid) {
        if (lbias) v = v + lbias[e];
        logits[(int64_t)s * E + e] = v;
    }
    if (!counters) return;                            // logits only
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(&counters[s], 1) == (int)gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    gate_topk_token(logits + (int64_t)s * E, E, K, act, cbias, use_bias, norm, sel + (int64_t)s * K, wout + (int64_t)s * K, sh);
    if (tid == 0) counters[s] = 0;
}

int sw_launch_router_topk(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                          const float *logit_bias, float *logits, int *counters, int K, int route_act,
                          const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w) {
    if (D % 128 || D > 8192 || E <= 0 || E > TK_MAXE || S <= 0 || K <= 0 || K > 64 || K > E) return -1;
    if (route_act < 0 || route_act > 2) return -1;
    dim3 grid((unsigned)((E + 15) / 16), (unsigned)S);
    const size_t lds = (size_t)16 * (D / 16 + 4) * sizeof(float);
    if (w_bf16)
        hipLaunchKernelGGL(k_router_topk<1>, grid, dim3(256), lds, st, Wc, x, D, E, logit_bias, logits, counters, K,
                           route_act, corr_bias, use_corr_bias, norm_topk, sel, w);
    else
        hipLaunchKernelGGL(k_router_topk<0>, grid, dim3(256), lds, st, Wc, x, D, E, logit_bias, logits, counters, K,
                           route_act, corr_bias, use_corr_bias, norm_topk, sel, w);
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
