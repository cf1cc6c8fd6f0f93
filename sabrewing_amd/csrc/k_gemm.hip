// k_gemm.hip -- grouped int4 and bf16 expert GEMMs on the gfx950 matrix cores.
//
// One wave owns one row tile of one group (an expert applied to a run of
// packed rows) and walks the whole of K itself, so every output follows the
// reduction contract stated in sw_hip.h whatever the batch.  Replaces the
// reference's warp-per-row mm_q4_kernel / mm_q4_group_kernel /
// grouped_*_g4 kernels (c/backend_cuda_laguna.cu:138-157,420-443;
// c/backend_cuda.cu:347-380): those re-read each weight row once per token;
// here a weight row is read once per launch and applied to every token of the
// group as MFMA columns (token t -> columns 2t (hi) and 2t+1 (lo)).
//
// int4 dequant (in registers, no LDS): a 32-bit word holds 8 nibbles of one
// row; OR-ing a nibble into the mantissa of f16 1024.0 gives 1024+n exactly,
// and one packed add (or packed fma for the nibbles sitting 4 bits higher)
// yields n-8 exactly.  Group scales (gs > 0) are folded into the f16 weight
// (f16(s*2^8) * (n-8), rounded once); per-row scales (gs == 0) are applied in
// f32 after the K loop, leaving the weights exact.
//
// Algorithmic bytes per launch (what the roofline divides): every distinct
// weight byte (nibbles + scales, or bf16) once, plus activations in and out.
#include "sw_hip.h"
#include "sw_libm.h"

enum { EPI_GLU = 0, EPI_ROWS = 1 };
#define PF 4          // super-steps of weight loads kept in flight per wave

__device__ __forceinline__ sw_half8 dq8(uint32_t w, sw_half2 s2, bool scaled) {
    const sw_half2 m1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const sw_half2 r16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const sw_half2 m72 = {(_Float16)-72.0f, (_Float16)-72.0f};
    const uint32_t w8 = w >> 8;
    sw_half2 h0 = __builtin_bit_cast(sw_half2, (w & 0x000F000Fu) | 0x64006400u) + m1032;
    sw_half2 h1 = __builtin_elementwise_fma(__builtin_bit_cast(sw_half2, (w & 0x00F000F0u) | 0x64006400u), r16, m72);
    sw_half2 h2 = __builtin_bit_cast(sw_half2, (w8 & 0x000F000Fu) | 0x64006400u) + m1032;
    sw_half2 h3 = __builtin_elementwise_fma(__builtin_bit_cast(sw_half2, (w8 & 0x00F000F0u) | 0x64006400u), r16, m72);
    if (scaled) { h0 = h0 * s2; h1 = h1 * s2; h2 = h2 * s2; h3 = h3 * s2; }
    sw_u32x4 u = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                  __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3)};
    return __builtin_bit_cast(sw_half8, u);
}

// position of element i inside an f16 plane row (8-blocks stored 0,4,1,5,2,6,3,7)
__device__ __forceinline__ int plane_pos(int i) {
    const int m = i & 7;
    return (i & ~7) | ((m & 3) << 1) | (m >> 2);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

__device__ __forceinline__ float silu_glu(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// ---------------------------------------------------------------- int4 ----
template <int EPI, int CB>
__global__ __launch_bounds__(256) void k_q4_gemm(SwQ4 W, const _Float16 *__restrict__ xp, SwGroups G,
                                                int I, void *__restrict__ out, int rowtiles) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = blockIdx.x;
    const int gvalid = G.G ? *G.G : G.ngroups_max;
    if (g >= gvalid) return;
    const int rt = blockIdx.y * 4 + wave;
    if (rt >= rowtiles) return;
    const int e = G.gexp[g], beg = G.gbeg[g], cnt = G.gcnt[g];
    const int r = lane & 15, kb = lane >> 4;
    const int wrow = (EPI == EPI_GLU) ? ((r < 8) ? (rt * 8 + r) : (I + rt * 8 + r - 8)) : (rt * 16 + r);
    const int K = W.K, gs = W.gs;
    const int ng = gs > 0 ? K / gs : 1;
    const int64_t wr = (int64_t)e * W.O + wrow;
    const uint8_t *arow = W.q + wr * (K / 2) + kb * 16;
    const float *srow = W.s + wr * ng;
    const int nss = K >> 7;
    const int c = lane & 15, tcol = c >> 1, plane = c & 1;
    const bool scaled = gs > 0;

    for (int t0 = 0; t0 < cnt; t0 += 8 * CB) {
        const int ncb = min(CB, (cnt - t0 + 7) >> 3);
        const _Float16 *bp[CB];
        bool bv[CB];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            const int t = t0 + cb * 8 + tcol;
            bv[cb] = (cb < ncb) && (t < cnt);
            const int src = bv[cb] ? (G.grow ? G.grow[beg + t] : beg + t) : 0;
            bp[cb] = xp + ((int64_t)(2 * src + plane)) * K + kb * 32;
        }
        sw_f32x4 acc[CB];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[cb] = (sw_f32x4){0.f, 0.f, 0.f, 0.f};

        sw_u32x4 ra[PF];
        float sa[PF];
#pragma unroll
        for (int u = 0; u < PF; u++) {
            if (u < nss) {
                ra[u] = *(const sw_u32x4 *)(arow + u * 64);
                sa[u] = scaled ? srow[(u * 128 + kb * 32) / gs] : 0.f;
            }
        }
        for (int ss0 = 0; ss0 < nss; ss0 += PF) {
#pragma unroll
            for (int u = 0; u < PF; u++) {
                const int ss = ss0 + u;
                if (ss < nss) {
                    const sw_u32x4 cur = ra[u];
                    const float cs = sa[u];
                    if (ss + PF < nss) {
                        ra[u] = *(const sw_u32x4 *)(arow + (ss + PF) * 64);
                        sa[u] = scaled ? srow[((ss + PF) * 128 + kb * 32) / gs] : 0.f;
                    }
                    sw_half8 bq[CB][4];
#pragma unroll
                    for (int cb = 0; cb < CB; cb++) {
                        if (cb < ncb) {
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                if (bv[cb]) bq[cb][q] = *(const sw_half8 *)(bp[cb] + ss * 128 + q * 8);
                                else bq[cb][q] = (sw_half8){0, 0, 0, 0, 0, 0, 0, 0};
                            }
                        }
                    }
                    const _Float16 s16 = (_Float16)(cs * SW_WPRESCALE);
                    const sw_half2 s2 = {s16, s16};
                    sw_half8 a[4];
                    a[0] = dq8(cur.x, s2, scaled);
                    a[1] = dq8(cur.y, s2, scaled);
                    a[2] = dq8(cur.z, s2, scaled);
                    a[3] = dq8(cur.w, s2, scaled);
#pragma unroll
                    for (int cb = 0; cb < CB; cb++) {
                        if (cb < ncb) {
#pragma unroll
                            for (int q = 0; q < 4; q++)
                                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[q], bq[cb][q], acc[cb], 0, 0, 0);
                        }
                    }
                }
            }
        }
        // epilogue: hi + lo, scale, then GLU or store
        const int rbase = 4 * (lane >> 4);
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            if (cb >= ncb) break;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float mine = acc[cb][j];
                const float other = __shfl_xor(mine, 1);
                v[j] = mine + other;       // even lanes: hi + lo
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (scaled) {
                    v[j] = v[j] * SW_WPRESCALE_INV;
                } else {
                    const int rr = rbase + j;
                    const int wrr = (EPI == EPI_GLU) ? ((rr < 8) ? (rt * 8 + rr) : (I + rt * 8 + rr - 8)) : (rt * 16 + rr);
                    v[j] = v[j] * W.s[(int64_t)e * W.O + wrr];
                }
            }
            const int t = t0 + cb * 8 + tcol;
            if (EPI == EPI_GLU) {
                float up[4];
#pragma unroll
                for (int j = 0; j < 4; j++) up[j] = __shfl_xor(v[j], 32);
                if (lane < 32 && plane == 0 && t < cnt) {
                    _Float16 *hp = (_Float16 *)out;
                    const int64_t row = 2 * (int64_t)(beg + t);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int i = rt * 8 + rbase + j;
                        const float h = silu_glu(v[j], up[j]);
                        const _Float16 hi = (_Float16)h;
                        const _Float16 lo = (_Float16)(h - (float)hi);
                        hp[row * I + plane_pos(i)] = hi;
                        hp[(row + 1) * I + plane_pos(i)] = lo;
                    }
                }
            } else {
                if (plane == 0 && t < cnt) {
                    float *Y = (float *)out;
                    *(sw_f32x4 *)(Y + (int64_t)(beg + t) * W.O + rt * 16 + rbase) = (sw_f32x4){v[0], v[1], v[2], v[3]};
                }
            }
        }
    }
}

// ---------------------------------------------------------------- bf16 ----
// Wg (and Wu for the GLU epilogue) bf16 [O, K]; one implicit group of S tokens.
template <int EPI, int CB>
__global__ __launch_bounds__(256) void k_bf16_gemm(SwBf16 Wg, SwBf16 Wu, const uint16_t *__restrict__ xp, int S,
                                                  void *__restrict__ out, int rowtiles) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rt = blockIdx.x * 4 + wave;
    if (rt >= rowtiles) return;
    const int tbase = blockIdx.y * 8 * CB;
    const int r = lane & 15, kb = lane >> 4;
    const int K = Wg.K;
    const uint16_t *arow;
    if (EPI == EPI_GLU) arow = (r < 8) ? (Wg.w + (int64_t)(rt * 8 + r) * K) : (Wu.w + (int64_t)(rt * 8 + r - 8) * K);
    else arow = Wg.w + (int64_t)(rt * 16 + r) * K;
    arow += kb * 32;
    const int nss = K >> 7;
    const int c = lane & 15, tcol = c >> 1, plane = c & 1;
    const int cnt = min(S - tbase, 8 * CB);
    const int ncb = (cnt + 7) >> 3;
    const uint16_t *bp[CB];
    bool bv[CB];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        const int t = cb * 8 + tcol;
        bv[cb] = (cb < ncb) && (t < cnt);
        bp[cb] = xp + (int64_t)(2 * (tbase + (bv[cb] ? t : 0)) + plane) * K + kb * 32;
    }
    sw_f32x4 acc[CB];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) acc[cb] = (sw_f32x4){0.f, 0.f, 0.f, 0.f};
    sw_u32x4 ra[PF][4];
#pragma unroll
    for (int u = 0; u < PF; u++)
        if (u < nss)
#pragma unroll
            for (int q = 0; q < 4; q++) ra[u][q] = *(const sw_u32x4 *)(arow + u * 128 + q * 8);
    for (int ss0 = 0; ss0 < nss; ss0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int ss = ss0 + u;
            if (ss < nss) {
                sw_u32x4 cur[4];
#pragma unroll
                for (int q = 0; q < 4; q++) cur[q] = ra[u][q];
                if (ss + PF < nss)
#pragma unroll
                    for (int q = 0; q < 4; q++) ra[u][q] = *(const sw_u32x4 *)(arow + (ss + PF) * 128 + q * 8);
#pragma unroll
                for (int cb = 0; cb < CB; cb++) {
                    if (cb < ncb) {
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            sw_u32x4 bw = {0u, 0u, 0u, 0u};
                            if (bv[cb]) bw = *(const sw_u32x4 *)(bp[cb] + ss * 128 + q * 8);
                            acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sw_bf16x8, cur[q]),
                                                                              __builtin_bit_cast(sw_bf16x8, bw), acc[cb], 0, 0, 0);
                        }
                    }
                }
            }
        }
    }
    const int rbase = 4 * (lane >> 4);
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        if (cb >= ncb) break;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float mine = acc[cb][j];
            v[j] = mine + __shfl_xor(mine, 1);
        }
        const int t = cb * 8 + tcol;
        if (EPI == EPI_GLU) {
            float up[4];
#pragma unroll
            for (int j = 0; j < 4; j++) up[j] = __shfl_xor(v[j], 32);
            if (lane < 32 && plane == 0 && t < cnt) {
                uint16_t *hp = (uint16_t *)out;
                const int Is = Wg.O;
                const int64_t row = 2 * (int64_t)(tbase + t);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int i = rt * 8 + rbase + j;
                    const float h = silu_glu(v[j], up[j]);
                    const uint16_t hi = f32_to_bf16_rne(h);
                    const uint16_t lo = f32_to_bf16_rne(h - bf16_to_f32(hi));
                    hp[row * Is + i] = hi;
                    hp[(row + 1) * Is + i] = lo;
                }
            }
        } else {
            if (plane == 0 && t < cnt) {
                float *Y = (float *)out;
                *(sw_f32x4 *)(Y + (int64_t)(tbase + t) * Wg.O + rt * 16 + rbase) = (sw_f32x4){v[0], v[1], v[2], v[3]};
            }
        }
    }
}

// ---------------------------------------------------------------- launch ----
static int launch_err(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

static int q4_ok(const SwQ4 &W) {
    if (W.K % 128) return 0;
    if (W.gs > 0 && (W.gs % 32 || W.K % W.gs)) return 0;
    return 1;
}

int sw_launch_q4_gateup(hipStream_t st, SwQ4 W, const _Float16 *xplanes, SwGroups g, int I, _Float16 *hplanes, int cb) {
    if (!q4_ok(W) || I % 8 || W.O != 2 * I || g.ngroups_max <= 0) return -1;
    const int rowtiles = I / 8;
    dim3 grid((unsigned)g.ngroups_max, (unsigned)((rowtiles + 3) / 4));
    if (cb <= 1)
        hipLaunchKernelGGL((k_q4_gemm<EPI_GLU, 1>), grid, dim3(256), 0, st, W, xplanes, g, I, (void *)hplanes, rowtiles);
    else
        hipLaunchKernelGGL((k_q4_gemm<EPI_GLU, 4>), grid, dim3(256), 0, st, W, xplanes, g, I, (void *)hplanes, rowtiles);
    return launch_err();
}

int sw_launch_q4_rows(hipStream_t st, SwQ4 W, const _Float16 *xplanes, SwGroups g, float *Y, int cb) {
    if (!q4_ok(W) || W.O % 16 || g.ngroups_max <= 0) return -1;
    const int rowtiles = W.O / 16;
    dim3 grid((unsigned)g.ngroups_max, (unsigned)((rowtiles + 3) / 4));
    if (cb <= 1)
        hipLaunchKernelGGL((k_q4_gemm<EPI_ROWS, 1>), grid, dim3(256), 0, st, W, xplanes, g, 0, (void *)Y, rowtiles);
    else
        hipLaunchKernelGGL((k_q4_gemm<EPI_ROWS, 4>), grid, dim3(256), 0, st, W, xplanes, g, 0, (void *)Y, rowtiles);
    return launch_err();
}

int sw_launch_bf16_gateup(hipStream_t st, SwBf16 Wg, SwBf16 Wu, const uint16_t *xplanes, int S, uint16_t *hplanes) {
    if (Wg.K % 128 || Wg.O % 8 || Wu.O != Wg.O || Wu.K != Wg.K || S <= 0) return -1;
    const int rowtiles = Wg.O / 8;
    if (S <= 8) {
        dim3 grid((unsigned)((rowtiles + 3) / 4), (unsigned)((S + 7) / 8));
        hipLaunchKernelGGL((k_bf16_gemm<EPI_GLU, 1>), grid, dim3(256), 0, st, Wg, Wu, xplanes, S, (void *)hplanes, rowtiles);
    } else {
        dim3 grid((unsigned)((rowtiles + 3) / 4), (unsigned)((S + 31) / 32));
        hipLaunchKernelGGL((k_bf16_gemm<EPI_GLU, 4>), grid, dim3(256), 0, st, Wg, Wu, xplanes, S, (void *)hplanes, rowtiles);
    }
    return launch_err();
}

int sw_launch_bf16_rows(hipStream_t st, SwBf16 W, const uint16_t *xplanes, int S, float *Y) {
    if (W.K % 128 || W.O % 16 || S <= 0) return -1;
    const int rowtiles = W.O / 16;
    if (S <= 8) {
        dim3 grid((unsigned)((rowtiles + 3) / 4), (unsigned)((S + 7) / 8));
        hipLaunchKernelGGL((k_bf16_gemm<EPI_ROWS, 1>), grid, dim3(256), 0, st, W, W, xplanes, S, (void *)Y, rowtiles);
    } else {
        dim3 grid((unsigned)((rowtiles + 3) / 4), (unsigned)((S + 31) / 32));
        hipLaunchKernelGGL((k_bf16_gemm<EPI_ROWS, 4>), grid, dim3(256), 0, st, W, W, xplanes, S, (void *)Y, rowtiles);
    }
    return launch_err();
}
