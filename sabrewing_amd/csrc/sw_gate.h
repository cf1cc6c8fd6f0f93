// sw_gate.h -- device functions shared by the routing kernels and the fused
// decode kernels: the gate + top-k of one token run by one wave, and the
// activation limbs of the int4 dot8 GEMV.
#ifndef SW_GATE_H
#define SW_GATE_H
#include "sw_hip.h"
#include "sw_libm.h"

// ------------------------------------------------------------ gate + top-k ----
// Gate with the reference's host expressions and glibc-exact expf/log1pf
// (c/moe_block.h:26; c/moe_math.h:54,68-72) -- sigmoid/softplus scores come
// from the logits kernel, softmax is done here -- then moe_topk
// (c/moe_arch.h:64-89): K passes of "largest score+bias among the unselected,
// valid only if > -1e30, ties to the lowest id", the all-invalid fallback to
// the lowest unselected id, weight = unbiased score, optional renormalisation
// summed in rank order (c/moe_block.h:121-122).
//
// A pass is one wave-wide max over 64-bit keys (order-preserving bits of
// key + 0.0 above ~id, so a larger key wins and equal keys go to the lower
// id; invalid or taken experts are key 0), reduced with DPP row operations.
#define TK_MAXE 1024

struct TopkLDS {
    float sc[TK_MAXE];
    float wk[64];
    int sk[64];
    uint64_t tab[32];
    float inv;
};

// LDS ordering between the lanes of one wave (its LDS operations run in order)
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

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

// The routing of one token, by the 64 lanes of one wave (no block barrier):
// src is the token's logits (act == 1) or its sigmoid/softplus scores.
// Leaves the picks in sh.sk[0..K) and their weights in sh.wk[0..K).
template <int NPER>   // expert slots per lane: E <= 64 * NPER
__device__ void gate_topk_wave(const float *__restrict__ src, int E, int K, int act, const float *__restrict__ bias,
                               int use_bias, int norm, TopkLDS &sh) {
    const int lane = threadIdx.x & 63;
    float v[NPER], b[NPER];
    // every load of the token issued before any is used (clamped indices)
    if (act == 1 && lane < 32) sh.tab[lane] = sw_exp2f_tab[lane];
    const bool hasb = use_bias && bias;
#pragma unroll
    for (int i = 0; i < NPER; i++) {
        const int e = min(lane + 64 * i, E - 1);
        v[i] = src[e];
        b[i] = hasb ? bias[e] : 0.f;
    }
    if (act == 1) {                                   // softmax
        wave_sync();
        float mx = -__builtin_inff();
        bool any = false;
#pragma unroll
        for (int i = 0; i < NPER; i++) {
            const int e = lane + 64 * i;
            if (e < E && v[i] == v[i]) { mx = any ? fmaxf(mx, v[i]) : v[i]; any = true; }
        }
        for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float r0 = __shfl(v[0], 0);
        if (r0 != r0) mx = r0;                        // a NaN in slot 0 propagates, as in the scan
#pragma unroll
        for (int i = 0; i < NPER; i++) {
            const int e = lane + 64 * i;
            if (e < E) sh.sc[e] = sw_expf_t(v[i] - mx, sh.tab);
        }
        wave_sync();
        if (lane == 0) {
            double sum = 0.0;
            for (int e = 0; e < E; e++) sum += (double)sh.sc[e];
            sh.inv = (float)(1.0 / sum);
        }
        wave_sync();
        const float inv = sh.inv;
#pragma unroll
        for (int i = 0; i < NPER; i++) {
            const int e = lane + 64 * i;
            if (e < E) v[i] = sh.sc[e] * inv;
        }
    }
#pragma unroll
    for (int i = 0; i < NPER; i++) {
        const int e = lane + 64 * i;
        if (e < E) sh.sc[e] = v[i];
    }
    wave_sync();
    uint64_t kk[NPER];
    bool fr[NPER];
#pragma unroll
    for (int i = 0; i < NPER; i++) {
        const int e = lane + 64 * i;
        const float key = v[i] + b[i];
        fr[i] = e < E;
        kk[i] = (e < E && key > -1e30f) ? (((uint64_t)ord_f32(key) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e)) : 0ull;
    }
    for (int a = 0; a < K; a++) {
        uint64_t m = kk[0];
#pragma unroll
        for (int i = 1; i < NPER; i++) m = max64(m, kk[i]);
        m = wave_max_u64(m);
        int bi;
        if (m != 0ull) {
            bi = (int)(0xFFFFFFFFu - (uint32_t)m);
        } else {                                      // nothing valid left: the lowest unselected id
            bi = 0x7fffffff;
#pragma unroll
            for (int i = NPER - 1; i >= 0; i--) {
                const unsigned long long bal = __ballot(fr[i]);
                if (bal) bi = 64 * i + __builtin_ctzll(bal);
            }
            if (bi >= E) bi = 0;
        }
        if ((bi & 63) == lane) {
#pragma unroll
            for (int i = 0; i < NPER; i++)
                if (i == (bi >> 6)) { kk[i] = 0ull; fr[i] = false; }
        }
        if (lane == 0) { sh.sk[a] = bi; sh.wk[a] = sh.sc[bi]; }
    }
    wave_sync();
    if (lane == 0 && norm) {
        float sm = 0.f;
        for (int a = 0; a < K; a++) sm += sh.wk[a];
        for (int a = 0; a < K; a++) sh.wk[a] = sh.wk[a] / sm;
    }
    wave_sync();
}

// ------------------------------------------------------------ limbs ----
// The activation side of the int4 dot8 GEMV (k_dot8.hip).  For each group of
// SW_RG consecutive inputs, with 2^e the smallest power of two above max|x|
// of the group, y = x * 2^-e in (-1, 1) is written as sum_{l=1..NL} d_l 8^-l
// with signed digits d_l in [-8, 7] (round to nearest, clamp, carry the exact
// remainder), so x ~= 2^(e - 3 NL) * D with D = sum_l d_l 8^(NL - l) and
// |error| <= 2^e 8^-NL.  Limb l of the group is 4 dwords of 32 nibbles (input
// 8j + i at bits 4i of dword j, the weights' nibble order); the factor is
// 2^(e - 3 NL), or NaN for a group holding a NaN or an infinity.
#define SW_RG 32
// one group by the 32 lanes of a half-wave; i = lane in the half
__device__ __forceinline__ void limbs_group(float v, int i, sw_u32x4 *__restrict__ dst, float *__restrict__ fdst) {
    float m = fabsf(v);
    bool bad = !(m <= 3.4028235e38f);                // NaN or inf
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
        m = fmaxf(m, __shfl_xor(m, o, 32));
        bad = bad | (__shfl_xor((int)bad, o, 32) != 0);
    }
    int e = 0;
    if (m > 0.f && !bad) (void)frexpf(m, &e);        // m = f 2^e, f in [0.5, 1): 2^e > m
    float y = ldexpf(v, -e);                          // exact: |y| < 1
    uint32_t dw[SW_NL];
#pragma unroll
    for (int l = 0; l < SW_NL; l++) {
        const float t = y * 8.0f;                     // exact
        float d = rintf(t);
        d = fminf(fmaxf(d, -8.0f), 7.0f);
        y = t - d;                                    // exact, |y| <= 1
        uint32_t nib = ((uint32_t)(int)d & 0xFu) << (4 * (i & 7));
        nib |= __shfl_xor(nib, 1, 32);
        nib |= __shfl_xor(nib, 2, 32);
        nib |= __shfl_xor(nib, 4, 32);
        dw[l] = nib;                                  // lanes 8j.. hold dword j of limb l
    }
    if ((i & 7) == 0) {
        const int j = i >> 3;
#pragma unroll
        for (int l = 0; l < SW_NL; l++) ((uint32_t *)(dst + l))[j] = bad ? 0u : dw[l];
    }
    if (i == 0) *fdst = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 3 * SW_NL);
}

#endif
