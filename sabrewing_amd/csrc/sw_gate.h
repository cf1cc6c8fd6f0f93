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
// A pass is one wave-wide max of the order-preserving bits of key + 0.0
// (invalid or taken experts are 0), then the lowest id holding that maximum:
// a larger key wins, equal keys go to the lower id.
#define TK_MAXE 1024

// LDS ordering between the lanes of one wave (its LDS operations run in order)
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// max over the 64 lanes, returned uniform: the max within each 16-lane row by
// DPP (0 fills nothing: the operations stay inside the row), then the rows'
// maxima by readlane
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
    return v > o ? v : o;
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
    v = dpp_umax<0xB1>(v);                  // quad_perm [1,0,3,2]
    v = dpp_umax<0x4E>(v);                  // quad_perm [2,3,0,1]
    v = dpp_umax<0x141>(v);                 // row_half_mirror
    v = dpp_umax<0x140>(v);                 // row_mirror
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    const uint32_t m01 = r0 > r1 ? r0 : r1, m23 = r2 > r3 ? r2 : r3;
    return m01 > m23 ? m01 : m23;
}

// The fixed summation order of every GEMV row here: a row's G terms (one per
// group of 32 inputs) are padded with zero terms to Gq = run_lanes(G) (the
// next power of two below 16, the next multiple of 16 above) and summed in
// runs of n = min(Gq, 16) consecutive groups held by n consecutive lanes
// (aligned to n), each run as the butterfly of pairs, quads, eights and
// sixteens -- every lane of the run ends with the same sum, since
// a + b == b + a -- then the run sums left to right.  It depends on nothing
// but the row's terms.
__host__ __device__ inline int run_lanes(int G) {
    if (G >= 16) return (G + 15) & ~15;
    int q = 1;
    while (q < G) q <<= 1;
    return q;
}
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// lane i of a 16-lane row gets v(i) + v(partner(i)), one v_add_f32_dpp
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// a lane's partner within its 16-lane row by rotation (row_ror:N): lane (i - N) mod 16.
// The tails of the butterflies below pair lanes at distance 8, 4, 2, 1 after the
// values already agree between lanes at every larger distance of the tree, so the
// rotation hands each lane the value of lane i ^ N, whichever way it turns, and the
// sums get the bits of the xor butterfly (a + b == b + a)
template <int N>
__device__ __forceinline__ float row_ror(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + N, 0xF, 0xF, true));
}
template <int N>
__device__ __forceinline__ double row_ror(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, 0x120 + N, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), 0x120 + N, 0xF, 0xF, true);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
// the reduce tree of a 16-lane row as __shfl_down by 8, 4, 2, 1: lane 0 ends with
// ((v0 + v8) + (v4 + v12)) + ... (the router chains' _mm512_reduce_add_ps order)
__device__ __forceinline__ float row_reduce16(float v) {
    v = v + row_ror<8>(v);
    v = v + row_ror<4>(v);
    v = v + row_ror<2>(v);
    return v + row_ror<1>(v);
}
// the xor butterfly over 64 lanes, pairs at distance 32, 16, 8, 4, 2, 1 in that order
__device__ __forceinline__ double wave_xor_sum(double v) {
    v += __shfl_xor(v, 32);
    v += __shfl_xor(v, 16);
    v += row_ror<8>(v);
    v += row_ror<4>(v);
    v += row_ror<2>(v);
    return v + row_ror<1>(v);
}
// the maximum over 64 lanes (fmaxf: any order gives the same value)
__device__ __forceinline__ float wave_fmax(float v) {
    v = fmaxf(v, __shfl_xor(v, 32));
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, row_ror<8>(v));
    v = fmaxf(v, row_ror<4>(v));
    v = fmaxf(v, row_ror<2>(v));
    return fmaxf(v, row_ror<1>(v));
}
__device__ __forceinline__ float run_sum16(float v) {
    v = dpp_add<0xB1>(v);                   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);                   // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);                  // row_half_mirror
    return dpp_add<0x140>(v);               // row_mirror
}
// the same butterfly over runs of n (a power of two <= 16) lanes
__device__ __forceinline__ float run_sum(float v, int n) {
    if (n >= 2) v = v + dppf<0xB1>(v);      // quad_perm [1,0,3,2]
    if (n >= 4) v = v + dppf<0x4E>(v);      // quad_perm [2,3,0,1]
    if (n >= 8) v = v + dppf<0x141>(v);     // row_half_mirror
    if (n >= 16) v = v + dppf<0x140>(v);    // row_mirror
    return v;
}

__device__ __forceinline__ uint32_t ord_f32(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f + 0.0f);   // -0 -> +0: equal keys tie on the id
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float lanef(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// The routing of one token, by the 64 lanes of one wave (no block barrier):
// src is the token's logits (a softmax act: 1, 3, 4) or its sigmoid/softplus scores; tab is
// 32 words of LDS for the expf table (softmax).  On return lane a < K holds
// pick a (rank order) in sk and its weight in wk.
//
// Lane l holds the NPER consecutive experts NPER l .. NPER l + NPER - 1, so a
// lower lane holds lower ids and the lowest id holding the maximum is the
// lowest such lane's first such slot: one ballot per pass.  Each lane keeps
// its own best slot and the state it leaves when that slot is taken ready
// before the wave maximum is known, so a pass is the maximum, one ballot and
// the winner's update.
// kp (0 < kp < K): only picks 0 .. kp-1 are wanted -- the first kp passes run and the
// weights are left unnormalised (a caller that needs one pick's expert, not the weights).
template <int NPER>   // expert slots per lane: E <= 64 * NPER
__device__ void gate_topk_wave(const float *__restrict__ src, int E, int K, int act, const float *__restrict__ bias,
                               int use_bias, int norm, uint64_t *tab, int &sk, float &wk, int ns = 0, float rs = 1.f,
                               float *__restrict__ wsh = nullptr, int kp = 0) {
    const int lane = threadIdx.x & 63;
    float v[NPER], b[NPER];
    // every load of the token issued before any is used (clamped indices)
    if ((act == 1 || act == 3 || act == 4) && lane < 32) tab[lane] = sw_exp2f_tab[lane];
    const bool hasb = use_bias && bias && act != 4;       // qwen35 selects on the probabilities alone
#pragma unroll
    for (int i = 0; i < NPER; i++) {
        const int e = min(NPER * lane + i, E - 1);
        v[i] = src[e];
        b[i] = hasb ? bias[e] : 0.f;
    }
    // the sums of the softmax paths in expert order: lane l's slots, then lane l + 1's
    auto sum_f = [&](float *p) {
        float sum = 0.f;
        for (int l = 0; l < 64 && NPER * l < E; l++) {
#pragma unroll
            for (int i = 0; i < NPER; i++)
                if (NPER * l + i < E) sum += lanef(p[i], l);
        }
        return sum;
    };
    // (in double, for terms in [0, 1]: when every nonzero term is at least 2^-19, all terms
    // are multiples of 2^-42 and every partial sum of at most 1024 of them is below 2^11,
    // so each addition is exact and any order gives the sequential sum's bits -- a wave
    // tree then replaces the 64-step scan; a NaN or a smaller term takes the scan)
    auto sum_d = [&](float *p) {
        bool small = false;
#pragma unroll
        for (int i = 0; i < NPER; i++)
            if (NPER * lane + i < E && !(p[i] == 0.f || p[i] >= 0x1p-19f)) small = true;
        if (__ballot(small) == 0ull) {
            double t = 0.0;
#pragma unroll
            for (int i = 0; i < NPER; i++)
                if (NPER * lane + i < E) t += (double)p[i];
            return wave_xor_sum(t);
        }
        double sum = 0.0;
        for (int l = 0; l < 64 && NPER * l < E; l++) {
#pragma unroll
            for (int i = 0; i < NPER; i++)
                if (NPER * l + i < E) sum += (double)lanef(p[i], l);
        }
        return sum;
    };
    if (act == 1) {                                   // softmax (c/moe_math.h:68-72)
        wave_sync();
        float mx = -__builtin_inff();
        bool any = false;
#pragma unroll
        for (int i = 0; i < NPER; i++) {
            const int e = NPER * lane + i;
            if (e < E && v[i] == v[i]) { mx = any ? fmaxf(mx, v[i]) : v[i]; any = true; }
        }
        mx = wave_fmax(mx);
        const float r0 = __shfl(v[0], 0);             // expert 0
        if (r0 != r0) mx = r0;                        // a NaN in slot 0 propagates, as in the scan
#pragma unroll
        for (int i = 0; i < NPER; i++) v[i] = sw_expf_t(v[i] - mx, tab);
        const double sum = sum_d(v);                  // in expert order, in double (every lane the same)
        const float inv = (float)(1.0 / sum);
#pragma unroll
        for (int i = 0; i < NPER; i++) v[i] = v[i] * inv;
    } else if (act == 3 || act == 4) {
        // act 3: OLMoE's softmax_row (c/olmoe.c:212-216): max from -1e30 by a strict
        // scan, a float sum in expert order, each term divided by it.
        // act 4: qwen35's moe_route (c/qwen35.c:570-574): max from -inf by a
        // strict scan, a double sum in expert order, each term (float)(p / sum)
        // in double.  A strict scan skips NaN: the maximum of the other keys.
        wave_sync();
        float mx = act == 3 ? -1e30f : -__builtin_inff();
#pragma unroll
        for (int i = 0; i < NPER; i++) {
            const int e = NPER * lane + i;
            if (e < E && v[i] > mx) mx = v[i];
        }
        mx = wave_fmax(mx);
#pragma unroll
        for (int i = 0; i < NPER; i++) v[i] = sw_expf_t(v[i] - mx, tab);
        if (act == 3) {
            const float sum = sum_f(v);
#pragma unroll
            for (int i = 0; i < NPER; i++) v[i] = v[i] / sum;
        } else {
            const double sum = sum_d(v);
#pragma unroll
            for (int i = 0; i < NPER; i++) v[i] = (float)((double)v[i] / sum);
        }
    }
    uint32_t ko[NPER];                                // order key, 0 = invalid or taken (valid keys order above 0)
    uint32_t frm = 0;                                 // bit i: slot i is an expert with an invalid key
#pragma unroll
    for (int i = 0; i < NPER; i++) {
        const int e = NPER * lane + i;
        const float key = v[i] + b[i];
        ko[i] = (e < E && key > -1e30f) ? ord_f32(key) : 0u;
        if (e < E && ko[i] == 0u) frm |= 1u << i;
    }
    sk = 0; wk = 0.f;
    // the passes that find a valid key (as many as there are valid experts), then the
    // all-invalid fallback for the rest: by then every valid expert is taken, so the
    // unselected ones are those of frm
    int nv = 0;
#pragma unroll
    for (int i = 0; i < NPER; i++) nv += __builtin_popcountll(__ballot(ko[i] != 0u));
    const int KP = kp > 0 && kp < K ? kp : K;
    const int kv = KP < nv ? KP : nv;
    int a = 0;
    for (; a < kv; a++) {
        // this lane's best: the largest key, its first slot and that slot's weight
        uint32_t lm = ko[0];
#pragma unroll
        for (int i = 1; i < NPER; i++) lm = lm > ko[i] ? lm : ko[i];
        int ls = NPER - 1;
#pragma unroll
        for (int i = NPER - 2; i >= 0; i--) ls = ko[i] == lm ? i : ls;
        float vs = v[0];
#pragma unroll
        for (int i = 1; i < NPER; i++) vs = ls == i ? v[i] : vs;
        const uint32_t m = wave_umax(lm);
        const int bl = __builtin_ctzll(__ballot(lm == m));    // the lowest lane holding the maximum
        const int slot = __builtin_amdgcn_readlane(ls, bl);
        const float wb = lanef(vs, bl);               // the pick's weight: its unbiased score
        const bool win = lane == bl;
#pragma unroll
        for (int i = 0; i < NPER; i++) ko[i] = (win && ls == i) ? 0u : ko[i];
        if (lane == a) { sk = NPER * bl + slot; wk = wb; }
    }
    for (; a < KP; a++) {                             // nothing valid left: the lowest unselected id
        const unsigned long long bal = __ballot(frm != 0u);
        const int ls = frm ? __builtin_ctz(frm) : 0;
        const int bl = bal ? __builtin_ctzll(bal) : 0;
        float vs = v[0];
#pragma unroll
        for (int i = 1; i < NPER; i++) vs = ls == i ? v[i] : vs;
        const int slot = __builtin_amdgcn_readlane(ls, bl);
        const float wb = lanef(vs, bl);
        if (lane == bl) frm &= ~(1u << ls);
        if (lane == a) { sk = NPER * bl + slot; wk = wb; }
    }
    if (KP < K) {                                     // picks only: no weights wanted
    } else if (act == 4) {                            // qwen35: always, in double (c/qwen35.c:585-587)
        double tot = 0.0;
        for (int a = 0; a < K; a++) tot += (double)lanef(wk, a);
        wk = (float)((double)wk / tot);
    } else if (act == SW_ROUTE_INKLING) {             // c/inkling.c:1040-1043: the picks' and the shared
        float sum = 0.f;                              // gates' sigmoids summed in that order, each
        for (int a = 0; a < K; a++) sum += lanef(wk, a);   // * (route_scale * global_scale) / sum
        for (int j = 0; j < ns; j++) sum += src[E + j];
        const float f = rs / sum;
        wk = wk * f;
        if (wsh && lane < ns) wsh[lane] = src[E + lane] * f;
    } else if (norm) {                                // renormalised: summed in rank order
        float sm = 0.f;
        for (int a = 0; a < K; a++) sm += lanef(wk, a);
        wk = wk / sm;
    }
}

// ------------------------------------------------------------ limbs ----
// The activation side of the int4 dot8 GEMV (k_dot8.hip).  For each group of
// SW_RG consecutive inputs, with 2^e the smallest power of two above max|x|
// of the group, y = x * 2^-e in (-1, 1) is written as sum_{l=1..ND} d_l 8^-l
// with signed digits d_l in [-8, 7] (round to nearest, clamp, carry the exact
// remainder), ND = SW_ND = 7, so x ~= 2^(e - 3 ND) * D with the integer
// D = sum_l d_l 8^(ND - l), |D| < 2^21.2, and |error| <= 2^e 8^-ND.  D is stored
// as SW_NL = 6 digits of balanced base 16 (every digit in [-8, 7], a complete
// digit set for base 16; six cover |D| <= 8 (16^6 - 1) / 15), most significant
// first, so the dot8 Horner runs 6 limbs with shifts of 4 instead of 7 with
// shifts of 3 over the same integer.  Limb l of the group is 4 dwords of 32
// nibbles (input 8j + i at bits 4i of dword j, the weights' nibble order); the
// factor is 2^(e - 3 ND), or NaN for a group holding a NaN or an infinity.
#define SW_RG 32
// the group's exponent e (by the 32 lanes of a half-wave, v = this lane's
// input): 2^e the smallest power of two above max|x|, 0 for an all-zero
// group; bad = the group holds a NaN or an infinity.  The maximum is taken over
// the bits of |x| (non-negative floats order as their bits, and an infinity or a
// NaN lies above every finite value): within each 16-lane row by DPP, then the
// half-wave's two rows by one shuffle
__device__ __forceinline__ int limbs_exp(float v, bool &bad) {
    uint32_t mb = __builtin_bit_cast(uint32_t, v) & 0x7FFFFFFFu;
    mb = dpp_umax<0xB1>(mb);                         // quad_perm [1,0,3,2]
    mb = dpp_umax<0x4E>(mb);                         // quad_perm [2,3,0,1]
    mb = dpp_umax<0x141>(mb);                        // row_half_mirror
    mb = dpp_umax<0x140>(mb);                        // row_mirror
    const uint32_t o = (uint32_t)__shfl_xor((int)mb, 16, 32);
    mb = mb > o ? mb : o;
    bad = mb > 0x7F7FFFFFu;                          // NaN or inf
    int e = 0;
    if (mb != 0u && !bad) (void)frexpf(__builtin_bit_cast(float, mb), &e);   // m = f 2^e, f in [0.5, 1): 2^e > m
    return e;
}
// OR over the 8 lanes of each aligned group of 8 (DPP within a row)
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_or(uint32_t v) {
    return v | (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
// the next digit of y (|y| <= 1): round to nearest, clamp to [-8, 7]; y keeps
// the exact remainder (|y| <= 1)
__device__ __forceinline__ float limb_digit(float &y) {
    const float t = y * 8.0f;                         // exact
    float d = rintf(t);
    d = fminf(fmaxf(d, -8.0f), 7.0f);
    y = t - d;                                        // exact
    return d;
}
// one group by the 32 lanes of a half-wave; i = lane in the half
__device__ __forceinline__ void limbs_group(float v, int i, sw_u32x4 *__restrict__ dst, float *__restrict__ fdst) {
    bool bad;
    const int e = limbs_exp(v, bad);
    float y = ldexpf(v, -e);                          // exact: |y| < 1
    int D = 0;
#pragma unroll
    for (int l = 0; l < SW_ND; l++) D = D * 8 + (int)limb_digit(y);
    uint32_t dw[SW_NL];
#pragma unroll
    for (int l = SW_NL - 1; l >= 0; l--) {            // the least significant digit first
        const int d = ((D + 8) & 15) - 8;             // in [-8, 7], D - d a multiple of 16
        D = (D - d) >> 4;                             // exact
        uint32_t nib = ((uint32_t)d & 0xFu) << (4 * (i & 7));
        nib = dpp_or<0xB1>(nib);                      // quad_perm [1,0,3,2]
        nib = dpp_or<0x4E>(nib);                      // quad_perm [2,3,0,1]
        nib = dpp_or<0x141>(nib);                     // row_half_mirror: the other quad of the 8
        dw[l] = nib;                                  // lanes 8j.. hold dword j of limb l
    }
    if ((i & 7) == 0) {
        const int j = i >> 3;
#pragma unroll
        for (int l = 0; l < SW_NL; l++) ((uint32_t *)(dst + l))[j] = bad ? 0u : dw[l];
    }
    if (i == 0) *fdst = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 3 * SW_ND);
}


// ---- RMSNorm (c/moe_math.h:58-62), the stack glue ----
// The factor inv = 1 / sqrtf((float)(ss / D) + eps) of row xr, the squares summed in
// double (a product of two floats is exact in double): threads 0..RN_NT-1 of the
// block each over a fixed stride in ascending order (chunks of RN_CH loads issued
// together; past the row a thread adds +0.0), then a fixed tree over the waves
// (xor shuffles, then the RN_NT/64 wave sums left to right).  Threads beyond RN_NT
// only meet the block barrier.  v keeps a thread's values of the last chunk (the
// whole row when D <= RN_NT * RN_CH).  The double sum differs from the reference's
// sequential one only in its last bits, so the float it rounds to is the same
// unless the two straddle a float rounding point.  k_rmsnorm (k_glue.hip) and the
// routing stage's normalising blocks (sw_router.h) both use this, so they give the
// same bits.
#define RN_NT 256
#define RN_CH 16
__device__ __forceinline__ float rms_inv_block(const float *__restrict__ xr, int D, float eps, double *part,
                                               float (&v)[RN_CH]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double ss = 0.0;
    if (tid < RN_NT) {
        for (int i0 = 0; i0 < D; i0 += RN_NT * RN_CH) {
#pragma unroll
            for (int k = 0; k < RN_CH; k++) {
                const int i = i0 + tid + k * RN_NT;
                v[k] = i < D ? xr[i] : 0.f;
            }
#pragma unroll
            for (int k = 0; k < RN_CH; k++) ss += (double)v[k] * (double)v[k];
        }
        ss = wave_xor_sum(ss);
        if (lane == 0) part[wave] = ss;
    }
    __syncthreads();
    double tot = part[0];
    for (int q = 1; q < RN_NT / 64; q++) tot += part[q];
    return 1.f / sqrtf((float)(tot / D) + eps);
}

#endif
