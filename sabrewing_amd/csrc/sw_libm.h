// sw_libm.h -- bit-exact restatements of the host libm functions the
// reference's routing depends on, for evaluation inside gfx950 kernels.
//
// The reference gate runs on the host: sigmoid 1/(1+expf(-x))
// (c/moe_block.h:26), softmax expf(x - max) (c/moe_math.h:68-72) and softplus
// x > 20 ? x : log1pf(expf(x)) (c/moe_math.h:54), all through glibc.  Routing
// must match it bit for bit, so the device evaluates the same algorithms:
//
//   sw_expf   -- glibc >= 2.28 expf (ARM optimized-routines design, as built
//                for x86-64 with FMA): x*N/ln2 = k + r, N = 32, table of
//                2^(i/N) as IEEE double bit patterns with i<<47 removed, cubic
//                in r evaluated in double, one final rounding to float.
//   sw_log1pf -- glibc's s_log1pf (fdlibm lineage): argument reduction to
//                [sqrt(2)/2, sqrt(2)], correction term c, degree-7 even
//                polynomial in s = f/(2+f), float arithmetic throughout.
//
// Both are checked exhaustively (every one of the 2^32 float inputs) against
// the host's glibc by tests/test_libm_exact.py (a CPU build of this header),
// and against the host on the device by the GPU tests.  All arithmetic here is
// plain IEEE with explicit fma where the glibc build fuses; the library is
// compiled with -ffp-contract=off so nothing else is fused.
#ifndef SW_LIBM_H
#define SW_LIBM_H
#include <hip/hip_runtime.h>
#include <stdint.h>

__host__ __device__ static inline uint32_t sw_asu32(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ static inline float sw_asf32(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ static inline uint64_t sw_asu64(double f) { return __builtin_bit_cast(uint64_t, f); }
__host__ __device__ static inline double sw_asf64(uint64_t u) { return __builtin_bit_cast(double, u); }

// tab[i] = bits(2^(i/32)) - (i << 47)
#define SW_EXP2F_TAB                                                                            \
    { 0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull }

// the table lives in memory on both sides (a per-lane index into a local
// array would otherwise be lowered to register moves or private memory)
#if defined(__HIP_DEVICE_COMPILE__)
__device__ static const uint64_t sw_exp2f_tab[32] = SW_EXP2F_TAB;
#else
static const uint64_t sw_exp2f_tab[32] = SW_EXP2F_TAB;
#endif

// tab: the 32 entries above (sw_exp2f_tab, or a copy of it in LDS)
__host__ __device__ static inline float sw_expf_t(float x, const uint64_t *tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+5;       // 32 / ln 2
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-20, c1 = 0x1.ebfce50fac4f3p-13, c2 = 0x1.62e42ff0c52d6p-6;
    uint32_t abstop = (sw_asu32(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                                 // |x| >= 88, inf or nan
        if (sw_asu32(x) == 0xff800000u) return 0.0f;       // -inf
        if (abstop >= 0x7f8) return x + x;                 // +inf, nan
        if (x > 0x1.62e42ep6f) return sw_asf32(0x7f800000u);   // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;               // underflow
    }
    double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    uint64_t ki = sw_asu64(kd);
    kd = kd - shift;
    double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki & 31] + (ki << 47);
    double s = sw_asf64(t);
    double z = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}
__host__ __device__ static inline float sw_expf(float x) { return sw_expf_t(x, sw_exp2f_tab); }

__host__ __device__ static inline float sw_log1pf(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
    const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f,
                Lp4 = 2.2222198546e-01f, Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
                Lp7 = 1.4798198640e-01f;
    float hfsq, f = 0.f, c = 0.f, s, z, R, u;
    int32_t k, hx, hu = 0, ax;
    hx = (int32_t)sw_asu32(x);
    ax = hx & 0x7fffffff;
    k = 1;
    if (hx < 0x3ed413d7) {                                 // x < 0.41422
        if (ax >= 0x3f800000) {                            // x <= -1
            if (x == -1.0f) return sw_asf32(0xff800000u);
            return sw_asf32(0x7fc00000u);
        }
        if (ax < 0x31000000) {                             // |x| < 2^-29
            if (ax < 0x24800000) return x;
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) { k = 0; f = x; hu = 1; }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)sw_asu32(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);
            c = c / u;
        } else {
            u = x;
            hu = (int32_t)sw_asu32(u);
            k = (hu >> 23) - 127;
            c = 0.f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = sw_asf32((uint32_t)hu | 0x3f800000u);
        } else {
            k += 1;
            u = sw_asf32((uint32_t)hu | 0x3f000000u);
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    hfsq = 0.5f * f * f;
    if (hu == 0) {
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += (float)k * ln2_lo;
            return (float)k * ln2_hi + c;
        }
        R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
    }
    s = f / (2.0f + f);
    z = s * s;
    R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

// gate activations with the reference's expressions
__host__ __device__ static inline float sw_sigmoid_ref_t(float x, const uint64_t *tab) { return 1.0f / (1.0f + sw_expf_t(-x, tab)); }
__host__ __device__ static inline float sw_softplus_ref_t(float x, const uint64_t *tab) {
    return x > 20.0f ? x : sw_log1pf(sw_expf_t(x, tab));
}
__host__ __device__ static inline float sw_sigmoid_ref(float x) { return sw_sigmoid_ref_t(x, sw_exp2f_tab); }
__host__ __device__ static inline float sw_softplus_ref(float x) { return sw_softplus_ref_t(x, sw_exp2f_tab); }

// IEEE sqrtf (round to nearest) from the hardware estimate: the result is the
// float whose rounding interval holds sqrt(x), decided by comparing x with the
// squares of the midpoints to its neighbours.  A midpoint has 25 significant
// bits, so its square is exact in double; sqrt(x) of a float x is never a
// midpoint.  Two corrections cover an estimate within 2 ulp.
__device__ static inline float sw_sqrt_rn(float x) {
    if (!(x > 0.f) || x == __builtin_inff()) return __builtin_sqrtf(x);   // +-0, negative, NaN, inf
    float sc = 1.f;
    if (x < 1.17549435e-38f) { x *= 18446744073709551616.0f; sc = 2.3283064365386963e-10f; }  // subnormal: x 2^64, result 2^-32 (exact)
    float r = __builtin_sqrtf(x);
    const double xd = x;
    for (int it = 0; it < 2; it++) {
        const float d = __uint_as_float(__float_as_uint(r) - 1u), u = __uint_as_float(__float_as_uint(r) + 1u);
        const double md = 0.5 * ((double)d + (double)r), mu = 0.5 * ((double)r + (double)u);
        if (md * md > xd) r = d;
        else if (mu * mu < xd) r = u;
        else break;
    }
    return r * sc;
}

#endif
