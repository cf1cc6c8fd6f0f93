// k_gen.hip -- seeded synthetic weights and activations, generated in HBM.
//
// Element i of a tensor with seed `seed` is a SplitMix64 counter draw pair
// (2p, 2p+1), p = i/2, through Box-Muller in double (z0 = r cos, z1 = r sin,
// r = sqrt(-2 ln u1)), scaled by sigma and rounded once to f32.  ln and
// sin/cos are fixed sequences of IEEE +,-,*,/ and fma (no library calls), so
// the host restatement (sabrewing_amd/synth.py documents the stream) and this
// kernel produce identical bits; tests compare tensor hashes.
// int4 quantisation follows the reference converters: per-row (gs = 0,
// c/tools/convert_laguna_int4.py:49-60) or per-group (gs > 0,
// c/tools/convert_fp8_to_int4.py:54-85), s = max(amax/7, 1e-8),
// q = clip(rint(w/s), -8, 7), byte = (q_even+8) | (q_odd+8) << 4.
#include "sw_hip.h"

static int launch_err(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

__device__ __forceinline__ uint64_t g_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t g_u64(uint64_t seed, uint64_t i) { return g_mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull); }

__device__ __forceinline__ double g_ln(double x) {
    const double C[13] = {0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
                          0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4,
                          0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
                          0x1.47ae147ae147bp-5};
    uint64_t b = __builtin_bit_cast(uint64_t, x);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    b = (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m = __builtin_bit_cast(double, b);
    if (m > 0x1.6a09e667f3bcdp+0) { m = m * 0.5; e += 1; }
    const double f = m - 1.0;
    const double s = f / (2.0 + f);
    const double z = s * s;
    double p = C[12];
#pragma unroll
    for (int k = 11; k >= 0; k--) p = __builtin_fma(p, z, C[k]);
    return __builtin_fma((double)e, 0x1.62e42fefa39efp-1, (2.0 * s) * p);
}

__device__ __forceinline__ void g_sincos2pi(double u, double *sn, double *cs) {
    const double SC[10] = {0x1.0000000000000p+0, -0x1.5555555555555p-3, 0x1.1111111111111p-7, -0x1.a01a01a01a01ap-13,
                           0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33, -0x1.ae7f3e733b81fp-41,
                           0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57};
    const double CC[10] = {0x1.0000000000000p+0, -0x1.0000000000000p-1, 0x1.5555555555555p-5, -0x1.6c16c16c16c17p-10,
                           0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37,
                           0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53};
    const double u4 = u * 4.0;
    const int q = (int)u4;
    const double r = u4 - (double)q;
    const double t = (r - 0.5) * 0x1.921fb54442d18p+0;
    const double t2 = t * t;
    double ps = SC[9], pc = CC[9];
#pragma unroll
    for (int k = 8; k >= 0; k--) { ps = __builtin_fma(ps, t2, SC[k]); pc = __builtin_fma(pc, t2, CC[k]); }
    const double st = t * ps, ct = pc;
    const double cphi = (ct - st) * 0x1.6a09e667f3bcdp-1, sphi = (ct + st) * 0x1.6a09e667f3bcdp-1;
    switch (q & 3) {
    case 0: *cs = cphi; *sn = sphi; break;
    case 1: *cs = -sphi; *sn = cphi; break;
    case 2: *cs = -cphi; *sn = -sphi; break;
    default: *cs = sphi; *sn = -cphi; break;
    }
}

// the normal pair of elements (2p, 2p+1)
__device__ __forceinline__ void g_normal_pair(uint64_t seed, uint64_t p, double *z0, double *z1) {
    const uint64_t a = g_u64(seed, 2 * p), b = g_u64(seed, 2 * p + 1);
    const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(b >> 11) * 0x1.0p-53;
    const double r = __builtin_sqrt(-2.0 * g_ln(u1));
    double sn, cs;
    g_sincos2pi(u2, &sn, &cs);
    *z0 = r * cs;
    *z1 = r * sn;
}

__device__ __forceinline__ uint16_t g_bf16(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// out[i] = f32(sigma * normal(seed, offset + i)), optionally rounded to bf16 (kept as f32)
__global__ void k_gen_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, double sigma, int to_bf16) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t gi = offset + (uint64_t)i;
        double z0, z1;
        g_normal_pair(seed, gi >> 1, &z0, &z1);
        float v = (float)(sigma * ((gi & 1) ? z1 : z0));
        if (to_bf16) v = __builtin_bit_cast(float, (uint32_t)g_bf16(v) << 16);
        out[i] = v;
    }
}

__global__ void k_gen_bf16(uint16_t *out, int64_t n, uint64_t seed, uint64_t offset, double sigma) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t gi = offset + (uint64_t)i;
        double z0, z1;
        g_normal_pair(seed, gi >> 1, &z0, &z1);
        out[i] = g_bf16((float)(sigma * ((gi & 1) ? z1 : z0)));
    }
}

// group-scale int4: one thread per (row, group of gs); gs even, gs <= 128, K % gs == 0
__global__ void k_gen_q4_group(uint8_t *q, float *s, uint64_t seed, double sigma, int64_t row0, int64_t nrows, int K, int gs) {
    const int ng = K / gs;
    const int64_t n = nrows * ng;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < n; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t / ng;
        const int g = (int)(t % ng);
        const uint64_t base = (uint64_t)(row0 + r) * (uint64_t)K + (uint64_t)g * gs;   // even
        float w[128];
        float am = 0.f;
        for (int i = 0; i < gs; i += 2) {
            double z0, z1;
            g_normal_pair(seed, (base + i) >> 1, &z0, &z1);
            w[i] = (float)(sigma * z0);
            w[i + 1] = (float)(sigma * z1);
            const float a = fabsf(w[i]), b = fabsf(w[i + 1]);
            if (a > am) am = a;
            if (b > am) am = b;
        }
        float sc = am / 7.f;
        if (sc < 1e-8f) sc = 1e-8f;
        s[r * ng + g] = sc;
        uint8_t *qr = q + r * (K / 2) + g * gs / 2;
        for (int i = 0; i < gs; i += 2) {
            int q0 = (int)rintf(w[i] / sc), q1 = (int)rintf(w[i + 1] / sc);
            q0 = q0 < -8 ? -8 : (q0 > 7 ? 7 : q0);
            q1 = q1 < -8 ? -8 : (q1 > 7 ? 7 : q1);
            qr[i >> 1] = (uint8_t)((q0 + 8) | ((q1 + 8) << 4));
        }
    }
}

// per-row int4: one block per row
__global__ __launch_bounds__(256) void k_gen_q4_row(uint8_t *q, float *s, uint64_t seed, double sigma, int64_t row0, int K) {
    __shared__ float red[256];
    const int64_t r = blockIdx.x;
    const uint64_t base = (uint64_t)(row0 + r) * (uint64_t)K;
    float am = 0.f;
    for (int i = 2 * threadIdx.x; i < K; i += 512) {
        double z0, z1;
        g_normal_pair(seed, (base + i) >> 1, &z0, &z1);
        const float a = fabsf((float)(sigma * z0)), b = fabsf((float)(sigma * z1));
        if (a > am) am = a;
        if (b > am) am = b;
    }
    red[threadIdx.x] = am;
    __syncthreads();
    for (int o = 128; o; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    float sc = red[0] / 7.f;
    if (sc < 1e-8f) sc = 1e-8f;
    if (threadIdx.x == 0) s[r] = sc;
    for (int i = 2 * threadIdx.x; i < K; i += 512) {
        double z0, z1;
        g_normal_pair(seed, (base + i) >> 1, &z0, &z1);
        int q0 = (int)rintf((float)(sigma * z0) / sc), q1 = (int)rintf((float)(sigma * z1) / sc);
        q0 = q0 < -8 ? -8 : (q0 > 7 ? 7 : q0);
        q1 = q1 < -8 ? -8 : (q1 > 7 ? 7 : q1);
        q[r * (K / 2) + (i >> 1)] = (uint8_t)((q0 + 8) | ((q1 + 8) << 4));
    }
}

int sw_launch_gen_normal(hipStream_t st, float *out, int64_t n, uint64_t seed, uint64_t offset, double sigma, int to_bf16) {
    if (n <= 0) return 0;
    SW_LAUNCH(k_gen_normal, dim3((unsigned)sw_imin64((n + 255) / 256, 65536)), dim3(256), 0, st, out, n, seed,
                       offset, sigma, to_bf16);
    return launch_err();
}

int sw_launch_gen_bf16(hipStream_t st, uint16_t *out, int64_t n, uint64_t seed, uint64_t offset, double sigma) {
    if (n <= 0) return 0;
    SW_LAUNCH(k_gen_bf16, dim3((unsigned)sw_imin64((n + 255) / 256, 65536)), dim3(256), 0, st, out, n, seed,
                       offset, sigma);
    return launch_err();
}

int sw_launch_gen_q4(hipStream_t st, uint8_t *q, float *s, uint64_t seed, double sigma, int64_t row0, int64_t nrows, int K, int gs) {
    if (nrows <= 0) return 0;
    if (K % 2) return -1;
    if (gs > 0) {
        if (gs % 2 || K % gs || gs > 128) return -1;
        const int64_t n = nrows * (K / gs);
        SW_LAUNCH(k_gen_q4_group, dim3((unsigned)sw_imin64((n + 255) / 256, 65536)), dim3(256), 0, st, q, s, seed,
                           sigma, row0, nrows, K, gs);
    } else {
        for (int64_t r0 = 0; r0 < nrows; r0 += 65536) {
            const int64_t nr = sw_imin64(65536, nrows - r0);
            SW_LAUNCH(k_gen_q4_row, dim3((unsigned)nr), dim3(256), 0, st, q + r0 * (K / 2), s + r0, seed, sigma,
                               row0 + r0, K);
        }
    }
    return launch_err();
}
