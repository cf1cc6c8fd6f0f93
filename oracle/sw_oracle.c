/* sw_oracle.c -- CPU restatement of the sabrewing MoE-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see sw_oracle.h).  Built with -ffp-contract=off:
 * every fused multiply-add the reference gets from GCC's default contraction
 * (-O3 -march=native, GNU C => -ffp-contract=fast) is written here as an
 * explicit fmaf(), and nothing else is fused.  The SIMD reductions are
 * restated lane by lane:
 *   _mm512_reduce_add_ps (GCC avx512fintrin.h __MM512_REDUCE_OP):
 *       t8[j]=a[j]+a[j+8]; t4[j]=t8[j]+t8[j+4]; (t4[0]+t4[2]) + (t4[1]+t4[3])
 *   hsum256 (c/quant.h:20-24):
 *       ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7))
 *
 * Pinning: tests/test_oracle_ref.py checks every kernel here bit-for-bit
 * against oracle/_ref (the reference headers compiled from /root/reference),
 * tests/test_oracle_golden.py against the committed golden vectors, and
 * tests/test_oracle_math.py against closed forms and brute force. */
#include "sw_oracle.h"
#include <immintrin.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ======================= seeded synthetic data ======================= */

uint64_t sw_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* i-th draw of the SplitMix64 stream seeded with `seed` */
uint64_t sw_u64(uint64_t seed, uint64_t i) { return sw_mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull); }

uint64_t sw_tensor_seed(uint64_t base, int layer, int tensor_id) {
    uint64_t k = ((uint64_t)(uint32_t)layer << 8) | (uint64_t)(uint32_t)tensor_id;
    return sw_mix64(base ^ sw_mix64(k + 0x632BE59BD9B4E019ull));
}

/* Fixed-sequence double ln / sincos: only IEEE +,-,*,/ and explicit fma, so
 * any IEEE-754 machine (the HIP generator included) evaluates the same bits. */
static const double SW_LN_C[13] = {
    0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
    0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4,
    0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
    0x1.47ae147ae147bp-5 };
static const double SW_SIN_C[10] = {
    0x1.0000000000000p+0, -0x1.5555555555555p-3, 0x1.1111111111111p-7, -0x1.a01a01a01a01ap-13,
    0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33, -0x1.ae7f3e733b81fp-41,
    0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57 };
static const double SW_COS_C[10] = {
    0x1.0000000000000p+0, -0x1.0000000000000p-1, 0x1.5555555555555p-5, -0x1.6c16c16c16c17p-10,
    0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37,
    0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53 };
#define SW_PIO2   0x1.921fb54442d18p+0
#define SW_LN2    0x1.62e42fefa39efp-1
#define SW_SQRT2  0x1.6a09e667f3bcdp+0
#define SW_SQRTH  0x1.6a09e667f3bcdp-1

static double sw_ln(double x) {                 /* x in [2^-53, 1] */
    uint64_t b; memcpy(&b, &x, 8);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    b = (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m; memcpy(&m, &b, 8);
    if (m > SW_SQRT2) { m = m * 0.5; e += 1; }
    double f = m - 1.0;
    double s = f / (2.0 + f);
    double z = s * s;
    double p = SW_LN_C[12];
    for (int k = 11; k >= 0; k--) p = fma(p, z, SW_LN_C[k]);
    return fma((double)e, SW_LN2, (2.0 * s) * p);
}

static void sw_sincos2pi(double u, double *sn, double *cs) {   /* u in [0,1) */
    double u4 = u * 4.0;
    int q = (int)u4;
    double r = u4 - (double)q;
    double t = (r - 0.5) * SW_PIO2;
    double t2 = t * t;
    double ps = SW_SIN_C[9], pc = SW_COS_C[9];
    for (int k = 8; k >= 0; k--) { ps = fma(ps, t2, SW_SIN_C[k]); pc = fma(pc, t2, SW_COS_C[k]); }
    double st = t * ps, ct = pc;
    double cphi = (ct - st) * SW_SQRTH, sphi = (ct + st) * SW_SQRTH;
    switch (q & 3) {
    case 0: *cs = cphi;  *sn = sphi;  break;
    case 1: *cs = -sphi; *sn = cphi;  break;
    case 2: *cs = -cphi; *sn = -sphi; break;
    default: *cs = sphi; *sn = -cphi; break;
    }
}

double sw_normal(uint64_t seed, uint64_t i) {
    uint64_t p = i >> 1;
    uint64_t a = sw_u64(seed, 2 * p), b = sw_u64(seed, 2 * p + 1);
    double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
    double u2 = (double)(b >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * sw_ln(u1));
    double sn, cs; sw_sincos2pi(u2, &sn, &cs);
    return (i & 1) ? r * sn : r * cs;
}

void sw_fill_normal_f32(float *out, int64_t n, uint64_t seed, uint64_t offset, double sigma) {
    #pragma omp parallel for schedule(static) if(n >= 65536)
    for (int64_t i = 0; i < n; i++) out[i] = (float)(sigma * sw_normal(seed, offset + (uint64_t)i));
}

/* f32 -> bf16 round-to-nearest-even (c/tools/kernel_check.c:23 f2bf16) */
uint16_t sw_f32_to_bf16(float f) { uint32_t u; memcpy(&u, &f, 4); u += 0x7FFF + ((u >> 16) & 1); return (uint16_t)(u >> 16); }
/* exact widening (c/moe_math.h:51 bf16_f32) */
float sw_bf16_to_f32(uint16_t b) { uint32_t u = (uint32_t)b << 16; float f; memcpy(&f, &u, 4); return f; }
float sw_round_bf16(float x) { return sw_bf16_to_f32(sw_f32_to_bf16(x)); }
void sw_round_bf16_inplace(float *x, int64_t n) { for (int64_t i = 0; i < n; i++) x[i] = sw_round_bf16(x[i]); }
void sw_f32_to_bf16_array(uint16_t *out, const float *x, int64_t n) { for (int64_t i = 0; i < n; i++) out[i] = sw_f32_to_bf16(x[i]); }

uint64_t sw_fnv1a64(const void *p, size_t n, uint64_t h) {
    const uint8_t *b = (const uint8_t *)p;
    if (!h) h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 0x100000001b3ull; }
    return h;
}

/* ======================= int4 container quantisers ======================= */

/* per-row: c/tools/convert_laguna_int4.py:49-60 (s = amax/7, floor 1e-8);
 * per-group: c/tools/convert_fp8_to_int4.py:54-85 (s = max(amax/7, 1e-8),
 * scale layout s[o*ng + g]).  Both: q = clip(rint(w/s), -8, 7) in f32,
 * byte = (q_even + 8) | (q_odd + 8) << 4; an odd I leaves the last high nibble 0. */
static void quant_row(uint8_t *p, float *scale, const float *w, int I, int gs) {
    int egs = gs > 0 ? gs : I, ng = gs > 0 ? (I + gs - 1) / gs : 1;
    int rb = (I + 1) / 2;
    memset(p, 0, (size_t)rb);
    for (int g = 0; g < ng; g++) {
        int base = g * egs, end = base + egs < I ? base + egs : I;
        float am = 0.f;
        for (int i = base; i < end; i++) { float a = fabsf(w[i]); if (a > am) am = a; }
        float s = am / 7.f;
        if (s < 1e-8f) s = 1e-8f;
        scale[g] = s;
        for (int i = base; i < end; i++) {
            int q = (int)rintf(w[i] / s);
            if (q < -8) q = -8;
            if (q > 7) q = 7;
            uint8_t nib = (uint8_t)(q + 8);
            if (i & 1) p[i >> 1] |= (uint8_t)(nib << 4); else p[i >> 1] |= nib;
        }
    }
}

void sw_quant_i4(uint8_t *packed, float *scale, const float *w, int O, int I, int gs) {
    int rb = (I + 1) / 2, ng = gs > 0 ? (I + gs - 1) / gs : 1;
    #pragma omp parallel for schedule(static) if(O >= 64)
    for (int o = 0; o < O; o++)
        quant_row(packed + (int64_t)o * rb, scale + (int64_t)o * ng, w + (int64_t)o * I, I, gs);
}

void sw_gen_q4(uint8_t *packed, float *scale, uint64_t seed, double sigma,
               int64_t row0, int64_t nrows, int I, int gs) {
    int rb = (I + 1) / 2, ng = gs > 0 ? (I + gs - 1) / gs : 1;
    #pragma omp parallel
    {
        float *w = (float *)malloc((size_t)I * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < nrows; r++) {
            uint64_t off = (uint64_t)(row0 + r) * (uint64_t)I;
            for (int i = 0; i < I; i++) w[i] = (float)(sigma * sw_normal(seed, off + (uint64_t)i));
            quant_row(packed + r * rb, scale + r * ng, w, I, gs);
        }
        free(w);
    }
}

/* ======================= reductions ======================= */

static float reduce16(const float *a) {         /* GCC _mm512_reduce_add_ps */
    float t8[8], t4[4];
    for (int j = 0; j < 8; j++) t8[j] = a[j + 8] + a[j];
    for (int j = 0; j < 4; j++) t4[j] = t8[j + 4] + t8[j];
    return (t4[0] + t4[2]) + (t4[1] + t4[3]);
}
static float hsum8(const float *v) {            /* hsum256, c/quant.h:20-24 */
    return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
}

/* ======================= GEMV / GEMM contracts ======================= */

/* GLM router (c/colibri.c:2871-2874): logits by c/quant.h:98-102's f32 matmul,
 * `a += xs[i] * w[i]` for i ascending.  As GCC -O3 builds it for AVX-512 the
 * products of the first I - I % 8 inputs are vectorised (16 and 8 wide) and
 * rounded, then added in order; the last I % 8 are a scalar fma chain.  The
 * sum order is the source's either way.  Then sigmoidf (c/colibri.c:833) with
 * glibc expf and the selection score logit + bias. */
static float glm_dot(const float *x, const float *w, int I) {
    const int nv = I - I % 8;
    float a = 0.f;
    for (int i = 0; i < nv; i++) { const float p = x[i] * w[i]; a = a + p; }
    for (int i = nv; i < I; i++) a = fmaf(x[i], w[i], a);
    return a;
}
void sw_glm_logits(const float *x, const float *W, const float *bias, int D, int E, float *logit, float *choice) {
    for (int e = 0; e < E; e++) {
        const float lg = 1.f / (1.f + expf(-glm_dot(x, W + (int64_t)e * D, D)));
        logit[e] = lg;
        choice[e] = lg + bias[e];
    }
}
/* the dot alone (to compare with the compiled c/quant.h matmul) */
void sw_glm_matmul(float *y, const float *x, const float *W, int S, int I, int O) {
    for (int o = 0; o < O; o++)
        for (int s = 0; s < S; s++) y[(int64_t)s * O + o] = glm_dot(x + (int64_t)s * I, W + (int64_t)o * I, I);
}

/* ---- row tiles for the lane contracts below ----
 * A batch of S rows re-reads every weight row once per token, so the
 * restatements walk tiles of MT weight rows (widened once into f32) against
 * one token at a time, four rows side by side.  _mm256_fmadd_ps is eight
 * independent fmaf() (one rounding each), so lane j of a vector accumulator
 * is exactly the scalar chain ln[j] of the contract; the reductions are the
 * scalar reduce16 / hsum8 on the stored lanes.  Tiling changes which rows
 * are computed when, never the operations of one (token, row) pair. */
#define MT 16
static void store16(float *ln, __m256 lo, __m256 hi) { _mm256_storeu_ps(ln, lo); _mm256_storeu_ps(ln + 8, hi); }

/* 16-lane SIMD contract of c/moe_matmul.h:25-43 for four widened rows w0..w3 */
static void lane16_rows4(float *y4, const float *xs, const float *w, int I) {
    __m256 lo[4], hi[4];
    for (int r = 0; r < 4; r++) { lo[r] = _mm256_setzero_ps(); hi[r] = _mm256_setzero_ps(); }
    int i = 0;
    for (; i + 16 <= I; i += 16) {
        const __m256 xa = _mm256_loadu_ps(xs + i), xb = _mm256_loadu_ps(xs + i + 8);
        for (int r = 0; r < 4; r++) {
            lo[r] = _mm256_fmadd_ps(xa, _mm256_loadu_ps(w + (int64_t)r * I + i), lo[r]);
            hi[r] = _mm256_fmadd_ps(xb, _mm256_loadu_ps(w + (int64_t)r * I + i + 8), hi[r]);
        }
    }
    for (int r = 0; r < 4; r++) {
        float ln[16];
        store16(ln, lo[r], hi[r]);
        float sm = reduce16(ln);
        for (int k = i; k < I; k++) sm = fmaf(xs[k], w[(int64_t)r * I + k], sm);
        y4[r] = sm;
    }
}

/* y[s, o] for rows o of W (widened by `widen` into MT-row tiles) under the
 * 16-lane contract */
static void lane16_matmul(float *y, const float *x, int S, int I, int O,
                          void (*widen)(float *dst, const void *W, int64_t o0, int n, int I), const void *W) {
    const int nt = (O + MT - 1) / MT;
    #pragma omp parallel if((int64_t)S * O >= 512)
    {
        float *wv = (float *)aligned_alloc(64, ((size_t)MT * I * 4 + 63) / 64 * 64);
        #pragma omp for schedule(static)
        for (int t = 0; t < nt; t++) {
            const int o0 = t * MT, no = O - o0 < MT ? O - o0 : MT;
            widen(wv, W, o0, no, I);
            memset(wv + (int64_t)no * I, 0, (size_t)(MT - no) * I * 4);
            for (int s = 0; s < S; s++) {
                const float *xs = x + (int64_t)s * I;
                for (int r0 = 0; r0 < no; r0 += 4) {
                    float y4[4];
                    lane16_rows4(y4, xs, wv + (int64_t)r0 * I, I);
                    for (int r = 0; r < 4 && r0 + r < no; r++) y[(int64_t)s * O + o0 + r0 + r] = y4[r];
                }
            }
        }
        free(wv);
    }
}
static void widen_f32(float *dst, const void *W, int64_t o0, int n, int I) {
    memcpy(dst, (const float *)W + o0 * I, (size_t)n * I * 4);
}
static void widen_bf16(float *dst, const void *W, int64_t o0, int n, int I) {
    const uint16_t *w = (const uint16_t *)W + o0 * I;
    for (int64_t k = 0; k < (int64_t)n * I; k++) dst[k] = sw_bf16_to_f32(w[k]);
}

/* c/moe_matmul.h:25-55.  SIMD: lane j sums i = j mod 16 ascending with FMA,
 * reduce16, then the scalar tail fused into the sum.  exact: double sum. */
void sw_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O, int exact) {
    if (!exact) { lane16_matmul(y, x, S, I, O, widen_f32, W); return; }
    #pragma omp parallel for schedule(static) if((int64_t)S * O >= 512)
    for (int o = 0; o < O; o++) {
        const float *w = W + (int64_t)o * I;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            double sm = 0; for (int i = 0; i < I; i++) sm += (double)xs[i] * w[i];
            y[(int64_t)s * O + o] = (float)sm;
        }
    }
}

/* c/moe_matmul.h:65-122 at round_x=0: weight widened bf16->f32 exactly, same
 * lane contract as matmul_f32 (so a bf16 router equals an f32 router holding
 * the widened values, c/laguna.c:126-128). */
void sw_matmul_bf16(float *y, const float *x, const uint16_t *W, int S, int I, int O, int exact) {
    if (!exact) { lane16_matmul(y, x, S, I, O, widen_bf16, W); return; }
    #pragma omp parallel for schedule(static) if((int64_t)S * O >= 512)
    for (int o = 0; o < O; o++) {
        const uint16_t *w = W + (int64_t)o * I;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            double sm = 0; for (int i = 0; i < I; i++) sm += (double)xs[i] * sw_bf16_to_f32(w[i]);
            y[(int64_t)s * O + o] = (float)sm;
        }
    }
}

/* ---- the bf16 activation contract (round_x = 1) ----
 * c/moe_matmul.h:64-90 on an AVX512-BF16 host, inkling's matmul_h
 * (c/inkling.c:166-169): every activation rounded to bf16 by vcvtne2ps2bf16,
 * then per row 16 lanes, lane j taking the bf16 pair (2j, 2j+1) of each
 * 32-column chunk through vdpbf16ps -- two FMAs in a row, the odd column
 * first, each with denormal inputs read as zero and a denormal result
 * flushed to zero (Intel SDM, VDPBF16PS) -- then _mm512_reduce_add_ps.
 * With I % 32 != 0 the reference takes its f32-activation path instead. */
static float daz(float v) {
    uint32_t u; memcpy(&u, &v, 4);
    if ((u & 0x7F800000u) == 0 && (u & 0x007FFFFFu)) { u &= 0x80000000u; memcpy(&v, &u, 4); }
    return v;
}
/* vcvtne2ps2bf16 of one float: NaN quieted, denormal to a signed zero, else RNE */
uint16_t sw_f32_to_bf16_ne(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
    if ((u & 0x7F800000u) == 0) return (uint16_t)((u >> 16) & 0x8000);
    u += 0x7FFF + ((u >> 16) & 1);
    return (uint16_t)(u >> 16);
}
static float dp_step(float acc, float a, float b) { return daz(fmaf(daz(a), daz(b), daz(acc))); }

void sw_matmul_bf16_rx(float *y, const float *x, const uint16_t *W, int S, int I, int O) {
    if (I % 32) { sw_matmul_bf16(y, x, W, S, I, O, 0); return; }
    float *xb = (float *)malloc((size_t)S * I * 4);
    for (int64_t k = 0; k < (int64_t)S * I; k++) xb[k] = sw_bf16_to_f32(sw_f32_to_bf16_ne(x[k]));
    #pragma omp parallel for schedule(static) if((int64_t)S * O >= 512)
    for (int o = 0; o < O; o++) {
        const uint16_t *w = W + (int64_t)o * I;
        for (int s = 0; s < S; s++) {
            const float *xs = xb + (int64_t)s * I;
            float ln[16] = {0};
            for (int c = 0; c < I; c += 32)
                for (int j = 0; j < 16; j++) {
                    ln[j] = dp_step(ln[j], xs[c + 2 * j + 1], sw_bf16_to_f32(w[c + 2 * j + 1]));
                    ln[j] = dp_step(ln[j], xs[c + 2 * j], sw_bf16_to_f32(w[c + 2 * j]));
                }
            y[(int64_t)s * O + o] = reduce16(ln);
        }
    }
    free(xb);
}

/* int8 weights [O,I] with f32 row scales, c/moe_quant.h:346-400 (matmul_q8_k),
 * each of the S rows of x on its own.  F32: 16 lanes fmaf(x, (float)w) over
 * i = j mod 16, reduce16, the scalar tail fused, * scale.  IDOT: x to int8 per
 * 32-block (amax/127, lrintf), exact int dot per block, acc = fma(xs_b, dot,
 * acc) in block order, * scale (I % 32 == 0, I <= 8192).  An IDOT call of
 * another shape takes the scalar route: a double sum, (float)(sum * scale). */
void sw_matmul_q8(float *y, const float *x, const int8_t *q, const float *scale, int S, int I, int O, int mode) {
    if (mode == SW_Q4_IDOT && !(I % 32 == 0 && I <= 8192)) {
        for (int o = 0; o < O; o++)
            for (int s = 0; s < S; s++) {
                const int8_t *w = q + (int64_t)o * I; const float *xs = x + (int64_t)s * I;
                double sm = 0; for (int i = 0; i < I; i++) sm += (double)xs[i] * w[i];
                y[(int64_t)s * O + o] = (float)(sm * scale[o]);
            }
        return;
    }
    if (mode == SW_Q4_IDOT && I % 32 == 0 && I <= 8192) {
        const int nb = I / 32;
        for (int s = 0; s < S; s++) {
            const float *xr = x + (int64_t)s * I;
            int8_t xi[8192]; float xsb[256];
            for (int b = 0; b < nb; b++) {
                float am = 0.f; for (int i = 0; i < 32; i++) { float a = fabsf(xr[b * 32 + i]); if (a > am) am = a; }
                float sc = am / 127.f; if (sc < 1e-12f) sc = 1e-12f;
                xsb[b] = sc; float inv = 1.f / sc;
                for (int i = 0; i < 32; i++) xi[b * 32 + i] = (int8_t)lrintf(xr[b * 32 + i] * inv);
            }
            #pragma omp parallel for schedule(static)
            for (int o = 0; o < O; o++) {
                const int8_t *w = q + (int64_t)o * I;
                float acc = 0.f;
                for (int b = 0; b < nb; b++) {
                    int dot = 0;
                    for (int i = 0; i < 32; i++) dot += (int)xi[b * 32 + i] * (int)w[b * 32 + i];
                    acc = fmaf(xsb[b], (float)dot, acc);
                }
                y[(int64_t)s * O + o] = acc * scale[o];
            }
        }
        return;
    }
    #pragma omp parallel for schedule(static) if((int64_t)S * O >= 512)
    for (int o = 0; o < O; o++) {
        const int8_t *w = q + (int64_t)o * I;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float ln[16] = {0};
            int i = 0;
            for (; i + 16 <= I; i += 16)
                for (int j = 0; j < 16; j++) ln[j] = fmaf(xs[i + j], (float)w[i + j], ln[j]);
            float sm = reduce16(ln);
            for (; i < I; i++) sm = fmaf(xs[i], (float)w[i], sm);
            y[(int64_t)s * O + o] = sm * scale[o];
        }
    }
}

static inline int nib_at(const uint8_t *p, int col) {
    uint8_t b = p[col >> 1];
    return (col & 1) ? (b >> 4) : (b & 0xF);
}

/* per-row int4, c/moe_quant.h:45-217 (matmul_q4_k / matmul_q4_kb; every row
 * reduces in the S=1 order).
 *   F32 SIMD: 16 lanes, per 16 packed bytes two FMAs per lane -- columns
 *             2c+j then 2c+16+j -- reduce16, byte tail, * scale.
 *   IDOT:     x per 32-block to int8 (amax/127, floor 1e-12, lrintf), exact
 *             integer dot per block, acc = fma(xs_b, dot, acc), * scale.
 *   exact:    double sum, (float)(s * scale); also what IDOT degrades to when
 *             I % 32 != 0 or I > 8192 (c/moe_quant.h:48,85,115). */
void sw_matmul_q4(float *y, const float *x, const uint8_t *packed, const float *scale,
                  int S, int I, int O, int mode, int exact) {
    int rb = I / 2;
    if (mode != SW_Q4_F32 && !(mode == SW_Q4_IDOT && I % 32 == 0 && I <= 8192)) exact = 1;
    if (mode == SW_Q4_IDOT && I % 32 == 0 && I <= 8192) {
        int nb = I / 32;
        int8_t *xi = (int8_t *)malloc((size_t)S * I);
        float *xs = (float *)malloc((size_t)S * nb * sizeof(float));
        for (int s = 0; s < S; s++) {
            const float *xr = x + (int64_t)s * I;
            for (int b = 0; b < nb; b++) {
                const float *xb = xr + b * 32;
                float am = 0.f; for (int i = 0; i < 32; i++) { float a = fabsf(xb[i]); if (a > am) am = a; }
                float sc = am / 127.f; if (sc < 1e-12f) sc = 1e-12f;
                xs[(int64_t)s * nb + b] = sc; float inv = 1.f / sc;
                for (int i = 0; i < 32; i++) xi[(int64_t)s * I + b * 32 + i] = (int8_t)lrintf(xb[i] * inv);
            }
        }
        #pragma omp parallel for schedule(static)
        for (int o = 0; o < O; o++) {
            const uint8_t *p = packed + (int64_t)o * rb;
            for (int s = 0; s < S; s++) {
                float acc = 0.f;
                for (int b = 0; b < nb; b++) {
                    int dot = 0;
                    for (int i = 0; i < 32; i++) dot += (int)xi[(int64_t)s * I + b * 32 + i] * (nib_at(p, b * 32 + i) - 8);
                    acc = fmaf(xs[(int64_t)s * nb + b], (float)dot, acc);
                }
                y[(int64_t)s * O + o] = acc * scale[o];
            }
        }
        free(xi); free(xs);
        return;
    }
    #pragma omp parallel for schedule(static) if((int64_t)S * O >= 512)
    for (int o = 0; o < O; o++) {
        const uint8_t *p = packed + (int64_t)o * rb;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            if (exact) {
                double sm = 0;
                for (int c = 0; c < rb; c++) {
                    uint8_t b = p[c];
                    sm += (double)xs[2 * c] * ((int)(b & 0xF) - 8) + (double)xs[2 * c + 1] * ((int)(b >> 4) - 8);
                }
                y[(int64_t)s * O + o] = (float)(sm * scale[o]);
                continue;
            }
            float ln[16] = {0};
            int c = 0;
            for (; c + 16 <= rb; c += 16) {
                for (int j = 0; j < 16; j++) ln[j] = fmaf(xs[2 * c + j], (float)(nib_at(p, 2 * c + j) - 8), ln[j]);
                for (int j = 0; j < 16; j++) ln[j] = fmaf(xs[2 * c + 16 + j], (float)(nib_at(p, 2 * c + 16 + j) - 8), ln[j]);
            }
            float sm = reduce16(ln);
            for (; c < rb; c++) {
                uint8_t b = p[c];
                sm = sm + fmaf(xs[2 * c], (float)((int)(b & 0xF) - 8), xs[2 * c + 1] * (float)((int)(b >> 4) - 8));
            }
            y[(int64_t)s * O + o] = sm * scale[o];
        }
    }
}

/* group-scale int4, c/quant.h:168-203 (AVX2 body): per group an 8-lane FMA
 * chain, two FMAs per 16 columns (cols i..i+7 then i+8..i+15), hsum256, then
 * a = fma(h, scale, a); scalar tail for a group length not divisible by 16. */
/* the AVX2 body of c/quant.h:168-203 for four rows of decoded nibble values
 * w (n - 8 as floats, row r at w + r*I) and one token, when every group is a
 * whole number of 16-column steps: lane j of a group's accumulator is the
 * fmaf chain ln[j] over cols i+j then i+8+j, hsum8, a = fma(h, scale, a) */
static void i4g_rows4(float *y4, const float *xs, const float *w, const float *sc, int ng, int I, int gs) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (int g = 0; g < ng; g++) {
        const int base = g * gs;
        __m256 ln[4];
        for (int r = 0; r < 4; r++) ln[r] = _mm256_setzero_ps();
        for (int i = base; i < base + gs; i += 16) {
            const __m256 xa = _mm256_loadu_ps(xs + i), xb = _mm256_loadu_ps(xs + i + 8);
            for (int r = 0; r < 4; r++) {
                ln[r] = _mm256_fmadd_ps(xa, _mm256_loadu_ps(w + (int64_t)r * I + i), ln[r]);
                ln[r] = _mm256_fmadd_ps(xb, _mm256_loadu_ps(w + (int64_t)r * I + i + 8), ln[r]);
            }
        }
        for (int r = 0; r < 4; r++) {
            float v[8];
            _mm256_storeu_ps(v, ln[r]);
            a[r] = fmaf(hsum8(v), sc[(int64_t)r * ng + g], a[r]);
        }
    }
    for (int r = 0; r < 4; r++) y4[r] = a[r];
}

/* byte b -> {low nibble - 8, high nibble - 8} as floats (the even, odd column) */
static float nib_pair[256][2];
static void nib_pair_init(void) {
    for (int b = 0; b < 256; b++) { nib_pair[b][0] = (float)((b & 0xF) - 8); nib_pair[b][1] = (float)((b >> 4) - 8); }
}

void sw_matmul_i4_grouped(float *y, const float *x, const uint8_t *q4, const float *scale,
                          int S, int I, int O, int gs) {
    int rb = (I + 1) / 2, ng = (I + gs - 1) / gs;
    if (gs % 16 == 0 && I % gs == 0) {              /* tiles of MT rows, decoded once */
        if (nib_pair[0][0] == 0.f) nib_pair_init();
        const int nt = (O + MT - 1) / MT;
        #pragma omp parallel
        {
            float *wv = (float *)aligned_alloc(64, ((size_t)MT * I * 4 + 63) / 64 * 64);
            float *sv = (float *)malloc((size_t)MT * ng * 4);
            #pragma omp for schedule(static)
            for (int t = 0; t < nt; t++) {
                const int o0 = t * MT, no = O - o0 < MT ? O - o0 : MT;
                for (int r = 0; r < MT; r++) {
                    const uint8_t *w = q4 + (int64_t)(o0 + r) * rb;
                    float *d = wv + (int64_t)r * I;
                    if (r < no) for (int c = 0; c < I / 2; c++) memcpy(d + 2 * c, nib_pair[w[c]], 8);
                    else memset(d, 0, (size_t)I * 4);
                    for (int g = 0; g < ng; g++) sv[r * ng + g] = r < no ? scale[(int64_t)(o0 + r) * ng + g] : 0.f;
                }
                for (int s = 0; s < S; s++) {
                    const float *xs = x + (int64_t)s * I;
                    for (int r0 = 0; r0 < no; r0 += 4) {
                        float y4[4];
                        i4g_rows4(y4, xs, wv + (int64_t)r0 * I, sv + r0 * ng, ng, I, gs);
                        for (int r = 0; r < 4 && r0 + r < no; r++) y[(int64_t)s * O + o0 + r0 + r] = y4[r];
                    }
                }
            }
            free(wv); free(sv);
        }
        return;
    }
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        const float *scl = scale + (int64_t)o * ng;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float a = 0;
            for (int g = 0; g * gs < I; g++) {
                int base = g * gs, glen = gs;
                if (base + glen > I) glen = I - base;
                float sc = scl[g];
                int i = base;
                float ln[8] = {0};
                for (; i + 16 <= base + glen; i += 16) {
                    for (int j = 0; j < 8; j++) ln[j] = fmaf(xs[i + j], (float)(nib_at(w, i + j) - 8), ln[j]);
                    for (int j = 0; j < 8; j++) ln[j] = fmaf(xs[i + 8 + j], (float)(nib_at(w, i + 8 + j) - 8), ln[j]);
                }
                a = fmaf(hsum8(ln), sc, a);
                for (; i < base + glen; i += 2) {
                    uint8_t byte = w[i >> 1];
                    float lo = (float)((int)(byte & 0xF) - 8), hi = (float)((int)(byte >> 4) - 8);
                    if (i + 1 < base + glen) a = fmaf(fmaf(xs[i + 1], hi, xs[i] * lo), sc, a);
                    else a = fmaf(xs[i] * lo, sc, a);
                }
            }
            y[(int64_t)s * O + o] = a;
        }
    }
}

/* ======================= scalar math ======================= */

float sw_siluf(float x) { return x / (1.f + expf(-x)); }                         /* c/moe_math.h:53 */
float sw_softplusf(float x) { return x > 20.f ? x : log1pf(expf(x)); }           /* c/moe_math.h:54 */
float sw_sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }                    /* c/moe_block.h:26 */

/* host libm over arrays (the values the device restatements must reproduce) */
void sw_expf_array(float *y, const float *x, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = expf(x[i]); }
void sw_log1pf_array(float *y, const float *x, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = log1pf(x[i]); }

/* c/moe_math.h:68-72: max, expf(x-mx) summed in double, (float)(1/s) multiply */
void sw_softmax_row(float *x, int n) {
    float mx = x[0]; for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    double s = 0; for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); s += x[i]; }
    float inv = (float)(1.0 / s); for (int i = 0; i < n; i++) x[i] *= inv;
}

/* OLMoE's softmax_row (c/olmoe.c:212-216): max from -1e30 by a strict scan,
 * expf(x-m) summed in float in order, each term divided by the sum */
void sw_softmax_row_olmoe(float *x, int n) {
    float m = -1e30f; for (int i = 0; i < n; i++) if (x[i] > m) m = x[i];
    float s = 0; for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); s += x[i]; }
    for (int i = 0; i < n; i++) x[i] /= s;
}

/* qwen35's moe_route (c/qwen35.c:558-589): max from -inf by a strict scan,
 * expf(x-mx) summed in double, p = (float)(p / sum) in double; K passes over
 * the unused experts keeping the first, replaced by a strictly larger p (ties
 * -> lowest id); w = p of the picks, renormalised by their double sum */
void sw_moe_route_qwen(const float *logit, int E, int K, int *sel, float *w) {
    float *p = (float *)malloc((size_t)E * sizeof(float));
    unsigned char *used = (unsigned char *)calloc((size_t)E, 1);
    float mx = -INFINITY; for (int e = 0; e < E; e++) if (logit[e] > mx) mx = logit[e];
    double sum = 0; for (int e = 0; e < E; e++) { p[e] = expf(logit[e] - mx); sum += p[e]; }
    for (int e = 0; e < E; e++) p[e] = (float)(p[e] / sum);
    for (int a = 0; a < K; a++) {
        int best = -1;
        for (int e = 0; e < E; e++) { if (used[e]) continue; if (best < 0 || p[e] > p[best]) best = e; }
        used[best] = 1; sel[a] = best; w[a] = p[best];
    }
    double tot = 0; for (int a = 0; a < K; a++) tot += w[a];
    for (int a = 0; a < K; a++) w[a] = (float)(w[a] / tot);
    free(p); free(used);
}

/* c/moe_arch.h:64-89: K passes, strict > from -1e30 (ties -> lowest id), bias
 * for selection only, all-non-finite -> lowest unselected expert */
void sw_moe_topk(const float *score, const float *corr_bias, int use_bias, int E, int K, int *sel) {
    for (int a = 0; a < K; a++) {
        int best = -1; float bv = -1e30f;
        for (int e = 0; e < E; e++) {
            int used = 0; for (int b = 0; b < a; b++) if (sel[b] == e) { used = 1; break; }
            if (used) continue;
            float s = score[e] + (use_bias && corr_bias ? corr_bias[e] : 0.f);
            if (s > bv) { bv = s; best = e; }
        }
        if (best < 0) {
            for (int e = 0; e < E && best < 0; e++) {
                int used = 0; for (int b = 0; b < a; b++) if (sel[b] == e) { used = 1; break; }
                if (!used) best = e;
            }
            if (best < 0) best = 0;
        }
        sel[a] = best;
    }
}

/* c/moe_math.h:58-62 */
void sw_rmsnorm_row(float *out, const float *x, const float *w, int D, float eps) {
    double ss = 0; for (int i = 0; i < D; i++) ss += (double)x[i] * x[i];
    float inv = 1.f / sqrtf((float)(ss / D) + eps);
    for (int i = 0; i < D; i++) out[i] = x[i] * inv * w[i];
}

/* greedy argmax, lowest index wins ties */
int sw_argmax(const float *v, int n) {
    int b = 0; for (int i = 1; i < n; i++) if (v[i] > v[b]) b = i;
    return b;
}

/* ======================= MoE block ======================= */

/* router rows: the E routed experts, plus Inkling's shared-expert gate rows */
static int router_rows(const SwMoeDesc *d, int E) { return E + (d->route_act == SW_ROUTE_INKLING ? d->n_shared : 0); }
/* weights per token: K, plus Inkling's shared-expert weights */
static int weight_cols(const SwMoeDesc *d) { return d->topk + (d->route_act == SW_ROUTE_INKLING ? d->n_shared : 0); }

static void router_logits(const SwMoeDesc *d, const SwMoeLayer *L, const float *x, int S, int mode, float *rl) {
    int exact = mode == SW_MODE_EXACT, R = router_rows(d, L->E);
    if (L->router_bf16) sw_matmul_bf16(rl, x, (const uint16_t *)L->router, S, L->D, R, exact);
    else sw_matmul_f32(rl, x, (const float *)L->router, S, L->D, R, exact);
    if (L->logit_bias)
        for (int s = 0; s < S; s++) for (int e = 0; e < L->E; e++) rl[(int64_t)s * R + e] += L->logit_bias[e];
}

/* moe_block.h:115-122 (and c/laguna.c:697-706 per row) */
static void route_row(const SwMoeDesc *d, const SwMoeLayer *L, float *rl, float *sc, int *sel, float *w) {
    int E = d->n_experts, K = d->topk;
    if (d->route_act == SW_ROUTE_SOFTMAX_QWEN) { sw_moe_route_qwen(rl, E, K, sel, w); return; }
    if (d->route_act == SW_ROUTE_INKLING) {         /* c/inkling.c:1027-1043; w gets K + n_shared */
        for (int e = 0; e < E; e++) sc[e] = sw_sigmoidf(rl[e]);
        sw_moe_topk(sc, L->corr_bias, d->use_corr_bias, E, K, sel);
        float sum = 0.f;
        for (int a = 0; a < K; a++) { w[a] = sw_sigmoidf(rl[sel[a]]); sum += w[a]; }
        for (int j = 0; j < d->n_shared; j++) { w[K + j] = sw_sigmoidf(rl[E + j]); sum += w[K + j]; }
        for (int a = 0; a < K + d->n_shared; a++) w[a] *= d->route_scale / sum;
        return;
    }
    if (d->route_act == SW_ROUTE_SOFTMAX_OLMOE) {   /* c/olmoe.c:607-632: softmax_row, the moe_topk scan, norm */
        sw_softmax_row_olmoe(rl, E); for (int e = 0; e < E; e++) sc[e] = rl[e];
    } else if (d->route_act == SW_ROUTE_SOFTMAX) { sw_softmax_row(rl, E); for (int e = 0; e < E; e++) sc[e] = rl[e]; }
    else if (d->route_act == SW_ROUTE_SOFTPLUS) { for (int e = 0; e < E; e++) sc[e] = sw_softplusf(rl[e]); }
    else if (d->route_act == SW_ROUTE_SQRT_SOFTPLUS) {   /* c/deepseek.c:854 */
        for (int e = 0; e < E; e++) sc[e] = sqrtf(sw_softplusf(rl[e]));
    }
    else for (int e = 0; e < E; e++) sc[e] = 1.f / (1.f + expf(-rl[e]));
    sw_moe_topk(sc, L->corr_bias, d->use_corr_bias, E, K, sel);
    for (int a = 0; a < K; a++) w[a] = sc[sel[a]];
    if (d->norm_topk) { float sm = 0; for (int a = 0; a < K; a++) sm += w[a]; for (int a = 0; a < K; a++) w[a] /= sm; }
}

/* the gate + top-k of S rows of given logits (route_row on a copy of each) */
void sw_route_logits(const SwMoeDesc *d, const float *logits, int S, int *sel, float *w) {
    int E = d->n_experts, K = d->topk, R = router_rows(d, E), W = weight_cols(d);
    SwMoeLayer L; memset(&L, 0, sizeof L); L.E = E;
    float *rl = (float *)malloc((size_t)R * sizeof(float)), *sc = (float *)malloc((size_t)E * sizeof(float));
    for (int s = 0; s < S; s++) {
        memcpy(rl, logits + (int64_t)s * R, (size_t)R * sizeof(float));
        route_row(d, &L, rl, sc, sel + s * K, w + s * W);
    }
    free(rl); free(sc);
}

void sw_moe_route(const SwMoeDesc *d, const SwMoeLayer *L, const float *x, int S,
                  int mode, float *logits, int *sel, float *w) {
    int E = d->n_experts, K = d->topk, R = router_rows(d, E), W = weight_cols(d);
    float *rl = (float *)malloc((size_t)S * R * sizeof(float)), *sc = (float *)malloc((size_t)E * sizeof(float));
    router_logits(d, L, x, S, mode, rl);
    if (logits) memcpy(logits, rl, (size_t)S * R * sizeof(float));
    for (int s = 0; s < S; s++) route_row(d, L, rl + (int64_t)s * R, sc, sel + s * K, w + s * W);
    free(rl); free(sc);
}

/* int4 expert matmul dispatch: gs>0 -> matmul_i4_grouped (the only group-scale
 * CPU kernel), gs==0 -> matmul_q4_kb at the caller's mode (c/laguna.c:248-252) */
static void q4mm(float *y, const float *x, const uint8_t *p, const float *s, int S, int I, int O, int gs, int mode) {
    if (gs > 0) sw_matmul_i4_grouped(y, x, p, s, S, I, O, gs);
    else sw_matmul_q4(y, x, p, s, S, I, O, mode == SW_MODE_IDOT ? SW_Q4_IDOT : SW_Q4_F32, mode == SW_MODE_EXACT);
}

/* routed expert over n rows (c/laguna.c:577-595, batched form :744-752) */
static void expert_rows(const SwMoeLayer *L, int e, const float *x, int n, float *out, int mode, float *gu, float *glu) {
    int D = L->D, I = L->I, gs = L->gs;
    int ngD = gs > 0 ? (D + gs - 1) / gs : 1, ngI = gs > 0 ? (I + gs - 1) / gs : 1;
    const uint8_t *p13 = L->gu_q + (int64_t)e * 2 * I * ((D + 1) / 2);
    const float *s13 = L->gu_s + (int64_t)e * 2 * I * ngD;
    const uint8_t *p2 = L->dn_q + (int64_t)e * D * ((I + 1) / 2);
    const float *s2 = L->dn_s + (int64_t)e * D * ngI;
    q4mm(gu, x, p13, s13, n, D, 2 * I, gs, mode);
    for (int j = 0; j < n; j++) {
        const float *g = gu + (int64_t)j * 2 * I; float *o = glu + (int64_t)j * I;
        for (int i = 0; i < I; i++) o[i] = sw_siluf(g[i]) * g[I + i];
    }
    q4mm(out, glu, p2, s2, n, I, D, gs, mode);
}

static void resmm(float *y, const float *x, const void *W, int S, int I, int O, int f32w, int mode) {
    int exact = mode == SW_MODE_EXACT;
    if (f32w) sw_matmul_f32(y, x, (const float *)W, S, I, O, exact);
    else sw_matmul_bf16(y, x, (const uint16_t *)W, S, I, O, exact);
}

/* shared expert over S rows (c/laguna.c:596-604, batched :776-781) */
static void shared_rows(const SwMoeLayer *L, const float *x, int S, float *out, int mode) {
    int D = L->D, SI = L->Is;
    float *sg = (float *)malloc((size_t)S * SI * 4), *su = (float *)malloc((size_t)S * SI * 4);
    resmm(sg, x, L->sg, S, D, SI, L->shared_f32, mode);
    resmm(su, x, L->su, S, D, SI, L->shared_f32, mode);
    for (int64_t i = 0; i < (int64_t)S * SI; i++) sg[i] = sw_siluf(sg[i]) * su[i];
    resmm(out, sg, L->sd, S, SI, D, L->shared_f32, mode);
    free(sg); free(su);
}

/* shared expert j of Inkling's gated pool over S rows (c/inkling.c:1177-1181):
 * gate and up rows j*Is.., SiLU-GLU, down block j, all through matmul_h */
static void gated_rows(const SwMoeLayer *L, int j, const float *x, int S, float *out) {
    int D = L->D, SI = L->Is;
    const uint16_t *sg = (const uint16_t *)L->sg + (int64_t)j * SI * D, *su = (const uint16_t *)L->su + (int64_t)j * SI * D;
    const uint16_t *sd = (const uint16_t *)L->sd + (int64_t)j * D * SI;
    float *g = (float *)malloc((size_t)S * SI * 4), *u = (float *)malloc((size_t)S * SI * 4);
    sw_matmul_bf16_rx(g, x, sg, S, D, SI);
    sw_matmul_bf16_rx(u, x, su, S, D, SI);
    for (int64_t i = 0; i < (int64_t)S * SI; i++) g[i] = sw_siluf(g[i]) * u[i];
    sw_matmul_bf16_rx(out, g, sd, S, SI, D);
    free(g); free(u);
}

/* moe_block.h:109-145 with laguna's hooks (c/laguna.c:574-617); with
 * SW_ROUTE_INKLING the weights already hold the route scale (no scaling of the
 * routed sum) and SW_SHARED_GATED adds the gated shared experts after the
 * routed ranks (c/inkling.c:1011-1183) */
void sw_moe_block_rows(const SwMoeDesc *d, const SwMoeLayer *L, const float *x, float *out, int S, int mode) {
    int E = d->n_experts, K = d->topk, D = L->D, I = L->I;
    const int inkling = d->route_act == SW_ROUTE_INKLING;
    float *rl = (float *)malloc((size_t)router_rows(d, E) * 4), *sc = (float *)malloc((size_t)E * 4);
    float *w = (float *)malloc((size_t)weight_cols(d) * 4);
    int *sel = (int *)malloc((size_t)K * sizeof(int));
    float *scr = (float *)malloc((size_t)D * 4), *acc = (float *)malloc((size_t)D * 4);
    float *gu = (float *)malloc((size_t)2 * I * 4), *glu = (float *)malloc((size_t)I * 4);
    for (int s = 0; s < S; s++) {
        const float *xs = x + (int64_t)s * D; float *os = out + (int64_t)s * D;
        router_logits(d, L, xs, 1, mode, rl);
        route_row(d, L, rl, sc, sel, w);
        for (int i = 0; i < D; i++) acc[i] = 0;
        for (int a = 0; a < K; a++) {
            expert_rows(L, sel[a], xs, 1, scr, mode, gu, glu);
            for (int i = 0; i < D; i++) acc[i] = fmaf(w[a], scr[i], acc[i]);
        }
        if (!inkling) for (int i = 0; i < D; i++) acc[i] *= d->route_scale;
        if (d->shared_mode == SW_SHARED_GATED) {
            for (int j = 0; j < d->n_shared; j++) {
                gated_rows(L, j, xs, 1, scr);
                for (int i = 0; i < D; i++) acc[i] = fmaf(w[K + j], scr[i], acc[i]);
            }
        } else if (d->shared_mode != SW_SHARED_NONE) {
            shared_rows(L, xs, 1, scr, mode);
            for (int i = 0; i < D; i++) acc[i] += scr[i];
        }
        for (int i = 0; i < D; i++) os[i] += acc[i];
    }
    free(rl); free(sc); free(w); free(sel); free(scr); free(acc); free(gu); free(glu);
}

/* counting sort of c/laguna.c:708-727: groups in ascending expert id, packed
 * rows stable in (s, a) order */
int sw_bucket(const int *sel, int S, int K, int E, int *gexp, int *gbeg, int *gcnt, int *grow, int *rowof) {
    int T = S * K;
    int *cnt = (int *)calloc((size_t)E, sizeof(int)), *pos = (int *)malloc((size_t)E * sizeof(int));
    for (int i = 0; i < T; i++) cnt[sel[i]]++;
    int G = 0, off = 0;
    for (int e = 0; e < E; e++) {
        if (!cnt[e]) continue;
        gexp[G] = e; gbeg[G] = off; gcnt[G] = cnt[e]; pos[e] = off; off += cnt[e]; G++;
    }
    for (int s = 0; s < S; s++) for (int a = 0; a < K; a++) {
        int slot = pos[sel[s * K + a]]++;
        grow[slot] = s; rowof[s * K + a] = slot;
    }
    free(cnt); free(pos);
    return G;
}

/* lag_moe_group, c/laguna.c:689-786 (CPU tier) */
void sw_moe_group_rows(const SwMoeDesc *d, const SwMoeLayer *L, const float *x, float *out, int S, int mode) {
    int E = d->n_experts, K = d->topk, D = L->D, I = L->I, T = S * K, W = weight_cols(d);
    const int inkling = d->route_act == SW_ROUTE_INKLING;
    float *w = (float *)malloc((size_t)S * W * 4);
    int *sel = (int *)malloc((size_t)T * sizeof(int));
    sw_moe_route(d, L, x, S, mode, NULL, sel, w);
    int *gexp = (int *)malloc((size_t)E * sizeof(int)), *gbeg = (int *)malloc((size_t)E * sizeof(int));
    int *gcnt = (int *)malloc((size_t)E * sizeof(int));
    int *grow = (int *)malloc((size_t)T * sizeof(int)), *rowof = (int *)malloc((size_t)T * sizeof(int));
    int G = sw_bucket(sel, S, K, E, gexp, gbeg, gcnt, grow, rowof);
    float *slots = (float *)malloc((size_t)T * D * 4), *xg = (float *)malloc((size_t)S * D * 4);
    float *gu = (float *)malloc((size_t)S * 2 * I * 4), *glu = (float *)malloc((size_t)S * I * 4);
    for (int g = 0; g < G; g++) {
        int e = gexp[g], n = gcnt[g], beg = gbeg[g];
        for (int j = 0; j < n; j++) memcpy(xg + (int64_t)j * D, x + (int64_t)grow[beg + j] * D, (size_t)D * 4);
        expert_rows(L, e, xg, n, slots + (int64_t)beg * D, mode, gu, glu);
    }
    float *acc = (float *)malloc((size_t)S * D * 4);
    for (int s = 0; s < S; s++) {
        float *o = acc + (int64_t)s * D;
        for (int i = 0; i < D; i++) o[i] = 0;
        for (int a = 0; a < K; a++) {
            const float *v = slots + (int64_t)rowof[s * K + a] * D; float wa = w[(int64_t)s * W + a];
            for (int i = 0; i < D; i++) o[i] = fmaf(wa, v[i], o[i]);
        }
    }
    if (!inkling) for (int64_t i = 0; i < (int64_t)S * D; i++) acc[i] *= d->route_scale;
    if (d->shared_mode == SW_SHARED_GATED) {
        float *so = (float *)malloc((size_t)S * D * 4);
        for (int j = 0; j < d->n_shared; j++) {
            gated_rows(L, j, x, S, so);
            for (int s = 0; s < S; s++)
                for (int i = 0; i < D; i++) acc[(int64_t)s * D + i] = fmaf(w[(int64_t)s * W + K + j], so[(int64_t)s * D + i], acc[(int64_t)s * D + i]);
        }
        for (int64_t i = 0; i < (int64_t)S * D; i++) out[i] += acc[i];
        free(so);
    } else if (d->shared_mode != SW_SHARED_NONE) {
        float *so = (float *)malloc((size_t)S * D * 4);
        shared_rows(L, x, S, so, mode);
        for (int64_t i = 0; i < (int64_t)S * D; i++) out[i] += acc[i] + so[i];
        free(so);
    } else {
        for (int64_t i = 0; i < (int64_t)S * D; i++) out[i] += acc[i];
    }
    free(w); free(sel); free(gexp); free(gbeg); free(gcnt); free(grow); free(rowof);
    free(slots); free(xg); free(gu); free(glu); free(acc);
}
