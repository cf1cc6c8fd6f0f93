// k_lanes.hip -- the reference CPU's 16-lane GEMV contracts on gfx950, bit for
// bit: y[s, o] of a row-major weight matrix W [O, I] against rows of x.
//
// The reference's SIMD matmuls reduce each output in a fixed order that is
// part of their result.  Lane j of 16 keeps one f32 chain; the chains are
// then added by GCC's _mm512_reduce_add_ps tree (t8[j] = a[j] + a[j+8],
// t4[j] = t8[j] + t8[j+4], (t4[0] + t4[2]) + (t4[1] + t4[3])).  Two chain
// shapes cover the contracts this file serves:
//   F32X  lane j: acc = fma(x[i], w[i], acc) for i = j, j+16, j+32, ... while
//         a whole 16 (32 for int4) remain, then a scalar tail fused into the
//         sum.  Weights widen exactly: bf16 (c/moe_matmul.h:92-110, round_x =
//         0), int8 (matmul_q8_k F32, c/moe_quant.h:378-391), int4 nibble - 8
//         (matmul_q4_k F32, c/moe_quant.h:85-109); the int ones end in * scale.
//   DP    vdpbf16ps (round_x = 1, c/moe_matmul.h:66-89; inkling's matmul_h):
//         x rounded to bf16 (RNE, NaN quieted, a denormal input to a signed
//         zero), lane j takes the bf16 pair (2j, 2j+1) of every 32 columns,
//         two FMAs in a row -- the odd column first -- with denormal inputs
//         read as zero and a denormal result flushed to a signed zero.
//   I4G   matmul_i4_grouped (c/quant.h:168-203, its AVX2 body): per scale group
//         of gs columns 8 lanes, lane j: fma over columns i + j then i + 8 + j
//         for every 16 of the group, hsum8 ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)),
//         then a = fma(h, scale[o][g], a) over the groups in order.  The 16
//         lanes of a row take two groups at a time (lanes 0-7 the even, 8-15
//         the odd one); the group sums go through LDS to the row's lane 0,
//         which runs the ordered scale chain.  A group wider than a tile (gs a
//         multiple of 256) is taken by lanes 0-7 alone, their chains carried
//         across its tiles.
// Each (row, token) is one lane chain, so a result never depends on the
// shape of the launch that computed it.
//
// Block: 256 threads = 16 rows x 16 lanes; tiles of CC columns of the 16
// rows (coalesced 16-byte loads) and of up to TS tokens go through LDS, and
// each token's chains stay in registers across tiles.
#include "sw_hip.h"
#include "sw_libm.h"

#define LN_ROWS 16
#define LN_CC 256                  // columns per LDS tile

enum { WK_BF16 = 0, WK_I8 = 1, WK_I4 = 2, WK_I4G = 3 };

__device__ __forceinline__ float bf16_widen(uint32_t h) { return __builtin_bit_cast(float, h << 16); }
// a denormal to a signed zero (the DAZ / FTZ of vdpbf16ps)
__device__ __forceinline__ float flush_dn(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x7F800000u) ? v : __builtin_bit_cast(float, u & 0x80000000u);
}
// vcvtne2ps2bf16 of one float, widened back to f32
__device__ __forceinline__ float round_bf16_ne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return bf16_widen((u >> 16) | 0x40);
    if ((u & 0x7F800000u) == 0) return bf16_widen((u >> 16) & 0x8000);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return bf16_widen(u >> 16);
}

template <int WK> struct WElem { static constexpr int bits = WK == WK_BF16 ? 16 : WK == WK_I8 ? 8 : 4; };
// wave-local LDS ordering (the 16 lanes of a row are in one wave)
__device__ __forceinline__ void lanes_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// element i of an LDS row tile, widened exactly
template <int WK>
__device__ __forceinline__ float w_at(const uint8_t *row, int i) {
    if constexpr (WK == WK_BF16) return bf16_widen(((const uint16_t *)row)[i]);
    else if constexpr (WK == WK_I8) return (float)((const int8_t *)row)[i];
    else {
        const uint8_t b = row[i >> 1];
        return (float)((int)((i & 1) ? (b >> 4) : (b & 15)) - 8);
    }
}

struct LanesArgs {
    const void *W;          // [O, I]
    const float *scale;     // [O] (int weights), [O][I/gs] (I4G) or null
    const float *x;         // [S, I]
    float *y;               // [S, O]
    int S, I, O;
    int gs;                 // I4G: columns per scale group (16..256, dividing I)
    int ldx, ldy;           // row strides of x and y
};

// reduce16 over the 16 lanes of a row (xor partners stay inside the row)
__device__ __forceinline__ float reduce16_lanes(float v) {
    v = v + __shfl_xor(v, 8, 16);
    v = v + __shfl_xor(v, 4, 16);
    v = v + __shfl_xor(v, 2, 16);
    return v + __shfl_xor(v, 1, 16);
}

template <int WK, int DP, int TS>
__global__ __launch_bounds__(256) void k_lanes16(LanesArgs A) {
    constexpr int EB = WElem<WK == WK_I4G ? WK_I4 : WK>::bits;
    constexpr int RB = LN_CC * EB / 8;                 // bytes of one row tile
    constexpr int RS = RB + 32;                        // its LDS stride (+8 banks per row)
    __shared__ __align__(16) uint8_t wt[LN_ROWS * RS];
    __shared__ __align__(16) float xt[TS * LN_CC];
    __shared__ float hg[WK == WK_I4G ? LN_ROWS * TS * (LN_CC / 16) : 1];   // I4G: group sums of a tile
    const int tid = threadIdx.x, r = tid >> 4, j = tid & 15;
    const int o0 = blockIdx.x * LN_ROWS, s0 = blockIdx.y * TS;
    const int I = A.I, O = A.O, S = A.S;
    const int ns = min(TS, S - s0);
    // columns of the lane chains; the rest is the scalar tail (F32X) -- DP needs I % 32 == 0
    const int imain = DP || WK == WK_I4G ? I : (WK == WK_I4 ? I & ~31 : I & ~15);
    const uint8_t *W = (const uint8_t *)A.W;
    const size_t rowb = (size_t)I * EB / 8;
    float acc[TS], lg[TS];                             // lg: the lane chains of a group wider than a tile
#pragma unroll
    for (int t = 0; t < TS; t++) { acc[t] = 0.f; lg[t] = 0.f; }
    for (int c0 = 0; c0 < imain; c0 += LN_CC) {
        const int cn = min(LN_CC, imain - c0);         // a multiple of 16 (32 for DP and int4)
        // the 16 rows' tile: cn * EB / 8 bytes each, in 16-byte pieces (rows past O: zeros)
        const int rb = cn * EB / 8, pieces = (rb + 15) / 16;
        for (int p = tid; p < LN_ROWS * pieces; p += 256) {
            const int rr = p / pieces, q = p - rr * pieces;
            sw_u32x4 v = {0u, 0u, 0u, 0u};
            if (o0 + rr < O) {
                const uint8_t *src = W + (size_t)(o0 + rr) * rowb + (size_t)c0 * EB / 8 + 16 * q;
                if (16 * q + 16 <= rb && (((uintptr_t)src) & 15) == 0) v = *(const sw_u32x4 *)src;
                else {
                    uint8_t tmp[16] = {0};
                    for (int b = 0; b < 16 && 16 * q + b < rb; b++) tmp[b] = src[b];
                    v = *(const sw_u32x4 *)tmp;
                }
            }
            *(sw_u32x4 *)(wt + rr * RS + 16 * q) = v;
        }
        for (int p = tid; p < TS * cn; p += 256) {
            const int t = p / cn, cc = p - t * cn;
            float v = t < ns ? A.x[(size_t)(s0 + t) * A.ldx + c0 + cc] : 0.f;
            xt[t * LN_CC + cc] = DP ? round_bf16_ne(v) : v;
        }
        __syncthreads();
        const uint8_t *row = wt + r * RS;
        if constexpr (DP) {
            for (int k = 0; k < cn; k += 32) {
                const float wo = flush_dn(w_at<WK>(row, k + 2 * j + 1)), we = flush_dn(w_at<WK>(row, k + 2 * j));
#pragma unroll
                for (int t = 0; t < TS; t++) {
                    // the converted activations are never denormal; the accumulator is always a flushed result
                    acc[t] = flush_dn(__builtin_fmaf(xt[t * LN_CC + k + 2 * j + 1], wo, acc[t]));
                    acc[t] = flush_dn(__builtin_fmaf(xt[t * LN_CC + k + 2 * j], we, acc[t]));
                }
            }
        } else if constexpr (WK == WK_I4G) {
            const int gs = A.gs, ngt = cn / gs, half = j >> 3, jj = j & 7;
            float *hrow = hg + r * TS * (LN_CC / 16);
            if (gs > LN_CC) {
                // a group spans gs / LN_CC whole tiles: lanes 0-7 carry its chains across them,
                // and its hsum8 and scale fma follow its last tile
                if (half == 0) {
                    for (int i = 0; i < cn; i += 16) {
                        const float w0 = w_at<WK_I4>(row, i + jj), w1 = w_at<WK_I4>(row, i + 8 + jj);
#pragma unroll
                        for (int t = 0; t < TS; t++) {
                            lg[t] = __builtin_fmaf(xt[t * LN_CC + i + jj], w0, lg[t]);
                            lg[t] = __builtin_fmaf(xt[t * LN_CC + i + 8 + jj], w1, lg[t]);
                        }
                    }
                }
                if ((c0 + cn) % gs == 0) {                 // uniform
                    const int o = o0 + r;
                    const float sg = A.scale[(size_t)(o < O ? o : 0) * (I / gs) + (c0 + cn) / gs - 1];
#pragma unroll
                    for (int t = 0; t < TS; t++) {
                        float v = lg[t] + __shfl_xor(lg[t], 4, 8);
                        v = v + __shfl_xor(v, 2, 8);
                        v = v + __shfl_xor(v, 1, 8);
                        if (j == 0) acc[t] = __builtin_fmaf(v, sg, acc[t]);
                        lg[t] = 0.f;
                    }
                }
            }
            for (int g = half; g < ngt; g += 2) {          // this half's groups of the tile
                float ln[TS];
#pragma unroll
                for (int t = 0; t < TS; t++) ln[t] = 0.f;
                for (int i = g * gs; i < g * gs + gs; i += 16) {
                    const float w0 = w_at<WK_I4>(row, i + jj), w1 = w_at<WK_I4>(row, i + 8 + jj);
#pragma unroll
                    for (int t = 0; t < TS; t++) {
                        ln[t] = __builtin_fmaf(xt[t * LN_CC + i + jj], w0, ln[t]);
                        ln[t] = __builtin_fmaf(xt[t * LN_CC + i + 8 + jj], w1, ln[t]);
                    }
                }
#pragma unroll
                for (int t = 0; t < TS; t++) {             // hsum8 inside the 8 lanes of the half
                    float v = ln[t] + __shfl_xor(ln[t], 4, 8);
                    v = v + __shfl_xor(v, 2, 8);
                    v = v + __shfl_xor(v, 1, 8);
                    if (jj == 0) hrow[t * (LN_CC / 16) + g] = v;
                }
            }
            lanes_wave_sync();
            if (j == 0) {                                  // the ordered scale chain of the row
                const int o = o0 + r;
                const float *sc = A.scale + (size_t)(o < O ? o : 0) * (I / gs) + c0 / gs;
                for (int g = 0; g < ngt; g++) {
                    const float sg = sc[g];
#pragma unroll
                    for (int t = 0; t < TS; t++) acc[t] = __builtin_fmaf(hrow[t * (LN_CC / 16) + g], sg, acc[t]);
                }
            }
            lanes_wave_sync();
        } else {
            for (int k = 0; k < cn; k += 16) {
                const float w = w_at<WK>(row, k + j);
#pragma unroll
                for (int t = 0; t < TS; t++) acc[t] = __builtin_fmaf(xt[t * LN_CC + k + j], w, acc[t]);
            }
        }
        __syncthreads();
    }
    const int o = o0 + r;
#pragma unroll
    for (int t = 0; t < TS; t++) {
        float sm = WK == WK_I4G ? acc[t] : reduce16_lanes(acc[t]);    // I4G: lane 0 holds the row's sum
        if (j == 0 && t < ns && o < O) {
            const float *xs = A.x + (size_t)(s0 + t) * A.ldx;
            const uint8_t *wr = W + (size_t)o * rowb;
            if constexpr (WK == WK_I4) {               // the byte tail of c/moe_quant.h:105-108
                for (int i = imain; i + 1 < I; i += 2) {
                    const uint8_t b = wr[i >> 1];
                    const float lo = (float)((int)(b & 15) - 8), hi = (float)((int)(b >> 4) - 8);
                    sm = sm + __builtin_fmaf(xs[i], lo, xs[i + 1] * hi);
                }
            } else if constexpr (!DP) {
                for (int i = imain; i < I; i++) {
                    const float w = WK == WK_BF16 ? bf16_widen(((const uint16_t *)wr)[i]) : (float)((const int8_t *)wr)[i];
                    sm = __builtin_fmaf(xs[i], w, sm);
                }
            }
            if (WK != WK_I4G && A.scale) sm = sm * A.scale[o];
            A.y[(size_t)(s0 + t) * A.ldy + o] = sm;
        }
    }
}

template <int WK, int DP>
static void launch_lanes(hipStream_t st, const LanesArgs &A) {
    const int ts = A.S >= 16 ? 16 : A.S >= 8 ? 8 : A.S >= 4 ? 4 : 1;
    const dim3 block(256);
    if (ts == 16) SW_LAUNCH((k_lanes16<WK, DP, 16>), dim3((A.O + 15) / 16, (A.S + 15) / 16), block, 0, st, A);
    else if (ts == 8) SW_LAUNCH((k_lanes16<WK, DP, 8>), dim3((A.O + 15) / 16, (A.S + 7) / 8), block, 0, st, A);
    else if (ts == 4) SW_LAUNCH((k_lanes16<WK, DP, 4>), dim3((A.O + 15) / 16, (A.S + 3) / 4), block, 0, st, A);
    else SW_LAUNCH((k_lanes16<WK, DP, 1>), dim3((A.O + 15) / 16, A.S), block, 0, st, A);
}

// wkind 0 bf16, 1 int8 (+ scale), 2 per-row int4 (+ scale), 3 group-scaled int4
// (+ scale [O][I/gs]; gs dividing I, a multiple of 16 dividing 256 or a multiple of
// 256); dp: the vdpbf16ps
// contract (bf16 weights, I % 32 == 0)
int sw_launch_lanes16(hipStream_t st, const void *W, int wkind, int dp, const float *scale, const float *x, int S,
                      int I, int O, float *y, int gs) {
    return sw_launch_lanes16_ld(st, W, wkind, dp, scale, x, I, S, I, O, y, O, gs);
}

int sw_launch_lanes16_ld(hipStream_t st, const void *W, int wkind, int dp, const float *scale, const float *x, int ldx,
                         int S, int I, int O, float *y, int ldy, int gs) {
    if (!W || !x || !y || S <= 0 || I <= 0 || O <= 0 || ldx < I || ldy < O) return -1;
    if (dp && (wkind != WK_BF16 || I % 32)) return -1;
    if ((wkind == WK_I4 || wkind == WK_I4G) && (I & 1)) return -1;
    if (wkind == WK_I4G && (gs < 16 || gs % 16 || (gs <= LN_CC ? LN_CC % gs : gs % LN_CC) || I % gs)) return -1;
    if (wkind != WK_BF16 && !scale) return -1;
    const LanesArgs A = {W, wkind == WK_BF16 ? nullptr : scale, x, y, S, I, O, gs, ldx, ldy};
    if (dp) launch_lanes<WK_BF16, 1>(st, A);
    else if (wkind == WK_BF16) launch_lanes<WK_BF16, 0>(st, A);
    else if (wkind == WK_I8) launch_lanes<WK_I8, 0>(st, A);
    else if (wkind == WK_I4) launch_lanes<WK_I4, 0>(st, A);
    else if (wkind == WK_I4G) launch_lanes<WK_I4G, 0>(st, A);
    else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------ SiLU-GLU ----
// h = siluf(g) * u elementwise, siluf(x) = x / (1 + expf(-x)) with the glibc-exact
// expf (c/moe_math.h:53): the bits of the CPU's `g[i] = siluf(g[i]) * u[i]`
__global__ void k_silu_mul(const float *__restrict__ g, const float *__restrict__ u, int64_t n, float *__restrict__ h) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = g[i];
        h[i] = (v / (1.0f + sw_expf(-v))) * u[i];
    }
}

int sw_launch_silu_mul(hipStream_t st, const float *g, const float *u, int64_t n, float *h) {
    if (!g || !u || !h || n <= 0) return -1;
    SW_LAUNCH(k_silu_mul, dim3((unsigned)sw_imin64((n + 255) / 256, 4096)), dim3(256), 0, st, g, u, n, h);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
