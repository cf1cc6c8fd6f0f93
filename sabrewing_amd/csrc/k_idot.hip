// k_idot.hip -- the reference's IDOT int4 contract on the device (opt-in,
// per-row scales): c/moe_quant.h:48-82 (matmul_q4_k) and :141-182
// (matmul_q4_kb), the CPU tier's LAG_IDOT=1 (c/laguna.c:204-207).
//
//   activations: per 32-block b, am = max |x|, s = am / 127 (floored at 1e-12),
//                x_i -> (int8) lrint(x_i * (1 / s))                (k_idot_quant)
//   per row o:   acc = 0; for b ascending: acc = fma(s_b, (float) dot_b, acc),
//                dot_b the exact int8 x int4 dot of block b; y = acc * scale_o
//
// Every step is an exact integer or a correctly rounded IEEE operation, so the
// device reproduces the CPU kernel bit for bit (the reference build contracts
// `acc += s * dot` into an fma, c/Makefile's GNU-mode default).  The SiLU-GLU
// between the two projections uses this build's glibc-exact expf (sw_libm.h),
// x / (1 + expf(-x)) * u as siluf (c/moe_math.h:53).
//
// Int8 activations are stored per block as 8 dwords, permuted to meet the
// cheap nibble expansion: dword 2j holds inputs 8j, 8j+2, 8j+4, 8j+6 and dword
// 2j+1 inputs 8j+1, 8j+3, 8j+5, 8j+7 (the even and odd nibbles of packed
// weight dword j); the block's dot is order-free, being an exact integer.
#include "sw_hip.h"
#include "sw_libm.h"

#define ID_NT 512          // threads per rows block
#define ID_RB 32           // weight rows per block (gate_up: 16 gate + 16 up)
#define ID_TT 2            // tokens per pass

// one block of 32 inputs by the 32 lanes of a half-wave (i = lane in the half)
__device__ __forceinline__ void idot_block(float v, int i, uint32_t *__restrict__ dst, float *__restrict__ sdst) {
    float am = fabsf(v);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) am = fmaxf(am, __shfl_xor(am, o, 32));   // NaN lanes never win (as `a > am`)
    float s = am / 127.f;
    if (s < 1e-12f) s = 1e-12f;
    const float inv = 1.f / s;
    const int q = (int)rintf(v * inv);                    // lrintf: |v * inv| <= 127.x, NaN -> 0
    // input i = 8j + c goes to dword 2j + (c & 1), byte c >> 1
    const int j = i >> 3, c = i & 7;
    uint32_t b = ((uint32_t)q & 0xFFu) << (8 * (c >> 1));
    b |= __shfl_xor(b, 2, 32);
    b |= __shfl_xor(b, 4, 32);
    if ((c & 6) == 0) dst[2 * j + (c & 1)] = b;          // lanes 8j and 8j+1
    if (i == 0) *sdst = s;
}

// rows x[r, K] -> int8 xi[r][K/32][8 dwords], scales xs[r][K/32]
__global__ __launch_bounds__(256) void k_idot_quant(const float *__restrict__ x, int K, int rows, uint32_t *__restrict__ xi,
                                                    float *__restrict__ xs) {
    const int G = K / 32;
    const int tid = threadIdx.x, g = blockIdx.x * 8 + (tid >> 5), r = blockIdx.y;
    if (r >= rows || g >= G) return;                       // whole half-waves leave together
    idot_block(x[(int64_t)r * K + g * 32 + (tid & 31)], tid & 31, xi + ((int64_t)r * G + g) * 8, xs + (int64_t)r * G + g);
}

int sw_launch_idot_quant(hipStream_t st, const float *x, int rows, int K, uint32_t *xi, float *xs) {
    if (K % 32 || K > 8192 || rows <= 0) return -1;
    const int G = K / 32;
    SW_LAUNCH(k_idot_quant, dim3((unsigned)((G + 7) / 8), (unsigned)rows), dim3(256), 0, st, x, K, rows, xi, xs);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// the signed bytes of packed dword w's even nibbles (k = 8j + 0, 2, 4, 6) and odd ones
__device__ __forceinline__ int idot_even(uint32_t w) { return (int)(((w & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u); }
__device__ __forceinline__ int idot_odd(uint32_t w) { return (int)((((w >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u); }

struct IdotArgs {
    const uint8_t *q;       // [E * O, K/2]
    const float *s;         // [E * O] row scales
    int O, K, I;            // GLU: O = 2 I, rows of a block are gate i0.. and up i0..
    const uint32_t *xi;     // [rows][K/32][8]
    const float *xs;        // [rows][K/32]
    SwGroups grp;           // whole groups (no pass list)
    float *Y;               // GLU: h [T][I]; else [T][O]
};

// block (group bx, row block by): the block's rows against every token of the group,
// ID_TT at a time; thread (row slot ro, block g) forms the exact dots into LDS, then
// one thread per (row, token) runs the block chain in order
template <int GLU>
__global__ __launch_bounds__(ID_NT) void k_idot_rows(IdotArgs A) {
    extern __shared__ __align__(16) int dots[];            // [ID_RB][ID_TT][G]
    __shared__ float ys[ID_RB * ID_TT];
    const int K = A.K, G = K / 32, O = A.O;
    const int tid = threadIdx.x;
    const int RPS = ID_NT / G, NS = (ID_RB + RPS - 1) / RPS;
    const int ro = tid / G, g = tid - ro * G;
    const bool worker = ro < RPS;
    int e, beg, t0, tend;
    if (!grp_work(A.grp, (int)blockIdx.x, 1 << 30, e, beg, t0, tend)) return;
    const int by = (int)blockIdx.y;
    auto srow = [&](int lr) -> int64_t {                   // weight row of local row lr
        if (GLU) {
            const int i0 = by * (ID_RB / 2);
            return (int64_t)e * O + (lr < ID_RB / 2 ? i0 + lr : A.I + i0 + lr - ID_RB / 2);
        }
        return (int64_t)e * O + by * ID_RB + lr;
    };
    const int nrow = GLU ? ID_RB : min(ID_RB, O - by * ID_RB);
    for (int tb = t0; tb < tend; tb += ID_TT) {
        const int nt = min(ID_TT, tend - tb);
        if (worker) {
            uint32_t X[ID_TT][8];
#pragma unroll
            for (int t = 0; t < ID_TT; t++) {
                const int pr = beg + tb + (t < nt ? t : 0);
                const int64_t tok = A.grp.grow ? A.grp.grow[pr] : pr;
                const sw_u32x4 *xp = (const sw_u32x4 *)(A.xi + (tok * G + g) * 8);
                const sw_u32x4 a = xp[0], b = xp[1];
                X[t][0] = a.x; X[t][1] = a.y; X[t][2] = a.z; X[t][3] = a.w;
                X[t][4] = b.x; X[t][5] = b.y; X[t][6] = b.z; X[t][7] = b.w;
            }
            for (int s = 0; s < NS; s++) {
                const int lr = ro * NS + s;
                if (lr < nrow) {
                    const sw_u32x4 w = *(const sw_u32x4 *)(A.q + srow(lr) * (K / 2) + g * 16);
                    const int we[4] = {idot_even(w.x), idot_even(w.y), idot_even(w.z), idot_even(w.w)};
                    const int wo[4] = {idot_odd(w.x), idot_odd(w.y), idot_odd(w.z), idot_odd(w.w)};
#pragma unroll
                    for (int t = 0; t < ID_TT; t++) {
                        if (t < nt) {
                            int d = 0;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                d = __builtin_amdgcn_sdot4(we[j], (int)X[t][2 * j], d, false);
                                d = __builtin_amdgcn_sdot4(wo[j], (int)X[t][2 * j + 1], d, false);
                            }
                            dots[(lr * ID_TT + t) * G + g] = d;
                        }
                    }
                }
            }
        }
        __syncthreads();
        // the block chain of each (row, token), in block order
        for (int p = tid; p < nrow * nt; p += ID_NT) {
            const int lr = p / nt, t = p - lr * nt;
            const int pr = beg + tb + t;
            const int64_t tok = A.grp.grow ? A.grp.grow[pr] : pr;
            const float *xs = A.xs + tok * G;
            const int *dr = dots + (lr * ID_TT + t) * G;
            float acc = 0.f;
            for (int b = 0; b < G; b++) acc = __builtin_fmaf(xs[b], (float)dr[b], acc);
            const float y = acc * A.s[srow(lr)];
            if (GLU) ys[lr * ID_TT + t] = y;
            else A.Y[(int64_t)pr * O + by * ID_RB + lr] = y;
        }
        if (GLU) {
            __syncthreads();
            const int NO = ID_RB / 2;
            for (int p = tid; p < NO * nt; p += ID_NT) {
                const int i = p / nt, t = p - i * nt;
                const float yg = ys[i * ID_TT + t], yu = ys[(NO + i) * ID_TT + t];
                A.Y[(int64_t)(beg + tb + t) * A.I + by * NO + i] = yg / (1.f + sw_expf(-yg)) * yu;
            }
        }
        __syncthreads();
    }
}

static size_t idot_lds(int K) { return (size_t)ID_RB * ID_TT * (K / 32) * 4; }
static int idot_check(const SwQ4 &W, const SwGroups &g) {
    return W.gs != 0 || W.K % 32 || W.K > 8192 || g.ngroups_max <= 0 || (W.K / 32) > ID_NT ||
                   idot_lds(W.K) + ID_RB * ID_TT * 4 > 65536 ? -1 : 0;
}

// h[packed row][I] = silu(gate) * up, both projections in the IDOT contract
int sw_launch_idot_glu(hipStream_t st, SwQ4 W, const uint32_t *xi, const float *xs, SwGroups g, int I, float *h) {
    if (idot_check(W, g) || W.O != 2 * I || I % (ID_RB / 2)) return -1;
    const IdotArgs A = {W.q, W.s, W.O, W.K, I, xi, xs, g, h};
    SW_LAUNCH(k_idot_rows<1>, dim3((unsigned)g.ngroups_max, (unsigned)(I / (ID_RB / 2))), dim3(ID_NT), idot_lds(W.K), st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Y[packed row][O] in the IDOT contract
int sw_launch_idot_rows(hipStream_t st, SwQ4 W, const uint32_t *xi, const float *xs, SwGroups g, float *Y) {
    if (idot_check(W, g)) return -1;
    const IdotArgs A = {W.q, W.s, W.O, W.K, 0, xi, xs, g, Y};
    SW_LAUNCH(k_idot_rows<0>, dim3((unsigned)g.ngroups_max, (unsigned)((W.O + ID_RB - 1) / ID_RB)), dim3(ID_NT), idot_lds(W.K),
              st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
