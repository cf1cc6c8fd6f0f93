// k_gemm.hip -- grouped int4 and bf16 expert GEMMs on the gfx950 matrix cores.
//
// Work unit: one wave owns one 16-row tile of one group (an expert applied to
// a run of packed rows) and walks K itself (int4), or one K-quarter of it
// (bf16, KSPLIT = 4, quarters summed in LDS as (q0+q1)+(q2+q3)).  Either way
// the reduction of every output is fixed by the weight format alone, never by
// the batch, so the grouped path is bit-identical to the per-token path.
// Replaces the reference's warp-per-row mm_q4_kernel / mm_q4_group_kernel /
// grouped_*_g4 kernels (c/backend_cuda_laguna.cu:138-157,420-443;
// c/backend_cuda.cu:347-380), which re-read a weight row once per token: here
// a weight row is read once per launch and applied to every token of its
// group as MFMA columns (token t -> columns 2t (hi) and 2t+1 (lo)).
//
// Data movement per wave: weights stream HBM -> VGPRs through a ring of PF
// super-steps in flight; a group's activation planes are staged in LDS by the
// whole workgroup, chunk by chunk along K, double-buffered, so MFMA B
// fragments come from LDS (one ds_read_b128 each).
//
// int4 dequant (in registers): a 32-bit word holds 8 nibbles of one row;
// OR-ing a nibble into the mantissa of f16 1024.0 gives 1024+n exactly, and
// one packed add (or packed fma for nibbles sitting 4 bits higher) yields
// n-8 exactly.  Group scales (gs > 0) are folded into the f16 weight
// (f16(s*2^8) * (n-8), one rounding); per-row scales (gs == 0) are applied in
// f32 after the K loop, leaving the weights exact.
#include "sw_hip.h"
#include "sw_libm.h"

#define PF 8          // weight super-steps in flight per wave
enum { FMT_Q4 = 0, FMT_BF16 = 1 };
enum { EPI_GLU = 0, EPI_ROWS = 1 };

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
__device__ __forceinline__ float silu_glu(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// ------------------------------------------------------------ staging ----
// LDS holds, per buffer, 2*ntok rows (hi, lo of each token) x KSPLIT slices of
// ck halves (+8 halves of padding per row).  Slice q of chunk c covers
// k in [q*K/KSPLIT + c*ck, +ck).  The source is either precomputed planes
// (XSRC_PLANES: [2*rows, K] 16-bit) or f32 rows (XSRC_F32: [rows, K]) split
// into hi/lo on the way into LDS (f16 in the permuted MFMA order, or bf16).
enum { XSRC_PLANES = 0, XSRC_F32 = 1 };
#define SREG 6        // 16-byte staging registers per thread per chunk (LDS budget 40 KB)
#define LDS_BUDGET 40960

template <int XSRC, int KSPLIT>
__device__ __forceinline__ void stage_load(sw_u32x4 *regs, int nper, const void *__restrict__ src, int K, int ck,
                                           int c, int ntok, const int *rowsrc, int tid) {
    const int segq = ck / 8, segrow = KSPLIT * segq;
    if (XSRC == XSRC_PLANES) {
        const uint16_t *planes = (const uint16_t *)src;
        const int nseg = 2 * ntok * segrow;
        for (int i = 0; i < nper; i++) {
            const int seg = tid + 256 * i;
            if (seg < nseg) {
                const int row = seg / segrow, rs = seg % segrow, q = rs / segq, k = (rs % segq) * 8;
                const int sr = rowsrc[row >> 1];
                regs[i] = *(const sw_u32x4 *)(planes + (int64_t)(2 * sr + (row & 1)) * K + q * (K / KSPLIT) + c * ck + k);
            }
        }
    } else {
        const float *x = (const float *)src;
        const int nseg = ntok * segrow;
        for (int i = 0; i < nper; i++) {
            const int seg = tid + 256 * i;
            if (seg < nseg) {
                const int t = seg / segrow, rs = seg % segrow, q = rs / segq, k = (rs % segq) * 8;
                const float *p = x + (int64_t)rowsrc[t] * K + q * (K / KSPLIT) + c * ck + k;
                regs[2 * i] = *(const sw_u32x4 *)p;
                regs[2 * i + 1] = *(const sw_u32x4 *)(p + 4);
            }
        }
    }
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

template <int FMT, int XSRC, int KSPLIT>
__device__ __forceinline__ void stage_store(const sw_u32x4 *regs, int nper, uint16_t *lds, int ck, int ntok, int tid) {
    const int segq = ck / 8, segrow = KSPLIT * segq, rowlen = KSPLIT * ck + 8;
    if (XSRC == XSRC_PLANES) {
        const int nseg = 2 * ntok * segrow;
        for (int i = 0; i < nper; i++) {
            const int seg = tid + 256 * i;
            if (seg < nseg) {
                const int row = seg / segrow, rs = seg % segrow;
                *(sw_u32x4 *)(lds + row * rowlen + rs * 8) = regs[i];
            }
        }
    } else {
        const int nseg = ntok * segrow;
        for (int i = 0; i < nper; i++) {
            const int seg = tid + 256 * i;
            if (seg < nseg) {
                const int t = seg / segrow, rs = seg % segrow;
                const sw_f32x4 v0 = __builtin_bit_cast(sw_f32x4, regs[2 * i]), v1 = __builtin_bit_cast(sw_f32x4, regs[2 * i + 1]);
                sw_u32x4 hi, lo;
                if (FMT == FMT_Q4) {          // f16, 8-block order 0,4,1,5,2,6,3,7
                    const float v[8] = {v0.x, v1.x, v0.y, v1.y, v0.z, v1.z, v0.w, v1.w};
                    sw_half8 h, l;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const _Float16 a = (_Float16)v[j];
                        h[j] = a;
                        l[j] = (_Float16)(v[j] - (float)a);
                    }
                    hi = __builtin_bit_cast(sw_u32x4, h);
                    lo = __builtin_bit_cast(sw_u32x4, l);
                } else {                       // bf16, natural order
                    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                    uint16_t h[8], l[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        h[j] = f32_to_bf16_rne(v[j]);
                        l[j] = f32_to_bf16_rne(v[j] - bf16_to_f32(h[j]));
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        hi[j] = (uint32_t)h[2 * j] | ((uint32_t)h[2 * j + 1] << 16);
                        lo[j] = (uint32_t)l[2 * j] | ((uint32_t)l[2 * j + 1] << 16);
                    }
                }
                *(sw_u32x4 *)(lds + (2 * t) * rowlen + rs * 8) = hi;
                *(sw_u32x4 *)(lds + (2 * t + 1) * rowlen + rs * 8) = lo;
            }
        }
    }
}

struct GemmArgs {
    const void *w0, *w1;      // weight bases: rows of expert e at (e*rpe + r); w1 = second tile of the GLU pair
    const float *s0, *s1;     // scale bases (int4), same row indexing
    int rpe, K, gs;           // rows per expert, inputs, group size (0: per-row)
    SwGroups g;
    const void *xsrc;         // activations: planes [2*rows, K] (XSRC_PLANES) or f32 rows [rows, K] (XSRC_F32)
    int I;                    // GLU: output width (rows of w0 / w1 used: I each)
    void *out;
    int rowtiles;             // 16-row tiles (ROWS) or 8-pair tiles (GLU)
    int ck;                   // staging chunk (halves per K slice)
    int srows;                // LDS rows per staging buffer (2 x tokens per pass)
};

// accumulate one super-step of MFMAs for CB column blocks from LDS
template <int FMT, int CB>
__device__ __forceinline__ void mma_step(sw_f32x4 *acc, const sw_half8 *a16, const sw_u32x4 *abf, const uint16_t *lds,
                                         int rowlen, int kofs, int lane, int ncb, int ntok_pass) {
    const int c = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        if (cb < ncb) {
            const int t = cb * 8 + (c >> 1);
            const bool valid = t < ntok_pass;
            const uint16_t *bp = lds + (2 * t + (c & 1)) * rowlen + kofs + kb * 32;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                sw_u32x4 b = {0u, 0u, 0u, 0u};
                if (valid) b = *(const sw_u32x4 *)(bp + q * 8);
                if (FMT == FMT_Q4)
                    acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a16[q], __builtin_bit_cast(sw_half8, b), acc[cb], 0, 0, 0);
                else
                    acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sw_bf16x8, abf[q]),
                                                                      __builtin_bit_cast(sw_bf16x8, b), acc[cb], 0, 0, 0);
            }
        }
    }
}

template <int FMT, int EPI, int CB, int KSPLIT, int XSRC>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs A) {
    extern __shared__ __align__(16) uint16_t lds[];
    __shared__ int rowsrc[8 * CB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.x;
    const int gvalid = A.g.G ? *A.g.G : A.g.ngroups_max;
    if (g >= gvalid) return;
    const int rt = (KSPLIT == 1) ? (int)blockIdx.y * 4 + wave : (int)blockIdx.y;
    const int quarter = (KSPLIT == 1) ? 0 : wave;
    if (KSPLIT == 1 && (int)blockIdx.y * 4 >= A.rowtiles) return;
    const bool active = rt < A.rowtiles;
    const int e = A.g.gexp ? A.g.gexp[g] : 0, beg = A.g.gbeg ? A.g.gbeg[g] : 0;
    const int cnt = A.g.gcnt ? A.g.gcnt[g] : A.g.cnt_const;
    const int r = lane & 15, kb = lane >> 4;
    const int K = A.K, gs = A.gs;
    const int Kq = K / KSPLIT;
    const int rtc = active ? rt : 0;
    // this lane's weight row
    const int64_t wrow = (EPI == EPI_GLU) ? ((int64_t)e * A.rpe + rtc * 8 + (r & 7)) : ((int64_t)e * A.rpe + rtc * 16 + r);
    const bool second = (EPI == EPI_GLU) && (r >= 8);
    const int ng = gs > 0 ? K / gs : 1;
    const uint8_t *arow8 = nullptr;
    const uint16_t *arow16 = nullptr;
    const float *srow = nullptr;
    if (FMT == FMT_Q4) {
        arow8 = (const uint8_t *)(second ? A.w1 : A.w0) + wrow * (K / 2) + quarter * (Kq / 2) + kb * 16;
        srow = (second ? A.s1 : A.s0) + wrow * ng;
    } else {
        arow16 = (const uint16_t *)(second ? A.w1 : A.w0) + wrow * K + quarter * Kq + kb * 32;
    }
    const bool scaled = (FMT == FMT_Q4) && gs > 0;
    const int nss = Kq >> 7;
    const int ck = A.ck, nchunk = Kq / ck, sspc = ck >> 7;
    const int rowlen = KSPLIT * ck + 8;
    const int bufh = A.srows * rowlen;               // halves per LDS buffer
    const int tpass = A.srows / 2;                   // tokens per pass

    for (int t0 = 0; t0 < cnt; t0 += tpass) {
        const int ntok = min(tpass, cnt - t0);
        const int ncb = (ntok + 7) >> 3;
        __syncthreads();
        if (tid < ntok) rowsrc[tid] = A.g.grow ? A.g.grow[beg + t0 + tid] : beg + t0 + tid;
        __syncthreads();
        const int nseg = (XSRC == XSRC_PLANES ? 2 : 1) * ntok * KSPLIT * (ck / 8);
        const int nper = (nseg + 255) / 256;            // <= SREG (or SREG/2 for f32 rows) by the LDS budget
        sw_u32x4 sreg[SREG];
        stage_load<XSRC, KSPLIT>(sreg, nper, A.xsrc, K, ck, 0, ntok, rowsrc, tid);
        stage_store<FMT, XSRC, KSPLIT>(sreg, nper, lds, ck, ntok, tid);
        __syncthreads();
        if (nchunk > 1) stage_load<XSRC, KSPLIT>(sreg, nper, A.xsrc, K, ck, 1, ntok, rowsrc, tid);

        sw_f32x4 acc[CB];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[cb] = (sw_f32x4){0.f, 0.f, 0.f, 0.f};
        // weight ring: super-step ss lives in slot ss % PF
        sw_u32x4 ra[PF][FMT == FMT_BF16 ? 4 : 1];
        float sa[PF];
        if (active) {
#pragma unroll
            for (int u = 0; u < PF; u++) {
                if (u < nss) {
                    if (FMT == FMT_Q4) {
                        ra[u][0] = *(const sw_u32x4 *)(arow8 + u * 64);
                        sa[u] = scaled ? srow[(quarter * Kq + u * 128 + kb * 32) / gs] : 0.f;
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; q++) ra[u][FMT == FMT_BF16 ? q : 0] = *(const sw_u32x4 *)(arow16 + u * 128 + q * 8);
                    }
                }
            }
        }
        for (int ss0 = 0; ss0 < nss; ss0 += PF) {
#pragma unroll
            for (int u = 0; u < PF; u++) {
                const int ss = ss0 + u;
                if (ss < nss) {
                    const int c = ss / sspc;
                    if (ss > 0 && ss % sspc == 0) {          // chunk boundary (uniform in the block)
                        stage_store<FMT, XSRC, KSPLIT>(sreg, nper, lds + (c & 1) * bufh, ck, ntok, tid);
                        __syncthreads();
                        if (c + 1 < nchunk) stage_load<XSRC, KSPLIT>(sreg, nper, A.xsrc, K, ck, c + 1, ntok, rowsrc, tid);
                    }
                    if (active) {
                        sw_half8 a16[4];
                        sw_u32x4 abf[4];
                        if (FMT == FMT_Q4) {
                            const sw_u32x4 cur = ra[u][0];
                            const float cs = sa[u];
                            if (ss + PF < nss) {
                                ra[u][0] = *(const sw_u32x4 *)(arow8 + (ss + PF) * 64);
                                sa[u] = scaled ? srow[(quarter * Kq + (ss + PF) * 128 + kb * 32) / gs] : 0.f;
                            }
                            const _Float16 s16 = (_Float16)(cs * SW_WPRESCALE);
                            const sw_half2 s2 = {s16, s16};
                            a16[0] = dq8(cur.x, s2, scaled);
                            a16[1] = dq8(cur.y, s2, scaled);
                            a16[2] = dq8(cur.z, s2, scaled);
                            a16[3] = dq8(cur.w, s2, scaled);
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; q++) abf[q] = ra[u][FMT == FMT_BF16 ? q : 0];
                            if (ss + PF < nss) {
#pragma unroll
                                for (int q = 0; q < 4; q++)
                                    ra[u][FMT == FMT_BF16 ? q : 0] = *(const sw_u32x4 *)(arow16 + (ss + PF) * 128 + q * 8);
                            }
                        }
                        mma_step<FMT, CB>(acc, a16, abf, lds + (c & 1) * bufh + quarter * ck, rowlen, (ss % sspc) * 128,
                                          lane, ncb, ntok);
                    }
                }
            }
        }
        __syncthreads();

        // K-split reduction: quarters through LDS, (q0+q1)+(q2+q3)
        if (KSPLIT > 1) {
            float *red = (float *)lds;                   // 4 waves x CB x 64 lanes x 4
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
#pragma unroll
                for (int j = 0; j < 4; j++) red[((wave * CB + cb) * 64 + lane) * 4 + j] = acc[cb][j];
            __syncthreads();
            if (wave == 0) {
#pragma unroll
                for (int cb = 0; cb < CB; cb++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float p0 = red[((0 * CB + cb) * 64 + lane) * 4 + j], p1 = red[((1 * CB + cb) * 64 + lane) * 4 + j];
                        const float p2 = red[((2 * CB + cb) * 64 + lane) * 4 + j], p3 = red[((3 * CB + cb) * 64 + lane) * 4 + j];
                        acc[cb][j] = (p0 + p1) + (p2 + p3);
                    }
            }
            __syncthreads();
        }
        const bool writer = active && (KSPLIT == 1 || wave == 0);
        // epilogue: hi + lo, scale, then GLU or store
        const int rbase = 4 * (lane >> 4);
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            if (cb >= ncb) break;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float mine = acc[cb][j];
                v[j] = mine + __shfl_xor(mine, 1);        // even lanes: hi + lo
            }
            if (FMT == FMT_Q4) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (scaled) {
                        v[j] = v[j] * SW_WPRESCALE_INV;
                    } else {
                        const int rr = rbase + j;
                        const int64_t wr = (EPI == EPI_GLU) ? ((int64_t)e * A.rpe + rtc * 8 + (rr & 7)) : ((int64_t)e * A.rpe + rtc * 16 + rr);
                        const float *sb = (EPI == EPI_GLU && rr >= 8) ? A.s1 : A.s0;
                        v[j] = v[j] * sb[wr];
                    }
                }
            }
            const int t = t0 + cb * 8 + ((lane & 15) >> 1);
            const bool evenc = (lane & 1) == 0;
            if (EPI == EPI_GLU) {
                float up[4];
#pragma unroll
                for (int j = 0; j < 4; j++) up[j] = __shfl_xor(v[j], 32);
                if (writer && lane < 32 && evenc && t < cnt) {
                    const int64_t row = 2 * (int64_t)(beg + t);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int i = rtc * 8 + rbase + j;
                        const float h = silu_glu(v[j], up[j]);
                        if (FMT == FMT_Q4) {
                            _Float16 *hp = (_Float16 *)A.out;
                            const _Float16 hi = (_Float16)h;
                            const _Float16 lo = (_Float16)(h - (float)hi);
                            hp[row * A.I + plane_pos(i)] = hi;
                            hp[(row + 1) * A.I + plane_pos(i)] = lo;
                        } else {
                            uint16_t *hp = (uint16_t *)A.out;
                            const uint16_t hi = f32_to_bf16_rne(h);
                            const uint16_t lo = f32_to_bf16_rne(h - bf16_to_f32(hi));
                            hp[row * A.I + i] = hi;
                            hp[(row + 1) * A.I + i] = lo;
                        }
                    }
                }
            } else {
                if (writer && evenc && t < cnt) {
                    float *Y = (float *)A.out;
                    *(sw_f32x4 *)(Y + (int64_t)(beg + t) * A.rpe + rtc * 16 + rbase) = (sw_f32x4){v[0], v[1], v[2], v[3]};
                }
            }
        }
    }
}

// ------------------------------------------------- down + combine (one token) ----
// For a single token: out[d] += (sum_a w[a] * y_a[d]) * route_scale (+ shared[d]),
// y_a = down_{sel[a]}(h_a), for one 16-row d tile per block.  Each wave runs
// the ranks a = wave, wave+4, ... with the same per-output MFMA chain as the
// grouped kernel (so y_a is bit-identical to its slot value there), parks y_a
// in LDS, and one wave sums the ranks in order with one fma per rank, the
// operation sequence of k_combine.
#define DC_MAXK 64
__global__ __launch_bounds__(256) void k_q4_down_combine(SwQ4 W, const _Float16 *__restrict__ hp, const int *__restrict__ sel,
                                                         const float *__restrict__ wts, int K, float route_scale,
                                                         const float *__restrict__ shared, float *__restrict__ out) {
    extern __shared__ __align__(16) uint16_t lds[];   // staged h planes: 2K rows x (I + 8) halves
    __shared__ float ys[DC_MAXK][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int I = W.K, D = W.O, gs = W.gs;
    const int dt = blockIdx.x;
    const int rowlen = I + 8;
    // stage every rank's planes (rows 2a hi, 2a+1 lo)
    {
        const int segrow = I / 8, nseg = 2 * K * segrow;
        for (int seg = tid; seg < nseg; seg += 256) {
            const int row = seg / segrow, k = (seg % segrow) * 8;
            *(sw_u32x4 *)(lds + row * rowlen + k) = *(const sw_u32x4 *)((const uint16_t *)hp + (int64_t)row * I + k);
        }
    }
    __syncthreads();
    const int r = lane & 15, kb = lane >> 4, c = lane & 15;
    const int ng = gs > 0 ? I / gs : 1;
    const bool scaled = gs > 0;
    const int nss = I >> 7;
    const int nmine = (K - wave + 3) / 4;               // ranks of this wave
    const int nsteps = nmine * nss;
    sw_u32x4 ra[PF];
    float sa[PF];
    auto arow_of = [&](int ai) -> const uint8_t * {
        const int e = sel[wave + 4 * ai];
        return W.q + ((int64_t)e * D + dt * 16 + r) * (I / 2) + kb * 16;
    };
    auto srow_of = [&](int ai) -> const float * {
        const int e = sel[wave + 4 * ai];
        return W.s + ((int64_t)e * D + dt * 16 + r) * ng;
    };
#pragma unroll
    for (int u = 0; u < PF; u++) {
        if (u < nsteps) {
            const int ai = u / nss, ss = u % nss;
            ra[u] = *(const sw_u32x4 *)(arow_of(ai) + ss * 64);
            sa[u] = scaled ? srow_of(ai)[(ss * 128 + kb * 32) / gs] : 0.f;
        }
    }
    sw_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < nsteps; i0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int i = i0 + u;
            if (i < nsteps) {
                const int ai = i / nss, ss = i % nss, a = wave + 4 * ai;
                const sw_u32x4 cur = ra[u];
                const float cs = sa[u];
                if (i + PF < nsteps) {
                    const int an = (i + PF) / nss, sn = (i + PF) % nss;
                    ra[u] = *(const sw_u32x4 *)(arow_of(an) + sn * 64);
                    sa[u] = scaled ? srow_of(an)[(sn * 128 + kb * 32) / gs] : 0.f;
                }
                const _Float16 s16 = (_Float16)(cs * SW_WPRESCALE);
                const sw_half2 s2 = {s16, s16};
                sw_half8 a16[4];
                a16[0] = dq8(cur.x, s2, scaled);
                a16[1] = dq8(cur.y, s2, scaled);
                a16[2] = dq8(cur.z, s2, scaled);
                a16[3] = dq8(cur.w, s2, scaled);
                const uint16_t *bp = lds + (2 * a + (c & 1)) * rowlen + ss * 128 + kb * 32;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    sw_u32x4 b = {0u, 0u, 0u, 0u};
                    if (c < 2) b = *(const sw_u32x4 *)(bp + q * 8);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a16[q], __builtin_bit_cast(sw_half8, b), acc, 0, 0, 0);
                }
                if (ss == nss - 1) {                    // rank finished: hi + lo, scale, park in LDS
                    const int rbase = 4 * (lane >> 4);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float mine = acc[j];
                        float v = mine + __shfl_xor(mine, 1);
                        if (scaled) v = v * SW_WPRESCALE_INV;
                        else v = v * W.s[(int64_t)sel[a] * D + dt * 16 + rbase + j];
                        if (c == 0) ys[a][rbase + j] = v;
                    }
                    acc = (sw_f32x4){0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    }
    __syncthreads();
    if (tid < 16) {
        const int d = dt * 16 + tid;
        float s = 0.f;
        for (int a = 0; a < K; a++) s = __builtin_fmaf(wts[a], ys[a][tid], s);
        s = s * route_scale;
        if (shared) s = s + shared[d];
        out[d] = out[d] + s;
    }
}

// ---------------------------------------------------------------- launch ----
static int launch_err(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

// staging chunk: the largest multiple of 128 dividing K/KSPLIT whose double
// buffer fits the LDS budget for 8*CB tokens
static int pick_ck(int Kq, int rows, int ksplit) {
    for (int ck = Kq; ck >= 128; ck -= 128) {
        if (Kq % ck) continue;
        const int bytes = 2 * rows * (ksplit * ck + 8) * 2;
        if (bytes <= LDS_BUDGET) return ck;
    }
    return 0;
}

// maxtok: an upper bound of the tokens of any group (sizes the LDS staging)
template <int FMT, int EPI, int KSPLIT, int XSRC>
static int launch_gemm(hipStream_t st, GemmArgs a, int cb, int maxtok) {
    const int Kq = a.K / KSPLIT;
    if (a.K % (128 * KSPLIT) || a.g.ngroups_max <= 0 || a.rowtiles <= 0) return -1;
    if (FMT == FMT_Q4 && a.gs > 0 && (a.gs % 32 || a.K % a.gs)) return -1;
    const int rows = 2 * (maxtok < 8 * cb ? maxtok : 8 * cb);
    a.ck = pick_ck(Kq, rows, KSPLIT);
    a.srows = rows;
    if (!a.ck) return -1;
    const size_t lds = (size_t)2 * rows * (KSPLIT * a.ck + 8) * 2;
    const size_t red = KSPLIT > 1 ? (size_t)4 * cb * 64 * 4 * 4 : 0;
    const size_t shm = lds > red ? lds : red;
    dim3 grid((unsigned)a.g.ngroups_max, (unsigned)(KSPLIT == 1 ? (a.rowtiles + 3) / 4 : a.rowtiles));
    if (cb <= 1) hipLaunchKernelGGL((k_gemm<FMT, EPI, 1, KSPLIT, XSRC>), grid, dim3(256), shm, st, a);
    else hipLaunchKernelGGL((k_gemm<FMT, EPI, 4, KSPLIT, XSRC>), grid, dim3(256), shm, st, a);
    return launch_err();
}

int sw_launch_q4_gateup(hipStream_t st, SwQ4 W, const float *x, SwGroups g, int I, _Float16 *hplanes, int maxtok) {
    if (I % 8 || W.O != 2 * I) return -1;
    const int ng = W.gs > 0 ? W.K / W.gs : 1;
    GemmArgs a = {W.q, W.q + (int64_t)I * (W.K / 2), W.s, W.s + (int64_t)I * ng, 2 * I, W.K, W.gs, g,
                  x, I, hplanes, I / 8, 0, 0};
    return launch_gemm<FMT_Q4, EPI_GLU, 1, XSRC_F32>(st, a, maxtok > 8 ? 4 : 1, maxtok);
}

int sw_launch_q4_rows(hipStream_t st, SwQ4 W, const _Float16 *planes, SwGroups g, float *Y, int maxtok) {
    if (W.O % 16) return -1;
    GemmArgs a = {W.q, W.q, W.s, W.s, W.O, W.K, W.gs, g, planes, 0, Y, W.O / 16, 0, 0};
    return launch_gemm<FMT_Q4, EPI_ROWS, 1, XSRC_PLANES>(st, a, maxtok > 8 ? 4 : 1, maxtok);
}

int sw_launch_q4_rows_x(hipStream_t st, SwQ4 W, const float *x, SwGroups g, float *Y, int maxtok) {
    if (W.O % 16) return -1;
    GemmArgs a = {W.q, W.q, W.s, W.s, W.O, W.K, W.gs, g, x, 0, Y, W.O / 16, 0, 0};
    return launch_gemm<FMT_Q4, EPI_ROWS, 1, XSRC_F32>(st, a, maxtok > 8 ? 4 : 1, maxtok);
}

int sw_launch_q4_down_combine(hipStream_t st, SwQ4 W, const _Float16 *hplanes, const int *sel, const float *w, int K,
                              float route_scale, const float *shared, float *out) {
    if (W.K % 128 || W.O % 16 || K <= 0 || K > DC_MAXK) return -1;
    if (W.gs > 0 && (W.gs % 32 || W.K % W.gs)) return -1;
    const size_t lds = (size_t)2 * K * (W.K + 8) * 2;
    if (lds > 65536) return -1;
    hipLaunchKernelGGL(k_q4_down_combine, dim3((unsigned)(W.O / 16)), dim3(256), lds, st, W, hplanes, sel, w, K,
                       route_scale, shared, out);
    return launch_err();
}

// bf16 GEMMs split K in four quarters when K allows it (K % 512 == 0), so a
// shape always reduces the same way whatever the batch
int sw_launch_bf16_gateup(hipStream_t st, SwBf16 Wg, SwBf16 Wu, const float *x, int S, uint16_t *hplanes) {
    if (Wg.O % 8 || Wu.O != Wg.O || Wu.K != Wg.K || S <= 0) return -1;
    SwGroups g = {nullptr, nullptr, nullptr, nullptr, nullptr, 1, S};
    GemmArgs a = {Wg.w, Wu.w, nullptr, nullptr, Wg.O, Wg.K, 0, g, x, Wg.O, hplanes, Wg.O / 8, 0, 0};
    if (Wg.K % 512 == 0) return launch_gemm<FMT_BF16, EPI_GLU, 4, XSRC_F32>(st, a, 1, S);
    return launch_gemm<FMT_BF16, EPI_GLU, 1, XSRC_F32>(st, a, 1, S);
}

int sw_launch_bf16_rows(hipStream_t st, SwBf16 W, const uint16_t *planes, int S, float *Y) {
    if (W.O % 16 || S <= 0) return -1;
    SwGroups g = {nullptr, nullptr, nullptr, nullptr, nullptr, 1, S};
    GemmArgs a = {W.w, W.w, nullptr, nullptr, W.O, W.K, 0, g, planes, 0, Y, W.O / 16, 0, 0};
    if (W.K % 512 == 0) return launch_gemm<FMT_BF16, EPI_ROWS, 4, XSRC_PLANES>(st, a, 1, S);
    return launch_gemm<FMT_BF16, EPI_ROWS, 1, XSRC_PLANES>(st, a, 1, S);
}

int sw_launch_bf16_rows_x(hipStream_t st, SwBf16 W, const float *x, int S, float *Y) {
    if (W.O % 16 || S <= 0) return -1;
    SwGroups g = {nullptr, nullptr, nullptr, nullptr, nullptr, 1, S};
    GemmArgs a = {W.w, W.w, nullptr, nullptr, W.O, W.K, 0, g, x, 0, Y, W.O / 16, 0, 0};
    if (W.K % 512 == 0) return launch_gemm<FMT_BF16, EPI_ROWS, 4, XSRC_F32>(st, a, 1, S);
    return launch_gemm<FMT_BF16, EPI_ROWS, 1, XSRC_F32>(st, a, 1, S);
}
