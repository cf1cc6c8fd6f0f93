// k_gemm.hip -- grouped int4 and bf16 expert GEMMs on the gfx950 matrix cores.
//
// Work unit: one wave owns one 16-row tile of one group (an expert applied to
// a run of packed rows) and one K-slice of it; a block holds 4/KSPLIT tiles x
// KSPLIT slices, and the slices of a tile are summed in LDS in a fixed order
// ((s0+s1) or (q0+q1)+(q2+q3)).  KSPLIT is a function of the operation and K
// alone (see q4_glu_ksplit / bf16_ksplit), never of the batch, so the
// reduction of every output is fixed and the grouped path is bit-identical to
// the per-token path.  Replaces the reference's warp-per-row mm_q4_kernel /
// mm_q4_group_kernel / grouped_*_g4 kernels (c/backend_cuda_laguna.cu:138-157,
// 420-443; c/backend_cuda.cu:347-380), which re-read a weight row once per
// token: here a weight row is read once per pass and applied to every token
// of the pass as MFMA columns (token t -> columns 2t (hi) and 2t+1 (lo)).
//
// Data movement per wave: weights stream HBM -> VGPRs through a ring of PF
// super-steps in flight (static register slots: the K loop is unrolled by
// PF and every chunk boundary falls on a multiple of PF); a pass's activation
// planes are staged in LDS by the whole block, the whole K-slice at once when
// it fits, else in chunks of a multiple of PF super-steps (next chunk's
// global loads in flight in registers while the current one is consumed),
// so MFMA B fragments come from LDS (one ds_read_b128 each).
//
// int4 dequant (in registers): a 32-bit word holds 8 nibbles of one row;
// OR-ing a nibble into the mantissa of f16 1024.0 gives 1024+n exactly, and
// one packed add (or packed fma for nibbles sitting 4 bits higher) yields
// n-8 exactly.  Group scales (gs > 0) are folded into the f16 weight
// (f16(s*2^8) * (n-8), one rounding); per-row scales (gs == 0) are applied in
// f32 after the K loop, leaving the weights exact.
#include "sw_hip.h"
#include "sw_libm.h"

#define PF_MAX 8          // weight super-steps in flight per wave (a template parameter PF <= PF_MAX
                          // that divides the super-steps of a slice; also the chunk granularity)
#define LDS_MAXH 32768    // staging budget in halves (64 KB)
#define TP_MAX 8          // tokens per pass: 16 MFMA columns
enum { FMT_Q4 = 0, FMT_BF16 = 1 };
enum { EPI_GLU = 0, EPI_ROWS = 1 };
enum { XSRC_PLANES = 0, XSRC_F32 = 1 };

// (a & m) | o in one VALU op (the compiler splits it in two when m and o are
// both literal constants)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

// s2 = (f16(s * 2^8), same) for group scales, (1, 1) for per-row scales (exact)
__device__ __forceinline__ sw_half8 dq8(uint32_t w, sw_half2 s2) {
    const sw_half2 m1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const sw_half2 r16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const sw_half2 m72 = {(_Float16)-72.0f, (_Float16)-72.0f};
    const uint32_t w8 = w >> 8, mg = 0x64006400u;
    sw_half2 h0 = __builtin_bit_cast(sw_half2, and_or(w, 0x000F000Fu, mg)) + m1032;
    sw_half2 h1 = __builtin_elementwise_fma(__builtin_bit_cast(sw_half2, and_or(w, 0x00F000F0u, mg)), r16, m72);
    sw_half2 h2 = __builtin_bit_cast(sw_half2, and_or(w8, 0x000F000Fu, mg)) + m1032;
    sw_half2 h3 = __builtin_elementwise_fma(__builtin_bit_cast(sw_half2, and_or(w8, 0x00F000F0u, mg)), r16, m72);
    h0 = h0 * s2; h1 = h1 * s2; h2 = h2 * s2; h3 = h3 * s2;
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

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// ------------------------------------------------------------ staging ----
// An LDS row holds, for one plane row (hi or lo of a token), the current
// chunk of every K-slice: [slice 0: ckh halves][slice 1] ... + 8 halves of
// padding.  A "line" is one (plane row | token, slice) run of ckh halves,
// moved in 16-byte segments (8 halves, or 8 f32 split into hi/lo on the way).
// Segments go out in batches of SB per thread (segment tid + 256 * (SB*b + i)),
// so only one batch is ever held in registers.
#define SB 4
template <int FMT, int XSRC, int KSPLIT>
struct Stage {
    sw_u32x4 r[XSRC == XSRC_PLANES ? SB : 2 * SB];

    // batch b of the chunk at slice offset k0; a last chunk shorter than ckh
    // loads only Kq - k0
    __device__ __forceinline__ void load(int b, const void *__restrict__ src, int K, int k0, int ckh, int ntok,
                                         const int *rowsrc, int tid) {
        const int Kq = K / KSPLIT, segq = ckh >> 3;
        const int segv = min(ckh, Kq - k0) >> 3;     // segments of a line inside the slice
        const int nlines = (XSRC == XSRC_PLANES ? 2 : 1) * ntok * KSPLIT;
        const int s0 = tid + 256 * SB * b;
        int line = s0 / segq, cs = s0 - line * segq;
#pragma unroll
        for (int i = 0; i < SB; i++) {
            if (line < nlines && cs < segv) {
                const int q = line % KSPLIT, rr = line / KSPLIT;
                if (XSRC == XSRC_PLANES) {
                    const uint16_t *p = (const uint16_t *)src + (int64_t)(2 * rowsrc[rr >> 1] + (rr & 1)) * K + q * Kq + k0 + cs * 8;
                    r[i] = *(const sw_u32x4 *)p;
                } else {
                    const float *p = (const float *)src + (int64_t)rowsrc[rr] * K + q * Kq + k0 + cs * 8;
                    r[2 * i] = *(const sw_u32x4 *)p;
                    r[2 * i + 1] = *(const sw_u32x4 *)(p + 4);
                }
            }
            cs += 256;
            while (cs >= segq) { cs -= segq; line++; }
        }
    }

    __device__ __forceinline__ void store(int b, uint16_t *lds, int ckh, int rowlen, int ntok, int tid) const {
        const int segq = ckh >> 3;
        const int nlines = (XSRC == XSRC_PLANES ? 2 : 1) * ntok * KSPLIT;
        const int s0 = tid + 256 * SB * b;
        int line = s0 / segq, cs = s0 - line * segq;
#pragma unroll
        for (int i = 0; i < SB; i++) {
            if (line < nlines) {
                const int q = line % KSPLIT, rr = line / KSPLIT;
                if (XSRC == XSRC_PLANES) {
                    *(sw_u32x4 *)(lds + rr * rowlen + q * ckh + cs * 8) = r[i];
                } else {
                    const sw_f32x4 v0 = __builtin_bit_cast(sw_f32x4, r[2 * i]), v1 = __builtin_bit_cast(sw_f32x4, r[2 * i + 1]);
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
                    *(sw_u32x4 *)(lds + (2 * rr) * rowlen + q * ckh + cs * 8) = hi;
                    *(sw_u32x4 *)(lds + (2 * rr + 1) * rowlen + q * ckh + cs * 8) = lo;
                }
            }
            cs += 256;
            while (cs >= segq) { cs -= segq; line++; }
        }
    }

    // batches of a chunk
    __device__ __forceinline__ static int nbatch(int ckh, int ntok) {
        const int nseg = (XSRC == XSRC_PLANES ? 2 : 1) * ntok * KSPLIT * (ckh >> 3);
        return (nseg + 256 * SB - 1) / (256 * SB);
    }
};

struct GemmArgs {
    const void *w0, *w1;      // weight bases: rows of expert e at (e*rpe + r); w1 = second tile of the GLU pair
    const float *s0, *s1;     // scale bases (int4), same row indexing
    int rpe, K, gs, gsh;      // rows per expert, inputs, group size (0: per-row), log2(gs)
    SwGroups g;
    const void *xsrc;         // activations: planes [2*rows, K] (XSRC_PLANES) or f32 rows [rows, K] (XSRC_F32)
    int I;                    // GLU: output width (rows of w0 / w1 used: I each)
    void *out;
    int rowtiles;             // 16-row tiles (ROWS) or 8-pair tiles (GLU)
    int tp;                   // tokens per pass
    int ldsh;                 // LDS halves allocated
};

// super-steps per chunk for a pass of ntok tokens: the whole slice when it
// fits, else the largest multiple of PF that does
__device__ __forceinline__ int chunk_ss(int nssq, int ntok, int ksplit, int ldsh, int pf) {
    if (2 * ntok * (ksplit * nssq * 128 + 8) <= ldsh) return nssq;
    const int per = (ldsh / (2 * ntok) - 8) / (ksplit * 128 * pf);
    return per * pf;
}

// CH = 0: every pass stages its whole K-slice at once (the host sizes passes
// so it fits); CH = 1: passes larger than that stage in chunks, the next
// chunk's loads in flight in registers across the K loop.
template <int FMT, int EPI, int KSPLIT, int XSRC, int PF, int CH>
__global__ __launch_bounds__(256, FMT == FMT_Q4 ? 3 : 2) void k_gemm(GemmArgs A) {   // waves per SIMD
    extern __shared__ __align__(16) uint16_t lds[];
    __shared__ int rowsrc[TP_MAX];
    constexpr int TPB = 4 / KSPLIT;                  // row tiles per block
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.x;
    const int gvalid = A.g.G ? *A.g.G : A.g.ngroups_max;
    if (g >= gvalid) return;
    const int rt = (int)blockIdx.y * TPB + wave / KSPLIT;
    const int slice = wave % KSPLIT;
    const bool active = rt < A.rowtiles;
    const int e = A.g.gexp ? A.g.gexp[g] : 0, beg = A.g.gbeg ? A.g.gbeg[g] : 0;
    const int cnt = A.g.gcnt ? A.g.gcnt[g] : A.g.cnt_const;
    const int r = lane & 15, kb = lane >> 4, c = lane & 15;
    const int K = A.K, gs = A.gs;
    const int Kq = K / KSPLIT, nssq = Kq >> 7;
    const int rtc = active ? rt : 0;
    // this lane's weight row
    const int64_t wrow = (EPI == EPI_GLU) ? ((int64_t)e * A.rpe + rtc * 8 + (r & 7)) : ((int64_t)e * A.rpe + rtc * 16 + r);
    const bool second = (EPI == EPI_GLU) && (r >= 8);
    const int ng = gs > 0 ? K / gs : 1;
    const uint8_t *arow8 = nullptr;
    const uint16_t *arow16 = nullptr;
    const float *srow = nullptr;
    if (FMT == FMT_Q4) {
        arow8 = (const uint8_t *)(second ? A.w1 : A.w0) + wrow * (K / 2) + slice * (Kq / 2) + kb * 16;
        srow = (second ? A.s1 : A.s0) + wrow * ng;
    } else {
        arow16 = (const uint16_t *)(second ? A.w1 : A.w0) + wrow * K + slice * Kq + kb * 32;
    }
    const bool scaled = (FMT == FMT_Q4) && gs > 0;
    const int sk0 = slice * Kq + kb * 32;            // k of this lane's first nibble at super-step 0
    const int gsh = gs > 0 ? A.gsh : 31;             // per-row scales: index 0 of the row, every step

    for (int t0 = 0; t0 < cnt; t0 += A.tp) {
        const int ntok = min(A.tp, cnt - t0);
        const int cks = CH ? chunk_ss(nssq, ntok, KSPLIT, A.ldsh, PF) : nssq;
        const int ckh = cks * 128, rowlen = KSPLIT * ckh + 8;
        __syncthreads();
        if (tid < ntok) rowsrc[tid] = A.g.grow ? A.g.grow[beg + t0 + tid] : beg + t0 + tid;
        __syncthreads();
        Stage<FMT, XSRC, KSPLIT> stg;
        const int nb = Stage<FMT, XSRC, KSPLIT>::nbatch(ckh, ntok);
        stg.load(0, A.xsrc, K, 0, ckh, ntok, rowsrc, tid);

        // weight ring: super-step ss lives in slot ss % PF (PF divides nssq).
        // Every round but the last refills each slot right after consuming it;
        // the last round is peeled and refills nothing, so the ring stays in
        // fixed registers, every load stays in flight and none is wasted.
        sw_u32x4 ra[PF][FMT == FMT_BF16 ? 4 : 1];
        float sa[PF];
#pragma unroll
        for (int u = 0; u < PF; u++) {
            if (FMT == FMT_Q4) {
                ra[u][0] = *(const sw_u32x4 *)(arow8 + u * 64);
                sa[u] = srow[(sk0 + u * 128) >> gsh];
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) ra[u][FMT == FMT_BF16 ? q : 0] = *(const sw_u32x4 *)(arow16 + u * 128 + q * 8);
            }
        }
        stg.store(0, lds, ckh, rowlen, ntok, tid);
        for (int b = 1; b < nb; b++) {
            stg.load(b, A.xsrc, K, 0, ckh, ntok, rowsrc, tid);
            stg.store(b, lds, ckh, rowlen, ntok, tid);
        }
        __syncthreads();
        if (CH && cks < nssq) stg.load(0, A.xsrc, K, ckh, ckh, ntok, rowsrc, tid);

        sw_f32x4 accq[4];                                // one chain per MFMA position q
#pragma unroll
        for (int q = 0; q < 4; q++) accq[q] = (sw_f32x4){0.f, 0.f, 0.f, 0.f};
        // columns past the pass read token 0's rows (their outputs are dropped)
        const int crow = ((c >> 1) < ntok) ? c : (c & 1);
        const uint16_t *bl = lds + crow * rowlen + slice * ckh + kb * 32;
        int cbeg = 0, cnext = cks;
        auto boundary = [&](int ss0) {
            if (CH && ss0 == cnext) {                    // chunk boundary (uniform in the block)
                __syncthreads();
                stg.store(0, lds, ckh, rowlen, ntok, tid);
                for (int b = 1; b < nb; b++) {
                    stg.load(b, A.xsrc, K, ss0 * 128, ckh, ntok, rowsrc, tid);
                    stg.store(b, lds, ckh, rowlen, ntok, tid);
                }
                __syncthreads();
                cbeg = ss0;
                cnext = ss0 + cks;
                if (cnext < nssq) stg.load(0, A.xsrc, K, cnext * 128, ckh, ntok, rowsrc, tid);
            }
        };
        auto round = [&](int ss0, bool refill) {
            const uint16_t *bss = bl + (ss0 - cbeg) * 128;
#pragma unroll
            for (int u = 0; u < PF; u++) {
                const int nx = ss0 + u + PF;
                sw_half8 a16[4];
                sw_u32x4 abf[4];
                if (FMT == FMT_Q4) {
                    const float cs = scaled ? sa[u] : (1.0f / SW_WPRESCALE);
                    const _Float16 s16 = (_Float16)(cs * SW_WPRESCALE);
                    const sw_half2 s2 = {s16, s16};
                    const sw_u32x4 cur = ra[u][0];
                    a16[0] = dq8(cur.x, s2);
                    a16[1] = dq8(cur.y, s2);
                    a16[2] = dq8(cur.z, s2);
                    a16[3] = dq8(cur.w, s2);
                    if (refill) {
                        ra[u][0] = *(const sw_u32x4 *)(arow8 + nx * 64);
                        sa[u] = srow[(sk0 + nx * 128) >> gsh];
                        __builtin_amdgcn_sched_barrier(0);  // keep the refill at its step
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) abf[q] = ra[u][FMT == FMT_BF16 ? q : 0];
                    if (refill) {
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            ra[u][FMT == FMT_BF16 ? q : 0] = *(const sw_u32x4 *)(arow16 + nx * 128 + q * 8);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const sw_u32x4 b = *(const sw_u32x4 *)(bss + u * 128 + q * 8);
                    if (FMT == FMT_Q4)
                        accq[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a16[q], __builtin_bit_cast(sw_half8, b), accq[q], 0, 0, 0);
                    else
                        accq[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sw_bf16x8, abf[q]),
                                                                          __builtin_bit_cast(sw_bf16x8, b), accq[q], 0, 0, 0);
                }
            }
        };
        int ss0 = 0;
        for (; ss0 + PF < nssq; ss0 += PF) {
            boundary(ss0);
            round(ss0, true);
        }
        boundary(ss0);
        round(ss0, false);
        sw_f32x4 acc = (accq[0] + accq[1]) + (accq[2] + accq[3]);
        __syncthreads();

        // K-split reduction: slices through LDS, (s0+s1) or (q0+q1)+(q2+q3)
        if (KSPLIT > 1) {
            float *red = (float *)lds;                   // 4 waves x 64 lanes x 4
#pragma unroll
            for (int j = 0; j < 4; j++) red[(wave * 64 + lane) * 4 + j] = acc[j];
            __syncthreads();
            if (slice == 0) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float p0 = red[((wave + 0) * 64 + lane) * 4 + j], p1 = red[((wave + 1) * 64 + lane) * 4 + j];
                    if (KSPLIT == 2) {
                        acc[j] = p0 + p1;
                    } else {
                        const float p2 = red[((wave + 2) * 64 + lane) * 4 + j], p3 = red[((wave + 3) * 64 + lane) * 4 + j];
                        acc[j] = (p0 + p1) + (p2 + p3);
                    }
                }
            }
            __syncthreads();
        }
        const bool writer = active && slice == 0;
        // epilogue: hi + lo, scale, then GLU or store
        const int rbase = 4 * (lane >> 4);
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float mine = acc[j];
            v[j] = mine + __shfl_xor(mine, 1);            // even lanes: hi + lo
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
        const int t = t0 + (c >> 1);
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

// ------------------------------------------------- down + combine (one token) ----
// For a single token: out[d] += (sum_a w[a] * y_a[d]) * route_scale (+ shared[d]),
// y_a = down_{sel[a]}(h_a), for one 16-row d tile per block.  Wave w runs the
// ranks a = w, w + nw, ... with the same per-output MFMA chain as the grouped
// kernel (KSPLIT 1: so y_a is bit-identical to its slot value there), its
// rank's two planes staged in a wave-private LDS region, parks y_a in LDS,
// and one wave sums the ranks in order with one fma per rank, the operation
// sequence of k_combine.
#define DC_MAXK 64
#define DC_MAXW 12         // waves per block (one rank each); 3 waves per SIMD leave 168 VGPRs
template <int PF>
__global__ __launch_bounds__(DC_MAXW * 64) void k_q4_down_combine(SwQ4 W, int gsh, const _Float16 *__restrict__ hp,
                                                                  const int *__restrict__ sel, const float *__restrict__ wts,
                                                                  int K, float route_scale, const float *__restrict__ shared,
                                                                  float *__restrict__ out) {
    extern __shared__ __align__(16) uint16_t lds[];   // per wave: 2 rows x (I + 8) halves
    __shared__ float ys[DC_MAXK][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int I = W.K, D = W.O, gs = W.gs;
    const int dt = blockIdx.x;
    const int rowlen = I + 8;
    uint16_t *my = lds + wave * 2 * rowlen;
    const int r = lane & 15, kb = lane >> 4, c = lane & 15;
    const int ng = gs > 0 ? I / gs : 1;
    const bool scaled = gs > 0;
    if (!scaled) gsh = 31;                           // per-row scales: index 0 of the row, every step
    const int nss = I >> 7;
    const int nseg = I / 4, segrow = I / 8;           // 16-byte segments of the two planes
    // the combine's operands, fetched before anything waits
    __shared__ float wk[DC_MAXK];
    if (tid < K) wk[tid] = wts[tid];
    float sh_d = 0.f, out_d = 0.f;
    if (tid < 16) {
        out_d = out[dt * 16 + tid];
        if (shared) sh_d = shared[dt * 16 + tid];
    }
    for (int a = wave; a < K; a += nw) {
        // this rank's planes (rows 2a hi, 2a+1 lo) do not depend on the routing:
        // their loads go out first, then the expert id, then its weights
        const uint16_t *src = (const uint16_t *)hp + (int64_t)(2 * a) * I;
        sw_u32x4 hv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int seg = min(lane + 64 * i, nseg - 1);
            const int row = seg >= segrow, k = (seg - row * segrow) * 8;
            hv[i] = *(const sw_u32x4 *)(src + (int64_t)row * I + k);
        }
        const int e = sel[a];
        const uint8_t *arow = W.q + ((int64_t)e * D + dt * 16 + r) * (I / 2) + kb * 16;
        const float *srow = W.s + ((int64_t)e * D + dt * 16 + r) * ng;
        sw_u32x4 ra[PF];
        float sa[PF];
#pragma unroll
        for (int u = 0; u < PF; u++) {
            ra[u] = *(const sw_u32x4 *)(arow + u * 64);
            sa[u] = srow[(kb * 32 + u * 128) >> gsh];
        }
        for (int s0 = 0; s0 < nseg; s0 += 4 * 64) {
            if (s0 > 0) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int seg = min(s0 + lane + 64 * i, nseg - 1);
                    const int row = seg >= segrow, k = (seg - row * segrow) * 8;
                    hv[i] = *(const sw_u32x4 *)(src + (int64_t)row * I + k);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int seg = s0 + lane + 64 * i;
                const int row = seg >= segrow, k = (seg - row * segrow) * 8;
                if (seg < nseg) *(sw_u32x4 *)(my + row * rowlen + k) = hv[i];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        sw_f32x4 accq[4];                                // one chain per MFMA position q
#pragma unroll
        for (int q = 0; q < 4; q++) accq[q] = (sw_f32x4){0.f, 0.f, 0.f, 0.f};
        const uint16_t *bl = my + (c & 1) * rowlen + kb * 32;   // columns 2.. duplicate the token (dropped)
        auto round = [&](int ss0, bool refill) {
#pragma unroll
            for (int u = 0; u < PF; u++) {
                const int ss = ss0 + u, nx = ss + PF;
                const float cs = scaled ? sa[u] : (1.0f / SW_WPRESCALE);
                const _Float16 s16 = (_Float16)(cs * SW_WPRESCALE);
                const sw_half2 s2 = {s16, s16};
                const sw_u32x4 cur = ra[u];
                sw_half8 a16[4];
                a16[0] = dq8(cur.x, s2);
                a16[1] = dq8(cur.y, s2);
                a16[2] = dq8(cur.z, s2);
                a16[3] = dq8(cur.w, s2);
                if (refill) {
                    ra[u] = *(const sw_u32x4 *)(arow + nx * 64);
                    sa[u] = srow[(kb * 32 + nx * 128) >> gsh];
                    __builtin_amdgcn_sched_barrier(0);      // keep the refill at its step
                }
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const sw_u32x4 b = *(const sw_u32x4 *)(bl + ss * 128 + q * 8);
                    accq[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a16[q], __builtin_bit_cast(sw_half8, b), accq[q], 0, 0, 0);
                }
            }
        };
        int ss0 = 0;
        for (; ss0 + PF < nss; ss0 += PF) round(ss0, true);
        round(ss0, false);
        const sw_f32x4 acc = (accq[0] + accq[1]) + (accq[2] + accq[3]);
        // rank finished: hi + lo, scale, park in LDS
        const int rbase = 4 * (lane >> 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float mine = acc[j];
            float v = mine + __shfl_xor(mine, 1);
            if (scaled) v = v * SW_WPRESCALE_INV;
            else v = v * W.s[(int64_t)e * D + dt * 16 + rbase + j];
            if (c == 0) ys[a][rbase + j] = v;
        }
        // the next rank of this wave overwrites the planes: every lane's reads are done
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    if (tid < 16) {
        float s = 0.f;
        for (int a = 0; a < K; a++) s = __builtin_fmaf(wk[a], ys[a][tid], s);
        s = s * route_scale;
        if (shared) s = s + sh_d;
        out[dt * 16 + tid] = out_d + s;
    }
}

// ---------------------------------------------------------------- launch ----
static int launch_err(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

static int log2_pow2(int v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int s = 0;
    while ((1 << s) < v) s++;
    return s;
}

// K-split rules: a function of the operation and K only (see the header)
static int q4_glu_ksplit(int K) { return (K >= 2048 && K % 256 == 0) ? 2 : 1; }
static int bf16_ksplit(int K) { return K % 512 == 0 ? 4 : 1; }

// ring depth: the largest power of two up to pfmax that divides the super-steps of a slice
static int pick_pf(int nssq, int pfmax = PF_MAX) {
    for (int pf = pfmax; pf > 1; pf >>= 1)
        if (nssq % pf == 0) return pf;
    return 1;
}

// maxtok: an upper bound of the tokens of any group (sizes the LDS staging)
template <int FMT, int EPI, int KSPLIT, int XSRC, int CH>
static void launch_pf(int pf, dim3 grid, size_t shm, hipStream_t st, const GemmArgs &a) {
    switch (pf) {
    case 8: SW_LAUNCH((k_gemm<FMT, EPI, KSPLIT, XSRC, FMT == FMT_BF16 ? 4 : 8, CH>), grid, dim3(256), shm, st, a); break;
    case 4: SW_LAUNCH((k_gemm<FMT, EPI, KSPLIT, XSRC, 4, CH>), grid, dim3(256), shm, st, a); break;
    case 2: SW_LAUNCH((k_gemm<FMT, EPI, KSPLIT, XSRC, 2, CH>), grid, dim3(256), shm, st, a); break;
    default: SW_LAUNCH((k_gemm<FMT, EPI, KSPLIT, XSRC, 1, CH>), grid, dim3(256), shm, st, a); break;
    }
}

// maxtok: an upper bound of the tokens of any group (sizes the LDS staging)
template <int FMT, int EPI, int KSPLIT, int XSRC>
static int launch_gemm(hipStream_t st, GemmArgs a, int maxtok) {
    const int Kq = a.K / KSPLIT;
    if (a.K % (128 * KSPLIT) || a.g.ngroups_max <= 0 || a.rowtiles <= 0 || maxtok <= 0) return -1;
    if (FMT == FMT_Q4 && a.gs > 0) {
        if (a.gs % 32 || a.K % a.gs) return -1;
        a.gsh = log2_pow2(a.gs);
        if (a.gsh < 0) return -1;                    // group sizes are powers of two
    }
    const int nssq = Kq / 128;
    // bf16 moves 64 bytes per lane per super-step: a ring of 4 keeps as much in flight
    const int pf = pick_pf(nssq, FMT == FMT_BF16 ? 4 : PF_MAX);
    const int whole1 = 2 * (KSPLIT * Kq + 8);        // halves to stage a full slice for one token
    const int tpw = LDS_MAXH / whole1;               // tokens per pass without chunking
    int ch = 0, tp;
    if (tpw >= (maxtok < TP_MAX ? maxtok : TP_MAX)) {
        tp = maxtok < TP_MAX ? maxtok : TP_MAX;
    } else {
        const int ck0 = nssq < pf ? nssq : pf;       // smallest chunk a pass may use
        tp = LDS_MAXH / (2 * (KSPLIT * ck0 * 128 + 8));
        if (tp > TP_MAX) tp = TP_MAX;
        if (tp > maxtok) tp = maxtok;
        ch = tp > tpw;
        if (!ch) tp = tpw;
    }
    if (tp < 1) return -1;
    a.tp = tp;
    const int whole = tp * whole1;
    int ldsh = whole < LDS_MAXH ? whole : LDS_MAXH;
    if (ldsh < 4 * 64 * 4 * 2) ldsh = 4 * 64 * 4 * 2; // room for the K-split reduction (f32)
    a.ldsh = ldsh;
    dim3 grid((unsigned)a.g.ngroups_max, (unsigned)((a.rowtiles + 4 / KSPLIT - 1) / (4 / KSPLIT)));
    const size_t shm = (size_t)ldsh * 2;
    if (ch) launch_pf<FMT, EPI, KSPLIT, XSRC, 1>(pf, grid, shm, st, a);
    else launch_pf<FMT, EPI, KSPLIT, XSRC, 0>(pf, grid, shm, st, a);
    return launch_err();
}

int sw_launch_q4_gateup(hipStream_t st, SwQ4 W, const float *x, SwGroups g, int I, _Float16 *hplanes, int maxtok) {
    if (I % 8 || W.O != 2 * I) return -1;
    const int ng = W.gs > 0 ? W.K / W.gs : 1;
    GemmArgs a = {W.q, W.q + (int64_t)I * (W.K / 2), W.s, W.s + (int64_t)I * ng, 2 * I, W.K, W.gs, 0, g,
                  x, I, hplanes, I / 8, 0, 0};
    if (q4_glu_ksplit(W.K) == 2) return launch_gemm<FMT_Q4, EPI_GLU, 2, XSRC_F32>(st, a, maxtok);
    return launch_gemm<FMT_Q4, EPI_GLU, 1, XSRC_F32>(st, a, maxtok);
}

int sw_launch_q4_rows(hipStream_t st, SwQ4 W, const _Float16 *planes, SwGroups g, float *Y, int maxtok) {
    if (W.O % 16) return -1;
    GemmArgs a = {W.q, W.q, W.s, W.s, W.O, W.K, W.gs, 0, g, planes, 0, Y, W.O / 16, 0, 0};
    return launch_gemm<FMT_Q4, EPI_ROWS, 1, XSRC_PLANES>(st, a, maxtok);
}

int sw_launch_q4_rows_x(hipStream_t st, SwQ4 W, const float *x, SwGroups g, float *Y, int maxtok) {
    if (W.O % 16) return -1;
    GemmArgs a = {W.q, W.q, W.s, W.s, W.O, W.K, W.gs, 0, g, x, 0, Y, W.O / 16, 0, 0};
    return launch_gemm<FMT_Q4, EPI_ROWS, 1, XSRC_F32>(st, a, maxtok);
}

int sw_launch_q4_down_combine(hipStream_t st, SwQ4 W, const _Float16 *hplanes, const int *sel, const float *w, int K,
                              float route_scale, const float *shared, float *out) {
    if (W.K % 128 || W.O % 16 || K <= 0 || K > DC_MAXK) return -1;
    int gsh = 0;
    if (W.gs > 0) {
        if (W.gs % 32 || W.K % W.gs) return -1;
        gsh = log2_pow2(W.gs);
        if (gsh < 0) return -1;
    }
    const int nw = K < DC_MAXW ? K : DC_MAXW;
    const size_t lds = (size_t)nw * 2 * (W.K + 8) * 2;
    if (lds > 65536) return -1;
    const dim3 grid((unsigned)(W.O / 16)), block(nw * 64);
    switch (pick_pf(W.K / 128)) {
    case 8: SW_LAUNCH(k_q4_down_combine<8>, grid, block, lds, st, W, gsh, hplanes, sel, w, K, route_scale, shared, out); break;
    case 4: SW_LAUNCH(k_q4_down_combine<4>, grid, block, lds, st, W, gsh, hplanes, sel, w, K, route_scale, shared, out); break;
    case 2: SW_LAUNCH(k_q4_down_combine<2>, grid, block, lds, st, W, gsh, hplanes, sel, w, K, route_scale, shared, out); break;
    default: SW_LAUNCH(k_q4_down_combine<1>, grid, block, lds, st, W, gsh, hplanes, sel, w, K, route_scale, shared, out); break;
    }
    return launch_err();
}

// bf16 GEMMs split K in four quarters when K allows it (K % 512 == 0), so a
// shape always reduces the same way whatever the batch
int sw_launch_bf16_gateup(hipStream_t st, SwBf16 Wg, SwBf16 Wu, const float *x, int S, uint16_t *hplanes) {
    if (Wg.O % 8 || Wu.O != Wg.O || Wu.K != Wg.K || S <= 0) return -1;
    SwGroups g = {nullptr, nullptr, nullptr, nullptr, nullptr, 1, S};
    GemmArgs a = {Wg.w, Wu.w, nullptr, nullptr, Wg.O, Wg.K, 0, 0, g, x, Wg.O, hplanes, Wg.O / 8, 0, 0};
    if (bf16_ksplit(Wg.K) == 4) return launch_gemm<FMT_BF16, EPI_GLU, 4, XSRC_F32>(st, a, S);
    return launch_gemm<FMT_BF16, EPI_GLU, 1, XSRC_F32>(st, a, S);
}

int sw_launch_bf16_rows(hipStream_t st, SwBf16 W, const uint16_t *planes, int S, float *Y) {
    if (W.O % 16 || S <= 0) return -1;
    SwGroups g = {nullptr, nullptr, nullptr, nullptr, nullptr, 1, S};
    GemmArgs a = {W.w, W.w, nullptr, nullptr, W.O, W.K, 0, 0, g, planes, 0, Y, W.O / 16, 0, 0};
    if (bf16_ksplit(W.K) == 4) return launch_gemm<FMT_BF16, EPI_ROWS, 4, XSRC_PLANES>(st, a, S);
    return launch_gemm<FMT_BF16, EPI_ROWS, 1, XSRC_PLANES>(st, a, S);
}

int sw_launch_bf16_rows_x(hipStream_t st, SwBf16 W, const float *x, int S, float *Y) {
    if (W.O % 16 || S <= 0) return -1;
    SwGroups g = {nullptr, nullptr, nullptr, nullptr, nullptr, 1, S};
    GemmArgs a = {W.w, W.w, nullptr, nullptr, W.O, W.K, 0, 0, g, x, 0, Y, W.O / 16, 0, 0};
    if (bf16_ksplit(W.K) == 4) return launch_gemm<FMT_BF16, EPI_ROWS, 4, XSRC_F32>(st, a, S);
    return launch_gemm<FMT_BF16, EPI_ROWS, 1, XSRC_F32>(st, a, S);
}
