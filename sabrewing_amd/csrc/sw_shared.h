// sw_shared.h -- the shared expert (bf16 weights, f32 activations) on the bf16
// MFMA: single-token block jobs of the decode stage kernels, and the pieces of
// the batch kernels (k_shared.hip).
//
// Each f32 input is split exactly into three bf16 parts, x = x0 + x1 + x2:
// x0 is x cut to its top 8 significant bits, x1 the next 8 bits of the
// remainder, x2 what is left (at most 8 significant bits, so exact in bf16
// for every normal remainder).  A product of a bf16 weight and a part is
// exact in f32.  Per output row and token, the K = 32 G inputs are walked in
// NSEG contiguous segments (NSEG: the largest power of two <= 8 dividing G);
// a segment is one chain of v_mfma_f32_16x16x32_bf16 from zero over its
// 32-input steps in order, each step three MFMAs against the parts 0, 1, 2;
// the row is the segments folded left to right, from -0.0 (which leaves the first
// segment's bits as they are).  A row's result depends only
// on its weights and its token's inputs (an MFMA output element is the dot of
// its own row and column), so the single-token blocks and the batch kernels
// give a token the same bits whatever batch it came in.
//
// A token's parts are stored per group of 32 inputs as [3][32] bf16 (192
// bytes): part p of input 32 g + k at element (3 g + p) * 32 + k.
#ifndef SW_SHARED_H
#define SW_SHARED_H
#include "sw_hip.h"

#define SH_RG 32               // inputs per MFMA step
#define SH_NT 512              // threads of the decode stage blocks (8 waves: one per segment)
#define SH_GLU_O 8             // outputs i per decode gate_up block: one 16-row tile, 8 gate + 8 up rows
#define SH_DN_O 32             // rows per decode down block: two 16-row tiles
#define SH_PF 8                // steps of weight loads in flight per wave

// K inputs in G = K/32 groups
__host__ __device__ inline bool sh_shape_ok(int K) { return K > 0 && K % SH_RG == 0; }
__host__ __device__ inline int sh_nseg(int G) {
    int n = 8;
    while (n > 1 && G % n) n >>= 1;
    return n;
}

// the bf16 bit patterns of the three parts of x (a NaN or an infinity is all in
// part 0, NaN kept NaN)
__device__ __forceinline__ void sh_split3(float x, uint32_t &a, uint32_t &b, uint32_t &c) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7F800000u) == 0x7F800000u) {
        a = (u >> 16) | ((u & 0x007FFFFFu) ? 0x40u : 0u);
        b = c = 0u;
        return;
    }
    const float r = x - __builtin_bit_cast(float, u & 0xFFFF0000u);      // exact
    const uint32_t ur = __builtin_bit_cast(uint32_t, r);
    const float t = r - __builtin_bit_cast(float, ur & 0xFFFF0000u);     // exact, <= 8 significant bits
    a = u >> 16;
    b = ur >> 16;
    c = __builtin_bit_cast(uint32_t, t) >> 16;
}
// the parts of 8 consecutive inputs as three 16-byte words (bf16 pairs, the even input low)
__device__ __forceinline__ void sh_split8(sw_f32x4 v0, sw_f32x4 v1, sw_u32x4 &p0, sw_u32x4 &p1, sw_u32x4 &p2) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float e = q < 2 ? v0[2 * q] : v1[2 * q - 4], o = q < 2 ? v0[2 * q + 1] : v1[2 * q - 3];
        uint32_t ea, eb, ec, oa, ob, oc;
        sh_split3(e, ea, eb, ec);
        sh_split3(o, oa, ob, oc);
        p0[q] = ea | (oa << 16);
        p1[q] = eb | (ob << 16);
        p2[q] = ec | (oc << 16);
    }
}
// one 32-input step: the weight word a against the parts b0, b1, b2 of the same inputs
__device__ __forceinline__ sw_f32x4 sh_mfma3(sw_u32x4 a, sw_u32x4 b0, sw_u32x4 b1, sw_u32x4 b2, sw_f32x4 acc) {
    const sw_bf16x8 A = __builtin_bit_cast(sw_bf16x8, a);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(sw_bf16x8, b0), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(sw_bf16x8, b1), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(sw_bf16x8, b2), acc, 0, 0, 0);
    return acc;
}

// ---- one token (the decode stages) ----
// LDS of a job: the token's parts (6 K bytes), then the segment results [8][32] f32
__host__ __device__ inline size_t sh_job_lds(int K) { return (size_t)K * 6 + 8 * 32 * 4; }
__host__ __device__ inline size_t sh_glu_lds(int D) { return sh_job_lds(D); }
__host__ __device__ inline size_t sh_down_lds(int Is) { return sh_job_lds(Is); }
__host__ __device__ inline int sh_down_blocks(int D) { return D / SH_DN_O; }

// The block's parts of one token's K inputs into LDS, in two halves, so a block can
// issue the loads of its first chunk of x before its weight loads (a wave's loads
// return in order: the x it waits on then does not queue behind the weights):
// sh_parts_first loads this thread's first chunk (8 inputs), sh_stage_parts stores it
// as parts and does the rest of x.
struct ShX { sw_f32x4 v0, v1; };
__device__ __forceinline__ ShX sh_parts_ld(const float *__restrict__ x, int c) {
    return ShX{((const sw_f32x4 *)x)[2 * c], ((const sw_f32x4 *)x)[2 * c + 1]};
}
__device__ __forceinline__ void sh_parts_st(const ShX &v, int c, uint16_t *pl) {
    sw_u32x4 p0, p1, p2;
    sh_split8(v.v0, v.v1, p0, p1, p2);
    uint16_t *dst = pl + (c >> 2) * 3 * SH_RG + (c & 3) * 8;
    *(sw_u32x4 *)dst = p0;
    *(sw_u32x4 *)(dst + SH_RG) = p1;
    *(sw_u32x4 *)(dst + 2 * SH_RG) = p2;
}
__device__ __forceinline__ ShX sh_parts_first(const float *__restrict__ x, int K) {
    return sh_parts_ld(x, min((int)threadIdx.x, K / 8 - 1));   // (clamped: no branch around the load)
}
__device__ __forceinline__ void sh_stage_parts(const float *__restrict__ x, int K, uint16_t *pl, const ShX &first) {
    if ((int)threadIdx.x < K / 8) sh_parts_st(first, threadIdx.x, pl);
    for (int c = threadIdx.x + blockDim.x; c < K / 8; c += blockDim.x) sh_parts_st(sh_parts_ld(x, c), c, pl);
}
__device__ __forceinline__ void sh_stage_parts(const float *__restrict__ x, int K, uint16_t *pl) {
    sh_stage_parts(x, K, pl, sh_parts_first(x, K));
}

// wave `seg` of the block: NRT 16-row tiles (row m of tile t at rowp(t, m)) over segment
// seg of the staged token; lane l keeps rows 4 (l / 16) .. +3 of column l % 16 (only
// column 0 holds the token; the other columns multiply zeros).  start() issues the
// first SH_PF steps' weight loads (before the block stages the token's parts, so the
// loads' latency overlaps that work); run() waits for the parts in LDS.
template <int NRT, int PFW = SH_PF>
struct ShSegWave {
    const uint16_t *wr[NRT];
    int GS, g0;
    sw_u32x4 ring[NRT][PFW];
    __device__ __forceinline__ sw_u32x4 ld(int t, int s) const {
        return *(const sw_u32x4 *)(wr[t] + (int64_t)(g0 + min(s, GS - 1)) * SH_RG);
    }
    template <class RowPtr>
    __device__ __forceinline__ void start(RowPtr rowp, int K, int seg, int nseg) {
        const int lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4;
        GS = K / SH_RG / nseg;
        g0 = seg * GS;
#pragma unroll
        for (int t = 0; t < NRT; t++) wr[t] = rowp(t, m) + 8 * kq;
        // unconditional (ld clamps a step past the segment to its last): loads under a
        // condition end at a join where the compiler waits for every load in flight,
        // and the caller's first loads (x) must not wait for the ring
#pragma unroll
        for (int u = 0; u < PFW; u++)
#pragma unroll
            for (int t = 0; t < NRT; t++) ring[t][u] = ld(t, u);
    }
    __device__ __forceinline__ void run(const uint16_t *pl, sw_f32x4 *acc) {
        const int lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4;
#pragma unroll
        for (int t = 0; t < NRT; t++) acc[t] = sw_f32x4{0.f, 0.f, 0.f, 0.f};
        const sw_u32x4 z = {0u, 0u, 0u, 0u};
        const bool col0 = m == 0;
        auto use = [&](int s, int u) {
            const uint16_t *pp = pl + (g0 + s) * 3 * SH_RG + 8 * kq;
            const sw_u32x4 b0 = *(const sw_u32x4 *)pp, b1 = *(const sw_u32x4 *)(pp + SH_RG),
                           b2 = *(const sw_u32x4 *)(pp + 2 * SH_RG);
#pragma unroll
            for (int t = 0; t < NRT; t++) acc[t] = sh_mfma3(ring[t][u], col0 ? b0 : z, col0 ? b1 : z, col0 ? b2 : z, acc[t]);
        };
        // full rounds with unconditional refills (clamped past the end), then the last
        // round without: no branch join inside a round, so the waits stay per step
        int s0 = 0;
        for (; s0 + PFW < GS; s0 += PFW) {
#pragma unroll
            for (int u = 0; u < PFW; u++) {
                use(s0 + u, u);
#pragma unroll
                for (int t = 0; t < NRT; t++) ring[t][u] = ld(t, s0 + u + PFW);
            }
        }
#pragma unroll
        for (int u = 0; u < PFW; u++)
            if (s0 + u < GS) use(s0 + u, u);               // uniform
    }
};

// the segment results of column 0 (rows 16 t + r) into red[seg][32], by the lanes holding them
template <int NRT>
__device__ __forceinline__ void sh_seg_store(const sw_f32x4 *acc, int seg, float *red) {
    const int lane = threadIdx.x & 63;
    if ((lane & 15) == 0) {
#pragma unroll
        for (int t = 0; t < NRT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[seg * 32 + 16 * t + 4 * (lane >> 4) + r] = acc[t][r];
    }
}
// the segments folded left to right from -0.0 (the identity of f32 addition, so the
// first segment is added like the others)
__device__ __forceinline__ float sh_fold(const float *red, int row, int nseg) {
    float y = -0.0f;
    for (int s = 0; s < nseg; s++) y = y + red[s * 32 + row];
    return y;
}

// gate_up of one token for outputs i0 = 8 bid .. +7: tile rows 0-7 the gate rows, 8-15 the
// up rows; h[i] = silu(gate) * up (f32)
__host__ __device__ inline int sh_glu_blocks(int Is) { return Is / SH_GLU_O; }
__device__ __forceinline__ void sh_glu_block(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu,
                                             const float *__restrict__ x, int D, int Is, float *__restrict__ h, int bid,
                                             float *smem) {
    uint16_t *pl = (uint16_t *)smem;
    float *red = smem + (size_t)D * 6 / 4;
    const int i0 = bid * SH_GLU_O, nseg = sh_nseg(D / SH_RG), wave = threadIdx.x >> 6;
    const ShX x0 = sh_parts_first(x, D);              // x ahead of the weights in every wave's queue
    ShSegWave<1> sw;
    if (wave < nseg)
        sw.start([&](int, int m) { return (m < 8 ? Wg + (int64_t)(i0 + m) * D : Wu + (int64_t)(i0 + m - 8) * D); }, D,
                 wave, nseg);
    sh_stage_parts(x, D, pl, x0);
    __syncthreads();
    if (wave < nseg) {
        sw_f32x4 acc[1];
        sw.run(pl, acc);
        sh_seg_store<1>(acc, wave, red);
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < SH_GLU_O) {
        const float yg = sh_fold(red, tid, nseg), yu = sh_fold(red, 8 + tid, nseg);
        h[i0 + tid] = (yg / (1.0f + expf(-yg))) * yu;
    }
}

// down of one token for rows d0 = 32 bid .. +31 (f32 out; PFW: steps of weight loads in
// flight per wave)
template <int PFW = SH_PF>
__device__ __forceinline__ void sh_down_block(const uint16_t *__restrict__ Wd, const float *__restrict__ h, int Is, int D,
                                              float *__restrict__ out, int bid, float *smem) {
    uint16_t *pl = (uint16_t *)smem;
    float *red = smem + (size_t)Is * 6 / 4;
    const int d0 = bid * SH_DN_O, nseg = sh_nseg(Is / SH_RG), wave = threadIdx.x >> 6;
    const ShX h0 = sh_parts_first(h, Is);             // h ahead of the weights in every wave's queue
    ShSegWave<2, PFW> sw;
    if (wave < nseg) sw.start([&](int t, int m) { return Wd + (int64_t)(d0 + 16 * t + m) * Is; }, Is, wave, nseg);
    sh_stage_parts(h, Is, pl, h0);
    __syncthreads();
    if (wave < nseg) {
        sw_f32x4 acc[2];
        sw.run(pl, acc);
        sh_seg_store<2>(acc, wave, red);
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < SH_DN_O) out[d0 + tid] = sh_fold(red, tid, nseg);
}

// ---- decode-sized batches: K split over the waves ----
// Block (bx, by) = (16-row tile, NC column tiles of 16 tokens), 8 waves: wave w runs
// segment w of the K inputs (the MFMA chain of that segment, as ShSegWave), the
// segment results go to LDS (red: [8][16][16 NC] floats) and are folded left to right
// there, so a token gets the bits of the single-token jobs while 8 waves stream one
// tile's weights.  Gate_up tiles: rows 0-7 the gate rows of outputs 8 bx .. +7,
// rows 8-15 the up rows.  The inputs come as parts (xp) or, FX, as f32 rows (xf)
// split into their parts at each step.  Run by k_sh_sk (k_shared.hip) and as extra
// blocks of the decode stage launches (k_dot8.hip).
struct ShSkArgs {
    const uint16_t *W0, *W1;   // gate and up rows (GLU), or the down rows
    const uint16_t *xp;        // the inputs' parts [S][K/32][3][32]
    const float *xf;           // FX: the inputs [S][K] f32
    int S, K, O;
    void *out;                 // GLU: h's parts [S][O/32][3][32]; else [S][O] f32
};
#define SH_SK_NT 512
#define SH_SK_MAX_S 128        // batches up to this many tokens take these blocks
// column tiles of 16 tokens per block: gate_up 1 up to 32 tokens (the grid then fills
// the chip), else 2; the down's segments are short: always 2
__host__ __device__ inline int sh_sk_nc(int GLU, int S) { return GLU && S <= 32 ? 1 : 2; }
__host__ __device__ inline int sh_sk_rows(int GLU, int O) { return GLU ? O / 8 : O / 16; }
__host__ __device__ inline int sh_sk_cols(int S, int nc) { return (S + 16 * nc - 1) / (16 * nc); }
__host__ __device__ inline size_t sh_sk_lds(int nc) { return (size_t)8 * 16 * 16 * nc * 4; }
// PF: steps in flight (weight and part words); 0: 8 with one column tile, else 4 (measured
// best at B = 8, 32 and 64)
template <int GLU, int NC, int FX, int PF = 0>
__device__ __forceinline__ void sh_sk_block(const ShSkArgs &A, int bx, int by, float *red) {
    const uint16_t *__restrict__ W0 = A.W0, *__restrict__ W1 = A.W1, *__restrict__ xp = A.xp;
    const int S = A.S, K = A.K, O = A.O;
    void *__restrict__ outp = A.out;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4;
    const int G = K / SH_RG, nseg = sh_nseg(G), GS = G / nseg;
    const int r0 = bx * (GLU ? 8 : 16), tok0 = by * 16 * NC;
    if (wave < nseg) {
        const uint16_t *wr = GLU ? (m < 8 ? W0 + (int64_t)(r0 + m) * K : W1 + (int64_t)(r0 + m - 8) * K)
                                 : W0 + (int64_t)(r0 + m) * K;
        wr += 8 * kq;
        const uint16_t *br[NC];
        const float *bf[NC];
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int64_t tok = min(tok0 + 16 * c + m, S - 1);
            if constexpr (FX) bf[c] = A.xf + tok * K + 8 * kq;
            else br[c] = xp + tok * K * 3 + 8 * kq;
        }
        const int g0 = wave * GS;
        // a step's words: the weights and, per column tile, the 3 part words (or the 8 f32
        // inputs they are split from)
        struct Step { sw_u32x4 a, b[NC][FX ? 2 : 3]; };
        auto load = [&](int s, Step &st) {
            const int g = g0 + min(s, GS - 1);
            st.a = *(const sw_u32x4 *)(wr + (int64_t)g * SH_RG);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if constexpr (FX) {
                    st.b[c][0] = *(const sw_u32x4 *)(bf[c] + g * SH_RG);
                    st.b[c][1] = *(const sw_u32x4 *)(bf[c] + g * SH_RG + 4);
                } else {
#pragma unroll
                    for (int p = 0; p < 3; p++) st.b[c][p] = *(const sw_u32x4 *)(br[c] + (g * 3 + p) * SH_RG);
                }
            }
        };
        sw_f32x4 acc[NC];
#pragma unroll
        for (int c = 0; c < NC; c++) acc[c] = sw_f32x4{0.f, 0.f, 0.f, 0.f};
        constexpr int SHK_PF = PF ? PF : NC == 1 ? 8 : 4;
        Step ring[SHK_PF];
#pragma unroll
        for (int u = 0; u < SHK_PF; u++) load(u, ring[u]);
        auto use = [&](const Step &st) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if constexpr (FX) {
                    sw_u32x4 p0, p1, p2;
                    sh_split8(__builtin_bit_cast(sw_f32x4, st.b[c][0]), __builtin_bit_cast(sw_f32x4, st.b[c][1]), p0, p1, p2);
                    acc[c] = sh_mfma3(st.a, p0, p1, p2, acc[c]);
                } else {
                    acc[c] = sh_mfma3(st.a, st.b[c][0], st.b[c][1], st.b[c][2], acc[c]);
                }
            }
        };
        // full rounds with unconditional refills (past the end they re-read the last step),
        // then the last round without: no branch join inside a round, so the waits stay
        // per step instead of draining the ring at every round
        int s0 = 0;
        for (; s0 + SHK_PF < GS; s0 += SHK_PF) {
#pragma unroll
            for (int u = 0; u < SHK_PF; u++) {
                use(ring[u]);
                load(s0 + u + SHK_PF, ring[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < SHK_PF; u++)
            if (s0 + u < GS) use(ring[u]);
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[(wave * 16 + 4 * kq + r) * 16 * NC + 16 * c + m] = acc[c][r];
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (GLU) {
        for (int it = tid; it < 8 * 16 * NC; it += SH_SK_NT) {
            const int r = it / (16 * NC), t = it - r * 16 * NC, tok = tok0 + t;
            float yg = -0.0f, yu = -0.0f;
            for (int sg = 0; sg < nseg; sg++) {
                yg = yg + red[(sg * 16 + r) * 16 * NC + t];
                yu = yu + red[(sg * 16 + 8 + r) * 16 * NC + t];
            }
            if (tok < S) {
                const int i = r0 + r;
                uint32_t pa, pb, pc;
                sh_split3((yg / (1.0f + expf(-yg))) * yu, pa, pb, pc);
                uint16_t *dst = (uint16_t *)outp + (int64_t)tok * O * 3 + (i >> 5) * 3 * SH_RG + (i & 31);
                dst[0] = (uint16_t)pa;
                dst[SH_RG] = (uint16_t)pb;
                dst[2 * SH_RG] = (uint16_t)pc;
            }
        }
    } else {
        for (int it = tid; it < 16 * 16 * NC; it += SH_SK_NT) {
            const int r = it / (16 * NC), t = it - r * 16 * NC, tok = tok0 + t;
            float y = -0.0f;
            for (int sg = 0; sg < nseg; sg++) y = y + red[(sg * 16 + r) * 16 * NC + t];
            if (tok < S) ((float *)outp)[(int64_t)tok * O + r0 + r] = y;
        }
    }
}

#endif
