// k_mfma.hip -- the grouped int4 expert GEMMs of prefill on the int8 matrix
// cores, bit-identical to the dot8 kernels of k_dot8.hip.
//
// For a weight row and a group of 32 inputs, dot8 forms the exact integer
// acc = sum_k w_k D_k (w_k = n_k - 8 in [-8, 7], D_k the 7-limb integer of
// input k, |D_k| < 2^21.2) and the term (float)acc * (s * xf).  Here every D
// is cut into two 12-bit digits, D = E1 2^12 + E0 with E0 the residue of D
// mod 4096 in [-2048, 2048), and every E into a low nibble and a signed high
// byte, E = lo + 16 hi (lo = E & 15, hi = E >> 4; both int8).  One
// v_mfma_i32_16x16x64_i8 has 64 k-slots: the 32 weights as bytes w against
// lo, and as bytes 16 w against hi, so it returns
//     R = sum_k (w_k lo_k + 16 w_k hi_k) = sum_k w_k E_k
// exactly (|R| < 2^19); the two of E0 and E1 give acc = (R1 << 12) + R0,
// dot8's int32.  The terms and the canonical row sum (pairwise trees over
// runs of 16 groups, padded with +0 terms, the runs added left to right)
// follow dot8's operations one for one, so a token's output has the same
// bits whichever kernel ran its group.
//
// Digits in memory: per (input row, group) 128 bytes, the B operands of the
// two MFMAs: byte op*64 + (k>>3)*16 + half*8 + (k&1)*4 + ((k&7)>>1) holds
// input k's lo (half 0) or hi (half 1) digit of E0 (op 0) or E1 (op 1).
// Lane l of the MFMA (column l % 16, k quarter q = l / 16) reads the 16
// bytes of quarter q, and its A operand holds the same k-slots of a weight
// row: [w of k = 8q+0,2,4,6 | w of 8q+1,3,5,7 | 16w of the same | 16w ...],
// expanded from packed dword q of the row's group (nibble k at bits 4(k&7)).
//
// Block: 128 weight rows (8 tiles of 16) x a tile of up to 64 tokens (4
// tiles of 16) of one group, 16 waves; wave w takes row tiles w&3 and (w&3)+4
// (for gate_up the gate and the up rows of the same 16 outputs) against
// token tile w>>2, so each lane holds 8 (row, token) sums and a wave stays
// within 128 registers: four waves per SIMD, which hide each other's MFMA,
// LDS and barrier waits.  The operands of 4 input groups at a time -- the
// rows' weights expanded once for the 16 waves, the tokens' digits, the
// scales and the token factors -- are staged in LDS in two buffers: while the
// waves compute one chunk from LDS, the next chunk's loads are in flight in
// registers, issued before each chunk's barrier so that the waves waiting there
// overlap them.  A tile's token tiles with no tokens compute nothing and have
// no digits staged; a prefill's tiles are mostly one full tile per expert plus
// a tail of 1-2 token tiles, whose fixed staging cost (the weights of all 128
// rows) is most of their time.  The inner loop reads LDS only, every wave read
// a contiguous 1 KB (conflict-free).
#include "sw_hip.h"
#include "sw_gate.h"

#define MF_DW 32           // digit dwords per (input row, group)
#define MF_ROWS 128        // weight rows per block
#define MF_TT SW_MF_TT     // tokens per block tile (64)
#define MF_NT 1024         // threads per block: 16 waves
#define MF_CG 4            // input groups per staged chunk
// one chunk buffer in LDS: expanded weights [g][tile 8][quarter 4][row 16] x 16 B,
// digits [g][token tile 4][op 2][quarter 4][token 16] x 16 B, scales [g][row],
// token factors [g][token]
#define MF_A_OFF 0
#define MF_B_OFF (MF_A_OFF + MF_CG * MF_ROWS * 64)
#define MF_S_OFF (MF_B_OFF + MF_CG * MF_TT * 128)
#define MF_X_OFF (MF_S_OFF + MF_CG * MF_ROWS * 4)
#define MF_BUF (MF_X_OFF + MF_CG * MF_TT * 4)
#define MF_HLD 65          // floats per token row of h in the gate_up epilogue

// ------------------------------------------------------------ digits ----
// one group by the 32 lanes of a half-wave (i = lane in the half): the same
// exponent and 7 limbs as limbs_group, written as the MFMA digits above;
// the factor 2^(e - 21) (NaN for a group holding a NaN or an infinity, whose
// digits are 0) is limbs_group's
__device__ __forceinline__ void digits_group(float v, int i, uint32_t *__restrict__ dst, float *__restrict__ fdst) {
    bool bad;
    const int e = limbs_exp(v, bad);
    float y = ldexpf(v, -e);
    int D = 0;
#pragma unroll
    for (int l = 0; l < SW_ND; l++) D = D * 8 + (int)limb_digit(y);
    if (bad) D = 0;
    const int E0 = ((D + 2048) & 4095) - 2048, E1 = (D - E0) >> 12;
    const int sh = 8 * ((i & 7) >> 1);
    uint32_t b[4] = {(uint32_t)(E0 & 15) << sh, (uint32_t)((E0 >> 4) & 255) << sh, (uint32_t)(E1 & 15) << sh,
                     (uint32_t)((E1 >> 4) & 255) << sh};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        b[q] |= __shfl_xor(b[q], 2, 32);
        b[q] |= __shfl_xor(b[q], 4, 32);
    }
    if ((i & 6) == 0) {                               // lane 8 kq + par holds the dwords of (kq, par)
        const int kq = i >> 3, par = i & 1;
        dst[kq * 4 + par] = b[0];
        dst[kq * 4 + 2 + par] = b[1];
        dst[16 + kq * 4 + par] = b[2];
        dst[16 + kq * 4 + 2 + par] = b[3];
    }
    if (i == 0) *fdst = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 3 * SW_ND);
}

// rows x[r, K] f32 -> digits dg[r][K/32][32 dwords], factors xs[r][K/32]
__global__ __launch_bounds__(256) void k_digits(const float *__restrict__ x, int K, int rows, uint32_t *__restrict__ dg,
                                                float *__restrict__ xs) {
    const int G = K / SW_RG;
    const int tid = threadIdx.x, g = blockIdx.x * 8 + (tid >> 5), r = blockIdx.y;
    if (r >= rows || g >= G) return;                  // whole half-waves leave together
    digits_group(x[(int64_t)r * K + g * SW_RG + (tid & 31)], tid & 31, dg + ((int64_t)r * G + g) * MF_DW,
                 xs + (int64_t)r * G + g);
}

int sw_launch_digits(hipStream_t st, const float *x, int rows, int K, uint32_t *dg, float *xs) {
    if (K % SW_RG || rows <= 0) return -1;
    const int G = K / SW_RG;
    SW_LAUNCH(k_digits, dim3((unsigned)((G + 7) / 8), (unsigned)rows), dim3(256), 0, st, x, K, rows, dg, xs);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------ GEMM ----
struct MfArgs {
    SwQ4 W;
    int gsh;
    const uint32_t *dg;     // input digits [rows][G][MF_DW]
    const float *xs;        // input factors [rows][G]
    SwGroups grp;           // tiles: items of up to MF_TT tokens, P live
    int I;                  // GLU: the intermediate size (W.O == 2 I)
    int nrb;                // row blocks
    uint32_t *hdg;          // GLU: h of every packed row as digits [T][I/32][MF_DW]
    float *hxs;             //      and factors [T][I/32]
    float *Y;               // rows: [T][O]
    const SwTab *tab;       // per-group tensors (the _tab launches) or null
};

// the pairwise tree of a run of CH terms (CH a power of two <= 16), fed one
// term at a time (gl = the term's index in the run, known at compile time
// after unrolling): L holds the pending single, pair, quad and eight; the
// run's sum lands in run after the last term
template <int CH>
__device__ __forceinline__ void tree_push(float p, int gl, float (&L)[4], float &run) {
    if (CH == 1) { run = p; return; }
    if ((gl & 1) == 0) { L[0] = p; return; }
    float s = L[0] + p;
    if (CH == 2) { run = s; return; }
    if ((gl & 2) == 0) { L[1] = s; return; }
    s = L[1] + s;
    if (CH == 4) { run = s; return; }
    if ((gl & 4) == 0) { L[2] = s; return; }
    s = L[2] + s;
    if (CH == 8) { run = s; return; }
    if ((gl & 8) == 0) { L[3] = s; return; }
    run = L[3] + s;
}

// the four int8 operand dwords of packed weight dword w (nibble n = w_k + 8
// of k = 8q + c at bits 4c): bytes w of the even k, w of the odd k, 16 w of
// the even k, 16 w of the odd k
__device__ __forceinline__ sw_i32x4 mf_expand(uint32_t w) {
    const uint32_t wx = w ^ 0x88888888u;             // nibbles w_k as 4-bit two's complement
    sw_i32x4 a;
    a[0] = (int)(((w & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u);          // n + 120 < 256, then bit 7 flipped: n - 8
    a[1] = (int)((((w >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u);
    a[2] = (int)((wx << 4) & 0xF0F0F0F0u);
    a[3] = (int)(wx & 0xF0F0F0F0u);
    return a;
}

template <int N>
struct MfIc { static constexpr int v = N; };

template <int GLU, int CH, int FULL, int PT>
__global__ __launch_bounds__(MF_NT, 1) void k_mf(MfArgs A) {
    static_assert(MF_NT == 1024 && MF_CG * MF_ROWS == 512 && MF_CG * MF_TT * 8 == 2 * MF_NT, "staging map");
    extern __shared__ __align__(16) uint8_t mf_lds[];
    const SwQ4 W = A.W;
    const SwGroups grp = A.grp;
    const int K = W.K, G = K / SW_RG, O = W.O;
    const int NC = G / MF_CG;                              // staged chunks (G % 4 == 0)
    const int NCV = (G + CH - 1) / CH * (CH / MF_CG);      // chunks of the padded runs
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, kq = lane >> 4;
    const int mp = wave & 3, tt = wave >> 2;               // row tiles mp, mp + 4; token tile tt

    // block -> (tile, row block), XCD-aware over the live blocks
    const int nlive = *grp.P * A.nrb;
    if ((int)blockIdx.x >= nlive) return;
    const int wk = sw_xcd_work((int)blockIdx.x, nlive);
    const int tile = wk / A.nrb, rb = wk - tile * A.nrb;
    int e, beg, t0, tend;
    if (!grp_work(grp, tile, MF_TT, e, beg, t0, tend)) return;
    const int nt = tend - t0;
    const int i0 = rb * 64, r0 = rb * MF_ROWS;
    // weight row of local row r (GLU: gate rows i0..i0+63, then the up rows)
    // (PT: row r of the group's own gate, up or down tensor)
    auto srow = [&](int r) -> uint32_t {
        const uint32_t eo = PT ? 0u : (uint32_t)e * (uint32_t)O;
        if (GLU) return eo + (uint32_t)(r < 64 ? i0 + r : (PT ? 0 : A.I) + i0 + r - 64);
        return eo + (uint32_t)(r0 + r);     // past O: the next expert's rows (PT: zeros), not stored
    };
    auto token = [&](int t) -> int64_t {                   // input row of tile token t (past the tile: its last)
        const int pr = beg + t0 + min(t, nt - 1);
        return grp.grow ? grp.grow[pr] : pr;
    };
    const int ng = W.gs > 0 ? K / W.gs : 1;
    const uint32_t rbytes = (uint32_t)K / 2;
    // staging roles by whole waves; for gate_up rotated so that in a tile of 1-3 token tiles the
    // computing waves (token tiles tt < nact: waves 0 .. 4 nact - 1) take the roles with no work
    // (the digits of token tiles that do not compute are not staged) or the lightest (C4:
    // gate_up 2.11 -> 2.04 ms; the down launch, 8 chunks, ran 1-2% slower with it, also when
    // rotated for one-column tiles only)
    const int nact = (nt + 15) >> 4;
    const int rot = GLU ? (nact == 1 ? 10 : nact < 4 ? 8 : 0) : 0;
    const int st = (tid + 64 * rot) & (MF_NT - 1);
    sw_rsrc rq, rs;
    if constexpr (PT) {
        // a staging thread's row ra = st & 127 is an up row iff (st >> 6) & 1: uniform per wave
        const SwTab tb_ = A.tab[e];
        if (GLU) {
            const bool up = __builtin_amdgcn_readfirstlane((st >> 6) & 1);
            rq = sw_make_rsrc(up ? tb_.u : tb_.g, (uint32_t)A.I * rbytes);
            rs = sw_make_rsrc(up ? tb_.us : tb_.gs, (uint32_t)A.I * (uint32_t)ng * 4);
        } else {
            rq = sw_make_rsrc(tb_.d, (uint32_t)O * rbytes);
            rs = sw_make_rsrc(tb_.ds, (uint32_t)O * (uint32_t)ng * 4);
        }
    } else {
        rq = sw_q4_rq(W);
        rs = sw_q4_rs(W);
    }

    // ---- staging: the units of a chunk of staging slot st (u = st & 511 within a group of 512 units)
    //  weights (slots < 512): row ra = st & 127 of group st >> 7 (16 B packed, expanded on
    //           the store) + its scale
    //  digits:  16 B (op, quarter) of token tb of groups st >> 9 and (st >> 9) + 2: unit u of a
    //           group is token tile u >> 7, op (u >> 6) & 1, quarter (u >> 4) & 3, token u & 15;
    //           staged only for the token tiles that compute (dact)
    //  factors (slots < 256): token tx of group st >> 6
    constexpr int DG_PER = MF_CG * MF_TT * 8 / MF_NT;      // digit units per slot (2)
    const bool wst = st < MF_CG * MF_ROWS;                 // uniform per wave
    const int ra = st & 127, ga = (st >> 7) & 3;
    const uint32_t rowa = srow(ra);
    const int tb = ((st >> 7) & 3) * 16 + (st & 15), opb = (st >> 6) & 1, kqb = (st >> 4) & 3, gb = st >> 9;
    const uint32_t *__restrict__ dgb = A.dg + token(tb) * G * MF_DW + opb * 16 + kqb * 4;
    const int tx = st & 63, gx = (st >> 6) & 3;
    const float *__restrict__ xsx = A.xs + token(tx) * G;
    const bool dact = ((st >> 7) & 3) < nact;             // uniform per wave
    sw_u32x4 pka, pkb[DG_PER];
    float psa = 1.0f, pxf = 0.f;
    auto stage_load = [&](int c) {
        const int g0 = c * MF_CG;
        if (wst) {
            pka = sw_ld16(rq, rowa * rbytes + (uint32_t)(g0 + ga) * 16, 0);
            if (W.gs > 0) psa = sw_ld4f(rs, (rowa * (uint32_t)ng + (uint32_t)(((g0 + ga) * SW_RG) >> A.gsh)) * 4, 0);
        }
        if (dact)
#pragma unroll
            for (int v = 0; v < DG_PER; v++) pkb[v] = *(const sw_u32x4 *)(dgb + (g0 + gb + 2 * v) * MF_DW);
        if (st < MF_CG * MF_TT) pxf = xsx[g0 + gx];
    };
    auto stage_store = [&](int buf) {
        uint8_t *base = mf_lds + buf * MF_BUF;
        sw_i32x4 *Al = (sw_i32x4 *)(base + MF_A_OFF);
        sw_u32x4 *Bl = (sw_u32x4 *)(base + MF_B_OFF);
        if (wst) {
            const int m = ra >> 4, i = ra & 15;
#pragma unroll
            for (int q = 0; q < 4; q++) Al[((ga * 8 + m) * 4 + q) * 16 + i] = mf_expand(pka[q]);
            ((float *)(base + MF_S_OFF))[ga * MF_ROWS + ra] = psa;
        }
        if (dact)
#pragma unroll
            for (int v = 0; v < DG_PER; v++) Bl[v * MF_NT + st] = pkb[v];
        if (st < MF_CG * MF_TT) ((float *)(base + MF_X_OFF))[gx * MF_TT + tx] = pxf;
    };

    const bool wact = tt * 16 < nt;                        // uniform over the wave
    float y[2][4], L[2][4][4], run[2][4];
    // the LDS operands of one group for this wave
    struct Frag {
        sw_i32x4 a[2], b[2];
        sw_f32x4 s4[2];
        float xf;
    };
    auto fetch = [&](Frag &F, const uint8_t *base, int g) {
        const sw_i32x4 *Al = (const sw_i32x4 *)(base + MF_A_OFF);
        const sw_i32x4 *Bl = (const sw_i32x4 *)(base + MF_B_OFF);
        const float *Sl = (const float *)(base + MF_S_OFF), *Xl = (const float *)(base + MF_X_OFF);
#pragma unroll
        for (int mi = 0; mi < 2; mi++) {
            const int m = mp + 4 * mi;
            F.a[mi] = Al[((g * 8 + m) * 4 + kq) * 16 + col];
            F.s4[mi] = *(const sw_f32x4 *)(Sl + g * MF_ROWS + 16 * m + 4 * kq);
        }
        F.b[0] = Bl[((g * 4 + tt) * 2 + 0) * 64 + lane];
        F.b[1] = Bl[((g * 4 + tt) * 2 + 1) * 64 + lane];
        F.xf = Xl[g * MF_TT + 16 * tt + col];
    };
    // the terms of one group (zero terms for the padding of a run: REAL = 0) into the trees
    auto group = [&](const Frag &F, int gl, bool first, auto RC) {
        constexpr bool REAL = decltype(RC)::v;
        sw_i32x4 R0[2], R1[2];
        if (REAL) {
            const sw_i32x4 z = {0, 0, 0, 0};
            // the MFMAs issue at raised wave priority: the SIMD's four waves, which leave
            // each chunk's barrier together, then spread out instead of waiting on their
            // products in step (C4: gate_up 2.33 -> 2.30 ms, down 1.32 -> 1.26 ms; the
            // priority raised for the whole group, or for the LDS fetches, gained less)
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                R0[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(F.a[mi], F.b[0], z, 0, 0, 0);
                R1[mi] = __builtin_amdgcn_mfma_i32_16x16x64_i8(F.a[mi], F.b[1], z, 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
        }
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float p = 0.f;                              // the +0 terms of a padded run
                if (REAL) {
                    const int acc = (R1[mi][j] << 12) + R0[mi][j];
                    p = (float)acc * (F.s4[mi][j] * F.xf);
                }
                tree_push<CH>(p, gl, L[mi][j], run[mi][j]);
                if (gl == CH - 1) y[mi][j] = first ? run[mi][j] : y[mi][j] + run[mi][j];
            }
    };
    // one chunk: its 4 groups at positions Q*4 .. Q*4+3 of the run (Q known at compile time)
    auto chunk = [&](auto QC, auto RC, int c) {
        constexpr int Q = decltype(QC)::v;
        const uint8_t *base = mf_lds + (c & 1) * MF_BUF;
        const bool first = c < CH / MF_CG;                 // in the first run
        // (one group's operands at a time: a second set for the next group measured slower,
        // its registers spill at 128)
#pragma unroll
        for (int g = 0; g < MF_CG; g++) {
            Frag F;
            if (decltype(RC)::v) fetch(F, base, g);
            group(F, Q * MF_CG + g, first, RC);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto chunk_q = [&](auto RC, int c) {
        switch (c % (CH / MF_CG)) {
            case 0: chunk(MfIc<0>{}, RC, c); break;
            case 1: if constexpr (CH / MF_CG > 1) chunk(MfIc<1 % (CH / MF_CG)>{}, RC, c); break;
            case 2: if constexpr (CH / MF_CG > 2) chunk(MfIc<2 % (CH / MF_CG)>{}, RC, c); break;
            default: if constexpr (CH / MF_CG > 3) chunk(MfIc<3 % (CH / MF_CG)>{}, RC, c); break;
        }
    };

    stage_load(0);
    stage_store(0);
    if (NC > 1) stage_load(1);
    __syncthreads();
    for (int c = 0; c < NCV; c++) {
        if (wact) {
            if (FULL || c < NC) chunk_q(MfIc<1>{}, c);
            else if constexpr (!FULL) chunk_q(MfIc<0>{}, c);
        }
        if (c + 1 < NC) stage_store((c + 1) & 1);          // read by no wave since the last barrier
        if (c + 2 < NC) stage_load(c + 2);                 // registers only: issued before the barrier's wait
        __syncthreads();
    }

    if constexpr (GLU) {
        // h = silu(gate) * up per (token, output), through LDS to the digit writers
        float *hl = (float *)mf_lds;                       // [MF_TT][MF_HLD]; every wave is past its last read
        const int I = A.I;
        if (wact) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int i = 16 * mp + 4 * kq + j, t = 16 * tt + col;
                    float yg = y[0][j], yu = y[1][j];
                    if (W.gs <= 0) {                        // per-row scales after the sum
                        if constexpr (PT) {
                            yg = yg * A.tab[e].gs[i0 + i];
                            yu = yu * A.tab[e].us[i0 + i];
                        } else {
                            yg = yg * W.s[(int64_t)e * (2 * I) + i0 + i];
                            yu = yu * W.s[(int64_t)e * (2 * I) + I + i0 + i];
                        }
                    }
                    hl[t * MF_HLD + i] = (yg / (1.0f + expf(-yg))) * yu;
                }
        }
        __syncthreads();
        // the block's 64 outputs are two limb groups of the down projection's input
        const int GI = I / SW_RG, hw = tid >> 5, i = tid & 31;
        for (int job = hw; job < 2 * nt; job += MF_NT / 32) {
            const int t = job >> 1, q = job & 1;
            const int64_t prow = beg + t0 + t;
            const int gi = 2 * rb + q;
            digits_group(hl[t * MF_HLD + 32 * q + i], i, A.hdg + (prow * GI + gi) * MF_DW, A.hxs + prow * GI + gi);
        }
    } else {
        if (wact) {
            const int t = 16 * tt + col;
            if (t < nt) {
                float *yrow = A.Y + (int64_t)(beg + t0 + t) * O;
#pragma unroll
                for (int mi = 0; mi < 2; mi++) {
                    const int row = r0 + 16 * (mp + 4 * mi) + 4 * kq;
                    if (row < O) {
                        sw_f32x4 o;
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            o[j] = W.gs > 0 ? y[mi][j] : y[mi][j] * (PT ? A.tab[e].ds[row + j] : W.s[(int64_t)e * O + row + j]);
                        *(sw_f32x4 *)(yrow + row) = o;
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------ launch ----
static size_t mf_lds_bytes() {
    const size_t h = (size_t)MF_TT * MF_HLD * 4;
    return 2 * MF_BUF > h ? 2 * MF_BUF : h;
}
// dynamic LDS above 64 KB, raised once per kernel, outside any stream work
template <int GLU, int CH, int FULL, int PT>
static int mf_go(hipStream_t st, unsigned nblocks, const MfArgs &A) {
    static size_t raised = 0;
    const size_t lds = mf_lds_bytes();
    if (lds > raised) {
        if (hipFuncSetAttribute((const void *)k_mf<GLU, CH, FULL, PT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) return -1;
        raised = lds;
    }
    SW_LAUNCH((k_mf<GLU, CH, FULL, PT>), dim3(nblocks), dim3(MF_NT), lds, st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
template <int GLU, int PT = 0>
static int mf_dispatch(hipStream_t st, unsigned nblocks, const MfArgs &A) {
    const int G = A.W.K / SW_RG, Gq = run_lanes(G), CH = Gq < 16 ? Gq : 16;
    const bool full = G == Gq;
    if (CH == 16) return full ? mf_go<GLU, 16, 1, PT>(st, nblocks, A) : mf_go<GLU, 16, 0, PT>(st, nblocks, A);
    if (CH == 8) return full ? mf_go<GLU, 8, 1, PT>(st, nblocks, A) : mf_go<GLU, 8, 0, PT>(st, nblocks, A);
    if (CH == 4) return full ? mf_go<GLU, 4, 1, PT>(st, nblocks, A) : mf_go<GLU, 4, 0, PT>(st, nblocks, A);
    return -1;
}
// shapes: K a multiple of 128 (whole chunks of 4 input groups), tiles listed (items, P)
static int mf_check(const SwQ4 &W, const SwGroups &g, int &gsh) {
    if (W.K % (SW_RG * MF_CG) || !g.items || !g.P || g.ngroups_max <= 0 || !sw_q4_extent_ok(W)) return -1;
    return sw_q4_gsh(W, gsh);
}

int sw_launch_mf_glu(hipStream_t st, SwQ4 W, const uint32_t *dg, const float *xs, SwGroups g, int I, uint32_t *hdg,
                     float *hxs) {
    int gsh;
    if (mf_check(W, g, gsh) || I % 64 || W.O != 2 * I) return -1;
    const int nrb = I / 64;
    const MfArgs A = {W, gsh, dg, xs, g, I, nrb, hdg, hxs, nullptr};
    return mf_dispatch<1>(st, (unsigned)(g.ngroups_max * nrb), A);
}

int sw_launch_mf_rows(hipStream_t st, SwQ4 W, const uint32_t *dg, const float *xs, SwGroups g, float *Y) {
    int gsh;
    if (mf_check(W, g, gsh) || W.O % 4) return -1;
    const int nrb = (W.O + MF_ROWS - 1) / MF_ROWS;
    const MfArgs A = {W, gsh, dg, xs, g, 0, nrb, nullptr, nullptr, Y};
    return mf_dispatch<0>(st, (unsigned)(g.ngroups_max * nrb), A);
}

// the same two GEMMs over per-group tensors: group c's gate/up/down are tab[gexp[c]]
// (W gives O, K and gs; each tensor holds one expert)
int sw_launch_mf_glu_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const uint32_t *dg, const float *xs, SwGroups g,
                         int I, uint32_t *hdg, float *hxs) {
    int gsh;
    W.E = 1;
    if (!tab || !hdg || !hxs || mf_check(W, g, gsh) || I % 64 || W.O != 2 * I) return -1;
    const int nrb = I / 64;
    const MfArgs A = {W, gsh, dg, xs, g, I, nrb, hdg, hxs, nullptr, tab};
    return mf_dispatch<1, 1>(st, (unsigned)(g.ngroups_max * nrb), A);
}
int sw_launch_mf_rows_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const uint32_t *dg, const float *xs, SwGroups g,
                          float *Y) {
    int gsh;
    W.E = 1;
    if (!tab || !Y || mf_check(W, g, gsh) || W.O % 4) return -1;
    const int nrb = (W.O + MF_ROWS - 1) / MF_ROWS;
    const MfArgs A = {W, gsh, dg, xs, g, 0, nrb, nullptr, nullptr, Y, tab};
    return mf_dispatch<0, 1>(st, (unsigned)(g.ngroups_max * nrb), A);
}
