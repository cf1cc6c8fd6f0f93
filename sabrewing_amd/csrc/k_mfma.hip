// k_mfma.hip -- the grouped int4 expert GEMMs of prefill on the matrix cores,
// bit-identical to the dot8 kernels of k_dot8.hip.
//
// For a weight row and a group of 32 inputs, dot8 forms the exact integer
// acc = sum_k w_k D_k (w_k = n_k - 8 in [-8, 7], D_k the 7-limb integer of
// input k, |D_k| < 2^21.2) and the term (float)acc * (s * xf).  Here every D
// is cut into two 12-bit digits, D = E1 2^12 + E0 with E0 the residue of D
// mod 4096 in [-2048, 2048) and |E1| <= 585.  The weights and both digits are
// integers that f16 holds exactly, and every product (|w E| <= 2^14) and
// every partial sum of 32 of them (< 2^19) is an integer that f32 holds
// exactly, so two v_mfma_f32_16x16x32_f16 return R0 = sum_k w_k E0_k and
// R1 = sum_k w_k E1_k exactly, whatever order the hardware adds in; then
// fma(R1, 4096, R0) rounds the exact acc = 4096 R1 + R0 once, to nearest even,
// which is (float)acc, dot8's conversion of its int32, bit for bit.  The
// terms and the canonical row sum (pairwise trees over runs of 16 groups,
// padded with +0 terms, the runs added left to right) follow dot8's
// operations one for one, so a token's output has the same bits whichever
// kernel ran its group.
//
// Digits in memory: per (input row, group) 128 bytes, E0 of the 32 inputs as
// f16, then E1: the B operands of the two MFMAs.  Lane l of an MFMA (column
// l % 16, k quarter q = l / 16) reads the 16 bytes of inputs 8q .. 8q+7 (in
// the slot order of mf_expand), and its A operand holds the same inputs of a
// weight row as f16, expanded from packed dword q of the row's group.
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
// overlap them.  Each staging wave load covers 16 rows (or tokens) with the
// chunk's 4 groups side by side in memory: 16 cache lines a load, not 64 (the
// staging loads' cache lines, more than the VALU, set the chunk's time).  A
// tile's token tiles with no tokens compute nothing and have no digits staged;
// a group's tokens are split into equal tiles of whole 16-token columns
// (sw_mf_tile).  The inner loop reads LDS only, every wave read a contiguous
// 1 KB (conflict-free).  A down block takes up to 4 row blocks of its tile with
// one staging pipeline running across them.
#include "sw_hip.h"
#include "sw_gate.h"

#define MF_DW 32           // digit dwords per (input row, group)
#define MF_ROWS 128        // weight rows per block
#define MF_TT SW_MF_TT     // tokens per block tile (64)
#define MF_NT 1024         // threads per block: 16 waves, four per SIMD
#define MF_CG 4            // input groups per staged chunk
// the two chunk buffers in LDS, each operand's pair side by side (so that one base
// register per operand and immediate offsets reach both): expanded weights
// [buf][g][tile 8][quarter 4][row 16] x 16 B, digits [buf][g][token tile 4][op 2]
// [quarter 4][token 16] x 16 B, scales [buf][g][row], token factors [buf][g][token]
#define MF_A_SZ (MF_CG * MF_ROWS * 64)
#define MF_B_SZ (MF_CG * MF_TT * 128)
#define MF_S_SZ (MF_CG * MF_ROWS * 4)
#define MF_X_SZ (MF_CG * MF_TT * 4)
#define MF_A_OFF 0
#define MF_B_OFF (MF_A_OFF + 2 * MF_A_SZ)
#define MF_S_OFF (MF_B_OFF + 2 * MF_B_SZ)
#define MF_X_OFF (MF_S_OFF + 2 * MF_S_SZ)
#define MF_LDS_STAGE (MF_X_OFF + 2 * MF_X_SZ)
#ifndef MF_PF
#define MF_PF 1            // the next group's operands fetched during this group's products
#endif
#define MF_YLD 129         // floats per token row of a row block's gate and up sums (<= 32 tokens)
#define MF_HLD 65          // floats per token row of h in the gate_up epilogue
#define MF_EP_OFF MF_LDS_STAGE                            // the epilogue's own LDS
#define MF_EP_SZ (MF_TT * MF_HLD * 4 > 32 * MF_YLD * 4 ? MF_TT * MF_HLD * 4 : 32 * MF_YLD * 4)

// ------------------------------------------------------------ digits ----
// one group by the 32 lanes of a half-wave (i = lane in the half): the same
// exponent and 7 limbs as limbs_group, written as the MFMA digits above (E0
// then E1 of the 32 inputs as f16, each quarter of 8 inputs in the operand
// order of mf_expand); the factor 2^(e - 21) (NaN for a group holding a NaN or
// an infinity, whose digits are 0) is limbs_group's
__device__ __forceinline__ void digits_group(float v, int i, uint32_t *__restrict__ dst, float *__restrict__ fdst) {
    bool bad;
    const int e = limbs_exp(v, bad);
    float y = ldexpf(v, -e);
    int D = 0;
#pragma unroll
    for (int l = 0; l < SW_ND; l++) D = D * 8 + (int)limb_digit(y);
    if (bad) D = 0;
    const int E0 = ((D + 2048) & 4095) - 2048, E1 = (D - E0) >> 12;
    // the odd inputs of a quarter meet weights 16 w: their digits are E / 16 (exact:
    // at most 11 significant bits, none below 2^-4)
    const float sc = (i & 1) ? 0.0625f : 1.0f;
    const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)((float)E0 * sc));
    const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)((float)E1 * sc));
    // input r = i & 7 of quarter q = i >> 3 sits at f16 slot (r & 1) * 4 + (r >> 1) of the
    // quarter's 4 dwords: inputs r and r ^ 2 share a dword (r & 2 the high half)
    const uint32_t o0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)h0, 0x4E, 0xF, 0xF, true);   // lane i ^ 2
    const uint32_t o1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)h1, 0x4E, 0xF, 0xF, true);
    if ((i & 2) == 0) {
        const int dw = (i >> 3) * 4 + (i & 1) * 2 + ((i >> 2) & 1);
        dst[dw] = h0 | (o0 << 16);
        dst[16 + dw] = h1 | (o1 << 16);
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
    int dg_rows;            // rows of dg and xs (dg_rows * K * 4 < 2^32)
    SwGroups grp;           // tiles: items of up to MF_TT tokens, P live
    int I;                  // GLU: the intermediate size (W.O == 2 I)
    int nrb;                // row blocks
    int rbper;              // row blocks per block (dividing nrb)
    uint32_t *hdg;          // GLU: h of every packed row as digits [T][I/32][MF_DW]
    float *hxs;             //      and factors [T][I/32]
    float *Y;               // rows: [T][O]
    const SwTab *tab;       // per-group tensors (the _tab launches) or null
};

// the A operand of packed weight dword w (nibble n_r = w_r + 8 of input r of the
// quarter at bits 4r) as f16 in the slot order of digits_group: (w0, w2), (w4, w6),
// (16 w1, 16 w3), (16 w5, 16 w7).  An even input's nibble is the low nibble of a
// byte, ORed under 0x64 into the f16 1024 + n; an odd input's is the high nibble,
// giving 1024 + 16 n.  Adding -1032, resp. -1152, leaves w, resp. 16 w, exactly.
__device__ __forceinline__ sw_i32x4 mf_expand(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = w & 0xF0F0F0F0u, magic = 0x64646464u;
    const sw_half2 off_lo = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const sw_half2 off_hi = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    // bytes (b0, 0x64, b1, 0x64) and (b2, 0x64, b3, 0x64) of lo and of hi
    const uint32_t p0 = __builtin_amdgcn_perm(magic, lo, 0x04010400u), p1 = __builtin_amdgcn_perm(magic, lo, 0x04030402u);
    const uint32_t p2 = __builtin_amdgcn_perm(magic, hi, 0x04010400u), p3 = __builtin_amdgcn_perm(magic, hi, 0x04030402u);
    sw_i32x4 a;
    a[0] = __builtin_bit_cast(int, __builtin_bit_cast(sw_half2, p0) + off_lo);
    a[1] = __builtin_bit_cast(int, __builtin_bit_cast(sw_half2, p1) + off_lo);
    a[2] = __builtin_bit_cast(int, __builtin_bit_cast(sw_half2, p2) + off_hi);
    a[3] = __builtin_bit_cast(int, __builtin_bit_cast(sw_half2, p3) + off_hi);
    return a;
}

template <int N>
struct MfIc { static constexpr int v = N; };

// the value of lane J of each lane's quad (DPP quad_perm [J, J, J, J])
template <int J>
__device__ __forceinline__ float mf_quad_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x55 * J, 0xF, 0xF, true));
}

template <int GLU, int CH, int FULL, int PT>
__global__ __launch_bounds__(MF_NT, 1) void k_mf(MfArgs A) {
    static_assert(MF_NT == 1024 && MF_CG * MF_ROWS == 512 && MF_CG * MF_TT * 8 == 2 * MF_NT, "staging map");
    extern __shared__ __align__(16) uint8_t mf_lds[];
    const SwQ4 W = A.W;
    const SwGroups grp = A.grp;
    const int K = W.K, G = K / SW_RG, O = W.O;
    const int NC = G / MF_CG;                              // staged chunks (G % 4 == 0)
    const int NCV = (G + CH - 1) / CH * (CH / MF_CG);      // chunks of the padded runs
    // (the wave index in a scalar register: what derives from it is uniform to the compiler)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, col = lane & 15,
              kq = lane >> 4;

    // block -> (tile, row block), XCD-aware over the live blocks
    // (a block takes rbper consecutive row blocks of one tile, its chunk pipeline running on
    // from one row block to the next: one start and one drain per rbper row blocks)
    const int rbper = GLU ? 1 : A.rbper;                   // (gate_up: one, known to the compiler)
    const int nrg = A.nrb / rbper;                         // row-block runs per tile
    const int nlive = *grp.P * nrg;
    if ((int)blockIdx.x >= nlive) return;
    const int wk = sw_xcd_work((int)blockIdx.x, nlive);
    const int tile = wk / nrg, rbf = (wk - tile * nrg) * rbper;     // the block's first row block
    int e, beg, t0, tend;
    if (!grp_work(grp, tile, MF_TT, e, beg, t0, tend)) return;
    const int nt = tend - t0, nact = (nt + 15) >> 4;       // tokens, token tiles with tokens
    const int i0 = rbf * 64, r0 = rbf * MF_ROWS;           // (of the first row block)
    constexpr int RPB = GLU ? 64 : MF_ROWS;                // weight rows a row block moves on by
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
    // computing waves take the roles with no work (the digits of token tiles that do not
    // compute are not staged) or the lightest
    const int rot = GLU ? (nact == 1 ? 10 : nact < 4 ? 8 : 0) : 0;
    const int st = (tid + 64 * rot) & (MF_NT - 1);
    const int sw_ = __builtin_amdgcn_readfirstlane(st >> 6);   // the staging role's wave index
    sw_rsrc rq, rs;
    if constexpr (PT) {
        // a staging thread's row ra (below) is an up row iff (st >> 9) & 1: uniform per wave
        const SwTab tb_ = A.tab[e];
        if (GLU) {
            const bool up = (sw_ >> 3) & 1;
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

    // ---- staging: the units of a chunk of staging slot st
    //  weights (every slot): half hq of row ra's 16 B packed of group ga (below; expanded on
    //           the store); slots of half 0 also the row's scale of the group
    //  digits:  16 B (op, quarter) of token tb of groups st >> 9 and (st >> 9) + 2: unit u of a
    //           group is token tile u >> 7, op (u >> 6) & 1, quarter (u >> 4) & 3, token u & 15;
    //           staged only for the token tiles that compute (dact)
    //  factors (the 4 waves with sw_ % 4 == 1): token tx of group gx (as ra, ga)
    // (the staging work spread evenly over the 16 waves: the chunk's barrier waits for the
    // slowest)
    // Every load is a buffer load: the slot's part of its offset in a register set once,
    // the chunk's in a scalar offset.
    constexpr int DG_PER = MF_CG * MF_TT * 8 / MF_NT;      // digit units per slot (2)
    // (a wave's 64 slots: one half of 16 rows, each with the chunk's 4 groups, side by side in
    // memory -- a wave load touches 16 lines, not 64 -- the rows fastest within each 16-slot
    // quarter, so that the LDS stores stay conflict-free)
    const int ra = ((st >> 7) << 4) | (st & 15), ga = (st >> 4) & 3, hq = (st >> 6) & 1;
    const bool sst = hq == 0;                              // uniform per wave
    const uint32_t rowa = srow(ra);
    const int tb = ((st >> 7) & 3) * 16 + (st & 15), opb = (st >> 6) & 1, kqb = (st >> 4) & 3, gb = st >> 9;
    const int xi = ((sw_ >> 2) << 6) | (st & 63);         // (factor slot)
    const int tx = ((xi >> 6) << 4) | (xi & 15), gx = (xi >> 4) & 3;   // (as ra, ga)
    const bool dact = ((sw_ >> 1) & 3) < nact;            // uniform per wave
    const bool xst = (sw_ & 3) == 1;
    const sw_rsrc rd = sw_make_rsrc(A.dg, (uint32_t)A.dg_rows * (uint32_t)G * MF_DW * 4);
    const sw_rsrc rx = sw_make_rsrc(A.xs, (uint32_t)A.dg_rows * (uint32_t)G * 4);
    const uint32_t vq = rowa * rbytes + (uint32_t)ga * 16 + (uint32_t)hq * 8;
    const uint32_t vs = (rowa * (uint32_t)ng + (uint32_t)((ga * SW_RG) >> A.gsh)) * 4;
    const uint32_t vd = ((uint32_t)token(tb) * (uint32_t)G + (uint32_t)gb) * MF_DW * 4 + (uint32_t)(opb * 16 + kqb * 4) * 4;
    const uint32_t vx = ((uint32_t)token(tx) * (uint32_t)G + (uint32_t)gx) * 4;
    uint2 pka;
    sw_u32x4 pkb[DG_PER];
    float psa = 1.0f, pxf = 0.f;
    // chunk q of the block: chunk q % NCV of its row block q / NCV (the row block's rows in
    // the vector offset, which the range check covers)
    auto stage_load = [&](int q) {
        const int rbi = GLU ? 0 : q / NCV, c = q - rbi * NCV;
        const uint32_t g0 = (uint32_t)__builtin_amdgcn_readfirstlane(c * MF_CG);
        const uint32_t dr = (uint32_t)(rbi * RPB);
        pka = sw_ld8(rq, vq + dr * rbytes, g0 * 16);
        // ((g0 + ga) * 32) >> gsh splits: g0 * 32 is a multiple of 128, ga * 32 < 128
        if (sst && W.gs > 0) psa = sw_ld4f(rs, vs + dr * (uint32_t)ng * 4, ((g0 * SW_RG) >> A.gsh) * 4);
        if (dact)
#pragma unroll
            for (int v = 0; v < DG_PER; v++) pkb[v] = sw_ld16(rd, vd + (uint32_t)v * 2 * MF_DW * 4, g0 * MF_DW * 4);
        if (xst) pxf = sw_ld4f(rx, vx, g0 * 4);
    };
    auto stage_store = [&](int buf) {
        sw_i32x4 *Al = (sw_i32x4 *)(mf_lds + MF_A_OFF + buf * MF_A_SZ);
        sw_u32x4 *Bl = (sw_u32x4 *)(mf_lds + MF_B_OFF + buf * MF_B_SZ);
        {
            const int m = ra >> 4, i = ra & 15;
            Al[((ga * 8 + m) * 4 + 2 * hq) * 16 + i] = mf_expand(pka.x);
            Al[((ga * 8 + m) * 4 + 2 * hq + 1) * 16 + i] = mf_expand(pka.y);
            if (sst) ((float *)(mf_lds + MF_S_OFF + buf * MF_S_SZ))[ga * MF_ROWS + ra] = psa;
        }
        if (dact)
#pragma unroll
            for (int v = 0; v < DG_PER; v++) Bl[v * MF_NT + st] = pkb[v];
        if (xst) ((float *)(mf_lds + MF_X_OFF + buf * MF_X_SZ))[gx * MF_TT + tx] = pxf;
    };

    // ---- the compute waves' (row tile, token tile) pairs: two per wave (row tiles m, m + 4
    // of token tile w >> 2) when 3-4 token tiles compute, else one (row tile w & 7 of token
    // tile w >> 3), so that a tail tile's pairs still spread over all four SIMDs, two or
    // four waves on each
    constexpr int NQ = CH / MF_CG;                         // chunks per run
    const int NR = NCV / NQ;                               // runs
    // the terms of one chunk's 4 groups summed as ((p0 + p1) + (p2 + p3)) per (row, token)
    // into q (REAL = 0: the +0 terms of a run's padding, whose sum is +0)
    auto quad = [&](auto NPC, auto RC, int buf, int tt, int m0, sw_f32x4 (&q)[2]) {
        constexpr int NP = decltype(NPC)::v;
        if constexpr (!decltype(RC)::v) {
#pragma unroll
            for (int mi = 0; mi < NP; mi++) q[mi] = sw_f32x4{0.f, 0.f, 0.f, 0.f};
            return;
        } else {
            // this lane's operands of group g: one base per operand plus immediate offsets
            const uint8_t *pa = mf_lds + MF_A_OFF + buf * MF_A_SZ + ((m0 * 4 + kq) * 16 + col) * 16;
            const uint8_t *pb = mf_lds + MF_B_OFF + buf * MF_B_SZ + (tt * 2 * 64 + lane) * 16;
            const uint8_t *ps = mf_lds + MF_S_OFF + buf * MF_S_SZ + (16 * m0 + 4 * kq) * 4;
            const uint8_t *px = mf_lds + MF_X_OFF + buf * MF_X_SZ + (16 * tt + col) * 4;
            sw_f32x4 h[NP];                                // the pending pair (p0 + p1)
            // a lane's four rows 4 kq + j take their scales from the four lanes of its quad
            // (lane col & 3 reads row 4 kq + (col & 3)), moved by DPP into the products: a
            // quarter of the LDS reads of one 16-byte read per lane
            struct Frag {
                sw_half8 a[NP], b0, b1;
                float s1[NP];
                float xf;
            };
            auto fetch = [&](Frag &F, int g) {
#pragma unroll
                for (int mi = 0; mi < NP; mi++) {
                    F.a[mi] = *(const sw_half8 *)(pa + (g * 8 + 4 * mi) * 4 * 16 * 16);
                    F.s1[mi] = *(const float *)(ps + (g * MF_ROWS + 64 * mi + (col & 3)) * 4);
                }
                F.b0 = *(const sw_half8 *)(pb + (g * 4 * 2 + 0) * 64 * 16);
                F.b1 = *(const sw_half8 *)(pb + (g * 4 * 2 + 1) * 64 * 16);
                F.xf = *(const float *)(px + g * MF_TT * 4);
            };
            Frag Fr[2];
            if (MF_PF) fetch(Fr[0], 0);
#pragma unroll
            for (int g = 0; g < MF_CG; g++) {
                if (!MF_PF) fetch(Fr[g & 1], g);
                const Frag &C = Fr[g & 1];
                const sw_f32x4 z = {0.f, 0.f, 0.f, 0.f};
                sw_f32x4 R0[NP], R1[NP];
                // the MFMAs issue at raised wave priority: the SIMD's waves, which leave each
                // chunk's barrier together, then spread out instead of waiting on their
                // products in step
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int mi = 0; mi < NP; mi++) {
                    R0[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(C.a[mi], C.b0, z, 0, 0, 0);
                    R1[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(C.a[mi], C.b1, z, 0, 0, 0);
                }
                __builtin_amdgcn_s_setprio(0);
                // (MF_PF: the next group's operands load while these products finish)
                if (MF_PF && g + 1 < MF_CG) fetch(Fr[(g + 1) & 1], g + 1);
#pragma unroll
                for (int mi = 0; mi < NP; mi++) {
                    // s * 2^(e - 21) of rows 4 kq + j (the DPP moves fold into the products)
                    const float t4[4] = {mf_quad_bcast<0>(C.s1[mi]) * C.xf, mf_quad_bcast<1>(C.s1[mi]) * C.xf,
                                         mf_quad_bcast<2>(C.s1[mi]) * C.xf, mf_quad_bcast<3>(C.s1[mi]) * C.xf};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        // (float)acc exactly, times (s * 2^(e - 21)), as dot8's term
                        const float p = __builtin_fmaf(R1[mi][j], 4096.0f, R0[mi][j]) * t4[j];
                        if (g == 0 || g == 2) h[mi][j] = p;
                        else if (g == 1) q[mi][j] = h[mi][j] + p;
                        else q[mi][j] = q[mi][j] + (h[mi][j] + p);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);         // one group's operands in flight at a time
            }
        }
    };
    // a row block's sums out: gate_up, h = silu(gate) * up to its digits (two limb
    // groups of the down's input per token); down, the rows of each token
    auto epilogue = [&](auto NPC, int rb, const sw_f32x4 (&y)[2], int tt, int m0, bool wact) {
        constexpr int NP = decltype(NPC)::v;
        const int ib = rb * 64, rr0 = rb * MF_ROWS;
        if constexpr (GLU) {
            const int I = A.I;
            float *el = (float *)(mf_lds + MF_EP_OFF);
            auto gsc = [&](int i) -> float { return PT ? A.tab[e].gs[ib + i] : W.s[(int64_t)e * (2 * I) + ib + i]; };
            auto usc = [&](int i) -> float { return PT ? A.tab[e].us[ib + i] : W.s[(int64_t)e * (2 * I) + I + ib + i]; };
            if constexpr (NP == 2) {
                // a lane holds the gate (row tile m0) and up (m0 + 4) sums of outputs 16 m0 + 4 kq + j
                if (wact)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int i = 16 * m0 + 4 * kq + j, t = 16 * tt + col;
                        float yg = y[0][j], yu = y[1][j];
                        if (W.gs <= 0) {                        // per-row scales after the sum
                            yg = yg * gsc(i);
                            yu = yu * usc(i);
                        }
                        el[t * MF_HLD + i] = (yg / (1.0f + expf(-yg))) * yu;
                    }
            } else {
                // (one row tile per wave: the gate and up sums of at most 32 tokens as they are)
                if (wact)
#pragma unroll
                    for (int j = 0; j < 4; j++) el[(16 * tt + col) * MF_YLD + 16 * m0 + 4 * kq + j] = y[0][j];
            }
            __syncthreads();
            // the row block's 64 outputs are two limb groups of the down projection's input
            const int GI = I / SW_RG, hw = tid >> 5, i = tid & 31;
            for (int job = hw; job < 2 * nt; job += MF_NT / 32) {
                const int t = job >> 1, q = job & 1;
                const int64_t prow = beg + t0 + t;
                const int gi = 2 * rb + q;
                float h;
                if constexpr (NP == 2) {
                    h = el[t * MF_HLD + 32 * q + i];
                } else {
                    const int o = 32 * q + i;
                    float yg = el[t * MF_YLD + o], yu = el[t * MF_YLD + 64 + o];
                    if (W.gs <= 0) {
                        yg = yg * gsc(o);
                        yu = yu * usc(o);
                    }
                    h = (yg / (1.0f + expf(-yg))) * yu;
                }
                digits_group(h, i, A.hdg + (prow * GI + gi) * MF_DW, A.hxs + prow * GI + gi);
            }
        } else {
            // a lane holds rows 16 m + 4 kq .. + 3 of token 16 tt + col: one 16-byte store each
            const int t = 16 * tt + col;
            if (wact && t < nt) {
                float *yrow = A.Y + (int64_t)(beg + t0 + t) * O;
#pragma unroll
                for (int mi = 0; mi < NP; mi++) {
                    const int row = rr0 + 16 * (m0 + 4 * mi) + 4 * kq;
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
    };
    // the main loop for NP pairs per wave: for each of the block's row blocks, runs of NQ
    // chunks, each run's quads summed ((q0 + q1) + (q2 + q3)) (NQ = 4), the runs added
    // left to right into y; then the row block's epilogue.  The staging runs over the
    // block's chunks q = rbi NCV + c without a break between row blocks.
    const int QT = rbper * NCV;
    auto real = [&](int q) { return GLU ? q < NC : q - q / NCV * NCV < NC; };
    auto main_loop = [&](auto NPC) {
        constexpr int NP = decltype(NPC)::v;
        const int tt = NP == 2 ? wave >> 2 : wave >> 3, m0 = NP == 2 ? wave & 3 : wave & 7;
        const bool wact = tt < nact;                       // uniform over the wave
        for (int rbi = 0; rbi < rbper; rbi++) {
            sw_f32x4 y[2];
            for (int r = 0; r < NR; r++) {
                sw_f32x4 ra[NP], rb[NP], q[2];
#pragma unroll
                for (int Q = 0; Q < NQ; Q++) {
                    const int c = r * NQ + Q, qg = rbi * NCV + c;
                    const int buf = NQ > 1 ? (Q & 1) : (qg & 1);   // (NCV is even when NQ > 1)
                    if (wact) {
                        // (a run-time test also for FULL: as a branch it keeps the compiler from
                        // interleaving the unrolled chunks, which spills at 128 registers)
                        if (c < NC) quad(NPC, MfIc<1>{}, buf, tt, m0, q);
                        else quad(NPC, MfIc<0>{}, buf, tt, m0, q);
#pragma unroll
                        for (int mi = 0; mi < NP; mi++) {
                            if (Q == 0) ra[mi] = q[mi];
                            else if (Q == 1 && NQ == 4) ra[mi] = ra[mi] + q[mi];
                            else if (Q == 2) rb[mi] = q[mi];
                            else if (Q == 3) ra[mi] = ra[mi] + (rb[mi] + q[mi]);
                            else ra[mi] = ra[mi] + q[mi];  // Q == 1 of NQ == 2
                        }
                    }
                    if (qg + 1 < QT && real(qg + 1)) stage_store((qg + 1) & 1);  // read by no wave since the last barrier
                    if (qg + 2 < QT && real(qg + 2)) stage_load(qg + 2);         // registers only: issued before the barrier's wait
                    __syncthreads();
                }
                if (wact)
#pragma unroll
                    for (int mi = 0; mi < NP; mi++) y[mi] = r == 0 ? ra[mi] : y[mi] + ra[mi];
            }
            epilogue(NPC, rbf + rbi, y, tt, m0, wact);
        }
    };

    stage_load(0);
    stage_store(0);
    if (QT > 1 && real(1)) stage_load(1);
    __syncthreads();
    if (nact > 2) main_loop(MfIc<2>{});
    else main_loop(MfIc<1>{});
}

// ------------------------------------------------------------ launch ----
static size_t mf_lds_bytes() { return (size_t)MF_EP_OFF + MF_EP_SZ; }
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
// row blocks per block: the down's 8-chunk row blocks four at a time (as nrb allows;
// C4 down 1064 -> 968 us); the gate_up's 32-chunk ones one at a time (two measured
// 1897 -> 1954 us: half the blocks balance worse over the CUs, and a start costs little
// against 32 chunks)
#ifndef MF_RBPER_ROWS
#define MF_RBPER_ROWS 4
#endif
static int mf_rbper(int nrb, int glu) {
    if (glu) return 1;
    for (int r = MF_RBPER_ROWS; r > 1; r >>= 1)
        if (nrb % r == 0) return r;
    return 1;
}
// shapes: K a multiple of 128 (whole chunks of 4 input groups), tiles listed (items, P),
// the digits addressed by 32-bit offsets
static int mf_check(const SwQ4 &W, const SwGroups &g, int &gsh, int dg_rows) {
    if (W.K % (SW_RG * MF_CG) || !g.items || !g.P || g.ngroups_max <= 0 || !sw_q4_extent_ok(W)) return -1;
    if (dg_rows <= 0 || (uint64_t)dg_rows * (uint64_t)W.K * 4 > 0xFFFFFFFFull) return -1;
    return sw_q4_gsh(W, gsh);
}

int sw_launch_mf_glu(hipStream_t st, SwQ4 W, const uint32_t *dg, const float *xs, int dg_rows, SwGroups g, int I,
                     uint32_t *hdg, float *hxs) {
    int gsh;
    if (mf_check(W, g, gsh, dg_rows) || I % 64 || W.O != 2 * I) return -1;
    const int nrb = I / 64;
    const int rp = mf_rbper(nrb, 1);
    const MfArgs A = {W, gsh, dg, xs, dg_rows, g, I, nrb, rp, hdg, hxs, nullptr};
    return mf_dispatch<1>(st, (unsigned)(g.ngroups_max * (nrb / rp)), A);
}

int sw_launch_mf_rows(hipStream_t st, SwQ4 W, const uint32_t *dg, const float *xs, int dg_rows, SwGroups g, float *Y) {
    int gsh;
    if (mf_check(W, g, gsh, dg_rows) || W.O % 4) return -1;
    const int nrb = (W.O + MF_ROWS - 1) / MF_ROWS;
    const int rp = mf_rbper(nrb, 0);
    const MfArgs A = {W, gsh, dg, xs, dg_rows, g, 0, nrb, rp, nullptr, nullptr, Y};
    return mf_dispatch<0>(st, (unsigned)(g.ngroups_max * (nrb / rp)), A);
}

// the same two GEMMs over per-group tensors: group c's gate/up/down are tab[gexp[c]]
// (W gives O, K and gs; each tensor holds one expert)
int sw_launch_mf_glu_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const uint32_t *dg, const float *xs, int dg_rows,
                         SwGroups g, int I, uint32_t *hdg, float *hxs) {
    int gsh;
    W.E = 1;
    if (!tab || !hdg || !hxs || mf_check(W, g, gsh, dg_rows) || I % 64 || W.O != 2 * I) return -1;
    const int nrb = I / 64;
    const int rp = mf_rbper(nrb, 1);
    const MfArgs A = {W, gsh, dg, xs, dg_rows, g, I, nrb, rp, hdg, hxs, nullptr, tab};
    return mf_dispatch<1, 1>(st, (unsigned)(g.ngroups_max * (nrb / rp)), A);
}
int sw_launch_mf_rows_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const uint32_t *dg, const float *xs, int dg_rows,
                          SwGroups g, float *Y) {
    int gsh;
    W.E = 1;
    if (!tab || !Y || mf_check(W, g, gsh, dg_rows) || W.O % 4) return -1;
    const int nrb = (W.O + MF_ROWS - 1) / MF_ROWS;
    const int rp = mf_rbper(nrb, 0);
    const MfArgs A = {W, gsh, dg, xs, dg_rows, g, 0, nrb, rp, nullptr, nullptr, Y, tab};
    return mf_dispatch<0, 1>(st, (unsigned)(g.ngroups_max * (nrb / rp)), A);
}
