// k_dot8.hip -- the int4 expert GEMV of decode on the gfx950 integer dot unit.
//
// v_dot8_i32_i4 multiplies eight signed 4-bit pairs and adds them to an int32
// in one VALU op.  A weight dword holds eight nibbles n (k = 8j + i at bits
// 4i, the container layout of c/moe_quant.h), and n ^ 8 read as a signed
// nibble is exactly n - 8, the weight's integer value: one XOR per eight
// weights is the whole dequant.  The activation side is an integer per input:
// for each group of 32 consecutive inputs, with 2^e the smallest power of two
// above max|x| of the group, y = x * 2^-e in (-1, 1) is written as
// sum_{l=1..ND} d_l 8^-l with signed digits d_l in [-8, 7] (round to nearest,
// clamp, carry the exact remainder), so
//     x ~= 2^(e - 3 ND) * D,   D = sum_l d_l 8^(ND - l)   (|error| <= 2^e 8^-ND).
// With ND = 7, |D| <= 8 (8^7 - 1) / 7 < 2^21.2 and the input error is at most
// 2^e 8^-7 (~2.4e-7 of the group's largest input, a few f32 ulps).  D is stored
// as NL = 6 "limbs", its digits in balanced base 16 (each in [-8, 7], a signed
// nibble like the weights).  For one weight row and one group, sum_k (n_k - 8) D_k
// is an exact int32 (Horner over the limbs: acc = (acc << 4) + four dot8;
// |acc| <= 32 * 8 * 2^21.2 < 2^29.2), turned into f32 once (correctly rounded, the
// same in every launch) and multiplied by s_row,group * 2^(e - 3 ND) (exact
// power-of-two scaling of the weight scale).  A row's output is then the sum
// of its group terms in the fixed order of run_sum (sw_gate.h): runs of up to
// 16 groups, each summed by a butterfly across the lanes holding them, the
// run sums left to right.  Nothing of it depends on which tokens share a
// launch, so grouped and per-token results are bit-identical.
//
// Per weight dword this is one XOR and NL dot8 (plus NL - 1 shift-adds and one
// fma per 32 weights), and each wave load is 1 KB of one row, contiguous.
#include "sw_hip.h"
#include "sw_libm.h"
#include "sw_gate.h"
#include "sw_router.h"
#include "sw_shared.h"

#define RG SW_RG              // inputs per limb group
#define CHG 16                // groups per run of the fixed row-sum order

// ------------------------------------------------------------ limbs ----
// rows x[r, K] f32 -> limbs (limbs_group in sw_gate.h), half a wave per group
__global__ __launch_bounds__(256) void k_limbs(const float *__restrict__ x, int K, int rows, sw_u32x4 *__restrict__ xl,
                                               float *__restrict__ xs) {
    const int G = K / RG;
    const int tid = threadIdx.x, g = blockIdx.x * 8 + (tid >> 5), r = blockIdx.y;
    if (r >= rows || g >= G) return;                 // whole half-waves leave together
    limbs_group(x[(int64_t)r * K + g * RG + (tid & 31)], tid & 31, xl + ((int64_t)r * G + g) * SW_NL, xs + (int64_t)r * G + g);
}

int sw_launch_limbs(hipStream_t st, const float *x, int rows, int K, sw_u32x4 *xl, float *xs) {
    if (K % RG || rows <= 0) return -1;
    const int G = K / RG;
    SW_LAUNCH(k_limbs, dim3((unsigned)((G + 7) / 8), (unsigned)rows), dim3(256), 0, st, x, K, rows, xl, xs);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// exact int32 sum_k (n_k - 8) D_k over one group: a = the group's 16 weight
// bytes with every nibble XOR 8 (signed nibbles n - 8).  Horner over the base-16
// limbs folded into dot8 chains -- acc = (acc << 4), then limb l's four dot8
// accumulate into it -- as two independent chains (limbs 0..2 and 3..5) joined
// at the end: acc = (hi << 12) + lo.  Every partial sum is an exact Horner
// prefix: |hi| <= 32 * 8 * 576, |hi << 12| < 2^29.2 + 32 * 8 * 2184 < 2^31.
__device__ __forceinline__ int dot8_chain(sw_u32x4 a, const sw_u32x4 *X, int l0, int l1) {
    int acc = __builtin_amdgcn_sdot8((int)a.x, (int)X[l0].x, 0, false);
    acc = __builtin_amdgcn_sdot8((int)a.y, (int)X[l0].y, acc, false);
    acc = __builtin_amdgcn_sdot8((int)a.z, (int)X[l0].z, acc, false);
    acc = __builtin_amdgcn_sdot8((int)a.w, (int)X[l0].w, acc, false);
#pragma unroll
    for (int l = l0 + 1; l < l1; l++) {
        acc = __builtin_amdgcn_sdot8((int)a.x, (int)X[l].x, acc << 4, false);
        acc = __builtin_amdgcn_sdot8((int)a.y, (int)X[l].y, acc, false);
        acc = __builtin_amdgcn_sdot8((int)a.z, (int)X[l].z, acc, false);
        acc = __builtin_amdgcn_sdot8((int)a.w, (int)X[l].w, acc, false);
    }
    return acc;
}
#define DOT8_SPLIT 3          // limbs of the high chain
__device__ __forceinline__ int dot8_group(sw_u32x4 a, const sw_u32x4 *X) {
    const int hi = dot8_chain(a, X, 0, DOT8_SPLIT), lo = dot8_chain(a, X, DOT8_SPLIT, SW_NL);
    return (hi << (4 * (SW_NL - DOT8_SPLIT))) + lo;
}

// A row's terms: one per group of 32 inputs, the lanes of a row padded to
// Gq = run_lanes(G).  C16 = 1 when G is a multiple of 16 (runs of 16 lanes,
// no padding), else runs of Gq lanes and padding lanes adding zero terms.
template <int C16>
__device__ __forceinline__ float row_term(float p, bool gv, int CH) {
    if constexpr (C16) return run_sum16(p);
    return run_sum(gv ? p : 0.f, CH);
}

// row slots of a block of nt threads: the largest power of two with rps * Gq <= nt, at most cap
__host__ __device__ inline int dg_rps(int Gq, int cap, int nt) {
    int r = 1;
    while (r * 2 * Gq <= nt && r < cap) r *= 2;
    return r;
}


// ------------------------------------------------------------ gate_up ----
// One block = RO (32; 128 or 64 for batches) consecutive intermediate outputs i
// of one group: gate rows i0..i0+RO-1 and up rows i0..i0+RO-1, every input
// group, for a tile of up to TT tokens of the group per pass over the block's
// weights (a group with more tokens takes further passes, which re-read the
// block's weights from L2).  Thread (row slot ro, input group g): Gq threads
// per row, RPS row slots; slot ro takes NSH = RO/RPS consecutive gate rows
// and the same up rows, one row per step (steps 0..NSH-1 gate, NSH..2NSH-1
// up), so its addresses are a fixed lane offset plus a per-step scalar one.
// The tile's limbs of its group stay in registers; PF steps of weight loads
// are in flight; a row's run sums go to LDS and the row sums, the SiLU-GLU
// and the limbs of h (the down projection's input) follow.
#define DG_TT SW_DG_TT        // tokens per weight pass in the grouped kernels
#define DG_NT 512             // threads per gate_up block
// One token (PICK = 1): block (rank a, set of outputs) takes pick a and
// writes h of packed row a.  With NP = 0 the picks come in sel (from the
// routing stage); with NP > 0 every block runs the token's gate + top-k on
// its first wave (gate_topk_wave: deterministic, so every block gets the
// same picks) while the others fetch the limbs, and block (0, 0) writes the
// picks and weights to sel / w for the down projection.
struct DotRoute {
    const float *src;          // the token's logits (act 1) or sigmoid/softplus scores
    const float *bias;         // selection bias (e_score_correction_bias) or null
    int E, K, act, use_bias, norm;
    float *w;
};
struct Dot8GluArgs {
    SwQ4 W;
    int gsh;
    const sw_u32x4 *xl;
    const float *xs;
    SwGroups grp;
    int I;
    sw_u32x4 *hl;
    float *hs;
    int *sel;
    DotRoute rt;
    const SwTab *tab;          // per-group tensors (the _tab launch) or null
};

// K inputs as G = K/32 groups, G <= 256
static bool dot8_shape_ok(int K) { return K > 0 && K % RG == 0 && K / RG <= 256; }
static int dot8_nc(int K) { const int G = K / RG; return G < CHG ? 1 : run_lanes(G) / CHG; }
static int dot8_c16(int K) { return (K / RG) % CHG == 0; }
// steps of weight loads in flight: min(8, steps per half) (a power of two dividing it)
static int dg_pf_glu(int K) { const int n = 32 / dg_rps(run_lanes(K / RG), 32, DG_NT); return n < 8 ? n : 8; }
static int dg_pf_rows(int K) { const int n = 64 / dg_rps(run_lanes(K / RG), 64, 256); return n < 8 ? n : 8; }

// block (bx = group or rank, by = set of RO outputs: 32, or up to 128 for groups --
// fewer, longer blocks per weight byte); runs: the dynamic LDS, [TT][2 RO][NC] floats;
// NTL: a block whose pass is its group's only one loads its weights non-temporal
template <int PF, int PICK, int NP, int TT, int C16, int RO, int PT = 0, int NTL = 1>
__device__ __forceinline__ void dot8_glu_block(const Dot8GluArgs &A, int bx, int by, float *runs) {
    static_assert(PT == 0 || PICK == 0, "per-group tensors come with groups");
    static_assert(PICK == 0 || TT == 1, "picks are of one token");
    static_assert(RO == 32 || RO == 64 || RO == 128, "1, 2 or 4 limb groups of h per block");
    const SwQ4 W = A.W;
    const int I = A.I;
    const sw_u32x4 *__restrict__ xl = A.xl;
    const float *__restrict__ xs = A.xs;
    const SwGroups grp = A.grp;
    const int K = W.K, G = K / RG, Gq = C16 ? G : run_lanes(G);
    const int CH = C16 ? CHG : (Gq < CHG ? Gq : CHG), NC = Gq / CH;
    const int RPS = dg_rps(Gq, RO, DG_NT), NSH = RO / RPS;    // a row slot: NSH gate rows and NSH up rows
    const int tid = threadIdx.x, ro = tid / Gq, gq = tid - ro * Gq, c = gq / CH;
    const bool worker = ro < RPS, lead = worker && (gq & (CH - 1)) == 0, gv = C16 || gq < G;
    const int g = gv ? gq : G - 1;                   // padding lanes load group G-1 and add 0
    const int roc = worker ? ro : 0;
    const int i0 = by * RO;
    const int ng = W.gs > 0 ? K / W.gs : 1;
    const int sg = W.gs > 0 ? (g * RG) >> A.gsh : 0;
    const uint32_t rb = (uint32_t)K / 2, sb = (uint32_t)ng * 4;
    int e, beg, tb, tend, gcnt = 0;
    sw_u32x4 X[TT][SW_NL];
    float xf[TT];
    if constexpr (PICK) {                             // one token: rank bx of its picks
        beg = bx; tb = 0; tend = 1;
#pragma unroll
        for (int l = 0; l < SW_NL; l++) X[0][l] = xl[(int64_t)g * SW_NL + l];
        xf[0] = xs[g];
        if constexpr (NP > 0) {                       // the token's routing by wave 0 of the block
            __shared__ int tk_sk[64];
            __shared__ float tk_wk[64];
            __shared__ uint64_t tk_tab[32];
            const DotRoute rt = A.rt;
            // a block needs its own pick only (passes 0 .. bx); the block of the last rank
            // and the first outputs runs all K passes and writes the picks and weights
            const bool writer = bx == rt.K - 1 && by == 0;
            if (tid < 64) {
                int sk;
                float wk;
                gate_topk_wave<NP>(rt.src, rt.E, rt.K, rt.act, rt.bias, rt.use_bias, rt.norm, tk_tab, sk, wk, 0, 1.f,
                                   nullptr, writer ? 0 : bx + 1);
                if (tid < rt.K) { tk_sk[tid] = sk; tk_wk[tid] = wk; }
            }
            __syncthreads();
            e = __builtin_amdgcn_readfirstlane(tk_sk[bx]);
            if (writer && tid < rt.K) { A.sel[tid] = tk_sk[tid]; rt.w[tid] = tk_wk[tid]; }
        } else {
            e = A.sel[bx];
        }
    } else {
        if (!grp_work(grp, bx, TT, e, beg, tb, tend, &gcnt)) return;
    }
    const bool once = PICK || (tb == 0 && gcnt <= TT);
    // gate rows through (rq, rs), up rows through (rq2, rs2): one [E*2I] tensor, or the
    // group's own gate and up tensors (PT)
    sw_rsrc rq, rs, rq2, rs2;
    uint32_t erow;
    if constexpr (PT) {
        const SwTab tb_ = A.tab[e];
        rq = sw_make_rsrc(tb_.g, (uint32_t)I * rb);
        rq2 = sw_make_rsrc(tb_.u, (uint32_t)I * rb);
        rs = sw_make_rsrc(tb_.gs, (uint32_t)I * sb);
        rs2 = sw_make_rsrc(tb_.us, (uint32_t)I * sb);
        erow = (uint32_t)i0;
    } else {
        rq = rq2 = sw_q4_rq(W);
        rs = rs2 = sw_q4_rs(W);
        erow = (uint32_t)e * (uint32_t)(2 * I) + (uint32_t)i0;
    }
    // lane offsets (this thread's first row of a half) and the scalar offset of step s
    const uint32_t voq = (uint32_t)(roc * NSH) * rb + (uint32_t)g * 16;
    const uint32_t vos = (uint32_t)(roc * NSH) * sb + (uint32_t)sg * 4;
    auto srow = [&](int s) -> uint32_t { return s < NSH ? erow + s : erow + (PT ? 0 : I) + (s - NSH); };
    auto wq = [&](int s) -> const sw_rsrc & { return s < NSH ? rq : rq2; };
    auto ws = [&](int s) -> const sw_rsrc & { return s < NSH ? rs : rs2; };
    const int NS = 2 * NSH;
    float *myruns = runs + (roc * NSH) * NC + c;      // this lane's run sum of step s: myruns[(t*64 + h*32 + j) * NC]
    // weight loads non-temporal (the nt policy) when this pass is the only one over the
    // block's weights; cached when other passes re-read them
    auto passes = [&](auto PC) {
        constexpr int POL = decltype(PC)::v;
        for (int t0 = tb; t0 < tend; t0 += TT) {
            const int nt = min(TT, tend - t0);
            if constexpr (PICK == 0) {
    #pragma unroll
                for (int t = 0; t < TT; t++) {
                    const int pr = beg + t0 + (t < nt ? t : 0);
                    const int64_t tok = grp.grow ? grp.grow[pr] : pr;
    #pragma unroll
                    for (int l = 0; l < SW_NL; l++) X[t][l] = xl[(tok * G + g) * SW_NL + l];
                    xf[t] = xs[tok * G + g];
                }
            }
            sw_u32x4 ra[PF];
            float sa[PF];
    #pragma unroll
            for (int u = 0; u < PF; u++) {
                ra[u] = sw_ld16<POL>(wq(u), voq, srow(u) * rb);
                sa[u] = sw_ld4f<POL>(ws(u), vos, srow(u) * sb);
            }
            auto step = [&](int s, int u, bool refill) {
                const sw_u32x4 w = ra[u] ^ 0x88888888u;
                const float sc = W.gs > 0 ? sa[u] : 1.0f;
                if (refill) {
                    ra[u] = sw_ld16<POL>(wq(s + PF), voq, srow(s + PF) * rb);
                    sa[u] = sw_ld4f<POL>(ws(s + PF), vos, srow(s + PF) * sb);
                    __builtin_amdgcn_sched_barrier(0);
                }
                const int urow = s < NSH ? s : RO + s - NSH;                 // local row minus roc * NSH
    #pragma unroll
                for (int t = 0; t < TT; t++) {
                    if (t < nt) {                          // uniform over the block
                        const float p = row_term<C16>((float)dot8_group(w, X[t]) * (sc * xf[t]), gv, CH);
                        if (lead) myruns[(t * 2 * RO + urow) * NC] = p;
                    }
                }
            };
            int s0 = 0;
            for (; s0 + PF < NS; s0 += PF) {
    #pragma unroll
                for (int u = 0; u < PF; u++) step(s0 + u, u, true);
            }
    #pragma unroll
            for (int u = 0; u < PF; u++) step(s0 + u, u, false);
            __syncthreads();
            // token t of the tile by the threads RO t .. RO t + RO - 1 (a half-wave per limb group)
            const int t = tid / RO, i = tid - t * RO;
            if (t < nt) {
                const float *rg = runs + (t * 2 * RO + i) * NC, *ru = runs + (t * 2 * RO + RO + i) * NC;
                float yg = rg[0], yu = ru[0];
                for (int cc = 1; cc < NC; cc++) { yg = yg + rg[cc]; yu = yu + ru[cc]; }
                if (W.gs <= 0) {                            // per-row scales after the sum
                    if constexpr (PT) {
                        yg = yg * A.tab[e].gs[i0 + i];
                        yu = yu * A.tab[e].us[i0 + i];
                    } else {
                        yg = yg * W.s[(int64_t)e * (2 * I) + i0 + i];
                        yu = yu * W.s[(int64_t)e * (2 * I) + I + i0 + i];
                    }
                }
                const float h = (yg / (1.0f + expf(-yg))) * yu;
                // every 32 of the block's outputs are one limb group of the down projection's input
                const int GI = I / RG, gi_out = (i0 + i) / RG;
                const int64_t prow = beg + t0 + t;
                limbs_group(h, i & 31, A.hl + (prow * GI + gi_out) * SW_NL, A.hs + prow * GI + gi_out);
            }
            __syncthreads();
        }
    };
    if constexpr (NTL) {
        if (once) passes(SwIc<2>{});
        else passes(SwIc<0>{});
    } else {
        passes(SwIc<0>{});
    }
}

template <int PF, int PICK, int TT, int C16, int RO>
__global__ __launch_bounds__(DG_NT) void k_dot8_glu(Dot8GluArgs A) {
    extern __shared__ __align__(16) float red[];
    dot8_glu_block<PF, PICK, 0, TT, C16, RO>(A, blockIdx.x, blockIdx.y, red);
}

// dispatch on the prefetch depth pf (1, 2, 4 or 8) and C16
template <template <int, int> class L, class... Args>
static void dispatch_pf_c16(int pf, int c16, Args &&...args) {
    if (c16) {
        if (pf >= 8) L<8, 1>::go(args...);
        else if (pf >= 4) L<4, 1>::go(args...);
        else if (pf >= 2) L<2, 1>::go(args...);
        else L<1, 1>::go(args...);
    } else {
        if (pf >= 8) L<8, 0>::go(args...);
        else if (pf >= 4) L<4, 0>::go(args...);
        else if (pf >= 2) L<2, 0>::go(args...);
        else L<1, 0>::go(args...);
    }
}
template <int PICK, int TT, int RO>
struct GluL {
    template <int PF, int C16>
    struct L {
        static void go(dim3 grid, size_t lds, hipStream_t st, const Dot8GluArgs &A) {
            SW_LAUNCH((k_dot8_glu<PF, PICK, TT, C16, RO>), grid, dim3(DG_NT), lds, st, A);
        }
    };
};
// outputs per gate_up block of a batch: 128 or 64 when I allows (fewer blocks, so less
// per-block start and epilogue per weight byte: B=32 gate_up 215 -> 190 us), else 32
static int dg_ro(int I) { return I % 128 == 0 ? 128 : I % 64 == 0 ? 64 : 32; }
// outputs per block of a grouped gate_up launch of nbx passes: 128 when that gives at
// least 1024 blocks (two rounds of the 512 that are resident at once), else 64, so a
// short grid ends in a smaller tail (C5 at B = 8: 768 blocks of 128 outputs took 95.7 us,
// 1536 of 64 take 87.9; at B = 16, 1280 blocks of 128 run 130 us against 134 with 64)
static int dg_ro_grid(int I, int nbx) {
    const int ro = dg_ro(I);
    return ro == 128 && (int64_t)nbx * (I / 128) < 1024 ? 64 : ro;
}

static int dot8_glu_check(SwQ4 W, int I, int &gsh) {
    if (!dot8_shape_ok(W.K) || I % 32 || W.O != 2 * I || !sw_q4_extent_ok(W)) return -1;
    return sw_q4_gsh(W, gsh);
}
static size_t dot8_glu_lds(int K, int TT, int RO = 32) { return (size_t)TT * 2 * RO * dot8_nc(K) * 4; }

int sw_launch_q4_dot8_glu(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, int I,
                          sw_u32x4 *hl, float *hs) {
    int gsh;
    if (dot8_glu_check(W, I, gsh) || g.ngroups_max <= 0 || (g.items && g.tt && g.tt != DG_TT)) return -1;
    const Dot8GluArgs A = {W, gsh, xl, xs, g, I, hl, hs, nullptr, DotRoute{}};
    const int RO = dg_ro_grid(I, g.ngroups_max);
    const dim3 grid((unsigned)g.ngroups_max, (unsigned)(I / RO));
    if (RO == 128) dispatch_pf_c16<GluL<0, DG_TT, 128>::L>(dg_pf_glu(W.K), dot8_c16(W.K), grid, dot8_glu_lds(W.K, DG_TT, 128), st, A);
    else if (RO == 64) dispatch_pf_c16<GluL<0, DG_TT, 64>::L>(dg_pf_glu(W.K), dot8_c16(W.K), grid, dot8_glu_lds(W.K, DG_TT, 64), st, A);
    else dispatch_pf_c16<GluL<0, DG_TT, 32>::L>(dg_pf_glu(W.K), dot8_c16(W.K), grid, dot8_glu_lds(W.K, DG_TT, 32), st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_q4_dot8_glu_picks(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, int I, sw_u32x4 *hl, float *hs,
                                const int *sel, int K) {
    int gsh;
    if (dot8_glu_check(W, I, gsh) || K <= 0 || K > 64 || !sel) return -1;
    const Dot8GluArgs A = {W, gsh, xl, xs, SwGroups{}, I, hl, hs, const_cast<int *>(sel), DotRoute{}};
    dispatch_pf_c16<GluL<1, 1, 32>::L>(dg_pf_glu(W.K), dot8_c16(W.K), dim3((unsigned)K, (unsigned)(I / 32)), dot8_glu_lds(W.K, 1), st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------ rows ----
// Y[packed row, O] = W_e . x for every packed row of every group (the down
// projection of the grouped path): block = RB (128, or 64 when O is not a
// multiple of 128) consecutive output rows of one group, a tile of up to
// DG_TT tokens per weight pass; thread (row slot ro, input group g) takes
// NS = RB/RPS rows, one per step (the RPS slots a step's RPS consecutive rows);
// same fixed-order row sums, f32 rows out.  O a multiple of 64.
struct Dot8RowsArgs {
    SwQ4 W;
    int gsh;
    const sw_u32x4 *xl;
    const float *xs;
    SwGroups grp;
    float *Y;
    const SwTab *tab;          // per-group tensors (the _tab launch) or null
};
// (a block whose pass is its group's only one loads its weights non-temporal; not with
// the 8-deep ring, which spills with both load paths)
// NT: threads per block (192 for rows of 48 lanes: four row slots, no idle lanes)
template <int PF, int TT, int C16, int RB, int PT = 0, int NTL = (PF < 8), int NT = 256>
__device__ __forceinline__ void dot8_rows_block(const Dot8RowsArgs &A, int bx, int by, float *runs) {
    const SwQ4 W = A.W;
    const sw_u32x4 *__restrict__ xl = A.xl;
    const float *__restrict__ xs = A.xs;
    const SwGroups grp = A.grp;
    float *__restrict__ Y = A.Y;
    const int K = W.K, G = K / RG, O = W.O, Gq = C16 ? G : run_lanes(G);
    const int CH = C16 ? CHG : (Gq < CHG ? Gq : CHG), NC = Gq / CH;
    const int RPS = dg_rps(Gq, RB, NT), NS = RB / RPS;
    const int tid = threadIdx.x, ro = tid / Gq, gq = tid - ro * Gq, c = gq / CH;
    const bool worker = ro < RPS, lead = worker && (gq & (CH - 1)) == 0, gv = C16 || gq < G;
    const int g = gv ? gq : G - 1;
    const int roc = worker ? ro : 0;
    int e, beg, tb, tend, gcnt;
    if (!grp_work(grp, bx, TT, e, beg, tb, tend, &gcnt)) return;
    const int r0 = by * RB;
    const int nrows = min(RB, O - r0);
    const int ng = W.gs > 0 ? K / W.gs : 1;
    const int sg = W.gs > 0 ? (g * RG) >> A.gsh : 0;
    const uint32_t rb = (uint32_t)K / 2, sb = (uint32_t)ng * 4;
    sw_rsrc rq, rs;
    if constexpr (PT) {                                  // the group's own down tensor
        rq = sw_make_rsrc(A.tab[e].d, (uint32_t)O * rb);
        rs = sw_make_rsrc(A.tab[e].ds, (uint32_t)O * sb);
    } else {
        rq = sw_q4_rq(W);
        rs = sw_q4_rs(W);
    }
    // step s of row slot roc takes row s RPS + roc: the block's slots read RPS consecutive
    // rows a step, one contiguous stretch of the tensor (B=32's down 89.8 -> 85.7 us, C5's
    // 41.8 -> 40.0 us against NS consecutive rows per slot), the row slot's part in the vector
    // offset and the step's in the scalar one.  RB divides O (the launches check), so every
    // row a block reads is one of its group's: the range check leaves the scalar offset out
    const uint32_t erow = (PT ? 0u : (uint32_t)e * (uint32_t)O) + (uint32_t)r0;
    const uint32_t voq = ((uint32_t)roc) * rb + (uint32_t)g * 16;
    const uint32_t vos = ((uint32_t)roc) * sb + (uint32_t)sg * 4;
    float *myruns = runs + roc * NC + c;
    // weight loads non-temporal (the nt policy) when this pass is the only one over the
    // block's weights; cached when other passes re-read them
    auto passes = [&](auto PC) {
        constexpr int POL = decltype(PC)::v;
        for (int t0 = tb; t0 < tend; t0 += TT) {
            const int nt = min(TT, tend - t0);
            sw_u32x4 X[TT][SW_NL];
            float xf[TT];
    #pragma unroll
            for (int t = 0; t < TT; t++) {
                const int pr = beg + t0 + (t < nt ? t : 0);
                const int64_t tok = grp.grow ? grp.grow[pr] : pr;
    #pragma unroll
                for (int l = 0; l < SW_NL; l++) X[t][l] = xl[(tok * G + g) * SW_NL + l];
                xf[t] = xs[tok * G + g];
            }
            sw_u32x4 ra[PF];
            float sa[PF];
            // the next step's offsets, moved on by RPS rows a step
            uint32_t vqn = voq, vsn = vos;
            const uint32_t dq = (uint32_t)RPS * rb, ds = (uint32_t)RPS * sb;
    #pragma unroll
            for (int u = 0; u < PF; u++) {
                ra[u] = sw_ld16<POL>(rq, voq, (erow + u * RPS) * rb);
                sa[u] = sw_ld4f<POL>(rs, vos, (erow + u * RPS) * sb);
            }
            auto step = [&](int s, int u, bool refill) {
                const sw_u32x4 w = ra[u] ^ 0x88888888u;
                const float sc = W.gs > 0 ? sa[u] : 1.0f;
                if (refill) {
                    ra[u] = sw_ld16<POL>(rq, voq, (erow + (s + PF) * RPS) * rb);
                    sa[u] = sw_ld4f<POL>(rs, vos, (erow + (s + PF) * RPS) * sb);
                    __builtin_amdgcn_sched_barrier(0);
                }
    #pragma unroll
                for (int t = 0; t < TT; t++) {
                    if (t < nt) {                          // uniform over the block
                        const float p = row_term<C16>((float)dot8_group(w, X[t]) * (sc * xf[t]), gv, CH);
                        if (lead) myruns[(t * RB + s * RPS) * NC] = p;
                    }
                }
            };
            int s0 = 0;
            for (; s0 + PF < NS; s0 += PF) {
    #pragma unroll
                for (int u = 0; u < PF; u++) step(s0 + u, u, true);
            }
    #pragma unroll
            for (int u = 0; u < PF; u++) step(s0 + u, u, false);
            __syncthreads();
            for (int it = tid; it < TT * RB; it += NT) {
                const int t = it / RB, r = it - t * RB;
                if (t < nt && r < nrows) {
                    const float *rr = runs + it * NC;
                    float y = rr[0];
                    for (int cc = 1; cc < NC; cc++) y = y + rr[cc];
                    if (W.gs <= 0) y = y * (PT ? A.tab[e].ds[r0 + r] : W.s[(int64_t)e * O + r0 + r]);
                    Y[(int64_t)(beg + t0 + t) * O + r0 + r] = y;
                }
            }
            __syncthreads();
        }
    };
    if constexpr (NTL) {
        if (tb == 0 && gcnt <= TT) passes(SwIc<2>{});
        else passes(SwIc<0>{});
    } else {
        passes(SwIc<0>{});
    }
}

template <int PF, int TT, int C16, int RB, int NT>
__global__ __launch_bounds__(NT, 4) void k_dot8_rows(Dot8RowsArgs A) {
    extern __shared__ __align__(16) float red[];
    const int nb = (int)(gridDim.x * gridDim.y);
    const int w = A.grp.items ? sw_xcd_work((int)(blockIdx.x + gridDim.x * blockIdx.y), nb)
                              : (int)(blockIdx.x + gridDim.x * blockIdx.y);
    dot8_rows_block<PF, TT, C16, RB, 0, (PF < 8), NT>(A, w % (int)gridDim.x, w / (int)gridDim.x, red);
}
#define RW_PF 4
template <int RB, int NT, int TT>
struct RowsL {
    template <int PF, int C16>
    struct L {
        static void go(dim3 grid, size_t lds, hipStream_t st, const Dot8RowsArgs &A) {
            SW_LAUNCH((k_dot8_rows<PF, TT, C16, RB, NT>), grid, dim3(NT), lds, st, A);
        }
    };
};

int sw_launch_q4_dot8_rows(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, float *Y) {
    int gsh;
    if (!dot8_shape_ok(W.K) || g.ngroups_max <= 0 || W.O <= 0 || !sw_q4_extent_ok(W) || sw_q4_gsh(W, gsh)) return -1;
    // 128 rows per block when O allows (half the blocks: half the per-block start and
    // epilogue per weight byte), else 64
    const int RB = W.O % 128 == 0 ? 128 : 64;          // (256 rows measured no faster at B=32)
    if (W.O % RB) return -1;                           // (no block reads past its group's rows)
    const dim3 grid((unsigned)g.ngroups_max, (unsigned)((W.O + RB - 1) / RB));
    const Dot8RowsArgs A = {W, gsh, xl, xs, g, Y};
    // a ring of at most RW_PF steps: within 128 VGPRs, four blocks per CU
    const int pf = dg_pf_rows(W.K) < RW_PF ? dg_pf_rows(W.K) : RW_PF;
    const int tt = g.tt ? g.tt : DG_TT;                // tokens per pass of the items
    if (tt != 1 && tt != DG_TT) return -1;
    const size_t lds = (size_t)tt * RB * dot8_nc(W.K) * 4;
    // rows of 48 lanes (K = 1536, C5's down) in blocks of 192 threads: four row slots and
    // no idle lanes, five blocks per CU (256 threads left 64 idle in each block)
    const int G = W.K / RG, Gq = dot8_c16(W.K) ? G : run_lanes(G);
#define SW_RW(T_) \
    do { \
        if (Gq == 48 && RB == 128) dispatch_pf_c16<RowsL<128, 192, T_>::L>(pf, dot8_c16(W.K), grid, lds, st, A); \
        else if (Gq == 48) dispatch_pf_c16<RowsL<64, 192, T_>::L>(pf, dot8_c16(W.K), grid, lds, st, A); \
        else if (RB == 128) dispatch_pf_c16<RowsL<128, 256, T_>::L>(pf, dot8_c16(W.K), grid, lds, st, A); \
        else dispatch_pf_c16<RowsL<64, 256, T_>::L>(pf, dot8_c16(W.K), grid, lds, st, A); \
    } while (0)
    if (tt == 1) SW_RW(1);
    else SW_RW(DG_TT);
#undef SW_RW
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------ per-group tensors (coli table) ----
// The two grouped kernels with group c's gate/up/down read from tab[gexp[c]]: the
// same blocks, steps and fixed-order sums, so a group's outputs are bit-identical to
// the same expert's outputs from the one-tensor launches above.
template <int PF, int C16, int RO, int TT>
__global__ __launch_bounds__(DG_NT) void k_dot8_glu_tab(Dot8GluArgs A) {
    extern __shared__ __align__(16) float red[];
    dot8_glu_block<PF, 0, 0, TT, C16, RO, 1>(A, blockIdx.x, blockIdx.y, red);
}
template <int RO, int TT>
struct GluTabL {
    template <int PF, int C16>
    struct L {
        static void go(dim3 grid, size_t lds, hipStream_t st, const Dot8GluArgs &A) {
            SW_LAUNCH((k_dot8_glu_tab<PF, C16, RO, TT>), grid, dim3(DG_NT), lds, st, A);
        }
    };
};
// one_row: every group holds one row (decode), so a weight pass carries one token
int sw_launch_q4_dot8_glu_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const sw_u32x4 *xl, const float *xs, SwGroups g,
                              int I, sw_u32x4 *hl, float *hs, int one_row) {
    int gsh;
    W.E = 1;                                              // each tensor holds one expert
    if (!tab || dot8_glu_check(W, I, gsh) || g.ngroups_max <= 0 || g.items) return -1;
    const Dot8GluArgs A = {W, gsh, xl, xs, g, I, hl, hs, nullptr, DotRoute{}, tab};
    // a decode-sized call (few groups) takes 32-output blocks, so the grid still fills the chip
    const int RO = g.ngroups_max * (I / 128) < 512 ? 32 : dg_ro(I);
    const dim3 grid((unsigned)g.ngroups_max, (unsigned)(I / RO));
    const int pf = dg_pf_glu(W.K), c16 = dot8_c16(W.K);
    if (one_row && RO == 32) dispatch_pf_c16<GluTabL<32, 1>::L>(pf, c16, grid, dot8_glu_lds(W.K, 1, 32), st, A);
    else if (RO == 128) dispatch_pf_c16<GluTabL<128, DG_TT>::L>(pf, c16, grid, dot8_glu_lds(W.K, DG_TT, 128), st, A);
    else if (RO == 64) dispatch_pf_c16<GluTabL<64, DG_TT>::L>(pf, c16, grid, dot8_glu_lds(W.K, DG_TT, 64), st, A);
    else dispatch_pf_c16<GluTabL<32, DG_TT>::L>(pf, c16, grid, dot8_glu_lds(W.K, DG_TT, 32), st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int PF, int C16, int RB>
__global__ __launch_bounds__(256, 4) void k_dot8_rows_tab(Dot8RowsArgs A) {
    extern __shared__ __align__(16) float red[];
    dot8_rows_block<PF, DG_TT, C16, RB, 1>(A, blockIdx.x, blockIdx.y, red);
}
template <int RB>
struct RowsTabL {
    template <int PF, int C16>
    struct L {
        static void go(dim3 grid, size_t lds, hipStream_t st, const Dot8RowsArgs &A) {
            SW_LAUNCH((k_dot8_rows_tab<PF, C16, RB>), grid, dim3(256), lds, st, A);
        }
    };
};
int sw_launch_q4_dot8_rows_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const sw_u32x4 *xl, const float *xs, SwGroups g,
                               float *Y) {
    int gsh;
    W.E = 1;
    if (!tab || !dot8_shape_ok(W.K) || g.ngroups_max <= 0 || g.items || W.O <= 0 || !sw_q4_extent_ok(W) ||
        sw_q4_gsh(W, gsh))
        return -1;
    const int RB = W.O % 128 == 0 && g.ngroups_max * (W.O / 128) >= 512 ? 128 : 64;
    if (W.O % RB) return -1;                           // (no block reads past its group's rows)
    const dim3 grid((unsigned)g.ngroups_max, (unsigned)((W.O + RB - 1) / RB));
    const Dot8RowsArgs A = {W, gsh, xl, xs, g, Y, tab};
    const int pf = dg_pf_rows(W.K) < RW_PF ? dg_pf_rows(W.K) : RW_PF;
    const size_t lds = (size_t)DG_TT * RB * dot8_nc(W.K) * 4;
    if (RB == 128) dispatch_pf_c16<RowsTabL<128>::L>(pf, dot8_c16(W.K), grid, lds, st, A);
    else dispatch_pf_c16<RowsTabL<64>::L>(pf, dot8_c16(W.K), grid, lds, st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------- down + combine (one token) ----
// out[d] += (sum_a w[a] * y_a[d]) * route_scale (+ shared[d]) with
// y_a = down_{sel[a]}(h_a), for DC_RB output rows per block and every rank:
// thread (rank a, input group g) keeps h_a's limbs of its group in registers
// and streams the block's rows of expert sel[a]; each y_a[d] gets the
// fixed-order row sum of the grouped rows kernel (so it is bit-identical to
// that kernel's slot value) and the ranks are summed in order with one fma
// each, the operation sequence of k_combine.
#ifndef DC_RB
#define DC_RB 8            // 4 and 16 measured slower at B=1 (10.2 and 10.9 us against 9.8)
#endif
#define DC_KU 16           // ranks whose run sums are read ahead of the fma chain
#define DC_NCM 4           // run sums per row read ahead (I <= 2048 at runs of 16 groups)
struct Dot8DownArgs {
    SwQ4 W;
    int gsh;
    const sw_u32x4 *hl;
    const float *hs;
    const int *sel;
    const float *wts;
    int K;
    float route_scale;
    const float *shared;
    float *out;
    const float *wsh;          // Inkling's gated shared experts: shared [ns][D] weighted by wsh[ns], or null
    int ns;
};
// block bx of DC_RB output rows; runs: [K][DC_RB][NC] floats
template <int C16>
__device__ __forceinline__ void dot8_down_combine_block(const Dot8DownArgs &A, int bx, float *runs) {
    const SwQ4 W = A.W;
    const int K = A.K;
    const sw_u32x4 *__restrict__ hl = A.hl;
    const float *__restrict__ hs = A.hs;
    const int *__restrict__ sel = A.sel;
    const float *__restrict__ wts = A.wts;
    const float route_scale = A.route_scale;
    const float *__restrict__ shared = A.shared;
    float *__restrict__ out = A.out;
    __shared__ float wk[64];
    const int I = W.K, G = I / RG, D = W.O, Gq = C16 ? G : run_lanes(G);
    const int CH = C16 ? CHG : (Gq < CHG ? Gq : CHG), NC = Gq / CH;
    const int tid = threadIdx.x, a = tid / Gq, gq = tid - a * Gq, c = gq / CH;
    const bool worker = a < K, lead = worker && (gq & (CH - 1)) == 0, gv = C16 || gq < G;
    const int g = gv ? gq : G - 1;
    const int ac = worker ? a : 0;
    const int d0 = bx * DC_RB;
    const int ng = W.gs > 0 ? I / W.gs : 1;
    const int sg = W.gs > 0 ? (g * RG) >> A.gsh : 0;
    const uint32_t rb = (uint32_t)I / 2, sb = (uint32_t)ng * 4;
    if (tid < K) wk[tid] = wts[tid];
    float sh_d = 0.f, out_d = 0.f;
    if (tid < DC_RB) {
        out_d = out[d0 + tid];
        if (shared && !A.wsh) sh_d = shared[d0 + tid];
    }
    sw_u32x4 X[SW_NL];
#pragma unroll
    for (int l = 0; l < SW_NL; l++) X[l] = hl[((int64_t)ac * G + g) * SW_NL + l];
    const float xf = hs[(int64_t)ac * G + g];
    const uint32_t e = (uint32_t)sel[ac];
    const sw_rsrc rq = sw_q4_rq(W), rs = sw_q4_rs(W);
    const uint32_t voq = (e * (uint32_t)D + (uint32_t)d0) * rb + (uint32_t)g * 16;
    const uint32_t vos = (e * (uint32_t)D + (uint32_t)d0) * sb + (uint32_t)sg * 4;
    sw_u32x4 ra[DC_RB];
    float sa[DC_RB];
#pragma unroll
    for (int r = 0; r < DC_RB; r++) {                // every row of the block in flight
        ra[r] = sw_ld16<2>(rq, voq, (uint32_t)r * rb);
        sa[r] = sw_ld4f<2>(rs, vos, (uint32_t)r * sb);
    }
    float *myruns = runs + (ac * DC_RB) * NC + c;
#pragma unroll
    for (int r = 0; r < DC_RB; r++) {
        const float sc = W.gs > 0 ? sa[r] : 1.0f;
        const float p = row_term<C16>((float)dot8_group(ra[r] ^ 0x88888888u, X) * (sc * xf), gv, CH);
        if (lead) myruns[r * NC] = p;
    }
    __syncthreads();
    if (tid < DC_RB) {
        float acc = 0.f;
        if (W.gs > 0 && NC <= DC_NCM) {
            // every rank's run sums and weight read from LDS first, then the same additions
            // and the rank-order fma chain (a loop over the ranks would wait out an LDS
            // latency for each of its loads in turn)
            for (int a0 = 0; a0 < K; a0 += DC_KU) {
                float yr[DC_KU][DC_NCM], wr[DC_KU];
#pragma unroll
                for (int u = 0; u < DC_KU; u++) {
                    const int aa = min(a0 + u, K - 1);
                    const float *rr = runs + (aa * DC_RB + tid) * NC;
#pragma unroll
                    for (int cc = 0; cc < DC_NCM; cc++) yr[u][cc] = rr[min(cc, NC - 1)];
                    wr[u] = wk[aa];
                }
#pragma unroll
                for (int u = 0; u < DC_KU; u++) {
                    if (a0 + u < K) {                 // (uniform)
                        float y = yr[u][0];
#pragma unroll
                        for (int cc = 1; cc < DC_NCM; cc++)
                            if (cc < NC) y = y + yr[u][cc];
                        acc = __builtin_fmaf(wr[u], y, acc);
                    }
                }
            }
        } else {
            for (int aa = 0; aa < K; aa++) {
                const float *rr = runs + (aa * DC_RB + tid) * NC;
                float y = rr[0];
                for (int cc = 1; cc < NC; cc++) y = y + rr[cc];
                if (W.gs <= 0) y = y * W.s[(int64_t)sel[aa] * D + d0 + tid];
                acc = __builtin_fmaf(wk[aa], y, acc);
            }
        }
        acc = acc * route_scale;
        if (A.wsh) {                                  // c/inkling.c:1176-1182: after the routed ranks
            for (int j = 0; j < A.ns; j++) acc = __builtin_fmaf(A.wsh[j], shared[(int64_t)j * D + d0 + tid], acc);
        } else if (shared) {
            acc = acc + sh_d;
        }
        out[d0 + tid] = out_d + acc;
    }
}

template <int C16>
__global__ __launch_bounds__(1024) void k_dot8_down_combine(Dot8DownArgs A) {
    extern __shared__ __align__(16) float red[];
    dot8_down_combine_block<C16>(A, blockIdx.x, red);
}

int sw_launch_q4_dot8_down_combine(hipStream_t st, SwQ4 W, const sw_u32x4 *hl, const float *hs, const int *sel, const float *w,
                                   int K, float route_scale, const float *shared, float *out, const float *wsh, int ns) {
    const int I = W.K, G = I / RG;
    int gsh;
    if (!dot8_shape_ok(I) || W.O % DC_RB || K <= 0 || K > 64 || K * run_lanes(G) > 1024 || !sw_q4_extent_ok(W) ||
        sw_q4_gsh(W, gsh)) return -1;
    const size_t lds = (size_t)K * DC_RB * dot8_nc(I) * 4;
    const int threads = (K * run_lanes(G) + 63) / 64 * 64;
    if (wsh && (!shared || ns <= 0)) return -1;
    const Dot8DownArgs A = {W, gsh, hl, hs, sel, w, K, route_scale, shared, out, wsh, ns};
    if (dot8_c16(I)) SW_LAUNCH(k_dot8_down_combine<1>, dim3((unsigned)(W.O / DC_RB)), dim3(threads), lds, st, A);
    else SW_LAUNCH(k_dot8_down_combine<0>, dim3((unsigned)(W.O / DC_RB)), dim3(threads), lds, st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------ fused stages ----
// A decode step of the MoE block is three launches on one stream:
//   stage 1: router logits / scores / limbs of x   + the shared expert's gate_up
//   stage 2: routed gate_up (routing fused for one token) + the shared expert's down
//   stage 3: routed down + rank-order combine (+ shared), or the grouped rows + combine
// The blocks of the two jobs of a stage share one grid (the critical-path job
// first), so the shared expert fills what the routed work leaves of the chip
// instead of running as its own launches.
static size_t lds_max(size_t a, size_t b) { return a > b ? a : b; }

struct ShGluArgs { const uint16_t *Wg, *Wu; const float *x; int D, Is; float *h; };

// the device's CUs (one device per process; 0 if it cannot be read)
static int sw_cu_count() {
    static int ncu = -1;
    if (ncu < 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            ncu = 0;
    }
    return ncu;
}

struct ShDownArgs { const uint16_t *Wd; const float *h; int Is, D; float *out; };

// SK: the extra blocks are a batch's shared gate_up over column tiles of SK x 16 tokens
// (sh_sk_block, inputs split from x), else the single token's (sh_glu_block)
// NORM: the rows of x are raw, normalised by the router blocks (RMSNorm, R.nw)
template <int BF16, int ONE, int SK, int NORM = 0>
__global__ __launch_bounds__(SH_NT) void k_stage_route(RouterArgs R, int nbr, int S, ShGluArgs G, ShSkArgs Sk) {
    extern __shared__ __align__(16) float smem[];
    const int b = blockIdx.x;
    if (b < nbr * S) {
        router_block<BF16, ONE, NORM>(R, b % nbr, b / nbr, nbr, smem);
    } else if constexpr (SK > 0) {
        const int w = b - nbr * S, nrb = sh_sk_rows(1, Sk.O);
        sh_sk_block<1, SK, 1>(Sk, w % nrb, w / nrb, smem);
    } else {
        sh_glu_block(G.Wg, G.Wu, G.x, G.D, G.Is, G.h, b - nbr * S, smem);
    }
}

// One token's gate_up units (rank a, 32 outputs c), unit u = a * nch + c (nch = I / 32),
// dealt over the blocks.  Blocks b and b + ncu share a CU (the dispatcher places one
// block on every CU before it places second ones), so when the units outnumber the
// CUs the CUs that take two hold blocks [0, h) and [ncu, nglu), h = nglu - ncu: those
// get the lowest ranks, whose routing (rank + 1 top-k passes) is the shortest.
__device__ __forceinline__ int b1_unit(int b, int nglu, int ncu) {
    const int h = nglu - ncu;
    if (h <= 0 || h > ncu) return b;                // (no CU takes two, or some take more)
    if (b < h) return b;
    if (b >= ncu) return h + (b - ncu);
    return 2 * h + (b - h);
}

// TTG: tokens per pass of the routed gate_up.  The extra blocks: the single token's
// shared down (sh_down_block), or with SKD a batch's shared expert: 1 its down
// (sh_sk_block over the parts of h), 2 its gate_up over column tiles of 16 tokens
// (sh_sk_block, inputs split from x).  ncu: the device's CUs (one token's unit order)
template <int PF, int PICK, int NP, int TTG, int C16, int RO, int SKD>
__global__ __launch_bounds__(DG_NT, PICK ? 1 : 4) void k_stage_experts(Dot8GluArgs A, int nbx, int nglu, ShDownArgs Sd,
                                                                    ShSkArgs Skd, int ncu) {
    extern __shared__ __align__(16) float smem[];
    const int b = blockIdx.x;
    if (b < nglu) {
        if constexpr (PICK) {
            const int u = b1_unit(b, nglu, ncu), nch = nglu / nbx;
            dot8_glu_block<PF, PICK, NP, TTG, C16, RO, 0, SKD != 1 && PF < 8>(A, u / nch, u % nch, smem);
        } else {
            const int w = A.grp.items ? sw_xcd_work(b, nglu) : b;
            // (cached loads with the batch shared down or the 8-deep ring, which spill with
            // both load paths)
            dot8_glu_block<PF, PICK, NP, TTG, C16, RO, 0, SKD != 1 && PF < 8>(A, w % nbx, w / nbx, smem);
        }
    } else if constexpr (SKD == 1) {
        const int w = b - nglu, nrb = sh_sk_rows(0, Skd.O);
        sh_sk_block<0, 2, 0>(Skd, w % nrb, w / nrb, smem);
    } else if constexpr (SKD == 2) {
        const int w = b - nglu, nrb = sh_sk_rows(1, Skd.O);
        sh_sk_block<1, 1, 1, 6>(Skd, w % nrb, w / nrb, smem);   // (a 6-step ring: within 128 registers)
    } else {
        sh_down_block(Sd.Wd, Sd.h, Sd.Is, Sd.D, Sd.out, b - nglu, smem);
    }
}
template <int PICK, int NP, int TTG, int RO = 32, int SKD = 0>
struct StageL {
    template <int PF, int C16>
    struct L {
        static void go(dim3 grid, size_t lds, hipStream_t st, const Dot8GluArgs &A, int nbx, int nglu, const ShDownArgs &Sd,
                       const ShSkArgs &Skd) {
            SW_LAUNCH((k_stage_experts<PF, PICK, NP, TTG, C16, RO, SKD>), grid, dim3(DG_NT), lds, st, A, nbx, nglu, Sd, Skd,
                      sw_cu_count());
        }
    };
};

template <int ONE, int SK, int NORM = 0>
static void launch_stage_route(int bf16, dim3 grid, size_t lds, hipStream_t st, const RouterArgs &R, int nbr, int S,
                               const ShGluArgs &G, const ShSkArgs &Sk, int nt = SH_NT) {
    if (bf16) SW_LAUNCH((k_stage_route<1, ONE, SK, NORM>), grid, dim3(nt), lds, st, R, nbr, S, G, Sk);
    else SW_LAUNCH((k_stage_route<0, ONE, SK, NORM>), grid, dim3(nt), lds, st, R, nbr, S, G, Sk);
}

// stage 1: router logits / scores and the limbs of x, and the shared
// expert's gate_up when sg is non-null
int sw_launch_stage_route(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                          const float *logit_bias, float *logits, float *scores, int route_act, sw_u32x4 *xl, float *xs,
                          const uint16_t *sg, const uint16_t *su, int Is, float *sh_h, uint16_t *xp, uint16_t *sh_hp,
                          const float *nw, float eps, float *xn) {
    if (D % 128 || E <= 0 || S <= 0 || route_act < 0 || route_act > SW_ROUTE_ACT_MAX || (!sw_act_softmax(route_act) && !scores)) return -1;
    if (xp && !sh_shape_ok(D)) return -1;
    const int one = router_one(S, E);
    const size_t rl = router_lds(D);
    // threads per router block of a batch without the shared expert's blocks or parts: 2
    // waves (8 experts per block, twice the blocks of 4 waves over the CUs: B=8 9.8 -> 7.6
    // us), 4 with the RMSNorm (rms_inv_block's fixed order is over 256 threads), more only
    // when x needs them to stage (D <= 4 RT_XB threads)
    int rnt = SH_NT;
    if (!one && !sg && !xp) {
        rnt = nw ? RN_NT : 128;
        while (rnt < SH_NT && D > 4 * RT_XB * rnt) rnt *= 2;
    }
    if (rl > 65536 || D > 4 * RT_XB * (one ? SH_NT - 64 : rnt)) return -1;
    const int nbr = (E + router_epb(one, rnt) - 1) / router_epb(one, rnt);
    // the RMSNorm of the rows (nw): not with the shared expert's blocks or parts, which
    // read x as given
    if (nw && (sg || xp || !xn)) return -1;
    const RouterArgs R = {Wc, x, D, E, logit_bias, logits, route_act, scores, xl, xs, xp, nw, eps, xn};
    const ShGluArgs G = {sg, su, x, D, Is, sh_h};
    // the shared expert's gate_up: one token's blocks (h to sh_h), or with sh_hp a batch's
    // split-K blocks (h's parts to sh_hp)
    if (sg && (!su || Is % 64 || !sh_shape_ok(D))) return -1;
    if (sg && !(S == 1 ? sh_h && !sh_hp : sh_hp && S <= SH_SK_MAX_S)) return -1;
    const int nc = sh_sk_nc(1, S);
    const ShSkArgs Sk = {sg, su, nullptr, x, S, D, Is, sh_hp};
    const int nsh = !sg ? 0 : S == 1 ? sh_glu_blocks(Is) : sh_sk_rows(1, Is) * sh_sk_cols(S, nc);
    const dim3 grid((unsigned)(nbr * S + nsh));
    const size_t lds = lds_max(rl, !sg ? 0 : S == 1 ? sh_glu_lds(D) : sh_sk_lds(nc));
    if (lds > 65536) return -1;
    const int sk = sg && S > 1 ? nc : 0;
    if (nw) {
        if (one) launch_stage_route<1, 0, 1>(w_bf16, grid, lds, st, R, nbr, S, G, Sk);
        else launch_stage_route<0, 0, 1>(w_bf16, grid, lds, st, R, nbr, S, G, Sk, rnt);
    } else if (one) {
        if (sk) launch_stage_route<1, 1>(w_bf16, grid, lds, st, R, nbr, S, G, Sk);   // (ONE: S <= 4, so nc = 1)
        else launch_stage_route<1, 0>(w_bf16, grid, lds, st, R, nbr, S, G, Sk);
    } else if (sk == 1) {
        launch_stage_route<0, 1>(w_bf16, grid, lds, st, R, nbr, S, G, Sk);
    } else if (sk == 2) {
        launch_stage_route<0, 2>(w_bf16, grid, lds, st, R, nbr, S, G, Sk);
    } else {
        launch_stage_route<0, 0>(w_bf16, grid, lds, st, R, nbr, S, G, Sk, rnt);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// stage 2.  Routed gate_up for the groups g (sel null), or for one token's K
// picks: from sel (route_src null) or, with route_src (the token's logits or
// scores), by a gate + top-k in every block, the picks and weights written to
// sel / w; plus the shared expert's down when sd is non-null.
int sw_launch_stage_experts(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, int I, sw_u32x4 *hl,
                            float *hs, int *sel, int K, const float *route_src, int E, int act, const float *bias,
                            int use_bias, int norm, float *w, const uint16_t *sd, const float *sh_h, int S, int Is, int D,
                            float *sh_out, uint16_t *sh_hp, const uint16_t *sg, const uint16_t *su, const float *x) {
    int gsh;
    if (dot8_glu_check(W, I, gsh)) return -1;
    const bool picks = sel != nullptr;
    if (picks && (S != 1 || K <= 0 || K > 64)) return -1;
    if (picks && route_src && (E <= 0 || E > 256 || K > E || !w || !(act == 1 || sw_act_scores(act)))) return -1;
    if (!picks && g.ngroups_max <= 0) return -1;
    // the shared expert's down: one token's blocks (from h in sh_h), or with sh_hp a
    // batch's split-K blocks (from h's parts); out to sh_out
    if (sd && (!sh_out || D % SH_DN_O || !sh_shape_ok(Is))) return -1;
    if (sd && !(S == 1 ? sh_h && !sh_hp : sh_hp && !picks && S <= SH_SK_MAX_S)) return -1;
    // or a batch's shared gate_up split-K blocks over 16-token column tiles (sg, su over x;
    // h's parts to sh_hp; up to 32 tokens), not both
    if (sg && (sd || picks || S > 32 || !su || !x || !sh_hp || Is % 64 || !sh_shape_ok(D))) return -1;
    const int gnc = 1;
    const int skd = sd && S > 1 ? 1 : sg ? 2 : 0;
    const int nbx = picks ? K : g.ngroups_max;
    const int RO = picks ? 32 : dg_ro_grid(I, nbx);   // outputs per gate_up block
    const int nglu = nbx * (I / RO);
    const int nsh = skd == 1 ? sh_sk_rows(0, D) * sh_sk_cols(S, 2) : skd ? sh_sk_rows(1, Is) * sh_sk_cols(S, gnc)
                    : sd ? sh_down_blocks(D) : 0;
    const DotRoute rt = route_src ? DotRoute{route_src, bias, E, K, act, use_bias, norm, w} : DotRoute{};
    const Dot8GluArgs A = {W, gsh, xl, xs, g, I, hl, hs, sel, rt};
    const ShDownArgs Sd = {sd, sh_h, Is, D, sh_out};
    const ShSkArgs Skd = skd == 1 ? ShSkArgs{sd, nullptr, sh_hp, nullptr, S, Is, D, sh_out}
                                  : ShSkArgs{sg, su, nullptr, x, S, D, Is, sh_hp};
    const dim3 grid((unsigned)(nglu + nsh));
    const size_t shl = skd == 1 ? sh_sk_lds(2) : skd ? sh_sk_lds(gnc) : sd ? sh_down_lds(Is) : 0;
    if (shl > 65536) return -1;
    const int pf0 = dg_pf_glu(W.K), c16 = dot8_c16(W.K);
    // groups: a 4-step ring, two blocks per CU (four waves per SIMD, 128 VGPRs); an
    // 8-step ring also fits but measured slower at B=32 (224 vs 215 us)
    const int pf = picks ? pf0 : (pf0 < 4 ? pf0 : 4);
    if (!picks) {
        // tokens per pass: one when the groups hold about one token each (the limbs of a
        // second token then only cost registers), else DG_TT
        const int tt = g.tt ? g.tt : DG_TT;
        if (tt != 1 && tt != DG_TT) return -1;
        const size_t lds = lds_max(dot8_glu_lds(W.K, tt, RO), shl);
#define SW_STG_T(T_, K_) \
    do { \
        if (RO == 128) dispatch_pf_c16<StageL<0, 0, T_, 128, K_>::L>(pf, c16, grid, lds, st, A, nbx, nglu, Sd, Skd); \
        else if (RO == 64) dispatch_pf_c16<StageL<0, 0, T_, 64, K_>::L>(pf, c16, grid, lds, st, A, nbx, nglu, Sd, Skd); \
        else dispatch_pf_c16<StageL<0, 0, T_, 32, K_>::L>(pf, c16, grid, lds, st, A, nbx, nglu, Sd, Skd); \
    } while (0)
#define SW_STG(K_) \
    do { \
        if (tt == 1) SW_STG_T(1, K_); \
        else SW_STG_T(DG_TT, K_); \
    } while (0)
        if (skd == 1) SW_STG(1);
        else if (skd == 2) SW_STG(2);
        else SW_STG(0);
#undef SW_STG
#undef SW_STG_T
    } else {
        const size_t lds = lds_max(dot8_glu_lds(W.K, 1), shl);
        if (!route_src) dispatch_pf_c16<StageL<1, 0, 1>::L>(pf, c16, grid, lds, st, A, nbx, nglu, Sd, Skd);
        else if (E <= 64) dispatch_pf_c16<StageL<1, 1, 1>::L>(pf, c16, grid, lds, st, A, nbx, nglu, Sd, Skd);
        else if (E <= 128) dispatch_pf_c16<StageL<1, 2, 1>::L>(pf, c16, grid, lds, st, A, nbx, nglu, Sd, Skd);
        else dispatch_pf_c16<StageL<1, 4, 1>::L>(pf, c16, grid, lds, st, A, nbx, nglu, Sd, Skd);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
