// k_dot8.hip -- the int4 expert GEMV of decode on the gfx950 integer dot unit.
//
// v_dot8_i32_i4 multiplies eight signed 4-bit pairs and adds them to an int32
// in one VALU op.  A weight dword holds eight nibbles n (k = 8j + i at bits
// 4i, the container layout of c/moe_quant.h), and n ^ 8 read as a signed
// nibble is exactly n - 8, the weight's integer value: one XOR per eight
// weights is the whole dequant.  The activation side is split into "limbs":
// for each group of 32 consecutive inputs, with 2^e the smallest power of two
// above max|x| of the group, y = x * 2^-e in (-1, 1) is written as
// sum_{l=1..NL} d_l 8^-l with signed digits d_l in [-8, 7] (round to nearest,
// clamp, carry the exact remainder), so
//     x ~= 2^(e - 3 NL) * D,   D = sum_l d_l 8^(NL - l)   (|error| <= 2^e 8^-NL).
// For one weight row and one group, sum_k (n_k - 8) D_k is an exact int32
// (Horner over the limbs: acc = (acc << 3) + four dot8), turned into f32 once
// (|acc| < 2^24, exact) and multiplied by s_row,group * 2^(e - 3 NL) (exact
// power-of-two scaling of the weight scale).  A row's output is then the sum
// of its group terms in a fixed order: runs of CH consecutive groups summed
// left to right, the run sums summed left to right.  Nothing of it depends on
// which tokens share a launch, so grouped and per-token results are
// bit-identical.
//
// Per weight byte this is ~2 VALU ops (XOR, dot8, shift over NL = 5 limbs,
// one fma per 32 weights) against ~3.3 for nibble-to-f16 dequant plus MFMA,
// and each wave load is 1 KB of one row, contiguous.
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
    hipLaunchKernelGGL(k_limbs, dim3((unsigned)((G + 7) / 8), (unsigned)rows), dim3(256), 0, st, x, K, rows, xl, xs);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// exact int32 sum_k (n_k - 8) D_k over one group (16 bytes of nibbles)
__device__ __forceinline__ int dot8_group(sw_u32x4 w, const sw_u32x4 *X) {
    const sw_u32x4 a = w ^ 0x88888888u;
    int acc = 0;
#pragma unroll
    for (int l = 0; l < SW_NL; l++) {
        acc <<= 3;
        acc = __builtin_amdgcn_sdot8((int)a.x, (int)X[l].x, acc, false);
        acc = __builtin_amdgcn_sdot8((int)a.y, (int)X[l].y, acc, false);
        acc = __builtin_amdgcn_sdot8((int)a.z, (int)X[l].z, acc, false);
        acc = __builtin_amdgcn_sdot8((int)a.w, (int)X[l].w, acc, false);
    }
    return acc;
}

// ------------------------------------------------------------ gate_up ----
// One block = 32 consecutive intermediate outputs i of one group: gate rows
// i0..i0+31 and up rows i0..i0+31 (64 weight rows), every input group, for
// each token of the group in turn (later tokens re-read the block's 160 KB
// from L2).  Thread (row offset ro, input group g) with TPR = G threads per
// row and RPS = 256 / G rows per step keeps its group's limbs in registers
// and streams one 16-byte weight load per step (PF steps in flight); the
// group terms go to LDS and the fixed-order row sums, the SiLU-GLU and the
// f16 hi/lo plane output (the down projection's input) follow.
#define DG_ROWS 64
// Fused routing for one token (NP > 0): every block runs the token's gate +
// top-k on its first wave (gate_topk_wave, deterministic, so every block gets
// the same picks) while the others fetch the limbs; block (0, 0) also writes
// the picks and weights out for the down projection.
struct DotRoute {
    const float *src;          // the token's logits (act 1) or sigmoid/softplus scores
    const float *bias;         // selection bias (e_score_correction_bias) or null
    int E, K, act, use_bias, norm;
    int *sel_out;
    float *w_out;
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
    DotRoute rt;
};
// block (bx = group or rank, by = set of 32 outputs); red: the dynamic LDS
// ([DG_ROWS][G + 1], then [DG_ROWS][G / CH] floats)
template <int PF, int NP>
__device__ __forceinline__ void dot8_glu_block(const Dot8GluArgs &A, int bx, int by, float *red) {
    const SwQ4 W = A.W;
    const int gsh = A.gsh, I = A.I;
    const sw_u32x4 *__restrict__ xl = A.xl;
    const float *__restrict__ xs = A.xs;
    const SwGroups grp = A.grp;
    sw_u32x4 *__restrict__ hl = A.hl;
    float *__restrict__ hs = A.hs;
    const DotRoute rt = A.rt;
    const int K = W.K, G = K / RG, Gp = G + 1;
    const int tid = threadIdx.x;
    const int RPS = 256 / G, NS = (DG_ROWS + RPS - 1) / RPS;
    const int ro = tid / G, g = tid - ro * G;
    const bool worker = ro < RPS;
    const int gi = bx;
    const int i0 = by * (DG_ROWS / 2);
    const int ng = W.gs > 0 ? K / W.gs : 1;
    const int gshift = W.gs > 0 ? gsh : 31;
    const int sg = (g * RG) >> gshift;               // this thread's weight-scale column
    int e, beg, cnt;
    int64_t tok0;
    sw_u32x4 X[SW_NL];
    if constexpr (NP > 0) {                           // one token: rank gi of its picks
        __shared__ TopkLDS tk;
        beg = gi; cnt = 1; tok0 = 0;
#pragma unroll
        for (int l = 0; l < SW_NL; l++) X[l] = xl[(int64_t)g * SW_NL + l];
        if (tid < 64) gate_topk_wave<NP>(rt.src, rt.E, rt.K, rt.act, rt.bias, rt.use_bias, rt.norm, tk);
        __syncthreads();
        e = tk.sk[gi];
        if (bx == 0 && by == 0 && tid < rt.K) { rt.sel_out[tid] = tk.sk[tid]; rt.w_out[tid] = tk.wk[tid]; }
    } else {
        const int gvalid = grp.G ? *grp.G : grp.ngroups_max;
        if (gi >= gvalid) return;
        e = grp.gexp ? grp.gexp[gi] : 0;
        beg = grp.gbeg ? grp.gbeg[gi] : 0;
        cnt = grp.gcnt ? grp.gcnt[gi] : grp.cnt_const;
        tok0 = grp.grow ? grp.grow[beg] : beg;
        if (cnt > 0) {
#pragma unroll
            for (int l = 0; l < SW_NL; l++) X[l] = xl[(tok0 * G + g) * SW_NL + l];
        }
    }
    // weight row of step s: local row lr = s*RPS + ro (clamped); gate rows first, then up rows
    auto wrow = [&](int s) -> int64_t {
        int lr = s * RPS + (worker ? ro : 0);
        lr = lr < DG_ROWS ? lr : DG_ROWS - 1;
        const int i = i0 + (lr & 31);
        return (int64_t)e * (2 * I) + (lr < 32 ? i : I + i);
    };
    const float *sbase = W.s + (W.gs > 0 ? sg : 0);   // per-row scales: read (and ignored) in the loop
    for (int t = 0; t < cnt; t++) {
        const int64_t tok = t == 0 ? tok0 : (grp.grow ? grp.grow[beg + t] : beg + t);
        if (t > 0) {
#pragma unroll
            for (int l = 0; l < SW_NL; l++) X[l] = xl[(tok * G + g) * SW_NL + l];
        }
        const float xf = xs[tok * G + g];
        sw_u32x4 ra[PF];
        float sa[PF];
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int64_t wr = wrow(u);
            ra[u] = *(const sw_u32x4 *)(W.q + wr * (K / 2) + g * 16);
            sa[u] = sbase[wr * ng];
        }
        auto step = [&](int s, int u, bool refill) {
            const int acc = dot8_group(ra[u], X);
            const float sx = (W.gs > 0 ? sa[u] : 1.0f) * xf;
            if (refill) {
                const int64_t wr = wrow(s + PF);
                ra[u] = *(const sw_u32x4 *)(W.q + wr * (K / 2) + g * 16);
                sa[u] = sbase[wr * ng];
                __builtin_amdgcn_sched_barrier(0);
            }
            const int lr = s * RPS + ro;
            if (worker && lr < DG_ROWS) red[lr * Gp + g] = (float)acc * sx;
        };
        int s0 = 0;
        for (; s0 + PF < NS; s0 += PF) {
#pragma unroll
            for (int u = 0; u < PF; u++) step(s0 + u, u, true);
        }
#pragma unroll
        for (int u = 0; u < PF; u++)
            if (s0 + u < NS) step(s0 + u, u, false);
        __syncthreads();
        // fixed-order row sums: runs of CH groups left to right, runs left to right
        const int CH = G < CHG ? G : CHG, NC = G / CH;
        float *runs = red + DG_ROWS * Gp;
        for (int it = tid; it < DG_ROWS * NC; it += 256) {
            const int r = it / NC, c = it - r * NC;
            const float *p = red + r * Gp + c * CH;
            float sum = p[0];
            for (int j = 1; j < CH; j++) sum = sum + p[j];
            runs[r * NC + c] = sum;
        }
        __syncthreads();
        if (tid < 32) {
            float yg = runs[tid * NC], yu = runs[(32 + tid) * NC];
            for (int c = 1; c < NC; c++) { yg = yg + runs[tid * NC + c]; yu = yu + runs[(32 + tid) * NC + c]; }
            if (W.gs <= 0) {                            // per-row scales after the sum
                yg = yg * W.s[(int64_t)e * (2 * I) + i0 + tid];
                yu = yu * W.s[(int64_t)e * (2 * I) + I + i0 + tid];
            }
            const float h = (yg / (1.0f + expf(-yg))) * yu;
            // the block's 32 outputs are one limb group of the down projection's input
            const int GI = I / RG, gi_out = i0 / RG;
            const int64_t prow = beg + t;
            limbs_group(h, tid, hl + (prow * GI + gi_out) * SW_NL, hs + prow * GI + gi_out);
        }
        __syncthreads();
    }
}

template <int PF, int NP>
__global__ __launch_bounds__(256) void k_dot8_glu(Dot8GluArgs A) {
    extern __shared__ __align__(16) float red[];
    dot8_glu_block<PF, NP>(A, blockIdx.x, blockIdx.y, red);
}

template <int NP>
static void launch_dot8_glu(int ns, dim3 grid, size_t lds, hipStream_t st, SwQ4 W, int gsh, const sw_u32x4 *xl, const float *xs,
                            SwGroups g, int I, sw_u32x4 *hl, float *hs, DotRoute rt) {
    const Dot8GluArgs A = {W, gsh, xl, xs, g, I, hl, hs, rt};
    if (ns >= 8) hipLaunchKernelGGL((k_dot8_glu<8, NP>), grid, dim3(256), lds, st, A);
    else if (ns >= 4) hipLaunchKernelGGL((k_dot8_glu<4, NP>), grid, dim3(256), lds, st, A);
    else hipLaunchKernelGGL((k_dot8_glu<2, NP>), grid, dim3(256), lds, st, A);
}

static int dot8_glu_check(SwQ4 W, int I, int &gsh) {
    const int K = W.K, G = K / RG;
    if (K % RG || I % 32 || W.O != 2 * I || G > 192) return -1;   // LDS: 64 rows x G terms
    const int CH = G < CHG ? G : CHG;
    if (G % CH) return -1;
    gsh = 0;
    if (W.gs > 0) {
        if (W.gs % RG || K % W.gs || (W.gs & (W.gs - 1))) return -1;
        while ((1 << gsh) < W.gs) gsh++;
    }
    return 0;
}
static size_t dot8_glu_lds(int K) {
    const int G = K / RG, CH = G < CHG ? G : CHG;
    return ((size_t)DG_ROWS * (G + 1) + (size_t)DG_ROWS * (G / CH)) * 4;
}

int sw_launch_q4_dot8_glu(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, int I,
                          sw_u32x4 *hl, float *hs) {
    int gsh;
    if (dot8_glu_check(W, I, gsh) || g.ngroups_max <= 0) return -1;
    const int G = W.K / RG, RPS = 256 / G, NS = (DG_ROWS + RPS - 1) / RPS;
    const DotRoute rt = {};
    launch_dot8_glu<0>(NS, dim3((unsigned)g.ngroups_max, (unsigned)(I / 32)), dot8_glu_lds(W.K), st, W, gsh, xl, xs, g, I,
                       hl, hs, rt);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_q4_dot8_glu_routed(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, int I, sw_u32x4 *hl, float *hs,
                                 const float *route_src, int E, int K, int act, const float *bias, int use_bias, int norm,
                                 int *sel, float *w) {
    int gsh;
    if (dot8_glu_check(W, I, gsh) || E <= 0 || E > 256 || K <= 0 || K > 64 || K > E) return -1;
    const int G = W.K / RG, RPS = 256 / G, NS = (DG_ROWS + RPS - 1) / RPS;
    const SwGroups g = {};
    const DotRoute rt = {route_src, bias, E, K, act, use_bias, norm, sel, w};
    const dim3 grid((unsigned)K, (unsigned)(I / 32));
    const size_t lds = dot8_glu_lds(W.K);
    if (E <= 64) launch_dot8_glu<1>(NS, grid, lds, st, W, gsh, xl, xs, g, I, hl, hs, rt);
    else if (E <= 128) launch_dot8_glu<2>(NS, grid, lds, st, W, gsh, xl, xs, g, I, hl, hs, rt);
    else launch_dot8_glu<4>(NS, grid, lds, st, W, gsh, xl, xs, g, I, hl, hs, rt);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ------------------------------------------------------------ rows ----
// Y[packed row, O] = W_e . x for every packed row of every group (the down
// projection of the grouped path): block = 64 consecutive output rows of one
// group, thread (row offset, input group) as in the gate_up, same fixed-order
// row sums, f32 rows out.
struct Dot8RowsArgs {
    SwQ4 W;
    int gsh;
    const sw_u32x4 *xl;
    const float *xs;
    SwGroups grp;
    float *Y;
};
template <int PF>
__device__ __forceinline__ void dot8_rows_block(const Dot8RowsArgs &A, int bx, int by, float *red) {
    const SwQ4 W = A.W;
    const int gsh = A.gsh;
    const sw_u32x4 *__restrict__ xl = A.xl;
    const float *__restrict__ xs = A.xs;
    const SwGroups grp = A.grp;
    float *__restrict__ Y = A.Y;
    const int K = W.K, G = K / RG, Gp = G + 1, O = W.O;
    const int tid = threadIdx.x;
    const int RPS = 256 / G, NS = (DG_ROWS + RPS - 1) / RPS;
    const int ro = tid / G, g = tid - ro * G;
    const bool worker = ro < RPS;
    const int gi = bx;
    const int gvalid = grp.G ? *grp.G : grp.ngroups_max;
    if (gi >= gvalid) return;
    const int e = grp.gexp ? grp.gexp[gi] : 0, beg = grp.gbeg ? grp.gbeg[gi] : 0;
    const int cnt = grp.gcnt ? grp.gcnt[gi] : grp.cnt_const;
    const int r0 = by * DG_ROWS;
    const int nrows = min(DG_ROWS, O - r0);
    const int ng = W.gs > 0 ? K / W.gs : 1;
    const int sg = W.gs > 0 ? (g * RG) >> gsh : 0;
    auto wrow = [&](int s) -> int64_t {
        int lr = s * RPS + (worker ? ro : 0);
        lr = lr < nrows ? lr : nrows - 1;
        return (int64_t)e * O + r0 + lr;
    };
    const float *sbase = W.s + sg;
    for (int t = 0; t < cnt; t++) {
        const int64_t tok = grp.grow ? grp.grow[beg + t] : beg + t;
        sw_u32x4 X[SW_NL];
#pragma unroll
        for (int l = 0; l < SW_NL; l++) X[l] = xl[(tok * G + g) * SW_NL + l];
        const float xf = xs[tok * G + g];
        sw_u32x4 ra[PF];
        float sa[PF];
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int64_t wr = wrow(u);
            ra[u] = *(const sw_u32x4 *)(W.q + wr * (K / 2) + g * 16);
            sa[u] = sbase[wr * ng];
        }
        auto step = [&](int s, int u, bool refill) {
            const int acc = dot8_group(ra[u], X);
            const float sx = (W.gs > 0 ? sa[u] : 1.0f) * xf;
            if (refill) {
                const int64_t wr = wrow(s + PF);
                ra[u] = *(const sw_u32x4 *)(W.q + wr * (K / 2) + g * 16);
                sa[u] = sbase[wr * ng];
                __builtin_amdgcn_sched_barrier(0);
            }
            const int lr = s * RPS + ro;
            if (worker && lr < DG_ROWS) red[lr * Gp + g] = (float)acc * sx;
        };
        int s0 = 0;
        for (; s0 + PF < NS; s0 += PF) {
#pragma unroll
            for (int u = 0; u < PF; u++) step(s0 + u, u, true);
        }
#pragma unroll
        for (int u = 0; u < PF; u++)
            if (s0 + u < NS) step(s0 + u, u, false);
        __syncthreads();
        const int CH = G < CHG ? G : CHG, NC = G / CH;
        float *runs = red + DG_ROWS * Gp;
        for (int it = tid; it < DG_ROWS * NC; it += 256) {
            const int r = it / NC, c = it - r * NC;
            const float *p = red + r * Gp + c * CH;
            float sum = p[0];
            for (int j = 1; j < CH; j++) sum = sum + p[j];
            runs[r * NC + c] = sum;
        }
        __syncthreads();
        if (tid < nrows) {
            float y = runs[tid * NC];
            for (int c = 1; c < NC; c++) y = y + runs[tid * NC + c];
            if (W.gs <= 0) y = y * W.s[(int64_t)e * O + r0 + tid];
            Y[(int64_t)(beg + t) * O + r0 + tid] = y;
        }
        __syncthreads();
    }
}

template <int PF>
__global__ __launch_bounds__(256) void k_dot8_rows(Dot8RowsArgs A) {
    extern __shared__ __align__(16) float red[];
    dot8_rows_block<PF>(A, blockIdx.x, blockIdx.y, red);
}

int sw_launch_q4_dot8_rows(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, float *Y) {
    const int K = W.K, G = K / RG;
    if (K % RG || G > 192 || g.ngroups_max <= 0 || W.O <= 0) return -1;
    const int CH = G < CHG ? G : CHG;
    if (G % CH) return -1;
    int gsh = 0;
    if (W.gs > 0) {
        if (W.gs % RG || K % W.gs || (W.gs & (W.gs - 1))) return -1;
        while ((1 << gsh) < W.gs) gsh++;
    }
    const int RPS = 256 / G, NS = (DG_ROWS + RPS - 1) / RPS;
    const dim3 grid((unsigned)g.ngroups_max, (unsigned)((W.O + DG_ROWS - 1) / DG_ROWS));
    const size_t lds = dot8_glu_lds(K);
    const Dot8RowsArgs A = {W, gsh, xl, xs, g, Y};
    if (NS >= 8) hipLaunchKernelGGL(k_dot8_rows<8>, grid, dim3(256), lds, st, A);
    else if (NS >= 4) hipLaunchKernelGGL(k_dot8_rows<4>, grid, dim3(256), lds, st, A);
    else hipLaunchKernelGGL(k_dot8_rows<2>, grid, dim3(256), lds, st, A);
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
#define DC_RB 16
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
};
// block bx of DC_RB output rows; red: [K][DC_RB][G + 1], then [K][DC_RB][G / CH] floats
template <int PF>
__device__ __forceinline__ void dot8_down_combine_block(const Dot8DownArgs &A, int bx, float *red) {
    const SwQ4 W = A.W;
    const int gsh = A.gsh, K = A.K;
    const sw_u32x4 *__restrict__ hl = A.hl;
    const float *__restrict__ hs = A.hs;
    const int *__restrict__ sel = A.sel;
    const float *__restrict__ wts = A.wts;
    const float route_scale = A.route_scale;
    const float *__restrict__ shared = A.shared;
    float *__restrict__ out = A.out;
    __shared__ float wk[64];
    const int I = W.K, G = I / RG, Gp = G + 1, D = W.O;
    const int tid = threadIdx.x, a = tid / G, g = tid - a * G;
    const bool worker = a < K;
    const int ac = worker ? a : 0;
    const int d0 = bx * DC_RB;
    const int ng = W.gs > 0 ? I / W.gs : 1;
    const int sg = W.gs > 0 ? (g * RG) >> gsh : 0;
    if (tid < K) wk[tid] = wts[tid];
    float sh_d = 0.f, out_d = 0.f;
    if (tid < DC_RB) {
        out_d = out[d0 + tid];
        if (shared) sh_d = shared[d0 + tid];
    }
    sw_u32x4 X[SW_NL];
#pragma unroll
    for (int l = 0; l < SW_NL; l++) X[l] = hl[((int64_t)ac * G + g) * SW_NL + l];
    const float xf = hs[(int64_t)ac * G + g];
    const int e = sel[ac];
    const uint8_t *wp = W.q + ((int64_t)e * D + d0) * (I / 2) + g * 16;
    const float *sp = W.s + ((int64_t)e * D + d0) * ng + sg;
    sw_u32x4 ra[PF];
    float sa[PF];
#pragma unroll
    for (int u = 0; u < PF; u++) {
        ra[u] = *(const sw_u32x4 *)(wp + (int64_t)u * (I / 2));
        sa[u] = sp[(int64_t)u * ng];
    }
    float *myred = red + (ac * DC_RB) * Gp + g;
    auto step = [&](int r, int u, bool refill) {
        const int acc = dot8_group(ra[u], X);
        const float sx = (W.gs > 0 ? sa[u] : 1.0f) * xf;
        if (refill) {
            ra[u] = *(const sw_u32x4 *)(wp + (int64_t)(r + PF) * (I / 2));
            sa[u] = sp[(int64_t)(r + PF) * ng];
            __builtin_amdgcn_sched_barrier(0);
        }
        if (worker) myred[r * Gp] = (float)acc * sx;
    };
    int r0 = 0;
    for (; r0 + PF < DC_RB; r0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; u++) step(r0 + u, u, true);
    }
#pragma unroll
    for (int u = 0; u < PF; u++) step(r0 + u, u, false);
    __syncthreads();
    const int CH = G < CHG ? G : CHG, NC = G / CH;
    float *runs = red + K * DC_RB * Gp;
    for (int it = tid; it < K * DC_RB * NC; it += blockDim.x) {
        const int ar = it / NC, c = it - ar * NC;
        const float *p = red + ar * Gp + c * CH;
        float sum = p[0];
        for (int j = 1; j < CH; j++) sum = sum + p[j];
        runs[ar * NC + c] = sum;
    }
    __syncthreads();
    if (tid < DC_RB) {
        float acc = 0.f;
        for (int aa = 0; aa < K; aa++) {
            const float *rr = runs + (aa * DC_RB + tid) * NC;
            float y = rr[0];
            for (int c = 1; c < NC; c++) y = y + rr[c];
            if (W.gs <= 0) y = y * W.s[(int64_t)sel[aa] * D + d0 + tid];
            acc = __builtin_fmaf(wk[aa], y, acc);
        }
        acc = acc * route_scale;
        if (shared) acc = acc + sh_d;
        out[d0 + tid] = out_d + acc;
    }
}

template <int PF>
__global__ __launch_bounds__(1024) void k_dot8_down_combine(Dot8DownArgs A) {
    extern __shared__ __align__(16) float red[];
    dot8_down_combine_block<PF>(A, blockIdx.x, red);
}

int sw_launch_q4_dot8_down_combine(hipStream_t st, SwQ4 W, const sw_u32x4 *hl, const float *hs, const int *sel, const float *w,
                                   int K, float route_scale, const float *shared, float *out) {
    const int I = W.K, G = I / RG;
    if (I % RG || W.O % DC_RB || K <= 0 || K > 64 || K * G > 1024) return -1;
    const int CH = G < CHG ? G : CHG;
    if (G % CH) return -1;
    int gsh = 0;
    if (W.gs > 0) {
        if (W.gs % RG || I % W.gs || (W.gs & (W.gs - 1))) return -1;
        while ((1 << gsh) < W.gs) gsh++;
    }
    const size_t lds = ((size_t)K * DC_RB * (G + 1) + (size_t)K * DC_RB * (G / CH)) * 4;
    if (lds > 65536) return -1;
    const int threads = (K * G + 63) / 64 * 64;
    const Dot8DownArgs A = {W, gsh, hl, hs, sel, w, K, route_scale, shared, out};
    hipLaunchKernelGGL(k_dot8_down_combine<8>, dim3((unsigned)(W.O / DC_RB)), dim3(threads), lds, st, A);
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
struct ShGluArgs { const uint16_t *Wg, *Wu; const float *x; int S, D, Is; float *h; };
struct ShDownArgs { const uint16_t *Wd; const float *h; int S, Is, D; float *out; };

template <int BF16, int TT>
__global__ __launch_bounds__(256) void k_stage_route(RouterArgs R, int nbr, int S, ShGluArgs G) {
    extern __shared__ __align__(16) float smem[];
    const int b = blockIdx.x;
    if (b < nbr * S) router_block<BF16>(R, b % nbr, b / nbr, nbr, smem);
    else sh_glu_block<TT>(G.Wg, G.Wu, G.x, G.S, G.D, G.Is, G.h, b - nbr * S, smem);
}

template <int PF, int NP, int TT>
__global__ __launch_bounds__(256) void k_stage_experts(Dot8GluArgs A, int nbx, int nglu, ShDownArgs Sd) {
    extern __shared__ __align__(16) float smem[];
    const int b = blockIdx.x;
    if (b < nglu) dot8_glu_block<PF, NP>(A, b % nbx, b / nbx, smem);
    else sh_down_block<TT>(Sd.Wd, Sd.h, Sd.S, Sd.Is, Sd.D, Sd.out, b - nglu, smem);
}

static size_t lds_max(size_t a, size_t b) { return a > b ? a : b; }

// stage 1: sh_glu may be null (no shared expert)
int sw_launch_stage_route(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                          const float *logit_bias, float *logits, float *scores, int route_act, sw_u32x4 *xl, float *xs,
                          const uint16_t *sg, const uint16_t *su, int Is, float *sh_h) {
    if (D % 128 || E <= 0 || S <= 0 || route_act < 0 || route_act > 2 || (route_act != 1 && !scores)) return -1;
    const int nw = 4;
    const size_t rl = router_lds(D, w_bf16, nw);
    if (rl > 65536) return -1;
    const int nbr = (E + nw - 1) / nw;
    const RouterArgs R = {Wc, x, D, E, logit_bias, logits, route_act, scores, xl, xs};
    const ShGluArgs G = {sg, su, x, S, D, Is, sh_h};
    const int TT = S >= 2 ? 2 : 1;
    const int nsh = sg ? sh_glu_blocks(S, Is, TT) : 0;
    if (sg && (Is % SH_GLU_O || (D / SH_RG) > 256)) return -1;
    const dim3 grid((unsigned)(nbr * S + nsh));
    if (TT == 2) {
        const size_t lds = lds_max(rl, sg ? sh_glu_lds<2>(D) : 0);
        if (w_bf16) hipLaunchKernelGGL((k_stage_route<1, 2>), grid, dim3(256), lds, st, R, nbr, S, G);
        else hipLaunchKernelGGL((k_stage_route<0, 2>), grid, dim3(256), lds, st, R, nbr, S, G);
    } else {
        const size_t lds = lds_max(rl, sg ? sh_glu_lds<1>(D) : 0);
        if (w_bf16) hipLaunchKernelGGL((k_stage_route<1, 1>), grid, dim3(256), lds, st, R, nbr, S, G);
        else hipLaunchKernelGGL((k_stage_route<0, 1>), grid, dim3(256), lds, st, R, nbr, S, G);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int NP, int TT>
static void launch_stage_experts(int ns, dim3 grid, size_t lds, hipStream_t st, const Dot8GluArgs &A, int nbx, int nglu,
                                 const ShDownArgs &Sd) {
    if (ns >= 8) hipLaunchKernelGGL((k_stage_experts<8, NP, TT>), grid, dim3(256), lds, st, A, nbx, nglu, Sd);
    else if (ns >= 4) hipLaunchKernelGGL((k_stage_experts<4, NP, TT>), grid, dim3(256), lds, st, A, nbx, nglu, Sd);
    else hipLaunchKernelGGL((k_stage_experts<2, NP, TT>), grid, dim3(256), lds, st, A, nbx, nglu, Sd);
}

// stage 2.  Routed gate_up for the groups g (route_src null), or for one token
// with its routing fused (route_src = its logits or scores; g ignored; picks
// to sel/w); plus the shared expert's down when sd is non-null.
int sw_launch_stage_experts(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, int I, sw_u32x4 *hl,
                            float *hs, const float *route_src, int E, int K, int act, const float *bias, int use_bias,
                            int norm, int *sel, float *w, const uint16_t *sd, const float *sh_h, int S, int Is, int D,
                            float *sh_out) {
    int gsh;
    if (dot8_glu_check(W, I, gsh)) return -1;
    const int G = W.K / RG, RPS = 256 / G, NS = (DG_ROWS + RPS - 1) / RPS;
    const bool fused = route_src != nullptr;
    if (fused && (S != 1 || E <= 0 || E > 256 || K <= 0 || K > 64 || K > E)) return -1;
    if (!fused && g.ngroups_max <= 0) return -1;
    if (sd && (D % SH_DN_O || (Is / SH_RG) > 256)) return -1;
    const int nbx = fused ? K : g.ngroups_max;
    const int nglu = nbx * (I / 32);
    const int TT = S >= 2 ? 2 : 1;
    const int nsh = sd ? sh_down_blocks(S, D, TT) : 0;
    const DotRoute rt = fused ? DotRoute{route_src, bias, E, K, act, use_bias, norm, sel, w} : DotRoute{};
    const Dot8GluArgs A = {W, gsh, xl, xs, g, I, hl, hs, rt};
    const ShDownArgs Sd = {sd, sh_h, S, Is, D, sh_out};
    const dim3 grid((unsigned)(nglu + nsh));
    const size_t lds = lds_max(dot8_glu_lds(W.K), sd ? (TT == 2 ? sh_down_lds<2>(Is) : sh_down_lds<1>(Is)) : 0);
    if (!fused) {
        if (TT == 2) launch_stage_experts<0, 2>(NS, grid, lds, st, A, nbx, nglu, Sd);
        else launch_stage_experts<0, 1>(NS, grid, lds, st, A, nbx, nglu, Sd);
    } else if (E <= 64) {
        launch_stage_experts<1, 1>(NS, grid, lds, st, A, nbx, nglu, Sd);
    } else if (E <= 128) {
        launch_stage_experts<2, 1>(NS, grid, lds, st, A, nbx, nglu, Sd);
    } else {
        launch_stage_experts<4, 1>(NS, grid, lds, st, A, nbx, nglu, Sd);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
