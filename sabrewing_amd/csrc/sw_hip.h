// sw_hip.h -- internal declarations of the gfx950 MoE backend.
//
// Device data layout (HBM):
//   weights    the reference container, unchanged (lag_hip_upload is a plain
//              byte copy, like lag_cuda_upload): int4 gate_up [E*2I, D/2]
//              (gate rows then up rows per expert), scales [E*2I, D/gs] f32,
//              down [E*D, I/2], scales [E*D, I/gs]; bf16 shared expert
//              [Is,D],[Is,D],[D,Is]; router in "chain-major" order (see below).
//   x, out     f32 [S, D] (out is accumulated into: out += MoE(x)).
//   activations of the int4 GEMMs as dot8 limbs (k_dot8.hip) or MFMA digits
//              (k_mfma.hip) per group of 32 inputs; of the bf16 shared expert
//              as three exact bf16 parts (sw_shared.h).
//
// MFMA operand convention for v_mfma_f32_16x16x32_{f16,bf16} (lane l):
//   A: row l%16, hardware k 8*(l/16)+h for element h of the 8-vector
//   B: col l%16, same k;   C: col l%16, rows 4*(l/16)+j, j = 0..3
// (checked on the device by lag_hip_selftest).
//
// Every reduction here is fixed by the operation and its shape alone, never
// by the batch: a token's output does not depend on which other tokens share
// its launch, so the grouped paths are bit-identical to the per-token path.
#ifndef SW_HIP_H
#define SW_HIP_H
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

typedef _Float16 sw_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 sw_half2 __attribute__((ext_vector_type(2)));
typedef __bf16 sw_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sw_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sw_u32x4 __attribute__((ext_vector_type(4)));
typedef int sw_i32x4 __attribute__((ext_vector_type(4)));

#ifdef __HIPCC__
#include <hip/hip_ext.h>
// Per-launch timing for the profile scopes of the backend: while a scope is
// open (sw_launch_events non-null), SW_LAUNCH records the scope's start event
// at the first kernel's dispatch and its stop event at each kernel's end
// (hipExtLaunchKernelGGL), so the pair times the kernels themselves.
struct SwLaunchEvents { hipEvent_t start, stop; int started; };
extern thread_local SwLaunchEvents *sw_launch_events;
#define SW_LAUNCH(kernel, grid, block, lds, st, ...)                                                              \
    do {                                                                                                          \
        if (sw_launch_events) {                                                                                   \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, st, sw_launch_events->started ? nullptr : sw_launch_events->start, \
                                  sw_launch_events->stop, 0, __VA_ARGS__);                                        \
            sw_launch_events->started = 1;                                                                        \
        } else {                                                                                                  \
            hipLaunchKernelGGL(kernel, grid, block, lds, st, __VA_ARGS__);                                        \
        }                                                                                                         \
    } while (0)
// Raw buffer access: a tensor is one descriptor (base and byte extent in
// scalar registers); each lane adds a 32-bit offset and each step a scalar
// one; a load past the extent returns 0 and touches no memory.
typedef __amdgpu_buffer_rsrc_t sw_rsrc;
__device__ __forceinline__ sw_rsrc sw_make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, bytes, 0x00020000);
}
// POL: the load's cache policy; 2 = nt (non-temporal)
template <int POL = 0>
__device__ __forceinline__ sw_u32x4 sw_ld16(sw_rsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, POL);
}
template <int POL = 0>
__device__ __forceinline__ uint2 sw_ld8(sw_rsrc r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, POL);
    return make_uint2(v[0], v[1]);
}
template <int POL = 0>
__device__ __forceinline__ float sw_ld4f(sw_rsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, POL));
}

// The rank-order combine of token s at outputs d .. d+3:
// out[s,d] (+)= (sum_a w[s,a] * slots[rowof[s,a], d]) * route_scale (+ shared[s,d])
// The sum runs in rank order from 0 with one fused multiply-add per rank, the
// operation sequence of moe_block's `acc[i] += w[a] * scr[i]` as the reference
// build compiles it (c/moe_block.h:124-142; c/laguna.c:761-782); with wsh,
// Inkling's ns gated shared outputs shared[s][ns][D] follow as fma(wsh[s,j], .).
// NTL: the slots with nontemporal loads (slots that no later launch reads).
template <int NTL = 0>
__device__ __forceinline__ void combine4(const float *__restrict__ slots, const int *__restrict__ rowof,
                                         const float *__restrict__ w, int64_t s, int K, int D, int d, float route_scale,
                                         const float *__restrict__ shared, float *__restrict__ out, int accumulate,
                                         const float *__restrict__ wsh, int ns) {
    sw_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int a0 = 0; a0 < K; a0 += 8) {
        sw_f32x4 v[8];
        float wa[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (a0 + u < K) {
                wa[u] = w[s * K + a0 + u];
                const sw_f32x4 *sp = (const sw_f32x4 *)(slots + (int64_t)rowof[s * K + a0 + u] * D + d);
                if constexpr (NTL) v[u] = __builtin_nontemporal_load(sp);
                else v[u] = *sp;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (a0 + u < K)
#pragma unroll
                for (int c = 0; c < 4; c++) acc[c] = __builtin_fmaf(wa[u], v[u][c], acc[c]);
    }
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = acc[c] * route_scale;
    if (wsh) {
        for (int j = 0; j < ns; j++) {
            const float wj = wsh[s * ns + j];
            const sw_f32x4 sh = *(const sw_f32x4 *)(shared + (s * ns + j) * D + d);
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = __builtin_fmaf(wj, sh[c], acc[c]);
        }
    } else if (shared) {
        const sw_f32x4 sh = *(const sw_f32x4 *)(shared + s * D + d);
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] = acc[c] + sh[c];
    }
    sw_f32x4 *o = (sw_f32x4 *)(out + s * D + d);
    if (accumulate) {
        sw_f32x4 cur = *o;
#pragma unroll
        for (int c = 0; c < 4; c++) cur[c] = cur[c] + acc[c];
        *o = cur;
    } else {
        *o = acc;
    }
}
#endif

#define SW_WAVE 64

static inline int64_t sw_imin64(int64_t a, int64_t b) { return a < b ? a : b; }

// ---- work description for the grouped GEMMs ----
// A "group" is one expert applied to gcnt consecutive packed rows starting at
// gbeg; packed row j takes its activation from row grow[j] of the input planes
// (or row j itself when grow is null).
struct SwGroups {
    const int *gexp, *gbeg, *gcnt;   // [ngroups]; null gexp/gbeg mean 0, null gcnt means cnt_const
    const int *grow;                 // [T] or null
    const int *G;                    // device count (null: use ngroups_max)
    int ngroups_max;                 // grid extent: groups, or passes when items is set
    int cnt_const;
    // passes (optional): items[j] = (t0 << 10) | group of pass j, P = the device count;
    // a block then takes one pass of up to DG_TT tokens from t0 instead of a whole group
    const int *items;
    const int *P;
    int tt;                          // tokens per pass of the items (1 or 2; 0: SW_DG_TT)
};
#define SW_DG_TT 2             // tokens per weight pass of the grouped dot8 kernels
// route activations whose gate is a softmax of the logits (computed with the
// top-k): 1 moe_block's, 3 OLMoE's, 4 qwen35's; 0 sigmoid and 2 softplus come
// as scores from the router
__host__ __device__ inline bool sw_act_softmax(int act) { return act == 1 || act == 3 || act == 4; }
// the gates whose router scores are selected by moe_topk and weighted as moe_block's
// sigmoid (c/moe_block.h:115-122): sigmoid, softplus, sqrt(softplus)
__host__ __device__ inline bool sw_act_scores(int act) { return act == 0 || act == 2 || act == 5; }
// the Inkling engine's routing (c/inkling.c:1027-1043): sigmoid scores selected as moe_topk
// does, weights normalised over the K picks and the n_shared shared-expert gates
#define SW_ROUTE_INKLING 6
#define SW_ROUTE_ACT_MAX 6
// extra layout of the gate + top-k: src rows of ld logits/scores (E routed first); with
// ns > 0 (Inkling) the ns shared gates follow them, the weights end in * rs / sum over
// the K picks and those gates, and the gates' weights go to wsh (row stride wshld);
// the pick weights to w with row stride wld
struct SwGateOpt { int ld, ns; float rs; int wld; float *wsh; int wshld; };
// the upper bound of the passes of T packed rows in at most min(T, E) groups, tt tokens each
__host__ __device__ inline int sw_npass_max(int T, int E, int tt) { return (T + (T < E ? T : E) * (tt - 1)) / tt; }
#define SW_MF_TT 64               // the prefill MFMA kernels' largest token tile
// the MFMA tiles of a group of n tokens: ceil(n / 64) of them (as 64-token tiles), each
// of the same whole number of 16-token columns (80 tokens: 48 + 32, not 64 + 16 -- a
// tail column costs most of what a full tile's staging does)
__host__ __device__ inline int sw_mf_tile(int n) {
    const int nt = (n + SW_MF_TT - 1) / SW_MF_TT, ts = ((n + nt - 1) / nt + 15) / 16 * 16;
    return ts < SW_MF_TT ? ts : SW_MF_TT;
}
// the token step between the passes (items) of a group of n tokens listed with tt
// tokens each: tt, or the balanced MFMA tile for tt = SW_MF_TT (the same count of passes)
__host__ __device__ inline int sw_item_step(int n, int tt) { return tt == SW_MF_TT ? sw_mf_tile(n) : tt; }
// XCD-aware block order: launches deal consecutive block ids to the 8 XCDs in
// turn; work index w gives XCD k the contiguous range [k n/8, (k+1) n/8) of
// the first n = 8 floor(nb/8) blocks, so neighbouring work (the passes of one
// group over the same weight rows) shares an L2
__device__ __forceinline__ int sw_xcd_work(int b, int nb) {
    const int n8 = nb & ~7;
    return b < n8 ? (b & 7) * (n8 >> 3) + (b >> 3) : b;
}

// the work of grouped block bx: expert e, the group's first packed row beg and
// its tokens [t0, tend) -- one pass from the pass list, or the whole group
// (false: nothing to do)
// (cnt: the group's token count, when asked for)
__device__ __forceinline__ bool grp_work(const SwGroups &grp, int bx, int TT, int &e, int &beg, int &t0, int &tend,
                                         int *cnt = nullptr) {
    // (uniform over the block: read into scalar registers)
    auto u = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    if (grp.items) {
        if (bx >= u(*grp.P)) return false;
        const int v = u(grp.items[bx]), gi = v & 1023;
        t0 = v >> 10;
        e = u(grp.gexp[gi]);
        beg = u(grp.gbeg[gi]);
        const int n = u(grp.gcnt[gi]);
        tend = min(t0 + sw_item_step(n, TT), n);
        if (cnt) *cnt = n;
        return true;
    }
    const int gvalid = grp.G ? u(*grp.G) : grp.ngroups_max;
    if (bx >= gvalid) return false;
    e = grp.gexp ? u(grp.gexp[bx]) : 0;
    beg = grp.gbeg ? u(grp.gbeg[bx]) : 0;
    t0 = 0;
    tend = grp.gcnt ? u(grp.gcnt[bx]) : grp.cnt_const;
    if (cnt) *cnt = tend;
    return true;
}
template <int N>
struct SwIc { static constexpr int v = N; };

// int4 weight tensor of E experts, O rows each, K inputs
struct SwQ4 {
    const uint8_t *q;     // [E*O, K/2]
    const float *s;       // [E*O, ng]
    int O, K, gs;         // gs = 0: per-row scale
    int E;                // experts in the tensor (the extent of its buffer descriptors)
};
// The int4 tensors are read through buffer descriptors over all E experts
// (extent E * O * K/2 bytes, and E * O * ng * 4 for the scales).
static inline bool sw_q4_extent_ok(const SwQ4 &W) {
    const int ng = W.gs > 0 ? W.K / W.gs : 1;
    return W.E > 0 && (uint64_t)W.E * W.O * (W.K / 2) < (1ull << 32) && (uint64_t)W.E * W.O * ng * 4 < (1ull << 32);
}
// One group's expert as three separate int4 tensors (the coli table's gate, up and
// down ColiCudaTensor, c/backend_cuda.cu:785-943): a group's rows address these
// instead of expert e of one [E*O] tensor.  Scales are [rows][ng] as in SwQ4.
struct SwTab {
    const uint8_t *g, *u, *d;
    const float *gs, *us, *ds;
};
__device__ __forceinline__ sw_rsrc sw_q4_rq(const SwQ4 &W) { return sw_make_rsrc(W.q, (uint32_t)W.E * W.O * (W.K / 2)); }
__device__ __forceinline__ sw_rsrc sw_q4_rs(const SwQ4 &W) {
    const int ng = W.gs > 0 ? W.K / W.gs : 1;
    return sw_make_rsrc(W.s, (uint32_t)W.E * W.O * ng * 4);
}
// scale groups of gs inputs (a power of two, a multiple of 32): group of
// input k is k >> gsh; gs <= 0 means one scale per row
static inline int sw_q4_gsh(const SwQ4 &W, int &gsh) {
    gsh = 0;
    if (W.gs > 0) {
        if (W.gs % 32 || W.K % W.gs || (W.gs & (W.gs - 1))) return -1;
        while ((1 << gsh) < W.gs) gsh++;
    }
    return 0;
}

// ---- kernels (launch wrappers, all async on `st`) ----
// router logits [S,E] (exact 16-lane FMA-chain contract; Wc chain-major), the
// sigmoid / softplus scores [S,E] next to them, with xl non-null the dot8
// limbs of x (xl, xs as sw_launch_limbs), and, with sel non-null, gate +
// top-k per token (a second kernel; softmax is computed there)
int sw_launch_router_topk(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                          const float *logit_bias, float *logits, float *scores, int K, int route_act,
                          const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w,
                          sw_u32x4 *xl, float *xs, const SwGateOpt *opt = nullptr);
// the router logits and scores alone (no limbs, no top-k) over tiles of tokens: one
// pass over the weights per tile, the same bits as sw_launch_router_topk; D % 256 == 0
int sw_launch_router_tiles(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                           const float *logit_bias, float *logits, float *scores, int route_act);
// gate + top-k of S tokens from their logits (act 1) or scores (one wave each)
int sw_launch_gate_topk(hipStream_t st, const float *logits, const float *scores, int S, int E, int K, int route_act,
                        const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w,
                        const SwGateOpt *opt = nullptr);
// counting sort by expert; with items non-null also the pass list of tt tokens (SwGroups)
// the gate + top-k and the bucketing of a batch of up to 32 tokens in one launch (the
// arguments of sw_launch_gate_topk, then those of sw_launch_bucket)
int sw_launch_gate_bucket(hipStream_t st, const float *logits, const float *scores, int S, int E, int K, int route_act,
                          const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w,
                          const SwGateOpt *opt, int *gexp, int *gbeg, int *gcnt, int *G, int *grow, int *rowof, int tt,
                          int *items, int *P);
// (hist: scratch of ceil(S K / 2048) * E ints for a sort split over blocks, or null for one
// block)
int sw_launch_bucket(hipStream_t st, const int *sel, int S, int K, int E, int *gexp, int *gbeg,
                     int *gcnt, int *G, int *grow, int *rowof, int tt, int *items, int *P, int *hist = nullptr);
// the reference CPU's 16-lane GEMV contracts (k_lanes.hip), bit for bit: wkind 0 bf16,
// 1 int8 (+ row scale), 2 per-row int4 (+ row scale), 3 group-scaled int4 (+ scales
// [O][I/gs], matmul_i4_grouped's lanes; gs a multiple of 16 dividing 256, or of 256);
// dp: bf16-rounded activations through the
// vdpbf16ps lane order
int sw_launch_lanes16(hipStream_t st, const void *W, int wkind, int dp, const float *scale, const float *x, int S,
                      int I, int O, float *y, int gs);
// the same with row strides: x row s at x + s*ldx, y row s at y + s*ldy
int sw_launch_lanes16_ld(hipStream_t st, const void *W, int wkind, int dp, const float *scale, const float *x, int ldx,
                         int S, int I, int O, float *y, int ldy, int gs);
// h[i] = siluf(g[i]) * u[i] with the glibc-exact expf (c/moe_math.h:53)
int sw_launch_silu_mul(hipStream_t st, const float *g, const float *u, int64_t n, float *h);
// activation limbs for the dot8 GEMV (k_dot8.hip): rows x[rows, K] f32 ->
// xl[rows][K/32][SW_NL] (32 signed nibbles each), xs[rows][K/32] f32.  An input's
// integer D is defined by SW_ND base-8 digits (limbs_group, sw_gate.h) and stored as
// SW_NL balanced base-16 digits
#define SW_ND 7
#define SW_NL 6
int sw_launch_limbs(hipStream_t st, const float *x, int rows, int K, sw_u32x4 *xl, float *xs);
// SiLU-GLU(gate, up) for every packed row of every group, on the dot8 unit;
// output h as limbs hl[packed row][I/32][SW_NL], hs[packed row][I/32]
int sw_launch_q4_dot8_glu(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, int I,
                          sw_u32x4 *hl, float *hs);
// the same for one token's K picks sel (block row a: expert sel[a], packed row a)
int sw_launch_q4_dot8_glu_picks(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, int I, sw_u32x4 *hl, float *hs,
                                const int *sel, int K);
// Y[packed row, O] f32 for every group, input as limbs (the grouped down projection);
// O a multiple of 64
int sw_launch_q4_dot8_rows(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, float *Y);
// the same two grouped kernels over per-group tensors: W gives O, K and gs (its q, s
// and E are unused); group c's tensors are tab[gexp[c]]
int sw_launch_q4_dot8_glu_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const sw_u32x4 *xl, const float *xs, SwGroups g,
                              int I, sw_u32x4 *hl, float *hs, int one_row);
int sw_launch_q4_dot8_rows_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const sw_u32x4 *xl, const float *xs, SwGroups g,
                               float *Y);
// the dot8 down projection fused with the rank-order combine for one token
// (h as limbs of the K packed rows in rank order)
// (wsh non-null: ns gated shared outputs shared[ns][D], added after the ranks as
// fma(wsh[j], shared[j], acc), Inkling's pass 3; route_scale 1)
int sw_launch_q4_dot8_down_combine(hipStream_t st, SwQ4 W, const sw_u32x4 *hl, const float *hs, const int *sel, const float *w,
                                   int K, float route_scale, const float *shared, float *out,
                                   const float *wsh = nullptr, int ns = 0);
// the int4 down projection fused with the rank-order combine for one token:
// out[d] += (sum_a w[a] * down_{sel[a]}(h_a)[d]) * route_scale (+ shared[d])
// out[s] (+)= route_scale * sum_a w[s,a] * slots[rowof[s,a]] (+ shared[s])
// (wsh non-null: shared [S][ns][D] gated by wsh [S][ns] after the ranks, as above)
// the shared expert's down of h's parts hp fused with the combine (accumulating into
// out, shared [S][D] its scratch): decode-sized batches (k_shared.hip)
int sw_launch_sh_combine(hipStream_t st, const uint16_t *Wd, const uint16_t *hp, int S, int Is, int D, float *shared,
                         const float *slots, const int *rowof, const float *w, int K, float route_scale, float *out);
int sw_launch_combine(hipStream_t st, const float *slots, const int *rowof, const float *w, int S, int K, int D,
                      float route_scale, const float *shared, float *out, int accumulate,
                      const float *wsh = nullptr, int ns = 0);
// fused decode stages (k_dot8.hip): stage 1 = router logits/scores/limbs
// and the shared expert's gate_up (sg null: none; one token's h to sh_h, or a
// batch's split-K blocks writing h's parts to sh_hp), with xp non-null also the
// bf16 parts of x (sw_shared.h); with nw the rows of x are raw and the router
// blocks apply the RMSNorm (weights nw, eps) as they stage them, writing the
// normalised rows to xn (no shared expert then); stage 2 = routed gate_up (sel non-null: one
// token's K picks, from sel or, with route_src, by a gate + top-k in every
// block; else the groups g) + the shared expert's down (sd null: none; from
// one token's h in sh_h, or a batch's from h's parts in sh_hp) or a batch's
// shared gate_up (sg, su over x; h's parts to sh_hp)
int sw_launch_stage_route(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                          const float *logit_bias, float *logits, float *scores, int route_act, sw_u32x4 *xl, float *xs,
                          const uint16_t *sg, const uint16_t *su, int Is, float *sh_h, uint16_t *xp = nullptr,
                          uint16_t *sh_hp = nullptr, const float *nw = nullptr, float eps = 0.f, float *xn = nullptr);
int sw_launch_stage_experts(hipStream_t st, SwQ4 W, const sw_u32x4 *xl, const float *xs, SwGroups g, int I, sw_u32x4 *hl,
                            float *hs, int *sel, int K, const float *route_src, int E, int act, const float *bias,
                            int use_bias, int norm, float *w, const uint16_t *sd, const float *sh_h, int S, int Is, int D,
                            float *sh_out, uint16_t *sh_hp = nullptr, const uint16_t *sg = nullptr,
                            const uint16_t *su = nullptr, const float *x = nullptr);
// the shared expert on the VALU (sw_shared.h): h[S, Is] = silu(Wg x) * (Wu x)
// and out[S, D] = Wd h, bf16 weights, f32 activations
// stack glue (k_glue.hip): RMSNorm rows, greedy argmax rows
// prefill expert GEMMs on the f16 MFMA (k_mfma.hip), bit-identical to the
// dot8 ones: activations as MFMA digits dg[rows][K/32][32 dwords] + factors
// xs[rows][K/32] (the limbs' exponent and integer, recut); tiles of up to 64
// tokens of a group listed in g.items / g.P (sw_launch_bucket with tt = SW_MF_TT)
#define SW_MF_DIGIT_BYTES 128     // MFMA digits of one (row, input group): 32 dwords
int sw_launch_digits(hipStream_t st, const float *x, int rows, int K, uint32_t *dg, float *xs);
// (dg_rows: the rows of dg and xs; dg_rows * K * 4 must stay below 2^32)
int sw_launch_mf_glu(hipStream_t st, SwQ4 W, const uint32_t *dg, const float *xs, int dg_rows, SwGroups g, int I,
                     uint32_t *hdg, float *hxs);
int sw_launch_mf_rows(hipStream_t st, SwQ4 W, const uint32_t *dg, const float *xs, int dg_rows, SwGroups g, float *Y);
int sw_launch_mf_glu_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const uint32_t *dg, const float *xs, int dg_rows,
                         SwGroups g, int I, uint32_t *hdg, float *hxs);
int sw_launch_mf_rows_tab(hipStream_t st, SwQ4 W, const SwTab *tab, const uint32_t *dg, const float *xs, int dg_rows,
                          SwGroups g, float *Y);
// the reference's IDOT int4 contract (k_idot.hip, per-row scales): int8 activations
// per 32-block xi[rows][K/32][8 dwords] + xs[rows][K/32], then grouped rows (whole groups)
int sw_launch_idot_quant(hipStream_t st, const float *x, int rows, int K, uint32_t *xi, float *xs);
int sw_launch_idot_glu(hipStream_t st, SwQ4 W, const uint32_t *xi, const float *xs, SwGroups g, int I, float *h);
int sw_launch_idot_rows(hipStream_t st, SwQ4 W, const uint32_t *xi, const float *xs, SwGroups g, float *Y);
int sw_launch_rmsnorm(hipStream_t st, const float *x, const float *w, float *out, int S, int D, float eps);
int sw_launch_argmax(hipStream_t st, const float *logits, int S, int V, int *tok);
// the shared expert of a batch on the bf16 MFMA (k_shared.hip): the three bf16 parts of
// rows of x ([S][K/32][3][32]); h = silu(Wg x) * (Wu x) as its parts; out = Wd h (f32)
int sw_launch_sh_parts(hipStream_t st, const float *x, int S, int K, uint16_t *parts);
int sw_launch_sh_glu(hipStream_t st, const uint16_t *Wg, const uint16_t *Wu, const uint16_t *xp, int S, int D, int Is,
                     uint16_t *hp);
int sw_launch_sh_down(hipStream_t st, const uint16_t *Wd, const uint16_t *hp, int S, int Is, int D, float *out);
// synthetic data
int sw_launch_gen_normal(hipStream_t st, float *out, int64_t n, uint64_t seed, uint64_t offset, double sigma, int to_bf16);
int sw_launch_gen_bf16(hipStream_t st, uint16_t *out, int64_t n, uint64_t seed, uint64_t offset, double sigma);
int sw_launch_gen_q4(hipStream_t st, uint8_t *q, float *s, uint64_t seed, double sigma, int64_t row0, int64_t nrows, int K, int gs);
int sw_launch_chain_major(hipStream_t st, const void *W, int w_bf16, int E, int D, void *Wc);
// self test kernels
int sw_launch_selftest(hipStream_t st, float *out, const float *xin, int n);

#endif
