// k_route.hip -- routing side of the MoE block on gfx950: activation planes,
// the router GEMV under the reference's exact FMA-chain contract, gate +
// top-k, the counting sort into expert groups, and the rank-order combine.
#include "sw_hip.h"
#include "sw_libm.h"
#include "sw_gate.h"

static int launch_err(void) { return hipGetLastError() == hipSuccess ? 0 : -1; }

// ------------------------------------------------------------ router ----
// Chain-major router copy: Wc[(e*16 + j)*M + m] = W[e*D + 16m + j], M = D/16,
// so lane j of expert e reads its FMA chain contiguously.
// The router in the order the routing kernel streams it (sw_router.h), in
// its own element type: experts in groups of 4, group g a run of 1 KB
// slices, slice q holding for each of the group's 64 chains c = 16*(e%4) + j
// (j = i%16) the next P elements m = Pq..Pq+P-1 (m = i/16) of that chain,
// P = 8 for bf16 and 4 for f32; experts past E in the last group are zero.
__global__ void k_chain_major(const void *__restrict__ W, int w_bf16, int E, int D, void *__restrict__ Wc) {
    const int P = w_bf16 ? 8 : 4, NQ = D / 16 / P;
    const int64_t n = (int64_t)((E + 3) / 4) * 4 * D;
    for (int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; o < n; o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t u = o % P, c = (o / P) & 63, q = (o / P / 64) % NQ, g = (o / P / 64) / NQ;
        const int64_t e = 4 * g + (c >> 4), j = c & 15, m = (int64_t)P * q + u, i = 16 * m + j;
        if (w_bf16) ((uint16_t *)Wc)[o] = e < E ? ((const uint16_t *)W)[e * D + i] : (uint16_t)0;
        else ((float *)Wc)[o] = e < E ? ((const float *)W)[e * D + i] : 0.f;
    }
}

int sw_launch_chain_major(hipStream_t st, const void *W, int w_bf16, int E, int D, void *Wc) {
    if (D % 128 || E <= 0) return -1;
    const int64_t n = (int64_t)((E + 3) / 4) * 4 * D;
    SW_LAUNCH(k_chain_major, dim3((unsigned)sw_imin64((n + 255) / 256, 8192)), dim3(256), 0, st, W, w_bf16, E, D, Wc);
    return launch_err();
}

// ------------------------------------------------------------ gate + top-k ----
// One wave per token (gate_topk_wave in sw_gate.h).
template <int NPER>   // expert slots per lane: E <= 64 * NPER
__global__ __launch_bounds__(64) void k_gate_topk(const float *__restrict__ logits, const float *__restrict__ scores,
                                                  int E, int K, int act, const float *__restrict__ bias, int use_bias,
                                                  int norm, int *__restrict__ sel_all, float *__restrict__ w_all,
                                                  SwGateOpt o) {
    __shared__ uint64_t tab[32];
    const int lane = threadIdx.x, s = blockIdx.x;
    int sk;
    float wk;
    gate_topk_wave<NPER>((sw_act_softmax(act) ? logits : scores) + (int64_t)s * o.ld, E, K, act, bias, use_bias, norm, tab,
                         sk, wk, o.ns, o.rs, o.wsh ? o.wsh + (int64_t)s * o.wshld : nullptr);
    if (lane < K) { sel_all[(int64_t)s * K + lane] = sk; w_all[(int64_t)s * o.wld + lane] = wk; }
}

#include "sw_router.h"

template <int BF16, int ONE>
__global__ __launch_bounds__(512) void k_router_logits(RouterArgs R) {
    extern __shared__ __align__(16) float smem[];
    router_block<BF16, ONE>(R, blockIdx.x, blockIdx.y, gridDim.x, smem);
}

// a 1-D grid of (expert block, token tile) pairs, dealt so that an XCD runs whole
// token tiles (all their expert blocks), whose x then comes from its L2
template <int BF16, int TT, int NW, int GPW>
__global__ __launch_bounds__(64 * NW) void k_router_tiles(RouterArgs R, int S, int nbx) {
    const int w = sw_xcd_work((int)blockIdx.x, (int)gridDim.x);
    router_tile_block<BF16, TT, NW, GPW>(R, S, w % nbx, w / nbx);
}

// token tile, waves per block and groups of 4 experts per wave.  bf16 weights: 8 waves of
// two groups each (64 experts per block sharing the tile's x in LDS; LDS reads per weight
// element halve against one group: C4 router 93 us against 111, C5 head 54 against 73), 16
// tokens for prefill-sized batches, else 8.  f32 weights keep one group per wave (two
// groups take 158-181 VGPRs): 16 tokens on 4 waves for prefill, else 8 tokens on 8 waves.
static void router_tile_shape(int S, int bf16, int &tt, int &nw, int &gpw) {
    tt = S >= 512 ? 16 : 8;
    nw = bf16 || S < 512 ? 8 : 4;
    gpw = bf16 ? 2 : 1;
}

int sw_launch_router_tiles(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                           const float *logit_bias, float *logits, float *scores, int route_act) {
    if (D % RT_CK || D > 65536 || E <= 0 || S <= 0 || route_act < 0 || route_act > SW_ROUTE_ACT_MAX) return -1;
    if ((int64_t)((E + 3) / 4) * 4 * D * (w_bf16 ? 2 : 4) > 0xFFFFFFFFll) return -1;
    int tt, nw, gpw;
    router_tile_shape(S, w_bf16, tt, nw, gpw);
    const RouterArgs R = {Wc, x, D, E, logit_bias, logits, route_act, scores, nullptr, nullptr, nullptr};
    const int ng4 = (E + 3) / 4;
    const int nbx = (ng4 + nw * gpw - 1) / (nw * gpw);
    const dim3 grid((unsigned)((int64_t)nbx * ((S + tt - 1) / tt)));
#define SW_RT(B, T, W, G) SW_LAUNCH((k_router_tiles<B, T, W, G>), grid, dim3(64 * W), 0, st, R, S, nbx)
    if (w_bf16) {
        if (tt == 16) SW_RT(1, 16, 8, 2); else SW_RT(1, 8, 8, 2);
    } else {
        if (tt == 16) SW_RT(0, 16, 4, 1); else SW_RT(0, 8, 8, 1);
    }
#undef SW_RT
    return launch_err();
}

int sw_launch_router_topk(hipStream_t st, const void *Wc, int w_bf16, const float *x, int S, int D, int E,
                          const float *logit_bias, float *logits, float *scores, int K, int route_act,
                          const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w,
                          sw_u32x4 *xl, float *xs, const SwGateOpt *opt) {
    if (D % 128 || D > 16384 || E <= 0 || S <= 0) return -1;
    // (logits only: any number of rows; with Inkling's ns shared gates the router has E + ns)
    const int ns = opt ? opt->ns : 0;
    if (sel && (E > TK_MAXE || K <= 0 || K > 64 || K > E)) return -1;
    E += ns;
    if (route_act < 0 || route_act > SW_ROUTE_ACT_MAX || (sel && !sw_act_softmax(route_act) && !scores)) return -1;
    // four experts per block (wave 0; the others stage x) while that stays within 256 blocks,
    // else four per wave of eight
    const int nt = 512, one = router_one(S, E), epb = router_epb(one, nt);
    if (router_lds(D) > 65536 || D > 4 * RT_XB * (one ? nt - 64 : nt)) return -1;
    dim3 grid((unsigned)((E + epb - 1) / epb), (unsigned)S);
    const RouterArgs R = {Wc, x, D, E, logit_bias, logits, route_act, scores, xl, xs, nullptr};
    if (one) {
        if (w_bf16) SW_LAUNCH((k_router_logits<1, 1>), grid, dim3(nt), router_lds(D), st, R);
        else SW_LAUNCH((k_router_logits<0, 1>), grid, dim3(nt), router_lds(D), st, R);
    } else {
        if (w_bf16) SW_LAUNCH((k_router_logits<1, 0>), grid, dim3(nt), router_lds(D), st, R);
        else SW_LAUNCH((k_router_logits<0, 0>), grid, dim3(nt), router_lds(D), st, R);
    }
    if (launch_err()) return -1;
    if (!sel) return 0;                              // logits only
    return sw_launch_gate_topk(st, logits, scores, S, E - ns, K, route_act, corr_bias, use_corr_bias, norm_topk, sel, w, opt);
}

int sw_launch_gate_topk(hipStream_t st, const float *logits, const float *scores, int S, int E, int K, int route_act,
                        const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w, const SwGateOpt *opt) {
    if (E <= 0 || E > TK_MAXE || S <= 0 || K <= 0 || K > 64 || K > E || route_act < 0 || route_act > SW_ROUTE_ACT_MAX) return -1;
    if (!sw_act_softmax(route_act) && !scores) return -1;
    const SwGateOpt o = opt ? *opt : SwGateOpt{E, 0, 1.f, K, nullptr, 0};
    if (o.ld < E + o.ns || o.wld < K || o.ns < 0 || o.ns > 64 || (o.ns && route_act != SW_ROUTE_INKLING)) return -1;
    const int nper = (E + 63) / 64;
#define SW_GATE(NP) SW_LAUNCH(k_gate_topk<NP>, dim3((unsigned)S), dim3(64), 0, st, logits, scores, E, K, route_act, \
                                       corr_bias, use_corr_bias, norm_topk, sel, w, o)
    if (nper <= 1) SW_GATE(1);
    else if (nper <= 2) SW_GATE(2);
    else if (nper <= 4) SW_GATE(4);
    else if (nper <= 8) SW_GATE(8);
    else SW_GATE(16);
#undef SW_GATE
    return launch_err();
}

// ------------------------------------------------------------ bucketing ----
// The counting sort of lag_moe_group (c/laguna.c:708-727) on the device:
// groups in ascending expert id, packed rows stable in (token, rank) order.
// One block of 1024 threads; pairs are taken 1024 at a time in order, and a
// pair's rank among earlier pairs of its expert comes from per-wave ballot
// match masks plus per-wave counts of the earlier waves (a wave holds at most
// 64 pairs of an expert, so each count is one byte: 16 KB for 1024 experts).
#define BK_THREADS 1024
#define BK_MAXE 1024
struct BucketArgs {
    int *gexp, *gbeg, *gcnt, *Gout, *grow, *rowof;
    int tt;
    int *items, *Pout;
};
// The parts of the sort, each by a block of BK_THREADS threads.
// (1) cnt[e] += the picks of expert e among sel[p0 .. p1)
__device__ __forceinline__ void bucket_count(const int *__restrict__ sel, int p0, int p1, int *cnt) {
    const int tid = threadIdx.x;
    // eight picks' loads in flight per thread before their atomics (one load latency per 8
    // BK_THREADS picks instead of one per BK_THREADS)
    for (int q0 = p0 + tid; q0 < p1; q0 += 8 * BK_THREADS) {
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = q0 + u * BK_THREADS < p1 ? sel[q0 + u * BK_THREADS] : 0;
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (q0 + u * BK_THREADS < p1) atomicAdd(&cnt[v[u]], 1);
    }
}
// (2) from the experts' counts: run[e] = the first packed row of expert e; with write, the
// group and pass tables.  Inclusive scans of cnt (packed offsets), of cnt > 0 (group index)
// and of the passes (pass list offsets), expert tid by thread tid: a shuffle scan within each
// wave, then the totals of the earlier waves (integer sums, so the order of the additions
// does not matter).
__device__ __forceinline__ void bucket_tables(const int *cnt, int E, const BucketArgs &B, bool write, int *run) {
    __shared__ int sa[BK_MAXE], sb[BK_MAXE], sp[BK_MAXE];
    __shared__ int wta[BK_THREADS / 64], wtb[BK_THREADS / 64], wtp[BK_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, tt = B.tt;
    {
        const int c0 = tid < E ? cnt[tid] : 0;
        int va = c0, vb = c0 > 0, vp = (c0 + tt - 1) / tt;
        for (int o = 1; o < 64; o <<= 1) {
            const int ta = __shfl_up(va, o), tb = __shfl_up(vb, o), tp = __shfl_up(vp, o);
            if (lane >= o) { va += ta; vb += tb; vp += tp; }
        }
        if (lane == 63) { wta[wave] = va; wtb[wave] = vb; wtp[wave] = vp; }
        __syncthreads();
        for (int w = 0; w < wave; w++) { va += wta[w]; vb += wtb[w]; vp += wtp[w]; }
        if (tid < E) { sa[tid] = va; sb[tid] = vb; sp[tid] = vp; }
    }
    if (tid < E) {
        const int c = cnt[tid];
        const int offx = sa[tid] - c, gi = sb[tid] - (c > 0);
        run[tid] = offx;
        if (write) {
            if (c > 0) { B.gexp[gi] = tid; B.gbeg[gi] = offx; B.gcnt[gi] = c; }
            if (tid == E - 1) *B.Gout = sb[tid];
            if (B.items) {
                const int np = (c + tt - 1) / tt, p0 = sp[tid] - np, ts = sw_item_step(c, tt);
                for (int k = 0; k < np; k++) B.items[p0 + k] = ((k * ts) << 10) | gi;
                if (tid == E - 1) *B.Pout = sp[tid];
            }
        }
    }
    __syncthreads();
}
// (3) the picks p0 .. p1 placed from run[] (advanced past them): rounds of two halves of
// BK_THREADS (pair base + h BK_THREADS + tid), three barriers a round: a pair's slot is its
// expert's run, plus its expert's pairs in the round's first half (for h = 1), in the earlier
// waves of its half, and in its wave before its lane -- the pairs' own order (stable).  (The
// next round's picks are loaded while a round runs.)
__device__ __forceinline__ void bucket_rounds(const int *__restrict__ sel, int p0, int p1, int K, int E,
                                              const BucketArgs &B, int *run) {
    __shared__ uint8_t wcnt[2][BK_THREADS / 64][BK_MAXE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int *__restrict__ grow = B.grow, *__restrict__ rowof = B.rowof;
    for (int i = tid; i < E; i += BK_THREADS)
        for (int w = 0; w < BK_THREADS / 64; w++) wcnt[0][w][i] = wcnt[1][w][i] = 0;
    __syncthreads();
    int nbits = 0;
    while ((1 << nbits) < E) nbits++;
    const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    auto pick = [&](int p) { return p < p1 ? sel[p] : 0; };
    int en[2] = {pick(p0 + tid), pick(p0 + BK_THREADS + tid)};
    for (int base = p0; base < p1; base += 2 * BK_THREADS) {
        const int nh = base + BK_THREADS < p1 ? 2 : 1;         // uniform over the block
        int e[2], rank[2];
        bool act[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            act[h] = h < nh && base + h * BK_THREADS + tid < p1;
            e[h] = act[h] ? en[h] : 0;
        }
        en[0] = pick(base + 2 * BK_THREADS + tid);
        en[1] = pick(base + 3 * BK_THREADS + tid);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            rank[h] = 0;
            if (h < nh) {
                unsigned long long peers = __ballot(act[h]);
                for (int b = 0; b < nbits; b++) {
                    const unsigned long long m = __ballot(act[h] && ((e[h] >> b) & 1));
                    peers &= ((e[h] >> b) & 1) ? m : ~m;
                }
                rank[h] = __popcll(peers & lt);
                if (act[h] && rank[h] == 0) wcnt[h][wave][e[h]] = (uint8_t)__popcll(peers);
            }
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; h++) {
            if (act[h]) {
                const int p = base + h * BK_THREADS + tid;
                int pre = 0;
                if (h == 1)
                    for (int w = 0; w < BK_THREADS / 64; w++) pre += wcnt[0][w][e[h]];
                for (int w = 0; w < wave; w++) pre += wcnt[h][w][e[h]];
                const int slot = run[e[h]] + pre + rank[h];
                grow[slot] = p / K;
                rowof[p] = slot;
            }
        }
        __syncthreads();
        for (int i = tid; i < E; i += BK_THREADS) {
            int tot = 0;
            for (int h = 0; h < nh; h++)
                for (int w = 0; w < BK_THREADS / 64; w++) { tot += wcnt[h][w][i]; wcnt[h][w][i] = 0; }
            run[i] += tot;
        }
        __syncthreads();
    }
}
// the whole sort by one block
__device__ __forceinline__ void bucket_block(const int *__restrict__ sel, int T, int K, int E, const BucketArgs &B) {
    __shared__ int cnt[BK_MAXE], run[BK_MAXE];
    for (int i = threadIdx.x; i < E; i += BK_THREADS) cnt[i] = 0;
    __syncthreads();
    bucket_count(sel, 0, T, cnt);
    __syncthreads();
    bucket_tables(cnt, E, B, true, run);
    bucket_rounds(sel, 0, T, K, E, B, run);
}

// The same counting sort for at most 128 picks of at most 256 experts, by one wave and no
// block barrier: lane l holds picks l and 64 + l; a pick's rank among its expert's picks of
// its half from ballots over the id bits, after the first half's picks of that expert (the
// pairs' own order: stable); the experts' counts, groups and passes by wave scans over 4
// experts a lane (integer sums).  The same tables as bucket_block.
#define WB_MAXN 128
__device__ __forceinline__ void wave_bucket(const int *sel, int n, int K, int E, const BucketArgs &B) {
    __shared__ int wb_cnt[2][256], wb_off[256];
    const int lane = threadIdx.x & 63, tt = B.tt;
    for (int i = lane; i < 256; i += 64) wb_cnt[0][i] = wb_cnt[1][i] = 0;
    wave_sync();
    bool act[2];
    int ex[2], rank[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        act[h] = 64 * h + lane < n;
        ex[h] = act[h] ? sel[64 * h + lane] : 0;
        unsigned long long peers = __ballot(act[h]);
        for (int b = 0; b < 8; b++) {
            const unsigned long long m = __ballot(act[h] && ((ex[h] >> b) & 1));
            peers &= ((ex[h] >> b) & 1) ? m : ~m;
        }
        rank[h] = __popcll(peers & (lane ? ~0ull >> (64 - lane) : 0ull));
        if (act[h] && rank[h] == 0) wb_cnt[h][ex[h]] = __popcll(peers);
    }
    wave_sync();
    int c[4], sc = 0, sg = 0, sp = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        c[i] = wb_cnt[0][4 * lane + i] + wb_cnt[1][4 * lane + i];
        sc += c[i];
        sg += c[i] > 0;
        sp += (c[i] + tt - 1) / tt;
    }
    int ic = sc, ig = sg, ip = sp;
    for (int o = 1; o < 64; o <<= 1) {
        const int a = __shfl_up(ic, o), b = __shfl_up(ig, o), q = __shfl_up(ip, o);
        if (lane >= o) { ic += a; ig += b; ip += q; }
    }
    int xc = ic - sc, xg = ig - sg, xp = ip - sp;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e4 = 4 * lane + i, np = (c[i] + tt - 1) / tt;
        wb_off[e4] = xc;
        if (c[i] > 0) {
            B.gexp[xg] = e4;
            B.gbeg[xg] = xc;
            B.gcnt[xg] = c[i];
            if (B.items) {
                const int ts = sw_item_step(c[i], tt);
                for (int q = 0; q < np; q++) B.items[xp + q] = ((q * ts) << 10) | xg;
            }
        }
        xc += c[i];
        xg += c[i] > 0;
        xp += np;
    }
    if (lane == 63) {
        *B.Gout = ig;
        if (B.items) *B.Pout = ip;
    }
    wave_sync();
#pragma unroll
    for (int h = 0; h < 2; h++)
        if (act[h]) {
            const int p = 64 * h + lane, slot = wb_off[ex[h]] + (h ? wb_cnt[0][ex[h]] : 0) + rank[h];
            B.grow[slot] = p / K;
            B.rowof[p] = slot;
        }
}

__global__ __launch_bounds__(BK_THREADS) void k_bucket(const int *__restrict__ sel, int T, int K, int E, BucketArgs B) {
    bucket_block(sel, T, K, E, B);
}

// The same sort of many picks over blocks of BK_CHUNK picks each (one round apiece): the
// counts of every chunk, then every chunk placed from the experts' totals (the same scans,
// block 0 writing the tables) plus the earlier chunks' counts of each expert -- the pairs'
// own order over the chunks (C4's 20,480 picks: 40 -> 14 us)
#define BK_CHUNK (2 * BK_THREADS)
__global__ __launch_bounds__(BK_THREADS) void k_bucket_count(const int *__restrict__ sel, int T, int E,
                                                             int *__restrict__ hist) {
    __shared__ int cnt[BK_MAXE];
    for (int i = threadIdx.x; i < E; i += BK_THREADS) cnt[i] = 0;
    __syncthreads();
    const int p0 = (int)blockIdx.x * BK_CHUNK;
    bucket_count(sel, p0, min(T, p0 + BK_CHUNK), cnt);
    __syncthreads();
    for (int i = threadIdx.x; i < E; i += BK_THREADS) hist[(int64_t)blockIdx.x * E + i] = cnt[i];
}
__global__ __launch_bounds__(BK_THREADS) void k_bucket_scatter(const int *__restrict__ sel, int T, int K, int E,
                                                               const int *__restrict__ hist, BucketArgs B) {
    __shared__ int cnt[BK_MAXE], run[BK_MAXE], pre[BK_MAXE];
    const int b = (int)blockIdx.x, nb = (int)gridDim.x;
    for (int i = threadIdx.x; i < E; i += BK_THREADS) {
        int tot = 0, before = 0;
        for (int c = 0; c < nb; c++) {
            const int h = hist[(int64_t)c * E + i];
            tot += h;
            if (c < b) before += h;
        }
        cnt[i] = tot;
        pre[i] = before;
    }
    __syncthreads();
    bucket_tables(cnt, E, B, b == 0, run);
    for (int i = threadIdx.x; i < E; i += BK_THREADS) run[i] += pre[i];
    __syncthreads();
    const int p0 = b * BK_CHUNK;
    bucket_rounds(sel, p0, min(T, p0 + BK_CHUNK), K, E, B, run);
}

int sw_launch_bucket(hipStream_t st, const int *sel, int S, int K, int E, int *gexp, int *gbeg,
                     int *gcnt, int *G, int *grow, int *rowof, int tt, int *items, int *P, int *hist) {
    if (E <= 0 || E > BK_MAXE || S <= 0 || K <= 0 || tt <= 0 || (items && !P)) return -1;
    if ((int64_t)S * K >= (1 << 21)) return -1;      // pass offsets in 21 bits of an item
    const BucketArgs B = {gexp, gbeg, gcnt, G, grow, rowof, tt, items, P};
    const int T = S * K, nb = (T + BK_CHUNK - 1) / BK_CHUNK;
    if (hist && nb > 1) {
        SW_LAUNCH(k_bucket_count, dim3((unsigned)nb), dim3(BK_THREADS), 0, st, sel, T, E, hist);
        SW_LAUNCH(k_bucket_scatter, dim3((unsigned)nb), dim3(BK_THREADS), 0, st, sel, T, K, E, (const int *)hist, B);
    } else {
        SW_LAUNCH(k_bucket, dim3(1), dim3(BK_THREADS), 0, st, sel, T, K, E, B);
    }
    return launch_err();
}

// The gate + top-k of a batch of up to GB_MAXS tokens and the bucketing of its picks in
// one block: wave w takes tokens w, w + 16, ... (each as k_gate_topk's wave), the block
// barrier, then bucket_block over the picks -- one launch instead of two.
#define GB_MAXS 32
template <int NPER>
__global__ __launch_bounds__(BK_THREADS) void k_gate_bucket(const float *__restrict__ logits, const float *__restrict__ scores,
                                                            int S, int E, int K, int act, const float *__restrict__ bias,
                                                            int use_bias, int norm, int *__restrict__ sel_all,
                                                            float *__restrict__ w_all, SwGateOpt o, BucketArgs B) {
    __shared__ uint64_t tab[32];
    __shared__ int lsel[GB_MAXS * 64];                // the picks again, for the bucketing
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int s = wave; s < S; s += BK_THREADS / 64) {
        int sk;
        float wk;
        gate_topk_wave<NPER>((sw_act_softmax(act) ? logits : scores) + (int64_t)s * o.ld, E, K, act, bias, use_bias, norm,
                             tab, sk, wk, o.ns, o.rs, o.wsh ? o.wsh + (int64_t)s * o.wshld : nullptr);
        if (lane < K) {
            sel_all[(int64_t)s * K + lane] = sk;
            w_all[(int64_t)s * o.wld + lane] = wk;
            lsel[s * K + lane] = sk;
        }
    }
    __syncthreads();                                  // the block's picks are in LDS
    if (S * K <= WB_MAXN && E <= 256) {              // (C5's 64 picks: 9.2 -> 6.7 us, C2 B=8's 80: 8.8 -> 7.2 us)
        if (wave == 0) wave_bucket(lsel, S * K, K, E, B);
        return;
    }
    bucket_block(lsel, S * K, K, E, B);
}

int sw_launch_gate_bucket(hipStream_t st, const float *logits, const float *scores, int S, int E, int K, int route_act,
                          const float *corr_bias, int use_corr_bias, int norm_topk, int *sel, float *w,
                          const SwGateOpt *opt, int *gexp, int *gbeg, int *gcnt, int *G, int *grow, int *rowof, int tt,
                          int *items, int *P) {
    if (E <= 0 || E > TK_MAXE || E > BK_MAXE || S <= 0 || S > GB_MAXS || K <= 0 || K > 64 || K > E || route_act < 0 ||
        route_act > SW_ROUTE_ACT_MAX || tt <= 0 || (items && !P)) return -1;
    if (!sw_act_softmax(route_act) && !scores) return -1;
    const SwGateOpt o = opt ? *opt : SwGateOpt{E, 0, 1.f, K, nullptr, 0};
    if (o.ld < E + o.ns || o.wld < K || o.ns < 0 || o.ns > 64 || (o.ns && route_act != SW_ROUTE_INKLING)) return -1;
    const BucketArgs B = {gexp, gbeg, gcnt, G, grow, rowof, tt, items, P};
    const int nper = (E + 63) / 64;
#define SW_GB(NP) SW_LAUNCH(k_gate_bucket<NP>, dim3(1), dim3(BK_THREADS), 0, st, logits, scores, S, E, K, route_act, \
                                     corr_bias, use_corr_bias, norm_topk, sel, w, o, B)
    if (nper <= 1) SW_GB(1);
    else if (nper <= 2) SW_GB(2);
    else if (nper <= 4) SW_GB(4);
    else if (nper <= 8) SW_GB(8);
    else SW_GB(16);
#undef SW_GB
    return launch_err();
}

// ------------------------------------------------------------ combine ----
// every (token, 4 outputs) by combine4 (sw_hip.h); NTL: the slots with nontemporal loads,
// for slot arrays beyond the caches (C4, 335 MB: 78.5 -> 70.4 us; a decode batch's few MB,
// still in L2 from the down launch, read slower so: 13.3 -> 15.5 us at B = 32)
#define CB_NT_BYTES (64ll << 20)
template <int NTL>
__global__ void k_combine(const float *__restrict__ slots, const int *__restrict__ rowof, const float *__restrict__ w,
                          int S, int K, int D, float route_scale, const float *__restrict__ shared,
                          float *__restrict__ out, int accumulate, const float *__restrict__ wsh, int ns) {
    const int64_t n4 = (int64_t)S * (D / 4);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t s = i / (D / 4);
        const int d = (int)(i % (D / 4)) * 4;
        combine4<NTL>(slots, rowof, w, s, K, D, d, route_scale, shared, out, accumulate, wsh, ns);
    }
}

int sw_launch_combine(hipStream_t st, const float *slots, const int *rowof, const float *w, int S, int K, int D,
                      float route_scale, const float *shared, float *out, int accumulate, const float *wsh, int ns) {
    if (D % 4 || S <= 0 || (wsh && (!shared || ns <= 0))) return -1;
    const int64_t n4 = (int64_t)S * (D / 4);
    const dim3 grid((unsigned)sw_imin64((n4 + 255) / 256, 4096));
    if ((int64_t)S * K * D * 4 >= CB_NT_BYTES)
        SW_LAUNCH(k_combine<1>, grid, dim3(256), 0, st, slots, rowof, w, S, K, D, route_scale, shared, out, accumulate,
                  wsh, ns);
    else
        SW_LAUNCH(k_combine<0>, grid, dim3(256), 0, st, slots, rowof, w, S, K, D, route_scale, shared, out, accumulate,
                  wsh, ns);
    return launch_err();
}

// ------------------------------------------------------------ self test ----
// MFMA lane-layout probe: A[i][k] = 32 i + k, B[k][j] = (k == j), so
// C[i][j] = 32 i + j under the layout in sw_hip.h; the int8 MFMA on fixed
// byte patterns (lane l byte b of A: (7 l + 13 b) % 17 - 8, of B:
// (5 l + 3 b + 1) % 23 - 11), whose C shows which A and B bytes meet; plus
// glibc-exact libm on host-chosen inputs.  out: [0,256) f16 MFMA C per lane
// (4 each), [256,512) bf16 MFMA, [512,768) i8 MFMA, [768, 768+n)
// sw_expf(xin), [768+n, 768+2n) sw_log1pf(xin), [768+2n, 768+3n) sw_sqrt_rn(xin).
#define ST_LIBM 768
__global__ void k_selftest_mfma(float *out) {
    const int l = threadIdx.x;
    sw_half8 a, b;
    sw_bf16x8 ab, bb;
    for (int h = 0; h < 8; h++) {
        const int k = 8 * (l >> 4) + h;
        const int i = l & 15;
        a[h] = (_Float16)(float)(32 * i + k);
        b[h] = (_Float16)(k == (l & 15) ? 1.0f : 0.0f);
        ab[h] = (__bf16)(float)(i * 2 + (k & 1));
        bb[h] = (__bf16)(k == (l & 15) ? 1.0f : 0.0f);
    }
    sw_f32x4 c = {0.f, 0.f, 0.f, 0.f}, c2 = {0.f, 0.f, 0.f, 0.f};
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, bb, c2, 0, 0, 0);
    for (int j = 0; j < 4; j++) { out[l * 4 + j] = c[j]; out[256 + l * 4 + j] = c2[j]; }
    sw_i32x4 ai, bi, ci = {0, 0, 0, 0};
    for (int d = 0; d < 4; d++) {
        uint32_t wa = 0, wb = 0;
        for (int q = 0; q < 4; q++) {
            const int b = 4 * d + q;
            wa |= (uint32_t)(uint8_t)(int8_t)((7 * l + 13 * b) % 17 - 8) << (8 * q);
            wb |= (uint32_t)(uint8_t)(int8_t)((5 * l + 3 * b + 1) % 23 - 11) << (8 * q);
        }
        ai[d] = (int)wa;
        bi[d] = (int)wb;
    }
    ci = __builtin_amdgcn_mfma_i32_16x16x64_i8(ai, bi, ci, 0, 0, 0);
    for (int j = 0; j < 4; j++) out[512 + l * 4 + j] = (float)ci[j];
}

__global__ void k_selftest_libm(float *out, const float *xin, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        out[ST_LIBM + i] = sw_expf(xin[i]);
        out[ST_LIBM + n + i] = sw_log1pf(xin[i]);
        out[ST_LIBM + 2 * n + i] = sw_sqrt_rn(xin[i]);
    }
}

int sw_launch_selftest(hipStream_t st, float *out, const float *xin, int n) {
    SW_LAUNCH(k_selftest_mfma, dim3(1), dim3(64), 0, st, out);
    if (n > 0) SW_LAUNCH(k_selftest_libm, dim3((unsigned)sw_imin64((n + 255) / 256, 4096)), dim3(256), 0, st, out, xin, n);
    return launch_err();
}
