// coli_hip.hip -- the GLM engine's coli_cuda_* table (c/backend_cuda.h:28-169) on
// gfx950: include/sabrewing_coli.h.
//
// Replaces c/backend_cuda.cu's host code for the MoE slots.  Process model: a
// context per configured device (stream, grow-only scratch, pinned staging,
// statistics), 1 ok / 0 fail everywhere, a failed HIP call logged and its
// sticky error consumed (c/backend_cuda.cu:63-69), COLI_GPU_FAIL_AFTER=N
// failing every compute entry after N calls (c/backend_cuda.cu:667-677).
//
// Different inside: a whole expert group is four launches whatever its count
// (limbs of x, gate/up + SiLU-GLU over every group, down over every group),
// the int4 bytes stay as stored (the signed-nibble XOR happens in registers),
// and each group reads its three tensors through a per-group table, so the
// projections are the dot8 kernels of the lag family, with their numerics.
#include "sw_hip.h"
#include "sw_libm.h"
#include "../../include/sabrewing_coli.h"
#include <mutex>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

struct ColiHipTensor {
    void *w;
    float *s;
    int fmt, I, O, device, gs, ng;
    size_t wbytes, sbytes;
};

namespace {

int ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return 1;
    fprintf(stderr, "[sabrewing-coli] %s: %s\n", what, hipGetErrorString(e));
    (void)hipGetLastError();
    return 0;
}

long g_calls = 0;
std::mutex g_calls_mu;
int fault_injected() {
    const char *fa = getenv("COLI_GPU_FAIL_AFTER");
    if (!fa) return 0;
    std::lock_guard<std::mutex> lk(g_calls_mu);
    return g_calls++ >= atol(fa);
}

struct DBuf { void *p = nullptr; size_t cap = 0; };
struct Ctx {
    int device = -1;
    hipStream_t st = nullptr;
    DBuf arena;                    // per-call scratch of the synchronous entries and issue
    DBuf res;                      // resident-issue scratch
    DBuf rout;                     // router scratch
    DBuf pipe[27];
    void *hin = nullptr, *hout = nullptr, *hiss_in = nullptr, *hiss_out = nullptr, *hres = nullptr, *hrout = nullptr;
    size_t hin_cap = 0, hout_cap = 0, hiss_in_cap = 0, hiss_out_cap = 0, hres_cap = 0;
    int pending = 0;
    hipEvent_t ev_done = nullptr, ev_res = nullptr;    // resident issue done; its meta copied
    int ev_done_ok = 0, ev_res_live = 0;
    hipEvent_t prof[4] = {};
    size_t tensor_count = 0, tensor_bytes = 0;
};
Ctx g_ctx[COLI_HIP_MAX_DEVICES];
std::mutex g_mu[COLI_HIP_MAX_DEVICES];
int g_nctx = 0;
std::mutex g_stats_mu;
uint64_t g_gcalls = 0, g_gexperts = 0, g_grows = 0;
double g_h2d = 0, g_kern = 0, g_d2h = 0;

Ctx *find_ctx(int device) {
    for (int i = 0; i < g_nctx; i++)
        if (g_ctx[i].device == device) return &g_ctx[i];
    return nullptr;
}
std::mutex &mu_of(Ctx *c) { return g_mu[c - g_ctx]; }
thread_local int t_current = -1;
int select_ctx(Ctx *c) {
    if (!c) return 0;
    if (t_current == c->device) return 1;
    if (!ok(hipSetDevice(c->device), "select device")) return 0;
    t_current = c->device;
    return 1;
}
// grow-only device scratch; the stream is drained before a buffer it may still read is freed
int grow(Ctx *c, DBuf &b, size_t need) {
    if (need <= b.cap) return 1;
    if (b.p) {
        if (!ok(hipStreamSynchronize(c->st), "scratch drain")) return 0;
        (void)hipFree(b.p);
    }
    b.p = nullptr;
    b.cap = 0;
    if (!ok(hipMalloc(&b.p, need * 2), "scratch allocation")) return 0;
    b.cap = need * 2;
    return 1;
}
int grow_pinned(Ctx *c, void *&p, size_t &cap, size_t need) {
    if (need <= cap) return 1;
    if (p) {
        if (!ok(hipStreamSynchronize(c->st), "staging drain")) return 0;
        (void)hipHostFree(p);
    }
    p = nullptr;
    cap = 0;
    if (!ok(hipHostMalloc(&p, need * 2, hipHostMallocDefault), "pinned staging allocation")) return 0;
    cap = need * 2;
    return 1;
}
struct Carve {
    size_t off = 0;
    size_t take(size_t n) { size_t o = (off + 255) & ~(size_t)255; off = o + n; return o; }
};

// ---- tensors ----
bool shape_ok(int fmt, int I, int O, int gs) {
    if ((fmt != 2 && fmt != 4) || I < 32 || O < 1 || I % 32 || I > 8192) return false;
    if (fmt == 4) return gs >= 32 && !(gs & (gs - 1)) && I % gs == 0;
    return true;
}

// ---- one call's groups ----
struct Groups {
    int device = -1, D = 0, I = 0, gs_gu = 0, gs_d = 0, total = 0, count = 0;
    std::vector<SwTab> tab;
    std::vector<int> beg, cnt;
};
// the reference's checks (c/backend_cuda.cu:788-808), plus one scale layout for all
// gates and ups and one for all downs (the kernels take gs per launch)
int collect(ColiHipTensor *const *gates, ColiHipTensor *const *ups, ColiHipTensor *const *downs, const int *rows,
            int count, Groups &G) {
    if (!gates || !ups || !downs || count < 1 || count > 64 || !gates[0]) return 0;
    const ColiHipTensor *f = gates[0];
    G.device = f->device; G.D = f->I; G.I = f->O; G.count = count;
    G.gs_gu = f->gs;
    G.gs_d = downs[0] ? downs[0]->gs : 0;
    G.tab.resize(count); G.beg.resize(count); G.cnt.resize(count);
    for (int c = 0; c < count; c++) {
        const ColiHipTensor *g = gates[c], *u = ups[c], *d = downs[c];
        const int r = rows ? rows[c] : 1;
        if (!g || !u || !d || r < 1 || g->device != G.device || u->device != G.device || d->device != G.device ||
            g->I != G.D || u->I != G.D || g->O != G.I || u->O != G.I || d->I != G.I || d->O != G.D)
            return 0;
        if (g->gs != G.gs_gu || u->gs != G.gs_gu || d->gs != G.gs_d) return 0;
        G.tab[c] = SwTab{(const uint8_t *)g->w, (const uint8_t *)u->w, (const uint8_t *)d->w, g->s, u->s, d->s};
        G.beg[c] = G.total;
        G.cnt[c] = r;
        G.total += r;
    }
    return 1;
}

// device scratch of a group call over T rows: x | gexp gbeg gcnt grow/items | tab |
// limbs (dot8) or digits (MFMA) of x and of h, with their factors | y
struct GLay { size_t x, ints, tab, xl, xs, hl, hs, y, end; };
// (T rows through the projections, xrows rows of x, ints: 3 per group + nextra)
GLay glay(const Groups &G, int T, int xrows, int nextra = 0, bool mf = false) {
    Carve cv;
    GLay L;
    const size_t per_group = mf ? (size_t)SW_MF_DIGIT_BYTES : (size_t)SW_NL * 16;
    L.x = cv.take((size_t)xrows * G.D * 4);
    L.ints = cv.take((size_t)(3 * G.count + nextra) * 4);
    L.tab = cv.take((size_t)G.count * sizeof(SwTab));
    L.xl = cv.take((size_t)xrows * (G.D / 32) * per_group);
    L.xs = cv.take((size_t)xrows * (G.D / 32) * 4);
    L.hl = cv.take((size_t)T * (G.I / 32) * per_group);
    L.hs = cv.take((size_t)T * (G.I / 32) * 4);
    L.y = cv.take((size_t)T * G.D * 4);
    L.end = cv.off;
    return L;
}
// the f16 MFMA GEMMs for prefill-sized groups (16-token tiles mostly full), as
// the lag family's automatic choice: whole chunks of 4 input groups, >= 8 rows per group
bool use_mf(const Groups &G) { return G.D % 128 == 0 && G.I % 128 == 0 && G.total >= 8 * G.count; }
size_t meta_bytes(const Groups &G, int T) { return (size_t)(3 * G.count + T) * 4 + (size_t)G.count * sizeof(SwTab); }
// the host image of the ints and the table: gexp = 0..count-1 (the table index),
// gbeg, gcnt, grow (or nothing), then the table
void pack_meta(const Groups &G, const int *grow, int T, char *dst) {
    int *h = (int *)dst;
    for (int c = 0; c < G.count; c++) { h[c] = c; h[G.count + c] = G.beg[c]; h[2 * G.count + c] = G.cnt[c]; }
    if (grow) memcpy(h + 3 * G.count, grow, (size_t)T * 4);
    memcpy(dst + (size_t)(3 * G.count + T) * 4, G.tab.data(), (size_t)G.count * sizeof(SwTab));
}

// the four launches: limbs of xrows rows, gate/up + GLU, down -> y [T][D]
int launch_group(Ctx *c, const Groups &G, char *A, const GLay &L, int T, int xrows, bool with_grow) {
    const int *d = (const int *)(A + L.ints);
    const SwTab *tab = (const SwTab *)(A + L.tab);
    sw_u32x4 *xl = (sw_u32x4 *)(A + L.xl), *hl = (sw_u32x4 *)(A + L.hl);
    float *xs = (float *)(A + L.xs), *hs = (float *)(A + L.hs);
    SwGroups g = {d, d + G.count, d + 2 * G.count, with_grow ? d + 3 * G.count : nullptr, nullptr, G.count, 0};
    const SwQ4 gu = {nullptr, nullptr, 2 * G.I, G.D, G.gs_gu, 1};
    const SwQ4 dn = {nullptr, nullptr, G.D, G.I, G.gs_d, 1};
    if (sw_launch_limbs(c->st, (const float *)(A + L.x), xrows, G.D, xl, xs)) return 0;
    if (sw_launch_q4_dot8_glu_tab(c->st, gu, tab, xl, xs, g, G.I, hl, hs, G.total == G.count)) return 0;
    SwGroups gd = g;
    gd.grow = nullptr;
    if (sw_launch_q4_dot8_rows_tab(c->st, dn, tab, hl, hs, gd, (float *)(A + L.y))) return 0;
    (void)T;
    return ok(hipGetLastError(), "expert group launch");
}

void count_group(const Groups &G) {
    std::lock_guard<std::mutex> lk(g_stats_mu);
    g_gcalls++;
    g_gexperts += (uint64_t)G.count;
    g_grows += (uint64_t)G.total;
}

// the MFMA form of the group: digits of x, gate/up + GLU, down, over 64-token tiles
// (items[j] = (t0 << 10) | group, then their count) listed after gexp gbeg gcnt
int launch_group_mf(Ctx *c, const Groups &G, char *A, const GLay &L, int ntile) {
    const int *d = (const int *)(A + L.ints);
    const int *items = d + 3 * G.count;
    const SwTab *tab = (const SwTab *)(A + L.tab);
    const SwGroups gt = {d, d + G.count, d + 2 * G.count, nullptr, nullptr, ntile, 0, items, items + ntile};
    const SwQ4 gu = {nullptr, nullptr, 2 * G.I, G.D, G.gs_gu, 1};
    const SwQ4 dn = {nullptr, nullptr, G.D, G.I, G.gs_d, 1};
    uint32_t *xd = (uint32_t *)(A + L.xl), *hd = (uint32_t *)(A + L.hl);
    float *xds = (float *)(A + L.xs), *hds = (float *)(A + L.hs);
    if (sw_launch_digits(c->st, (const float *)(A + L.x), G.total, G.D, xd, xds)) return 0;
    if (sw_launch_mf_glu_tab(c->st, gu, tab, xd, xds, G.total, gt, G.I, hd, hds)) return 0;
    if (sw_launch_mf_rows_tab(c->st, dn, tab, hd, hds, G.total, gt, (float *)(A + L.y))) return 0;
    return ok(hipGetLastError(), "expert group launch");
}

// the synchronous group (expert_group, expert_mlp, shared_mlp_w4a16)
int group_sync(const Groups &G, float *y, const float *x) {
    Ctx *c = find_ctx(G.device);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    const int T = G.total;
    const bool mf = use_mf(G);
    std::vector<int> items;
    if (mf) {
        for (int g = 0; g < G.count; g++)
            for (int t0 = 0; t0 < G.cnt[g]; t0 += sw_mf_tile(G.cnt[g])) items.push_back((t0 << 10) | g);
        items.push_back((int)items.size());
    }
    const int ni = (int)items.size();
    const GLay L = glay(G, T, T, ni, mf);
    const size_t xb = (size_t)T * G.D * 4, ib = (size_t)(3 * G.count + ni) * 4, mb = ib + (size_t)G.count * sizeof(SwTab);
    if (!grow(c, c->arena, L.end) || !grow_pinned(c, c->hin, c->hin_cap, xb + mb) ||
        !grow_pinned(c, c->hout, c->hout_cap, xb))
        return 0;
    char *A = (char *)c->arena.p, *H = (char *)c->hin;
    const char *pe = getenv("COLI_CUDA_PROFILE");
    const bool prof = pe && atoi(pe);
    if (prof && !c->prof[0])
        for (auto &e : c->prof)
            if (!ok(hipEventCreate(&e), "profile event")) return 0;
    memcpy(H, x, xb);
    pack_meta(G, nullptr, 0, H + xb);                      // gexp gbeg gcnt, then the table
    if (mf) {                                              // the tiles between the ints and the table
        memmove(H + xb + ib, H + xb + (size_t)(3 * G.count) * 4, (size_t)G.count * sizeof(SwTab));
        memcpy(H + xb + (size_t)(3 * G.count) * 4, items.data(), (size_t)ni * 4);
    }
    if (prof) (void)hipEventRecord(c->prof[0], c->st);
    // the table follows the ints in the image; in the arena it has its own aligned slot
    if (!ok(hipMemcpyAsync(A + L.x, H, xb, hipMemcpyHostToDevice, c->st), "expert group input upload") ||
        !ok(hipMemcpyAsync(A + L.ints, H + xb, ib, hipMemcpyHostToDevice, c->st), "expert group descriptors") ||
        !ok(hipMemcpyAsync(A + L.tab, H + xb + ib, (size_t)G.count * sizeof(SwTab), hipMemcpyHostToDevice, c->st),
            "expert group table"))
        return 0;
    if (prof) (void)hipEventRecord(c->prof[1], c->st);
    if (mf ? !launch_group_mf(c, G, A, L, ni - 1) : !launch_group(c, G, A, L, T, T, false)) return 0;
    if (prof) (void)hipEventRecord(c->prof[2], c->st);
    if (!ok(hipMemcpyAsync(c->hout, A + L.y, xb, hipMemcpyDeviceToHost, c->st), "expert group output download")) return 0;
    if (prof) (void)hipEventRecord(c->prof[3], c->st);
    if (!ok(hipStreamSynchronize(c->st), "expert group synchronize")) return 0;
    memcpy(y, c->hout, xb);
    if (prof) {
        float a = 0, b = 0, d = 0;
        (void)hipEventElapsedTime(&a, c->prof[0], c->prof[1]);
        (void)hipEventElapsedTime(&b, c->prof[1], c->prof[2]);
        (void)hipEventElapsedTime(&d, c->prof[2], c->prof[3]);
        std::lock_guard<std::mutex> sl(g_stats_mu);
        g_h2d += a; g_kern += b; g_d2h += d;
    }
    count_group(G);
    return 1;
}

// ---- small kernels ----
// out[i] = sum_c w[c] * y[c][i] in c order, one fma each
struct WArgs { float w[64]; int count, D; };
__global__ __launch_bounds__(256) void k_coli_wsum(float *__restrict__ out, const float *__restrict__ y, WArgs a) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.D; i += gridDim.x * blockDim.x) {
        float acc = 0.f;
        for (int c = 0; c < a.count; c++) acc = __builtin_fmaf(a.w[c], y[(size_t)c * a.D + i], acc);
        out[i] = acc;
    }
}
// dst[i] = sum_s slots[s][i] in slot order
__global__ __launch_bounds__(256) void k_coli_sum_slots(float *__restrict__ dst, const float *__restrict__ slots, int n, int D) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < D; i += gridDim.x * blockDim.x) {
        float acc = 0.f;
        for (int s = 0; s < n; s++) acc = acc + slots[(size_t)s * D + i];
        dst[i] = acc;
    }
}
__global__ __launch_bounds__(256) void k_coli_add(float *__restrict__ x, const float *__restrict__ t, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) x[i] = x[i] + t[i];
}
__global__ __launch_bounds__(256) void k_coli_rows_add(float *__restrict__ x, const float *__restrict__ p,
                                                       const int *__restrict__ rows, int D) {
    float *xr = x + (size_t)rows[blockIdx.x] * D;
    const float *pr = p + (size_t)blockIdx.x * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) xr[i] = xr[i] + pr[i];
}
// gate = silu(gate) * up, siluf of c/moe_math.h:53 with glibc's expf
__global__ __launch_bounds__(256) void k_coli_silu_mul(float *__restrict__ g, const float *__restrict__ u, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float v = g[i];
        g[i] = v / (1.0f + sw_expf(-v)) * u[i];
    }
}
unsigned blocks_for(size_t n) { size_t b = (n + 255) / 256; return (unsigned)(b < 1024 ? (b ? b : 1) : 1024); }

// ---- the device router (c/colibri.c:2871-2999 on one row) ----
// logits: lane e runs its expert's dot in input order as the CPU engine's
// `a += xs[i] * w[i]` (c/quant.h:98-102) runs built by GCC -O3 for AVX-512: the
// products of the first D - D % 8 inputs rounded and added in order (its
// vector loops), the last D % 8 as an fma chain (its scalar tail); x is staged
// in LDS
#define GR_XMAX 16384
__global__ __launch_bounds__(256) void k_glm_logits(const float *__restrict__ x, const float *__restrict__ W,
                                                    const float *__restrict__ bias, int D, int E,
                                                    float *__restrict__ logit, float *__restrict__ choice) {
#pragma clang fp contract(off)
    __shared__ float xs[GR_XMAX];
    for (int i = threadIdx.x; i < D; i += blockDim.x) xs[i] = x[i];
    __syncthreads();
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const float *w = W + (size_t)e * D;
    float a = 0.f;
    int i = 0;
    for (; i + 8 <= D; i += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = w[i + j];
#pragma unroll
        for (int j = 0; j < 8; j++) a = a + xs[i + j] * v[j];       // rounded product, then the add
    }
    for (; i < D; i++) a = __builtin_fmaf(xs[i], w[i], a);
    const float lg = 1.f / (1.f + sw_expf(-a));            // sigmoidf, c/colibri.c:833
    logit[e] = lg;
    choice[e] = lg + bias[e];
}
// selection, top-p, norm_topk, routed_scale by one wave: out = idx[K] | w[K] | keff
__global__ __launch_bounds__(64) void k_glm_select(const float *__restrict__ logit, const float *__restrict__ choice,
                                                   int E, int Ksel, float topp, int norm_topk, float routed_scale,
                                                   int *__restrict__ out) {
    __shared__ uint32_t taken[128];
    __shared__ int idx[64];
    __shared__ float w[64];
    const int l = threadIdx.x;
    for (int i = l; i < 128; i += 64) taken[i] = 0;
    __syncthreads();
    for (int kk = 0; kk < Ksel; kk++) {
        // lane: the first strict maximum of its experts l, l+64, ... (values <= -1e30 and NaN never win)
        float bv = -1e30f;
        int best = -1;
        for (int e = l; e < E; e += 64)
            if (!((taken[e >> 5] >> (e & 31)) & 1u) && choice[e] > bv) { bv = choice[e]; best = e; }
        // the wave's: larger value, then lower id
#pragma unroll
        for (int o = 32; o; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int ob = __shfl_xor(best, o, 64);
            if (ob >= 0 && (best < 0 || ov > bv || (ov == bv && ob < best))) { bv = ov; best = ob; }
        }
        if (l == 0) {
            if (best < 0) best = kk < E ? kk : 0;           // router_best_or_fallback, c/colibri.c:2776-2782
            idx[kk] = best;
            w[kk] = logit[best];
            taken[best >> 5] |= 1u << (best & 31);
        }
        __syncthreads();
    }
    if (l) return;
    int Ke = Ksel;
    if (topp > 0.f && topp < 1.f) {                         // c/colibri.c:2979-2984
        for (int a = 1; a < Ksel; a++) {
            const int ii = idx[a];
            const float ww = w[a];
            int b = a - 1;
            while (b >= 0 && w[b] < ww) { w[b + 1] = w[b]; idx[b + 1] = idx[b]; b--; }
            w[b + 1] = ww;
            idx[b + 1] = ii;
        }
        float tot = 1e-20f;
        for (int kk = 0; kk < Ksel; kk++) tot = tot + w[kk];
        float cum = 0.f;
        for (int kk = 0; kk < Ksel; kk++) {
            cum = cum + w[kk];
            if (cum >= topp * tot) { Ke = kk + 1; break; }
        }
    }
    if (norm_topk) {                                        // c/colibri.c:2997
        float sm = 0.f;
        for (int kk = 0; kk < Ke; kk++) sm = sm + w[kk];
        sm = sm + 1e-20f;
        for (int kk = 0; kk < Ke; kk++) w[kk] = w[kk] / sm;
    }
    for (int kk = 0; kk < Ke; kk++) w[kk] = w[kk] * routed_scale;
    for (int kk = 0; kk < Ksel; kk++) { out[kk] = idx[kk]; ((float *)out)[Ksel + kk] = w[kk]; }
    out[2 * Ksel] = Ke;
}

}  // namespace

// ============================================================== contexts ====
extern "C" int coli_hip_init(const int *devices, int count) {
    int available = 0;
    if (!devices || count < 1 || count > COLI_HIP_MAX_DEVICES) return 0;
    if (g_nctx) coli_hip_shutdown();
    if (!ok(hipGetDeviceCount(&available), "device discovery")) return 0;
    for (int i = 0; i < count; i++) {
        const int dev = devices[i];
        if (dev < 0 || dev >= available || find_ctx(dev)) {
            fprintf(stderr, "[sabrewing-coli] device %d: %s\n", dev, dev < 0 || dev >= available ? "invalid" : "duplicate");
            coli_hip_shutdown();
            return 0;
        }
        Ctx *c = &g_ctx[g_nctx];
        *c = Ctx{};
        c->device = dev;
        t_current = -1;
        if (!select_ctx(c) || !ok(hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking), "stream creation")) {
            coli_hip_shutdown();
            return 0;
        }
        g_nctx++;
    }
    return 1;
}

extern "C" void coli_hip_shutdown(void) {
    for (int i = 0; i < g_nctx; i++) {
        Ctx *c = &g_ctx[i];
        std::lock_guard<std::mutex> lk(g_mu[i]);
        if (!select_ctx(c)) continue;
        if (c->st) (void)hipStreamSynchronize(c->st);
        DBuf *bs[] = {&c->arena, &c->res, &c->rout};
        for (DBuf *b : bs) if (b->p) (void)hipFree(b->p);
        for (DBuf &b : c->pipe) if (b.p) (void)hipFree(b.p);
        void *hs[] = {c->hin, c->hout, c->hiss_in, c->hiss_out, c->hres, c->hrout};
        for (void *h : hs) if (h) (void)hipHostFree(h);
        if (c->ev_done) (void)hipEventDestroy(c->ev_done);
        if (c->ev_res) (void)hipEventDestroy(c->ev_res);
        for (auto e : c->prof) if (e) (void)hipEventDestroy(e);
        if (c->st) (void)hipStreamDestroy(c->st);
        *c = Ctx{};
    }
    g_nctx = 0;
    t_current = -1;
}

extern "C" int coli_hip_device_count(void) { return g_nctx; }
extern "C" int coli_hip_device_at(int index) { return index >= 0 && index < g_nctx ? g_ctx[index].device : -1; }

extern "C" int coli_hip_mem_info(int device, size_t *free_bytes, size_t *total_bytes) {
    Ctx *c = find_ctx(device);
    if (!free_bytes || !total_bytes || !select_ctx(c)) return 0;
    return ok(hipMemGetInfo(free_bytes, total_bytes), "memory info");
}

extern "C" void coli_hip_stats(int device, size_t *tensor_count, size_t *tensor_bytes) {
    size_t n = 0, b = 0;
    for (int i = 0; i < g_nctx; i++)
        if (device < 0 || g_ctx[i].device == device) { n += g_ctx[i].tensor_count; b += g_ctx[i].tensor_bytes; }
    if (tensor_count) *tensor_count = n;
    if (tensor_bytes) *tensor_bytes = b;
}

extern "C" void coli_hip_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows, double *h2d_ms,
                                     double *kernel_ms, double *d2h_ms) {
    std::lock_guard<std::mutex> lk(g_stats_mu);
    if (calls) *calls = g_gcalls;
    if (experts) *experts = g_gexperts;
    if (rows) *rows = g_grows;
    if (h2d_ms) *h2d_ms = g_h2d;
    if (kernel_ms) *kernel_ms = g_kern;
    if (d2h_ms) *d2h_ms = g_d2h;
}

// =============================================================== tensors ====
extern "C" int coli_hip_tensor_upload_g(ColiHipTensor **tensor, const void *weights, const float *scales, int fmt, int I,
                                        int O, int device, int gs) {
    if (!tensor) return 0;
    const int want_gs = fmt == 4 && gs > 0 ? gs : 0;
    if (*tensor) {
        const ColiHipTensor *t = *tensor;
        return t->fmt == fmt && t->I == I && t->O == O && t->device == device && t->gs == want_gs;
    }
    Ctx *c = find_ctx(device);
    if (!weights || !scales || !shape_ok(fmt, I, O, want_gs) || !c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    ColiHipTensor *t = (ColiHipTensor *)calloc(1, sizeof(ColiHipTensor));
    if (!t) return 0;
    t->fmt = fmt; t->I = I; t->O = O; t->device = device; t->gs = want_gs;
    t->ng = want_gs ? I / want_gs : 1;
    t->wbytes = (size_t)O * (I / 2);
    t->sbytes = (size_t)O * t->ng * 4;
    if (!ok(hipMalloc(&t->w, t->wbytes), "tensor allocation") ||
        !ok(hipMalloc((void **)&t->s, t->sbytes), "scale allocation") ||
        !ok(hipMemcpy(t->w, weights, t->wbytes, hipMemcpyHostToDevice), "tensor upload") ||
        !ok(hipMemcpy(t->s, scales, t->sbytes, hipMemcpyHostToDevice), "scale upload")) {
        if (t->w) (void)hipFree(t->w);
        if (t->s) (void)hipFree(t->s);
        free(t);
        return 0;
    }
    c->tensor_count++;
    c->tensor_bytes += t->wbytes + t->sbytes;
    *tensor = t;
    return 1;
}

extern "C" int coli_hip_tensor_upload(ColiHipTensor **tensor, const void *weights, const float *scales, int fmt, int I,
                                      int O, int device) {
    return coli_hip_tensor_upload_g(tensor, weights, scales, fmt, I, O, device, 0);
}

extern "C" void coli_hip_tensor_free(ColiHipTensor *t) {
    if (!t) return;
    Ctx *c = find_ctx(t->device);
    if (c) {
        std::lock_guard<std::mutex> lk(mu_of(c));
        if (select_ctx(c)) {
            (void)hipStreamSynchronize(c->st);              // no queued work may still read it
            if (c->tensor_count) c->tensor_count--;
            const size_t b = t->wbytes + t->sbytes;
            c->tensor_bytes = c->tensor_bytes >= b ? c->tensor_bytes - b : 0;
        }
    }
    if (t->w) (void)hipFree(t->w);
    if (t->s) (void)hipFree(t->s);
    free(t);
}

extern "C" size_t coli_hip_tensor_bytes(const ColiHipTensor *t) { return t ? t->wbytes + t->sbytes : 0; }
extern "C" int coli_hip_tensor_device(const ColiHipTensor *t) { return t ? t->device : -1; }

extern "C" int coli_hip_tensor_update(ColiHipTensor *t, const void *weights, const float *scales) {
    if (!t || !weights || !scales) return 0;
    Ctx *c = find_ctx(t->device);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c) || !ok(hipStreamSynchronize(c->st), "tensor refresh drain")) return 0;
    return ok(hipMemcpy(t->w, weights, t->wbytes, hipMemcpyHostToDevice), "tensor refresh") &&
           ok(hipMemcpy(t->s, scales, t->sbytes, hipMemcpyHostToDevice), "scale refresh");
}

// =============================================================== compute ====
namespace {
// y_dev[S][O] = x_dev[S][I] . W^T on the context's stream, in the CPU's f32 contract:
// matmul_q4_k (per-row scales, fmt 2) or matmul_i4_grouped (group scales, fmt 4), the
// 16-lane kernels of k_lanes.hip
int gemm_dev(Ctx *c, const ColiHipTensor *t, float *y, const float *x, int S) {
    const int gs = t->fmt == 4 ? t->gs : 0;
    if (sw_launch_lanes16(c->st, t->w, gs > 0 ? 3 : 2, 0, t->s, x, S, t->I, t->O, y, gs)) return ok(hipErrorInvalidValue, "matmul launch (shape unsupported?)");
    return ok(hipGetLastError(), "matmul launch");
}
}  // namespace

extern "C" int coli_hip_matmul(ColiHipTensor **tensor, float *y, const float *x, const void *weights,
                               const float *scales, int fmt, int S, int I, int O, int device, int gs) {
    if (fault_injected()) return 0;
    if ((fmt == 4 && gs <= 0) || S < 1 || !y || !x) return 0;
    if (!coli_hip_tensor_upload_g(tensor, weights, scales, fmt, I, O, device, gs)) return 0;
    const ColiHipTensor *t = *tensor;
    Ctx *c = find_ctx(t->device);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    Carve cv;
    const size_t ox = cv.take((size_t)S * I * 4), oy = cv.take((size_t)S * O * 4);
    const size_t xb = (size_t)S * I * 4, yb = (size_t)S * O * 4;
    if (!grow(c, c->arena, cv.off) || !grow_pinned(c, c->hin, c->hin_cap, xb) || !grow_pinned(c, c->hout, c->hout_cap, yb))
        return 0;
    char *A = (char *)c->arena.p;
    memcpy(c->hin, x, xb);
    if (!ok(hipMemcpyAsync(A + ox, c->hin, xb, hipMemcpyHostToDevice, c->st), "input upload") ||
        !gemm_dev(c, t, (float *)(A + oy), (const float *)(A + ox), S) ||
        !ok(hipMemcpyAsync(c->hout, A + oy, yb, hipMemcpyDeviceToHost, c->st), "output download") ||
        !ok(hipStreamSynchronize(c->st), "matmul synchronize"))
        return 0;
    memcpy(y, c->hout, yb);
    return 1;
}

extern "C" int coli_hip_expert_mlp(ColiHipTensor *gate, ColiHipTensor *up, ColiHipTensor *down, float *y,
                                   const float *x, int S) {
    if (fault_injected()) return 0;
    if (!x || !y || S < 1) return 0;
    Groups G;
    if (!collect(&gate, &up, &down, &S, 1, G)) return 0;
    return group_sync(G, y, x);
}

extern "C" int coli_hip_shared_mlp_w4a16(ColiHipTensor *gate, ColiHipTensor *up, ColiHipTensor *down, float *y,
                                         const float *x, int S) {
    if (fault_injected()) return 0;
    if (!gate || !up || !down || gate->fmt != 2 || up->fmt != 2 || down->fmt != 2 || !x || !y || S < 1) return 0;
    Groups G;
    if (!collect(&gate, &up, &down, &S, 1, G)) return 0;
    return group_sync(G, y, x);
}

extern "C" int coli_hip_expert_group(ColiHipTensor *const *gates, ColiHipTensor *const *ups, ColiHipTensor *const *downs,
                                     const int *rows, int count, float *y, const float *x) {
    if (fault_injected()) return 0;
    if (!rows || !x || !y) return 0;
    Groups G;
    if (!collect(gates, ups, downs, rows, count, G)) return 0;
    return group_sync(G, y, x);
}

extern "C" int coli_hip_expert_group_issue(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                           ColiHipTensor *const *downs, const int *rows, int count, const float *x) {
    if (!rows || !x) return 0;
    Groups G;
    if (!collect(gates, ups, downs, rows, count, G) || G.total > 8) return 0;     // decode-scale only
    Ctx *c = find_ctx(G.device);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (c->pending || !select_ctx(c)) return 0;
    const int T = G.total;
    const GLay L = glay(G, T, T);
    const size_t xb = (size_t)T * G.D * 4, mb = meta_bytes(G, 0);
    if (!grow(c, c->arena, L.end) || !grow_pinned(c, c->hiss_in, c->hiss_in_cap, xb + mb) ||
        !grow_pinned(c, c->hiss_out, c->hiss_out_cap, xb))
        return 0;
    char *A = (char *)c->arena.p, *H = (char *)c->hiss_in;
    memcpy(H, x, xb);
    pack_meta(G, nullptr, 0, H + xb);
    if (!ok(hipMemcpyAsync(A + L.x, H, xb, hipMemcpyHostToDevice, c->st), "expert group issue upload") ||
        !ok(hipMemcpyAsync(A + L.ints, H + xb, (size_t)(3 * G.count) * 4, hipMemcpyHostToDevice, c->st), "issue descriptors") ||
        !ok(hipMemcpyAsync(A + L.tab, H + xb + (size_t)(3 * G.count) * 4, (size_t)G.count * sizeof(SwTab),
                           hipMemcpyHostToDevice, c->st), "issue table") ||
        !launch_group(c, G, A, L, T, T, false) ||
        !ok(hipMemcpyAsync(c->hiss_out, A + L.y, xb, hipMemcpyDeviceToHost, c->st), "expert group issue download"))
        return 0;
    c->pending = 1;
    count_group(G);
    return 1;
}

extern "C" const float *coli_hip_expert_group_take(int device) {
    Ctx *c = find_ctx(device);
    if (!c) return nullptr;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!c->pending) return nullptr;
    c->pending = 0;
    if (!select_ctx(c) || !ok(hipStreamSynchronize(c->st), "expert group take")) return nullptr;
    return (const float *)c->hiss_out;
}

extern "C" int coli_hip_expert_group_resident_issue(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                                    ColiHipTensor *const *downs, const float *weights, int count,
                                                    int home_device, const float *x_src_dev, float *partial_slot_dev) {
    if (!weights || !x_src_dev || !partial_slot_dev) return 0;
    Groups G;
    if (!collect(gates, ups, downs, nullptr, count, G) || G.gs_gu != 0 || G.gs_d != 0) return 0;   // per-row int4 only
    for (int i = 0; i < count; i++)
        if (gates[i]->fmt != 2) return 0;
    Ctx *c = find_ctx(G.device);
    if (!c || !find_ctx(home_device)) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    if (!c->ev_done_ok) {
        if (!ok(hipEventCreateWithFlags(&c->ev_done, hipEventDisableTiming), "resident group event") ||
            !ok(hipEventCreateWithFlags(&c->ev_res, hipEventDisableTiming), "resident meta event"))
            return 0;
        c->ev_done_ok = 1;
    }
    // every group is one row, all reading x (grow = 0...): limbs of one row
    const int T = count;
    std::vector<int> zeros((size_t)T, 0);
    // scratch for the 64-expert cap at this (D, I), so a later issue never regrows it under queued work
    Groups cap = G;
    cap.count = 64;
    const GLay Lc = glay(cap, 64, 1, 64);
    const GLay L = glay(G, T, 1, T);
    if (!grow(c, c->res, Lc.end + (size_t)G.D * 4 + 256)) return 0;
    // the pinned meta image: wait until the previous issue's copy of it has run
    if (c->ev_res_live && !ok(hipEventSynchronize(c->ev_res), "resident meta wait")) return 0;
    if (!grow_pinned(c, c->hres, c->hres_cap, meta_bytes(cap, 64))) return 0;
    char *A = (char *)c->res.p, *H = (char *)c->hres;
    pack_meta(G, zeros.data(), T, H);
    float *partial = (float *)(A + ((Lc.end + 255) & ~(size_t)255));
    const bool same = home_device == G.device;
    hipError_t xe = same ? hipMemcpyAsync(A + L.x, x_src_dev, (size_t)G.D * 4, hipMemcpyDeviceToDevice, c->st)
                         : hipMemcpyPeerAsync(A + L.x, G.device, x_src_dev, home_device, (size_t)G.D * 4, c->st);
    if (!ok(xe, "resident group x copy") ||
        !ok(hipMemcpyAsync(A + L.ints, H, (size_t)(3 * G.count + T) * 4, hipMemcpyHostToDevice, c->st), "resident descriptors") ||
        !ok(hipMemcpyAsync(A + L.tab, H + (size_t)(3 * G.count + T) * 4, (size_t)G.count * sizeof(SwTab),
                           hipMemcpyHostToDevice, c->st), "resident table") ||
        !ok(hipEventRecord(c->ev_res, c->st), "resident meta event"))
        return 0;
    c->ev_res_live = 1;
    if (!launch_group(c, G, A, L, T, 1, true)) return 0;
    WArgs wa;
    for (int i = 0; i < count; i++) wa.w[i] = weights[i];
    wa.count = count;
    wa.D = G.D;
    float *dst = same ? partial_slot_dev : partial;
    hipLaunchKernelGGL(k_coli_wsum, dim3(blocks_for((size_t)G.D)), dim3(256), 0, c->st, dst, (const float *)(A + L.y), wa);
    if (!ok(hipGetLastError(), "resident weighted sum")) return 0;
    if (!same && !ok(hipMemcpyPeerAsync(partial_slot_dev, home_device, partial, G.device, (size_t)G.D * 4, c->st),
                     "resident partial copy"))
        return 0;
    if (!ok(hipEventRecord(c->ev_done, c->st), "resident event record")) return 0;
    count_group(G);
    return 1;
}

extern "C" int coli_hip_expert_group_resident_take(int home_device, const int *devices, int n_issued, float *slots_dev,
                                                   float *acc_dev, int D) {
    if (n_issued < 1 || !devices || !slots_dev || !acc_dev || D < 1) return 0;
    Ctx *h = find_ctx(home_device);
    if (!h) return 0;
    std::lock_guard<std::mutex> lk(mu_of(h));
    if (!select_ctx(h)) return 0;
    for (int i = 0; i < n_issued; i++) {
        Ctx *s = find_ctx(devices[i]);
        if (!s || !s->ev_done_ok) return 0;
        if (s != h && !ok(hipStreamWaitEvent(h->st, s->ev_done, 0), "resident take wait")) return 0;
    }
    hipLaunchKernelGGL(k_coli_sum_slots, dim3(blocks_for((size_t)D)), dim3(256), 0, h->st, acc_dev, (const float *)slots_dev,
                       n_issued, D);
    return ok(hipGetLastError(), "resident take reduce");
}

// ========================================================= not on gfx950 ====
extern "C" int coli_hip_attention_absorb(ColiHipTensor *, float *, const float *, const float *, const float *, int, int,
                                         int, int, int, int, float) { return 0; }
extern "C" int coli_hip_attention_absorb_batch(ColiHipTensor *, float *, const float *, const float *, const float *, int,
                                               int, int, int, int, int, int, float) { return 0; }
extern "C" int coli_hip_attention_project_batch(ColiHipTensor *, ColiHipTensor *, float *, const float *, const float *,
                                                const float *, int, int, int, int, int, int, int, float) { return 0; }
extern "C" int coli_hip_attention_project_ragged(ColiHipTensor *, ColiHipTensor *, float *, const float *,
                                                 const void *const *, const float *const *, const float *const *,
                                                 const int *, int, int, int, int, int, int, int, float) { return 0; }
extern "C" int coli_hip_attention_project_batch_dev(ColiHipTensor *, ColiHipTensor *, float *, const float *,
                                                    const float *, const float *, int, int, int, int, int, int, int,
                                                    float) { return 0; }
extern "C" int coli_hip_attention_absorb_batch_dev(ColiHipTensor *, float *, const float *, const float *, const float *,
                                                   int, int, int, int, int, int, int, float) { return 0; }
extern "C" int coli_hip_attention_absorb_kvdev(ColiHipTensor *, float *, const float *, const float *, const float *, int,
                                               int, int, int, int, int, float) { return 0; }
extern "C" int coli_hip_attention_project_batch_dev_out(ColiHipTensor *, ColiHipTensor *, float *, const float *,
                                                        const float *, const float *, int, int, int, int, int, int, int,
                                                        float) { return 0; }
extern "C" int coli_hip_pipe_rmsnorm(int, float *, const float *, const float *, int, int, float) { return 0; }
extern "C" int coli_hip_pipe_rmsnorm_s(int, float *, const float *, const float *, int, int, float, int, int) { return 0; }
extern "C" int coli_hip_pipe_rope(int, float *, const int *, int, int, int, int, int, float) { return 0; }
extern "C" int coli_hip_pipe_rope_base(int, float *, int, int, int, int, int, int, float) { return 0; }

// ============================================================ pipe plane ====
extern "C" float *coli_hip_pipe_scratch(int device, int slot, size_t bytes) {
    Ctx *c = find_ctx(device);
    if (!c || slot < 0 || slot >= 27) return nullptr;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c) || !grow(c, c->pipe[slot], bytes)) return nullptr;
    return (float *)c->pipe[slot].p;
}

extern "C" void *coli_hip_pipe_alloc(int device, size_t bytes) {
    Ctx *c = find_ctx(device);
    if (!select_ctx(c)) return nullptr;
    void *p = nullptr;
    if (!ok(hipMalloc(&p, bytes), "pipe alloc")) return nullptr;
    return p;
}

extern "C" void coli_hip_pipe_free(int device, void *p) {
    Ctx *c = find_ctx(device);
    if (!p || !c) return;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return;
    (void)hipStreamSynchronize(c->st);
    (void)hipFree(p);
}

extern "C" int coli_hip_pipe_upload(int device, void *dst, const void *src, size_t bytes) {
    Ctx *c = find_ctx(device);
    if (!c || !dst || !src) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    return select_ctx(c) && ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->st), "pipe upload") &&
           ok(hipStreamSynchronize(c->st), "pipe upload sync");
}

extern "C" int coli_hip_pipe_download(int device, const void *src, void *dst, size_t bytes) {
    Ctx *c = find_ctx(device);
    if (!c || !dst || !src) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    return select_ctx(c) && ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->st), "pipe download") &&
           ok(hipStreamSynchronize(c->st), "pipe download sync");
}

extern "C" int coli_hip_pipe_silu_mul(int device, float *gate_dev, const float *up_dev, size_t n) {
    if (fault_injected()) return 0;
    Ctx *c = find_ctx(device);
    if (!c || !n || !gate_dev || !up_dev) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    hipLaunchKernelGGL(k_coli_silu_mul, dim3(blocks_for(n)), dim3(256), 0, c->st, gate_dev, up_dev, n);
    return ok(hipGetLastError(), "pipe silu mul");
}

extern "C" int coli_hip_pipe_add(int device, float *x_dev, const float *t_dev, size_t n) {
    if (fault_injected()) return 0;
    Ctx *c = find_ctx(device);
    if (!c || !n || !x_dev || !t_dev) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    hipLaunchKernelGGL(k_coli_add, dim3(blocks_for(n)), dim3(256), 0, c->st, x_dev, t_dev, n);
    return ok(hipGetLastError(), "pipe add");
}

extern "C" int coli_hip_pipe_rows_add(int device, float *x_dev, const float *partial_dev, const int *rows_dev, int nrows,
                                      int D) {
    if (fault_injected()) return 0;
    Ctx *c = find_ctx(device);
    if (!c || nrows < 1 || D < 1 || !x_dev || !partial_dev || !rows_dev) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    hipLaunchKernelGGL(k_coli_rows_add, dim3((unsigned)nrows), dim3(256), 0, c->st, x_dev, partial_dev, rows_dev, D);
    return ok(hipGetLastError(), "pipe rows add");
}

extern "C" int coli_hip_pipe_gemm(ColiHipTensor *t, float *y_dev, const float *x_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || !y_dev || !x_dev || S < 1) return 0;
    Ctx *c = find_ctx(t->device);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    return select_ctx(c) && gemm_dev(c, t, y_dev, x_dev, S);
}

extern "C" int coli_hip_pipe_copy2d(int device, float *dst, int dpitch, const float *src, int spitch, int width,
                                    int height) {
    Ctx *c = find_ctx(device);
    if (!c || !dst || !src || width < 0 || height < 0 || dpitch < width || spitch < width) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    return select_ctx(c) && ok(hipMemcpy2DAsync(dst, (size_t)dpitch * 4, src, (size_t)spitch * 4, (size_t)width * 4,
                                                (size_t)height, hipMemcpyDeviceToDevice, c->st), "pipe copy2d");
}

extern "C" int coli_hip_pipe_peer_copy(int dst_dev, float *dst, int src_dev, const float *src, size_t bytes) {
    if (!dst || !src) return 0;
    Ctx *c = find_ctx(dst_dev);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    if (dst_dev == src_dev)
        return ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->st), "pipe intra copy") &&
               ok(hipStreamSynchronize(c->st), "pipe intra copy sync");
    return ok(hipMemcpyPeer(dst, dst_dev, src, src_dev, bytes), "pipe peer copy");
}

extern "C" int coli_hip_pipe_sync(int device) {
    Ctx *c = find_ctx(device);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    return select_ctx(c) && ok(hipStreamSynchronize(c->st), "pipe sync");
}

extern "C" int coli_hip_pipe_router(int device, const float *x_dev, const void *rw_dev, const void *rb_dev, int D, int E,
                                    int Ksel, float topp, int norm_topk, float routed_scale, int *idx_host,
                                    float *w_host, int *keff_host) {
    Ctx *c = find_ctx(device);
    if (!c || !x_dev || !rw_dev || !rb_dev || D < 1 || D > GR_XMAX || E < 1 || E > 4096 || Ksel < 1 || Ksel > 64 ||
        !idx_host || !w_host || !keff_host)
        return 0;
    std::lock_guard<std::mutex> lk(mu_of(c));
    if (!select_ctx(c)) return 0;
    const size_t pack = (size_t)(2 * Ksel + 1) * 4;
    Carve cv;
    const size_t ol = cv.take((size_t)E * 4), oc = cv.take((size_t)E * 4), oo = cv.take(pack);
    if (!grow(c, c->rout, cv.off)) return 0;
    if (!c->hrout && !ok(hipHostMalloc(&c->hrout, (size_t)(2 * 64 + 1) * 4, hipHostMallocDefault), "router staging"))
        return 0;
    char *A = (char *)c->rout.p;
    hipLaunchKernelGGL(k_glm_logits, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, c->st, x_dev, (const float *)rw_dev,
                       (const float *)rb_dev, D, E, (float *)(A + ol), (float *)(A + oc));
    hipLaunchKernelGGL(k_glm_select, dim3(1), dim3(64), 0, c->st, (const float *)(A + ol), (const float *)(A + oc), E, Ksel,
                       topp, norm_topk, routed_scale, (int *)(A + oo));
    if (!ok(hipGetLastError(), "pipe router launch") ||
        !ok(hipMemcpyAsync(c->hrout, A + oo, pack, hipMemcpyDeviceToHost, c->st), "pipe router readback") ||
        !ok(hipStreamSynchronize(c->st), "pipe router sync"))
        return 0;
    const int *o = (const int *)c->hrout;
    memcpy(idx_host, o, (size_t)Ksel * 4);
    memcpy(w_host, o + Ksel, (size_t)Ksel * 4);
    *keff_host = o[2 * Ksel];
    return 1;
}
