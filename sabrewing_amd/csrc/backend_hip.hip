// backend_hip.hip -- host side of the gfx950 MoE backend (include/sabrewing_hip.h).
//
// Replaces c/backend_cuda_laguna.cu's host code.  Same process model: one
// device, one stream, pinned staging grown on demand, results of the
// host-pointer entries valid on return.  Different inside: every MoE entry is
// a fixed short sequence of launches over device-side groups (no per-expert
// launch loop, no host bounce of intermediate results), and the device-side
// forward keeps routing, bucketing and the combine on the GPU.
#include "sw_hip.h"
#include "sw_shared.h"
#include "../../include/sabrewing_hip.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>
#include <string>

static int g_ok = 0;
static int g_dev = 0;
static int g_capturing = 0;             // between lag_hip_graph_begin and _end: nothing may allocate or sync
static hipStream_t g_st = nullptr;      // the backend stream (all entry points are ordered on it)
static char g_err[256] = "";

static int fail(const char *what, hipError_t e) {
    snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
    fprintf(stderr, "[sabrewing-hip] %s\n", g_err);
    (void)hipGetLastError();                     // consume the sticky error
    return -1;
}
#define CK(call, what)                        \
    do {                                      \
        hipError_t e_ = (call);               \
        if (e_ != hipSuccess) return fail(what, e_); \
    } while (0)
static int fail_msg(const char *what) {
    snprintf(g_err, sizeof g_err, "%s", what);
    return -1;
}

// COLI_GPU_FAIL_AFTER=N: compute entries report failure after N successful calls
static long g_calls = 0;
static int fault_injected(void) {
    const char *fa = getenv("COLI_GPU_FAIL_AFTER");
    return fa && g_calls++ >= atol(fa);
}

// ------------------------------------------------------------ profiling ----
struct ProfRec { std::string name; double ms; long long n; };
struct Pending { int rec; hipEvent_t a, b; };
static int g_prof = 0;
static std::vector<ProfRec> g_prof_recs;
static std::vector<Pending> g_pending;
static std::vector<hipEvent_t> g_evpool;

static hipEvent_t ev_get(void) {
    if (!g_evpool.empty()) { hipEvent_t e = g_evpool.back(); g_evpool.pop_back(); return e; }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
static int prof_rec(const char *name) {
    for (size_t i = 0; i < g_prof_recs.size(); i++) if (g_prof_recs[i].name == name) return (int)i;
    g_prof_recs.push_back({name, 0.0, 0});
    return (int)g_prof_recs.size() - 1;
}
static void prof_flush(void) {
    if (g_pending.empty()) return;
    (void)hipStreamSynchronize(g_st);
    for (auto &p : g_pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) { g_prof_recs[p.rec].ms += ms; g_prof_recs[p.rec].n++; }
        g_evpool.push_back(p.a); g_evpool.push_back(p.b);
    }
    g_pending.clear();
}
thread_local SwLaunchEvents *sw_launch_events = nullptr;
// Time one launch when profiling: kernels launched through SW_LAUNCH carry the
// scope's events themselves (dispatch to end); otherwise the events are
// recorded on the stream around the scope.
struct ProfScope {
    Pending p; bool on; hipStream_t st; SwLaunchEvents le;
    ProfScope(const char *name, hipStream_t s) : on(g_prof != 0 && !g_capturing), st(s) {
        if (!on) return;
        p.rec = prof_rec(name); p.a = ev_get(); p.b = ev_get();
        if (!p.a || !p.b) { on = false; return; }
        le = {p.a, p.b, 0};
        sw_launch_events = &le;
    }
    ~ProfScope() {
        if (!on) return;
        sw_launch_events = nullptr;
        if (!le.started) {                              // no kernel took the events: time the scope on the stream
            (void)hipEventRecord(p.a, st);
            (void)hipEventRecord(p.b, st);
        }
        g_pending.push_back(p);
        if (g_pending.size() > 4096) prof_flush();
    }
};
#define PROF(name) ProfScope prof_scope_(name, g_st)

// ------------------------------------------------------------ buffers ----
// grow-only device arena and pinned staging (2x slack, as the reference)
struct Buf { void *p = nullptr; size_t cap = 0; };
static int grow_dev(Buf &b, size_t need) {
    if (need <= b.cap) return 0;
    if (g_capturing) return fail_msg("device scratch too small while recording a graph (run the same shapes once first)");
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr; b.cap = 0;
    CK(hipMalloc(&b.p, need * 2), "device scratch allocation");
    b.cap = need * 2;
    return 0;
}
// pinned host staging of the host-pointer entries, grown like the arena
static int grow_pinned(Buf &b, size_t need) {
    if (need <= b.cap) return 0;
    if (b.p) (void)hipHostFree(b.p);
    b.p = nullptr; b.cap = 0;
    CK(hipHostMalloc(&b.p, need * 2, hipHostMallocDefault), "pinned staging allocation");
    b.cap = need * 2;
    return 0;
}
static Buf g_arena, g_hin, g_hout;

// carve aligned sub-buffers out of the arena
struct Carve {
    size_t off = 0;
    size_t take(size_t n) { size_t o = (off + 255) & ~(size_t)255; off = o + n; return o; }
};

static int noalloc_setup(int dev);

// ------------------------------------------------------------ lag family ----
// One device per process, as the reference backend: the stream, the arena and the
// uploaded weights all belong to the first device initialised, so a later call
// naming another device is refused instead of silently keeping the first one's.
extern "C" int lag_hip_init(int dev) {
    if (g_ok) {
        if (dev == g_dev) return 0;
        snprintf(g_err, sizeof g_err, "lag_hip_init(%d): already initialised on device %d (one device per process)", dev,
                 g_dev);
        return -1;
    }
    CK(hipSetDevice(dev), "hipSetDevice");
    if (!g_st) CK(hipStreamCreateWithFlags(&g_st, hipStreamNonBlocking), "stream creation");
    void *probe = nullptr;
    CK(hipMalloc(&probe, 1 << 20), "probe allocation");
    (void)hipFree(probe);
    g_dev = dev;
    g_ok = 1;
    // the allocation-free forward's scratch address: a failure here leaves that one
    // entry unavailable (it reports not initialised) and every other entry working
    (void)noalloc_setup(dev);
    return 0;
}

extern "C" size_t lag_hip_free_bytes(void) {
    size_t fr = 0, to = 0;
    if (hipMemGetInfo(&fr, &to) != hipSuccess) { (void)hipGetLastError(); return 0; }
    return fr;
}
extern "C" size_t lag_hip_total_bytes(void) {
    size_t fr = 0, to = 0;
    if (hipMemGetInfo(&fr, &to) != hipSuccess) { (void)hipGetLastError(); return 0; }
    return to;
}

extern "C" void *lag_hip_upload(const void *h, size_t n) {
    if (!g_ok || !h || !n) return nullptr;
    void *d = nullptr;
    if (hipMalloc(&d, n) != hipSuccess) { fail("upload allocation", hipErrorOutOfMemory); return nullptr; }
    if (hipMemcpy(d, h, n, hipMemcpyHostToDevice) != hipSuccess) { (void)hipFree(d); fail("upload copy", hipErrorUnknown); return nullptr; }
    return d;
}
extern "C" void lag_hip_free(void *d) { if (d) (void)hipFree(d); }

extern "C" void *lag_hip_alloc(size_t n) {
    if (!g_ok || !n) return nullptr;
    void *d = nullptr;
    if (hipMalloc(&d, n) != hipSuccess) { fail("alloc", hipErrorOutOfMemory); return nullptr; }
    return d;
}
extern "C" int lag_hip_h2d(void *dst, const void *src, size_t n) {
    if (!g_ok) return -1;
    CK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g_st), "h2d");
    CK(hipStreamSynchronize(g_st), "h2d sync");
    return 0;
}
extern "C" int lag_hip_d2h(void *dst, const void *src, size_t n) {
    if (!g_ok) return -1;
    CK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g_st), "d2h");
    CK(hipStreamSynchronize(g_st), "d2h sync");
    return 0;
}
extern "C" int lag_hip_d2d(void *dst, const void *src, size_t n) {
    if (!g_ok) return -1;
    CK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, g_st), "d2d");
    return 0;
}
extern "C" int lag_hip_memset(void *dst, int v, size_t n) {
    if (!g_ok) return -1;
    CK(hipMemsetAsync(dst, v, n, g_st), "memset");
    return 0;
}
extern "C" int lag_hip_sync(void) {
    if (!g_ok) return -1;
    CK(hipStreamSynchronize(g_st), "stream sync");
    if (g_prof) prof_flush();
    return 0;
}

// The grouped expert GEMMs of a batch: dot8 (k_dot8.hip) or the f16 MFMA
// (k_mfma.hip), bit-identical; auto takes the MFMA when the groups average at
// least 6.5 tokens (SW_MF_MIN_AVG2 / 2).  Measured on the C2 layer (dot8 against MFMA
// per step): B=160 1,009 against 1,055 us, B=176 1,088 against 1,065, B=192 1,167 against
// 1,072, B=256 1,476 against 1,105.
static int g_grouped_kernel = 0;        // 0 auto, 1 dot8, 2 MFMA
#define SW_MF_MIN_AVG2 13
static bool use_mfma(int T, int E, int D, int I) {
    if (g_grouped_kernel == 1 || D % 128 || I % 128) return false;      // whole chunks of 4 input groups
    if (g_grouped_kernel == 2) return true;
    return 2 * (int64_t)T >= SW_MF_MIN_AVG2 * (int64_t)(T < E ? T : E);
}
extern "C" int lag_hip_set_grouped_kernel(int mode) {
    if (mode < 0 || mode > 2) return -1;
    const int prev = g_grouped_kernel;
    g_grouped_kernel = mode;
    return prev;
}

// The int4 activation contract of the device-resident layer for per-row scales
// (gs == 0): 0 this build's exact-integer dot8/MFMA form, 1 the reference's IDOT
// (int8 activations per 32-block, c/moe_quant.h:48-82; its LAG_IDOT=1, c/laguna.c:204-207).
static int g_q4_mode = 0;
extern "C" int lag_hip_set_q4_mode(int mode) {
    if (mode < 0 || mode > 1) return -1;
    const int prev = g_q4_mode;
    g_q4_mode = mode;
    return prev;
}

// the int4 expert pipeline over device groups:
//   h <- silu_glu(gate_up . x);  slots <- down . h
// (limbs_ready: xl/xs already hold the limbs of dx)
static int run_experts(SwQ4 gu, SwQ4 dn, const float *dx, int S, sw_u32x4 *xl, float *xs, int limbs_ready, SwGroups g,
                       int I, sw_u32x4 *hl, float *hs, float *slots, int maxtok) {
    if (!limbs_ready) {
        PROF("x_limbs");
        if (sw_launch_limbs(g_st, dx, S, gu.K, xl, xs)) return fail_msg("limbs launch (shape unsupported?)");
    }
    { PROF("q4_gateup_glu"); if (sw_launch_q4_dot8_glu(g_st, gu, xl, xs, g, I, hl, hs)) return fail_msg("gate_up launch (shape unsupported?)"); }
    SwGroups gd = g;
    gd.grow = nullptr;                     // down reads the packed rows directly
    { PROF("q4_down"); if (sw_launch_q4_dot8_rows(g_st, dn, hl, hs, gd, slots)) return fail_msg("down launch (shape unsupported?)"); }
    (void)maxtok;
    return 0;
}

// host-index grouped entry shared by moe_experts / moe_group / expert_q4
static int grouped_host(float *outh, const float *x, int S, const void *gu_q, const float *gu_s,
                        const void *dn_q, const float *dn_s, const int *gexp, const int *gbeg, const int *gcnt, int G,
                        const int *grow, const int *rowof, const float *w, int K, int I, int D, int gs, int combine) {
    if (!g_ok || fault_injected()) return -1;
    if (D <= 0 || I <= 0 || G <= 0 || S <= 0) return -1;
    const int T = S * K;
    // the MFMA kernels for prefill-sized groups: tiles of up to 64 tokens, listed here
    int ntile = 0;
    for (int i = 0; i < G; i++) ntile += (gcnt[i] + SW_MF_TT - 1) / SW_MF_TT;
    const bool mf = G < 1024 && T < (1 << 21) && use_mfma(T, G, D, I);
    Carve cv;
    const size_t idxn = (size_t)(3 * G + 2 * T) * 4 + (size_t)T * 4 + (mf ? (size_t)(ntile + 1) * 4 : 0);
    const size_t o_x = cv.take((size_t)S * D * 4), o_idx = cv.take(idxn);
    const size_t o_hl = cv.take((size_t)T * (I / 32) * SW_NL * 16), o_hs = cv.take((size_t)T * (I / 32) * 4);
    const size_t o_slot = cv.take((size_t)T * D * 4), o_out = cv.take((size_t)S * D * 4);
    const size_t o_xl = cv.take((size_t)S * (D / 32) * SW_NL * 16), o_xs = cv.take((size_t)S * (D / 32) * 4);
    size_t o_xd = 0, o_hd = 0;
    if (mf) { o_xd = cv.take((size_t)S * (D / 32) * 128); o_hd = cv.take((size_t)T * (I / 32) * 128); }
    if (grow_dev(g_arena, cv.off)) return -1;
    char *A = (char *)g_arena.p;
    // one pinned blob: x | gexp gbeg gcnt grow rowof w [| items P]
    const size_t xn = (size_t)S * D * 4;
    if (grow_pinned(g_hin, xn + idxn) || grow_pinned(g_hout, (size_t)S * D * 4)) return -1;
    char *H = (char *)g_hin.p;
    memcpy(H, x, xn);
    int *hi = (int *)(H + xn);
    memcpy(hi, gexp, (size_t)G * 4);
    memcpy(hi + G, gbeg, (size_t)G * 4);
    memcpy(hi + 2 * G, gcnt, (size_t)G * 4);
    memcpy(hi + 3 * G, grow, (size_t)T * 4);
    memcpy(hi + 3 * G + T, rowof, (size_t)T * 4);
    memcpy(hi + 3 * G + 2 * T, w, (size_t)T * 4);
    if (mf) {
        int *it = hi + 3 * G + 3 * T, n = 0;
        for (int i = 0; i < G; i++)
            for (int t0 = 0; t0 < gcnt[i]; t0 += sw_mf_tile(gcnt[i])) it[n++] = (t0 << 10) | i;
        it[n] = n;
    }
    CK(hipMemcpyAsync(A + o_x, H, xn, hipMemcpyHostToDevice, g_st), "x upload");
    CK(hipMemcpyAsync(A + o_idx, H + xn, idxn, hipMemcpyHostToDevice, g_st), "index upload");
    const int *d_gexp = (const int *)(A + o_idx), *d_gbeg = d_gexp + G, *d_gcnt = d_gexp + 2 * G;
    const int *d_grow = d_gexp + 3 * G, *d_rowof = d_grow + T;
    const float *d_w = (const float *)(d_rowof + T);
    int nexp = 0;                                     // the tensors hold experts 0..max(gexp)
    for (int i = 0; i < G; i++) {
        if (gexp[i] < 0) return fail_msg("negative expert id");
        nexp = gexp[i] + 1 > nexp ? gexp[i] + 1 : nexp;
    }
    SwQ4 gu = {(const uint8_t *)gu_q, gu_s, 2 * I, D, gs, nexp};
    SwQ4 dn = {(const uint8_t *)dn_q, dn_s, D, I, gs, nexp};
    SwGroups g = {d_gexp, d_gbeg, d_gcnt, d_grow, nullptr, G, 0};
    int maxcnt = 0;
    for (int i = 0; i < G; i++) maxcnt = gcnt[i] > maxcnt ? gcnt[i] : maxcnt;
    if (mf) {
        const int *d_items = (const int *)(d_w + T);
        const SwGroups gt = {d_gexp, d_gbeg, d_gcnt, d_grow, nullptr, ntile, 0, d_items, d_items + ntile};
        SwGroups gd = gt;
        gd.grow = nullptr;
        uint32_t *xd = (uint32_t *)(A + o_xd), *hd = (uint32_t *)(A + o_hd);
        float *xds = (float *)(A + o_xs), *hds = (float *)(A + o_hs);     // the factors: same sizes as the limbs'
        { PROF("digits"); if (sw_launch_digits(g_st, (const float *)(A + o_x), S, D, xd, xds)) return fail_msg("digits launch"); }
        { PROF("mf_glu"); if (sw_launch_mf_glu(g_st, gu, xd, xds, S, gt, I, hd, hds)) return fail_msg("MFMA gate_up launch (shape unsupported?)"); }
        { PROF("mf_down"); if (sw_launch_mf_rows(g_st, dn, hd, hds, T, gd, (float *)(A + o_slot))) return fail_msg("MFMA down launch (shape unsupported?)"); }
    } else if (run_experts(gu, dn, (const float *)(A + o_x), S, (sw_u32x4 *)(A + o_xl), (float *)(A + o_xs), 0, g, I,
                           (sw_u32x4 *)(A + o_hl), (float *)(A + o_hs), (float *)(A + o_slot), maxcnt)) return -1;
    const float *res = (const float *)(A + o_slot);
    if (combine) {
        PROF("combine");
        if (sw_launch_combine(g_st, (const float *)(A + o_slot), d_rowof, d_w, S, K, D, 1.0f, nullptr,
                              (float *)(A + o_out), 0)) return fail_msg("combine launch");
        res = (const float *)(A + o_out);
    }
    CK(hipMemcpyAsync(g_hout.p, res, (size_t)S * D * 4, hipMemcpyDeviceToHost, g_st), "result download");
    CK(hipStreamSynchronize(g_st), "stream sync");
    memcpy(outh, g_hout.p, (size_t)S * D * 4);
    if (g_prof) prof_flush();
    return 0;
}

extern "C" int lag_hip_moe_group_g(float *acc, const float *x, const void *gu_q, const float *gu_s,
                                   const void *dn_q, const float *dn_s, const int *gexp, const int *gbeg,
                                   const int *gcnt, int G, const int *grow, const int *rowof, const float *w,
                                   int S, int K, int I, int D, int gs) {
    if ((D & 1) || (I & 1)) return -1;
    return grouped_host(acc, x, S, gu_q, gu_s, dn_q, dn_s, gexp, gbeg, gcnt, G, grow, rowof, w, K, I, D, gs, 1);
}
extern "C" int lag_hip_moe_group(float *acc, const float *x, const void *gu_q, const float *gu_s,
                                 const void *dn_q, const float *dn_s, const int *gexp, const int *gbeg,
                                 const int *gcnt, int G, const int *grow, const int *rowof, const float *w,
                                 int S, int K, int I, int D) {
    return lag_hip_moe_group_g(acc, x, gu_q, gu_s, dn_q, dn_s, gexp, gbeg, gcnt, G, grow, rowof, w, S, K, I, D, 0);
}

extern "C" int lag_hip_moe_experts_g(float *out, const float *x, const void *gu_q, const float *gu_s,
                                     const void *dn_q, const float *dn_s, const int *sel, const float *w,
                                     int K, int I, int D, int gs) {
    if (K <= 0 || K > 1024 || (D & 1) || (I & 1)) return -1;
    std::vector<int> gbeg(K), gcnt(K, 1), grow(K, 0), rowof(K);
    for (int a = 0; a < K; a++) { gbeg[a] = a; rowof[a] = a; }
    return grouped_host(out, x, 1, gu_q, gu_s, dn_q, dn_s, sel, gbeg.data(), gcnt.data(), K, grow.data(), rowof.data(),
                        w, K, I, D, gs, 1);
}
extern "C" int lag_hip_moe_experts(float *out, const float *x, const void *gu_q, const float *gu_s,
                                   const void *dn_q, const float *dn_s, const int *sel, const float *w,
                                   int K, int I, int D) {
    return lag_hip_moe_experts_g(out, x, gu_q, gu_s, dn_q, dn_s, sel, w, K, I, D, 0);
}

extern "C" int lag_hip_expert_q4_g(float *out, const float *x, const void *p13, const void *s13,
                                   const void *p2, const void *s2, int I, int D, int gs) {
    const int zero = 0, one = 1;
    const float wone = 1.0f;
    return grouped_host(out, x, 1, p13, (const float *)s13, p2, (const float *)s2, &zero, &zero, &one, 1, &zero, &zero,
                        &wone, 1, I, D, gs, 0);
}
extern "C" int lag_hip_expert_q4(float *out, const float *x, const void *p13, const void *s13,
                                 const void *p2, const void *s2, int I, int D) {
    return lag_hip_expert_q4_g(out, x, p13, s13, p2, s2, I, D, 0);
}

// The reference CPU's 16-lane GEMV contracts, bit for bit (k_lanes.hip): host
// x and y, device weights.  Every row of every call takes them, so a token's
// result does not depend on how many rows share its call (an engine's
// per-token and chunked paths agree bit for bit, as on the CPU).
static int lanes_host(float *y, const float *x, const void *W, int wkind, int dp, const void *scale, int S, int I, int O,
                      int gs = 0) {
    if (!g_ok || fault_injected()) return -1;
    if (S <= 0 || I <= 0 || O <= 0 || !W) return -1;
    Carve cv;
    const size_t o_x = cv.take((size_t)S * I * 4), o_y = cv.take((size_t)S * O * 4);
    if (grow_dev(g_arena, cv.off) || grow_pinned(g_hin, (size_t)S * I * 4) || grow_pinned(g_hout, (size_t)S * O * 4)) return -1;
    char *A = (char *)g_arena.p;
    memcpy(g_hin.p, x, (size_t)S * I * 4);
    CK(hipMemcpyAsync(A + o_x, g_hin.p, (size_t)S * I * 4, hipMemcpyHostToDevice, g_st), "x upload");
    { PROF("lanes16");
      if (sw_launch_lanes16(g_st, W, wkind, dp, (const float *)scale, (const float *)(A + o_x), S, I, O, (float *)(A + o_y), gs))
          return fail_msg("lanes launch (shape unsupported?)"); }
    CK(hipMemcpyAsync(g_hout.p, A + o_y, (size_t)S * O * 4, hipMemcpyDeviceToHost, g_st), "result download");
    CK(hipStreamSynchronize(g_st), "stream sync");
    memcpy(y, g_hout.p, (size_t)S * O * 4);
    if (g_prof) prof_flush();
    return 0;
}

extern "C" int lag_hip_matmul_bf16_rx(float *y, const float *x, const void *W, int S, int I, int O) {
    return lanes_host(y, x, W, 0, I % 32 == 0, nullptr, S, I, O);
}
extern "C" int lag_hip_matmul_q8_s(float *y, const float *x, const void *q8, const void *scale, int S, int I, int O) {
    if (!scale) return -1;
    return lanes_host(y, x, q8, 1, 0, scale, S, I, O);
}
extern "C" int lag_hip_matmul_q8(float *y, const float *x, const void *W, int S, int I, int O) {
    if (!W) return -1;
    return lag_hip_matmul_q8_s(y, x, W, (const char *)W + (size_t)I * O, S, I, O);
}

extern "C" int lag_hip_matmul_q4_g(float *y, const float *x, const void *packed, const void *scale,
                                   int S, int I, int O, int gs) {
    // per-row scales: matmul_q4_k's lanes; group scales: matmul_i4_grouped's lanes, the
    // scales applied in f32 per group
    if (gs <= 0) return (I & 1) ? -1 : lanes_host(y, x, packed, 2, 0, scale, S, I, O);
    if (gs % 16 || I % gs || (gs <= 256 ? 256 % gs : gs % 256))
        return fail_msg("matmul_q4_g: group size unsupported (a multiple of 16 dividing 256, or of 256, dividing I)");
    return lanes_host(y, x, packed, 3, 0, scale, S, I, O, gs);
}
extern "C" int lag_hip_matmul_q4(float *y, const float *x, const void *packed, const void *scale, int S, int I, int O) {
    if (I & 1) return -1;
    return lag_hip_matmul_q4_g(y, x, packed, scale, S, I, O, 0);
}

extern "C" int lag_hip_matmul_bf16(float *y, const float *x, const void *W, int S, int I, int O) {
    return lanes_host(y, x, W, 0, 0, nullptr, S, I, O);
}

// ------------------------------------------------------------ device MoE block ----
extern "C" void *lag_hip_router_upload(const void *W, int E, int D, int w_bf16) {
    if (!g_ok || !W || E <= 0 || D % 128) return nullptr;
    const size_t n = (size_t)E * D * (w_bf16 ? 2 : 4);
    void *tmp = lag_hip_upload(W, n);
    if (!tmp) return nullptr;
    void *out = nullptr;
    if (hipMalloc(&out, (size_t)((E + 3) / 4) * 4 * D * (w_bf16 ? 2 : 4)) != hipSuccess) { (void)hipFree(tmp); fail("router allocation", hipErrorOutOfMemory); return nullptr; }
    if (sw_launch_chain_major(g_st, tmp, w_bf16, E, D, out) || hipStreamSynchronize(g_st) != hipSuccess) {
        (void)hipFree(tmp); (void)hipFree(out); fail("router transform", hipErrorUnknown); return nullptr;
    }
    (void)hipFree(tmp);
    return out;
}

extern "C" int lag_hip_router_chain(const void *W, void *Wc, int E, int D, int w_bf16) {
    if (!g_ok || !W || !Wc) return -1;
    if (sw_launch_chain_major(g_st, W, w_bf16, E, D, Wc)) return fail_msg("router transform launch");
    return 0;
}

struct FwdScratch {
    float *logits, *scores, *w, *slots, *sout;
    float *wsh;             // Inkling: the shared gates' weights [S, ns]
    float *shu;             // GATED: the shared experts' up rows [S, ns * Is]
    int *sel, *gexp, *gbeg, *gcnt, *G, *grow, *rowof, *items, *P;
    sw_u32x4 *hl;           // h of every packed row as dot8 limbs
    float *hs;
    float *shh;             // shared expert h [S, Is] (one token: f32)
    uint16_t *shx, *shp;    // a batch's shared expert: the bf16 parts of x [S][D/32][3][32] and of h
    sw_u32x4 *xl;
    float *xs;
    uint32_t *xd, *hd;      // MFMA digits of x [S][D/32] and of h [T][I/32] (prefill)
    float *xds, *hds;
    uint32_t *xq, *hq;      // IDOT int8 activations of x [S][D/32][8] and of h [T][I/32][8]
    float *xqs, *hqs, *hf;  // their block scales; h [T][I] f32
};
static int g_last_G_dev = 0;            // 1: last forward's groups live in the arena
static FwdScratch g_last;
static int g_last_ng = 0;

// router rows and the Inkling gate pool; the shared experts of a layer
static int ink_ns(const LagHipMoeDesc *d) { return d->route_act == SW_ROUTE_INKLING ? d->n_shared : 0; }
static int router_rows(const LagHipMoeDesc *d) { return d->n_experts + ink_ns(d); }
static int shared_count(const LagHipMoeDesc *d) {
    return d->shared_mode == LAG_HIP_SHARED_GATED ? d->n_shared : d->shared_mode ? 1 : 0;
}
// the scale the combine applies to the routed sum: Inkling's weights already hold it
static float combine_scale(const LagHipMoeDesc *d) { return d->route_act == SW_ROUTE_INKLING ? 1.0f : d->route_scale; }

static int desc_ok(const LagHipMoeDesc *d, const LagHipMoeWeights *w) {
    if (!d || !w) return 0;
    if (d->shared_mode != LAG_HIP_SHARED_NONE && d->shared_mode != LAG_HIP_SHARED_UNSCALED &&
        d->shared_mode != LAG_HIP_SHARED_GATED) return 0;
    if (d->route_act == SW_ROUTE_INKLING) {          // its own gate pool; no router-hook bias
        if (d->n_shared < 0 || d->n_shared > 64 || w->logit_bias) return 0;
        if (d->shared_mode == LAG_HIP_SHARED_UNSCALED) return 0;
        if (d->n_experts + d->n_shared > 1024) return 0;
    }
    if (d->shared_mode == LAG_HIP_SHARED_GATED && (d->route_act != SW_ROUTE_INKLING || d->n_shared < 1)) return 0;
    // (E <= 1024: the gate/top-k wave and the counting sort hold every expert on chip)
    if (d->n_experts <= 0 || d->n_experts > 1024 || d->topk <= 0 || d->topk > d->n_experts || d->topk > 64) return 0;
    if (d->route_act < 0 || d->route_act > SW_ROUTE_ACT_MAX) return 0;
    if (d->hidden % 128 || d->moe_inter % 128) return 0;
    if (d->gs > 0 && (d->gs % 32 || d->hidden % d->gs || d->moe_inter % d->gs)) return 0;
    if (d->shared_mode && (!w->sg || !w->su || !w->sd || d->shared_inter % 128)) return 0;
    if (!w->router || !w->gu_q || !w->gu_s || !w->dn_q || !w->dn_s) return 0;
    return 1;
}

// Where a forward's scratch comes from: the growing arena (fixed null), or a
// caller-provided region of fixed capacity that nothing may outgrow.
struct ScratchSrc { char *fixed; size_t cap; };
static const ScratchSrc kArena = {nullptr, 0};

// need: only report the bytes the layout takes (nothing allocated or assigned)
static int carve_fwd(const LagHipMoeDesc *d, int S, FwdScratch &f, const ScratchSrc &src, bool idot = false,
                     size_t *need = nullptr) {
    const int E = d->n_experts, K = d->topk, D = d->hidden, I = d->moe_inter, Is = d->shared_inter;
    const int T = S * K, R = router_rows(d), nsx = shared_count(d);
    Carve cv;
    const size_t o_lg = cv.take((size_t)S * R * 4), o_sc = cv.take((size_t)S * R * 4);
    const size_t o_wsh = cv.take((size_t)S * (ink_ns(d) > 0 ? ink_ns(d) : 1) * 4);
    const size_t o_sel = cv.take((size_t)T * 4), o_w = cv.take((size_t)T * 4);
    const size_t o_gexp = cv.take((size_t)E * 4), o_gbeg = cv.take((size_t)E * 4), o_gcnt = cv.take((size_t)E * 4);
    const size_t o_G = cv.take(4), o_grow = cv.take((size_t)T * 4), o_rowof = cv.take((size_t)T * 4);
    const size_t o_items = cv.take((size_t)sw_npass_max(T, E, 1) * 4), o_P = cv.take(4);   // (one token per pass at most)
    const size_t o_hl = cv.take((size_t)T * (I / 32) * SW_NL * 16), o_hs = cv.take((size_t)T * (I / 32) * 4);
    const size_t o_slot = cv.take(S > 1 || idot ? (size_t)T * D * 4 : 4);
    size_t o_sh = 0, o_so = 0, o_su = 0;
    if (d->shared_mode) { o_sh = cv.take((size_t)S * nsx * Is * 4); o_so = cv.take((size_t)S * nsx * D * 4); }
    if (d->shared_mode == LAG_HIP_SHARED_GATED) o_su = cv.take((size_t)S * nsx * Is * 4);
    // the batch kernels of the unscaled shared expert (also the IDOT forward's at S = 1)
    const bool shb = d->shared_mode == LAG_HIP_SHARED_UNSCALED && (S > 1 || idot);
    size_t o_shx = 0, o_shp = 0;
    if (shb) { o_shx = cv.take((size_t)S * D * 6); o_shp = cv.take((size_t)S * Is * 6); }
    const size_t o_xl = cv.take((size_t)S * (D / 32) * SW_NL * 16), o_xs = cv.take((size_t)S * (D / 32) * 4);
    size_t o_xd = 0, o_xds = 0, o_hd = 0, o_hds = 0;
    if (S > 1) {
        o_xd = cv.take((size_t)S * (D / 32) * 128); o_xds = cv.take((size_t)S * (D / 32) * 4);
        o_hd = cv.take((size_t)T * (I / 32) * 128); o_hds = cv.take((size_t)T * (I / 32) * 4);
    }
    size_t o_xq = 0, o_xqs = 0, o_hq = 0, o_hqs = 0, o_hf = 0;
    if (idot) {
        o_xq = cv.take((size_t)S * (D / 32) * 32); o_xqs = cv.take((size_t)S * (D / 32) * 4);
        o_hq = cv.take((size_t)T * (I / 32) * 32); o_hqs = cv.take((size_t)T * (I / 32) * 4);
        o_hf = cv.take((size_t)T * I * 4);
    }
    if (need) { *need = cv.off; return 0; }
    char *A;
    if (src.fixed) {
        if (cv.off > src.cap) {
            snprintf(g_err, sizeof g_err, "moe_forward: S=%d needs %zu bytes of scratch, above the fixed region's %zu",
                     S, cv.off, src.cap);
            return -1;
        }
        A = src.fixed;
    } else {
        if (grow_dev(g_arena, cv.off)) return -1;
        A = (char *)g_arena.p;
    }
    f.xq = idot ? (uint32_t *)(A + o_xq) : nullptr; f.xqs = idot ? (float *)(A + o_xqs) : nullptr;
    f.hq = idot ? (uint32_t *)(A + o_hq) : nullptr; f.hqs = idot ? (float *)(A + o_hqs) : nullptr;
    f.hf = idot ? (float *)(A + o_hf) : nullptr;
    f.logits = (float *)(A + o_lg); f.scores = (float *)(A + o_sc); f.sel = (int *)(A + o_sel); f.w = (float *)(A + o_w);
    f.gexp = (int *)(A + o_gexp); f.gbeg = (int *)(A + o_gbeg); f.gcnt = (int *)(A + o_gcnt); f.G = (int *)(A + o_G);
    f.items = (int *)(A + o_items); f.P = (int *)(A + o_P);
    f.grow = (int *)(A + o_grow); f.rowof = (int *)(A + o_rowof);
    f.hl = (sw_u32x4 *)(A + o_hl); f.hs = (float *)(A + o_hs); f.slots = (float *)(A + o_slot);
    f.shh = d->shared_mode ? (float *)(A + o_sh) : nullptr;
    f.sout = d->shared_mode ? (float *)(A + o_so) : nullptr;
    f.shu = d->shared_mode == LAG_HIP_SHARED_GATED ? (float *)(A + o_su) : nullptr;
    f.shx = shb ? (uint16_t *)(A + o_shx) : nullptr;
    f.shp = shb ? (uint16_t *)(A + o_shp) : nullptr;
    f.wsh = (float *)(A + o_wsh);
    f.xl = (sw_u32x4 *)(A + o_xl); f.xs = (float *)(A + o_xs);
    f.xd = S > 1 ? (uint32_t *)(A + o_xd) : nullptr; f.xds = S > 1 ? (float *)(A + o_xds) : nullptr;
    f.hd = S > 1 ? (uint32_t *)(A + o_hd) : nullptr; f.hds = S > 1 ? (float *)(A + o_hds) : nullptr;
    return 0;
}


// A prefill-sized batch's router, and a head-sized one (R rows), run over token tiles
// (each weight slice read once per tile, the same bits as the per-token blocks), then
// the limbs of x as a kernel of their own; smaller batches keep the fused routing stage
// (B = 32: 11 us against 22 + 4 us tiled, the tiles' x chunks waiting on one wave per CU)
static bool router_tiled(int S, int D, int R) { return S >= 2 && D % 256 == 0 && (S >= 512 || R >= 4096); }
static int router_batch(const void *Wc, int w_bf16, const float *x, int S, int D, int R, const float *lbias,
                        float *logits, float *scores, int act, sw_u32x4 *xl, float *xs) {
    { PROF("router_tiles");
      if (sw_launch_router_tiles(g_st, Wc, w_bf16, x, S, D, R, lbias, logits, scores, act))
          return fail_msg("router launch (shape unsupported?)"); }
    if (xl) {
        PROF("limbs");
        if (sw_launch_limbs(g_st, x, S, D, xl, xs)) return fail_msg("limbs launch");
    }
    return 0;
}

// router logits (+ scores); with sel, gate + top-k; with xl, the dot8 limbs of x
static int route_dev(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, int S, float *logits,
                     float *scores, int *sel, float *wts, sw_u32x4 *xl = nullptr, float *xs = nullptr) {
    PROF("router_topk");
    // Inkling: the picks' weights then the shared gates' in one row of K + ns
    const int ns = ink_ns(d), K = d->topk;
    const SwGateOpt o = {router_rows(d), ns, d->route_scale, K + ns, ns ? wts + K : nullptr, K + ns};
    if (router_tiled(S, d->hidden, router_rows(d))) {
        if (router_batch(w->router, d->router_bf16, x, S, d->hidden, router_rows(d), w->logit_bias, logits, scores,
                         d->route_act, xl, xs)) return -1;
        if (sel && sw_launch_gate_topk(g_st, logits, scores, S, d->n_experts, K, d->route_act, w->corr_bias,
                                       d->use_corr_bias, d->norm_topk, sel, wts, &o)) return fail_msg("gate/top-k launch");
        return 0;
    }
    if (sw_launch_router_topk(g_st, w->router, d->router_bf16, x, S, d->hidden, d->n_experts, w->logit_bias, logits,
                              scores, d->topk, d->route_act, w->corr_bias, d->use_corr_bias, d->norm_topk,
                              sel, wts, xl, xs, &o)) return fail_msg("router launch");
    return 0;
}

// the gate + top-k launch of the forward: weights [S, K], Inkling's shared gates' to f.wsh
static int gate_dev(const LagHipMoeDesc *d, const LagHipMoeWeights *w, int S, FwdScratch &f) {
    PROF("gate_topk");
    const int ns = ink_ns(d);
    const SwGateOpt o = {router_rows(d), ns, d->route_scale, d->topk, ns ? f.wsh : nullptr, ns};
    if (sw_launch_gate_topk(g_st, f.logits, f.scores, S, d->n_experts, d->topk, d->route_act, w->corr_bias,
                            d->use_corr_bias, d->norm_topk, f.sel, f.w, &o)) return fail_msg("gate/top-k launch");
    return 0;
}

// a batch's unscaled shared expert, gate_up: the parts of x (unless the routing stage
// wrote them), then h's parts (f.shp)
static int shared_glu_batch(const LagHipMoeWeights *w, const float *x, int S, int D, int Is, FwdScratch &f,
                            bool have_parts = false) {
    PROF("shared_glu");
    if (!have_parts && sw_launch_sh_parts(g_st, x, S, D, f.shx)) return fail_msg("shared parts launch");
    if (sw_launch_sh_glu(g_st, (const uint16_t *)w->sg, (const uint16_t *)w->su, f.shx, S, D, Is, f.shp))
        return fail_msg("shared gate_up launch (shape unsupported?)");
    return 0;
}

// Inkling's gated shared experts over S rows (c/inkling.c:1166-1183) in matmul_h's
// contract: gate and up rows of all ns experts, SiLU-GLU, then expert j's down into
// sout[s][j][D]
static int gated_shared(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, int S, FwdScratch &f) {
    PROF("gated_shared");
    const int D = d->hidden, Is = d->shared_inter, ns = d->n_shared;
    if (sw_launch_lanes16(g_st, w->sg, 0, 1, nullptr, x, S, D, ns * Is, f.shh, 0) ||
        sw_launch_lanes16(g_st, w->su, 0, 1, nullptr, x, S, D, ns * Is, f.shu, 0) ||
        sw_launch_silu_mul(g_st, f.shh, f.shu, (int64_t)S * ns * Is, f.shh)) return fail_msg("gated shared gate/up launch");
    for (int j = 0; j < ns; j++)
        if (sw_launch_lanes16_ld(g_st, (const uint16_t *)w->sd + (size_t)j * D * Is, 0, 1, nullptr, f.shh + (size_t)j * Is,
                                 ns * Is, S, Is, D, f.sout + (size_t)j * D, ns * D, 0))
            return fail_msg("gated shared down launch");
    return 0;
}

extern "C" int lag_hip_route(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, int S,
                             float *logits, int *sel, float *wts) {
    if (!g_ok || fault_injected() || !desc_ok(d, w) || S <= 0) return -1;
    FwdScratch f;
    if (carve_fwd(d, S, f, kArena)) return -1;
    return route_dev(d, w, x, S, logits ? logits : f.logits, f.scores, sel, wts);
}

// The layer in the IDOT contract (any S): router, gate + top-k, the counting sort, int8
// activations, grouped gate_up GLU, int8 h, grouped down into slots, combine; the
// shared expert as in batches (the same arithmetic as the decode stages).
static int forward_idot(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out, int S,
                        const ScratchSrc &sc) {
    const int E = d->n_experts, K = d->topk, D = d->hidden, I = d->moe_inter, Is = d->shared_inter;
    FwdScratch f;
    if (carve_fwd(d, S, f, sc, true)) return -1;
    SwQ4 gu = {(const uint8_t *)w->gu_q, w->gu_s, 2 * I, D, 0, E};
    SwQ4 dn = {(const uint8_t *)w->dn_q, w->dn_s, D, I, 0, E};
    const bool sh = d->shared_mode == LAG_HIP_SHARED_UNSCALED, gated = d->shared_mode == LAG_HIP_SHARED_GATED;
    if (router_tiled(S, D, router_rows(d))) {
        if (router_batch(w->router, d->router_bf16, x, S, D, router_rows(d), w->logit_bias, f.logits, f.scores,
                         d->route_act, nullptr, nullptr)) return -1;
    } else {
        PROF("stage_route");
        if (sw_launch_stage_route(g_st, w->router, d->router_bf16, x, S, D, router_rows(d), w->logit_bias, f.logits, f.scores,
                                  d->route_act, nullptr, f.xs, nullptr, nullptr, Is, f.shh)) return fail_msg("routing stage launch");
    }
    if (sh && shared_glu_batch(w, x, S, D, Is, f)) return -1;
    if (gated && gated_shared(d, w, x, S, f)) return -1;
    if (gate_dev(d, w, S, f)) return -1;
    { PROF("bucket");
      if (sw_launch_bucket(g_st, f.sel, S, K, E, f.gexp, f.gbeg, f.gcnt, f.G, f.grow, f.rowof, 1, nullptr, nullptr))
          return fail_msg("bucket launch"); }
    const SwGroups g = {f.gexp, f.gbeg, f.gcnt, f.grow, f.G, S * K < E ? S * K : E, 0, nullptr, nullptr};
    SwGroups gd = g;
    gd.grow = nullptr;                     // the down reads the packed rows directly
    { PROF("idot_quant"); if (sw_launch_idot_quant(g_st, x, S, D, f.xq, f.xqs)) return fail_msg("IDOT quant launch"); }
    { PROF("idot_glu"); if (sw_launch_idot_glu(g_st, gu, f.xq, f.xqs, g, I, f.hf)) return fail_msg("IDOT gate_up launch"); }
    if (sh) {
        PROF("shared_down");
        if (sw_launch_sh_down(g_st, (const uint16_t *)w->sd, f.shp, S, Is, D, f.sout)) return fail_msg("shared down launch");
    }
    { PROF("idot_quant"); if (sw_launch_idot_quant(g_st, f.hf, S * K, I, f.hq, f.hqs)) return fail_msg("IDOT quant launch"); }
    { PROF("idot_down"); if (sw_launch_idot_rows(g_st, dn, f.hq, f.hqs, gd, f.slots)) return fail_msg("IDOT down launch"); }
    { PROF("combine");
      if (sw_launch_combine(g_st, f.slots, f.rowof, f.w, S, K, D, combine_scale(d), f.sout, out, 1,
                            gated ? f.wsh : nullptr, gated ? d->n_shared : 0))
          return fail_msg("combine launch"); }
    g_last_G_dev = 1; g_last_ng = 0;
    g_last = f;
    return 0;
}

// One decode step (sabrewing's moe_block over S tokens, device pointers).
// S == 1, three launches:
//   stage 1  router logits / scores / limbs of x + the shared expert's gate_up
//   stage 2  every block re-derives the gate + top-k (E <= 256), then the
//            routed gate_up; + the shared expert's down
//   stage 3  routed down fused with the rank-order combine (+ shared, residual)
// S > 1: routing stage, gate + top-k, shared gate_up over token tiles, the
// counting sort, grouped gate_up, shared down, grouped down into slots, combine;
// the grouped GEMMs on dot8 (passes of 2 tokens) or, for prefill-sized batches,
// on the f16 MFMA (tiles of up to 64 tokens, the inputs as MFMA digits).
// nw: x holds raw rows, normalised by the routing launch's router blocks (RMSNorm with
// weights nw, eps) into xn, which every later launch reads in x's place
static int forward(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out, int S,
                   const ScratchSrc &sc, const float *nw = nullptr, float eps = 0.f, float *xn = nullptr) {
    if (!g_ok || fault_injected()) return -1;
    if (!desc_ok(d, w) || S <= 0) return fail_msg("moe_forward: unsupported descriptor/shape");
    if (g_q4_mode == 1 && d->gs == 0) return forward_idot(d, w, x, out, S, sc);
    const int E = d->n_experts, K = d->topk, D = d->hidden, I = d->moe_inter, Is = d->shared_inter;
    const int T = S * K;
    FwdScratch f;
    if (carve_fwd(d, S, f, sc)) return -1;
    SwQ4 gu = {(const uint8_t *)w->gu_q, w->gu_s, 2 * I, D, d->gs, E};
    SwQ4 dn = {(const uint8_t *)w->dn_q, w->dn_s, D, I, d->gs, E};
    // sh: moe_block's unscaled shared expert (the laguna contract); gated: Inkling's pool
    const bool sh = d->shared_mode == LAG_HIP_SHARED_UNSCALED, gated = d->shared_mode == LAG_HIP_SHARED_GATED;
    const uint16_t *sg = sh ? (const uint16_t *)w->sg : nullptr, *su = sh ? (const uint16_t *)w->su : nullptr;
    const uint16_t *sd = sh ? (const uint16_t *)w->sd : nullptr;
    const float rs_c = combine_scale(d);
    const float *wsh = gated ? f.wsh : nullptr;
    const int nsg = gated ? d->n_shared : 0;
    // one token with E <= 256: its gate + top-k runs in every block of the
    // expert stage (no device-scope handoff); otherwise a gate + top-k launch
    // after the routing stage
    const bool in_experts = E <= 256 && S == 1 && (d->route_act == 1 || sw_act_scores(d->route_act));
    // S == 1: the shared expert's gate_up and down run as extra blocks of stages 1 and 2
    // (they fill the chip while the routed chain waits on its router and top-k);
    // S > 1: as extra blocks of other launches (below) or, for prefill-sized batches, as
    // kernels of their own over token tiles (the same arithmetic per token either way)
    const bool sh_in = sh && S == 1;
    const bool mf = S > 1 && use_mfma(T, E, D, I);
    // a decode-sized batch on the dot8 kernels: the shared expert's split-K blocks ride in
    // other launches -- up to 32 tokens in the expert stage (gate_up) and the combine
    // (down); beyond, in the routing stage (gate_up) and the expert stage (down), where
    // the down's 32-token tiles re-read its weights less often than the combine's would
    const bool sh_fused = sh && S > 1 && !mf && S <= SH_SK_MAX_S && !router_tiled(S, D, router_rows(d));
    const bool sh_late = sh_fused && S <= 32;
    if (router_tiled(S, D, router_rows(d))) {
        if (router_batch(w->router, d->router_bf16, x, S, D, router_rows(d), w->logit_bias, f.logits, f.scores,
                         d->route_act, mf ? nullptr : f.xl, f.xs)) return -1;
    } else {
        PROF("stage_route");
        if (sw_launch_stage_route(g_st, w->router, d->router_bf16, x, S, D, router_rows(d), w->logit_bias, f.logits, f.scores,
                                  d->route_act, mf ? nullptr : f.xl, f.xs, sh_in || (sh_fused && !sh_late) ? sg : nullptr, su,
                                  Is, f.shh, sh && !sh_in && !sh_fused ? f.shx : nullptr,
                                  sh_fused && !sh_late ? f.shp : nullptr, nw, eps, xn))
            return fail_msg("routing stage launch");
    }
    if (nw) x = xn;                      // the normalised rows from here on
    if (gated && gated_shared(d, w, x, S, f)) return -1;
    if (mf) {
        PROF("digits");
        if (sw_launch_digits(g_st, x, S, D, f.xd, f.xds)) return fail_msg("digits launch");
    }
    if (sh && !sh_in && !sh_fused && shared_glu_batch(w, x, S, D, Is, f, !router_tiled(S, D, router_rows(d)))) return -1;
    // a small batch on the dot8 kernels: its gate + top-k and the bucketing in one launch
    // (up to 8 tokens, a wave each; beyond, a wave's several top-ks in a row cost more
    // than the launch saves: 10.9 against 9.2 us at 16 tokens)
    const bool gate_bucket = !in_experts && S > 1 && S <= 8 && !mf && E <= 1024;
    if (!in_experts && !gate_bucket && gate_dev(d, w, S, f)) return -1;
    if (S == 1) {                        // one token: its K picks in rank order, fused down + combine
        { PROF("stage_experts");
          if (sw_launch_stage_experts(g_st, gu, f.xl, f.xs, SwGroups{}, I, f.hl, f.hs, f.sel, K,
                                      in_experts ? (sw_act_softmax(d->route_act) ? f.logits : f.scores) : nullptr, E, d->route_act,
                                      w->corr_bias, d->use_corr_bias, d->norm_topk, f.w, sh_in ? sd : nullptr, f.shh, S, Is, D,
                                      f.sout))
              return fail_msg("expert stage launch"); }
        { PROF("q4_down_combine");
          if (sw_launch_q4_dot8_down_combine(g_st, dn, f.hl, f.hs, f.sel, f.w, K, rs_c, sh || gated ? f.sout : nullptr, out,
                                             wsh, nsg))
              return fail_msg("down/combine launch"); }
        g_last_G_dev = 0; g_last_ng = K;
    } else if (mf) {                     // prefill: tiles of up to 64 tokens of a group on the f16 MFMA
        { PROF("bucket");
          // (the split sort's counts in the slots, which the down launch writes later)
          if (sw_launch_bucket(g_st, f.sel, S, K, E, f.gexp, f.gbeg, f.gcnt, f.G, f.grow, f.rowof, SW_MF_TT, f.items, f.P,
                               (int *)f.slots))
              return fail_msg("bucket launch"); }
        SwGroups g = {f.gexp, f.gbeg, f.gcnt, f.grow, f.G, sw_npass_max(T, E, SW_MF_TT), 0, f.items, f.P};
        { PROF("mf_glu");
          if (sw_launch_mf_glu(g_st, gu, f.xd, f.xds, S, g, I, f.hd, f.hds)) return fail_msg("MFMA gate_up launch"); }
        if (sh) {
            PROF("shared_down");
            if (sw_launch_sh_down(g_st, sd, f.shp, S, Is, D, f.sout)) return fail_msg("shared down launch");
        }
        SwGroups gd = g;
        gd.grow = nullptr;                 // the down reads the packed rows directly
        { PROF("mf_down"); if (sw_launch_mf_rows(g_st, dn, f.hd, f.hds, T, gd, f.slots)) return fail_msg("MFMA down launch"); }
        { PROF("combine");
          if (sw_launch_combine(g_st, f.slots, f.rowof, f.w, S, K, D, rs_c, sh || gated ? f.sout : nullptr, out, 1, wsh, nsg))
              return fail_msg("combine launch"); }
        g_last_G_dev = 1; g_last_ng = 0;
    } else {
        // tokens per pass of the grouped kernels: one when the pairs number at most 0.3 E
        // (about one token per group: C5's 64 pairs of 256 experts, 7.19 -> 6.91 ms per
        // step), else SW_DG_TT (B=32: 300 against 316 us with one)
        const int tt = (int64_t)T * 10 <= (int64_t)E * 3 ? 1 : SW_DG_TT;
        if (gate_bucket) {
            PROF("gate_bucket");
            const int ns = ink_ns(d);
            const SwGateOpt o = {router_rows(d), ns, d->route_scale, d->topk, ns ? f.wsh : nullptr, ns};
            if (sw_launch_gate_bucket(g_st, f.logits, f.scores, S, E, K, d->route_act, w->corr_bias, d->use_corr_bias,
                                      d->norm_topk, f.sel, f.w, &o, f.gexp, f.gbeg, f.gcnt, f.G, f.grow, f.rowof, tt,
                                      f.items, f.P))
                return fail_msg("gate/top-k + bucket launch");
        } else {
            PROF("bucket");
            if (sw_launch_bucket(g_st, f.sel, S, K, E, f.gexp, f.gbeg, f.gcnt, f.G, f.grow, f.rowof, tt, f.items, f.P))
                return fail_msg("bucket launch");
        }
        // one block per pass of up to tt tokens of a group (the passes of a group with many
        // tokens spread over blocks instead of queueing in one)
        SwGroups g = {f.gexp, f.gbeg, f.gcnt, f.grow, f.G, sw_npass_max(T, E, tt), 0, f.items, f.P, tt};
        { PROF("stage_experts");
          if (sw_launch_stage_experts(g_st, gu, f.xl, f.xs, g, I, f.hl, f.hs, nullptr, K, nullptr, E, d->route_act,
                                      w->corr_bias, d->use_corr_bias, d->norm_topk, f.w, sh_fused && !sh_late ? sd : nullptr,
                                      f.shh, S, Is, D, f.sout, sh_fused ? f.shp : nullptr, sh_late ? sg : nullptr, su, x))
              return fail_msg("expert stage launch"); }
        if (sh && !sh_fused) {
            PROF("shared_down");
            if (sw_launch_sh_down(g_st, sd, f.shp, S, Is, D, f.sout)) return fail_msg("shared down launch");
        }
        SwGroups gd = g;
        gd.grow = nullptr;                 // the down reads the packed rows directly
        { PROF("q4_down"); if (sw_launch_q4_dot8_rows(g_st, dn, f.hl, f.hs, gd, f.slots)) return fail_msg("down launch"); }
        if (sh_late) {
            PROF("shared_down_combine");
            if (sw_launch_sh_combine(g_st, sd, f.shp, S, Is, D, f.sout, f.slots, f.rowof, f.w, K, rs_c, out))
                return fail_msg("shared down + combine launch");
        } else {
            PROF("combine");
            if (sw_launch_combine(g_st, f.slots, f.rowof, f.w, S, K, D, rs_c, sh || gated ? f.sout : nullptr, out, 1, wsh, nsg))
                return fail_msg("combine launch");
        }
        g_last_G_dev = 1; g_last_ng = 0;
    }
    g_last = f;
    return 0;
}

extern "C" int lag_hip_moe_forward(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out, int S) {
    return forward(d, w, x, out, S, kArena);
}

// a stack layer: xn = rmsnorm(h), h += MoE(xn) -- the norm inside the routing launch
// when the routing stage runs (below 512 tokens), no shared expert reads x, and the
// default contract is on; else the two launches of lag_hip_rmsnorm and the forward
extern "C" int lag_hip_moe_forward_rmsnorm(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *norm_w,
                                           float eps, float *xn, float *h, int S) {
    if (!g_ok || !d || !w || !norm_w || !xn || !h || S <= 0) return -1;
    if (!desc_ok(d, w)) return fail_msg("moe_forward_rmsnorm: unsupported descriptor/shape");
    const bool fuse = d->shared_mode == LAG_HIP_SHARED_NONE && !router_tiled(S, d->hidden, router_rows(d)) &&
                      !(g_q4_mode == 1 && d->gs == 0);
    if (!fuse) {
        if (lag_hip_rmsnorm(h, norm_w, xn, S, d->hidden, eps)) return -1;
        return forward(d, w, xn, h, S, kArena);
    }
    return forward(d, w, h, h, S, kArena, norm_w, eps, xn);
}

// ------------------------------------------------- the allocation-free forward ----
// lag_hip_moe_forward with its scratch in a file-scope device array instead of
// the arena: no allocation of any kind, for callers that cannot allocate (code
// under graph capture, tight serving loops).  Each device holds its own copy of
// the array; the host name `scratch` is only a stand-in, so its device address
// is looked up once per device (lag_hip_init, with that device current) and
// only that address is ever handed to kernels.  Nothing in it must start at
// zero: every word a launch reads was written earlier in the same call.
// Calls that overlap on one device share the array and race.
#define SW_NOALLOC_MAX_DEV 64
#define SW_NOALLOC_SCRATCH_BYTES LAG_HIP_NOALLOC_SCRATCH_BYTES
static __device__ __align__(256) char scratch[SW_NOALLOC_SCRATCH_BYTES];
static char *g_scratch_ptr[SW_NOALLOC_MAX_DEV];

static int noalloc_setup(int dev) {
    if (dev < 0 || dev >= SW_NOALLOC_MAX_DEV) return fail_msg("device index beyond the static scratch table");
    if (g_scratch_ptr[dev]) return 0;
    void *p = nullptr;
    CK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "static scratch address");
    g_scratch_ptr[dev] = (char *)p;
    return 0;
}

extern "C" size_t lag_hip_moe_forward_scratch_bytes(const LagHipMoeDesc *d, const LagHipMoeWeights *w, int S) {
    if (!desc_ok(d, w) || S <= 0) return 0;
    FwdScratch f;
    size_t n = 0;
    return carve_fwd(d, S, f, kArena, g_q4_mode == 1 && d->gs == 0, &n) ? 0 : n;
}

extern "C" int lag_hip_moe_forward_noalloc(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out,
                                           int S) {
    if (!g_ok) return fail_msg("moe_forward_noalloc: backend not initialised");
    if (g_dev < 0 || g_dev >= SW_NOALLOC_MAX_DEV || !g_scratch_ptr[g_dev])
        return fail_msg("moe_forward_noalloc: the static scratch of this device is unavailable");
    const int prof = g_prof;
    g_prof = 0;                                  // the per-launch timing pool allocates events
    const int rc = forward(d, w, x, out, S, ScratchSrc{g_scratch_ptr[g_dev], SW_NOALLOC_SCRATCH_BYTES});
    g_prof = prof;
    return rc;
}

// ------------------------------------------------------------ stack glue ----
extern "C" int lag_hip_rmsnorm(const float *x, const float *w, float *out, int S, int D, float eps) {
    if (!g_ok || fault_injected() || !x || !w || !out) return -1;
    PROF("rmsnorm");
    if (sw_launch_rmsnorm(g_st, x, w, out, S, D, eps)) return fail_msg("rmsnorm launch");
    return 0;
}

extern "C" int lag_hip_argmax(const float *logits, int S, int V, int *tok) {
    if (!g_ok || fault_injected() || !logits || !tok) return -1;
    PROF("argmax");
    if (sw_launch_argmax(g_st, logits, S, V, tok)) return fail_msg("argmax launch");
    return 0;
}

extern "C" int lag_hip_head_argmax(const void *Wc, int w_bf16, const float *x, int S, int D, int V, float *logits, int *tok) {
    if (!g_ok || fault_injected() || !Wc || !x || !logits || S <= 0 || V <= 0) return -1;
    { PROF("head_logits");
      if (router_tiled(S, D, V) ? sw_launch_router_tiles(g_st, Wc, w_bf16, x, S, D, V, nullptr, logits, nullptr, 1)
                             : sw_launch_router_topk(g_st, Wc, w_bf16, x, S, D, V, nullptr, logits, nullptr, 1, 1, nullptr, 0, 0,
                                                     nullptr, nullptr, nullptr, nullptr))
          return fail_msg("head launch (shape unsupported?)"); }
    if (tok) {
        PROF("argmax");
        if (sw_launch_argmax(g_st, logits, S, V, tok)) return fail_msg("argmax launch");
    }
    return 0;
}

extern "C" int lag_hip_last_groups(int *G, int *gexp, int *gbeg, int *gcnt, int cap) {
    if (!g_ok) return -1;
    CK(hipStreamSynchronize(g_st), "stream sync");
    if (!g_last_G_dev) { *G = g_last_ng; return 0; }
    CK(hipMemcpy(G, g_last.G, 4, hipMemcpyDeviceToHost), "G download");
    const int n = *G < cap ? *G : cap;
    if (n > 0) {
        CK(hipMemcpy(gexp, g_last.gexp, (size_t)n * 4, hipMemcpyDeviceToHost), "gexp download");
        CK(hipMemcpy(gbeg, g_last.gbeg, (size_t)n * 4, hipMemcpyDeviceToHost), "gbeg download");
        CK(hipMemcpy(gcnt, g_last.gcnt, (size_t)n * 4, hipMemcpyDeviceToHost), "gcnt download");
    }
    return 0;
}

extern "C" int lag_hip_moe_block(const LagHipMoeDesc *d, const LagHipMoeWeights *w, const float *x, float *out, int S) {
    if (!g_ok || !d || S <= 0) return -1;
    static Buf dx, dout;
    const size_t n = (size_t)S * d->hidden * 4;
    if (grow_dev(dx, n) || grow_dev(dout, n) || grow_pinned(g_hin, n) || grow_pinned(g_hout, n)) return -1;
    memcpy(g_hin.p, x, n);
    memcpy(g_hout.p, out, n);
    CK(hipMemcpyAsync(dx.p, g_hin.p, n, hipMemcpyHostToDevice, g_st), "x upload");
    CK(hipMemcpyAsync(dout.p, g_hout.p, n, hipMemcpyHostToDevice, g_st), "out upload");
    if (lag_hip_moe_forward(d, w, (const float *)dx.p, (float *)dout.p, S)) return -1;
    CK(hipMemcpyAsync(g_hout.p, dout.p, n, hipMemcpyDeviceToHost, g_st), "out download");
    CK(hipStreamSynchronize(g_st), "stream sync");
    memcpy(out, g_hout.p, n);
    if (g_prof) prof_flush();
    return 0;
}

// ------------------------------------------------------------ events / profile ----
extern "C" void *lag_hip_event_create(void) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return (void *)e;
}
extern "C" int lag_hip_event_record(void *ev) {
    if (!g_ok || !ev) return -1;
    CK(hipEventRecord((hipEvent_t)ev, g_st), "event record");
    return 0;
}
extern "C" float lag_hip_event_elapsed_ms(void *a, void *b) {
    float ms = -1.f;
    if (hipEventSynchronize((hipEvent_t)b) != hipSuccess) return -1.f;
    if (hipEventElapsedTime(&ms, (hipEvent_t)a, (hipEvent_t)b) != hipSuccess) return -1.f;
    return ms;
}
extern "C" void lag_hip_event_destroy(void *ev) { if (ev) (void)hipEventDestroy((hipEvent_t)ev); }

extern "C" int lag_hip_profile(int enable) {
    if (!enable) prof_flush();
    g_prof = enable ? 1 : 0;
    return 0;
}
extern "C" int lag_hip_profile_count(void) { prof_flush(); return (int)g_prof_recs.size(); }
extern "C" int lag_hip_profile_read(int idx, char *name, int cap, double *total_ms, long long *launches) {
    prof_flush();
    if (idx < 0 || idx >= (int)g_prof_recs.size()) return -1;
    if (name && cap > 0) { strncpy(name, g_prof_recs[idx].name.c_str(), (size_t)cap - 1); name[cap - 1] = 0; }
    if (total_ms) *total_ms = g_prof_recs[idx].ms;
    if (launches) *launches = g_prof_recs[idx].n;
    return 0;
}
extern "C" void lag_hip_profile_reset(void) { prof_flush(); g_prof_recs.clear(); }

// ------------------------------------------------------------ generators ----
extern "C" int lag_hip_gen_normal(float *out, int64_t n, uint64_t seed, uint64_t offset, double sigma, int to_bf16) {
    if (!g_ok) return -1;
    if (sw_launch_gen_normal(g_st, out, n, seed, offset, sigma, to_bf16)) return fail_msg("gen launch");
    return 0;
}
extern "C" int lag_hip_gen_bf16(uint16_t *out, int64_t n, uint64_t seed, uint64_t offset, double sigma) {
    if (!g_ok) return -1;
    if (sw_launch_gen_bf16(g_st, out, n, seed, offset, sigma)) return fail_msg("gen launch");
    return 0;
}
extern "C" int lag_hip_gen_q4(uint8_t *q, float *s, uint64_t seed, double sigma, int64_t row0, int64_t nrows, int K, int gs) {
    if (!g_ok) return -1;
    if (sw_launch_gen_q4(g_st, q, s, seed, sigma, row0, nrows, K, gs)) return fail_msg("gen launch");
    return 0;
}

// ------------------------------------------------------------ diagnostics ----
extern "C" int lag_hip_selftest(float *out_host, const float *xin_host, int n) {
    if (!g_ok || n < 0) return -1;
    float *dout = nullptr, *din = nullptr;
    CK(hipMalloc(&dout, (size_t)(768 + 3 * n) * 4), "selftest alloc");
    if (n > 0 && hipMalloc(&din, (size_t)n * 4) != hipSuccess) { (void)hipFree(dout); return fail_msg("selftest alloc"); }
    if (n > 0) CK(hipMemcpy(din, xin_host, (size_t)n * 4, hipMemcpyHostToDevice), "selftest upload");
    int rc = sw_launch_selftest(g_st, dout, din, n);
    if (rc == 0 && hipStreamSynchronize(g_st) != hipSuccess) rc = -1;
    if (rc == 0 && hipMemcpy(out_host, dout, (size_t)(768 + 3 * n) * 4, hipMemcpyDeviceToHost) != hipSuccess) rc = -1;
    (void)hipFree(dout);
    if (din) (void)hipFree(din);
    return rc ? fail_msg("selftest") : 0;
}

extern "C" const char *lag_hip_last_error(void) { return g_err; }

// ------------------------------------------------------------ graphs ----
// Every device-pointer entry issued between begin and end (moe_forward,
// route, d2d) is recorded into one graph, replayed by lag_hip_graph_launch
// with one submission.  The recorded kernels hold raw pointers into the
// scratch arena, so a finished recording takes the arena with it (freed by
// lag_hip_graph_destroy) and no later call, whatever its size, can free or
// move memory that a live graph replays over.  A recording that starts with
// no arena (the previous recording took it) first allocates one of the
// capacity the last arena had, so graphs of the same shapes can be recorded
// back to back; shapes beyond that capacity need an eager call first.
// Destroying a graph while another recording is open is deferred to the end
// of that recording (a stream synchronisation would break the capture).
struct GraphRec { hipGraphExec_t exec; Buf arena; };
static size_t g_arena_last_cap = 0;
static std::vector<GraphRec *> g_graph_deferred;
static void graph_free(GraphRec *r) {
    (void)hipStreamSynchronize(g_st);   // no replay may still be reading the buffers
    (void)hipGraphExecDestroy(r->exec);
    if (r->arena.p) (void)hipFree(r->arena.p);
    delete r;
}
extern "C" int lag_hip_graph_begin(void) {
    if (!g_ok || g_capturing) return -1;
    prof_flush();
    if (!g_arena.p && g_arena_last_cap) {
        CK(hipMalloc(&g_arena.p, g_arena_last_cap), "device scratch allocation");
        g_arena.cap = g_arena_last_cap;
    }
    CK(hipStreamBeginCapture(g_st, hipStreamCaptureModeRelaxed), "begin capture");
    g_capturing = 1;
    return 0;
}
extern "C" void *lag_hip_graph_end(void) {
    if (!g_ok || !g_capturing) return nullptr;
    g_capturing = 0;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(g_st, &graph);
    for (GraphRec *r : g_graph_deferred) graph_free(r);
    g_graph_deferred.clear();
    if (e != hipSuccess || !graph) { fail("end capture", e); return nullptr; }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) { fail("graph instantiate", e); return nullptr; }
    GraphRec *r = new GraphRec{exec, g_arena};
    if (g_arena.cap) g_arena_last_cap = g_arena.cap;
    g_arena = Buf{};
    g_last_G_dev = 0;                   // the last groups now live in the graph's arena
    g_last_ng = 0;
    return (void *)r;
}
extern "C" int lag_hip_graph_launch(void *g) {
    if (!g_ok || !g || g_capturing) return -1;
    CK(hipGraphLaunch(((GraphRec *)g)->exec, g_st), "graph launch");
    return 0;
}
extern "C" void lag_hip_graph_destroy(void *g) {
    if (!g) return;
    if (g_capturing) g_graph_deferred.push_back((GraphRec *)g);
    else graph_free((GraphRec *)g);
}
