// k_shared.hip -- the shared expert for batches (S > 1): gate_up + SiLU-GLU
// and down as standalone kernels over token tiles staged in LDS
// (sh_tile_job, sw_shared.h).  Per (row, token) the arithmetic is that of
// the single-token block jobs the decode stages run, so a token's shared
// expert output does not depend on the batch it came in.
#include "sw_hip.h"

// Per-block timeline, for a build with -DSW_TRACE only: kernel k (0 gate_up,
// 1 down), linear block b: marks (0 start, 1 tile staged, 2.. row batches
// done, 7 end) in sw_trace_mid[(k, b)].
#ifdef SW_TRACE
#define TS_MARK(k, i)                                                                         \
    do {                                                                                      \
        const unsigned b_ = blockIdx.x + gridDim.x * blockIdx.y;                              \
        if (threadIdx.x == 0 && b_ < SW_TRACE_SLOT)                                           \
            sw_trace_mid[((k) * SW_TRACE_SLOT + b_) * 8 + (i)] = wall_clock64();              \
    } while (0)
#define SH_TILE_MARK(i) TS_MARK(NR == 32 ? 0 : 1, i)     // gate_up jobs have 2 * 16 rows
extern "C" int sw_trace_read_mid_shared(void *dst, size_t n) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(sw_trace_mid), n) == hipSuccess ? 0 : -1;
}
#else
#define TS_MARK(k, i)
#endif
#include "sw_shared.h"

// block (set of SHT_GLU_O outputs, token tile): h[tok][i] = silu(gate) * up
__global__ __launch_bounds__(SHT_NT) void k_sh_glu_tile(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu,
                                                      const float *__restrict__ x, int S, int D, int Is,
                                                      float *__restrict__ h) {
    extern __shared__ __align__(16) float lds[];
    __shared__ float ys[2 * SHT_GLU_O * SHT_T];
    TS_MARK(0, 0);
    const int i0 = blockIdx.x * SHT_GLU_O, tok0 = blockIdx.y * SHT_T;
    const int nt = min(SHT_T, S - tok0);
    sh_tile_job([&](int lr) { return (lr < SHT_GLU_O ? Wg : Wu) + (int64_t)(i0 + (lr & (SHT_GLU_O - 1))) * D; },
                2 * SHT_GLU_O, D, x, tok0, nt, [&](int lr, int t, float y) { ys[lr * SHT_T + t] = y; }, lds);
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < SHT_GLU_O * SHT_T) {
        const int lr = tid / SHT_T, t = tid - lr * SHT_T;
        if (t < nt) {
            const float yg = ys[lr * SHT_T + t], yu = ys[(SHT_GLU_O + lr) * SHT_T + t];
            h[(int64_t)(tok0 + t) * Is + i0 + lr] = (yg / (1.0f + expf(-yg))) * yu;
        }
    }
    TS_MARK(0, 7);
}

// block (set of SHT_DN_O output rows, token tile): out[tok][d]
__global__ __launch_bounds__(SHT_NT) void k_sh_down_tile(const uint16_t *__restrict__ Wd, const float *__restrict__ h,
                                                       int S, int Is, int D, float *__restrict__ out) {
    extern __shared__ __align__(16) float lds[];
    TS_MARK(1, 0);
    const int d0 = blockIdx.x * SHT_DN_O, tok0 = blockIdx.y * SHT_T;
    const int nt = min(SHT_T, S - tok0);
    sh_tile_job([&](int lr) { return Wd + (int64_t)(d0 + lr) * Is; }, SHT_DN_O, Is, h, tok0, nt,
                [&](int lr, int t, float y) { out[(int64_t)(tok0 + t) * D + d0 + lr] = y; }, lds);
    TS_MARK(1, 7);
}

// dynamic LDS above 64 KB (gfx950 gives a workgroup up to 160 KB): raised once per
// kernel to the largest size asked so far, outside any stream work
static int set_lds(const void *fn, size_t bytes, size_t &raised) {
    if (bytes > 160 * 1024) return -1;
    if (bytes <= raised) return 0;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) return -1;
    raised = bytes;
    return 0;
}
static size_t g_glu_lds = 0, g_down_lds = 0;

int sw_launch_sh_glu(hipStream_t st, const uint16_t *Wg, const uint16_t *Wu, const float *x, int S, int D, int Is, float *h) {
    if (S <= 0 || Is % SHT_GLU_O || !sh_shape_ok(D) || run_lanes(D / SH_RG) > SHT_NT) return -1;
    const size_t lds = sh_tile_lds(D, 2 * SHT_GLU_O);
    if (set_lds((const void *)k_sh_glu_tile, lds, g_glu_lds)) return -1;
    const dim3 grid((unsigned)(Is / SHT_GLU_O), (unsigned)((S + SHT_T - 1) / SHT_T));
    SW_LAUNCH(k_sh_glu_tile, grid, dim3(SHT_NT), lds, st, Wg, Wu, x, S, D, Is, h);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_sh_down(hipStream_t st, const uint16_t *Wd, const float *h, int S, int Is, int D, float *out) {
    if (S <= 0 || D % SHT_DN_O || !sh_shape_ok(Is) || run_lanes(Is / SH_RG) > SHT_NT) return -1;
    const size_t lds = sh_tile_lds(Is, SHT_DN_O);
    if (set_lds((const void *)k_sh_down_tile, lds, g_down_lds)) return -1;
    const dim3 grid((unsigned)(D / SHT_DN_O), (unsigned)((S + SHT_T - 1) / SHT_T));
    SW_LAUNCH(k_sh_down_tile, grid, dim3(SHT_NT), lds, st, Wd, h, S, Is, D, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
