// k_shared.hip -- the shared expert for batches (S > 1) on the bf16 MFMA: the
// three bf16 parts of the inputs, gate_up + SiLU-GLU (writing the parts of h),
// and down.  Per (row, token) the arithmetic is that of the single-token jobs
// of the decode stages (sw_shared.h), so a token's shared expert output does
// not depend on the batch it came in.
//
#include "sw_hip.h"
#include "sw_shared.h"

// parts of the rows of x [S, K] f32 -> [S][K/32][3][32] bf16, 8 inputs per thread
__global__ __launch_bounds__(256) void k_sh_parts(const float *__restrict__ x, int64_t n8, int K,
                                                  uint16_t *__restrict__ parts) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= n8) return;
    const int k8 = K / 8;
    const int64_t tok = c / k8;
    const int cc = (int)(c - tok * k8);
    const sw_f32x4 *xv = (const sw_f32x4 *)(x + tok * K + 8 * cc);
    sw_u32x4 p0, p1, p2;
    sh_split8(xv[0], xv[1], p0, p1, p2);
    uint16_t *dst = parts + tok * K * 3 + (cc >> 2) * 3 * SH_RG + (cc & 3) * 8;
    *(sw_u32x4 *)dst = p0;
    *(sw_u32x4 *)(dst + SH_RG) = p1;
    *(sw_u32x4 *)(dst + 2 * SH_RG) = p2;
}

// Prefill-sized batches.  Block: 4 waves, 128 rows x 64 tokens; wave w takes rows
// 32 w .. +31 (two 16-row tiles) against the four 16-token column tiles.  The
// tokens' part words of a step go through LDS (two buffers: the next step's
// loads are in flight in registers while the waves read this one, issued
// before each step's barrier; C4: 214 -> 202 us for gate_up + down), each
// token's 192 bytes at a padded stride; the waves' weight words come from
// global memory a step ahead.  Blocks are dealt so that an XCD runs whole
// token tiles (all their row blocks), whose part words then come from its L2.
// The fold starts from -0.0, the identity of
// f32 addition (-0 + y == y bit for bit), so every segment is added the same way.
#define SHB_TOK 64             // tokens per block
#define SHB_TS 208             // LDS bytes per token and step: 192 + 16 of padding
#define SHB_STAGE (SHB_TOK * SHB_TS)
#define SHB_CH (SHB_TOK * 12 / 256)   // 16-byte chunks staged per thread per step
template <class RowPtr>
__device__ __forceinline__ void sh_block_tiles(RowPtr rowp, const uint16_t *__restrict__ xp, int S, int K, int tok0,
                                               uint8_t *lds, sw_f32x4 tot[2][4]) {
    const int tid = threadIdx.x, lane = tid & 63, m = lane & 15, kq = lane >> 4;
    const int G = K / SH_RG, GS = G / sh_nseg(G);
    const uint16_t *wr[2];
#pragma unroll
    for (int t = 0; t < 2; t++) wr[t] = rowp(t, m) + 8 * kq;
    // staging: chunk q = u * 256 + tid of a step -> token q / 12, chunk q % 12
    const uint16_t *sp[SHB_CH];
    int so[SHB_CH];
#pragma unroll
    for (int u = 0; u < SHB_CH; u++) {
        const int q = u * 256 + tid, tk = q / 12, ch = q - tk * 12;
        sp[u] = xp + (int64_t)min(tok0 + tk, S - 1) * G * 3 * SH_RG + ch * 8;
        so[u] = tk * SHB_TS + ch * 16;
    }
    auto stage_load = [&](int g, sw_u32x4 *r) {
#pragma unroll
        for (int u = 0; u < SHB_CH; u++) r[u] = *(const sw_u32x4 *)(sp[u] + (int64_t)g * 3 * SH_RG);
    };
    auto stage_store = [&](int buf, const sw_u32x4 *r) {
#pragma unroll
        for (int u = 0; u < SHB_CH; u++) *(sw_u32x4 *)(lds + buf * SHB_STAGE + so[u]) = r[u];
    };
    auto ald = [&](int t, int g) { return *(const sw_u32x4 *)(wr[t] + (int64_t)min(g, G - 1) * SH_RG); };
    sw_f32x4 acc[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            acc[t][c] = sw_f32x4{0.f, 0.f, 0.f, 0.f};
            tot[t][c] = sw_f32x4{-0.f, -0.f, -0.f, -0.f};
        }
    sw_u32x4 an[2] = {ald(0, 0), ald(1, 0)};
    sw_u32x4 sr[SHB_CH];
    stage_load(0, sr);
    stage_store(0, sr);
    if (G > 1) stage_load(1, sr);
    __syncthreads();
    for (int g = 0; g < G; g++) {
        const uint8_t *base = lds + (g & 1) * SHB_STAGE + m * SHB_TS + kq * 16;
        const sw_u32x4 a0 = an[0], a1 = an[1];
        an[0] = ald(0, g + 1);
        an[1] = ald(1, g + 1);
        // column tile c's part words from LDS, tile c + 1's read while c's MFMAs run
        sw_u32x4 b[2][3];
        auto bld = [&](int c, sw_u32x4 *bb) {
#pragma unroll
            for (int p = 0; p < 3; p++) bb[p] = *(const sw_u32x4 *)(base + 16 * c * SHB_TS + 64 * p);
        };
        bld(0, b[0]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            if (c + 1 < 4) bld(c + 1, b[(c + 1) & 1]);
            acc[0][c] = sh_mfma3(a0, b[c & 1][0], b[c & 1][1], b[c & 1][2], acc[0][c]);
            acc[1][c] = sh_mfma3(a1, b[c & 1][0], b[c & 1][1], b[c & 1][2], acc[1][c]);
        }
        if ((g + 1) % GS == 0) {                       // a segment ends: fold it in
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    tot[t][c] = tot[t][c] + acc[t][c];
                    acc[t][c] = sw_f32x4{0.f, 0.f, 0.f, 0.f};
                }
        }
        if (g + 1 < G) stage_store((g + 1) & 1, sr);     // read by no wave since the last barrier
        if (g + 2 < G) stage_load(g + 2, sr);            // registers only: issued before the barrier's wait
        __syncthreads();
    }
}

// block (64 outputs i0 = 64 bx.., 64 tokens): wave w's tile t holds gate rows i0 + 16 w + 8 t
// + 0..7 (tile rows 0-7) and the same up rows (8-15); h's parts [S][Is/32][3][32]
__global__ __launch_bounds__(256) void k_sh_glu_mf(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu,
                                                   const uint16_t *__restrict__ xp, int S, int D, int Is,
                                                   uint16_t *__restrict__ hp) {
    __shared__ __align__(16) uint8_t lds[2 * SHB_STAGE];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4;
    const int nrb = Is / 64, w = sw_xcd_work((int)blockIdx.x, (int)gridDim.x);   // an XCD's blocks: whole token tiles
    const int ib = (w % nrb) * 64 + 16 * wave, tok0 = (w / nrb) * SHB_TOK;
    sw_f32x4 tot[2][4];
    sh_block_tiles([&](int t, int r) {
        const int i = ib + 8 * t + (r & 7);
        return (r < 8 ? Wg : Wu) + (int64_t)i * D;
    }, xp, S, D, tok0, lds, tot);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            // lanes kq < 2 hold gate rows 4 kq + r; lane + 32 holds the up rows of the same outputs
            float hv[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float yg = tot[t][c][r], yu = __shfl_xor(tot[t][c][r], 32);
                hv[r] = (yg / (1.0f + expf(-yg))) * yu;
            }
            const int tok = tok0 + 16 * c + m;
            if (kq < 2 && tok < S) {
                const int i = ib + 8 * t + 4 * kq;      // four consecutive outputs of one group
                uint32_t pa[4], pb[4], pc[4];
#pragma unroll
                for (int r = 0; r < 4; r++) sh_split3(hv[r], pa[r], pb[r], pc[r]);
                uint16_t *dst = hp + (int64_t)tok * Is * 3 + (i >> 5) * 3 * SH_RG + (i & 31);
                *(uint2 *)dst = make_uint2(pa[0] | (pa[1] << 16), pa[2] | (pa[3] << 16));
                *(uint2 *)(dst + SH_RG) = make_uint2(pb[0] | (pb[1] << 16), pb[2] | (pb[3] << 16));
                *(uint2 *)(dst + 2 * SH_RG) = make_uint2(pc[0] | (pc[1] << 16), pc[2] | (pc[3] << 16));
            }
        }
}

// block (128 rows d0 = 128 bx.., 64 tokens): out[tok][d] f32
__global__ __launch_bounds__(256) void k_sh_down_mf(const uint16_t *__restrict__ Wd, const uint16_t *__restrict__ hp, int S,
                                                    int Is, int D, float *__restrict__ out) {
    __shared__ __align__(16) uint8_t lds[2 * SHB_STAGE];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4;
    const int nrb = D / 128, w = sw_xcd_work((int)blockIdx.x, (int)gridDim.x);
    const int db = (w % nrb) * 128 + 32 * wave, tok0 = (w / nrb) * SHB_TOK;
    sw_f32x4 tot[2][4];
    sh_block_tiles([&](int t, int r) { return Wd + (int64_t)(db + 16 * t + r) * Is; }, hp, S, Is, tok0, lds, tot);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int tok = tok0 + 16 * c + m;
            if (tok < S) *(sw_f32x4 *)(out + (int64_t)tok * D + db + 16 * t + 4 * kq) = tot[t][c];
        }
}

// ---- decode-sized batches: K split over the waves (sh_sk_block, sw_shared.h) ----
template <int GLU, int NC>
__global__ __launch_bounds__(SH_SK_NT) void k_sh_sk(ShSkArgs A) {
    __shared__ float red[8 * 16 * 16 * NC];                // [segment][row][token]
    sh_sk_block<GLU, NC, 0>(A, blockIdx.x, blockIdx.y, red);
}
// The shared expert's down fused with the rank-order combine of a decode-sized batch:
// block (bx, by) runs the down of rows 16 bx .. +15 for the 32 tokens of column tile
// by (sh_sk_block, written to shared [S][D]), then combines those outputs of those
// tokens (combine4, the combine launch's arithmetic) into out.  A block's 16 outputs
// are half of each 128-byte line of the slot rows it reads: the row blocks go to the
// XCDs in contiguous ranges, so both halves of a line are read through one L2.
__global__ __launch_bounds__(SH_SK_NT) void k_sh_combine(ShSkArgs A, const float *__restrict__ slots,
                                                        const int *__restrict__ rowof, const float *__restrict__ w, int K,
                                                        float route_scale, float *__restrict__ out) {
    __shared__ float red[8 * 16 * 16 * 2];
    const int rb = sw_xcd_work((int)blockIdx.x, (int)gridDim.x);
    sh_sk_block<0, 2, 0>(A, rb, blockIdx.y, red);
    __syncthreads();                                    // the tile's shared outputs are written
    const int tid = threadIdx.x;
    if (tid < 32 * 4) {
        const int64_t s = (int64_t)blockIdx.y * 32 + (tid >> 2);
        if (s < A.S) combine4(slots, rowof, w, s, K, A.O, rb * 16 + 4 * (tid & 3), route_scale,
                              (const float *)A.out, out, 1, nullptr, 0);
    }
}

// decode-sized batches take the split-K blocks: the gate_up 16-token column tiles up to
// 32 tokens (the grid then fills the chip), else 32-token tiles
template <int GLU>
static int launch_sk(hipStream_t st, const uint16_t *W0, const uint16_t *W1, const uint16_t *xp, int S, int K, int O,
                     void *out) {
    const int nc = sh_sk_nc(GLU, S);
    const dim3 grid((unsigned)sh_sk_rows(GLU, O), (unsigned)sh_sk_cols(S, nc));
    const ShSkArgs A = {W0, W1, xp, nullptr, S, K, O, out};
    if (nc == 1) SW_LAUNCH((k_sh_sk<GLU, 1>), grid, dim3(SH_SK_NT), 0, st, A);
    else SW_LAUNCH((k_sh_sk<GLU, 2>), grid, dim3(SH_SK_NT), 0, st, A);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_sh_parts(hipStream_t st, const float *x, int S, int K, uint16_t *parts) {
    if (S <= 0 || !sh_shape_ok(K)) return -1;
    const int64_t n8 = (int64_t)S * (K / 8);
    SW_LAUNCH(k_sh_parts, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, x, n8, K, parts);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_sh_glu(hipStream_t st, const uint16_t *Wg, const uint16_t *Wu, const uint16_t *xp, int S, int D, int Is,
                     uint16_t *hp) {
    if (S <= 0 || Is % 64 || !sh_shape_ok(D)) return -1;
    if (S <= SH_SK_MAX_S) return launch_sk<1>(st, Wg, Wu, xp, S, D, Is, hp);
    const dim3 grid((unsigned)(Is / 64 * ((S + SHB_TOK - 1) / SHB_TOK)));
    SW_LAUNCH(k_sh_glu_mf, grid, dim3(256), 0, st, Wg, Wu, xp, S, D, Is, hp);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_sh_down(hipStream_t st, const uint16_t *Wd, const uint16_t *hp, int S, int Is, int D, float *out) {
    if (S <= 0 || D % 128 || !sh_shape_ok(Is)) return -1;
    if (S <= SH_SK_MAX_S) return launch_sk<0>(st, Wd, nullptr, hp, S, Is, D, out);
    const dim3 grid((unsigned)(D / 128 * ((S + SHB_TOK - 1) / SHB_TOK)));
    SW_LAUNCH(k_sh_down_mf, grid, dim3(256), 0, st, Wd, hp, S, Is, D, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_sh_combine(hipStream_t st, const uint16_t *Wd, const uint16_t *hp, int S, int Is, int D, float *shared,
                         const float *slots, const int *rowof, const float *w, int K, float route_scale, float *out) {
    if (S <= 0 || S > SH_SK_MAX_S || D % 16 || K <= 0 || !sh_shape_ok(Is)) return -1;
    const ShSkArgs A = {Wd, nullptr, hp, nullptr, S, Is, D, shared};
    const dim3 grid((unsigned)sh_sk_rows(0, D), (unsigned)sh_sk_cols(S, 2));
    SW_LAUNCH(k_sh_combine, grid, dim3(SH_SK_NT), 0, st, A, slots, rowof, w, K, route_scale, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
