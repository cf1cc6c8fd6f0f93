// k_shared.hip -- the shared expert's gate_up and down as standalone kernels
// (the block jobs of sw_shared.h; the decode kernels run the same jobs as
// extra blocks).
#include "sw_hip.h"
#include "sw_shared.h"

template <int TT>
__global__ __launch_bounds__(SH_NT) void k_sh_glu(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu,
                                                const float *__restrict__ x, int S, int D, int Is, float *__restrict__ h) {
    extern __shared__ __align__(16) float red[];
    sh_glu_block<TT>(Wg, Wu, x, S, D, Is, h, blockIdx.x, red);
}

template <int TT>
__global__ __launch_bounds__(SH_NT) void k_sh_down(const uint16_t *__restrict__ Wd, const float *__restrict__ h, int S, int Is,
                                                 int D, float *__restrict__ out) {
    extern __shared__ __align__(16) float red[];
    sh_down_block<TT>(Wd, h, S, Is, D, out, blockIdx.x, red);
}

int sw_launch_sh_glu(hipStream_t st, const uint16_t *Wg, const uint16_t *Wu, const float *x, int S, int D, int Is, float *h) {
    if (S <= 0 || Is % SH_GLU_O || !sh_shape_ok(D)) return -1;
    if (S >= 2)
        SW_LAUNCH(k_sh_glu<SH_TT>, dim3((unsigned)sh_glu_blocks(S, Is, SH_TT)), dim3(SH_NT), sh_glu_lds<SH_TT>(D), st, Wg, Wu, x, S, D, Is, h);
    else
        SW_LAUNCH(k_sh_glu<1>, dim3((unsigned)sh_glu_blocks(S, Is, 1)), dim3(SH_NT), sh_glu_lds<1>(D), st, Wg, Wu, x, S, D, Is, h);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sw_launch_sh_down(hipStream_t st, const uint16_t *Wd, const float *h, int S, int Is, int D, float *out) {
    if (S <= 0 || D % SH_DN_O || !sh_shape_ok(Is)) return -1;
    if (S >= 2)
        SW_LAUNCH(k_sh_down<SH_TT>, dim3((unsigned)sh_down_blocks(S, D, SH_TT)), dim3(SH_NT), sh_down_lds<SH_TT>(Is), st, Wd, h, S, Is, D, out);
    else
        SW_LAUNCH(k_sh_down<1>, dim3((unsigned)sh_down_blocks(S, D, 1)), dim3(SH_NT), sh_down_lds<1>(Is), st, Wd, h, S, Is, D, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
