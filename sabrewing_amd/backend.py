"""ctypes binding of libsabrewing_hip.so (include/sabrewing_hip.h).

Plumbing for tests and the benchmark: host arrays are numpy, device memory is
owned by `DevBuf` handles from the backend's own allocator.  There is no CPU
fallback here: if the library is missing or the device cannot be initialised,
`Backend()` raises.
"""
import ctypes as C
import os
import numpy as np

from . import synth
from .configs import WEIGHT_SIGMA

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsabrewing_hip.so")
LOADER_PATH = os.path.join(HERE, "libsabrewing_loader.so")

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
VP = C.c_void_p

# every symbol include/sabrewing_hip.h declares (tests check the export table)
EXPORTS = [
    "lag_hip_init", "lag_hip_free_bytes", "lag_hip_total_bytes", "lag_hip_upload", "lag_hip_free",
    "lag_hip_matmul_bf16", "lag_hip_matmul_q4", "lag_hip_expert_q4", "lag_hip_moe_experts", "lag_hip_moe_group",
    "lag_hip_matmul_q8", "lag_hip_matmul_q8_s", "lag_hip_matmul_bf16_rx",
    "lag_hip_matmul_q4_g", "lag_hip_expert_q4_g", "lag_hip_moe_experts_g", "lag_hip_moe_group_g",
    "lag_hip_router_upload", "lag_hip_router_chain", "lag_hip_moe_forward", "lag_hip_moe_forward_noalloc",
    "lag_hip_moe_forward_scratch_bytes",
    "lag_hip_moe_block", "lag_hip_route",
    "lag_hip_last_groups", "lag_hip_rmsnorm", "lag_hip_moe_forward_rmsnorm", "lag_hip_head_argmax", "lag_hip_argmax", "lag_hip_set_grouped_kernel",
    "lag_hip_set_q4_mode",
    "lag_hip_alloc", "lag_hip_h2d", "lag_hip_d2h", "lag_hip_d2d", "lag_hip_memset",
    "lag_hip_graph_begin", "lag_hip_graph_end", "lag_hip_graph_launch", "lag_hip_graph_destroy", "lag_hip_sync",
    "lag_hip_event_create", "lag_hip_event_record", "lag_hip_event_elapsed_ms", "lag_hip_event_destroy",
    "lag_hip_profile", "lag_hip_profile_count", "lag_hip_profile_read", "lag_hip_profile_reset",
    "lag_hip_gen_normal", "lag_hip_gen_bf16", "lag_hip_gen_q4", "lag_hip_selftest", "lag_hip_last_error",
]
LOADER_EXPORTS = [
    "lag_cuda_init", "lag_cuda_free_bytes", "lag_cuda_total_bytes", "lag_cuda_upload", "lag_cuda_free",
    "lag_cuda_matmul_bf16", "lag_cuda_matmul_q8", "lag_cuda_matmul_q4", "lag_cuda_expert_q4",
    "lag_cuda_moe_experts", "lag_cuda_moe_group", "lag_cuda_matmul_fp4", "lag_cuda_moe_experts_fp4",
    "sabrewing_loader_available", "sabrewing_loader_path",
]
# the Inkling engine's table (c/backend_cuda_ink.h:14-34), exported by the loader
INK_EXPORTS = [
    "ink_cuda_init", "ink_cuda_free_bytes", "ink_cuda_total_bytes", "ink_cuda_upload", "ink_cuda_matmul_bf16",
    "ink_cuda_matmul_q4", "ink_cuda_matmul_q8", "ink_cuda_expert_q4", "sabrewing_loader_ink_available",
]


class LagHipMoeDesc(C.Structure):
    _fields_ = [("n_experts", C.c_int), ("topk", C.c_int), ("route_act", C.c_int), ("use_corr_bias", C.c_int),
                ("norm_topk", C.c_int), ("route_scale", C.c_float), ("shared_mode", C.c_int),
                ("hidden", C.c_int), ("moe_inter", C.c_int), ("shared_inter", C.c_int), ("gs", C.c_int),
                ("router_bf16", C.c_int), ("n_shared", C.c_int)]


class LagHipMoeWeights(C.Structure):
    _fields_ = [("router", VP), ("corr_bias", VP), ("logit_bias", VP), ("gu_q", VP), ("gu_s", VP),
                ("dn_q", VP), ("dn_s", VP), ("sg", VP), ("su", VP), ("sd", VP)]


def desc_of(cfg):
    return LagHipMoeDesc(cfg.E, cfg.K, cfg.route_act, cfg.use_corr_bias, cfg.norm_topk, cfg.route_scale,
                         cfg.shared_mode, cfg.D, cfg.I, cfg.Is, cfg.gs, int(cfg.router_bf16), cfg.n_shared)


class BackendError(RuntimeError):
    pass


def load_library(path=None):
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise BackendError(f"{path} is not built (python -m sabrewing_amd.build)")
    lib = C.CDLL(path)
    L = lib
    L.lag_hip_init.argtypes = [C.c_int]
    L.lag_hip_free_bytes.restype = C.c_size_t
    L.lag_hip_total_bytes.restype = C.c_size_t
    L.lag_hip_upload.restype = VP; L.lag_hip_upload.argtypes = [VP, C.c_size_t]
    L.lag_hip_free.argtypes = [VP]
    L.lag_hip_alloc.restype = VP; L.lag_hip_alloc.argtypes = [C.c_size_t]
    L.lag_hip_h2d.argtypes = [VP, VP, C.c_size_t]
    L.lag_hip_d2h.argtypes = [VP, VP, C.c_size_t]
    L.lag_hip_memset.argtypes = [VP, C.c_int, C.c_size_t]
    L.lag_hip_d2d.argtypes = [VP, VP, C.c_size_t]
    L.lag_hip_graph_end.restype = VP
    L.lag_hip_graph_launch.argtypes = [VP]
    L.lag_hip_graph_destroy.argtypes = [VP]
    L.lag_hip_matmul_bf16.argtypes = [F32P, F32P, VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_matmul_q4.argtypes = [F32P, F32P, VP, VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_matmul_q4_g.argtypes = [F32P, F32P, VP, VP, C.c_int, C.c_int, C.c_int, C.c_int]
    L.lag_hip_expert_q4.argtypes = [F32P, F32P, VP, VP, VP, VP, C.c_int, C.c_int]
    L.lag_hip_expert_q4_g.argtypes = [F32P, F32P, VP, VP, VP, VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_matmul_q8.argtypes = [F32P, F32P, VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_matmul_q8_s.argtypes = [F32P, F32P, VP, VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_matmul_bf16_rx.argtypes = [F32P, F32P, VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_moe_experts.argtypes = [F32P, F32P, VP, VP, VP, VP, I32P, F32P, C.c_int, C.c_int, C.c_int]
    L.lag_hip_moe_experts_g.argtypes = [F32P, F32P, VP, VP, VP, VP, I32P, F32P, C.c_int, C.c_int, C.c_int, C.c_int]
    L.lag_hip_moe_group.argtypes = [F32P, F32P, VP, VP, VP, VP, I32P, I32P, I32P, C.c_int, I32P, I32P, F32P,
                                    C.c_int, C.c_int, C.c_int, C.c_int]
    L.lag_hip_moe_group_g.argtypes = L.lag_hip_moe_group.argtypes + [C.c_int]
    L.lag_hip_router_upload.restype = VP; L.lag_hip_router_upload.argtypes = [VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_router_chain.argtypes = [VP, VP, C.c_int, C.c_int, C.c_int]
    L.lag_hip_rmsnorm.argtypes = [VP, VP, VP, C.c_int, C.c_int, C.c_float]
    L.lag_hip_head_argmax.argtypes = [VP, C.c_int, VP, C.c_int, C.c_int, C.c_int, VP, VP]
    L.lag_hip_argmax.argtypes = [VP, C.c_int, C.c_int, VP]
    DP, WP = C.POINTER(LagHipMoeDesc), C.POINTER(LagHipMoeWeights)
    L.lag_hip_moe_forward.argtypes = [DP, WP, VP, VP, C.c_int]
    L.lag_hip_moe_forward_rmsnorm.argtypes = [DP, WP, VP, C.c_float, VP, VP, C.c_int]
    L.lag_hip_moe_forward_noalloc.argtypes = [DP, WP, VP, VP, C.c_int]
    L.lag_hip_moe_forward_scratch_bytes.restype = C.c_size_t
    L.lag_hip_moe_forward_scratch_bytes.argtypes = [DP, WP, C.c_int]
    L.lag_hip_moe_block.argtypes = [DP, WP, F32P, F32P, C.c_int]
    L.lag_hip_route.argtypes = [DP, WP, VP, C.c_int, VP, VP, VP]
    L.lag_hip_last_groups.argtypes = [C.POINTER(C.c_int), I32P, I32P, I32P, C.c_int]
    L.lag_hip_event_create.restype = VP
    L.lag_hip_event_record.argtypes = [VP]
    L.lag_hip_event_elapsed_ms.restype = C.c_float; L.lag_hip_event_elapsed_ms.argtypes = [VP, VP]
    L.lag_hip_event_destroy.argtypes = [VP]
    L.lag_hip_profile.argtypes = [C.c_int]
    L.lag_hip_set_grouped_kernel.argtypes = [C.c_int]
    L.lag_hip_set_q4_mode.argtypes = [C.c_int]
    L.lag_hip_profile_read.argtypes = [C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_longlong)]
    L.lag_hip_gen_normal.argtypes = [VP, C.c_int64, C.c_uint64, C.c_uint64, C.c_double, C.c_int]
    L.lag_hip_gen_bf16.argtypes = [VP, C.c_int64, C.c_uint64, C.c_uint64, C.c_double]
    L.lag_hip_gen_q4.argtypes = [VP, VP, C.c_uint64, C.c_double, C.c_int64, C.c_int64, C.c_int, C.c_int]
    L.lag_hip_selftest.argtypes = [F32P, F32P, C.c_int]
    L.lag_hip_last_error.restype = C.c_char_p
    return lib


class DevBuf:
    """Device allocation from the backend (freed with lag_hip_free)."""

    def __init__(self, be, nbytes, ptr=None):
        self.be, self.nbytes = be, int(nbytes)
        self.ptr = ptr if ptr is not None else be.lib.lag_hip_alloc(max(1, self.nbytes))
        if not self.ptr:
            raise BackendError(f"device allocation of {nbytes} bytes failed: {be.last_error()}")

    def free(self):
        if self.ptr:
            self.be.lib.lag_hip_free(self.ptr)
            self.ptr = None

    def __int__(self):
        return int(self.ptr)


class Backend:
    def __init__(self, device=0, path=None):
        self.lib = load_library(path)
        rc = self.lib.lag_hip_init(device)
        if rc != 0:
            raise BackendError(f"lag_hip_init({device}) failed: {self.last_error()}")

    def last_error(self):
        e = self.lib.lag_hip_last_error()
        return e.decode() if e else ""

    def check(self, rc, what):
        if rc != 0:
            raise BackendError(f"{what} failed: {self.last_error()}")

    # ---- memory ----
    def alloc(self, nbytes):
        return DevBuf(self, nbytes)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.lib.lag_hip_upload(arr.ctypes.data_as(VP), arr.nbytes)
        if not p:
            raise BackendError(f"upload of {arr.nbytes} bytes failed: {self.last_error()}")
        return DevBuf(self, arr.nbytes, p)

    def h2d(self, buf, arr):
        arr = np.ascontiguousarray(arr)
        self.check(self.lib.lag_hip_h2d(VP(int(buf)), arr.ctypes.data_as(VP), arr.nbytes), "h2d")

    def d2h(self, buf, shape, dtype, offset=0):
        out = np.empty(shape, dtype)
        self.check(self.lib.lag_hip_d2h(out.ctypes.data_as(VP), VP(int(buf) + offset), out.nbytes), "d2h")
        return out

    def sync(self):
        self.check(self.lib.lag_hip_sync(), "sync")

    # ---- lag family (host activations) ----
    def matmul_bf16(self, x, W, O):
        x = np.ascontiguousarray(x, np.float32); S, I = x.shape
        y = np.empty((S, O), np.float32)
        self.check(self.lib.lag_hip_matmul_bf16(y, x, VP(int(W)), S, I, O), "lag_hip_matmul_bf16")
        return y

    def matmul_bf16_rx(self, x, W, O):
        x = np.ascontiguousarray(x, np.float32); S, I = x.shape
        y = np.empty((S, O), np.float32)
        self.check(self.lib.lag_hip_matmul_bf16_rx(y, x, VP(int(W)), S, I, O), "lag_hip_matmul_bf16_rx")
        return y

    def matmul_q8(self, x, q, s, O):
        x = np.ascontiguousarray(x, np.float32); S, I = x.shape
        y = np.empty((S, O), np.float32)
        self.check(self.lib.lag_hip_matmul_q8_s(y, x, VP(int(q)), VP(int(s)), S, I, O), "lag_hip_matmul_q8_s")
        return y

    def matmul_q4(self, x, p, s, O, gs=0):
        x = np.ascontiguousarray(x, np.float32); S, I = x.shape
        y = np.empty((S, O), np.float32)
        self.check(self.lib.lag_hip_matmul_q4_g(y, x, VP(int(p)), VP(int(s)), S, I, O, gs), "lag_hip_matmul_q4_g")
        return y

    def expert_q4(self, x, p13, s13, p2, s2, I, D, gs=0):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty(D, np.float32)
        self.check(self.lib.lag_hip_expert_q4_g(out, x, VP(int(p13)), VP(int(s13)), VP(int(p2)), VP(int(s2)), I, D, gs),
                   "lag_hip_expert_q4_g")
        return out

    def moe_experts(self, x, L, sel, w, gs=0):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty(L.D, np.float32)
        self.check(self.lib.lag_hip_moe_experts_g(out, x, VP(int(L.gu_q)), VP(int(L.gu_s)), VP(int(L.dn_q)),
                                                  VP(int(L.dn_s)), np.ascontiguousarray(sel, np.int32),
                                                  np.ascontiguousarray(w, np.float32), len(sel), L.I, L.D, gs),
                   "lag_hip_moe_experts_g")
        return out

    def moe_group(self, x, L, gexp, gbeg, gcnt, grow, rowof, w, K, gs=0):
        x = np.ascontiguousarray(x, np.float32); S = x.shape[0]
        acc = np.empty((S, L.D), np.float32)
        i32 = lambda a: np.ascontiguousarray(a, np.int32).reshape(-1)
        self.check(self.lib.lag_hip_moe_group_g(acc, x, VP(int(L.gu_q)), VP(int(L.gu_s)), VP(int(L.dn_q)),
                                                VP(int(L.dn_s)), i32(gexp), i32(gbeg), i32(gcnt), len(gexp),
                                                i32(grow), i32(rowof), np.ascontiguousarray(w, np.float32).reshape(-1),
                                                S, K, L.I, L.D, gs), "lag_hip_moe_group_g")
        return acc

    # ---- device MoE block ----
    def router_upload(self, W, bf16):
        W = np.ascontiguousarray(W)
        E, D = W.shape
        p = self.lib.lag_hip_router_upload(W.ctypes.data_as(VP), E, D, int(bf16))
        if not p:
            raise BackendError(f"router upload failed: {self.last_error()}")
        return DevBuf(self, W.nbytes, p)

    def moe_forward(self, desc, weights, x_dev, out_dev, S):
        self.check(self.lib.lag_hip_moe_forward(C.byref(desc), C.byref(weights), VP(int(x_dev)), VP(int(out_dev)), S),
                   "lag_hip_moe_forward")

    def moe_forward_noalloc(self, desc, weights, x_dev, out_dev, S):
        """the allocation-free forward (scratch in the library's static device array)"""
        self.check(self.lib.lag_hip_moe_forward_noalloc(C.byref(desc), C.byref(weights), VP(int(x_dev)),
                                                        VP(int(out_dev)), S), "lag_hip_moe_forward_noalloc")

    def moe_block(self, desc, weights, x, out):
        x = np.ascontiguousarray(x, np.float32); out = np.ascontiguousarray(out, np.float32).copy()
        self.check(self.lib.lag_hip_moe_block(C.byref(desc), C.byref(weights), x, out, x.shape[0]), "lag_hip_moe_block")
        return out

    def route(self, desc, weights, x_dev, S):
        """(logits [S, R], sel [S, K], w [S, W]); Inkling's routing (act 6) has R = E + n_shared
        router rows and W = K + n_shared weights (the picks', then the shared gates')"""
        K = desc.topk
        ns = desc.n_shared if desc.route_act == 6 else 0
        R, W = desc.n_experts + ns, K + ns
        lg, sel, w = self.alloc(S * R * 4), self.alloc(S * K * 4), self.alloc(S * W * 4)
        self.check(self.lib.lag_hip_route(C.byref(desc), C.byref(weights), VP(int(x_dev)), S, VP(int(lg)),
                                          VP(int(sel)), VP(int(w))), "lag_hip_route")
        out = (self.d2h(lg, (S, R), np.float32), self.d2h(sel, (S, K), np.int32), self.d2h(w, (S, W), np.float32))
        for b in (lg, sel, w):
            b.free()
        return out

    def moe_forward_rmsnorm(self, desc, weights, norm_w_dev, eps, xn_dev, h_dev, S):
        """one stack layer: xn = rmsnorm(h), h += MoE(xn) (the norm inside the routing launch)"""
        self.check(self.lib.lag_hip_moe_forward_rmsnorm(C.byref(desc), C.byref(weights), VP(int(norm_w_dev)),
                                                        C.c_float(eps), VP(int(xn_dev)), VP(int(h_dev)), S),
                   "lag_hip_moe_forward_rmsnorm")

    def rmsnorm(self, x_dev, w_dev, out_dev, S, D, eps):
        self.check(self.lib.lag_hip_rmsnorm(VP(int(x_dev)), VP(int(w_dev)), VP(int(out_dev)), S, D, C.c_float(eps)),
                   "lag_hip_rmsnorm")

    def head_argmax(self, Wc, w_bf16, x_dev, S, D, V, logits_dev, tok_dev=None):
        self.check(self.lib.lag_hip_head_argmax(VP(int(Wc)), int(w_bf16), VP(int(x_dev)), S, D, V, VP(int(logits_dev)),
                                                VP(int(tok_dev)) if tok_dev is not None else None),
                   "lag_hip_head_argmax")

    def argmax(self, logits_dev, S, V, tok_dev):
        self.check(self.lib.lag_hip_argmax(VP(int(logits_dev)), S, V, VP(int(tok_dev))), "lag_hip_argmax")

    def last_groups(self, cap=4096):
        G = C.c_int(0)
        gexp, gbeg, gcnt = (np.zeros(cap, np.int32) for _ in range(3))
        self.check(self.lib.lag_hip_last_groups(C.byref(G), gexp, gbeg, gcnt, cap), "lag_hip_last_groups")
        n = min(G.value, cap)
        return G.value, gexp[:n], gbeg[:n], gcnt[:n]

    # ---- generators ----
    def gen_normal(self, buf, n, seed, sigma, offset=0, to_bf16=False):
        self.check(self.lib.lag_hip_gen_normal(VP(int(buf)), n, seed, offset, sigma, int(to_bf16)), "gen_normal")

    def gen_bf16(self, buf, n, seed, sigma, offset=0):
        self.check(self.lib.lag_hip_gen_bf16(VP(int(buf)), n, seed, offset, sigma), "gen_bf16")

    def gen_q4(self, qbuf, sbuf, seed, sigma, rows, K, gs, row0=0):
        self.check(self.lib.lag_hip_gen_q4(VP(int(qbuf)), VP(int(sbuf)), seed, sigma, row0, rows, K, gs), "gen_q4")

    # ---- graphs ----
    def graph_begin(self):
        self.check(self.lib.lag_hip_graph_begin(), "graph begin")

    def graph_end(self):
        g = self.lib.lag_hip_graph_end()
        if not g:
            raise BackendError(f"graph end failed: {self.last_error()}")
        return g

    def graph_launch(self, g):
        self.check(self.lib.lag_hip_graph_launch(g), "graph launch")

    def graph_destroy(self, g):
        self.lib.lag_hip_graph_destroy(g)

    # ---- timing / profile ----
    def event(self):
        return self.lib.lag_hip_event_create()

    def record(self, ev):
        self.check(self.lib.lag_hip_event_record(ev), "event record")

    def elapsed_ms(self, a, b):
        return float(self.lib.lag_hip_event_elapsed_ms(a, b))

    def profile(self, on):
        self.lib.lag_hip_profile(int(on))

    GROUPED_AUTO, GROUPED_DOT8, GROUPED_MFMA = 0, 1, 2

    def set_grouped_kernel(self, mode):
        """the grouped expert GEMMs of batches: 0 auto, 1 dot8, 2 f16 MFMA
        (bit-identical); returns the previous mode"""
        prev = self.lib.lag_hip_set_grouped_kernel(int(mode))
        if prev < 0:
            raise BackendError(f"bad grouped-kernel mode {mode}")
        return prev

    Q4_DOT8, Q4_IDOT = 0, 1

    def set_q4_mode(self, mode):
        """the int4 activation contract of moe_forward for per-row scales: 0 this
        build's exact-integer form, 1 the reference's IDOT (LAG_IDOT=1); returns the
        previous mode"""
        prev = self.lib.lag_hip_set_q4_mode(int(mode))
        if prev < 0:
            raise BackendError(f"bad q4 mode {mode}")
        return prev

    def profile_reset(self):
        self.lib.lag_hip_profile_reset()

    def profile_read(self):
        out = {}
        buf = C.create_string_buffer(128)
        for i in range(self.lib.lag_hip_profile_count()):
            ms, n = C.c_double(0), C.c_longlong(0)
            if self.lib.lag_hip_profile_read(i, buf, 128, C.byref(ms), C.byref(n)) == 0:
                out[buf.value.decode()] = (ms.value, n.value)
        return out

    def selftest(self, xin):
        xin = np.ascontiguousarray(xin, np.float32)
        out = np.zeros(768 + 3 * xin.size, np.float32)
        self.check(self.lib.lag_hip_selftest(out, xin, xin.size), "lag_hip_selftest")
        return out


class DeviceLayer:
    """One MoE layer resident in HBM (the reference container layout), with
    the descriptor and weight-pointer structs lag_hip_moe_forward takes."""

    def __init__(self, be, cfg):
        self.be, self.cfg = be, cfg
        self.bufs = []
        self.router = self.corr_bias = self.logit_bias = None
        self.gu_q = self.gu_s = self.dn_q = self.dn_s = self.sg = self.su = self.sd = None
        self.D, self.I = cfg.D, cfg.I

    def _keep(self, b):
        self.bufs.append(b)
        return b

    @classmethod
    def from_host(cls, be, cfg, L):
        """Upload a host layer (oracle.synth.Layer)."""
        self = cls(be, cfg)
        self.router = self._keep(be.router_upload(L.router, cfg.router_bf16))
        self.gu_q, self.gu_s = self._keep(be.upload(L.gu_q)), self._keep(be.upload(L.gu_s))
        self.dn_q, self.dn_s = self._keep(be.upload(L.dn_q)), self._keep(be.upload(L.dn_s))
        if L.corr_bias is not None:
            self.corr_bias = self._keep(be.upload(L.corr_bias))
        if L.logit_bias is not None:
            self.logit_bias = self._keep(be.upload(L.logit_bias))
        if cfg.shared_mode:
            self.sg, self.su, self.sd = (self._keep(be.upload(a)) for a in (L.sg, L.su, L.sd))
        return self

    @classmethod
    def from_container(cls, be, snap, i):
        """MoE layer i of a Laguna int4 snapshot (sabrewing_amd.container.Snapshot);
        the layer's descriptor is self.cfg"""
        from .container import load_layer
        cfg, L = load_layer(snap, i)
        return cls.from_host(be, cfg, L)

    @classmethod
    def generate(cls, be, cfg, base_seed, layer=0):
        """Generate a seeded layer directly in HBM (same bits as the host generator)."""
        self = cls(be, cfg)
        D, I, Is, E, gs = cfg.D, cfg.I, cfg.Is, cfg.E, cfg.gs
        ts = lambda tid: synth.tensor_seed(base_seed, layer, tid)
        ngD = D // gs if gs > 0 else 1
        ngI = I // gs if gs > 0 else 1
        rb = 2 if cfg.router_bf16 else 4
        R = cfg.router_rows                      # Inkling: the shared gate rows follow the E routed
        tmp = be.alloc(R * D * rb)
        if cfg.router_bf16:
            be.gen_bf16(tmp, R * D, ts(synth.T_ROUTER), WEIGHT_SIGMA)
        else:
            be.gen_normal(tmp, R * D, ts(synth.T_ROUTER), WEIGHT_SIGMA)
        self.router = self._keep(be.alloc((R + 3) // 4 * 4 * D * rb))    # streaming order
        be.check(be.lib.lag_hip_router_chain(VP(int(tmp)), VP(int(self.router)), R, D, int(cfg.router_bf16)), "router chain")
        be.sync()
        tmp.free()
        self.gu_q, self.gu_s = self._keep(be.alloc(E * 2 * I * D // 2)), self._keep(be.alloc(E * 2 * I * ngD * 4))
        self.dn_q, self.dn_s = self._keep(be.alloc(E * D * I // 2)), self._keep(be.alloc(E * D * ngI * 4))
        be.gen_q4(self.gu_q, self.gu_s, ts(synth.T_GATE_UP), WEIGHT_SIGMA, E * 2 * I, D, gs)
        be.gen_q4(self.dn_q, self.dn_s, ts(synth.T_DOWN), WEIGHT_SIGMA, E * D, I, gs)
        if cfg.use_corr_bias:
            self.corr_bias = self._keep(be.alloc(E * 4))
            be.check(be.lib.lag_hip_memset(VP(int(self.corr_bias)), 0, E * 4), "memset")
        if cfg.zipf > 0:
            lb = synth.zipf_bias(E, cfg.zipf, ts(synth.T_ROUTER) ^ 0x5A5A)
            self.logit_bias = self._keep(be.upload(lb))
        if cfg.shared_mode:                       # ns shared experts stacked (GATED: Inkling's pool)
            ns = cfg.n_shared_experts
            self.sg, self.su, self.sd = (self._keep(be.alloc(ns * Is * D * 2)) for _ in range(3))
            be.gen_bf16(self.sg, ns * Is * D, ts(synth.T_SH_GATE), WEIGHT_SIGMA)
            be.gen_bf16(self.su, ns * Is * D, ts(synth.T_SH_UP), WEIGHT_SIGMA)
            be.gen_bf16(self.sd, ns * D * Is, ts(synth.T_SH_DOWN), WEIGHT_SIGMA)
        be.sync()
        return self

    def desc(self):
        return desc_of(self.cfg)

    def weights(self):
        p = lambda b: VP(int(b)) if b is not None else None
        return LagHipMoeWeights(p(self.router), p(self.corr_bias), p(self.logit_bias), p(self.gu_q), p(self.gu_s),
                                p(self.dn_q), p(self.dn_s), p(self.sg), p(self.su), p(self.sd))

    def free(self):
        for b in self.bufs:
            b.free()
        self.bufs = []


def gen_x(be, cfg, base_seed, S, stream=0):
    """S tokens of N(0,1) activations in HBM (bf16-valued when cfg.x_bf16)."""
    buf = be.alloc(S * cfg.D * 4)
    be.gen_normal(buf, S * cfg.D, synth.tensor_seed(base_seed, 1000 + stream, synth.T_X), 1.0, to_bf16=cfg.x_bf16)
    return buf
