"""ctypes bindings for the CPU checker (test infrastructure only).

`Oracle` wraps oracle/liboracle.so (the C restatement, sw_oracle.c);
`Ref` wraps oracle/_ref/libref_*.so (the reference's own kernels and its
laguna.c MoE entry point, compiled from the reference sources).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use this module.
"""
import ctypes as C
import os
import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
U8P = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
I8P = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")

ROUTE_SIGMOID, ROUTE_SOFTMAX, ROUTE_SOFTPLUS = 0, 1, 2
SHARED_NONE, SHARED_UNSCALED = 0, 1
MODE_F32, MODE_IDOT, MODE_EXACT = 0, 1, 2
T_ROUTER, T_GATE_UP, T_DOWN, T_SH_GATE, T_SH_UP, T_SH_DOWN, T_X, T_CORR_BIAS, T_NORM, T_HEAD = range(1, 11)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def route_shape(desc):
    """(router rows, weights per token): Inkling's routing (act 6) adds its
    n_shared shared-expert gates to both"""
    ns = getattr(desc, "n_shared", 0) if desc.route_act == 6 else 0
    return desc.E + ns, desc.K + ns


class SwMoeDesc(C.Structure):
    _fields_ = [("n_experts", C.c_int), ("topk", C.c_int), ("route_act", C.c_int),
                ("use_corr_bias", C.c_int), ("norm_topk", C.c_int), ("route_scale", C.c_float),
                ("shared_mode", C.c_int), ("n_shared", C.c_int)]


class SwMoeLayer(C.Structure):
    _fields_ = [("D", C.c_int), ("I", C.c_int), ("Is", C.c_int), ("E", C.c_int), ("gs", C.c_int),
                ("router_bf16", C.c_int), ("shared_f32", C.c_int),
                ("router", C.c_void_p), ("corr_bias", C.c_void_p), ("logit_bias", C.c_void_p),
                ("gu_q", C.c_void_p), ("dn_q", C.c_void_p), ("gu_s", C.c_void_p), ("dn_s", C.c_void_p),
                ("sg", C.c_void_p), ("su", C.c_void_p), ("sd", C.c_void_p)]


class Oracle:
    def __init__(self, path=None):
        self.lib = C.CDLL(path or os.path.join(HERE, "liboracle.so"))
        L = self.lib
        L.sw_mix64.restype = C.c_uint64; L.sw_mix64.argtypes = [C.c_uint64]
        L.sw_u64.restype = C.c_uint64; L.sw_u64.argtypes = [C.c_uint64, C.c_uint64]
        L.sw_normal.restype = C.c_double; L.sw_normal.argtypes = [C.c_uint64, C.c_uint64]
        L.sw_tensor_seed.restype = C.c_uint64; L.sw_tensor_seed.argtypes = [C.c_uint64, C.c_int, C.c_int]
        L.sw_fill_normal_f32.argtypes = [F32P, C.c_int64, C.c_uint64, C.c_uint64, C.c_double]
        L.sw_round_bf16.restype = C.c_float; L.sw_round_bf16.argtypes = [C.c_float]
        L.sw_f32_to_bf16_array.argtypes = [U16P, F32P, C.c_int64]
        L.sw_round_bf16_inplace.argtypes = [F32P, C.c_int64]
        L.sw_quant_i4.argtypes = [U8P, F32P, F32P, C.c_int, C.c_int, C.c_int]
        L.sw_gen_q4.argtypes = [U8P, F32P, C.c_uint64, C.c_double, C.c_int64, C.c_int64, C.c_int, C.c_int]
        L.sw_matmul_f32.argtypes = [F32P, F32P, F32P] + [C.c_int] * 4
        L.sw_matmul_bf16.argtypes = [F32P, F32P, U16P] + [C.c_int] * 4
        L.sw_matmul_q4.argtypes = [F32P, F32P, U8P, F32P] + [C.c_int] * 5
        L.sw_matmul_bf16_rx.argtypes = [F32P, F32P, U16P] + [C.c_int] * 3
        L.sw_f32_to_bf16_ne.restype = C.c_uint16; L.sw_f32_to_bf16_ne.argtypes = [C.c_float]
        L.sw_matmul_q8.argtypes = [F32P, F32P, I8P, F32P] + [C.c_int] * 4
        L.sw_matmul_i4_grouped.argtypes = [F32P, F32P, U8P, F32P] + [C.c_int] * 4
        for f in ("sw_siluf", "sw_softplusf", "sw_sigmoidf"):
            getattr(L, f).restype = C.c_float; getattr(L, f).argtypes = [C.c_float]
        L.sw_softmax_row.argtypes = [F32P, C.c_int]
        L.sw_softmax_row_olmoe.argtypes = [F32P, C.c_int]
        L.sw_moe_route_qwen.argtypes = [F32P, C.c_int, C.c_int, I32P, F32P]
        L.sw_expf_array.argtypes = [F32P, F32P, C.c_int64]
        L.sw_log1pf_array.argtypes = [F32P, F32P, C.c_int64]
        L.sw_moe_topk.argtypes = [F32P, C.c_void_p, C.c_int, C.c_int, C.c_int, I32P]
        L.sw_rmsnorm_row.argtypes = [F32P, F32P, F32P, C.c_int, C.c_float]
        L.sw_argmax.restype = C.c_int; L.sw_argmax.argtypes = [F32P, C.c_int]
        L.sw_moe_route.argtypes = [C.POINTER(SwMoeDesc), C.POINTER(SwMoeLayer), F32P, C.c_int, C.c_int,
                                   C.c_void_p, I32P, F32P]
        L.sw_moe_block_rows.argtypes = [C.POINTER(SwMoeDesc), C.POINTER(SwMoeLayer), F32P, F32P, C.c_int, C.c_int]
        L.sw_route_logits.argtypes = [C.POINTER(SwMoeDesc), F32P, C.c_int, I32P, F32P]
        L.sw_moe_group_rows.argtypes = [C.POINTER(SwMoeDesc), C.POINTER(SwMoeLayer), F32P, F32P, C.c_int, C.c_int]
        L.sw_glm_logits.argtypes = [F32P, F32P, F32P, C.c_int, C.c_int, F32P, F32P]
        L.sw_glm_matmul.argtypes = [F32P, F32P, F32P] + [C.c_int] * 3
        L.sw_bucket.restype = C.c_int
        L.sw_bucket.argtypes = [I32P, C.c_int, C.c_int, C.c_int, I32P, I32P, I32P, I32P, I32P]

    # ---- data ----
    def tensor_seed(self, base, layer, tid):
        return self.lib.sw_tensor_seed(base, layer, tid)

    def normal(self, n, seed, sigma=1.0, offset=0):
        out = np.empty(n, np.float32)
        self.lib.sw_fill_normal_f32(out, n, seed, offset, sigma)
        return out

    def bf16_round(self, x):
        x = np.ascontiguousarray(x, np.float32).copy()
        self.lib.sw_round_bf16_inplace(x, x.size)
        return x

    def to_bf16(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.sw_f32_to_bf16_array(out, x, x.size)
        return out

    def quant_i4(self, w, gs):
        w = np.ascontiguousarray(w, np.float32)
        O, I = w.shape
        ng = (I + gs - 1) // gs if gs > 0 else 1
        p = np.empty((O, (I + 1) // 2), np.uint8)
        s = np.empty((O, ng), np.float32)
        self.lib.sw_quant_i4(p, s, w, O, I, gs)
        return p, s

    def gen_q4(self, seed, sigma, rows, I, gs, row0=0):
        ng = (I + gs - 1) // gs if gs > 0 else 1
        p = np.empty((rows, (I + 1) // 2), np.uint8)
        s = np.empty((rows, ng), np.float32)
        self.lib.sw_gen_q4(p, s, seed, sigma, row0, rows, I, gs)
        return p, s

    # ---- kernels ----
    def matmul_f32(self, x, W, exact=0):
        S, I = x.shape; O = W.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.sw_matmul_f32(y, np.ascontiguousarray(x), np.ascontiguousarray(W), S, I, O, exact)
        return y

    def matmul_bf16(self, x, Wb, exact=0):
        S, I = x.shape; O = Wb.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.sw_matmul_bf16(y, np.ascontiguousarray(x), np.ascontiguousarray(Wb), S, I, O, exact)
        return y

    def matmul_bf16_rx(self, x, Wb):
        """bf16 weights against bf16-rounded activations (the vdpbf16ps contract)"""
        S, I = x.shape; O = Wb.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.sw_matmul_bf16_rx(y, np.ascontiguousarray(x, np.float32), np.ascontiguousarray(Wb), S, I, O)
        return y

    def matmul_q8(self, x, q, s, mode=0):
        S, I = x.shape; O = q.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.sw_matmul_q8(y, np.ascontiguousarray(x, np.float32), np.ascontiguousarray(q, np.int8),
                              np.ascontiguousarray(s, np.float32), S, I, O, mode)
        return y

    def matmul_q4(self, x, p, s, mode=0, exact=0):
        S, I = x.shape; O = p.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.sw_matmul_q4(y, np.ascontiguousarray(x), p, np.ascontiguousarray(s, np.float32).reshape(-1), S, I, O, mode, exact)
        return y

    def matmul_i4_grouped(self, x, p, s, gs):
        S, I = x.shape; O = p.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.sw_matmul_i4_grouped(y, np.ascontiguousarray(x), p, np.ascontiguousarray(s, np.float32).reshape(-1), S, I, O, gs)
        return y

    def softmax_row(self, x):
        x = np.ascontiguousarray(x, np.float32).copy()
        self.lib.sw_softmax_row(x, x.size)
        return x

    def rmsnorm_rows(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32); w = np.ascontiguousarray(w, np.float32)
        out = np.empty_like(x)
        for s in range(x.shape[0]):
            self.lib.sw_rmsnorm_row(out[s], x[s], w, x.shape[1], eps)
        return out

    def argmax_rows(self, v):
        v = np.ascontiguousarray(v, np.float32)
        return np.array([self.lib.sw_argmax(v[s], v.shape[1]) for s in range(v.shape[0])], np.int32)

    def stack(self, desc, layers, norms, final_norm, head, h0, eps):
        """h += moe_block(rmsnorm(h, w_l)) per layer, then rmsnorm, the bf16 head
        (matmul_bf16, the SIMD contract) and the greedy pick: (h, logits, tok)"""
        h = np.ascontiguousarray(h0, np.float32).copy()
        for l, L in enumerate(layers):
            xn = self.rmsnorm_rows(h, norms[l], eps)
            h = self.moe_block_rows(desc, L, xn, h)
        xn = self.rmsnorm_rows(h, final_norm, eps)
        logits = self.matmul_bf16(xn, head)
        return h, logits, self.argmax_rows(logits)

    def softmax_row_olmoe(self, x):
        x = np.ascontiguousarray(x, np.float32).copy()
        self.lib.sw_softmax_row_olmoe(x, x.size)
        return x

    def route_qwen(self, logits, K):
        sel = np.empty(K, np.int32); w = np.empty(K, np.float32)
        self.lib.sw_moe_route_qwen(np.ascontiguousarray(logits, np.float32), logits.size, K, sel, w)
        return sel, w

    def route_logits(self, desc, logits):
        """gate + top-k of given logits [S, R] under desc (no correction bias)"""
        d, _ = self.make(desc, None)
        S = logits.shape[0]
        sel = np.empty((S, desc.K), np.int32); w = np.empty((S, route_shape(desc)[1]), np.float32)
        self.lib.sw_route_logits(C.byref(d), np.ascontiguousarray(logits, np.float32), S, sel, w)
        return sel, w

    # ---- the GLM engine's routing (c/colibri.c:2871-2999, plain path) ----
    def glm_matmul(self, x, W):
        """c/quant.h:98-102 as GCC -O3 builds it for AVX-512: inputs ascending, rounded products
        added in order, the last I % 8 as an fma chain"""
        x = np.ascontiguousarray(x, np.float32); W = np.ascontiguousarray(W, np.float32)
        y = np.empty((x.shape[0], W.shape[0]), np.float32)
        self.lib.sw_glm_matmul(y, x, W, x.shape[0], x.shape[1], W.shape[0])
        return y

    def glm_logits(self, x, W, bias):
        """(logit, choice) of one row: sigmoidf of the chain (c/colibri.c:833, 2873), + bias"""
        E, D = W.shape
        lg = np.empty(E, np.float32); ch = np.empty(E, np.float32)
        self.lib.sw_glm_logits(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(W, np.float32),
                               np.ascontiguousarray(bias, np.float32), D, E, lg, ch)
        return lg, ch

    @staticmethod
    def glm_select(logit, choice, Ksel, topp=0.0, norm_topk=1, routed_scale=1.0):
        """(idx[Ksel], w[Ksel], keff): Ksel passes of the first strict maximum of choice over the
        experts not yet taken (from -1e30, so NaN and <= -1e30 never win; none: kk < E ? kk : 0,
        c/colibri.c:2776-2782, 2955-2961); with 0 < topp < 1 the stable descending insertion sort
        and the cumulative cut (:2979-2984); norm_topk (:2997) and routed_scale (:2998) over the
        kept ones.  Every operation in float32, in the reference's order."""
        f = np.float32
        E = len(choice)
        idx, w, taken = [], [], set()
        for kk in range(Ksel):
            best, bv = -1, f(-1e30)
            for e in range(E):
                if e not in taken and choice[e] > bv:
                    bv, best = choice[e], e
            if best < 0:
                best = kk if kk < E else 0
            idx.append(best); w.append(f(logit[best])); taken.add(best)
        Ke = Ksel
        topp = f(topp)
        if f(0) < topp < f(1):
            for a in range(1, Ksel):
                ii, ww, b = idx[a], w[a], a - 1
                while b >= 0 and w[b] < ww:
                    w[b + 1] = w[b]; idx[b + 1] = idx[b]; b -= 1
                w[b + 1] = ww; idx[b + 1] = ii
            tot = f(1e-20)
            for v in w:
                tot = f(tot + v)
            cum = f(0)
            for kk in range(Ksel):
                cum = f(cum + w[kk])
                if cum >= f(topp * tot):
                    Ke = kk + 1
                    break
        if norm_topk:
            sm = f(0)
            for kk in range(Ke):
                sm = f(sm + w[kk])
            sm = f(sm + f(1e-20))
            for kk in range(Ke):
                w[kk] = f(w[kk] / sm)
        for kk in range(Ke):
            w[kk] = f(w[kk] * f(routed_scale))
        return np.array(idx, np.int32), np.array(w, np.float32), Ke

    def glm_route(self, x, W, bias, Ksel, topp=0.0, norm_topk=1, routed_scale=1.0):
        lg, ch = self.glm_logits(x, W, bias)
        return self.glm_select(lg, ch, Ksel, topp, norm_topk, routed_scale)

    def expf(self, x):
        x = np.ascontiguousarray(x, np.float32); y = np.empty_like(x)
        self.lib.sw_expf_array(y, x, x.size)
        return y

    def log1pf(self, x):
        x = np.ascontiguousarray(x, np.float32); y = np.empty_like(x)
        self.lib.sw_log1pf_array(y, x, x.size)
        return y

    def topk(self, score, K, bias=None):
        sel = np.empty(K, np.int32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.sw_moe_topk(np.ascontiguousarray(score, np.float32), _ptr(b), 1 if b is not None else 0,
                             score.size, K, sel)
        return sel

    def bucket(self, sel, S, K, E):
        T = S * K
        gexp = np.zeros(E, np.int32); gbeg = np.zeros(E, np.int32); gcnt = np.zeros(E, np.int32)
        grow = np.zeros(T, np.int32); rowof = np.zeros(T, np.int32)
        G = self.lib.sw_bucket(np.ascontiguousarray(sel, np.int32).reshape(-1), S, K, E, gexp, gbeg, gcnt, grow, rowof)
        return G, gexp[:G], gbeg[:G], gcnt[:G], grow, rowof

    # ---- MoE block ----
    @staticmethod
    def make(desc, layer):
        d = SwMoeDesc(desc.E, desc.K, desc.route_act, desc.use_corr_bias, desc.norm_topk,
                      desc.route_scale, desc.shared_mode, getattr(desc, "n_shared", 0))
        if layer is None:
            return d, None
        L = SwMoeLayer(layer.D, layer.I, layer.Is, layer.E, layer.gs, int(layer.router_bf16), 0,
                       _ptr(layer.router), _ptr(layer.corr_bias), _ptr(layer.logit_bias),
                       _ptr(layer.gu_q), _ptr(layer.dn_q), _ptr(layer.gu_s), _ptr(layer.dn_s),
                       _ptr(layer.sg), _ptr(layer.su), _ptr(layer.sd))
        return d, L

    def route(self, desc, layer, x, mode=MODE_F32):
        d, L = self.make(desc, layer)
        S = x.shape[0]
        R, W = route_shape(desc)
        sel = np.empty((S, desc.K), np.int32); w = np.empty((S, W), np.float32)
        lg = np.empty((S, R), np.float32)
        self.lib.sw_moe_route(C.byref(d), C.byref(L), np.ascontiguousarray(x, np.float32), S, mode,
                              lg.ctypes.data_as(C.c_void_p), sel, w)
        return lg, sel, w

    def moe_block_rows(self, desc, layer, x, out, mode=MODE_F32):
        d, L = self.make(desc, layer)
        out = np.ascontiguousarray(out, np.float32).copy()
        self.lib.sw_moe_block_rows(C.byref(d), C.byref(L), np.ascontiguousarray(x, np.float32), out, x.shape[0], mode)
        return out

    def moe_group_rows(self, desc, layer, x, out, mode=MODE_F32):
        d, L = self.make(desc, layer)
        out = np.ascontiguousarray(out, np.float32).copy()
        self.lib.sw_moe_group_rows(C.byref(d), C.byref(L), np.ascontiguousarray(x, np.float32), out, x.shape[0], mode)
        return out


class RefInkling:
    """The Inkling engine's own moe() (c/inkling.c:1011-1185, compiled in
    oracle/_ref/libref_inkling_avx512.so by ref_inkling.c) on host weights.  Its
    routed matmuls take IDOT from the environment once per process."""

    def __init__(self):
        self.lib = C.CDLL(os.path.join(HERE, "_ref", "libref_inkling_avx512.so"))
        self.lib.ref_inkling_moe.restype = C.c_int
        self.lib.ref_inkling_moe.argtypes = ([C.c_int] * 3 + [C.c_float] * 2 + [C.c_int] * 2 + [C.c_void_p] * 9
                                             + [F32P, F32P, C.c_int])

    @staticmethod
    def available():
        return os.path.exists(os.path.join(HERE, "_ref", "libref_inkling_avx512.so"))

    def moe(self, E, K, ns, route_scale, gscale, layer, x):
        """out[S, D] = moe(x) with out starting at zero"""
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        L = layer
        rc = self.lib.ref_inkling_moe(E, K, ns, route_scale, gscale, L.D, L.I, _ptr(L.router), _ptr(L.corr_bias),
                                      _ptr(L.gu_q), _ptr(L.gu_s), _ptr(L.dn_q), _ptr(L.dn_s),
                                      _ptr(L.sg), _ptr(L.su), _ptr(L.sd), x, out, x.shape[0])
        assert rc == 0
        return out


class RefGlm:
    """The GLM engine's router GEMV (c/quant.h matmul), compiled from the reference."""

    def __init__(self):
        self.lib = C.CDLL(os.path.join(HERE, "_ref", "libref_glm_avx512.so"))
        self.lib.ref_glm_matmul.argtypes = [F32P, F32P, F32P] + [C.c_int] * 3

    @staticmethod
    def available():
        return os.path.exists(os.path.join(HERE, "_ref", "libref_glm_avx512.so"))

    def matmul(self, x, W):
        x = np.ascontiguousarray(x, np.float32); W = np.ascontiguousarray(W, np.float32)
        y = np.empty((x.shape[0], W.shape[0]), np.float32)
        self.lib.ref_glm_matmul(y, x, W, x.shape[0], x.shape[1], W.shape[0])
        return y


class Ref:
    """The reference's own kernels (oracle/_ref), when built."""

    def __init__(self, isa=None):
        isa = isa or "avx512"
        self.lib = C.CDLL(os.path.join(HERE, "_ref", f"libref_kernels_{isa}.so"))
        L = self.lib
        L.ref_matmul_f32.argtypes = [F32P, F32P, F32P] + [C.c_int] * 4
        L.ref_matmul_bf16.argtypes = [F32P, F32P, U16P] + [C.c_int] * 5
        L.ref_matmul_q4_kb.argtypes = [F32P, F32P, U8P, F32P] + [C.c_int] * 5
        L.ref_matmul_q8.argtypes = [F32P, F32P, I8P, F32P] + [C.c_int] * 3
        L.ref_matmul_i4_grouped.argtypes = [F32P, F32P, U8P, F32P] + [C.c_int] * 4
        L.ref_softmax_row.argtypes = [F32P, C.c_int]
        L.ref_moe_topk.argtypes = [F32P, C.c_void_p, C.c_int, C.c_int, C.c_int, I32P]
        for f in ("ref_siluf", "ref_softplusf", "ref_expf", "ref_log1pf"):
            getattr(L, f).restype = C.c_float; getattr(L, f).argtypes = [C.c_float]
        L.ref_rmsnorm_row.argtypes = [F32P, F32P, F32P, C.c_int, C.c_float]
        L.ref_physical_cores.restype = C.c_int
        L.ref_moe_block_rows.restype = C.c_int
        L.ref_moe_block_rows.argtypes = ([C.c_int] * 5 + [C.c_float] + [C.c_int] * 6
                                         + [C.c_void_p] * 3 + [C.c_void_p] * 4 + [C.c_void_p] * 3
                                         + [F32P, F32P, C.c_int, C.c_int, C.c_int])

    @staticmethod
    def available(isa="avx512"):
        return os.path.exists(os.path.join(HERE, "_ref", f"libref_kernels_{isa}.so"))

    def matmul_f32(self, x, W, exact=0):
        S, I = x.shape; O = W.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.ref_matmul_f32(y, np.ascontiguousarray(x), np.ascontiguousarray(W), S, I, O, exact)
        return y

    def matmul_bf16(self, x, Wb, exact=0, round_x=0):
        S, I = x.shape; O = Wb.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.ref_matmul_bf16(y, np.ascontiguousarray(x), np.ascontiguousarray(Wb), S, I, O, round_x, exact)
        return y

    def matmul_q8(self, x, q, s, mode=0):
        """matmul_q8_k, one row of x at a time (the reference kernel is single-row)"""
        S, I = x.shape; O = q.shape[0]
        y = np.empty((S, O), np.float32)
        for r in range(S):
            self.lib.ref_matmul_q8(y[r], np.ascontiguousarray(x[r], np.float32), np.ascontiguousarray(q, np.int8),
                                   np.ascontiguousarray(s, np.float32), I, O, mode)
        return y

    def matmul_q4(self, x, p, s, mode=0, exact=0):
        S, I = x.shape; O = p.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.ref_matmul_q4_kb(y, np.ascontiguousarray(x), p, np.ascontiguousarray(s, np.float32).reshape(-1), S, I, O, mode, exact)
        return y

    def matmul_i4_grouped(self, x, p, s, gs):
        S, I = x.shape; O = p.shape[0]
        y = np.empty((S, O), np.float32)
        self.lib.ref_matmul_i4_grouped(y, np.ascontiguousarray(x), p, np.ascontiguousarray(s, np.float32).reshape(-1), S, I, O, gs)
        return y

    def softmax_row(self, x):
        x = np.ascontiguousarray(x, np.float32).copy()
        self.lib.ref_softmax_row(x, x.size)
        return x

    def topk(self, score, K, bias=None):
        sel = np.empty(K, np.int32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.ref_moe_topk(np.ascontiguousarray(score, np.float32), _ptr(b), 1 if b is not None else 0,
                              score.size, K, sel)
        return sel

    def rmsnorm_row(self, x, w, eps):
        out = np.empty(x.size, np.float32)
        self.lib.ref_rmsnorm_row(out, np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32),
                                 x.size, eps)
        return out

    def moe_block_rows(self, desc, layer, x, out, mode=0, exact=0):
        out = np.ascontiguousarray(out, np.float32).copy()
        rc = self.lib.ref_moe_block_rows(
            desc.E, desc.K, desc.route_act, desc.use_corr_bias, desc.norm_topk, desc.route_scale,
            desc.shared_mode, layer.D, layer.I, layer.Is, layer.gs, int(layer.router_bf16),
            _ptr(layer.router), _ptr(layer.corr_bias), _ptr(layer.logit_bias),
            _ptr(layer.gu_q), _ptr(layer.gu_s), _ptr(layer.dn_q), _ptr(layer.dn_s),
            _ptr(layer.sg), _ptr(layer.su), _ptr(layer.sd),
            np.ascontiguousarray(x, np.float32), out, x.shape[0], mode, exact)
        assert rc == 0
        return out


class RefLaguna:
    """The reference Laguna engine's lag_moe_rows (gs = 0 container)."""

    def __init__(self):
        self.lib = C.CDLL(os.path.join(HERE, "_ref", "libref_laguna_avx512.so"))
        f = self.lib.ref_laguna_moe_rows
        f.restype = C.c_int
        f.argtypes = ([C.c_int] * 3 + [C.c_float] + [C.c_int] * 3 + [C.c_void_p] * 2 + [C.c_void_p] * 4
                      + [C.c_void_p] * 3 + [F32P, F32P, C.c_int, C.c_int, C.c_int])

    @staticmethod
    def available():
        return os.path.exists(os.path.join(HERE, "_ref", "libref_laguna_avx512.so"))

    def moe_rows(self, desc, layer, x, h, exact=0, group=1):
        assert layer.gs == 0 and not layer.router_bf16
        h = np.ascontiguousarray(h, np.float32).copy()
        rc = self.lib.ref_laguna_moe_rows(
            desc.E, desc.K, desc.norm_topk, desc.route_scale, layer.D, layer.I, layer.Is,
            _ptr(layer.router), _ptr(layer.corr_bias),
            _ptr(layer.gu_q), _ptr(layer.gu_s), _ptr(layer.dn_q), _ptr(layer.dn_s),
            _ptr(layer.sg), _ptr(layer.su), _ptr(layer.sd),
            np.ascontiguousarray(x, np.float32), h, x.shape[0], exact, group)
        assert rc == 0
        return h


class RefLagunaHip:
    """The reference Laguna engine's lag_moe_rows built with -DCOLI_CUDA and
    linked against libsabrewing_loader.so (oracle/_ref/libref_laguna_hip.so):
    the engine's own batched driver calling this backend through lag_cuda_*."""

    def __init__(self):
        self.lib = C.CDLL(os.path.join(HERE, "_ref", "libref_laguna_hip.so"))
        f = self.lib.ref_laguna_moe_rows_dev
        f.restype = C.c_int
        f.argtypes = ([C.c_int] * 3 + [C.c_float] + [C.c_int] * 3 + [C.c_void_p] * 2 + [C.c_void_p] * 4
                      + [C.c_void_p] * 3 + [C.c_void_p] * 7 + [F32P, F32P, C.c_int, C.c_int])

    @staticmethod
    def available():
        return os.path.exists(os.path.join(HERE, "_ref", "libref_laguna_hip.so"))

    def moe_rows(self, desc, layer, dev, x, h, group=1):
        """dev: device pointers (ints) gu_q, gu_s, dn_q, dn_s, sg, su, sd"""
        assert layer.gs == 0 and not layer.router_bf16
        h = np.ascontiguousarray(h, np.float32).copy()
        rc = self.lib.ref_laguna_moe_rows_dev(
            desc.E, desc.K, desc.norm_topk, desc.route_scale, layer.D, layer.I, layer.Is,
            _ptr(layer.router), _ptr(layer.corr_bias),
            _ptr(layer.gu_q), _ptr(layer.gu_s), _ptr(layer.dn_q), _ptr(layer.dn_s),
            _ptr(layer.sg), _ptr(layer.su), _ptr(layer.sd),
            *[C.c_void_p(int(p)) for p in dev],
            np.ascontiguousarray(x, np.float32), h, x.shape[0], group)
        assert rc == 0
        return h


class RefQwen35Hip:
    """The reference qwen35 engine's moe_forward_rows (c/qwen35.c:595-700) built
    with -DCOLI_CUDA and linked against libsabrewing_loader.so
    (oracle/_ref/libref_qwen35_hip.so): with device pointers, the engine's own
    routing and counting sort hand the groups to lag_cuda_moe_group and its
    shared expert to lag_cuda_matmul_bf16; with none, the engine's CPU path."""

    def __init__(self):
        self.lib = C.CDLL(os.path.join(HERE, "_ref", "libref_qwen35_hip.so"))
        f = self.lib.ref_qwen35_moe_rows
        f.restype = C.c_int
        f.argtypes = [C.c_int] * 5 + [C.c_void_p] * 2 + [C.c_void_p] * 4 + [C.c_void_p] * 3 + [C.c_void_p] * 7 + \
            [F32P, F32P, C.c_int]

    @staticmethod
    def available():
        return os.path.exists(os.path.join(HERE, "_ref", "libref_qwen35_hip.so"))

    def moe_rows(self, E, K, layer, sgate, x, dev=None):
        """out [S, D] = the engine's MoE (routed + gated shared) of x; layer: per-row int4
        experts, f32 router, bf16 shared expert; dev: device pointers (ints) gu_q, gu_s,
        dn_q, dn_s, sg, su, sd, or None for the CPU path"""
        assert layer.gs == 0 and not layer.router_bf16
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        sgate = np.ascontiguousarray(sgate, np.float32)
        rc = self.lib.ref_qwen35_moe_rows(
            E, K, layer.D, layer.I, layer.Is, _ptr(layer.router), _ptr(sgate),
            _ptr(layer.gu_q), _ptr(layer.gu_s), _ptr(layer.dn_q), _ptr(layer.dn_s),
            _ptr(layer.sg), _ptr(layer.su), _ptr(layer.sd),
            *[C.c_void_p(int(p) if dev else None) for p in (dev or [0] * 7)],
            x, out, x.shape[0])
        assert rc == 0
        return out


class RefCallers:
    """The OLMoE and qwen35 engines' routing from their own sources
    (oracle/_ref/libref_olmoe_*.so, libref_qwen35_*.so)."""

    def __init__(self):
        self.olmoe = C.CDLL(os.path.join(HERE, "_ref", "libref_olmoe_avx512.so"))
        self.qwen = C.CDLL(os.path.join(HERE, "_ref", "libref_qwen35_avx512.so"))
        self.olmoe.ref_olmoe_route.argtypes = [F32P, C.c_int, C.c_int, C.c_int, I32P, F32P]
        self.olmoe.ref_olmoe_softmax_row.argtypes = [F32P, C.c_int]
        self.qwen.ref_qwen35_route.argtypes = [F32P, C.c_int, C.c_int, I32P, F32P]

    @staticmethod
    def available():
        return all(os.path.exists(os.path.join(HERE, "_ref", f)) for f in
                   ("libref_olmoe_avx512.so", "libref_qwen35_avx512.so"))

    def olmoe_route(self, logits, K, norm):
        E = logits.size
        sel = np.empty(K, np.int32); w = np.empty(K, np.float32)
        self.olmoe.ref_olmoe_route(np.ascontiguousarray(logits, np.float32), E, K, norm, sel, w)
        return sel, w

    def olmoe_softmax_row(self, x):
        x = np.ascontiguousarray(x, np.float32).copy()
        self.olmoe.ref_olmoe_softmax_row(x, x.size)
        return x

    def qwen_route(self, logits, K):
        E = logits.size
        sel = np.empty(K, np.int32); w = np.empty(K, np.float32)
        self.qwen.ref_qwen35_route(np.ascontiguousarray(logits, np.float32), E, K, sel, w)
        return sel, w
