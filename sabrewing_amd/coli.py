"""Python mirror of the GLM engine's coli_cuda_* table (include/sabrewing_coli.h).

`Coli` binds libsabrewing_hip.so's coli_hip_* entries with the reference's
argument meaning and its 1 ok / 0 fail convention (c/backend_cuda.h:28-169).  A
0 is raised as ColiError here, so a test reads like the engine's own checks
(c/colibri.c:3580-3600).  Weights arrive as the container stores them:
packed int4 bytes [O][I/2], low nibble = even input, offset 8; scales [O] for
fmt 2, or [O][I/gs] for fmt 4.  There is no CPU path: the library is required.
"""
import ctypes as C

import numpy as np

from . import backend as B

FMT_INT4, FMT_INT4_GROUPED = 2, 4
P = C.c_void_p
I_ = C.c_int
SZ = C.c_size_t
F = C.c_float

# name -> (restype, argtypes) of every entry of include/sabrewing_coli.h
SIGS = {
    "init": (I_, [P, I_]), "shutdown": (None, []), "device_count": (I_, []), "device_at": (I_, [I_]),
    "mem_info": (I_, [I_, P, P]), "stats": (None, [I_, P, P]), "group_stats": (None, [P] * 6),
    "tensor_upload_g": (I_, [P, P, P, I_, I_, I_, I_, I_]), "tensor_upload": (I_, [P, P, P, I_, I_, I_, I_]),
    "matmul": (I_, [P, P, P, P, P, I_, I_, I_, I_, I_, I_]),
    "expert_mlp": (I_, [P, P, P, P, P, I_]), "shared_mlp_w4a16": (I_, [P, P, P, P, P, I_]),
    "expert_group_issue": (I_, [P, P, P, P, I_, P]), "expert_group_take": (P, [I_]),
    "expert_group": (I_, [P, P, P, P, I_, P, P]),
    "attention_absorb": (I_, [P] * 5 + [I_] * 6 + [F]),
    "attention_absorb_batch": (I_, [P] * 5 + [I_] * 7 + [F]),
    "attention_project_batch": (I_, [P] * 6 + [I_] * 7 + [F]),
    "attention_project_ragged": (I_, [P] * 8 + [I_] * 7 + [F]),
    "attention_project_batch_dev": (I_, [P] * 6 + [I_] * 7 + [F]),
    "attention_absorb_batch_dev": (I_, [P] * 5 + [I_] * 7 + [F]),
    "attention_absorb_kvdev": (I_, [P] * 5 + [I_] * 6 + [F]),
    "attention_project_batch_dev_out": (I_, [P] * 6 + [I_] * 7 + [F]),
    "tensor_free": (None, [P]), "tensor_bytes": (SZ, [P]), "tensor_device": (I_, [P]),
    "tensor_update": (I_, [P, P, P]),
    "pipe_scratch": (P, [I_, I_, SZ]), "pipe_alloc": (P, [I_, SZ]), "pipe_free": (None, [I_, P]),
    "pipe_upload": (I_, [I_, P, P, SZ]), "pipe_download": (I_, [I_, P, P, SZ]),
    "pipe_rmsnorm": (I_, [I_, P, P, P, I_, I_, F]), "pipe_rope": (I_, [I_, P, P, I_, I_, I_, I_, I_, F]),
    "pipe_silu_mul": (I_, [I_, P, P, SZ]), "pipe_add": (I_, [I_, P, P, SZ]),
    "pipe_rows_add": (I_, [I_, P, P, P, I_, I_]), "pipe_gemm": (I_, [P, P, P, I_]),
    "pipe_rmsnorm_s": (I_, [I_, P, P, P, I_, I_, F, I_, I_]),
    "pipe_rope_base": (I_, [I_, P, I_, I_, I_, I_, I_, I_, F]),
    "pipe_copy2d": (I_, [I_, P, I_, P, I_, I_, I_]), "pipe_peer_copy": (I_, [I_, P, I_, P, SZ]),
    "pipe_sync": (I_, [I_]),
    "expert_group_resident_issue": (I_, [P, P, P, P, I_, I_, P, P]),
    "expert_group_resident_take": (I_, [I_, P, I_, P, P, I_]),
    "pipe_router": (I_, [I_, P, P, P, I_, I_, I_, F, I_, F, P, P, P]),
}
COLI_EXPORTS = ["coli_hip_" + n for n in SIGS]


class ColiError(RuntimeError):
    pass


def _p(a):
    return None if a is None else (a if isinstance(a, int) else a.ctypes.data)


def _tensors(ts):
    arr = (P * len(ts))(*[t.ptr for t in ts])
    return C.cast(arr, P), arr


class Tensor:
    """A resident int4 tensor W[O][I] (ColiCudaTensor)."""

    def __init__(self, coli, ptr, fmt, I, O, gs):
        self.coli, self.ptr, self.fmt, self.I, self.O, self.gs = coli, ptr, fmt, I, O, gs

    def free(self):
        if self.ptr:
            self.coli.f.tensor_free(self.ptr)
            self.ptr = None


class Coli:
    def __init__(self, devices=(0,), path=None):
        self.lib = B.load_library(path)
        self.f = _Fns(self.lib)
        devs = np.asarray(devices, np.int32)
        if not self.f.init(devs.ctypes.data, len(devs)):
            raise ColiError("coli_hip_init failed")
        self.devices = list(devices)

    def close(self):
        self.f.shutdown()

    # ---- tensors ----
    def upload(self, packed, scales, I, O, device=0, gs=0):
        """fmt 2 (gs 0) or fmt 4 (gs > 0) from the stored bytes"""
        packed = np.ascontiguousarray(packed, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        h = P(0)
        fmt = FMT_INT4_GROUPED if gs else FMT_INT4
        if not self.f.tensor_upload_g(C.addressof(h), packed.ctypes.data, scales.ctypes.data, fmt, I, O, device, gs):
            raise ColiError(f"tensor_upload_g(fmt {fmt}, I {I}, O {O}, gs {gs}) failed")
        return Tensor(self, h.value, fmt, I, O, gs)

    # ---- compute ----
    def matmul(self, t, x):
        x = np.ascontiguousarray(x, np.float32)
        S = x.shape[0]
        y = np.empty((S, t.O), np.float32)
        h = P(t.ptr)
        if not self.f.matmul(C.addressof(h), y.ctypes.data, x.ctypes.data, None, None, t.fmt, S, t.I, t.O,
                             self.f.tensor_device(t.ptr), t.gs):
            raise ColiError("matmul failed")
        return y

    def expert_mlp(self, g, u, d, x, shared=False):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], g.I), np.float32)
        fn = self.f.shared_mlp_w4a16 if shared else self.f.expert_mlp
        if not fn(g.ptr, u.ptr, d.ptr, y.ctypes.data, x.ctypes.data, x.shape[0]):
            raise ColiError("expert_mlp failed")
        return y

    def expert_group(self, gates, ups, downs, rows, x):
        x = np.ascontiguousarray(x, np.float32)
        rows = np.ascontiguousarray(rows, np.int32)
        y = np.empty_like(x)
        (pg, kg), (pu, ku), (pd, kd) = _tensors(gates), _tensors(ups), _tensors(downs)
        if not self.f.expert_group(pg, pu, pd, rows.ctypes.data, len(gates), y.ctypes.data, x.ctypes.data):
            raise ColiError("expert_group failed")
        return y

    def issue(self, gates, ups, downs, rows, x):
        x = np.ascontiguousarray(x, np.float32)
        rows = np.ascontiguousarray(rows, np.int32)
        (pg, kg), (pu, ku), (pd, kd) = _tensors(gates), _tensors(ups), _tensors(downs)
        return bool(self.f.expert_group_issue(pg, pu, pd, rows.ctypes.data, len(gates), x.ctypes.data))

    def take(self, device, shape):
        p = self.f.expert_group_take(device)
        if not p:
            return None
        n = int(np.prod(shape))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(n,)).reshape(shape).copy()

    def resident_issue(self, gates, ups, downs, weights, home, x_dev, slot_dev):
        w = np.ascontiguousarray(weights, np.float32)
        (pg, kg), (pu, ku), (pd, kd) = _tensors(gates), _tensors(ups), _tensors(downs)
        return bool(self.f.expert_group_resident_issue(pg, pu, pd, w.ctypes.data, len(gates), home, x_dev, slot_dev))

    def resident_take(self, home, devices, slots_dev, acc_dev, D):
        d = np.ascontiguousarray(devices, np.int32)
        return bool(self.f.expert_group_resident_take(home, d.ctypes.data, len(d), slots_dev, acc_dev, D))

    def router(self, device, x_dev, rw_dev, rb_dev, D, E, Ksel, topp=0.0, norm_topk=1, routed_scale=1.0):
        idx = np.empty(Ksel, np.int32)
        w = np.empty(Ksel, np.float32)
        ke = np.empty(1, np.int32)
        if not self.f.pipe_router(device, x_dev, rw_dev, rb_dev, D, E, Ksel, topp, norm_topk, routed_scale,
                                  idx.ctypes.data, w.ctypes.data, ke.ctypes.data):
            raise ColiError("pipe_router failed")
        return idx, w, int(ke[0])

    # ---- device memory ----
    def dev_put(self, a, device=0):
        a = np.ascontiguousarray(a)
        p = self.f.pipe_alloc(device, max(a.nbytes, 4))
        if not p or not self.f.pipe_upload(device, p, a.ctypes.data, a.nbytes):
            raise ColiError("pipe_alloc/upload failed")
        return p

    def dev_get(self, p, shape, dtype=np.float32, device=0):
        out = np.empty(shape, dtype)
        if not self.f.pipe_download(device, p, out.ctypes.data, out.nbytes):
            raise ColiError("pipe_download failed")
        return out

    def dev_free(self, p, device=0):
        self.f.pipe_free(device, p)


class _Fns:
    def __init__(self, lib):
        for n, (rt, at) in SIGS.items():
            fn = getattr(lib, "coli_hip_" + n)
            fn.restype = rt
            fn.argtypes = at
            setattr(self, n, fn)
