"""The Laguna int4 container on disk -> MoE layers for the device.

A colibri snapshot (`c/tools/convert_laguna_int4.py`, read by `c/laguna.c:349-452`) is an
HF directory: `config.json` plus safetensors shards (`model.safetensors.index.json` ->
shard files, or one `model.safetensors`).  Per MoE layer i it holds
(`docs/laguna.md:34-44`):

  model.layers.{i}.mlp.gate.weight                       f32 [E, D]    router
  model.layers.{i}.mlp.experts.e_score_correction_bias   f32 [E]       (optional: zeros)
  model.layers.{i}.mlp.experts.gate_up_proj              u8  [E*2I, D/2] packed int4
  model.layers.{i}.mlp.experts.gate_up_proj.qs           f32 [E*2I] row scales (or [E*2I, D/gs])
  model.layers.{i}.mlp.experts.down_proj                 u8  [E*D, I/2]
  model.layers.{i}.mlp.experts.down_proj.qs              f32 [E*D] (or [E*D, I/gs])
  model.layers.{i}.mlp.shared_expert.{gate,up}_proj.weight  bf16 [Is, D]
  model.layers.{i}.mlp.shared_expert.down_proj.weight       bf16 [D, Is]

Dense layers are listed by `mlp_only_layers` (or `mlp_layer_types` "dense"), as
`cfg_load` reads them (`c/laguna.c:279-286`).  The descriptor is the one the engine
builds for every MoE layer (`c/laguna.c:817-819`): sigmoid routing with the correction
bias in the selection, `norm_topk_prob`, `moe_routed_scaling_factor`, one unscaled shared
expert.

Files are memory-mapped; a tensor is a zero-copy view of its bytes.  The header is
parsed here (8-byte little-endian length, then the JSON table of dtype, shape and byte
offsets): the bf16 tensors stay raw (uint16), as the device takes them.
"""
import json
import mmap
import os
import struct
from dataclasses import dataclass
from typing import Optional

import numpy as np

from .configs import MoeConfig, ROUTE_SIGMOID, SHARED_UNSCALED

ST_MAX_HEADER = 512 << 20          # a crafted header length is refused before any allocation
_DT = {"F32": (np.float32, 4), "BF16": (np.uint16, 2), "F16": (np.float16, 2), "U8": (np.uint8, 1),
       "I8": (np.int8, 1), "I32": (np.int32, 4), "I64": (np.int64, 8), "F64": (np.float64, 8)}


class ContainerError(ValueError):
    pass


@dataclass
class TensorInfo:
    path: str
    dtype: str
    shape: tuple
    offset: int          # absolute byte offset in the file
    nbytes: int

    @property
    def numel(self):
        n = 1
        for d in self.shape:
            n *= d
        return n


def read_header(path):
    """name -> TensorInfo of one safetensors file (validated against the file size)"""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ContainerError(f"{path}: shorter than a safetensors header")
        (hlen,) = struct.unpack("<Q", head)
        if hlen > ST_MAX_HEADER or 8 + hlen > size:
            raise ContainerError(f"{path}: header length {hlen} out of range")
        try:
            table = json.loads(f.read(hlen))
        except ValueError as e:
            raise ContainerError(f"{path}: bad header JSON ({e})") from None
    base = 8 + hlen
    out = {}
    for name, t in table.items():
        if name == "__metadata__":
            continue
        dt = t.get("dtype")
        if dt not in _DT:
            raise ContainerError(f"{path}: {name}: unsupported dtype {dt}")
        shape = tuple(int(d) for d in t["shape"])
        b0, b1 = (int(v) for v in t["data_offsets"])
        info = TensorInfo(path, dt, shape, base + b0, b1 - b0)
        if b0 < 0 or b1 < b0 or base + b1 > size or info.nbytes != info.numel * _DT[dt][1]:
            raise ContainerError(f"{path}: {name}: data offsets [{b0}, {b1}) do not fit {dt}{list(shape)}")
        out[name] = info
    return out


class Snapshot:
    """A snapshot directory: config.json and its tensors, memory-mapped on first use."""

    def __init__(self, snap):
        self.dir = snap
        with open(os.path.join(snap, "config.json")) as f:
            self.config = json.load(f)
        idx = os.path.join(snap, "model.safetensors.index.json")
        if os.path.exists(idx):
            with open(idx) as f:
                files = sorted(set(json.load(f)["weight_map"].values()))
        elif os.path.exists(os.path.join(snap, "model.safetensors")):
            files = ["model.safetensors"]
        else:
            files = sorted(p for p in os.listdir(snap) if p.endswith(".safetensors"))
        if not files:
            raise ContainerError(f"{snap}: no safetensors files")
        self.tensors = {}
        for fn in files:
            self.tensors.update(read_header(os.path.join(snap, fn)))
        self._maps = {}

    def has(self, name):
        return name in self.tensors

    def info(self, name):
        if name not in self.tensors:
            raise ContainerError(f"missing tensor {name}")
        return self.tensors[name]

    def array(self, name):
        """the tensor as stored (bf16 as raw uint16), a read-only view of the mapped file"""
        t = self.info(name)
        m = self._maps.get(t.path)
        if m is None:
            with open(t.path, "rb") as f:
                m = self._maps[t.path] = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        dt = _DT[t.dtype][0]
        return np.frombuffer(m, dtype=dt, count=t.numel, offset=t.offset).reshape(t.shape)

    def f32(self, name):
        """the tensor widened to f32 (bf16 and f16 exactly), as st_read_f32 does"""
        a = self.array(name)
        if self.info(name).dtype == "BF16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        return a.astype(np.float32)

    def close(self):
        """drop the snapshot's maps (a file stays mapped while an array viewing it lives)"""
        self._maps = {}

    # ---- the layers ----
    def n_layers(self):
        return int(self.config.get("num_hidden_layers", 0))

    def is_moe(self, i):
        c = self.config
        mol, mlt = c.get("mlp_only_layers"), c.get("mlp_layer_types")
        if isinstance(mol, list):
            return i not in [int(v) for v in mol]
        if isinstance(mlt, list) and i < len(mlt):
            return mlt[i] != "dense"
        return True

    def moe_layers(self):
        return [i for i in range(self.n_layers()) if self.is_moe(i)]


@dataclass
class HostLayer:
    """One MoE layer in host memory, in the device's upload layout (the fields
    DeviceLayer.from_host reads)."""
    D: int
    I: int
    Is: int
    E: int
    gs: int
    router_bf16: bool
    router: np.ndarray
    corr_bias: Optional[np.ndarray]
    logit_bias: Optional[np.ndarray]
    gu_q: np.ndarray
    gu_s: np.ndarray
    dn_q: np.ndarray
    dn_s: np.ndarray
    sg: Optional[np.ndarray]
    su: Optional[np.ndarray]
    sd: Optional[np.ndarray]


def _group_size(qs_numel, rows, K):
    """gs from a .qs tensor as `detect_group_size` finds it (`c/colibri.c:980-993`):
    one scale per row -> 0; else the finest candidate gs whose ceil(K / gs) groups
    per row give the scale count.  The device takes gs a power of two, a multiple of
    32, dividing K."""
    if qs_numel == rows:
        return 0
    for gs in (16, 32, 48, 64, 96, 128, 192, 256):
        if gs > K:
            break
        if qs_numel == rows * ((K + gs - 1) // gs):
            if gs % 32 or gs & (gs - 1) or K % gs:
                raise ContainerError(f"group size {gs} over {K} inputs is not supported on the device")
            return gs
    raise ContainerError(f"{qs_numel} scales over {rows} rows of {K} inputs match no group size")


def load_layer(snap: Snapshot, i: int, name: str = None):
    """(MoeConfig, HostLayer) of MoE layer i of a Laguna int4 snapshot"""
    c = snap.config
    if not snap.is_moe(i):
        raise ContainerError(f"layer {i} is dense")
    p = f"model.layers.{i}.mlp."
    D, E = int(c["hidden_size"]), int(c["num_experts"])
    K, I = int(c["num_experts_per_tok"]), int(c["moe_intermediate_size"])
    Is = int(c.get("shared_expert_intermediate_size", 0) or 0)
    if not snap.has(p + "experts.gate_up_proj.qs"):
        raise ContainerError(f"layer {i}: not an int4 container (no experts.gate_up_proj.qs)")
    gu_q, gu_s = snap.array(p + "experts.gate_up_proj"), snap.f32(p + "experts.gate_up_proj.qs")
    dn_q, dn_s = snap.array(p + "experts.down_proj"), snap.f32(p + "experts.down_proj.qs")
    if gu_q.dtype != np.uint8 or gu_q.shape != (E * 2 * I, D // 2):
        raise ContainerError(f"layer {i}: gate_up_proj is {gu_q.dtype}{list(gu_q.shape)}, want u8[{E * 2 * I}, {D // 2}]")
    if dn_q.dtype != np.uint8 or dn_q.shape != (E * D, I // 2):
        raise ContainerError(f"layer {i}: down_proj is {dn_q.dtype}{list(dn_q.shape)}, want u8[{E * D}, {I // 2}]")
    gs = _group_size(gu_s.size, E * 2 * I, D)
    if _group_size(dn_s.size, E * D, I) != gs:
        raise ContainerError(f"layer {i}: gate_up and down scale groups differ")
    rw = snap.info(p + "gate.weight")
    if rw.shape != (E, D):
        raise ContainerError(f"layer {i}: router is {list(rw.shape)}, want [{E}, {D}]")
    router_bf16 = rw.dtype == "BF16"
    router = snap.array(p + "gate.weight") if router_bf16 else snap.f32(p + "gate.weight")
    cb_name = p + "experts.e_score_correction_bias"
    corr = snap.f32(cb_name).reshape(E) if snap.has(cb_name) else np.zeros(E, np.float32)
    sg = su = sd = None
    if Is:
        sh = p + "shared_expert."
        sg, su, sd = (snap.array(sh + n + "_proj.weight") for n in ("gate", "up", "down"))
        for a, shp, n in ((sg, (Is, D), "gate"), (su, (Is, D), "up"), (sd, (D, Is), "down")):
            if a.dtype != np.uint16 or a.shape != shp:
                raise ContainerError(f"layer {i}: shared {n}_proj is {a.dtype}{list(a.shape)}, want bf16{list(shp)}")
    nt = c.get("norm_topk_prob", True)
    cfg = MoeConfig(name or f"laguna-layer{i}", D=D, E=E, K=K, I=I, Is=Is, route_act=ROUTE_SIGMOID, use_corr_bias=1,
                    norm_topk=int(bool(nt)) if isinstance(nt, bool) else 1,
                    route_scale=float(c.get("moe_routed_scaling_factor", 1.0)),
                    shared_mode=SHARED_UNSCALED if Is else 0, gs=gs, router_bf16=router_bf16)
    layer = HostLayer(D, I, Is, E, gs, router_bf16, router, corr, None, gu_q, gu_s.reshape(-1), dn_q,
                      dn_s.reshape(-1), sg, su, sd)
    return cfg, layer
