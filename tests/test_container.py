"""The Laguna int4 container reader (sabrewing_amd/container.py).

A small snapshot is written here with the standard safetensors library, in the
layout c/tools/convert_laguna_int4.py produces and c/laguna.c:349-452 reads: two
shards behind an index, a dense layer 0 (mlp_only_layers), MoE layers with the
fused packed-int4 experts and f32 `.qs` row scales (or group scales), the f32
router and correction bias, and the bf16 shared expert.  The CPU tests check the
header parser, the layer mapping and the descriptor; the GPU test runs a loaded
layer through lag_hip_moe_block against the oracle on the same tensors."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from sabrewing_amd import configs as cf
from sabrewing_amd import container as ct

D, E, K, I, Is = 256, 16, 4, 128, 128


def quant_rows(w, gs=0):
    """int4 with offset 8, low nibble = even column; per-row (gs 0) or per-gs-group
    scales amax/7 floored at 1e-8 (c/tools/convert_laguna_int4.py:49-60;
    c/tools/convert_fp8_to_int4.py:54-85)"""
    O, n = w.shape
    g = n if gs == 0 else gs
    wg = w.reshape(O, n // g, g)
    s = np.maximum(np.abs(wg).max(axis=2, keepdims=True) / 7.0, 1e-8).astype(np.float32)
    q = np.clip(np.rint(wg / s), -8, 7).astype(np.int32).reshape(O, n)
    packed = ((q[:, 0::2] + 8) | ((q[:, 1::2] + 8) << 4)).astype(np.uint8)
    return packed, (s[:, :, 0] if gs else s[:, 0, 0]).astype(np.float32)


def bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


def write_snapshot(d, gs=0, corr=True, seed=5):
    rng = np.random.default_rng(seed)
    cfg = {"hidden_size": D, "num_hidden_layers": 3, "num_experts": E, "num_experts_per_tok": K,
           "moe_intermediate_size": I, "shared_expert_intermediate_size": Is, "intermediate_size": 512,
           "moe_routed_scaling_factor": 2.5, "norm_topk_prob": True, "mlp_only_layers": [0]}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)
    shards = [{}, {}]
    shards[0]["model.layers.0.mlp.gate_proj.weight"] = bf16(rng.normal(0, 0.02, (512, D)))
    for i in (1, 2):
        p = f"model.layers.{i}.mlp."
        sh = shards[i - 1]
        gu_q, gu_s = quant_rows(rng.normal(0, 0.02, (E * 2 * I, D)).astype(np.float32), gs)
        dn_q, dn_s = quant_rows(rng.normal(0, 0.02, (E * D, I)).astype(np.float32), gs)
        sh[p + "experts.gate_up_proj"] = torch.from_numpy(gu_q)
        sh[p + "experts.gate_up_proj.qs"] = torch.from_numpy(gu_s)
        sh[p + "experts.down_proj"] = torch.from_numpy(dn_q)
        sh[p + "experts.down_proj.qs"] = torch.from_numpy(dn_s)
        sh[p + "gate.weight"] = torch.from_numpy(rng.normal(0, 0.02, (E, D)).astype(np.float32))
        if corr:
            sh[p + "experts.e_score_correction_bias"] = torch.from_numpy(rng.normal(0, 0.01, E).astype(np.float32))
        for n, shp in (("gate", (Is, D)), ("up", (Is, D)), ("down", (D, Is))):
            sh[p + f"shared_expert.{n}_proj.weight"] = bf16(rng.normal(0, 0.02, shp))
    wm = {}
    for k, sh in enumerate(shards):
        fn = f"model-{k + 1:05d}-of-00002.safetensors"
        save_file(sh, os.path.join(d, fn))
        wm.update({n: fn for n in sh})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    return shards


def test_header_and_arrays(tmp_path):
    shards = write_snapshot(str(tmp_path))
    s = ct.Snapshot(str(tmp_path))
    assert s.moe_layers() == [1, 2] and not s.is_moe(0)
    p = "model.layers.2.mlp."
    assert s.info(p + "experts.gate_up_proj").dtype == "U8"
    assert s.info(p + "shared_expert.gate_proj.weight").dtype == "BF16"
    # every tensor reads back with the bytes that were written
    for sh in shards:
        for n, t in sh.items():
            got = s.array(n)
            want = t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()
            assert got.shape == tuple(t.shape) and np.array_equal(got, want), n
    # bf16 widened exactly to f32
    w = s.f32(p + "shared_expert.up_proj.weight")
    assert np.array_equal(w, shards[1][p + "shared_expert.up_proj.weight"].float().numpy())
    s.close()


def test_layer_descriptor(tmp_path):
    write_snapshot(str(tmp_path))
    s = ct.Snapshot(str(tmp_path))
    cfg, L = ct.load_layer(s, 1)
    assert (cfg.D, cfg.E, cfg.K, cfg.I, cfg.Is) == (D, E, K, I, Is)
    # c/laguna.c:817-819: sigmoid, corr-bias selection, norm_topk, route_scale, unscaled shared
    assert cfg.route_act == cf.ROUTE_SIGMOID and cfg.use_corr_bias == 1 and cfg.norm_topk == 1
    assert cfg.route_scale == 2.5 and cfg.shared_mode == cf.SHARED_UNSCALED
    assert cfg.gs == 0 and not cfg.router_bf16
    assert L.gu_q.shape == (E * 2 * I, D // 2) and L.gu_s.shape == (E * 2 * I,)
    assert L.corr_bias.shape == (E,) and L.sg.dtype == np.uint16
    with pytest.raises(ct.ContainerError):
        ct.load_layer(s, 0)                          # the dense layer
    s.close()


def test_group_scales_and_missing_bias(tmp_path):
    write_snapshot(str(tmp_path), gs=32, corr=False)
    s = ct.Snapshot(str(tmp_path))
    cfg, L = ct.load_layer(s, 2)
    assert cfg.gs == 32 and L.gu_s.size == E * 2 * I * (D // 32) and L.dn_s.size == E * D * (I // 32)
    assert np.array_equal(L.corr_bias, np.zeros(E, np.float32))   # calloc'd zeros (c/laguna.c:414)
    s.close()


def test_bad_headers_refused(tmp_path):
    p = tmp_path / "model.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ct.ContainerError):
        ct.read_header(str(p))
    hdr = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 64]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)   # offsets past the file
    with pytest.raises(ct.ContainerError):
        ct.read_header(str(p))
    hdr = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)   # size does not match the shape
    with pytest.raises(ct.ContainerError):
        ct.read_header(str(p))


@pytest.mark.gpu
@pytest.mark.parametrize("gs", [0, 32])
def test_container_layer_on_device(be, orc, tmp_path, gs):
    from oracle import synth
    from sabrewing_amd.backend import DeviceLayer, desc_of
    write_snapshot(str(tmp_path), gs=gs)
    s = ct.Snapshot(str(tmp_path))
    cfg, L = ct.load_layer(s, 2)
    OL = synth.Layer(**{k: getattr(L, k) for k in synth.Layer.__dataclass_fields__})
    rng = np.random.default_rng(11)
    for S_ in (1, 5, 40):
        x = rng.standard_normal((S_, D)).astype(np.float32)
        base = rng.standard_normal((S_, D)).astype(np.float32)
        want = orc.moe_block_rows(synth.desc_of(cfg), OL, x, base)
        dl = DeviceLayer.from_container(be, s, 2)
        assert dl.cfg == cfg
        got = be.moe_block(desc_of(cfg), dl.weights(), x, base)
        xd = be.upload(x)
        _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, S_)
        xd.free(); dl.free()
        _, sel_w, _ = orc.route(synth.desc_of(cfg), OL, x)
        assert np.array_equal(sel, sel_w)
        dw = want - base
        assert float(np.max(np.abs((got - base) - dw))) / float(np.max(np.abs(dw))) <= 2e-3
    s.close()
