"""Workload byte/flop accounting (the roofline denominators) against the
closed forms of the benchmark definition."""
from sabrewing_amd import configs as cf


def test_expert_bytes():
    assert cf.C1.expert_bytes() == 3 * 2048 * 1024 // 2 + 3 * 2048 * 1024 // 32 * 4 == 3_932_160
    assert cf.C2.expert_bytes() == 7_864_320
    assert cf.C2.router_bytes() == 256 * 4096 * 2 and cf.C1.router_bytes() == 64 * 2048 * 4
    assert cf.C2.shared_bytes() == 3 * 4096 * 1024 * 2


def test_step_bytes_batch1():
    # K distinct experts + router + shared (+ activations) per token
    # weights: the benchmark's per-token figures less their 6 B/element of activations
    assert cf.C2.step_bytes(1, 10) - 3 * 4096 * 4 == 105_930_752 - 6 * 4096
    assert cf.C1.step_bytes(1, 8) - 3 * 2048 * 4 == 31_993_856 - 6 * 2048
    # activations here: x read (f32) + out read-modify-write (f32) = 12 B per element
    assert cf.C2.step_bytes(3, 10) - cf.C2.step_bytes(1, 10) == 2 * 12 * 4096


def test_flops_prefill():
    f = cf.C2.flops(2048)
    assert abs(f - 5.71e11) / 5.71e11 < 0.01
