"""Device self-checks: MFMA lane layout, the device libm against the host's
glibc, and the device generator against the host generator (bit for bit)."""
import numpy as np
import pytest

from sabrewing_amd import synth as S
from sabrewing_amd.configs import WEIGHT_SIGMA

pytestmark = pytest.mark.gpu


def test_mfma_layout(be):
    out = be.selftest(np.zeros(0, np.float32))
    lane = np.arange(64)[:, None]; j = np.arange(4)[None, :]
    row, col = 4 * (lane // 16) + j, lane % 16
    assert np.array_equal(out[:256].reshape(64, 4), (32 * row + col).astype(np.float32))
    assert np.array_equal(out[256:512].reshape(64, 4), (2 * row + (col & 1)).astype(np.float32))
    # int8 16x16x64: lane l = (row or column l % 16, k quarter l // 16), its 16
    # bytes meeting the same bytes of the other operand's lane
    b = np.arange(16)[None, :]
    A = ((7 * np.arange(64)[:, None] + 13 * b) % 17 - 8).reshape(4, 16, 16)     # [quarter][row][byte]
    B = ((5 * np.arange(64)[:, None] + 3 * b + 1) % 23 - 11).reshape(4, 16, 16)
    C = np.einsum("qib,qjb->ij", A, B)
    assert np.array_equal(out[512:768].reshape(64, 4), C[row, col].astype(np.float32))


def test_device_libm_matches_host(be, orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    xs = np.concatenate([bits.view(np.float32),
                         np.linspace(-110, 95, 1 << 18).astype(np.float32),         # the expf domain
                         np.linspace(-30, 25, 1 << 18).astype(np.float32),          # gate range
                         np.array([0.0, -0.0, np.inf, -np.inf, 88.72283, -103.97208, 1e-30, -1.0,
                                   -0.99999994, 0.41421, 3e38], np.float32)])
    xs = xs[~np.isnan(xs)]
    out = be.selftest(xs)
    n = xs.size
    e_dev, l_dev = out[768:768 + n], out[768 + n:768 + 2 * n]
    e_host, l_host = orc.expf(xs), orc.log1pf(xs)
    assert np.array_equal(e_dev.view(np.uint32), e_host.view(np.uint32))
    ok = (l_dev.view(np.uint32) == l_host.view(np.uint32)) | (np.isnan(l_dev) & np.isnan(l_host))
    assert ok.all()
    # sqrt rounded to nearest (the SQRT_SOFTPLUS gate): numpy's float32 sqrt is IEEE, and the
    # positive inputs include subnormals and every exponent
    pos = xs >= 0
    s_dev, s_host = out[768 + 2 * n:768 + 3 * n], np.sqrt(np.where(pos, xs, np.float32(0)))
    assert np.array_equal(s_dev[pos].view(np.uint32), s_host[pos].view(np.uint32))
    assert np.isnan(s_dev[xs < 0]).all()


def test_generator_matches_host(be, orc):
    seed = S.tensor_seed(99, 3, S.T_ROUTER)
    n = 1 << 20
    buf = be.alloc(n * 4)
    be.gen_normal(buf, n, seed, WEIGHT_SIGMA, offset=12345)
    got = be.d2h(buf, n, np.float32)
    want = orc.normal(n, seed, WEIGHT_SIGMA, offset=12345)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    be.gen_normal(buf, n, seed, 1.0, to_bf16=True)
    assert np.array_equal(be.d2h(buf, n, np.float32).view(np.uint32), orc.bf16_round(orc.normal(n, seed, 1.0)).view(np.uint32))
    b16 = be.alloc(n * 2)
    be.gen_bf16(b16, n, seed, WEIGHT_SIGMA)
    assert np.array_equal(be.d2h(b16, n, np.uint16), orc.to_bf16(orc.normal(n, seed, WEIGHT_SIGMA)))
    buf.free(); b16.free()
    for gs, K, rows in ((32, 4096, 96), (32, 1024, 64), (64, 2048, 16), (0, 1024, 40)):
        ng = K // gs if gs else 1
        q, s = be.alloc(rows * K // 2), be.alloc(rows * ng * 4)
        be.gen_q4(q, s, seed, WEIGHT_SIGMA, rows, K, gs, row0=7)
        wq, ws = orc.gen_q4(seed, WEIGHT_SIGMA, rows, K, gs, row0=7)
        assert np.array_equal(be.d2h(q, (rows, K // 2), np.uint8), wq), gs
        assert np.array_equal(be.d2h(s, (rows, ng), np.float32).view(np.uint32), ws.view(np.uint32)), gs
        q.free(); s.free()
