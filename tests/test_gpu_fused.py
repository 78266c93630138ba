"""Activation quant fused into its producers (rmsnorm, silu * up): scales and
codes against the act quant applied to the same producer computed in fp64."""
import numpy as np
import pytest
import torch

from gpu_util import host, to_dev

pytestmark = pytest.mark.gpu


def ref_quant(y):
    """quant.cpp:179-193 on fp64-computed values rounded to fp32."""
    y = y.astype(np.float32)
    am = np.max(np.abs(y), axis=1)
    s = (am / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(s[:, None] > 0, np.rint(y / s[:, None]), 0)
    return np.clip(q, -127, 127).astype(np.int8), s


def check(xq, s, y_ref):
    q_ref, s_ref = ref_quant(y_ref)
    s = host(s)
    assert np.allclose(s, s_ref, rtol=2e-6, atol=0), np.max(np.abs(s / s_ref - 1))
    d = np.abs(host(xq).astype(np.int32) - q_ref.astype(np.int32))
    assert d.max() <= 1                      # a rounding boundary may fall either way
    assert (d > 0).mean() < 1e-3


@pytest.mark.parametrize("m,k,dt", [(1, 1536, torch.float16), (7, 1536, torch.float32), (512, 1536, torch.float16),
                                    (3, 8960, torch.float16), (5, 100, torch.float32), (2, 40000, torch.float16),
                                    (256, 8960, torch.float16)])
def test_rmsnorm_quant(dev, nq, m, k, dt):
    rng = np.random.default_rng(m * 7 + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = (1 + 0.1 * rng.normal(0, 1, k)).astype(np.float32)
    xd = to_dev(x, dev).to(dt)
    xq, s = nq.rmsnorm_quant(xd, to_dev(w, dev), 1e-6)
    xs = host(xd.float()).astype(np.float64)
    y = xs / np.sqrt((xs * xs).mean(1, keepdims=True) + 1e-6) * w
    check(xq, s, y)


@pytest.mark.parametrize("m,k,dt", [(1, 8960, torch.float16), (16, 8960, torch.float32), (512, 8960, torch.float16),
                                    (4, 72, torch.float32), (300, 16384, torch.float32), (256, 8200, torch.float16)])
def test_silu_mul_quant_on_fused_halves(dev, nq, m, k, dt):
    rng = np.random.default_rng(m + k)
    gu = rng.normal(0, 2, (m, 2 * k)).astype(np.float32)
    gd = to_dev(gu, dev).to(dt)
    xq, s = nq.silu_mul_quant(gd[:, :k], gd[:, k:])
    g = host(gd[:, :k].float()).astype(np.float64)
    u = host(gd[:, k:].float()).astype(np.float64)
    check(xq, s, g / (1 + np.exp(-g)) * u)


def test_fused_errors(dev, nq):
    x = torch.zeros((2, 16), device=dev)
    with pytest.raises(ValueError):
        nq.rmsnorm_quant(x, torch.ones(8, device=dev), 1e-6)
    with pytest.raises(ValueError):
        nq.silu_mul_quant(x[:, :8], x[:, :4])


@pytest.mark.parametrize("m,k,dt,inplace", [(1, 1536, torch.float16, False), (512, 1536, torch.float16, True),
                                            (7, 1536, torch.float32, True), (5, 100, torch.float32, False),
                                            (300, 8960, torch.float16, False)])
def test_add_rmsnorm_quant(dev, nq, m, k, dt, inplace):
    """h equals the tensor add x + r bit for bit; codes and scales follow the
    fused rmsnorm quant of h (and equal nq.rmsnorm_quant(h) exactly)."""
    rng = np.random.default_rng(m + k)
    x = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32), dev).to(dt)
    r = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32), dev).to(dt)
    w = to_dev((1 + 0.1 * rng.normal(0, 1, k)).astype(np.float32), dev)
    h_ref = x + r
    x_in = x.clone()
    h, xq, s = nq.add_rmsnorm_quant(x_in, r, w, 1e-6, inplace=inplace)
    assert torch.equal(h, h_ref)
    if inplace:
        assert h.data_ptr() == x_in.data_ptr()
    xq2, s2 = nq.rmsnorm_quant(h_ref, w, 1e-6)
    assert torch.equal(xq, xq2) and torch.equal(s, s2)


@pytest.mark.parametrize("h,s,d,dt", [(12, 512, 128, torch.float16), (2, 7, 64, torch.float32), (12, 1, 128, torch.float16),
                                      (3, 300, 24, torch.float16)])
def test_act_quant_heads(dev, nq, h, s, d, dt):
    """Codes and scales of the head-major variant equal nq.act_quant of the
    transposed matrix bit for bit."""
    g = torch.Generator(device=dev).manual_seed(h * s + d)
    a = torch.randn((h, s, d), generator=g, device=dev).to(dt)
    xq, sc = nq.act_quant_heads(a)
    xq2, sc2 = nq.act_quant(a.transpose(0, 1).reshape(s, h * d).contiguous())
    assert torch.equal(xq, xq2) and torch.equal(sc, sc2)
