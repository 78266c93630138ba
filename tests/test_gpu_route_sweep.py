"""Route sweep: shapes and dtypes chosen to launch every kernel instantiation of
the dispatch trees (checked by tests/test_route_coverage.py against the kernel
trace of this suite), each against an independent reference.

* activation quants (plain, head-major, rmsnorm-, add-rmsnorm- and silu*up-
  fused): codes and scales bit-exact with the numpy restatement of
  quant.cpp:179-193 (plain / head-major) or within one code of the fp64
  producer (fused), over every vector width and workgroup size;
* weight-only linears: against torch fp64 on the dequantized weight (whose
  dequant is bit-exact with the oracle), 1e-3 * RMS (+ half an fp16 ulp for
  fp16 outputs), over m buckets, row groups, split-K plans, long K (several
  chunks per lane), activation / output / scale dtypes and group sizes;
* W8A8: every AUTO route's output equals the bounds-checked generic kernel's
  bit for bit (one shared epilogue), its int32 accumulators equal the exact
  integer product, and the generic output is within 1e-3 * RMS of fp64.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close_rms, host

pytestmark = pytest.mark.gpu

F32, F16 = torch.float32, torch.float16


def _gen(dev, seed):
    return torch.Generator(device=dev).manual_seed(seed)


def _ref_quant_np(y):
    """quant.cpp:179-193 on fp32 values: absmax / 127, round half even, clamp."""
    y = y.astype(np.float32)
    am = np.max(np.abs(y), axis=1)
    s = (am / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(s[:, None] > 0, np.rint(y / s[:, None]), 0)
    return np.clip(q, -127, 127).astype(np.int8), s


def _check_close_codes(xq, s, y_ref):
    q_ref, s_ref = _ref_quant_np(y_ref)
    s = host(s)
    assert np.allclose(s, s_ref, rtol=2e-6, atol=0), np.max(np.abs(s / s_ref - 1))
    d = np.abs(host(xq).astype(np.int32) - q_ref.astype(np.int32))
    assert d.max() <= 1
    assert (d > 0).mean() < 1e-3


# vectors of 8 per row (k / 8) that select each workgroup size and vector count
ACT_STEPS = [40, 200, 300, 500, 700, 900, 1100, 1300, 1500, 1700, 1900, 2048]


@pytest.mark.parametrize("m", [1, 5, 260])
@pytest.mark.parametrize("dt", [F32, F16])
def test_sweep_act_quant(dev, nq, m, dt):
    for steps in ACT_STEPS + [2500, 3750, 7500, None]:
        k = 8 * steps if steps else 100                           # 100: the scalar row kernel
        x = (torch.randn((m, k), generator=_gen(dev, m + k), device=dev) * 3).to(dt)
        xq, s = nq.act_quant(x)
        q_ref, s_ref = _ref_quant_np(host(x.float()))
        assert np.array_equal(host(s), s_ref), (m, k)
        assert np.array_equal(host(xq), q_ref), (m, k)


@pytest.mark.parametrize("dt", [F32, F16])
def test_sweep_act_quant_heads(dev, nq, dt):
    for heads, d in ((2, 64), (12, 128), (16, 128), (24, 128), (32, 128), (40, 128), (64, 128), (16, 1024)):
        s_len = 3
        a = torch.randn((heads, s_len, d), generator=_gen(dev, heads * d), device=dev).to(dt)
        xq, sc = nq.act_quant_heads(a)
        flat = host(a.float()).transpose(1, 0, 2).reshape(s_len, heads * d)
        q_ref, s_ref = _ref_quant_np(flat)
        assert np.array_equal(host(sc), s_ref) and np.array_equal(host(xq), q_ref), (heads, d)


FUSED_K = [64, 72, 1536, 2048, 3072, 4096, 5120, 6144, 7168, 8192, 8960, 12288, 16384, 20000, 30000]


@pytest.mark.parametrize("m", [1, 7, 300])
@pytest.mark.parametrize("dt", [F32, F16])
def test_sweep_rmsnorm_quant(dev, nq, m, dt):
    for k in FUSED_K:
        x = torch.randn((m, k), generator=_gen(dev, m * k), device=dev).to(dt)
        w = 1 + 0.1 * torch.randn(k, generator=_gen(dev, k), device=dev)
        xq, s = nq.rmsnorm_quant(x, w, 1e-6)
        xs = host(x.float()).astype(np.float64)
        y = xs / np.sqrt((xs * xs).mean(1, keepdims=True) + 1e-6) * host(w).astype(np.float64)
        _check_close_codes(xq, s, y)
        r = torch.randn((m, k), generator=_gen(dev, m * k + 1), device=dev).to(dt)
        h, xq2, s2 = nq.add_rmsnorm_quant(x, r, w, 1e-6)
        assert torch.equal(h, x + r)
        hs = host(h.float()).astype(np.float64)
        _check_close_codes(xq2, s2, hs / np.sqrt((hs * hs).mean(1, keepdims=True) + 1e-6) * host(w).astype(np.float64))


@pytest.mark.parametrize("m", [1, 7, 300])
@pytest.mark.parametrize("dt", [F32, F16])
def test_sweep_silu_mul_quant(dev, nq, m, dt):
    for k in FUSED_K + [100]:                                     # 100: the bounds-checked kernel
        gu = (torch.randn((m, 2 * k), generator=_gen(dev, m + k), device=dev) * 2).to(dt)
        xq, s = nq.silu_mul_quant(gu[:, :k], gu[:, k:])
        g = host(gu[:, :k].float()).astype(np.float64)
        u = host(gu[:, k:].float()).astype(np.float64)
        _check_close_codes(xq, s, g / (1 + np.exp(-g)) * u)


@pytest.mark.parametrize("sdt", [F32, F16])
def test_sweep_quantize_dequant_q4g(dev, nq, orc, sdt):
    """Every vector width of the group quantizer (group = 8 * 2^j) and the
    per-block / per-byte kernels, bit-exact with the oracle; dequantize to fp32
    and fp16 equals codes x stored scale."""
    for n, k, g in ((64, 1024, 8), (64, 1024, 16), (64, 1024, 32), (64, 1024, 64), (64, 1024, 128),
                    (64, 1024, 256), (64, 1024, 512), (33, 96, 24), (17, 101, 32), (9, 64, 3)):
        w = (torch.randn((n, k), generator=_gen(dev, n * k + g), device=dev) * 0.02)
        t = nq.quantize_q4g(w, g, scale_dtype=sdt)
        p, sc = orc.quantize_q4g(host(w), g)
        assert np.array_equal(host(t.q), p), (n, k, g)
        assert np.array_equal(host(t.scale.float()), sc.astype(np.float16).astype(np.float32) if sdt == F16 else sc)
        codes = torch.stack([t.q.int() & 15, t.q.int() >> 4], -1).reshape(n, -1)[:, :k] - 8
        ref = codes.float() * t.scale.float().repeat_interleave(g, 1)[:, :k]
        for odt in (F32, F16):
            assert torch.equal(nq.dequantize_q4g(t, out_dtype=odt), ref.to(odt)), (n, k, g, odt)


# ---- weight-only linears ------------------------------------------------------------------
def _wq_ref(nq, mode, t, g, x, bias):
    wd = (nq.dequantize_q8(t) if mode == "q8" else nq.dequantize_q4g(t)).double()
    y = x.double() @ wd.t()
    return y + bias.double() if bias is not None else y


WQ_SHAPES = [  # (m, n, k): GEMV buckets, row-group rules, GEMM tile plans, split K
    # one fp16 row, 9216 < k <= 16384: half chunks over up to 16 waves, 3 / 4 / 6 rows per workgroup
    (1, 1000, 11008), (1, 4100, 12288), (1, 8200, 10240),
    # m = 3..4 fp16 on wide weights: 4 weight rows per workgroup (int8 n >= 6144, int4 n >= 3584, k <= 4096)
    (3, 6200, 2560), (4, 3600, 3072),
    # fp32 x at m = 2..4 past k = 10240: pairs of 4-row workgroups on the 576-thread bound
    (2, 1100, 12288), (4, 1100, 12288),
    # one fp16 row, int8, 9216 < k <= 12288: one chunk per lane over up to 16 waves, 4 rows
    (1, 1030, 11008),
    # int4 short rows (k <= 1024, or 2048 with two half chunks per lane): one wave, 2 or 4 weight rows
    (1, 8300, 640), (2, 1100, 1024), (2, 8200, 512), (3, 2000, 768), (8, 9000, 640), (1, 9000, 1088), (3, 9000, 1984),
    # the one-chunk int4 GEMV forms that now start past k = 2048
    (1, 2000, 3072), (2, 1536, 3072), (3, 700, 3072), (8, 1536, 2560),
    # one fp16 row of int4 from k = 2048 on tall weights: the half-chunk GEMV, 6 rows
    (1, 4100, 2080),
    # int8 1024 < k <= 2048 in one wave: m = 1 up to 6144 rows, fp16 m = 3..4 from 6144
    (1, 1100, 2048), (4, 6200, 1088),
    (1, 1536, 1536), (1, 4864, 896), (1, 1536, 8960), (1, 8960, 5120), (1, 40000, 1536), (1, 1024, 4096),
    (2, 1536, 8960), (2, 4864, 896), (2, 40000, 1536), (2, 256, 1536), (2, 8960, 1536),
    (3, 1536, 2048), (4, 4864, 896), (4, 1536, 8960), (4, 256, 1536),
    (5, 8960, 1536), (6, 1536, 8960), (7, 4864, 896), (8, 2048, 8192), (8, 512, 1536),
    (9, 896, 896), (12, 4608, 896), (12, 1536, 8960), (15, 1536, 4224),
    (16, 1536, 1536), (24, 8960, 1536), (32, 1536, 8960), (33, 8960, 1536), (48, 4864, 896),
    (64, 1536, 8960), (64, 896, 4864), (65, 1536, 1536), (100, 2000, 1024), (130, 9000, 512),
    (256, 1536, 1536), (300, 4864, 896), (1100, 640, 512), (2048, 1536, 1536),
    # each tile of the wide kernels' tables, as the tile picker chooses them (k = 256)
    (32, 8960, 256), (32, 17920, 256), (96, 17920, 256), (192, 17920, 256), (256, 17920, 256),
    (300, 17920, 256), (512, 17920, 256), (640, 17920, 256), (1024, 17920, 256),
    # split K: the shallow wide tiles (k % 128 == 0) and the 16-row kernel (k % 128 == 32),
    # one to four 16-row blocks, one or two 16-column blocks
    (16, 1536, 4096), (40, 1536, 4096), (100, 1536, 4096),
    (16, 1536, 4128), (24, 1536, 4128), (24, 6000, 4128), (40, 1536, 4128), (56, 1536, 4128), (100, 1536, 4128), (16, 6000, 4128),
    (24, 1536, 1536), (40, 6000, 1024),
    # one activation row on tall weights: 4 and 8 weight rows per workgroup
    (1, 24600, 2560), (1, 65600, 1056),
    # m = 5..8 on large weights (int8 with fp16 x; fp32 x from n, k >= 4096 or on long K): the MFMA GEMM
    (6, 4160, 4096), (8, 17920, 1024), (7, 64, 9728), (5, 3100, 18464), (6, 2100, 9344), (3, 3100, 4224), (8, 1000, 4160), (2, 4100, 4096), (2, 2048, 8192), (4, 8200, 3072), (4, 1536, 2560), (8, 1100, 2560),
    # split wide tiles from k = 2048 (k % 128 == 0)
    (40, 4608, 3584), (16, 1536, 2048),
    # long K (several chunks per lane): int8 past k = 9216, int4 past k = 18432, each m bucket
    (1, 100, 9232), (2, 37, 14336), (4, 70, 9744), (7, 50, 10240),
    (1, 60, 18944), (2, 37, 18464), (3, 50, 20480), (8, 45, 18944), (1, 8200, 9232), (1, 8200, 18464),
    # outside the fast paths (k % 32 != 0: the bounds-checked kernels)
    (3, 300, 100), (1, 129, 90),
]
WQ_MODES = [("q8", 0, None), ("q4g", 32, F16), ("q4g", 32, F32), ("q4g", 64, F16), ("q4g", 64, F32),
            ("q4g", 128, F16), ("q4g", 128, F32), ("q4g", 256, F32)]


@pytest.mark.parametrize("mode,g,sdt", WQ_MODES)
@pytest.mark.parametrize("xdt,ydt", [(F16, F16), (F16, F32), (F32, F32), (F32, F16)])
def test_sweep_weight_only(dev, nq, mode, g, sdt, xdt, ydt):
    for i, (m, n, k) in enumerate(WQ_SHAPES):
        print(f"{mode} g{g} {m}x{n}x{k} {xdt}->{ydt}", flush=True)
        gen = _gen(dev, m * 31 + n * 7 + k + g)
        w = torch.randn((n, k), generator=gen, device=dev) * 0.02
        t = nq.quantize_q8(w) if mode == "q8" else nq.quantize_q4g(w, g, scale_dtype=sdt)
        x = torch.randn((m, k), generator=gen, device=dev).to(xdt)
        b = torch.randn(n, generator=gen, device=dev) if i % 3 == 0 else None
        y = nq.linear_q8(x, t, b, out_dtype=ydt) if mode == "q8" else nq.linear_q4g(x, t, b, out_dtype=ydt)
        ref = _wq_ref(nq, mode, t, g, x, b)
        assert_close_rms(host(y.double()), host(ref), f"{mode} g{g} {m}x{n}x{k} {xdt}->{ydt}", fp16_out=ydt == F16)
        if 5 <= m <= 8 and k > 9216:  # the GEMV slices AUTO leaves to the GEMM there (fp32 x): forced
            from nanoinfer_amd import _lib as L
            lin = nq.linear_q8 if mode == "q8" else nq.linear_q4g
            y2 = lin(x, t, b, out_dtype=ydt, path=L.NQ_PATH_GEMV)
            assert_close_rms(host(y2.double()), host(ref), f"GEMV {mode} {m}x{n}x{k}", fp16_out=ydt == F16)


# ---- W8A8 ---------------------------------------------------------------------------------
W8A8_SHAPES = [
    (1, 1536, 1536), (1, 4864, 896), (1, 1536, 8960), (1, 64, 4096), (1, 700, 512),
    (2, 1536, 1536), (2, 4864, 896), (2, 8960, 1536), (2, 1536, 8960), (3, 8960, 1536), (3, 1536, 4096),
    (4, 256, 1536), (4, 8960, 1536), (4, 1536, 8960), (5, 1536, 8960), (6, 2048, 4096), (8, 256, 1536),
    (8, 1536, 1536), (8, 4864, 896), (8, 8960, 1536), (8, 1536, 8960), (8, 17920, 1536), (8, 1536, 3072),
    # the decode kernel's in-kernel quant at m = 2..8 (k up to 4096 at m <= 4)
    (2, 1536, 4096), (2, 8960, 3072), (4, 8960, 1024), (3, 1536, 2560), (5, 8960, 768), (8, 256, 512),
    # m = 5..8 on large weights with long rows or many rows: the K-split tile GEMV over the codes
    (6, 4700, 3584), (8, 2100, 8192),
    # the skinny kernel: k % 64 != 0 (no wide tiles), one to four 16-row blocks, 64-row blocks past 64;
    # m <= 16 on long K
    (12, 8960, 1040), (24, 8960, 1040), (40, 8960, 1040), (64, 8960, 1040), (100, 8960, 1040), (12, 8960, 8192),
    # each wide tile the cost model picks (k = 128), and long K on 64 x 64 tiles in K ranges
    (65, 64, 128), (65, 8960, 128), (192, 8960, 128), (768, 12288, 128), (384, 4096, 128), (65, 17920, 128),
    (384, 17920, 128), (512, 17920, 128), (1536, 12288, 128), (256, 17920, 128), (640, 17920, 128),
    (1024, 17920, 128), (65, 64, 4096), (512, 512, 65536),
    (9, 1536, 1536), (12, 256, 8960), (16, 256, 1536), (16, 1536, 1536), (16, 8960, 1536), (16, 1536, 8960),
    (16, 4864, 896), (16, 2048, 3072), (17, 1536, 1536), (24, 8960, 1536), (32, 256, 1536), (32, 1536, 1536),
    (32, 1536, 4096), (32, 8960, 1536), (32, 1536, 8960), (33, 512, 1536), (48, 1536, 1536), (64, 256, 1536),
    (64, 1536, 1536), (64, 8960, 1536), (64, 1536, 8960), (64, 17920, 1536), (65, 1536, 1536), (100, 1000, 960),
    (128, 256, 8960), (128, 1536, 8960), (128, 8960, 1536), (200, 1003, 192), (256, 1536, 1536),
    (300, 640, 4096), (512, 1536, 8960), (512, 2048, 1536), (512, 17920, 1536), (1024, 8960, 1536),
    (2048, 8960, 1536), (2048, 1536, 1536),
    # 64 x 128 tiles over more than one round (more than 256 of them, k <= 4096)
    (17, 33000, 256), (40, 33000, 512),
    # long K on the GEMV (several chunks per lane past k = 9216), each m bucket
    (1, 100, 9232), (2, 37, 14336), (3, 70, 9744), (7, 2100, 9232), (1, 64, 32768),
]


@pytest.mark.parametrize("xdt,ydt", [(F16, F16), (F32, F32), (F16, F32), (F32, F16)])
def test_sweep_w8a8(dev, nq, xdt, ydt):
    from nanoinfer_amd import _lib as L
    for i, (m, n, k) in enumerate(W8A8_SHAPES):
        gen = _gen(dev, m * 13 + n + k)
        w = torch.randn((n, k), generator=gen, device=dev) * 0.02
        t = nq.quantize_q8(w)
        x = torch.randn((m, k), generator=gen, device=dev).to(xdt)
        b = torch.randn(n, generator=gen, device=dev) if i % 2 else None
        print(f"w8a8 {m}x{n}x{k} {xdt}->{ydt}", flush=True)
        bits = torch.int16 if ydt == F16 else torch.int32
        y = nq.linear_w8a8(x, t, b, out_dtype=ydt)
        # the bounds-checked generic kernel where it is quick, else the forced MFMA path
        other = L.NQ_PATH_GENERIC if m * n * k <= 1 << 30 else L.NQ_PATH_MFMA
        y_gen = nq.linear_w8a8(x, t, b, out_dtype=ydt, path=other)
        assert torch.equal(y.view(bits), y_gen.view(bits)), (m, n, k, xdt, ydt)
        xq, a_s = nq.act_quant(x)
        acc_ref = (xq.double() @ t.q.double().t())
        acc = nq.w8a8_acc_i32(xq, t.q)
        assert torch.equal(acc.double(), acc_ref), (m, n, k)
        y_pre = nq.gemm_w8a8(xq, a_s, t, b, out_dtype=ydt)                     # the pre-quantized entry
        assert torch.equal(y_pre.view(bits), y_gen.view(bits)), ("gemm", m, n, k)
        ref = acc_ref * a_s.double()[:, None] * t.scale.double()[None, :]
        if b is not None:
            ref = ref + b.double()
        assert_close_rms(host(y_gen.double()), host(ref), f"w8a8 {m}x{n}x{k}", fp16_out=ydt == F16)


@pytest.mark.parametrize("xdt", [F32, F16])
def test_sweep_lm_head_argmax(dev, nq, xdt):
    """The fused greedy pick over every GEMV form it runs (m buckets, 2 / 4 / 8
    weight rows): ids equal the reference scan over nq_linear_q8's fp32 logits."""
    for m in (1, 2, 3, 4, 5, 8):
        for n, k in ((1024, 1536), (4096, 896), (40000, 1536)):
            gen = _gen(dev, m * n + k)
            t = nq.quantize_q8(torch.randn((n, k), generator=gen, device=dev) * 0.02)
            x = torch.randn((m, k), generator=gen, device=dev).to(xdt)
            ids = host(nq.lm_head_argmax(x, t))
            logits = host(nq.linear_q8(x, t, out_dtype=F32))
            assert ids.tolist() == [int(np.argmax(r)) for r in logits], (m, n, k, xdt)
