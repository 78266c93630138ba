"""GPU parity of the three linears against the oracle.

Integer work is bit-exact (W8A8 int32 accumulators on every kernel path);
floating-point outputs meet max|err| <= 1e-3 * RMS(y) (plus half an fp16 ulp
for fp16 outputs); the W8A8 GEMV and MFMA paths give bit-identical outputs
(cpp/tests/test_cuda.cpp:217-251's gemv==tiled claim)."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close_rms, host, rms, to_dev
from test_oracle import same_bits

pytestmark = pytest.mark.gpu

F32, F16 = torch.float32, torch.float16


def data(m, n, k, seed, wsig=0.02, bias=False):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = rng.normal(0, wsig, (n, k)).astype(np.float32)
    b = rng.normal(0, 1, n).astype(np.float32) if bias else None
    return x, w, b


# ---- weight-only int8 -----------------------------------------------------------------
Q8_CASES = [
    (1, 4864, 896, False, F32, F32),      # config 1
    (1, 151936, 1536, False, F16, F16),   # config 5 LM head
    (4, 8192, 896, False, F32, F32),      # test_cuda.cpp:437 batched decode
    (2, 896, 896, True, F32, F32),        # :438 +bias
    (8, 100, 90, False, F32, F32),        # :441 ragged k (generic kernel)
    (3, 1536, 1536, True, F16, F32),
    (16, 896, 896, True, F32, F16),       # m > 8: slices of 8 rows
    (100, 896, 4864, False, F32, F32),    # :440 ragged m, wide k
    (5, 64, 16384, False, F32, F32),      # k beyond one workgroup (generic)
    (8, 1536, 8960, True, F32, F32),      # fp32 x, m = 5..8, long K: 4 weight x 4 activation rows, pairs
    (6, 4864, 896, False, F32, F16),      # fp32 x, m = 5..8: 4 x 4 rows per workgroup, pairs
    (7, 1001, 2048, True, F32, F32),      # fp32 x, m = 5..8, small: pairs, ragged n
    (5, 8960, 1536, True, F32, F32),      # fp32 x, short K, tall: 8 x 4 rows, pairs, 1 row in the second
    (8, 2048, 8192, False, F32, F16),     # fp32 x, long K, 256 groups of 8: one 8 x 8 workgroup
    (7, 2051, 8192, True, F32, F32),      # ragged n on the 8 x 8 route
    (8, 8963, 1536, True, F16, F16),      # fp16 x, short K: pairs, ragged n
    (5, 1536, 8960, False, F16, F32),     # fp16 x, long K: no pairs
    (4, 4864, 896, True, F32, F32),       # fp32 x, m = 3..4: 4 rows per workgroup
    (3, 1537, 2048, False, F32, F16),     # fp32 x, m = 3..4: 4 rows, ragged n
    (2, 1537, 8960, True, F16, F16),      # m = 2: a workgroup per activation row, ragged n
    (2, 4864, 896, False, F32, F32),      # m = 2 pairs, fp32 x
    (2, 40000, 1536, False, F16, F16),    # m = 2, very tall: 8 rows, no pairs
    (6, 2100, 8192, True, F16, F16),      # fp16 x, m = 5..8, long K: the split wide tiles
]


@pytest.mark.parametrize("m,n,k,bias,xdt,ydt", Q8_CASES)
def test_linear_q8(dev, nq, orc, m, n, k, bias, xdt, ydt):
    x, w, b = data(m, n, k, m * 7 + n + k, bias=bias)
    t = nq.quantize_q8(to_dev(w, dev))
    xd = to_dev(x, dev, xdt)
    y = nq.linear_q8(xd, t, None if b is None else to_dev(b, dev), out_dtype=ydt)
    q, s = orc.quantize_q8(w)
    ref = orc.linear_q8(host(xd.float()), q, s, b)
    assert_close_rms(host(y.float()), ref, f"linear_q8 {m}x{n}x{k}", fp16_out=(ydt == F16))


def ref_argmax(v):
    """sampling.cpp:14-20: scan left to right with a strict >; logit 0 NaN -> 0."""
    v = np.asarray(v, np.float32)
    if np.isnan(v[0]):
        return 0
    u = np.where(np.isnan(v), -np.inf, v)
    return int(np.argmax(u))          # numpy: first index of the maximum


def gemv_logits(nq, xd, t, b):
    """fp32 logits of the q8 GEMV, in slices of 8 rows (the GEMV's batch)."""
    return torch.cat([nq.linear_q8(xd[r:r + 8], t, b, out_dtype=F32) for r in range(0, xd.shape[0], 8)])


@pytest.mark.parametrize("m,n,k,bias,xdt", [
    (1, 151936, 1536, False, F16),    # config 5 LM head (8 rows per workgroup)
    (1, 4864, 896, True, F32),
    (2, 151936, 1536, True, F32),
    (3, 8192, 896, False, F16),       # 2 rows per workgroup
    (8, 1000, 512, True, F32),
    (11, 5000, 256, False, F16),      # two slices of 8
    (8, 9000, 1024, True, F32),       # fp32 x: 8 rows per workgroup
    (6, 4864, 896, False, F32),       # fp32 x: 4 rows per workgroup
    (4, 9000, 1024, False, F32),      # fp32 x, m = 3..4: 4 rows per workgroup
    (13, 20000, 512, True, F32),      # a slice of 8 and one of 5, 8 rows per workgroup
    (3, 700, 90, True, F32),          # ragged k: logits in the workspace, then argmax
    (2, 200000, 64, False, F16),      # 25000 partials per row: 13 final workgroups
])
def test_lm_head_argmax(dev, nq, orc, m, n, k, bias, xdt):
    x, w, b = data(m, n, k, m * 13 + n + k, bias=bias)
    t = nq.quantize_q8(to_dev(w, dev))
    xd = to_dev(x, dev, xdt)
    bd = None if b is None else to_dev(b, dev)
    ids = nq.lm_head_argmax(xd, t, bd)
    logits = host(gemv_logits(nq, xd, t, bd))
    assert ids.dtype == torch.int64 and ids.shape == (m,)
    assert host(ids).tolist() == [ref_argmax(r) for r in logits]
    # against the oracle's CPU logits where the top-2 margin dwarfs the 1e-3 RMS tolerance
    q, s = orc.quantize_q8(w)
    ref = orc.linear_q8(host(xd.float()), q, s, b)
    for i in range(m):
        rms = np.sqrt(np.mean(ref[i] ** 2))
        top = np.sort(ref[i])[-2:]
        if top[1] - top[0] > 4e-3 * rms:
            assert int(host(ids)[i]) == int(np.argmax(ref[i])), i
        # every row: the chosen logit is a maximum of the oracle's logits up to
        # twice the 1e-3 RMS logit tolerance (GEMV logit of the id >= the GEMV
        # logit of the oracle's argmax, each within 1e-3 RMS of the oracle)
        assert ref[i][int(host(ids)[i])] >= top[1] - 2e-3 * rms, i


def test_lm_head_argmax_many_inputs(dev, nq, orc):
    """The fused LM head's final reduction combines workgroup keys with
    device-scope atomics across the XCDs: 24 inputs on one vocabulary-sized
    weight, each id equal to the argmax of the GEMV's own logits, and every
    fourth input's ids a maximum of the oracle's logits up to twice the logit
    tolerance."""
    rng = np.random.default_rng(5)
    n, k = 151936, 1536
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    t = nq.quantize_q8(to_dev(w, dev))
    q, s = orc.quantize_q8(w)
    for it in range(24):
        m = 1 + it % 3
        xd = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32), dev, F16 if it % 2 else F32)
        ids = host(nq.lm_head_argmax(xd, t, None)).tolist()
        logits = host(gemv_logits(nq, xd, t, None))
        assert ids == [ref_argmax(r) for r in logits], it
        if it % 4 == 0:
            ref = orc.linear_q8(host(xd.float()), q, s, None)
            for i in range(m):
                assert ref[i][ids[i]] >= ref[i].max() - 2e-3 * np.sqrt(np.mean(ref[i] ** 2)), (it, i)


def test_lm_head_argmax_tie_far_apart(dev, nq):
    """A tie between rows far apart in a 200000-row head (25000 workgroup
    partials, reduced by 13 final workgroups) goes to the first of them."""
    n, k = 200000, 64                                   # 8 rows per workgroup, 25000 partials
    rng = np.random.default_rng(9)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    x = rng.normal(0, 1, (1, k)).astype(np.float32)
    for r in (170001, 199999):
        w[r] = np.sign(x[0]) * 0.05
    t = nq.quantize_q8(to_dev(w, dev))
    xd = to_dev(x, dev, F16)
    got = int(nq.lm_head_argmax(xd, t, None)[0])
    assert got == ref_argmax(host(gemv_logits(nq, xd, t, None))[0]) == 170001


def test_lm_head_argmax_ties_nan_inf(dev, nq):
    """Ties go to the first index (within and across workgroups); a NaN logit 0
    gives 0; other NaN logits are skipped; all -inf gives 0. Each case is also
    checked against the scan over the GEMV's own logits."""
    n, k = 40000, 256                                   # 8 rows per workgroup at m = 1
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    x = rng.normal(0, 1, (1, k)).astype(np.float32)
    top = np.sign(x[0]) * 0.05                          # the largest dot product by far
    for r in (9, 10, 30001):                            # 9 and 10 share a workgroup, 30001 does not
        w[r] = top
    t = nq.quantize_q8(to_dev(w, dev))
    xd = to_dev(x, dev)

    def run(xv, b, expect):
        bd = None if b is None else to_dev(b, dev)
        got = int(nq.lm_head_argmax(xv, t, bd)[0])
        assert got == ref_argmax(host(gemv_logits(nq, xv, t, bd))[0])
        assert got == expect
        return got

    lg = host(gemv_logits(nq, xd, t, None))[0]
    assert lg[9] == lg[10] == lg[30001]                 # identical rows give identical logits
    run(xd, None, 9)
    b = np.zeros(n, np.float32)
    b[9] = np.nan                                       # skipped: 10 is next among the equals
    run(xd, b, 10)
    b[10] = np.nan
    run(xd, b, 30001)                                   # the tie across workgroups
    b[0] = np.nan                                       # logit 0 NaN -> 0
    run(xd, b, 0)
    run(xd, np.full(n, -np.inf, np.float32), 0)         # all -inf -> 0
    xn = xd.clone()
    xn[0, 5] = float("nan")                             # every logit NaN -> 0
    run(xn, None, 0)
    b = np.zeros(n, np.float32)
    b[n - 1] = 1e30                                     # the last row, in the last workgroup
    run(xd, b, n - 1)


def test_linear_q8_golden(dev, nq, golden):
    g = golden("q8_linear")
    for i in range(6):
        t = nq.QTensor(to_dev(g[f"c{i}_q"], dev), to_dev(g[f"c{i}_s"], dev), *g[f"c{i}_q"].shape)
        b = to_dev(g[f"c{i}_b"], dev) if f"c{i}_b" in g.files else None
        y = nq.linear_q8(to_dev(g[f"c{i}_x"], dev), t, b)
        assert_close_rms(host(y), g[f"c{i}_y"], f"golden q8 c{i}")


# ---- group-wise int4 -----------------------------------------------------------------------
Q4_CASES = [
    (1, 1536, 8960, 32, False, F16, F16, F16),   # config 2
    (1, 1536, 8960, 32, False, F16, F16, F32),   # same kernel, fp32 output (bare bound)
    (4, 896, 4864, 32, True, F32, F32, F32),
    (8, 512, 2048, 64, False, F16, F32, F16),
    (3, 40, 32, 8, True, F32, F32, F32),        # group < 32: generic kernel
    (16, 64, 40, 8, False, F32, F32, F32),      # test_quant.cpp:265-280 shapes
    (2, 33, 137, 5, True, F32, F32, F32),       # odd k, odd group
    (9, 7, 40, 16, True, F32, F32, F32),
    (8, 1536, 8960, 32, False, F32, F16, F32),  # fp32 x, m = 5..8: 4 rows, 320-thread bound
    (6, 1001, 4096, 64, True, F32, F32, F16),   # fp32 x, 4 rows, ragged n
    (4, 4864, 896, 128, False, F32, F32, F32),  # fp32 x, m = 3..4: 4 rows
    (7, 300, 12288, 32, True, F32, F16, F32),   # fp32 x, k > 10240: 2 rows, 576 threads
    # short rows (k <= 1024): half chunks in one wave; k % group != 0, ragged n, 4 rows on tall weights
    (1, 301, 992, 64, True, F16, F16, F16),
    (2, 9000, 1024, 256, False, F32, F32, F32),
    (4, 517, 96, 32, True, F32, F16, F16),
    (8, 4864, 896, 128, False, F16, F16, F32),
    (2, 8960, 1536, 32, False, F32, F16, F16),  # fp32 x, m = 2: 4 rows
    (1, 1536, 8960, 32, True, F32, F32, F32),   # fp32 x, m = 1, k >= 4096: 4 rows, unsigned group math
    (1, 1000, 2048, 64, False, F32, F16, F16),  # fp32 x, m = 1, small: 2 rows
    (1, 24600, 1024, 32, True, F32, F16, F32),  # fp32 x, m = 1, tall: 8 rows
    (4, 1100, 12288, 32, True, F32, F16, F32),  # fp32 x, m = 3..4, k > 10240: pairs of 4-row workgroups
    (2, 1030, 14336, 64, False, F32, F32, F16), # fp32 x, m = 2, k > 10240: the same
    (3, 1536, 8960, 32, True, F16, F16, F16),   # m = 3..4: workgroup pairs over activation rows
    (4, 4867, 896, 32, False, F16, F32, F32),   # pairs, ragged n
    (3, 2048, 1536, 64, True, F32, F32, F16),   # fp32 x pairs, 4 rows, 320-thread bound
    (5, 8960, 1536, 32, True, F16, F16, F16),   # m = 5..8 fp16 short K: pairs, 1 row in the second
    (8, 1027, 2048, 32, False, F32, F16, F32),  # m = 5..8 fp32 pairs, ragged n
    (7, 1536, 8960, 32, True, F16, F16, F32),   # fp16 long K: no pairs
    (2, 1539, 8960, 32, True, F32, F16, F16),   # m = 2 fp32 long K: pairs, ragged n
    # one fp16 row, 5120 <= k <= 9216: half a chunk per lane
    (1, 1537, 8960, 32, True, F16, F16, F32),   # ragged n: the last workgroup has one row
    (1, 7, 5120, 64, False, F16, F32, F16),     # group 64, fewer rows than a workgroup pair
    (1, 999, 9216, 128, True, F16, F16, F16),   # 576 threads, group 128
    (1, 640, 7168, 96, False, F16, F32, F32),   # group 96, k % group = 64: a short last group
    (3, 500, 1568, 64, True, F32, F32, F32),    # k % group = 32: scale rows of ceil(k / group)
    # fp16 x at m = 5..8 on n, k >= 4096: the split wide tiles (workspace) instead of the GEMV
    (8, 4100, 4096, 64, True, F16, F32, F16),   # ragged n, fp32 scales, group 64
    (5, 4096, 4224, 32, False, F16, F16, F32),  # 33 slabs of 128 codes
]


@pytest.mark.parametrize("m,n,k,g,bias,xdt,sdt,ydt", Q4_CASES)
def test_linear_q4g(dev, nq, orc, m, n, k, g, bias, xdt, sdt, ydt):
    x, w, b = data(m, n, k, m * 13 + n + k + g, bias=bias)
    t = nq.quantize_q4g(to_dev(w, dev), g, scale_dtype=sdt)
    xd = to_dev(x, dev, xdt)
    y = nq.linear_q4g(xd, t, None if b is None else to_dev(b, dev), out_dtype=ydt)
    q = host(t.q)
    s = host(t.scale.float())                  # the scales the kernel used (fp16-rounded if fp16)
    ref = orc.linear_q4g(host(xd.float()), q, s, g, b)
    assert_close_rms(host(y.float()), ref, f"linear_q4g {m}x{n}x{k} g{g}", fp16_out=(ydt == F16))


WQ_GEMM_CASES = [  # m > 8: the fp16 MFMA GEMM (m >= 16 or n >= 4096) or GEMV slices
    ("q8", 9, 896, 896, 0, True, F16, F16, F16),       # k <= 1024: the GEMM
    ("q8", 9, 896, 4864, 0, True, F16, F16, F16),      # narrow, long rows: GEMV slices 8 + 1
    ("q4g", 13, 1600, 2048, 32, False, F32, F32, F16),  # m = 9..15 from 1536 rows: the GEMM
    ("q8", 9, 4608, 896, 0, True, F16, F16, F16),      # GEMM, tall weight
    ("q4g", 12, 4104, 512, 32, False, F32, F16, F32),  # GEMM, ragged last tile
    ("q8", 64, 4864, 896, 0, False, F32, F32, F32),    # fp32 x: exact three-part bf16 split
    ("q8", 300, 1536, 1536, 0, True, F16, F32, F16),   # several 64-row blocks
    ("q8", 33, 8960, 1536, 0, False, F16, F32, F16),   # 32 rows per workgroup
    ("q4g", 16, 1536, 8960, 32, False, F16, F16, F16),
    ("q4g", 40, 8960, 1536, 32, True, F32, F32, F32),
    ("q4g", 64, 896, 4864, 64, False, F16, F32, F16),  # group 64
    ("q4g", 130, 512, 2048, 128, True, F16, F16, F32),
    ("q4g", 20, 256, 1536, 96, False, F16, F32, F16),  # group 96 (3 chunks): GEMV slices
    # m > 64, fp16 x, k % 128 == 0: the wide-tile kernel (LDS-DMA ring)
    ("q4g", 300, 1536, 1536, 32, True, F16, F16, F16),
    ("q4g", 200, 2000, 1024, 64, False, F16, F16, F32),  # fp32 y: direct stores
    ("q4g", 130, 1000, 2048, 128, True, F16, F32, F16),  # fp32 scales, one group per slab
    ("q4g", 96, 700, 1536, 256, False, F16, F32, F16),   # a group spans two slabs
    ("q4g", 16, 1536, 1568, 64, False, F16, F16, F16),   # k % group = 32: a short last group
    ("q4g", 130, 1000, 1664, 256, True, F16, F32, F16),  # wide kernel, k % group = 128
    ("q4g", 64, 1536, 4224, 256, False, F16, F16, F16),  # wide split K over the workspace, k % group = 128
    ("q4g", 16, 1536, 4128, 64, True, F16, F32, F16),    # 16-row split K, k % group = 32
    ("q8", 12, 1536, 4224, 0, False, F16, F16, F16),     # m = 9..15, wide split K
    ("q8", 257, 2900, 1024, 0, True, F16, F32, F32),
    ("q4g", 1100, 640, 512, 32, True, F16, F16, F16),
    ("q4g", 40, 8960, 1536, 64, True, F16, F16, F16),    # m >= 32 with >= 128 tiles
    # fp32 x on the wide tiles: three exact bf16 parts, 64-column slabs
    ("q8", 300, 1536, 1536, 0, True, F32, F32, F32),
    ("q4g", 200, 2000, 1024, 32, False, F32, F16, F16),
    ("q4g", 130, 9000, 512, 32, True, F32, F32, F32),
    # m > 128 with few unsplit tiles: the split wide tiles (64 x 128, K ranges)
    ("q8", 200, 1536, 8960, 0, True, F16, F32, F16),
    ("q4g", 300, 1000, 8192, 64, False, F16, F16, F16),  # ragged n, k >= 8192 rule
    ("q8", 160, 896, 4864, 0, False, F32, F32, F32),     # fp32 x, 64-column slabs
    ("q4g", 520, 896, 4864, 32, True, F16, F16, F32),
    ("q8", 100, 17000, 2048, 0, False, F16, F32, F16),   # m > 64 with >= 256 split tiles: unsplit wide
]


def _wq_random_cases():
    """Seeded shapes over the weight-only wide-tile plans (m >= 32, fp16 x,
    k % 128 == 0): every tile shape, fp16 / fp32 scales, group 32..256."""
    rng = np.random.default_rng(77)
    cases = []
    for i in range(14):
        mode = "q8" if i % 3 == 0 else "q4g"
        m = int(rng.integers(32, 1600))
        n = int(rng.integers(64, 12000))
        k = 128 * int(rng.integers(1, 24))
        if m * n * k > 4e9:
            n = max(64, int(4e9 / (m * k)))
        sdt = F16 if i % 2 else F32
        g = int(rng.choice([32, 64])) if sdt == F16 else int(rng.choice([32, 64, 128, 256]))
        while k % g:
            g //= 2
        cases.append((mode, m, n, k, g, bool(i % 4 == 1), sdt, F16 if i % 5 else F32, F32 if i % 3 == 1 else F16))
    return cases


def _dequant_q4g(t, g):
    q = t.q.to(torch.int32)
    codes = torch.stack([q & 15, q >> 4], dim=-1).reshape(t.out, -1)[:, :t.in_] - 8
    return codes.float() * t.scale.float().repeat_interleave(g, dim=1)[:, :t.in_]


@pytest.mark.parametrize("mode,m,n,k,g,bias,sdt,ydt,xdt", _wq_random_cases())
def test_weight_only_random_shapes(dev, nq, mode, m, n, k, g, bias, sdt, ydt, xdt):
    """Weight-only linears on fp16 or fp32 activations against a torch fp32 reference
    on the dequantized weight (the reference's own test_quant.cpp:100-116
    invariant linear(x, dequant(w)))."""
    gen = torch.Generator(device=dev).manual_seed(m * 7 + n * 3 + k)
    x = torch.randn((m, k), generator=gen, device=dev).to(xdt)
    w = torch.randn((n, k), generator=gen, device=dev) * 0.05
    b = torch.randn(n, generator=gen, device=dev) if bias else None
    if mode == "q8":
        t = nq.quantize_q8(w)
        deq = t.q.float() * t.scale[:, None]
        y = nq.linear_q8(x, t, b, out_dtype=ydt)
    else:
        t = nq.quantize_q4g(w, g, scale_dtype=sdt)
        deq = _dequant_q4g(t, g)
        y = nq.linear_q4g(x, t, b, out_dtype=ydt)
    ref = x.float() @ deq.t() + (b if b is not None else 0.0)
    assert_close_rms(host(y.float()), host(ref), f"{mode} {m}x{n}x{k} g{g}", fp16_out=(ydt == F16))


@pytest.mark.parametrize("mode,m,n,k,g,bias,xdt,sdt,ydt", WQ_GEMM_CASES)
def test_weight_only_gemm_batched(dev, nq, orc, mode, m, n, k, g, bias, xdt, sdt, ydt):
    x, w, b = data(m, n, k, m * 31 + n + k + g, bias=bias)
    xd = to_dev(x, dev, xdt)
    bd = None if b is None else to_dev(b, dev)
    xo = host(xd.float())
    if mode == "q8":
        t = nq.quantize_q8(to_dev(w, dev))
        y = nq.linear_q8(xd, t, bd, out_dtype=ydt)
        q, s = orc.quantize_q8(w)
        ref = orc.linear_q8(xo, q, s, b)
    else:
        t = nq.quantize_q4g(to_dev(w, dev), g, scale_dtype=sdt)
        y = nq.linear_q4g(xd, t, bd, out_dtype=ydt)
        ref = orc.linear_q4g(xo, host(t.q), host(t.scale.float()), g, b)
    assert_close_rms(host(y.float()), ref, f"{mode} gemm {m}x{n}x{k}", fp16_out=(ydt == F16))


# 256 x 288 Q8 tiles (one round at m ~ 2048, n in (8192, 9216]) run as 2 x 6
# waves of 128 x 48; ragged m and n, with and without bias, sampled rows against
# the oracle and the whole output against the 16-row kernel's (fp32 y).
@pytest.mark.parametrize("m,n,k,bias", [(1900, 8800, 512, True), (2048, 8960, 256, False)])
def test_weight_only_q8_wide_2x6(dev, nq, orc, m, n, k, bias):
    x, w, b = data(m, n, k, m + n + k, bias=bias)
    xd = to_dev(x, dev, F16)
    bd = None if b is None else to_dev(b, dev)
    t = nq.quantize_q8(to_dev(w, dev))
    y = nq.linear_q8(xd, t, bd, out_dtype=F32)
    rows = np.random.default_rng(m).choice(m, 16, replace=False)
    q, s = orc.quantize_q8(w)
    ref = orc.linear_q8(host(xd.float())[rows], q, s, b)
    assert_close_rms(host(y)[rows], ref, f"q8 wide 2x6 {m}x{n}x{k}")
    y16 = torch.cat([nq.linear_q8(xd[i:i + 64], t, bd, out_dtype=F32) for i in range(0, 128, 64)])
    assert_close_rms(host(y[:128]), host(y16), f"q8 wide 2x6 vs 16-row kernel {m}x{n}x{k}")


# Split K over a workspace (nq_linear_q8_ws / nq_linear_q4g_ws, which the
# Python linears call): weights with few rows at batched m run K in ranges whose
# fp32 planes a reduce kernel sums in order. 16-row kernel splits (fp32 x below
# m = 32, or short K with a tiny grid), wide 64-row tile splits with the
# two-slot ring (16 <= m <= 128, k >= 4096; fp32 x takes 64-column slabs),
# ragged m and n (n % 4 != 0: the scalar reduce), fp16 / fp32 scales, groups 32,
# 64 and 128. Against the oracle, and against the unsplit entry point on the
# same inputs.
WQ_SPLIT_CASES = [
    ("q8", 16, 896, 4864, 0, False, F16, F32, F16),
    ("q4g", 24, 1536, 8960, 32, True, F32, F16, F32),
    ("q8", 48, 896, 4864, 0, True, F32, F32, F16),
    ("q4g", 64, 1536, 8960, 32, False, F16, F16, F32),
    ("q4g", 100, 896, 4864, 128, True, F16, F32, F16),
    ("q8", 128, 2048, 8192, 0, False, F16, F32, F32),
    ("q8", 40, 256, 1536, 0, True, F32, F32, F32),
    ("q4g", 72, 202, 1536, 64, False, F16, F16, F16),
    ("q8", 97, 1001, 4096, 0, True, F16, F32, F16),
    ("q4g", 32, 1000, 4096, 64, False, F16, F16, F32),
    ("q4g", 17, 4100, 4224, 32, True, F16, F32, F16),
    ("q8", 12, 1536, 8960, 0, True, F16, F32, F16),     # m = 9..15 with a workspace
    ("q4g", 9, 2000, 4096, 32, False, F16, F16, F32),
]


@pytest.mark.parametrize("mode,m,n,k,g,bias,xdt,sdt,ydt", WQ_SPLIT_CASES)
def test_weight_only_split_k(dev, nq, orc, mode, m, n, k, g, bias, xdt, sdt, ydt):
    from nanoinfer_amd import _lib
    lib = _lib.load()
    nbytes = lib.nq_linear_wq_workspace_size(m, n, k)
    assert nbytes > 0, "shape must plan a split"
    x, w, b = data(m, n, k, m * 13 + n + k, bias=bias)
    xd = to_dev(x, dev, xdt)
    bd = None if b is None else to_dev(b, dev)
    xo = host(xd.float())
    y0 = torch.empty((m, n), dtype=ydt, device=dev)
    xc, yc = (1 if xdt == F16 else 0), (1 if ydt == F16 else 0)
    s = torch.cuda.current_stream().cuda_stream
    P = lambda t: None if t is None else t.data_ptr()
    if mode == "q8":
        t = nq.quantize_q8(to_dev(w, dev))
        y = nq.linear_q8(xd, t, bd, out_dtype=ydt)
        _lib.check(lib.nq_linear_q8(P(xd), xc, P(t.q), P(t.scale), P(bd), P(y0), yc, m, n, k, s))
        q, sc = orc.quantize_q8(w)
        ref = orc.linear_q8(xo, q, sc, b)
    else:
        t = nq.quantize_q4g(to_dev(w, dev), g, scale_dtype=sdt)
        y = nq.linear_q4g(xd, t, bd, out_dtype=ydt)
        _lib.check(lib.nq_linear_q4g(P(xd), xc, P(t.q), P(t.scale), 0 if sdt == F32 else 1, g, P(bd), P(y0),
                                     yc, m, n, k, s))
        ref = orc.linear_q4g(xo, host(t.q), host(t.scale.float()), g, b)
    assert_close_rms(host(y.float()), ref, f"{mode} split {m}x{n}x{k}", fp16_out=(ydt == F16))
    assert_close_rms(host(y.float()), host(y0.float()), f"{mode} split vs whole {m}x{n}x{k}", fp16_out=(ydt == F16))


def _split_random_cases():
    rng = np.random.default_rng(11)
    cases = []
    for i in range(14):
        mode = "q8" if i % 2 else "q4g"
        m = int(rng.integers(9, 129))
        n = int(rng.integers(64, 3000))
        k = 128 * int(rng.integers(32, 80))          # k >= 4096: the split routes
        sdt = F16 if i % 3 else F32
        g = 32 if sdt == F16 or i % 4 else 128
        xdt = F32 if i % 5 == 0 else F16
        cases.append((mode, m, n, k, g, bool(i % 3 == 1), xdt, sdt, F16 if i % 2 else F32))
    return cases


@pytest.mark.parametrize("mode,m,n,k,g,bias,xdt,sdt,ydt", _split_random_cases())
def test_weight_only_split_random_shapes(dev, nq, mode, m, n, k, g, bias, xdt, sdt, ydt):
    """Random batched shapes with long K through the workspace entries (split
    wide tiles, split 16-row kernel or unsplit, as planned) against a torch fp32
    reference on the dequantized weight."""
    gen = torch.Generator(device=dev).manual_seed(m * 7 + n * 3 + k)
    x = torch.randn((m, k), generator=gen, device=dev).to(xdt)
    w = torch.randn((n, k), generator=gen, device=dev) * 0.05
    b = torch.randn(n, generator=gen, device=dev) if bias else None
    if mode == "q8":
        t = nq.quantize_q8(w)
        deq = t.q.float() * t.scale[:, None]
        y = nq.linear_q8(x, t, b, out_dtype=ydt)
    else:
        t = nq.quantize_q4g(w, g, scale_dtype=sdt)
        deq = _dequant_q4g(t, g)
        y = nq.linear_q4g(x, t, b, out_dtype=ydt)
    ref = x.float() @ deq.t() + (b if b is not None else 0.0)
    assert_close_rms(host(y.float()), host(ref), f"{mode} split random {m}x{n}x{k} g{g}", fp16_out=(ydt == F16))


# fp32 activations far outside fp16's range and deep in its subnormals, on both
# weight-only MFMA kernels (16-row tiles: k % 128 != 0 or small m; wide tiles:
# m > 128, k % 128 == 0): the exact bf16 split keeps every row at the accuracy of
# an fp32 dot product, so each row is held to 1e-5 of its own RMS.
@pytest.mark.parametrize("mode,m,n,k,g", [("q8", 24, 4864, 896, 0), ("q4g", 40, 1536, 960, 32),
                                          ("q8", 300, 1536, 1536, 0), ("q4g", 200, 2000, 1024, 32)])
def test_weight_only_fp32_x_extreme_range(dev, nq, orc, mode, m, n, k, g):
    rng = np.random.default_rng(m + n + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    x[0::4] *= 1e5            # |x| up to ~5e5 > 65504
    x[1::4] *= 1e-6           # fp16 subnormal range
    x[2::4, 7] = 3e5          # one large outlier among ordinary values
    x[3::4] *= np.float32(2.0 ** -100)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    xd = to_dev(x, dev)
    if mode == "q8":
        t = nq.quantize_q8(to_dev(w, dev))
        y = host(nq.linear_q8(xd, t, out_dtype=F32))
        q, s = orc.quantize_q8(w)
        ref = orc.linear_q8(x, q, s)
    else:
        t = nq.quantize_q4g(to_dev(w, dev), g)
        y = host(nq.linear_q4g(xd, t, out_dtype=F32))
        ref = orc.linear_q4g(x, host(t.q), host(t.scale), g)
    assert np.isfinite(y).all()
    for r in range(m):
        rr = rms(ref[r])
        err = np.abs(y[r].astype(np.float64) - ref[r]).max()
        assert err <= 1e-5 * rr, (mode, r, err, rr)


def test_linear_q4g_golden(dev, nq, golden):
    gd = golden("q4g")
    for i in range(6):
        q, s, g = gd[f"lin{i}_q"], gd[f"lin{i}_s"], int(gd[f"lin{i}_g"])
        k = gd[f"lin{i}_x"].shape[1]
        t = nq.Q4GTensor(to_dev(q, dev), to_dev(s, dev), q.shape[0], k, g)
        b = to_dev(gd[f"lin{i}_b"], dev) if f"lin{i}_b" in gd.files else None
        y = nq.linear_q4g(to_dev(gd[f"lin{i}_x"], dev), t, b)
        assert_close_rms(host(y), gd[f"lin{i}_y"], f"golden q4g lin{i}")


def test_linear_q4_per_row(dev, nq, golden):
    gd = golden("q4g")
    for m in (3, 16):
        q, s = gd[f"q4lin{m}_q"], gd[f"q4lin{m}_s"]
        t = nq.Q4GTensor(to_dev(q, dev), to_dev(s, dev), q.shape[0], 40, 40)
        y = nq.linear_q4(to_dev(gd[f"q4lin{m}_x"], dev), t, to_dev(gd[f"q4lin{m}_b"], dev))
        assert_close_rms(host(y), gd[f"q4lin{m}_y"], f"golden q4 m={m}")


# ---- W8A8 -----------------------------------------------------------------------------------
W8A8_SHAPES = [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960)]  # q/o, k/v, gate/up, down


@pytest.mark.parametrize("m", [1, 8, 16, 32, 64])
@pytest.mark.parametrize("n,k", W8A8_SHAPES)
def test_w8a8_acc_exact_all_paths(dev, nq, orc, m, n, k):
    rng = np.random.default_rng(m + n + k)
    xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
    xq[0, :] = 127
    wq[0, :] = 127                              # largest positive int32 sum
    ref = orc.w8a8_acc(xq, wq)
    xd, wd = to_dev(xq, dev), to_dev(wq, dev)
    for path in (nq._lib.NQ_PATH_GEMV, nq._lib.NQ_PATH_MFMA, nq._lib.NQ_PATH_AUTO):
        acc = host(nq.w8a8_acc_i32(xd, wd, path))
        assert np.array_equal(acc, ref), (m, n, k, path)


def test_w8a8_acc_generic_and_ragged(dev, nq, orc):
    rng = np.random.default_rng(3)
    for m, n, k in [(3, 70, 90), (20, 33, 100), (130, 65, 48), (1, 1, 0)]:
        xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
        wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
        ref = orc.w8a8_acc(xq, wq)
        for path in (nq._lib.NQ_PATH_GENERIC, nq._lib.NQ_PATH_AUTO, nq._lib.NQ_PATH_MFMA):
            assert np.array_equal(host(nq.w8a8_acc_i32(to_dev(xq, dev), to_dev(wq, dev), path)), ref), (m, n, k, path)


@pytest.mark.parametrize("m", [1, 8, 16, 64])
@pytest.mark.parametrize("n,k", W8A8_SHAPES)
def test_linear_w8a8_sweep(dev, nq, orc, m, n, k):
    x, w, _ = data(m, n, k, 100 + m + n + k)
    t = nq.quantize_q8(to_dev(w, dev))
    xd = to_dev(x, dev, F16)
    xo = host(xd.float())
    q, s = orc.quantize_q8(w)
    ref = orc.linear_w8a8(xo, q, s)
    y32 = nq.linear_w8a8(xd, t, out_dtype=F32)
    assert_close_rms(host(y32), ref, f"w8a8 {m}x{n}x{k} fp32-out")
    y16 = nq.linear_w8a8(xd, t, out_dtype=F16)
    assert_close_rms(host(y16.float()), ref, f"w8a8 {m}x{n}x{k} fp16-out", fp16_out=True)
    # the fp16 store is the only difference between the two outputs
    assert same_bits(host(y16), host(y32).astype(np.float16))


@pytest.mark.parametrize("m,n,k,bias", [(1, 896, 896, True), (8, 4864, 896, False), (16, 896, 4864, False),
                                        (5, 1536, 1536, True)])
def test_w8a8_gemv_equals_mfma_bitwise(dev, nq, m, n, k, bias):
    x, w, b = data(m, n, k, m + n, wsig=0.5, bias=bias)       # test_cuda.cpp:217-251, :425-427
    t = nq.quantize_q8(to_dev(w, dev))
    bd = None if b is None else to_dev(b, dev)
    xd = to_dev(x, dev)
    yg = host(nq.linear_w8a8(xd, t, bd, path=nq._lib.NQ_PATH_GEMV))
    ym = host(nq.linear_w8a8(xd, t, bd, path=nq._lib.NQ_PATH_MFMA))
    assert same_bits(yg, ym)


@pytest.mark.parametrize("m,n,k,bias", [(128, 896, 896, True), (128, 4864, 896, False), (100, 896, 4864, False),
                                        (1, 896, 896, True), (16, 896, 4864, False)])
def test_w8a8_reference_shapes(dev, nq, orc, m, n, k, bias):
    rng = np.random.default_rng(1234 + m)                      # test_cuda.cpp:418-423, uniform(-1,1)
    x = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    w = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32) if bias else None
    t = nq.quantize_q8(to_dev(w, dev))
    y = host(nq.linear_w8a8(to_dev(x, dev), t, None if b is None else to_dev(b, dev)))
    q, s = orc.quantize_q8(w)
    ref = orc.linear_w8a8(x, q, s, b)
    assert np.abs(y - ref).max() < 2e-3                        # the reference GPU tolerance
    assert_close_rms(y, ref, "w8a8 ref shape")


def test_w8a8_golden(dev, nq, golden):
    g = golden("w8a8")
    for i in range(6):
        t = nq.QTensor(to_dev(g[f"c{i}_q"], dev), to_dev(g[f"c{i}_s"], dev), *g[f"c{i}_q"].shape)
        b = to_dev(g[f"c{i}_b"], dev) if f"c{i}_b" in g.files else None
        y = host(nq.linear_w8a8(to_dev(g[f"c{i}_x"], dev), t, b))
        ref = g[f"c{i}_y"]
        ok = ~np.isnan(ref)
        assert_close_rms(y[ok], ref[ok], f"golden w8a8 c{i}")


def test_w8a8_prefill_config5(dev, nq, orc):
    """M=2048, K=1536, N=8960: the MFMA accumulators equal the independent
    GEMV kernel's everywhere, and the oracle's on sampled rows."""
    m, n, k = 2048, 8960, 1536
    rng = np.random.default_rng(5)
    xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
    xd, wd = to_dev(xq, dev), to_dev(wq, dev)
    acc_m = nq.w8a8_acc_i32(xd, wd, nq._lib.NQ_PATH_MFMA)
    acc_g = nq.w8a8_acc_i32(xd, wd, nq._lib.NQ_PATH_GEMV)
    assert torch.equal(acc_m, acc_g)
    rows = rng.choice(m, 24, replace=False)
    assert np.array_equal(host(acc_m)[rows], orc.w8a8_acc(xq[rows], wq))


@pytest.mark.parametrize("m", [9, 24, 40, 57])
@pytest.mark.parametrize("n,k", [(1536, 1536), (8960, 1536), (1536, 8960), (100, 272)])
def test_w8a8_skinny_ragged_m(dev, nq, orc, m, n, k):
    x, w, b = data(m, n, k, 7 * m + n + k, bias=True)
    t = nq.quantize_q8(to_dev(w, dev))
    y = host(nq.linear_w8a8(to_dev(x, dev), t, to_dev(b, dev)))
    q, s = orc.quantize_q8(w)
    assert_close_rms(y, orc.linear_w8a8(x, q, s, b), f"w8a8 skinny {m}x{n}x{k}")


def test_w8a8_workspace_reuse_and_gemm_entry(dev, nq, orc):
    """Split-K counters re-arm between calls sharing one workspace; the
    pre-quantized entry (nq_gemm_w8a8) gives the same bits as the linear."""
    import ctypes  # noqa: F401
    from nanoinfer_amd import _lib
    lib = _lib.load()
    m, n, k = 32, 1536, 8960
    rng = np.random.default_rng(77)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    t = nq.quantize_q8(to_dev(w, dev))
    q, s = orc.quantize_q8(w)
    ws = torch.empty(lib.nq_linear_w8a8_workspace_size(m, n, k), dtype=torch.uint8, device=dev)
    ws.fill_(0xAB)                                     # garbage: the call must not depend on it
    for it in range(3):
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        xd = to_dev(x, dev)
        y = torch.empty((m, n), dtype=torch.float32, device=dev)
        _lib.check(lib.nq_linear_w8a8(xd.data_ptr(), 0, t.q.data_ptr(), t.scale.data_ptr(), None, y.data_ptr(), 0,
                                      m, n, k, ws.data_ptr(), ws.numel(), 0, torch.cuda.current_stream().cuda_stream))
        assert_close_rms(host(y), orc.linear_w8a8(x, q, s), f"reuse {it}")
        xq, a_s = nq.act_quant(xd)
        y2 = nq.gemm_w8a8(xq, a_s, t, out_dtype=torch.float32)
        assert same_bits(host(y2), host(y))


@pytest.mark.parametrize("m,n,k", [(32, 1536, 8960), (200, 1003, 4096), (16, 1536, 8960)])
def test_w8a8_split_workspace_too_small(dev, nq, m, n, k):
    """Plans with K ranges need their partial planes: one byte short of the
    reported size is NQ_BAD_ARG, before anything is launched."""
    from nanoinfer_amd import _lib
    lib = _lib.load()
    need = lib.nq_gemm_w8a8_workspace_size(m, n, k)
    assert need > 0
    xq = torch.zeros((m, k), dtype=torch.int8, device=dev)
    a_s = torch.ones(m, device=dev)
    wq = torch.zeros((n, k), dtype=torch.int8, device=dev)
    w_s = torch.ones(n, device=dev)
    y = torch.empty((m, n), dtype=torch.float16, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    st = lib.nq_gemm_w8a8(xq.data_ptr(), a_s.data_ptr(), wq.data_ptr(), w_s.data_ptr(), None, y.data_ptr(), 1,
                          m, n, k, ws.data_ptr(), need - 256, 0, torch.cuda.current_stream().cuda_stream)
    assert st == _lib.NQ_BAD_ARG, st


@pytest.mark.parametrize("m,n,k", [(512, 256, 1536), (512, 1536, 1536), (512, 1536, 8960), (300, 1000, 960),
                                   (2048, 8960, 1536), (200, 1003, 192), (77, 517, 1024), (129, 36, 2048),
                                   # wide-tile plans: 256 x 256 / 288 / 320 tiles, ragged m and n, n % 8 != 0
                                   (1800, 6000, 192), (1900, 7996, 128), (2048, 10000, 64), (1700, 8191, 64),
                                   (1537, 9000, 64),
                                   # 128-row wide tiles (m = 512 class), ragged m and n, n odd
                                   (512, 17920, 192), (400, 15000, 64), (450, 16001, 64),
                                   # config 4 gate|up at its real k (12 slabs through the 3-slot ring),
                                   # and ragged m and n on the same plan
                                   (512, 17920, 1536), (500, 17917, 1536),
                                   # k % 64 != 0: the skinny kernel over 64-row blocks in one launch,
                                   # with split K and its partial planes for the long k
                                   (200, 1000, 528), (130, 512, 6160),
                                   # long K, fewer than 128 tiles: 64 x 64 wide tiles with K in 5 / 4 / 4 / 6
                                   # ranges (k % 128 == 64 puts the half slab in the last range; ragged m, n)
                                   (128, 1536, 8960), (200, 896, 4864), (256, 1000, 4160), (100, 700, 4096),
                                   # 128 tiles on K >= 8192: two ranges (half slab at the end)
                                   (100, 4096, 8256)])
def test_w8a8_prefill_plans_exact(dev, nq, orc, m, n, k):
    """Every prefill plan (wide 256 x 256..320 tiles, 256x128 / 128x128 tiles,
    split K with int32 partial planes) gives the GEMV path's accumulators bit for bit, and the linear's
    fp16 output equals the GEMM entry's and the oracle's within tolerance."""
    rng = np.random.default_rng(m + n + k)
    xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
    xd, wd = to_dev(xq, dev), to_dev(wq, dev)
    acc_m = nq.w8a8_acc_i32(xd, wd, nq._lib.NQ_PATH_MFMA)
    acc_g = nq.w8a8_acc_i32(xd, wd, nq._lib.NQ_PATH_GEMV)
    assert torch.equal(acc_m, acc_g)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    b = rng.normal(0, 0.1, n).astype(np.float32)
    t = nq.quantize_q8(to_dev(w, dev))
    xdv = to_dev(x, dev).half()
    for _ in range(2):                                   # the split accumulator re-arms between calls
        y = nq.linear_w8a8(xdv, t, to_dev(b, dev))
        xq2, a_s = nq.act_quant(xdv)
        y2 = nq.gemm_w8a8(xq2, a_s, t, to_dev(b, dev), out_dtype=torch.float16)
        assert torch.equal(y, y2)
    rows = rng.choice(m, 16, replace=False)
    q, s = orc.quantize_q8(w)
    ref = orc.linear_w8a8(host(xdv.float())[rows], q, s, b)
    assert_close_rms(host(y.float())[rows], ref, f"w8a8 prefill {m}x{n}x{k}", fp16_out=True)
    y32 = nq.linear_w8a8(xdv, t, to_dev(b, dev), out_dtype=torch.float32)   # fp32 epilogue path
    assert_close_rms(host(y32)[rows], ref, f"w8a8 prefill fp32-out {m}x{n}x{k}")


def _small_m_shapes():
    """Seeded decode-batch shapes (m <= 64) over the skinny kernel, the 64-row
    wide tiles (tall weights) and their K ranges (long K), k % 128 == 64 tails."""
    rng = np.random.default_rng(4242)
    shapes = []
    for _ in range(14):
        m = int(rng.integers(3, 65))
        n = int(rng.choice([int(rng.integers(16, 3000)), int(rng.integers(4096, 20000))]))
        k = int(rng.choice([64, 192, 1536, 1600, 4160, 6080, 8960]))
        if m * n * k > 3e9:
            n = max(16, int(3e9 / (m * k)))
        shapes.append((m, n, k))
    return shapes


@pytest.mark.parametrize("m,n,k", _small_m_shapes())
def test_w8a8_small_m_random_shapes(dev, nq, m, n, k):
    """int32 accumulators of the m <= 64 MFMA plans equal the GEMV path's bit for bit."""
    g = torch.Generator(device=dev).manual_seed(m * 17 + n * 5 + k)
    xq = torch.randint(-127, 128, (m, k), generator=g, device=dev, dtype=torch.int8)
    wq = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
    acc_m = nq.w8a8_acc_i32(xq, wq, nq._lib.NQ_PATH_MFMA)
    acc_g = nq.w8a8_acc_i32(xq, wq, nq._lib.NQ_PATH_GEMV)
    assert torch.equal(acc_m, acc_g), (m, n, k)


def _plan_shapes():
    """Seeded shapes spread over the W8A8 plans for m > 64: wide tiles in one
    or more rounds, 128x128 and 64x128 prefill tiles, split K, and k % 64 != 0
    (the skinny kernel over 64-row blocks); wide shapes whose last 128-byte
    K slab is half empty."""
    rng = np.random.default_rng(2026)
    shapes = [(2304, 16384, 128), (2048, 8200, 128), (200, 1003, 4096), (96, 5000, 6144)]   # 2 rounds, wide, split
    shapes += [(2048, 8200, 192), (512, 17000, 320), (1900, 8900, 64), (200, 1003, 4160)]   # last 128-byte slab half empty
    for _ in range(12):
        m = int(rng.integers(65, 2300))
        n = int(rng.integers(16, 20000))
        k = int(rng.choice([64, 128, 192, 320, 1536, 2560, 4096, 48, 208]))
        if m * n * k > 6e9:
            n = max(16, int(6e9 / (m * k)))
        shapes.append((m, n, k))
    return shapes


# One shape per wide-kernel tile (rows x cols): 64x32, 64x64, 64x96, 64x128, 128x64,
# 128x128, 128x256, 128x320, 256x128, 256x256, 256x320 (256x288 and 128x288 are
# the config shapes above), each with a half-empty last 128-byte K slab or not.
WIDE_TILE_SHAPES = [(512, 2048, 1536), (1024, 1536, 1536), (1088, 1920, 320), (1024, 2048, 192),
                    (1000, 4000, 448), (512, 16384, 320), (512, 20480, 192), (1024, 8192, 448),
                    (2048, 8192, 256), (2048, 10240, 192), (4096, 8960, 192), (3000, 5000, 320),
                    # m <= 64 with a tall weight: 64 x 32..128 tiles, rows past m read as zeros
                    (16, 8960, 1536), (64, 17920, 1536), (8, 8960, 192), (33, 4100, 320), (64, 16384, 1600),
                    # ... and long K in ranges (partial planes + reduction)
                    (32, 1536, 8960), (64, 1536, 8960), (40, 3000, 6080)]


@pytest.mark.parametrize("m,n,k", WIDE_TILE_SHAPES)
def test_w8a8_wide_tiles(dev, nq, m, n, k):
    """Every wide tile: int32 accumulators and the fp32 / fp16 epilogue with
    bias equal the GEMV path bit for bit."""
    g = torch.Generator(device=dev).manual_seed(m + 3 * n + 7 * k)
    xq = torch.randint(-127, 128, (m, k), generator=g, device=dev, dtype=torch.int8)
    wq = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
    assert torch.equal(nq.w8a8_acc_i32(xq, wq, nq._lib.NQ_PATH_MFMA), nq.w8a8_acc_i32(xq, wq, nq._lib.NQ_PATH_GEMV))
    x = torch.randn((m, k), generator=g, device=dev)
    w = torch.randn((n, k), generator=g, device=dev) * 0.05
    b = torch.randn(n, generator=g, device=dev)
    t = nq.quantize_q8(w)
    yg = nq.linear_w8a8(x, t, b, path=nq._lib.NQ_PATH_GEMV, out_dtype=F32)
    ym = nq.linear_w8a8(x, t, b, path=nq._lib.NQ_PATH_MFMA, out_dtype=F32)
    assert torch.equal(ym, yg), (m, n, k)
    y16 = nq.linear_w8a8(x, t, b, path=nq._lib.NQ_PATH_MFMA, out_dtype=F16)
    assert torch.equal(y16, ym.half()), (m, n, k)


@pytest.mark.parametrize("m,n,k", _plan_shapes())
def test_w8a8_plans_random_shapes(dev, nq, m, n, k):
    """int32 accumulators of the MFMA plans equal the GEMV path's bit for bit."""
    g = torch.Generator(device=dev).manual_seed(m * 131 + n * 7 + k)
    xq = torch.randint(-127, 128, (m, k), generator=g, device=dev, dtype=torch.int8)
    wq = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
    acc_m = nq.w8a8_acc_i32(xq, wq, nq._lib.NQ_PATH_MFMA)
    acc_g = nq.w8a8_acc_i32(xq, wq, nq._lib.NQ_PATH_GEMV)
    assert torch.equal(acc_m, acc_g), (m, n, k)


# The decode-batch routes of nq_linear_w8a8 (AUTO, m <= 64): the act quant fused
# into the decode kernel (m <= 8, m * k <= 4096), the decode kernel over
# pre-quantized codes (n, k <= 2048; m <= 8 with k <= 1024 to n = 5120; m = 5..8
# with k >= 8192 to n = 2048; m = 17..32
# as one 32-row batch to n = 1536, m = 33..64 as one of 64 to n = 512; waves
# sharing a row group over slices of the activation rows), and the GEMV / MFMA
# paths otherwise. All share the act
# quant's codes, exact int32 sums and the epilogue, so every route's output
# equals the forced MFMA path's bit for bit.
@pytest.mark.parametrize("m,n,k", [(1, 256, 1536), (2, 8960, 1536), (2, 1536, 2048), (1, 1, 16), (2, 3, 2048),
                                   (8, 1536, 1536), (8, 256, 1536), (5, 2000, 1024), (3, 1000, 2048),
                                   (7, 129, 528), (8, 2048, 2048), (4, 8960, 1536), (8, 1536, 8960),
                                   (9, 1536, 1536), (12, 256, 1536), (16, 2048, 2048), (16, 256, 1536),
                                   (13, 1000, 1040), (16, 8960, 1536), (16, 1536, 8960),
                                   (8, 4864, 896), (6, 5120, 1024), (17, 256, 1536), (24, 256, 1536),
                                   (32, 512, 2048), (31, 100, 528), (20, 33, 16), (32, 513, 2048),
                                   (48, 256, 1536), (64, 512, 2048), (33, 300, 1040), (64, 1, 16),
                                   (30, 1536, 1536), (40, 512, 528), (5, 256, 1536), (6, 1536, 8960),
                                   (8, 2000, 8192), (7, 33, 9216), (1, 4864, 896), (1, 1001, 1024),
                                   (1, 3, 16)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                     (torch.float16, torch.float32)])
def test_w8a8_decode_routes_equal_mfma(dev, nq, m, n, k, xdt, ydt):
    g = torch.Generator(device=dev).manual_seed(m * 1000 + n + k)
    x = torch.randn((m, k), generator=g, device=dev).to(xdt)
    w = torch.randn((n, k), generator=g, device=dev) * 0.02
    b = torch.randn(n, generator=g, device=dev)
    t = nq.quantize_q8(w)
    y = nq.linear_w8a8(x, t, b, out_dtype=ydt)
    y_mfma = nq.linear_w8a8(x, t, b, out_dtype=ydt, path=nq._lib.NQ_PATH_MFMA)
    assert torch.isfinite(y).all()
    assert torch.equal(y, y_mfma), (m, n, k, float((y.float() - y_mfma.float()).abs().max()))
