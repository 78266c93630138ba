"""GPU parity: quantize/pack, activation quant and the int8 embedding gather are
bit-exact with the oracle (and through it with the reference quant.cpp)."""
import numpy as np
import pytest
import torch

from gpu_util import host, to_dev
from test_oracle import same_bits

pytestmark = pytest.mark.gpu


def test_quantize_q8_golden(dev, nq, golden):
    g = golden("q8_quantize")
    for n in sorted({k.rsplit("_", 1)[0] for k in g.files}):
        t = nq.quantize_q8(to_dev(g[n + "_w"], dev))
        assert same_bits(host(t.q), g[n + "_q"]), n
        assert same_bits(host(t.scale), g[n + "_s"]), n


@pytest.mark.parametrize("shape", [(4864, 896), (1536, 8960), (151936, 1536), (7, 90), (3, 0)])
def test_quantize_q8_full(dev, nq, orc, shape):
    rng = np.random.default_rng(sum(shape))
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    if w.size:
        w[0, 0] = np.nan
        w[-1] = 0
    t = nq.quantize_q8(to_dev(w, dev))
    q, s = orc.quantize_q8(w)
    assert same_bits(host(t.q), q) and same_bits(host(t.scale), s)


def test_quantize_q4g_golden(dev, nq, golden):
    g = golden("q4g")
    for n in ("g8", "partial", "g1", "g3odd", "g32", "nonfinite"):
        t = nq.quantize_q4g(to_dev(g[n + "_w"], dev), int(g[n + "_g"]))
        assert same_bits(host(t.q), g[n + "_q"]), n
        assert same_bits(host(t.scale), g[n + "_s"]), n
    for n in ("kat", "odd", "outlier"):
        t = nq.quantize_q4(to_dev(g[n + "_w"], dev))
        assert same_bits(host(t.q), g[n + "_q"]), n
        assert same_bits(host(t.scale).reshape(-1), g[n + "_s"]), n


# The vector path (group = 8 * 2^j <= 512, in % 8 == 0) and the scalar ones:
# partial last blocks (1000 % 32, 200 % 128), 64-lane blocks (g = 512), g = 8,
# a non-power-of-two lane count (g = 96) and in % 8 != 0 take the scalar kernels.
@pytest.mark.parametrize("shape,group", [((1536, 8960), 32), ((64, 896), 64), ((33, 137), 32), ((17, 45), 5),
                                         ((40, 1000), 32), ((9, 1024), 8), ((5, 4096), 512), ((11, 200), 128),
                                         ((7, 960), 96), ((3, 8192), 256)])
def test_quantize_q4g_full(dev, nq, orc, shape, group):
    rng = np.random.default_rng(shape[0] * 7 + shape[1])
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    w[0, 1] = np.nan                              # skipped by the absmax, code 0 (nibble 8)
    w[-1, -3:] = 0
    w[shape[0] // 2, 0] = 3.0                     # one block dominated by an outlier
    q, s = orc.quantize_q4g(w, group)
    t = nq.quantize_q4g(to_dev(w, dev), group)
    assert same_bits(host(t.q), q) and same_bits(host(t.scale), s)
    # fp16 scale storage: same codes, scale rounded to nearest-even fp16
    t16 = nq.quantize_q4g(to_dev(w, dev), group, scale_dtype=torch.float16)
    assert same_bits(host(t16.q), q)
    assert same_bits(host(t16.scale), s.astype(np.float16))


def test_q4_byte_layout_known_answer(dev, nq):
    t = nq.quantize_q4(to_dev(np.array([[7, -7]], np.float32), dev))       # test_quant.cpp:199-211
    assert host(t.q).tolist() == [[0x1F]] and host(t.scale).tolist() == [[1.0]]


@pytest.mark.parametrize("m,k", [(1, 896), (8, 1536), (16, 8960), (64, 1536), (512, 1536), (3, 90), (2, 0),
                                 (300, 8960), (256, 16384)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_act_quant(dev, nq, orc, m, k, xdt):
    rng = np.random.default_rng(m * 31 + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    if k:
        x[0, 0] = np.nan
        if m > 1:
            x[1] = 0
        if m > 2:
            x[2, -1] = 1e4                       # outlier dominates the row scale
    xw = to_dev(x, dev, xdt)
    xq, s = nq.act_quant(xw)
    xo = host(xw.float())                        # fp16 widens exactly; oracle sees the same values
    q_ref, s_ref = orc.act_quant(xo)
    assert same_bits(host(xq), q_ref) and same_bits(host(s), s_ref)


def test_act_quant_golden(dev, nq, golden):
    g = golden("w8a8")
    for i in range(6):
        xq, s = nq.act_quant(to_dev(g[f"c{i}_x"], dev))
        assert same_bits(host(xq), g[f"c{i}_xq"]) and same_bits(host(s), g[f"c{i}_xs"]), i


def test_embedding_q8(dev, nq, orc, golden):
    g = golden("embedding_q8")
    t = nq.quantize_q8(to_dev(g["table"], dev))
    assert same_bits(host(nq.embedding_q8(t, g["ids"])), g["out"])
    rng = np.random.default_rng(11)                                          # test_cuda.cpp:434
    table = rng.uniform(-1, 1, (2048, 896)).astype(np.float32)
    ids = rng.integers(0, 2048, 300)
    t = nq.quantize_q8(to_dev(table, dev))
    q, s = orc.quantize_q8(table)
    assert same_bits(host(nq.embedding_q8(t, ids)), orc.embedding_q8(q, s, ids))
    h = host(nq.embedding_q8(t, ids, out_dtype=torch.float16))
    assert same_bits(h, orc.embedding_q8(q, s, ids).astype(np.float16))
    with pytest.raises(ValueError):
        nq.embedding_q8(t, [2048])


def test_act_quant_ties_and_extremes(dev, nq, orc):
    """Rows whose quotients hit exact half-integers (the fast reciprocal path must
    hand them to the exact divide), tiny and huge scales, and non-finite values."""
    rows = [
        [127, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 2.5, 126.5, -126.5, 3.5, 4.5] + [0] * 4,
        [1e-38, 5e-39, -1e-39, 3e-40] + [0] * 12,                 # denormal-range scale
        [3e38, -1e38, 1e30, 7] + [0] * 12,
        [np.inf, 1, -2, 3] + [0] * 12,
        [np.nan, np.nan, 1, -1] + [0] * 12,
        list(np.linspace(-127, 127, 16)),
    ]
    x = np.array(rows, np.float32)
    xq, s = nq.act_quant(to_dev(x, dev))
    q_ref, s_ref = orc.act_quant(x)
    assert same_bits(host(xq), q_ref) and same_bits(host(s), s_ref)
    t = nq.quantize_q8(to_dev(x, dev))
    assert same_bits(host(t.q), q_ref) and same_bits(host(t.scale), s_ref)


# ---- dequantize (quant.cpp:110-119, 323-335) ------------------------------------------
def test_dequantize_golden(dev, nq, golden):
    g = golden("ops")
    for i in range(2):
        q, s = g[f"dq8_{i}_q"], g[f"dq8_{i}_s"]
        t = nq.QTensor(to_dev(q, dev), to_dev(s, dev), *q.shape)
        assert same_bits(host(nq.dequantize_q8(t)), g[f"dq8_{i}_w"]), i
    for i in range(3):
        q, s, k, gr = g[f"dq4_{i}_q"], g[f"dq4_{i}_s"], int(g[f"dq4_{i}_k"]), int(g[f"dq4_{i}_g"])
        t = nq.Q4GTensor(to_dev(q, dev), to_dev(s, dev), q.shape[0], k, gr)
        assert same_bits(host(nq.dequantize_q4g(t)), g[f"dq4_{i}_w"]), i


@pytest.mark.parametrize("shape", [(4864, 896), (151936, 1536), (7, 90), (3, 0), (0, 5)])
def test_dequantize_q8_full(dev, nq, orc, shape):
    rng = np.random.default_rng(shape[0] + 3 * shape[1])
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    t = nq.quantize_q8(to_dev(w, dev))
    q, s = host(t.q), host(t.scale)
    ref = orc.dequantize_q8(q, s)
    assert same_bits(host(nq.dequantize_q8(t)), ref)
    h = host(nq.dequantize_q8(t, torch.float16))
    assert same_bits(h, ref.astype(np.float16))


@pytest.mark.parametrize("shape,group", [((1536, 8960), 32), ((33, 137), 32), ((17, 45), 5), ((9, 1024), 3),
                                         ((5, 96), 96), ((4, 64), 200)])
def test_dequantize_q4g_full(dev, nq, orc, shape, group):
    rng = np.random.default_rng(shape[0] * 5 + shape[1])
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    q = rng.integers(0, 256, (shape[0], (shape[1] + 1) // 2), dtype=np.uint8)   # all 16 nibbles
    nb = (shape[1] + group - 1) // group
    s = np.abs(rng.normal(0, 0.01, (shape[0], nb))).astype(np.float32)
    t = nq.Q4GTensor(to_dev(q, dev), to_dev(s, dev), shape[0], shape[1], group)
    ref = orc.dequantize_q4g(q, s, shape[1], group)
    assert same_bits(host(nq.dequantize_q4g(t)), ref)
    # fp16 scale storage: the oracle on the widened fp16 scales
    s16 = s.astype(np.float16)
    t16 = nq.Q4GTensor(to_dev(q, dev), to_dev(s16, dev), shape[0], shape[1], group)
    ref16 = orc.dequantize_q4g(q, s16.astype(np.float32), shape[1], group)
    assert same_bits(host(nq.dequantize_q4g(t16)), ref16)
    assert same_bits(host(nq.dequantize_q4g(t16, torch.float16)), ref16.astype(np.float16))
