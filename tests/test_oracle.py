"""Pins the CPU oracle (oracle/nq_oracle.c) before it is trusted as the checker.

Three independent anchors, chosen so a plausible slip (wrong rounding mode, a
dropped clamp, swapped nibbles, a missing block scale, a transposed operand)
fails at least one:
  * golden fixtures written by the reference's own compiled quant.cpp
    (tests/golden/gen_golden.py) — bit-exact;
  * the known answers of cpp/tests/test_quant.cpp and test_simd.cpp;
  * closed forms computed here with numpy, independently of the C code
    (float32 divide + np.rint for the codes, int64 brute force for dot_qq,
    float64 matmul for the linears).
"""
import numpy as np
import pytest


def same_bits(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype.kind == "f":
        return a.shape == b.shape and np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else np.uint16),
                                                     b.view(np.uint32 if b.dtype == np.float32 else np.uint16))
    return a.shape == b.shape and np.array_equal(a, b)


def np_quant_rows(w, qmax):
    """Closed form of round_clamp over per-row absmax (quant.cpp:31-38, :98-106)."""
    w = np.asarray(w, np.float32)
    a = np.abs(w)
    a = np.where(np.isnan(a), np.float32(0), a)          # NaN never wins std::max
    absmax = a.max(axis=1) if w.shape[1] else np.zeros(w.shape[0], np.float32)
    scale = (absmax / np.float32(qmax)).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.rint(w / scale[:, None]).astype(np.float32)
    r = np.clip(r, -qmax, qmax)
    r = np.where(np.isnan(r) | (scale[:, None] <= 0), 0, r)
    return r.astype(np.int8), scale


# ---- golden fixtures (reference build) ------------------------------------------------
def test_quantize_q8_golden(orc, golden):
    g = golden("q8_quantize")
    names = sorted({k.rsplit("_", 1)[0] for k in g.files})
    assert len(names) >= 7
    for n in names:
        q, s = orc.quantize_q8(g[n + "_w"])
        assert same_bits(q, g[n + "_q"]), n
        assert same_bits(s, g[n + "_s"]), n


def test_linear_q8_golden(orc, golden):
    g = golden("q8_linear")
    for i in range(6):
        b = g[f"c{i}_b"] if f"c{i}_b" in g.files else None
        y = orc.linear_q8(g[f"c{i}_x"], g[f"c{i}_q"], g[f"c{i}_s"], b)
        assert same_bits(y, g[f"c{i}_y"]), i


def test_w8a8_golden(orc, golden):
    g = golden("w8a8")
    for i in range(6):
        x = g[f"c{i}_x"]
        xq, xs = orc.act_quant(x)
        assert same_bits(xq, g[f"c{i}_xq"]) and same_bits(xs, g[f"c{i}_xs"]), i
        assert same_bits(orc.w8a8_acc(xq, g[f"c{i}_q"]), g[f"c{i}_acc"]), i
        b = g[f"c{i}_b"] if f"c{i}_b" in g.files else None
        y = orc.linear_w8a8(x, g[f"c{i}_q"], g[f"c{i}_s"], b)
        assert same_bits(y, g[f"c{i}_y"]), i


def test_q4g_golden(orc, golden):
    g = golden("q4g")
    for n in ("kat", "odd", "outlier"):
        q, s = orc.quantize_q4(g[n + "_w"])
        assert same_bits(q, g[n + "_q"]) and same_bits(s, g[n + "_s"]), n
    for n in ("g8", "partial", "g1", "g3odd", "g32", "nonfinite"):
        q, s = orc.quantize_q4g(g[n + "_w"], int(g[n + "_g"]))
        assert same_bits(q, g[n + "_q"]) and same_bits(s, g[n + "_s"]), n
    for i in range(6):
        b = g[f"lin{i}_b"] if f"lin{i}_b" in g.files else None
        y = orc.linear_q4g(g[f"lin{i}_x"], g[f"lin{i}_q"], g[f"lin{i}_s"], int(g[f"lin{i}_g"]), b)
        assert same_bits(y, g[f"lin{i}_y"]), i
    for m in (3, 16):
        y = orc.linear_q4(g[f"q4lin{m}_x"], g[f"q4lin{m}_q"], g[f"q4lin{m}_s"], g[f"q4lin{m}_b"])
        assert same_bits(y, g[f"q4lin{m}_y"]), m


def test_simd_golden(orc, golden):
    g = golden("simd")
    for n in range(71):
        assert same_bits(orc.unpack_q4(g[f"unpack{n}_p"], n), g[f"unpack{n}_c"]), n
    a, b = g["dotqq_a"], g["dotqq_b"]
    for i in range(41):
        assert orc.w8a8_acc(a[i:i + 1, :i], b[i:i + 1, :i])[0, 0] == g["dotqq_acc"][i]


def test_embedding_golden(orc, golden):
    g = golden("embedding_q8")
    q, s = orc.quantize_q8(g["table"])
    assert same_bits(q, g["q"]) and same_bits(s, g["s"])
    assert same_bits(orc.embedding_q8(q, s, g["ids"]), g["out"])


# ---- known answers (cpp/tests/test_quant.cpp, test_simd.cpp) -----------------------------
def test_q8_known_answers(orc):
    q, s = orc.quantize_q8(np.array([[1, 2, 4], [-8, 0, 8]], np.float32))   # test_quant.cpp:24-34
    assert abs(s[0] - 4 / 127) < 1e-9 and abs(s[1] - 8 / 127) < 1e-9
    assert q[0, 2] == 127 and q[1, 0] == -127 and q[1, 1] == 0
    q, s = orc.quantize_q8(np.array([[0, 0], [3, -3]], np.float32))          # :87-96
    assert s[0] == 0 and (q[0] == 0).all()
    q, _ = orc.quantize_q8(np.array([[5, 5, 5, 5], [1e30, -1e30, 1e-30, 0]], np.float32))  # :79-85
    assert q.min() >= -127 and q.max() <= 127


def test_q8_half_step_bound(orc):
    rng = np.random.default_rng(0)                                          # test_quant.cpp:36-49
    w = rng.normal(0, 3, (8, 32)).astype(np.float32)
    q, s = orc.quantize_q8(w)
    dq = orc.dequantize_q8(q, s)
    assert (np.abs(dq.astype(np.float64) - w) <= s[:, None] / 2 + 1e-6).all()


def test_q4_known_answers(orc):
    q, s = orc.quantize_q4(np.array([[7, -7]], np.float32))                 # test_quant.cpp:199-211
    assert s[0] == 1.0 and q.shape == (1, 1) and q[0, 0] == 0x1F
    q, s = orc.quantize_q4g(np.array([[3, -1, 0, 7, -2]], np.float32), 1)  # :322-330 group == 1 exact
    dq = orc.dequantize_q4g(q, s, 5, 1)
    assert np.allclose(dq, [[3, -1, 0, 7, -2]], atol=1e-5)
    rng = np.random.default_rng(8)                                          # :311-320 group == in is Q4
    w = rng.normal(0, 1, (4, 16)).astype(np.float32)
    a = orc.dequantize_q4g(*orc.quantize_q4g(w, 16), 16, 16)
    q4, s4 = orc.quantize_q4(w)
    assert np.allclose(a, orc.dequantize_q4g(q4, s4[:, None], 16, 16), atol=1e-6)
    w = np.array([[100] + [0.5] * 15], np.float32)                          # :285-296 outliers
    e4 = np.abs(orc.dequantize_q4g(*orc.quantize_q4(w)[:1], orc.quantize_q4(w)[1][:, None], 16, 16)[0, 8:] - 0.5).max()
    e4g = np.abs(orc.dequantize_q4g(*orc.quantize_q4g(w, 8), 16, 8)[0, 8:] - 0.5).max()
    assert e4g < e4 / 5


def test_q4g_rejects_bad_group(orc):
    import oracle
    with pytest.raises(oracle.OracleError):
        orc.quantize_q4g(np.zeros((2, 8), np.float32), 0)


def test_embedding_rejects_bad_id(orc):
    import oracle
    q, s = orc.quantize_q8(np.arange(12, dtype=np.float32).reshape(3, 4))
    with pytest.raises(oracle.OracleError):
        orc.embedding_q8(q, s, [3])                                          # test_quant.cpp:403-411


# ---- closed forms computed independently in numpy ----------------------------------------
@pytest.mark.parametrize("shape,sigma", [((64, 896), 0.02), ((33, 137), 3.0), ((5, 8960), 1.0)])
def test_quantize_closed_form(orc, shape, sigma):
    rng = np.random.default_rng(shape[1])
    w = rng.normal(0, sigma, shape).astype(np.float32)
    w[0, :3] = [np.nan, np.inf, -0.0]
    w[1] = 0
    q, s = orc.quantize_q8(w)
    qn, sn = np_quant_rows(w, 127)
    assert same_bits(s, sn) and np.array_equal(q, qn)


def test_q4g_closed_form(orc):
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (16, 256)).astype(np.float32)
    q, s = orc.quantize_q4g(w, 32)
    codes, scales = np_quant_rows(w.reshape(-1, 32), 7)
    assert same_bits(s.reshape(-1), scales)
    nib = (codes.reshape(16, 256).astype(np.int32) + 8).astype(np.uint8)
    packed = nib[:, 0::2] | (nib[:, 1::2] << 4)                              # even col -> low nibble
    assert np.array_equal(q, packed)


def test_unpack_all_nibbles(orc):
    packed = np.arange(256, dtype=np.uint8)
    c = orc.unpack_q4(packed, 512)
    assert np.array_equal(c[0::2], (packed & 15).astype(np.int8) - 8)
    assert np.array_equal(c[1::2], (packed >> 4).astype(np.int8) - 8)


def test_dot_qq_brute_force(orc):
    rng = np.random.default_rng(5)
    xq = rng.integers(-127, 128, (7, 8960), dtype=np.int8)
    wq = rng.integers(-127, 128, (9, 8960), dtype=np.int8)
    xq[0] = 127
    wq[0] = -127                                                             # the int32 extreme
    ref = xq.astype(np.int64) @ wq.astype(np.int64).T
    assert np.array_equal(orc.w8a8_acc(xq, wq), ref.astype(np.int32))


def test_linears_vs_float64(orc):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (5, 320)).astype(np.float32)
    w = rng.normal(0, 0.02, (40, 320)).astype(np.float32)
    b = rng.normal(0, 1, 40).astype(np.float32)
    q, s = orc.quantize_q8(w)
    ref = (x.astype(np.float64) @ (q.astype(np.float64) * s[:, None].astype(np.float64)).T) + b
    assert np.abs(orc.linear_q8(x, q, s, b) - ref).max() < 1e-4               # test_quant.cpp:51-64
    xq, xs = np_quant_rows(x, 127)
    ref = ((xq.astype(np.float64) * xs[:, None]) @ (q.astype(np.float64) * s[:, None]).T) + b
    assert np.abs(orc.linear_w8a8(x, q, s, b) - ref).max() < 1e-3             # :100-116
    p, t = orc.quantize_q4g(w, 32)
    deq = orc.dequantize_q4g(p, t, 320, 32).astype(np.float64)
    assert np.abs(orc.linear_q4g(x, p, t, 32, b) - (x.astype(np.float64) @ deq.T + b)).max() < 1e-4


def test_thread_count_invariance(orc):
    rng = np.random.default_rng(7)                                           # test_simd.cpp:84-109
    x = rng.normal(0, 1, (3, 137)).astype(np.float32)
    w = rng.normal(0, 1, (200, 137)).astype(np.float32)
    q, s = orc.quantize_q8(w)
    n0 = orc.max_threads()
    orc.set_threads(1)
    y1 = orc.linear_q8(x, q, s)
    orc.set_threads(max(2, n0))
    y2 = orc.linear_q8(x, q, s)
    orc.set_threads(n0)
    assert same_bits(y1, y2)


def test_reference_build_matches_when_present(orc):
    import oracle
    ref = oracle.reference()
    if ref is None:
        pytest.skip("oracle/_ref not built here (reference sources absent)")
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (9, 200)).astype(np.float32)
    w = rng.normal(0, 0.02, (130, 200)).astype(np.float32)
    q, s = orc.quantize_q8(w)
    assert same_bits(q, ref.quantize_q8(w)[0])
    assert same_bits(orc.linear_w8a8(x, q, s), ref.linear_w8a8(x, q, s))
    p, t = orc.quantize_q4g(w, 40)
    assert same_bits(orc.linear_q4g(x, p, t, 40), ref.linear_q4g(x, p, t, 40))


# ---- linear_f32 (ops.cpp:42-69, the dequant-matmul reference of test_quant.cpp) ----------
def test_linear_f32_golden(orc, golden):
    g = golden("ops")
    for i in range(3):
        b = g[f"lin{i}_b"] if f"lin{i}_b" in g.files else None
        y = orc.linear_f32(g[f"lin{i}_x"], g[f"lin{i}_w"], b)
        assert same_bits(y, g[f"lin{i}_y"]), i


def test_linear_f32_closed_form(orc):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (5, 77)).astype(np.float32)
    w = rng.normal(0, 1, (9, 77)).astype(np.float32)
    b = rng.normal(0, 1, 9).astype(np.float32)
    y = orc.linear_f32(x, w, b)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    # a transposed operand or a dropped bias fails this
    assert not np.allclose(orc.linear_f32(x, w), ref, atol=1e-3)


def test_dequantize_golden(orc, golden):
    g = golden("ops")
    for i in range(2):
        assert same_bits(orc.dequantize_q8(g[f"dq8_{i}_q"], g[f"dq8_{i}_s"]), g[f"dq8_{i}_w"]), i
    for i in range(3):
        w = orc.dequantize_q4g(g[f"dq4_{i}_q"], g[f"dq4_{i}_s"], int(g[f"dq4_{i}_k"]), int(g[f"dq4_{i}_g"]))
        assert same_bits(w, g[f"dq4_{i}_w"]), i
