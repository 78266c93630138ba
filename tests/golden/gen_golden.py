"""Write the golden fixtures for the quant path from the REFERENCE's own build.

Runs in the build container only (it needs ``oracle/_ref/libnqref.so``, which is
``/root/reference/cpp/src/quant.cpp`` compiled by ``oracle/Makefile``). Every
fixture is data: seeded inputs plus the reference's outputs for them
(``quant.cpp`` ``quantize_q8`` / ``linear_q8`` / ``linear_w8a8`` /
``quantize_q4g`` / ``linear_q4g`` / ``quantize_q4`` / ``linear_q4`` /
``embedding_q8`` and ``simd::dot_qq`` / ``simd::unpack_q4``). The cases follow
``cpp/tests/test_quant.cpp`` and ``cpp/tests/test_simd.cpp`` (known answers,
zero rows, clamps, odd widths, partial groups, both Q4 m-paths) plus seeded
random cases at small versions of the benchmark shapes and non-finite inputs.

Usage:  python tests/golden/gen_golden.py     (rewrites tests/golden/*.npz)
        python tests/golden/gen_golden.py --ops-only   (only ops.npz)
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def main():
    oracle.build(ref=True)
    ref = oracle.reference()
    assert ref is not None, "reference build missing"
    rng = np.random.default_rng(20261201)

    # ---- Q8 quantize (quant.cpp:88-108) --------------------------------------
    q8 = {}
    cases = [
        ("kat", np.array([[1, 2, 4], [-8, 0, 8]], np.float32)),             # test_quant.cpp:24-34
        ("clamp", np.array([[5, 5, 5, 5], [1e30, -1e30, 1e-30, 0]], np.float32)),  # :79-85
        ("zero_row", np.array([[0, 0], [3, -3]], np.float32)),             # :87-96
        ("ties", np.array([[127, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 2.5]], np.float32)),
        ("nonfinite", np.array([[np.nan, 1, -2, 3], [np.inf, 1, 2, 3], [1, 2, np.nan, np.nan]], np.float32)),
        ("rand_896", rng.normal(0, 0.02, (48, 896)).astype(np.float32)),
        ("rand_odd", rng.normal(0, 3.0, (13, 137)).astype(np.float32)),
    ]
    for name, w in cases:
        q, s = ref.quantize_q8(w)
        q8[name + "_w"], q8[name + "_q"], q8[name + "_s"] = w, q, s
    np.savez_compressed(os.path.join(OUT, "q8_quantize.npz"), **q8)

    # ---- Q8 linear (quant.cpp:136-163) ---------------------------------------
    lin = {}
    for i, (m, n, k, bias) in enumerate([(1, 64, 896, False), (3, 5, 16, True), (2, 7, 12, False),
                                         (8, 100, 90, False), (4, 96, 1536, True), (16, 33, 64, False)]):
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32) if bias else None
        q, s = ref.quantize_q8(w)
        y = ref.linear_q8(x, q, s, b)
        lin[f"c{i}_x"], lin[f"c{i}_q"], lin[f"c{i}_s"], lin[f"c{i}_y"] = x, q, s, y
        if b is not None:
            lin[f"c{i}_b"] = b
    np.savez_compressed(os.path.join(OUT, "q8_linear.npz"), **lin)

    # ---- W8A8 (quant.cpp:165-210, simd.hpp:160-197) --------------------------
    wa = {}
    for i, (m, n, k, bias) in enumerate([(1, 64, 1536, False), (3, 5, 16, True), (8, 48, 1536, False),
                                         (16, 40, 256, True), (5, 24, 8960, False), (64, 16, 128, False)]):
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        if i == 3:
            x[1] = 0.0           # all-zero activation row -> a_scale 0
            x[2, 5] = np.nan     # NaN activation -> code 0, ignored by absmax
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32) if bias else None
        q, s = ref.quantize_q8(w)
        xq, xs = ref.quantize_q8(x)          # the activation quant is quantize_q8's per-row scheme
        acc = ref.w8a8_acc(xq, q)
        y = ref.linear_w8a8(x, q, s, b)
        for key, v in dict(x=x, q=q, s=s, xq=xq, xs=xs, acc=acc, y=y).items():
            wa[f"c{i}_{key}"] = v
        if b is not None:
            wa[f"c{i}_b"] = b
    np.savez_compressed(os.path.join(OUT, "w8a8.npz"), **wa)

    # ---- Q4G / Q4 (quant.cpp:212-389) ----------------------------------------
    q4 = {}
    q4["kat_w"] = np.array([[7, -7]], np.float32)                      # test_quant.cpp:199-211
    q4["kat_q"], q4["kat_s"] = ref.quantize_q4(q4["kat_w"])
    q4["odd_w"] = np.array([[1, -2, 4], [7, 0, -7]], np.float32)      # :231-241
    q4["odd_q"], q4["odd_s"] = ref.quantize_q4(q4["odd_w"])
    q4["outlier_w"] = np.array([[100, 1, -1, 0]], np.float32)         # :213-219
    q4["outlier_q"], q4["outlier_s"] = ref.quantize_q4(q4["outlier_w"])
    gcases = [("g8", 8, rng.normal(0, 2, (4, 40))), ("partial", 4, np.arange(20).reshape(2, 10) - 5.0),
              ("g1", 1, np.array([[3, -1, 0, 7, -2]])), ("g3odd", 3, rng.normal(0, 1, (3, 11))),
              ("g32", 32, rng.normal(0, 0.02, (24, 896))),
              ("nonfinite", 4, np.array([[np.nan, 1, 2, 3, np.inf, 1, 1, 1, 0, 0, 0, 0]]))]
    for name, g, w in gcases:
        w = np.asarray(w, np.float32)
        q, s = ref.quantize_q4g(w, g)
        q4[f"{name}_w"], q4[f"{name}_q"], q4[f"{name}_s"] = w, q, s
        q4[f"{name}_g"] = np.int64(g)
    for i, (m, n, k, g, bias) in enumerate([(3, 5, 32, 8, True), (16, 5, 32, 8, False), (1, 48, 896, 32, False),
                                            (2, 24, 8960, 32, True), (8, 16, 256, 64, False), (9, 7, 40, 16, True)]):
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32) if bias else None
        q, s = ref.quantize_q4g(w, g)
        y = ref.linear_q4g(x, q, s, g, b)
        for key, v in dict(x=x, q=q, s=s, y=y, g=np.int64(g)).items():
            q4[f"lin{i}_{key}"] = v
        if b is not None:
            q4[f"lin{i}_b"] = b
    # per-row Q4 linear at both m paths (test_quant.cpp:177-197)
    for m in (3, 16):
        x = rng.normal(0, 1, (m, 40)).astype(np.float32)
        w = rng.normal(0, 1, (5, 40)).astype(np.float32)
        b = rng.normal(0, 1, 5).astype(np.float32)
        q, s = ref.quantize_q4(w)
        q4[f"q4lin{m}_x"], q4[f"q4lin{m}_q"], q4[f"q4lin{m}_s"], q4[f"q4lin{m}_b"] = x, q, s, b
        q4[f"q4lin{m}_y"] = ref.linear_q4(x, q, s, b)
    np.savez_compressed(os.path.join(OUT, "q4g.npz"), **q4)

    # ---- simd: dot_qq / unpack_q4 (test_simd.cpp:58-82) -----------------------
    sm = {}
    for n in range(0, 71):
        packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
        sm[f"unpack{n}_p"] = packed
        sm[f"unpack{n}_c"] = ref.unpack_q4(packed, n)
    a = rng.integers(-127, 128, (41, 40), dtype=np.int8)
    bq = rng.integers(-127, 128, (41, 40), dtype=np.int8)
    sm["dotqq_acc"] = np.array([ref.w8a8_acc(a[i:i + 1, :i], bq[i:i + 1, :i])[0, 0] for i in range(41)], np.int32)
    sm["dotqq_a"], sm["dotqq_b"] = a, bq
    np.savez_compressed(os.path.join(OUT, "simd.npz"), **sm)

    # ---- embedding_q8 (quant.cpp:121-134, test_quant.cpp:383-411) -------------
    table = rng.normal(0, 1, (6, 8)).astype(np.float32)
    q, s = ref.quantize_q8(table)
    ids = np.array([0, 5, 3, 3, 1], np.int64)
    np.savez_compressed(os.path.join(OUT, "embedding_q8.npz"), table=table, q=q, s=s, ids=ids,
                        out=ref.embedding_q8(q, s, ids))
    print("golden fixtures written to", OUT)


def ops_fixtures():
    """ops.cpp fixtures for tests/model_ref.py (rmsnorm :272-290, build_rope_cache /
    apply_rope :120-166, attention :206-270, silu :86-92) and for the oracle's
    linear_f32 (ops.cpp:42-69), written from the reference build."""
    oracle.build(ref=True)
    ref, ops = oracle.reference(), oracle.reference_ops()
    assert ref is not None and ops is not None, "reference build missing"
    rng = np.random.default_rng(20261202)
    o = {}
    for i, (rows, d, eps) in enumerate([(2, 1536, 1e-6), (3, 256, 1e-5), (2, 7, 1e-6)]):
        x = rng.normal(0, 1, (rows, d)).astype(np.float32)
        if i == 1:
            x[1] = 0.0                                       # zero row: scale = 1/sqrt(eps)
        w = (1 + rng.normal(0, 0.02, d)).astype(np.float32)
        o[f"rms{i}_x"], o[f"rms{i}_w"], o[f"rms{i}_eps"] = x, w, np.float32(eps)
        o[f"rms{i}_y"] = ops.rmsnorm(x, w, eps)
    for i, (seq, dim, theta) in enumerate([(40, 128, 1e6), (32, 64, 1e4)]):
        c, s = ops.rope_cache(seq, dim, theta)
        o[f"ropec{i}_seq"], o[f"ropec{i}_dim"], o[f"ropec{i}_theta"] = np.int64(seq), np.int64(dim), np.float32(theta)
        o[f"ropec{i}_cos"], o[f"ropec{i}_sin"] = c, s
        x = rng.normal(0, 1, (2, 16, dim)).astype(np.float32)
        o[f"rope{i}_x"] = x
        for off in (0, 9):
            o[f"rope{i}_{off}_y"] = ops.apply_rope(x, c, s, off)
    for i, (h, sq, sk, d, causal) in enumerate([(2, 21, 21, 64, True), (2, 5, 19, 64, True), (3, 4, 17, 32, False),
                                                 (1, 1, 1, 16, True)]):
        q = rng.normal(0, 1, (h, sq, d)).astype(np.float32)
        k = rng.normal(0, 1, (h, sk, d)).astype(np.float32)
        v = rng.normal(0, 1, (h, sk, d)).astype(np.float32)
        off = sk - sq if causal else 0
        for key, val in dict(q=q, k=k, v=v, causal=np.int64(causal), off=np.int64(off),
                             y=ops.attention(q, k, v, causal, off)).items():
            o[f"attn{i}_{key}"] = val
    g = np.concatenate([rng.normal(0, 4, 2000), [0.0, -0.0, 1e-30, -90.0, 90.0, 88.7, -88.7]]).astype(np.float32)
    o["silu_x"], o["silu_y"] = g, ops.silu(g)
    for i, (m, n, k, bias) in enumerate([(1, 24, 896, False), (3, 17, 40, True), (4, 9, 1536, True)]):
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32) if bias else None
        o[f"lin{i}_x"], o[f"lin{i}_w"] = x, w
        if b is not None:
            o[f"lin{i}_b"] = b
        o[f"lin{i}_y"] = ref.linear_f32(x, w, b)
    # dequantize_q8 / dequantize_q4g (quant.cpp:110-119, 323-335) of reference-quantized weights
    for i, (n, k) in enumerate([(5, 24), (3, 37)]):
        w = rng.normal(0, 0.05, (n, k)).astype(np.float32)
        q, s = ref.quantize_q8(w)
        o[f"dq8_{i}_q"], o[f"dq8_{i}_s"], o[f"dq8_{i}_w"] = q, s, ref.dequantize_q8(q, s)
    for i, (n, k, g) in enumerate([(4, 64, 32), (3, 37, 5), (2, 40, 16)]):
        w = rng.normal(0, 0.05, (n, k)).astype(np.float32)
        q, s = ref.quantize_q4g(w, g)
        q[0, 0] = 0x0F if k > 1 else q[0, 0]             # nibbles 15 and 0: codes +7 and -8
        o[f"dq4_{i}_q"], o[f"dq4_{i}_s"], o[f"dq4_{i}_g"] = q, s, np.int64(g)
        o[f"dq4_{i}_k"], o[f"dq4_{i}_w"] = np.int64(k), ref.dequantize_q4g(q, s, k, g)
    np.savez_compressed(os.path.join(OUT, "ops.npz"), **o)
    print("ops fixtures written to", OUT)


if __name__ == "__main__":
    if "--ops-only" not in sys.argv:
        main()
    ops_fixtures()
