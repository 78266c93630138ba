"""Pins the CPU reference decoder used for greedy-token parity (tests/model_ref.py).

* Its quantized projections: the oracle's quant path and the reference's own
  quant.cpp build give the same tokens.
* Its non-quant ops (rmsnorm, RoPE, attention, silu), restated in numpy, against
  fixtures written by the reference's own ops.cpp build (tests/golden/ops.npz):
  rmsnorm and the RoPE tables bit for bit; apply_rope, attention and silu within
  the stated bounds (the compiled reference contracts or re-associates a few
  float operations and calls libm's expf, so their last bits may differ):
    apply_rope  |d| <= 4 * 2^-24 * (|x*cos| + |rot*sin|)     (half-ulps of the two terms)
    attention   |d| <= 8 * 2^-24 * max_j |v[j, d]|           (per head and column)
    silu        |d| <= 16 * 2^-24 * |y|                       (8 ulp relative)
  and against closed-form properties that a slip in the restatement would break.
"""
import numpy as np
import pytest

import model_ref as M

PROMPT = [3, 17, 42, 7, 99, 5, 250, 11]
E24 = 2.0 ** -24


@pytest.mark.parametrize("mode", ["w8a8", "q8", "q4g"])
def test_ref_model_oracle_matches_reference_build(orc, mode):
    import oracle
    from nanoinfer_amd.model import Config, random_weights
    ref = oracle.reference()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) not present")
    cfg = Config(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=1024,
                 max_pos=64, tie_embeddings=False)
    w = random_weights(cfg, 0)
    a = M.RefModel(orc, cfg, w, mode)
    b = M.RefModel(ref, cfg, w, mode)
    assert a.generate(PROMPT, 8) == b.generate(PROMPT, 8)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_rmsnorm_golden(golden):
    g = golden("ops")
    for i in range(3):
        y = M.rmsnorm(g[f"rms{i}_x"], g[f"rms{i}_w"], float(g[f"rms{i}_eps"]))
        assert np.array_equal(bits(y), bits(g[f"rms{i}_y"])), i


def test_rope_cache_golden(golden):
    g = golden("ops")
    for i in range(2):
        c, s = M.rope_cache(int(g[f"ropec{i}_seq"]), int(g[f"ropec{i}_dim"]), float(g[f"ropec{i}_theta"]))
        assert np.array_equal(bits(c), bits(g[f"ropec{i}_cos"])), i
        assert np.array_equal(bits(s), bits(g[f"ropec{i}_sin"])), i


def test_apply_rope_golden(golden):
    g = golden("ops")
    for i in range(2):
        c, s, x = g[f"ropec{i}_cos"], g[f"ropec{i}_sin"], g[f"rope{i}_x"]
        half = x.shape[-1] // 2
        rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
        for off in (0, 9):
            y = M.apply_rope(x, c, s, off)
            cs, sn = c[off:off + x.shape[1]], s[off:off + x.shape[1]]
            bound = 4 * E24 * (np.abs(x * cs).astype(np.float64) + np.abs(rot * sn))
            assert (np.abs(y.astype(np.float64) - g[f"rope{i}_{off}_y"]) <= bound).all(), (i, off)


def test_attention_golden(golden):
    g = golden("ops")
    for i in range(4):
        q, k, v = g[f"attn{i}_q"], g[f"attn{i}_k"], g[f"attn{i}_v"]
        y = M.attention(q, k, v, bool(g[f"attn{i}_causal"]), int(g[f"attn{i}_off"]))
        bound = 8 * E24 * np.abs(v).max(axis=1, keepdims=True).astype(np.float64)
        assert (np.abs(y.astype(np.float64) - g[f"attn{i}_y"]) <= bound).all(), i


def test_silu_golden(golden):
    g = golden("ops")
    y = M.silu(g["silu_x"])
    assert (np.abs(y.astype(np.float64) - g["silu_y"]) <= 16 * E24 * np.abs(g["silu_y"])).all()


def test_ops_closed_forms():
    """Properties the mathematics fixes, independent of the fixtures."""
    rng = np.random.default_rng(3)
    # rmsnorm: unit weight gives rows of RMS 1 (up to eps)
    x = rng.normal(0, 3, (4, 512)).astype(np.float32)
    y = M.rmsnorm(x, np.ones(512, np.float32), 1e-12)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-5)
    # RoPE is a rotation: it keeps each (i, i + half) pair's norm; position 0 is identity
    c, s = M.rope_cache(16, 64, 1e4)
    q = rng.normal(0, 1, (2, 16, 64)).astype(np.float32)
    r = M.apply_rope(q, c, s)
    n0 = q[..., :32] ** 2 + q[..., 32:] ** 2
    n1 = r[..., :32] ** 2 + r[..., 32:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
    assert np.array_equal(r[:, 0], q[:, 0])
    # relative-position property: <rope(q, i), rope(k, j)> depends on i - j only
    qv = np.tile(q[:1, :1], (1, 16, 1))
    kv = np.tile(rng.normal(0, 1, (1, 1, 64)).astype(np.float32), (1, 16, 1))
    rq, rk = M.apply_rope(qv, c, s)[0], M.apply_rope(kv, c, s)[0]
    assert abs(float(rq[5] @ rk[3]) - float(rq[9] @ rk[7])) < 1e-4
    # attention: first causal query sees only key 0; uniform scores average v
    k = rng.normal(0, 1, (1, 6, 8)).astype(np.float32)
    v = rng.normal(0, 1, (1, 6, 8)).astype(np.float32)
    qa = rng.normal(0, 1, (1, 6, 8)).astype(np.float32)
    a = M.attention(qa, k, v)
    assert np.allclose(a[0, 0], v[0, 0], atol=1e-7)
    a0 = M.attention(np.zeros_like(qa), k, v, causal=False)
    assert np.allclose(a0[0], v[0].mean(0), atol=1e-6)
    # brute-force softmax for one causal row
    sc = (qa[0, 3] @ k[0, :4].T) / np.sqrt(8.0)
    p = np.exp(sc - sc.max())
    p /= p.sum()
    assert np.allclose(a[0, 3], p @ v[0, :4], atol=1e-6)
    # silu closed form
    z = np.linspace(-20, 20, 101).astype(np.float32)
    assert np.allclose(M.silu(z), z / (1 + np.exp(-z.astype(np.float64))), rtol=1e-6, atol=1e-30)
