"""Per-call kernel choice of the weight-only linears, the W8A8 LM-head prefill
route and the fused greedy pick on the nicpp seam.

* nq_linear_q8_ex / nq_linear_q4g_ex with every forced path (the per-call
  form of the reference's CudaPolicy::force_tiled_q8, cuda_quant.cu:308): each
  path within 1e-3 * RMS of the oracle, GEMV against MFMA at the same shapes.
* use_w8a8_lmhead (cuda_quant.cu:362-372): the int8 embedding's linear at
  m > 8 runs W8A8 on the same codes; checked against the oracle's linear_w8a8
  at (128, 151936, 1536) on sampled vocabulary rows (the linear is row
  independent, and the codes of those rows are the same per-row quantize).
* nicpp.Model.next_token / generate take the LM-head GEMV with the argmax
  fused in: the id equals the reference scan over forward()'s last row.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close_rms, host, to_dev

pytestmark = pytest.mark.gpu

F32, F16 = torch.float32, torch.float16


def _data(m, n, k, seed):
    rng = np.random.default_rng(seed)
    return (rng.normal(0, 1, (m, k)).astype(np.float32), rng.normal(0, 0.02, (n, k)).astype(np.float32),
            rng.normal(0, 1, n).astype(np.float32))


PATH_CASES = [
    (1, 4864, 896, F32),      # config 1 (decode)
    (3, 1536, 1536, F16),
    (12, 1536, 8960, F16),    # m = 9..15 on long K (AUTO splits K over the workspace)
    (40, 896, 896, F32),
    (1, 1537, 8960, F16),     # config 2's K, ragged n
]


@pytest.mark.parametrize("m,n,k,xdt", PATH_CASES)
def test_q8_every_path_matches_oracle(dev, nq, orc, m, n, k, xdt):
    from nanoinfer_amd import _lib as L
    x, w, b = _data(m, n, k, 11 * m + n)
    t = nq.quantize_q8(to_dev(w, dev))
    xd, bd = to_dev(x, dev, xdt), to_dev(b, dev)
    q, s = orc.quantize_q8(w)
    ref = orc.linear_q8(host(xd.float()), q, s, b)
    outs = {}
    for path in (L.NQ_PATH_AUTO, L.NQ_PATH_GEMV, L.NQ_PATH_MFMA, L.NQ_PATH_GENERIC):
        print(f"q8 path {path} m={m} n={n} k={k} {xdt}", flush=True)
        y = nq.linear_q8(xd, t, bd, out_dtype=F32, path=path)
        outs[path] = host(y)
        assert_close_rms(outs[path], ref, f"linear_q8 path {path} {m}x{n}x{k}")
    # GEMV and MFMA sum the same products in another order: they agree to rounding
    assert_close_rms(outs[L.NQ_PATH_MFMA], outs[L.NQ_PATH_GEMV], "q8 MFMA vs GEMV", rel=2e-6 * np.sqrt(k))


@pytest.mark.parametrize("m,n,k,xdt", PATH_CASES)
@pytest.mark.parametrize("group", [32, 128])
def test_q4g_every_path_matches_oracle(dev, nq, orc, m, n, k, xdt, group):
    from nanoinfer_amd import _lib as L
    x, w, b = _data(m, n, k, 13 * m + n + group)
    t = nq.quantize_q4g(to_dev(w, dev), group, scale_dtype=F16)
    xd, bd = to_dev(x, dev, xdt), to_dev(b, dev)
    p, s = orc.quantize_q4g(w, group)
    s16 = s.astype(np.float16).astype(np.float32)   # the fp16 storage variant's scales, widened
    ref = orc.linear_q4g(host(xd.float()), p, s16, group, b)
    outs = {}
    for path in (L.NQ_PATH_AUTO, L.NQ_PATH_GEMV, L.NQ_PATH_MFMA, L.NQ_PATH_GENERIC):
        print(f"q4g path {path} m={m} n={n} k={k} g={group} {xdt}", flush=True)
        y = nq.linear_q4g(xd, t, bd, out_dtype=F32, path=path)
        outs[path] = host(y)
        assert_close_rms(outs[path], ref, f"linear_q4g path {path} {m}x{n}x{k} g{group}")
    assert_close_rms(outs[L.NQ_PATH_MFMA], outs[L.NQ_PATH_GEMV], "q4g MFMA vs GEMV", rel=2e-6 * np.sqrt(k))


def test_forced_mfma_refuses_off_contract(dev, nq):
    """k % 32 != 0 has no MFMA form: the forced path raises instead of running
    another kernel."""
    from nanoinfer_amd import _lib as L
    w = torch.randn(64, 48, device=dev) * 0.02
    t = nq.quantize_q8(w)
    with pytest.raises(ValueError, match="MFMA path"):
        nq.linear_q8(torch.randn(2, 48, device=dev), t, path=L.NQ_PATH_MFMA)


def _lm_head(dev, nq, n=151936, k=1536, seed=5):
    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    emb = nq.make_q8_embed(w)
    return w, emb


def test_w8a8_lmhead_prefill_route(dev, nq, orc):
    """use_w8a8_lmhead: m = 128 prefill rows through the int8 LM head run as
    W8A8 on the embedding's own codes, within 1e-3 * RMS of the oracle's
    linear_w8a8 (quant.cpp:165-210) on 4096 sampled vocabulary rows; the
    codes of those rows are bit-exact. Decode (m <= 8) stays weight-only."""
    m, n, k = 128, 151936, 1536
    w, emb = _lm_head(dev, nq, n, k)
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    xd = to_dev(x, dev)
    rows = np.sort(rng.choice(n, 4096, replace=False))
    wr = host(w[torch.from_numpy(rows).to(dev)])
    q, s = orc.quantize_q8(wr)
    assert np.array_equal(host(emb.t.q[torch.from_numpy(rows).to(dev)]), q)
    pol = nq.policy()
    try:
        pol.use_w8a8_lmhead = True
        print("w8a8 lm head m=128", flush=True)
        y = host(emb.linear(xd))
        assert y.shape == (m, n)
        assert_close_rms(y[:, rows], orc.linear_w8a8(x, q, s), "W8A8 LM head m=128")
        # the same as the W8A8 linear on those codes, bit for bit
        assert np.array_equal(y, host(nq.linear_w8a8(xd, emb.t)))
        # decode stays on the weight-only GEMV (the reference's m <= kGemvMaxM branch)
        y8 = host(emb.linear(xd[:8]))
        assert np.array_equal(y8, host(nq.linear_q8(xd[:8], emb.t)))
        assert_close_rms(y8[:, rows], orc.linear_q8(x[:8], q, s), "weight-only LM head m=8")
    finally:
        pol.use_w8a8_lmhead = False
    # policy off: the weight-only linear at m = 128
    y = host(emb.linear(xd))
    assert_close_rms(y[:, rows], orc.linear_q8(x, q, s), "weight-only LM head m=128")


def test_force_tiled_q8_lm_head(dev, nq, orc):
    """force_tiled_q8 runs the LM head's weight-only linear on the MFMA GEMM at
    decode m; same results to rounding."""
    from nanoinfer_amd import _lib as L
    n, k = 32768, 1536
    w, emb = _lm_head(dev, nq, n, k, seed=6)
    x = torch.randn(2, k, device=dev)
    base = host(emb.linear(x))
    pol = nq.policy()
    try:
        pol.force_tiled_q8 = True
        tiled = host(emb.linear(x))
    finally:
        pol.force_tiled_q8 = False
    assert np.array_equal(tiled, host(nq.linear_q8(x, emb.t, path=L.NQ_PATH_MFMA)))
    assert_close_rms(tiled, base, "tiled vs GEMV LM head", rel=1e-5)


def test_nicpp_w8a8_lmhead_policy(dev, orc):
    """The C++ HipEmbedQ8Weight follows nicpp.set_policy as the reference's
    CudaEmbedQ8Weight follows cuda_policy()."""
    from nanoinfer_amd import nicpp
    m, n, k = 64, 8192, 1536
    rng = np.random.default_rng(21)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    be = nicpp.make_backend("hip")
    emb = be.make_embed_weight(w)
    q, s = orc.quantize_q8(w)
    assert nicpp.policy() == {"use_w8a8_lmhead": False, "force_tiled_q8": False}
    assert_close_rms(emb.linear(x), orc.linear_q8(x, q, s), "nicpp LM head weight-only")
    try:
        nicpp.set_policy(use_w8a8_lmhead=True)
        assert_close_rms(emb.linear(x), orc.linear_w8a8(x, q, s), "nicpp LM head W8A8")
        assert_close_rms(emb.linear(x[:8]), orc.linear_q8(x[:8], q, s), "nicpp LM head decode stays q8")
        nicpp.set_policy(force_tiled_q8=True)
        assert_close_rms(emb.linear(x[:3]), orc.linear_q8(x[:3], q, s), "nicpp LM head forced tiled")
    finally:
        nicpp.set_policy()


def _ref_scan(row):
    """sampling.cpp:14-20: left-to-right strict >, logit 0 NaN never beaten."""
    best, bv = 0, row[0]
    for i in range(1, len(row)):
        if row[i] > bv:
            best, bv = i, row[i]
    return best


@pytest.mark.parametrize("mode", ["w8a8", "q4g"])
def test_nicpp_next_token_is_fused_argmax_of_forward(tmp_path, mode):
    """next_token (the fused argmax on the last position) equals the reference
    scan over forward()'s last row, and generate() continues with those ids."""
    from nanoinfer_amd import model, nicpp
    from test_gpu_nicpp_model import PROMPT, _cfg, _write_dir
    cfg = _cfg()
    _write_dir(tmp_path, cfg, model.random_weights(cfg, 31))
    m = nicpp.Model(str(tmp_path), nicpp.quant_mode(mode), "hip")
    ids = list(PROMPT)
    gen = m.generate(PROMPT, 6)
    for t in gen:
        lg = m.forward(ids)
        assert m.next_token(ids) == _ref_scan(lg[-1]) == t
        ids.append(t)


def test_nicpp_untied_without_lm_head_uses_embedding(tmp_path):
    """An untied config with no lm_head.weight file keeps the embedding as the
    head (model.cpp:187, 290-296), giving the tied model's logits."""
    import dataclasses

    from nanoinfer_amd import model, nicpp
    from test_gpu_nicpp_model import PROMPT, _cfg, _write_dir
    cfg = _cfg(tie=True)
    w = model.random_weights(cfg, 41)
    a, b = tmp_path / "tied", tmp_path / "untied"
    a.mkdir()
    b.mkdir()
    _write_dir(a, cfg, w)
    _write_dir(b, dataclasses.replace(cfg, tie_embeddings=False), w)   # no lm_head.weight written
    ma = nicpp.Model(str(a), nicpp.QuantMode.W8A8, "hip")
    mb = nicpp.Model(str(b), nicpp.QuantMode.W8A8, "hip")
    assert mb.config.tie_word_embeddings == 0
    assert np.array_equal(ma.forward(PROMPT), mb.forward(PROMPT))
    assert ma.weight_bytes() == mb.weight_bytes()
