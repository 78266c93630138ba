"""nicpp.Model — the reference's Python seam (cpp/bindings/nicpp.cpp:207-233, 317)
over the C++ host Model: a random-init Qwen2-style model written as a weights
directory (config.txt + NIT0 / NIT1 files, the exporter's layout), loaded with
device="hip", against the CPU reference decoder (tests/model_ref.py over the
oracle) on the same weights: logits within 2e-2 * RMS (an activation code may
round the other way in W8A8), greedy tokens equal."""
import dataclasses

import numpy as np
import pytest

from model_ref import RefModel
from nit_util import bf16_exact, write_nit0, write_nit1

pytestmark = pytest.mark.gpu

PROMPT = [3, 17, 42, 7, 99, 5, 250, 11]


def _cfg(tie=True):
    from nanoinfer_amd.model import Config
    return Config(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=1024,
                  max_pos=64, tie_embeddings=tie)


def _write_dir(path, cfg, weights, nit1=False):
    lines = {"vocab_size": cfg.vocab, "hidden_size": cfg.hidden, "intermediate_size": cfg.intermediate,
             "num_layers": cfg.layers, "num_attention_heads": cfg.heads, "num_kv_heads": cfg.kv_heads,
             "head_dim": cfg.head_dim, "max_position_embeddings": cfg.max_pos, "rms_norm_eps": cfg.eps,
             "rope_theta": cfg.rope_theta, "tie_word_embeddings": int(cfg.tie_embeddings),
             "eos_token_id": -1, "qkv_bias": int(cfg.qkv_bias), "some_future_key": 7}
    with open(path / "config.txt", "w") as f:
        for k, v in lines.items():
            f.write(f"{k} {v}\n")
    for name, t in weights.items():
        if nit1:
            write_nit1(str(path / f"{name}.bin"), t.numpy(), 1)
        else:
            write_nit0(str(path / f"{name}.bin"), t.numpy())


def _nicpp():
    from nanoinfer_amd import nicpp
    return nicpp


@pytest.mark.parametrize("mode", ["w8a8", "q8", "q4g", "q4"])
def test_nicpp_model_matches_reference_decoder(orc, tmp_path, mode):
    from nanoinfer_amd import model
    nicpp = _nicpp()
    cfg = _cfg(tie=mode != "q8")                 # one untied checkpoint (own lm_head.weight)
    w = model.random_weights(cfg, 5)
    _write_dir(tmp_path, cfg, w)
    m = nicpp.Model(str(tmp_path), nicpp.quant_mode(mode), "hip")
    c = m.config
    assert (c.hidden_size, c.num_layers, c.num_attention_heads, c.num_kv_heads, c.n_rep) == (256, 2, 4, 2, 2)
    if mode == "q4":
        ref = RefModel(orc, cfg, w, "q4g")       # per-row int4 = Q4G with one group per row
        ref.proj = {k: orc.quantize_q4g(w[k + ".weight"].numpy(), w[k + ".weight"].shape[1]) for k in ref.proj}
        in_g = {k: w[k + ".weight"].shape[1] for k in ref.proj}
        ref.project = lambda x, name: orc.linear_q4g(x, *ref.proj[name], in_g[name], ref.bias.get(name))
    else:
        ref = RefModel(orc, cfg, w, mode)
    lg = m.forward(PROMPT)
    lr = ref.forward(PROMPT)
    assert lg.shape == (len(PROMPT), cfg.vocab)
    rms = float(np.sqrt(np.mean(lr.astype(np.float64) ** 2)))
    assert np.max(np.abs(lg - lr)) <= 2e-2 * rms, (np.max(np.abs(lg - lr)), rms)
    assert m.generate(PROMPT, 12) == ref.generate(PROMPT, 12)


def test_nicpp_model_nit1_bf16_and_weight_bytes(tmp_path):
    """bf16 payloads load to the same model as the fp32 files of the same
    (bf16-exact) values; weight_bytes counts int8 projections + int8
    embedding + fp32 norms and biases (model.cpp:298-322)."""
    import torch

    from nanoinfer_amd import model
    nicpp = _nicpp()
    cfg = _cfg()
    w = {k: torch.from_numpy(bf16_exact(v.numpy())) for k, v in model.random_weights(cfg, 6).items()}
    a_dir, b_dir = tmp_path / "a", tmp_path / "b"
    a_dir.mkdir()
    b_dir.mkdir()
    _write_dir(a_dir, cfg, w)
    _write_dir(b_dir, cfg, w, nit1=True)
    a = nicpp.Model(str(a_dir), nicpp.QuantMode.W8A8, "hip")
    b = nicpp.Model(str(b_dir), nicpp.QuantMode.W8A8, "hip")
    assert np.array_equal(a.forward(PROMPT), b.forward(PROMPT))
    actual, fp32 = a.weight_bytes()
    proj = sum(o * i + 4 * o for o, i in model.proj_shapes(cfg).values()) * cfg.layers
    raw = (2 * cfg.hidden + (cfg.heads + 2 * cfg.kv_heads) * cfg.head_dim) * cfg.layers * 4 + cfg.hidden * 4
    emb = cfg.vocab * cfg.hidden + 4 * cfg.vocab
    assert actual == proj + raw + emb
    assert fp32 == sum(t.numel() for t in w.values()) * 4


def test_nicpp_model_errors(tmp_path):
    from nanoinfer_amd import model
    nicpp = _nicpp()
    cfg = _cfg()
    _write_dir(tmp_path, cfg, model.random_weights(cfg, 7))
    with pytest.raises(ValueError):
        nicpp.Model(str(tmp_path), nicpp.QuantMode.W8A8, "cpu")
    with pytest.raises(ValueError):
        nicpp.Model(str(tmp_path), nicpp.QuantMode.NONE, "hip")
    with pytest.raises(RuntimeError):
        nicpp.Model(str(tmp_path / "missing"), nicpp.QuantMode.W8A8, "hip")
    m = nicpp.Model(str(tmp_path), nicpp.QuantMode.Q8, "hip")
    with pytest.raises(ValueError):
        m.forward([1, cfg.vocab])                 # id out of range
    with pytest.raises(ValueError):
        m.forward([])
    with pytest.raises(ValueError):
        m.forward([1, 2], cache=object())
    (tmp_path / "config.txt").write_text("vocab_size 1024\nhidden_size 256\n")
    with pytest.raises(RuntimeError):
        nicpp.Model(str(tmp_path), nicpp.QuantMode.Q8, "hip")   # missing dimensions
    bad = dataclasses.replace(cfg)
    _write_dir(tmp_path, bad, model.random_weights(cfg, 7))
    with open(tmp_path / "config.txt", "a") as f:
        f.write("n_experts 8\n")
    with pytest.raises(RuntimeError):
        nicpp.Model(str(tmp_path), nicpp.QuantMode.Q8, "hip")   # an architecture this path does not implement
