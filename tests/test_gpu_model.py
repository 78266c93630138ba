"""Greedy-token parity of a random-init Qwen2-style model: projections, int8
embedding and int8 LM head on libnq_hip.so (GPU) vs the CPU quant path
(tests/model_ref.py over the oracle) on identical seeded weights."""
import numpy as np
import pytest
import torch

from model_ref import RefModel

pytestmark = pytest.mark.gpu

PROMPT = [3, 17, 42, 7, 99, 5, 250, 11]


def tiny():
    from nanoinfer_amd.model import Config
    return Config(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=1024,
                  max_pos=64)


@pytest.mark.parametrize("mode", ["w8a8", "q8", "q4g"])
@pytest.mark.parametrize("seed", [0, 1])
def test_greedy_tokens_match(orc, dev, mode, seed):
    from nanoinfer_amd import model, quant
    cfg = tiny()
    w = model.random_weights(cfg, seed)
    qm = {"w8a8": quant.QuantMode.W8A8, "q8": quant.QuantMode.Q8, "q4g": quant.QuantMode.Q4G}[mode]
    gpu = model.Model(cfg, w, qm, dev)
    ref = RefModel(orc, cfg, w, mode)
    lg = gpu.forward(PROMPT).cpu().numpy()
    lr = ref.forward(PROMPT)
    rms = float(np.sqrt(np.mean(lr.astype(np.float64) ** 2)))
    assert np.max(np.abs(lg - lr)) <= 2e-2 * rms, (np.max(np.abs(lg - lr)), rms)
    toks_gpu = gpu.generate(PROMPT, 12)
    toks_ref = ref.generate(PROMPT, 12)
    assert toks_gpu == toks_ref


def test_model_uses_quant_weights(dev):
    from nanoinfer_amd import model, quant
    cfg = tiny()
    m = model.Model(cfg, model.random_weights(cfg, 0), quant.QuantMode.W8A8, dev, layers=1)
    assert m.proj["layers.0.mlp.down_proj"].format() == quant.Format.W8A8
    assert m.embed.format() == quant.Format.Q8


@pytest.mark.parametrize("payload", [0, 1])
def test_model_from_nit_dir(dev, tmp_path, payload):
    """The model loaded from a directory of NIT files (fp32 / bf16 payloads,
    quantized on the device) generates the same tokens as the in-memory build
    of the same (bf16-exact) weights."""
    from nanoinfer_amd import model, quant
    from nit_util import bf16_exact, write_nit1
    cfg = tiny()
    w = {k: torch.from_numpy(bf16_exact(v.numpy())) for k, v in model.random_weights(cfg, 3).items()}
    for name, t in w.items():
        write_nit1(str(tmp_path / f"{name}.bin"), t.numpy(), payload)
    loaded = model.load_weights_dir(str(tmp_path), dev)
    assert set(loaded) == set(w)
    for name, t in w.items():
        assert torch.equal(loaded[name].cpu(), t), name
    a = model.Model(cfg, loaded, quant.QuantMode.W8A8, dev)
    b = model.Model(cfg, w, quant.QuantMode.W8A8, dev)
    assert a.generate(PROMPT, 6) == b.generate(PROMPT, 6)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_rope_qkv_matches_torch(dev, dt):
    """nq_rope_qkv equals the tensor-op RoPE (apply_rope) on the split heads."""
    from nanoinfer_amd import model
    cfg = model.Config(hidden=256, heads=12, kv_heads=2, head_dim=128, intermediate=512, layers=1, vocab=64,
                       max_pos=96)
    cos, sin = model.rope_tables(cfg, dev)
    s, hq, hkv = 77, 12 * 128, 2 * 128
    g = torch.Generator(device=dev).manual_seed(4)
    qkv = torch.randn((s, hq + 2 * hkv + 8), generator=g, device=dev).to(dt)[:, : hq + 2 * hkv]   # ld > width
    q, k, v = model.rope_qkv(qkv, 12, 2, 128, cos, sin)
    rq, rk, rv = qkv.float().split([hq, hkv, hkv], 1)
    rq = model.apply_rope(rq.reshape(s, 12, 128).transpose(0, 1), cos, sin)
    rk = model.apply_rope(rk.reshape(s, 2, 128).transpose(0, 1), cos, sin)
    rv = rv.reshape(s, 2, 128).transpose(0, 1)
    tol = 1e-5 if dt == torch.float32 else 2e-3
    assert torch.allclose(q.float(), rq, atol=tol, rtol=tol) and torch.allclose(k.float(), rk, atol=tol, rtol=tol)
    assert torch.equal(v.float(), rv)
