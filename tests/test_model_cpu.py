"""CPU checks of the decoder's torch helpers (no GPU): the fp16 fast paths
agree with the fp32 reference-semantics paths."""
import torch

from nanoinfer_amd import model


def test_attention_fast_path_matches_reference():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(4, 9, 32, generator=g)
    k = torch.randn(2, 9, 32, generator=g)
    v = torch.randn(2, 9, 32, generator=g)
    ref = model.attention(q, k, v, 2)
    fast = model.attention(q.half(), k.half(), v.half(), 2).float()
    assert torch.allclose(ref, fast, atol=5e-3, rtol=5e-3)


def test_rmsnorm_paths_agree():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 64, generator=g)
    w = 1 + 0.02 * torch.randn(64, generator=g)
    ref = model.rmsnorm(x, w, 1e-6)
    assert torch.allclose(model.rmsnorm(x.half(), w, 1e-6).float(), ref, atol=5e-3, rtol=5e-3)
    manual = x / torch.sqrt((x.double() ** 2).mean(-1, keepdim=True).float() + 1e-6) * w
    assert torch.allclose(ref, manual, atol=1e-6)


def test_rope_rotates_pairs():
    cfg = model.Config(hidden=64, heads=2, kv_heads=1, head_dim=32, intermediate=64, layers=1, vocab=8, max_pos=16)
    cos, sin = model.rope_tables(cfg, "cpu")
    x = torch.randn(2, 7, 32)
    y = model.apply_rope(x, cos, sin)
    # a rotation keeps the norm of every (d, d + half) pair
    h = 16
    nx = x[..., :h] ** 2 + x[..., h:] ** 2
    ny = y[..., :h] ** 2 + y[..., h:] ** 2
    assert torch.allclose(nx, ny, atol=1e-5)
    assert torch.allclose(y[:, 0], x[:, 0])  # position 0 is the identity
