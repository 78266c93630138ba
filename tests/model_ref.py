"""CPU reference decoder for the greedy-token parity test (test infrastructure).

The quantized projections, the int8 embedding gather and the int8 LM head run
through the CPU quant path (the oracle's C restatement of cpp/src/quant.cpp, or
the reference's own quant.cpp build when it is available); rmsnorm, RoPE,
causal GQA attention and SwiGLU follow cpp/src/ops.cpp in numpy with the same
fp64 accumulations:
  rmsnorm     ops.cpp:272-290   sum of squares in double, x * scale * w
  rope        ops.cpp:120-166   half-split tables built in double
  attention   ops.cpp:206-270   fp32 scores, double softmax denominator and PV sums
  silu / mul  ops.cpp:86-100
  layer       model.cpp:154-193 pre-norm attention and SwiGLU blocks
"""
from __future__ import annotations

import math

import numpy as np


class RefModel:
    def __init__(self, cpu, cfg, weights: dict, mode: str = "w8a8", layers=None, quantize_embed=True):
        self.cpu, self.cfg, self.mode = cpu, cfg, mode
        self.n_layers = cfg.layers if layers is None else layers
        f = lambda t: np.ascontiguousarray(t.numpy(), np.float32)
        self.proj, self.bias, self.norm = {}, {}, {}
        from nanoinfer_amd.model import PROJ
        for li in range(self.n_layers):
            L = f"layers.{li}."
            for p in PROJ:
                w = f(weights[L + p + ".weight"])
                if mode in ("w8a8", "q8"):
                    self.proj[L + p] = cpu.quantize_q8(w)
                elif mode == "q4g":
                    self.proj[L + p] = cpu.quantize_q4g(w, 32)
                else:
                    raise ValueError(mode)
            if cfg.qkv_bias:
                for p in ("q_proj", "k_proj", "v_proj"):
                    self.bias[L + f"self_attn.{p}"] = f(weights[L + f"self_attn.{p}.bias"])
            for nme in ("input_layernorm", "post_attention_layernorm"):
                self.norm[L + nme] = f(weights[L + nme + ".weight"])
        self.final_norm = f(weights["norm.weight"])
        self.embed = cpu.quantize_q8(f(weights["embed_tokens.weight"]))
        self.head = self.embed if cfg.tie_embeddings else cpu.quantize_q8(f(weights["lm_head.weight"]))
        self.cos, self.sin = rope_cache(cfg.max_pos, cfg.head_dim, cfg.rope_theta)

    def project(self, x, name):
        b = self.bias.get(name)
        if self.mode == "w8a8":
            q, s = self.proj[name]
            return self.cpu.linear_w8a8(x, q, s, b)
        if self.mode == "q8":
            q, s = self.proj[name]
            return self.cpu.linear_q8(x, q, s, b)
        q, s = self.proj[name]
        return self.cpu.linear_q4g(x, q, s, 32, b)

    def run_layers(self, x):
        """The decoder layers (model.cpp:166-190) on hidden states x [s, hidden]."""
        cfg = self.cfg
        s = x.shape[0]
        for li in range(self.n_layers):
            L = f"layers.{li}."
            h = rmsnorm(x, self.norm[L + "input_layernorm"], cfg.eps)
            q = self.project(h, L + "self_attn.q_proj").reshape(s, cfg.heads, cfg.head_dim).transpose(1, 0, 2)
            k = self.project(h, L + "self_attn.k_proj").reshape(s, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
            v = self.project(h, L + "self_attn.v_proj").reshape(s, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
            q, k = apply_rope(q, self.cos, self.sin), apply_rope(k, self.cos, self.sin)
            a = gqa_attention(q, k, v, cfg.n_rep).transpose(1, 0, 2).reshape(s, -1)
            x = x + self.project(np.ascontiguousarray(a), L + "self_attn.o_proj")
            hm = rmsnorm(x, self.norm[L + "post_attention_layernorm"], cfg.eps)
            g = silu(self.project(hm, L + "mlp.gate_proj"))
            u = self.project(hm, L + "mlp.up_proj")
            x = x + self.project(np.ascontiguousarray(g * u), L + "mlp.down_proj")
        return x

    def forward(self, ids):
        eq, es = self.embed
        x = self.run_layers(self.cpu.embedding_q8(eq, es, np.asarray(ids, np.int64)))
        x = rmsnorm(x, self.final_norm, self.cfg.eps)
        hq, hs = self.head
        return self.cpu.linear_q8(x, hq, hs)

    def generate(self, prompt, max_new):
        ids, out = list(prompt), []
        for _ in range(max_new):
            logits = self.forward(ids)
            nxt = int(np.argmax(logits[-1]))
            out.append(nxt)
            ids.append(nxt)
        return out


def rmsnorm(x, w, eps):
    """ops.cpp:272-290: sum of squares in double, scale = 1 / sqrt(float(ss / d) + eps)."""
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        ss = float(np.sum(x[r].astype(np.float64) ** 2))
        scale = np.float32(1.0) / np.sqrt(np.float32(ss / x.shape[1]) + np.float32(eps))
        out[r] = x[r] * scale * w
    return out


def rope_cache(seq, head_dim, theta):
    """ops.cpp:120-142: inv_freq and angles in double, cos/sin rounded to float,
    each frequency duplicated over both halves."""
    half = head_dim // 2
    inv = 1.0 / np.power(float(theta), np.arange(half, dtype=np.float64) * 2.0 / head_dim)
    ang = np.arange(seq, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    return np.concatenate([c, c], 1), np.concatenate([s, s], 1)


def apply_rope(x, cos, sin, pos_offset=0):
    """ops.cpp:144-166 on [heads, seq, dim]: x * cos + rotate_half(x) * sin in float."""
    s, d = x.shape[1], x.shape[2]
    half = d // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
    c, sn = cos[pos_offset:pos_offset + s], sin[pos_offset:pos_offset + s]
    return (x * c + rot * sn).astype(np.float32)


def attention(q, k, v, causal=True, query_offset=0):
    """ops.cpp:206-270 on [heads, seq, dim] (k and v already repeated per head):
    fp32 scores (double dot, scaled in float), float exp, double denominator,
    PV sums of double(e) * inv * v in double."""
    h, sq, d = q.shape
    sk = k.shape[1]
    scale = np.float32(1.0 / math.sqrt(d))
    out = np.empty_like(q)
    for hh in range(h):
        sc = (q[hh].astype(np.float64) @ k[hh].astype(np.float64).T).astype(np.float32) * scale
        for i in range(sq):
            lim = query_offset + i + 1 if causal else sk
            row = sc[i, :lim]
            e = np.exp(row - row.max()).astype(np.float32)
            inv = np.float32(1.0 / float(np.sum(e.astype(np.float64))))
            p = e.astype(np.float64) * np.float64(inv)
            out[hh, i] = (p @ v[hh, :lim].astype(np.float64)).astype(np.float32)
    return out


def gqa_attention(q, k, v, n_rep):
    """repeat_kv (ops.cpp:190-204) then causal attention."""
    return attention(q, np.repeat(k, n_rep, 0), np.repeat(v, n_rep, 0))


def silu(x):
    """ops.cpp:86-92: v / (1 + exp(-v)) in float."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore"):
        return x / (np.float32(1.0) + np.exp(-x))
