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
        half = cfg.head_dim // 2
        inv = 1.0 / np.power(float(cfg.rope_theta), np.arange(half, dtype=np.float64) * 2.0 / cfg.head_dim)
        ang = np.arange(cfg.max_pos, dtype=np.float64)[:, None] * inv[None, :]
        c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        self.cos, self.sin = np.concatenate([c, c], 1), np.concatenate([s, s], 1)

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

    @staticmethod
    def rmsnorm(x, w, eps):
        out = np.empty_like(x)
        for r in range(x.shape[0]):
            ss = float(np.sum(x[r].astype(np.float64) ** 2))
            scale = np.float32(1.0) / np.sqrt(np.float32(ss / x.shape[1]) + np.float32(eps))
            out[r] = x[r] * scale * w
        return out

    def rope(self, x):
        s, d = x.shape[1], x.shape[2]
        half = d // 2
        rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
        return (x * self.cos[:s] + rot * self.sin[:s]).astype(np.float32)

    @staticmethod
    def attention(q, k, v, n_rep):
        k = np.repeat(k, n_rep, 0)
        v = np.repeat(v, n_rep, 0)
        h, s, d = q.shape
        scale = np.float32(1.0 / math.sqrt(d))
        out = np.empty_like(q)
        for hh in range(h):
            sc = (q[hh].astype(np.float64) @ k[hh].astype(np.float64).T).astype(np.float32) * scale
            for i in range(s):
                row = sc[i, : i + 1]
                e = np.exp(row - row.max()).astype(np.float32)
                inv = np.float32(1.0 / float(np.sum(e.astype(np.float64))))
                p = (e * inv).astype(np.float64)
                out[hh, i] = (p @ v[hh, : i + 1].astype(np.float64)).astype(np.float32)
        return out

    def forward(self, ids):
        cfg = self.cfg
        eq, es = self.embed
        x = self.cpu.embedding_q8(eq, es, np.asarray(ids, np.int64))
        s = x.shape[0]
        for li in range(self.n_layers):
            L = f"layers.{li}."
            h = self.rmsnorm(x, self.norm[L + "input_layernorm"], cfg.eps)
            q = self.project(h, L + "self_attn.q_proj").reshape(s, cfg.heads, cfg.head_dim).transpose(1, 0, 2)
            k = self.project(h, L + "self_attn.k_proj").reshape(s, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
            v = self.project(h, L + "self_attn.v_proj").reshape(s, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
            q, k = self.rope(q), self.rope(k)
            a = self.attention(q, k, v, cfg.n_rep).transpose(1, 0, 2).reshape(s, -1)
            x = x + self.project(np.ascontiguousarray(a), L + "self_attn.o_proj")
            hm = self.rmsnorm(x, self.norm[L + "post_attention_layernorm"], cfg.eps)
            g = self.project(hm, L + "mlp.gate_proj")
            g = g / (np.float32(1.0) + np.exp(-g))
            u = self.project(hm, L + "mlp.up_proj")
            x = x + self.project(np.ascontiguousarray(g * u), L + "mlp.down_proj")
        x = self.rmsnorm(x, self.final_norm, cfg.eps)
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
