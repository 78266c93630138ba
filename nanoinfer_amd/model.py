"""Qwen2-style decoder driven through the quantized-weight path.

This is the caller of the quant linears that the reference's Model is
(cpp/src/model.cpp:154-193): every projection is a device Weight from
quant.make_quantized (W8A8 / Q8 / Q4 / Q4G kernels of libnq_hip.so), the tied
embedding / LM head is the weight-only int8 Weight of quant.make_q8_embed
(model.cpp:146-149, the reference's quantize_embed), and the remaining ops
(rmsnorm, RoPE, causal GQA attention, SwiGLU gate, residual adds) are plain
torch device math with the reference's semantics (cpp/src/ops.cpp:86-300).
There is no KV cache: forward() recomputes the whole sequence, as the
reference's uncached path does (model.cpp:166-172).

Weights are named as the reference's exporter names them
("layers.N.self_attn.q_proj.weight", ...), fp32 on the host.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass

import torch

from . import quant


@dataclass(frozen=True)
class Config:
    """The Qwen2 fields the forward reads (cpp/src/model.hpp config)."""
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    layers: int
    vocab: int
    rope_theta: float = 1_000_000.0
    eps: float = 1e-6
    qkv_bias: bool = True
    max_pos: int = 4096
    tie_embeddings: bool = True

    @property
    def n_rep(self) -> int:
        return self.heads // self.kv_heads


def qwen25_15b(layers: int = 28) -> Config:
    """Qwen2.5-1.5B shapes (hidden 1536, 12 Q / 2 KV heads of 128, SwiGLU 8960)."""
    return Config(hidden=1536, heads=12, kv_heads=2, head_dim=128, intermediate=8960,
                  layers=layers, vocab=151936)


PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
        "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def proj_shapes(cfg: Config) -> dict:
    """[out, in] of the seven projections of one layer."""
    h, q, kv, i = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim, cfg.intermediate
    return {"self_attn.q_proj": (q, h), "self_attn.k_proj": (kv, h), "self_attn.v_proj": (kv, h),
            "self_attn.o_proj": (h, q), "mlp.gate_proj": (i, h), "mlp.up_proj": (i, h),
            "mlp.down_proj": (h, i)}


def random_weights(cfg: Config, seed: int = 0, layers=None) -> dict:
    """Random-init fp32 host weights: projections and embedding N(0, 0.02),
    q/k/v biases N(0, 0.02), norm weights 1 + N(0, 0.02) (seeded CPU generator)."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.02
    w = {"embed_tokens.weight": r(cfg.vocab, cfg.hidden), "norm.weight": 1.0 + r(cfg.hidden)}
    if not cfg.tie_embeddings:
        w["lm_head.weight"] = r(cfg.vocab, cfg.hidden)
    for li in range(cfg.layers if layers is None else layers):
        L = f"layers.{li}."
        for p, (o, i) in proj_shapes(cfg).items():
            w[L + p + ".weight"] = r(o, i)
        if cfg.qkv_bias:
            for p in ("q_proj", "k_proj", "v_proj"):
                w[L + f"self_attn.{p}.bias"] = r(proj_shapes(cfg)[f"self_attn.{p}"][0])
        w[L + "input_layernorm.weight"] = 1.0 + r(cfg.hidden)
        w[L + "post_attention_layernorm.weight"] = 1.0 + r(cfg.hidden)
    return w


def rope_tables(cfg: Config, device) -> tuple:
    """cos/sin [max_pos, head_dim], half-split layout (ops.cpp:120-143), in double."""
    half = cfg.head_dim // 2
    inv = 1.0 / torch.pow(torch.tensor(cfg.rope_theta, dtype=torch.float64),
                          torch.arange(half, dtype=torch.float64) * 2.0 / cfg.head_dim)
    ang = torch.arange(cfg.max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    return torch.cat([cos, cos], 1).to(device), torch.cat([sin, sin], 1).to(device)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """ops.cpp:272-290: x * (1 / sqrt(mean(x^2) + eps)) * w. fp32 activations sum
    the squares in fp64 as the reference does; fp16 activations in fp32."""
    xf = x.float()
    if x.dtype == torch.float32:
        ms = (x.double() * x.double()).mean(-1, keepdim=True).float()
    else:
        ms = (xf * xf).mean(-1, keepdim=True)
    return (xf * torch.rsqrt(ms + eps) * w).to(x.dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """ops.cpp:145-166 on [heads, seq, dim] at positions 0..seq-1."""
    s, d = x.shape[1], x.shape[2]
    half = d // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], -1)
    return x * cos[:s].to(x.dtype) + rot * sin[:s].to(x.dtype)


def rope_qkv(qkv: torch.Tensor, heads: int, kv_heads: int, head_dim: int, cos: torch.Tensor, sin: torch.Tensor):
    """One launch for the fused q|k|v output [s, (heads + 2 kv) d]: RoPE on q and
    k (ops.cpp:145-166) and all three written head-major [h, s, d]."""
    from ._lib import check, load
    s = qkv.shape[0]
    if qkv.stride(1) != 1 or cos.dtype != torch.float32 or cos.shape[0] < s:
        raise ValueError("rope_qkv: unit column stride, fp32 tables of >= s rows required")
    q = torch.empty((heads, s, head_dim), dtype=qkv.dtype, device=qkv.device)
    k = torch.empty((kv_heads, s, head_dim), dtype=qkv.dtype, device=qkv.device)
    v = torch.empty_like(k)
    dt = quant._dtype_code(qkv, "qkv")
    check(load().nq_rope_qkv(qkv.data_ptr(), dt, s, qkv.stride(0), heads, kv_heads, head_dim, cos.data_ptr(),
                             sin.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), quant._stream()))
    return q, k, v


def attention(q, k, v, n_rep: int) -> torch.Tensor:
    """ops.cpp:206-270: causal softmax(q k^T / sqrt(d)) v with the KV heads
    repeated n_rep times (GQA); scores and softmax in fp32. fp16 activations use
    torch's fused scaled-dot-product attention (fp32 softmax inside)."""
    if q.dtype == torch.float16:
        return torch.nn.functional.scaled_dot_product_attention(
            q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), is_causal=True, enable_gqa=n_rep > 1).squeeze(0)
    k = k.repeat_interleave(n_rep, 0)
    v = v.repeat_interleave(n_rep, 0)
    s = q.shape[1]
    scores = torch.matmul(q.float(), k.float().transpose(1, 2)) / math.sqrt(q.shape[2])
    mask = torch.ones(s, s, dtype=torch.bool, device=q.device).triu(1)
    scores.masked_fill_(mask, float("-inf"))
    p = torch.softmax(scores, -1)
    return torch.matmul(p, v.float()).to(q.dtype)


def load_weights_dir(path: str, device="cuda") -> dict:
    """Every NIT0 / NIT1 ``<name>.bin`` in ``path`` as a device fp32 tensor keyed
    by ``<name>`` (model.cpp:50-57: the file stem keeps the dotted name, e.g.
    "layers.0.self_attn.q_proj.weight"). bf16 payloads are uploaded at 2 bytes
    per element and inflated on the device; Model then quantizes on the device."""
    names = sorted(f for f in os.listdir(path) if f.endswith(".bin"))
    if not names:
        raise RuntimeError(f"load_weights_dir: no .bin weights in {path}")
    return {f[:-4]: quant.load_nit(os.path.join(path, f), device) for f in names}


class Model:
    """Decoder whose projections and embedding run on libnq_hip.so.

    mode: quant.QuantMode of the projections (NONE keeps them dense torch fp32).
    act_dtype: activation dtype between ops (torch.float32 or torch.float16).
    """

    def __init__(self, cfg: Config, weights: dict, mode=quant.QuantMode.W8A8, device="cuda",
                 act_dtype=torch.float32, quantize_embed: bool = True, layers=None):
        self.cfg, self.mode, self.act_dtype = cfg, quant.QuantMode(mode), act_dtype
        self.device = torch.device(device)
        self.n_layers = cfg.layers if layers is None else layers
        dev = lambda t: t.to(self.device, torch.float32).contiguous()
        self.proj, self.bias, self.norm = {}, {}, {}
        # W8A8 fuses the projections that share an input: q|k|v and gate|up are
        # concatenated along the output rows (per-row quantization, so the codes
        # and scales equal the separate projections'), their activation quant is
        # fused into rmsnorm, and the down projection's into silu * up.
        self.fused = self.mode == quant.QuantMode.W8A8
        for li in range(self.n_layers):
            L = f"layers.{li}."
            groups = {p: (p,) for p in PROJ}
            if self.fused:
                groups = {"self_attn.qkv_proj": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
                          "self_attn.o_proj": ("self_attn.o_proj",),
                          "mlp.gate_up_proj": ("mlp.gate_proj", "mlp.up_proj"),
                          "mlp.down_proj": ("mlp.down_proj",)}
            for name, parts in groups.items():
                wt = torch.cat([dev(weights[L + p + ".weight"]) for p in parts], 0)
                q = quant.make_quantized(wt, self.mode)
                self.proj[L + name] = q if q is not None else wt
                del wt
            if cfg.qkv_bias:
                bs = {p: dev(weights[L + f"self_attn.{p}.bias"]) for p in ("q_proj", "k_proj", "v_proj")}
                if self.fused:
                    self.bias[L + "self_attn.qkv_proj"] = torch.cat([bs["q_proj"], bs["k_proj"], bs["v_proj"]])
                else:
                    for p, b in bs.items():
                        self.bias[L + f"self_attn.{p}"] = b
            for nme in ("input_layernorm", "post_attention_layernorm"):
                self.norm[L + nme] = dev(weights[L + nme + ".weight"])
        self.final_norm = dev(weights["norm.weight"])
        emb = dev(weights["embed_tokens.weight"])
        self.embed = quant.make_q8_embed(emb) if quantize_embed else emb
        # An untied checkpoint has its own output projection (model.cpp:148-150).
        self.head = self.embed
        if not cfg.tie_embeddings:
            hw = dev(weights["lm_head.weight"])
            self.head = quant.make_q8_embed(hw) if quantize_embed else hw
        self.cos, self.sin = rope_tables(cfg, self.device)

    def project(self, x: torch.Tensor, name: str) -> torch.Tensor:
        """model.cpp:209-215: one Weight::linear per projection."""
        w, b = self.proj[name], self.bias.get(name)
        if isinstance(w, torch.Tensor):
            y = torch.nn.functional.linear(x.float(), w, b)
        else:
            y = w.linear(x, b)
        return y.to(self.act_dtype)

    def embed_tokens(self, ids) -> torch.Tensor:
        if isinstance(self.embed, torch.Tensor):
            return self.embed[torch.as_tensor(list(ids), device=self.device)].to(self.act_dtype)
        return self.embed.gather(list(ids)).to(self.act_dtype)

    def lm_head(self, x: torch.Tensor) -> torch.Tensor:
        """model.cpp:290-296: the output projection (the tied embedding unless the
        model has its own lm_head), fp32 logits."""
        if isinstance(self.head, torch.Tensor):
            return torch.nn.functional.linear(x.float(), self.head)
        return quant.lm_head_linear(x, self.head.t, None, out_dtype=torch.float32)

    def gemm(self, xq_as, name: str) -> torch.Tensor:
        """W8A8 projection of activations quantized by a fused producer."""
        xq, a_s = xq_as
        return quant.gemm_w8a8(xq, a_s, self.proj[name].t, self.bias.get(name), out_dtype=self.act_dtype)

    def layer(self, x: torch.Tensor, li: int, pending=None):
        """One pre-norm decoder layer (model.cpp:166-190). In W8A8 mode the MLP
        output is returned unadded, as (x, y): the residual add joins the next
        norm (add_rmsnorm_quant); settle() adds a pending y. Other modes return x."""
        cfg, L = self.cfg, f"layers.{li}."
        s = x.shape[0]
        hq, hkv = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        if self.fused:
            if pending is None:
                xq = quant.rmsnorm_quant(x, self.norm[L + "input_layernorm"], cfg.eps)
            else:
                x, *xq = quant.add_rmsnorm_quant(x, pending, self.norm[L + "input_layernorm"], cfg.eps)
            qkv = self.gemm(tuple(xq), L + "self_attn.qkv_proj")
            q, k, v = rope_qkv(qkv, cfg.heads, cfg.kv_heads, cfg.head_dim, self.cos, self.sin)
        else:
            h = rmsnorm(x, self.norm[L + "input_layernorm"], cfg.eps)
            q = self.project(h, L + "self_attn.q_proj").reshape(s, cfg.heads, cfg.head_dim).transpose(0, 1)
            k = self.project(h, L + "self_attn.k_proj").reshape(s, cfg.kv_heads, cfg.head_dim).transpose(0, 1)
            v = self.project(h, L + "self_attn.v_proj").reshape(s, cfg.kv_heads, cfg.head_dim).transpose(0, 1)
            q, k = apply_rope(q, self.cos, self.sin), apply_rope(k, self.cos, self.sin)
        a = attention(q, k, v, cfg.n_rep)
        if self.fused:
            o = self.gemm(quant.act_quant_heads(a.contiguous()), L + "self_attn.o_proj")
            x, *xq = quant.add_rmsnorm_quant(x, o, self.norm[L + "post_attention_layernorm"], cfg.eps)
            gu = self.gemm(tuple(xq), L + "mlp.gate_up_proj")
            i = cfg.intermediate
            return x, self.gemm(quant.silu_mul_quant(gu[:, :i], gu[:, i:]), L + "mlp.down_proj")
        a = a.transpose(0, 1).reshape(s, hq).contiguous()
        x = x + self.project(a, L + "self_attn.o_proj")
        hm = rmsnorm(x, self.norm[L + "post_attention_layernorm"], cfg.eps)
        gate = torch.nn.functional.silu(self.project(hm, L + "mlp.gate_proj").float())
        up = self.project(hm, L + "mlp.up_proj").float()
        return x + self.project((gate * up).to(self.act_dtype).contiguous(), L + "mlp.down_proj")

    @staticmethod
    def settle(out) -> torch.Tensor:
        """The residual stream after layer(): x, or x + the pending MLP output."""
        return out[0] + out[1] if isinstance(out, tuple) else out

    def run_layers(self, x: torch.Tensor) -> torch.Tensor:
        out = x
        for li in range(self.n_layers):
            out = self.layer(out[0], li, out[1]) if isinstance(out, tuple) else self.layer(out, li)
        return self.settle(out)

    def hidden(self, ids) -> torch.Tensor:
        """Final-norm hidden states [len(ids), hidden] for positions 0..len-1."""
        x = self.run_layers(self.embed_tokens(ids))
        return rmsnorm(x, self.final_norm, self.cfg.eps).contiguous()

    def forward(self, ids) -> torch.Tensor:
        """Logits [len(ids), vocab] (fp32, on the device) for positions 0..len-1."""
        return self.lm_head(self.hidden(ids))

    def next_token(self, ids) -> int:
        """Greedy pick for the last position (sampling.cpp:95). With the int8
        head the argmax is fused into the LM-head GEMV (no logits written)."""
        h = self.hidden(ids)[-1:]
        if isinstance(self.head, torch.Tensor):
            return int(torch.argmax(self.lm_head(h)[0]).item())
        return int(quant.lm_head_argmax(h, self.head.t)[0].item())

    @torch.no_grad()
    def generate(self, prompt, max_new: int) -> list:
        """Greedy decoding by full recompute; returns the new token ids."""
        ids = list(prompt)
        out = []
        for _ in range(max_new):
            nxt = self.next_token(ids)
            out.append(nxt)
            ids.append(nxt)
        return out
