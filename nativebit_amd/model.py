"""Packed NativeBit decoder: the reference's PackedGPT and its loader.

Mirrors inference/generate_torch.py:29-277 module for module: RMSNorm
(29-38), interleaved-pair RoPE (41-60), causal attention with a static KV
cache (63-106), SwiGLU (109-117), pre-norm blocks (120-132), a tied,
soft-capped LM head (135-162), ``load_packed_model`` (176-266) and
``init_kv_cache`` (269-277).  Every quantized linear is a PackedLinear on
the gfx950 kernels; the non-quantized arithmetic here is plain torch, in
fp32 as in the reference.  ``nativebit_amd.decode`` runs the same model as
fused HIP kernels for speed; this module is its functional statement.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import formats, synth
from .linear import PackedLinear


@dataclass
class ModelConfig:
    """TPU2BConfig's shape (configs/tpu.py:137-183)."""
    vocab_size: int = 50257
    n_layers: int = 26
    n_embd: int = 2560
    n_head: int = 20
    ffn_hidden: int = 6912
    context_len: int = 1024
    block_size: int = 128
    n_entries: int = 8
    rope_theta: float = 10000.0
    norm_eps: float = 1e-6


class RMSNorm(nn.Module):
    """x / sqrt(mean(x^2) + eps) * w, in fp32 (generate_torch.py:29-38)."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim), requires_grad=False)
        self.eps = eps

    def forward(self, x):
        dtype = x.dtype
        norm = torch.sqrt(x.float().pow(2).mean(-1, keepdim=True) + self.eps)
        return (x.float() / norm * self.weight.float()).to(dtype)


def precompute_rope(dim, max_len, theta=10000.0):
    """cos/sin tables (max_len, dim/2) in fp32 (generate_torch.py:41-45)."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    t = torch.arange(max_len, dtype=torch.float32)
    freqs = torch.outer(t, freqs)
    return torch.cos(freqs), torch.sin(freqs)


def apply_rope(q, k, cos, sin, pos_offset=0):
    """Rotation of (even, odd) pairs (generate_torch.py:48-60)."""
    dtype = q.dtype
    T = q.shape[2]
    cos = cos[pos_offset:pos_offset + T][None, None, :, :]
    sin = sin[pos_offset:pos_offset + T][None, None, :, :]
    cos2 = cos.repeat_interleave(2, dim=-1)
    sin2 = sin.repeat_interleave(2, dim=-1)

    def rotate(x):
        x1, x2 = x[..., ::2], x[..., 1::2]
        return torch.stack((-x2, x1), dim=-1).reshape(x.shape)

    q_rot = (q.float() * cos2 + rotate(q.float()) * sin2).to(dtype)
    k_rot = (k.float() * cos2 + rotate(k.float()) * sin2).to(dtype)
    return q_rot, k_rot


class CausalAttention(nn.Module):
    def __init__(self, n_embd, n_head, context_len, qkv, out_proj, theta=10000.0):
        super().__init__()
        self.n_head = n_head
        self.head_dim = n_embd // n_head
        self.qkv = qkv
        self.out_proj = out_proj
        cos, sin = precompute_rope(self.head_dim, context_len, theta)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    def forward(self, x, kv_cache=None, pos_offset=0):
        B, T, C = x.shape
        qkv = self.qkv(x)
        q, k, v = qkv.chunk(3, dim=-1)
        q = q.reshape(B, T, self.n_head, self.head_dim).transpose(1, 2)
        k = k.reshape(B, T, self.n_head, self.head_dim).transpose(1, 2)
        v = v.reshape(B, T, self.n_head, self.head_dim).transpose(1, 2)
        if kv_cache is not None:
            pos_offset = kv_cache[2]
        q, k = apply_rope(q, k, self.cos, self.sin, pos_offset)
        if kv_cache is not None:
            k_buf, v_buf, cache_len = kv_cache
            k_buf[:, :, cache_len:cache_len + T] = k
            v_buf[:, :, cache_len:cache_len + T] = v
            new_len = cache_len + T
            scale = self.head_dim ** -0.5
            # (b h q d) x (b h d k): batched matmul in fp32 on a contiguous
            # right operand
            attn = torch.matmul(q * scale, k_buf.transpose(-1, -2).contiguous())
            q_pos = cache_len + torch.arange(T, device=x.device)
            k_pos = torch.arange(k_buf.shape[2], device=x.device)
            mask = (k_pos[None, :] <= q_pos[:, None]) & (k_pos[None, :] < new_len)
            attn = attn.masked_fill(~mask[None, None], torch.finfo(attn.dtype).min)
            out = torch.matmul(F.softmax(attn, dim=-1), v_buf)
            new_cache = (k_buf, v_buf, new_len)
        else:
            out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
            new_cache = None
        out = out.transpose(1, 2).reshape(B, T, C)
        return self.out_proj(out), new_cache


class SwiGLU(nn.Module):
    def __init__(self, gate, up, down):
        super().__init__()
        self.gate, self.up, self.down = gate, up, down

    def forward(self, x):
        return self.down(F.silu(self.gate(x)) * self.up(x))


class TransformerBlock(nn.Module):
    def __init__(self, cfg: ModelConfig, lin: dict):
        super().__init__()
        self.ln1 = RMSNorm(cfg.n_embd, cfg.norm_eps)
        self.attn = CausalAttention(cfg.n_embd, cfg.n_head, cfg.context_len, lin["qkv"],
                                    lin["out_proj"], cfg.rope_theta)
        self.ln2 = RMSNorm(cfg.n_embd, cfg.norm_eps)
        self.ffn = SwiGLU(lin["gate"], lin["up"], lin["down"])

    def forward(self, x, kv_cache=None, pos_offset=0):
        attn_out, new_cache = self.attn(self.ln1(x), kv_cache, pos_offset=pos_offset)
        x = x + attn_out
        x = x + self.ffn(self.ln2(x))
        return x, new_cache


# order of a block's quantized linears (module order of generate_torch.py:
# qkv, out_proj, gate, up, down -- replace_linears walks them in this order)
LINEAR_NAMES = ("qkv", "out_proj", "gate", "up", "down")


class PackedGPT(nn.Module):
    """generate_torch.py:135-162 with PackedLinear layers."""

    def __init__(self, cfg: ModelConfig, linears: list, embedding: torch.Tensor):
        super().__init__()
        self.cfg = cfg
        self.n_layers = cfg.n_layers
        self.n_embd = cfg.n_embd
        self.n_head = cfg.n_head
        self.context_len = cfg.context_len
        self.embedding = nn.Embedding(embedding.shape[0], embedding.shape[1])
        self.embedding.weight = nn.Parameter(embedding, requires_grad=False)
        self.blocks = nn.ModuleList([TransformerBlock(cfg, lin) for lin in linears])
        self.ln_f = RMSNorm(cfg.n_embd, cfg.norm_eps)

    @torch.no_grad()
    def forward(self, idx, kv_caches=None, pos_offset=0):
        x = self.embedding(idx)
        new_caches = []
        for i, block in enumerate(self.blocks):
            cache = kv_caches[i] if kv_caches is not None else None
            x, new_cache = block(x, cache, pos_offset=pos_offset)
            new_caches.append(new_cache)
        x = self.ln_f(x)
        logits = x.to(self.embedding.weight.dtype) @ self.embedding.weight.T
        logits = 30.0 * torch.tanh(logits.float() / 30.0)
        if kv_caches is not None:
            return logits, new_caches
        return logits


def init_kv_cache(model: PackedGPT, batch_size=1, device="cuda", dtype=torch.float32):
    """Static per-layer K/V buffers (generate_torch.py:269-277)."""
    head_dim = model.n_embd // model.n_head
    caches = []
    for _ in range(model.n_layers):
        k = torch.zeros(batch_size, model.n_head, model.context_len, head_dim, device=device,
                        dtype=dtype)
        caches.append((k, torch.zeros_like(k), 0))
    return caches


@torch.no_grad()
def greedy_generate(model: PackedGPT, prompt_tokens, n_generate: int, device="cuda"):
    """Prefill the prompt, then decode greedily with the KV cache; returns
    the generated token ids (generate_torch.py:298-313)."""
    caches = init_kv_cache(model, device=device)
    x = torch.tensor([list(prompt_tokens)], dtype=torch.long, device=device)
    logits, caches = model(x, kv_caches=caches)
    token = int(logits[0, -1].argmax())
    out = []
    for _ in range(n_generate):
        out.append(token)
        x1 = torch.tensor([[token]], dtype=torch.long, device=device)
        logits, caches = model(x1, kv_caches=caches)
        token = int(logits[0, -1].argmax())
    return out


# ---------------------------------------------------------------------------
# construction
# ---------------------------------------------------------------------------

def load_packed_model(path: str, cfg: ModelConfig | None = None, device="cuda") -> PackedGPT:
    """Build a PackedGPT from a .nbpack.npz (generate_torch.py:176-266).

    Quantized layers are taken in natural-sorted key order, five per block
    (qkv, out_proj, gate, up, down); the embedding and norm weights come
    from ``params/embedding``, ``params/block_<i>/RMSNorm_<j>/weight`` and
    ``params/ln_f/weight`` when present (ones otherwise, as the reference's
    freshly built modules).
    """
    cfg = cfg or ModelConfig()
    pack = formats.load_nbpack(path)
    need = cfg.n_layers * len(LINEAR_NAMES)
    if len(pack.layers) < need:
        raise ValueError(f"{path}: {len(pack.layers)} quantized layers, {need} needed")
    it = iter(pack.layers)
    linears = []
    for _ in range(cfg.n_layers):
        linears.append({n: formats.packed_linear(next(it), device) for n in LINEAR_NAMES})
    emb = pack.params.get("params/embedding")
    if emb is None:
        raise ValueError(f"{path}: no params/embedding")
    model = PackedGPT(cfg, linears, torch.from_numpy(np.array(emb, dtype=np.float32)).to(device))
    for i, blk in enumerate(model.blocks):
        for j, name in enumerate(("ln1", "ln2")):
            w = pack.params.get(f"params/block_{i}/RMSNorm_{j}/weight")
            if w is not None:
                getattr(blk, name).weight.data = torch.from_numpy(
                    np.array(w, dtype=np.float32)).to(device)
    w = pack.params.get("params/ln_f/weight")
    if w is not None:
        model.ln_f.weight.data = torch.from_numpy(np.array(w, dtype=np.float32)).to(device)
    return model.to(device)


def random_packed_model(cfg: ModelConfig, seed: int = 0, device="cuda",
                        keep_indices: bool = False) -> PackedGPT:
    """Random-init packed model: every linear built as synth.make_layer
    (N(0, 0.02) latent weights, per-block quantile codebooks, nearest-entry
    indices), embedding N(0, 0.02), norm weights one."""
    linears = []
    shapes = {"qkv": (3 * cfg.n_embd, cfg.n_embd), "out_proj": (cfg.n_embd, cfg.n_embd),
              "gate": (cfg.ffn_hidden, cfg.n_embd), "up": (cfg.ffn_hidden, cfg.n_embd),
              "down": (cfg.n_embd, cfg.ffn_hidden)}
    for l in range(cfg.n_layers):
        lin = {}
        for j, name in enumerate(LINEAR_NAMES):
            N, K = shapes[name]
            lay = synth.make_layer(N, K, cfg.n_entries, cfg.block_size,
                                   seed=seed * 1000 + l * 10 + j, device=device,
                                   keep_indices=keep_indices)
            pl = PackedLinear(lay.packed, lay.codebook, N, K, block_size=cfg.block_size,
                              bits=lay.bits)
            if keep_indices:
                pl.indices = lay.indices
            lin[name] = pl
        linears.append(lin)
    gen = torch.Generator(device=torch.device(device)).manual_seed(seed + 7)
    emb = torch.randn(cfg.vocab_size, cfg.n_embd, generator=gen, device=device) * 0.02
    return PackedGPT(cfg, linears, emb).to(device)


def to_nbpack_params(model: PackedGPT) -> dict:
    """The model as .nbpack.npz contents (key -> array), in the layout
    load_packed_model reads; used to round-trip a model through a file."""
    out = {}
    for i, blk in enumerate(model.blocks):
        lin = [blk.attn.qkv, blk.attn.out_proj, blk.ffn.gate, blk.ffn.up, blk.ffn.down]
        names = ["CausalSelfAttention_0.NativeBitDense_0", "CausalSelfAttention_0.NativeBitDense_1",
                 "SwiGLU_0.NativeBitDense_0", "SwiGLU_0.NativeBitDense_1",
                 "SwiGLU_0.NativeBitDense_2"]
        for pl, n in zip(lin, names):
            p = f"params.block_{i}.{n}"
            nb = pl.codebook.shape[0]
            out[f"idx.{p}"] = pl.packed_indices.cpu().numpy()
            out[f"cb.{p}"] = pl.codebook.cpu().numpy()
            out[f"shape.{p}"] = np.array([pl.out_features, pl.in_features])
            out[f"idxshape.{p}"] = np.array([nb, pl.block_size])
        out[f"param.params.block_{i}.RMSNorm_0.weight"] = blk.ln1.weight.cpu().numpy()
        out[f"param.params.block_{i}.RMSNorm_1.weight"] = blk.ln2.weight.cpu().numpy()
    out["param.params.embedding"] = model.embedding.weight.cpu().numpy()
    out["param.params.ln_f.weight"] = model.ln_f.weight.cpu().numpy()
    n_q = 5 * len(model.blocks)
    out["__metadata__"] = np.array([model.cfg.block_size, model.cfg.n_entries, n_q,
                                    2 * len(model.blocks) + 2])
    return out


@torch.no_grad()
def benchmark(model: PackedGPT, prompt_tokens, n_generate=128, n_runs=3, device="cuda"):
    """Decode tokens/s with the KV cache (generate_torch.py:280-320)."""
    greedy_generate(model, prompt_tokens, 2, device)
    torch.cuda.synchronize()
    times = []
    for _ in range(n_runs):
        caches = init_kv_cache(model, device=device)
        x = torch.tensor([list(prompt_tokens)], dtype=torch.long, device=device)
        logits, caches = model(x, kv_caches=caches)
        torch.cuda.synchronize()
        token = int(logits[0, -1].argmax())
        t0 = time.time()
        for _ in range(n_generate):
            x1 = torch.tensor([[token]], dtype=torch.long, device=device)
            logits, caches = model(x1, kv_caches=caches)
            token = int(logits[0, -1].argmax())
        torch.cuda.synchronize()
        times.append(time.time() - t0)
    t = sum(times) / len(times)
    return {"generate_tps": round(n_generate / t, 1), "per_token_ms": round(t / n_generate * 1e3, 3)}
