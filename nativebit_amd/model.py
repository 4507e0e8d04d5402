"""Packed NativeBit decoder: the reference's PackedGPT API on the gfx950
kernels, and its loader.

The module names, constructor arguments and forward signatures are those of
inference/generate_torch.py:29-277 (RMSNorm, precompute_rope / apply_rope,
CausalAttention with a static cache, SwiGLU, TransformerBlock, PackedGPT,
load_packed_model, init_kv_cache), so code written against the reference's
model runs unchanged.  The arithmetic runs in this library's kernels: the
packed linears are PackedLinear (fused dequant-GEMV for up to 16 rows, a
device gather + dense GEMM beyond), the norms nb_rmsnorm_rows (with the
residual add fused into the second norm of a block), RoPE and the cache
appends nb_rope_kv_rows, attention nb_attention_rows, the SwiGLU product
nb_silu_pairs_rows.  Activations stay fp32 (the reference's module
numerics); ``nativebit_amd.decode.DecodeEngine`` runs the same model with
bf16 GEMV inputs, one HIP graph per token, for speed.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn as nn

from . import _lib, formats, synth
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


def _stream(dev) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _rows(x: torch.Tensor, width: int) -> torch.Tensor:
    """x as contiguous fp32 rows of `width` (a copy when it is not already)."""
    return x.reshape(-1, width).to(torch.float32).contiguous()


class RMSNorm(nn.Module):
    """Root-mean-square norm of the last dimension times a weight, in fp32
    (generate_torch.py:29-38), by the row kernel nb_rmsnorm_rows; the result
    takes x's dtype."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim), requires_grad=False)
        self.eps = eps

    def forward(self, x):
        C = x.shape[-1]
        rows = _rows(x, C)
        out = torch.empty_like(rows)
        w = self.weight.detach().to(torch.float32).contiguous()
        _lib.check(_lib.load().nb_rmsnorm_rows(
            _p(rows), None, None, None, _p(w), _p(out), _lib.NB_F32, rows.shape[0], C,
            float(self.eps), _stream(x.device)))
        return out.reshape(x.shape).to(x.dtype)


def precompute_rope(dim, max_len, theta=10000.0):
    """cos / sin tables (max_len, dim / 2) fp32 of the angles pos * theta^(-2i
    / dim) -- the reference's fp32 arithmetic (generate_torch.py:41-45), so
    the rotations match it bit for bit."""
    inv = torch.arange(0, dim, 2, dtype=torch.float32).div(dim)
    inv = torch.pow(torch.tensor(theta, dtype=torch.float32), inv).reciprocal()
    ang = torch.arange(max_len, dtype=torch.float32).unsqueeze(1) * inv.unsqueeze(0)
    return ang.cos(), ang.sin()


def apply_rope(q, k, cos, sin, pos_offset=0):
    """Rotates each (even, odd) pair of the last dimension of q and k (B, H,
    T, D) by the angles of positions pos_offset .. pos_offset + T - 1
    (generate_torch.py:48-60), in fp32, results in the inputs' dtype."""
    T = q.shape[2]
    c = cos[pos_offset:pos_offset + T].to(q.device)
    s_ = sin[pos_offset:pos_offset + T].to(q.device)

    def turn(x):
        pairs = x.float().unflatten(-1, (-1, 2))
        a, b = pairs[..., 0], pairs[..., 1]
        return torch.stack((a * c - b * s_, b * c + a * s_), dim=-1).flatten(-2).to(x.dtype)

    return turn(q), turn(k)


class CausalAttention(nn.Module):
    """Causal self-attention over a static cache (generate_torch.py:63-106):
    the packed q|k|v and output projections around nb_rope_kv_rows (RoPE,
    cache append) and nb_attention_rows (masked softmax over the cache).
    A cache is (keys [B][H][D][ctx], values [B][H][ctx][D], length), the
    layout of the GPU decode step; without one the sequence attends to
    itself from position pos_offset on."""

    def __init__(self, n_embd, n_head, context_len, qkv, out_proj, theta=10000.0):
        super().__init__()
        self.n_head = n_head
        self.head_dim = n_embd // n_head
        self.context_len = context_len
        self.qkv = qkv
        self.out_proj = out_proj
        cos, sin = precompute_rope(self.head_dim, context_len, theta)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    def forward(self, x, kv_cache=None, pos_offset=0):
        B, T, C = x.shape
        H, D = self.n_head, self.head_dim
        dev = x.device
        qkv = self.qkv(x).reshape(B, T, 3 * C).to(torch.float32).contiguous()
        if kv_cache is not None:
            k_buf, v_buf, pos0 = kv_cache
            ctx = k_buf.shape[-1]
        else:
            pos0, ctx = pos_offset, pos_offset + T
            k_buf = torch.zeros(B, H, D, ctx, device=dev)
            v_buf = torch.zeros(B, H, ctx, D, device=dev)
        cos, sin = self.cos.to(dev).contiguous(), self.sin.to(dev).contiguous()
        if pos0 + T > cos.shape[0]:
            raise ValueError(f"positions up to {pos0 + T} exceed the RoPE tables")
        q = torch.empty(T, C, device=dev)
        att = torch.empty(B, T, C, device=dev)
        lib, s = _lib.load(), _stream(dev)
        for b in range(B):
            _lib.check(lib.nb_rope_kv_rows(_p(qkv[b]), _p(k_buf[b]), _p(v_buf[b]), _p(cos),
                                           _p(sin), pos0, T, _p(q), H, D, ctx, s))
            _lib.check(lib.nb_attention_rows(_p(q), _p(k_buf[b]), _p(v_buf[b]), pos0, T,
                                             _p(att[b]), _lib.NB_F32, H, D, ctx, s))
        out = self.out_proj(att)
        return out, ((k_buf, v_buf, pos0 + T) if kv_cache is not None else None)


class SwiGLU(nn.Module):
    """down(silu(gate(x)) * up(x)) (generate_torch.py:109-117); the product is
    nb_silu_pairs_rows over the gate and up outputs side by side."""

    def __init__(self, gate, up, down):
        super().__init__()
        self.gate, self.up, self.down = gate, up, down

    def forward(self, x):
        g, u = self.gate(x), self.up(x)
        F = g.shape[-1]
        pairs = torch.stack((g.float(), u.float()), dim=-1).reshape(-1, 2 * F).contiguous()
        act = torch.empty(pairs.shape[0], F, device=x.device)
        _lib.check(_lib.load().nb_silu_pairs_rows(_p(pairs), _p(act), _lib.NB_F32,
                                                  pairs.shape[0], F, _stream(x.device)))
        return self.down(act.reshape(*g.shape[:-1], F).to(x.dtype))


class TransformerBlock(nn.Module):
    """Pre-norm block (generate_torch.py:120-132): the attention's residual
    add and the second norm are one nb_rmsnorm_rows (add form)."""

    def __init__(self, cfg: ModelConfig, lin: dict):
        super().__init__()
        self.ln1 = RMSNorm(cfg.n_embd, cfg.norm_eps)
        self.attn = CausalAttention(cfg.n_embd, cfg.n_head, cfg.context_len, lin["qkv"],
                                    lin["out_proj"], cfg.rope_theta)
        self.ln2 = RMSNorm(cfg.n_embd, cfg.norm_eps)
        self.ffn = SwiGLU(lin["gate"], lin["up"], lin["down"])

    def forward(self, x, kv_cache=None, pos_offset=0):
        C = x.shape[-1]
        a, new_cache = self.attn(self.ln1(x), kv_cache, pos_offset=pos_offset)
        res = x.reshape(-1, C).to(torch.float32, copy=True)   # becomes x + a (a fresh copy)
        h = torch.empty_like(res)
        w2 = self.ln2.weight.detach().to(torch.float32).contiguous()
        _lib.check(_lib.load().nb_rmsnorm_rows(
            _p(res), _p(_rows(a, C)), None, None, _p(w2), _p(h), _lib.NB_F32, res.shape[0], C,
            float(self.ln2.eps), _stream(x.device)))
        f = self.ffn(h.reshape(x.shape).to(x.dtype))
        return (res.reshape(x.shape) + f.float()).to(x.dtype), new_cache


# order of a block's quantized linears (module order of generate_torch.py:
# qkv, out_proj, gate, up, down -- replace_linears walks them in this order)
LINEAR_NAMES = ("qkv", "out_proj", "gate", "up", "down")


class PackedGPT(nn.Module):
    """The packed decoder (generate_torch.py:135-162): token embedding, the
    blocks, a final norm and the tied, soft-capped head 30 tanh(l / 30).
    Activations are fp32 through the packed linears (exact fp32 weights, the
    reference's module numerics); ``nativebit_amd.decode.DecodeEngine`` runs
    the same model on bf16 GEMV inputs for speed."""

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
        """Logits (B, T, vocab) fp32 of tokens idx (B, T); with kv_caches
        (from init_kv_cache) the caches are read and extended and the new
        caches are returned too."""
        emb = self.embedding.weight
        x = emb.index_select(0, idx.reshape(-1)).reshape(*idx.shape, emb.shape[1]).float()
        caches = []
        for i, block in enumerate(self.blocks):
            x, c = block(x, kv_caches[i] if kv_caches is not None else None, pos_offset)
            caches.append(c)
        h = self.ln_f(x)
        logits = torch.tanh(h.to(emb.dtype) @ emb.t() / 30.0).float() * 30.0
        return (logits, caches) if kv_caches is not None else logits


def init_kv_cache(model: PackedGPT, batch_size=1, device="cuda", dtype=torch.float32):
    """Empty static caches, one (keys [B][H][D][ctx], values [B][H][ctx][D],
    length 0) per block -- the generate_torch.py:269-277 caches in the GPU
    decode step's layout (keys transposed); fp32 only."""
    if dtype != torch.float32:
        raise ValueError("the caches are fp32")
    D = model.n_embd // model.n_head
    shape_k = (batch_size, model.n_head, D, model.context_len)
    shape_v = (batch_size, model.n_head, model.context_len, D)
    return [(torch.zeros(shape_k, device=device), torch.zeros(shape_v, device=device), 0)
            for _ in range(model.n_layers)]


@torch.no_grad()
def greedy_generate(model: PackedGPT, prompt_tokens, n_generate: int, device="cuda"):
    """The reference's greedy loop (generate_torch.py:298-313) on the module
    forward: the prompt as one pass over the caches, then one token per
    pass, each the argmax of the last logits."""
    caches = init_kv_cache(model, device=device)
    logits, caches = model(torch.tensor([list(prompt_tokens)], device=device), kv_caches=caches)
    out = []
    for _ in range(n_generate):
        out.append(int(logits[0, -1].argmax()))
        if len(out) == n_generate:
            break
        logits, caches = model(torch.tensor([[out[-1]]], device=device), kv_caches=caches)
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


def benchmark(model: PackedGPT, prompt_tokens, n_generate=128, n_runs=3, device="cuda"):
    """Decode tokens/s (the measurement of generate_torch.py:280-320) on the
    device-resident decoder: the prompt as one batched pass, then one HIP
    graph replay per generated token."""
    from .decode import DecodeEngine
    eng = DecodeEngine(model, max_steps=len(prompt_tokens) + n_generate)
    r = eng.benchmark(prompt_tokens, n_generate, n_runs)
    return {"generate_tps": round(r["generate_tps"], 1), "per_token_ms": round(r["per_token_ms"], 3)}
