"""Packed NativeBit decoder: the reference's PackedGPT API on the gfx950
kernels, and its loader.

The classes and functions are those of inference/generate_torch.py:29-277,
with the reference's constructor signatures: ``RMSNorm(dim, eps)``,
``CausalAttention(n_embd, n_head, context_len, make_linear)``,
``SwiGLU(n_embd, ffn_hidden, make_linear)``,
``TransformerBlock(n_embd, n_head, ffn_hidden, context_len, make_linear)``,
``PackedGPT(vocab_size, n_layers, n_embd, n_head, ffn_hidden, context_len,
make_linear)`` (``make_linear(out_features, in_features)`` builds each linear),
``load_packed_model(path, config, device)`` with a ``TPU2BConfig``-shaped
config (configs/tpu.py:137-151), ``init_kv_cache(model, batch_size, device)``
and the ``forward(idx, kv_caches=None, pos_offset=0)`` contract.  The keyword
arguments after those (norm epsilon, RoPE base, format) default to the
reference's constants.

The arithmetic runs in this library's kernels: the packed linears are
PackedLinear (fused dequant-GEMV for up to 16 rows, the packed MFMA kernels or
a device gather + dense GEMM beyond), the norms nb_rmsnorm_rows (the residual
add fused into the second norm of a block), RoPE and the cache appends
nb_rope_kv_rows, attention nb_attention_rows, the SwiGLU product
nb_silu_pairs_rows.  Activations stay fp32 (the reference's module numerics);
``nativebit_amd.decode.DecodeEngine`` runs the same model with bf16 GEMV
inputs, one HIP graph per token, for speed.

KV caches: ``init_kv_cache`` returns the reference's shapes, keys and values
(B, H, ctx, head_dim).  The keys are a transposed view of (B, H, head_dim,
ctx) storage -- the layout the attention kernels read, 64 consecutive
positions per wave load -- so indexing them as the reference does
(``k_buf[:, :, :n]``) gives positions.  A cache built by the caller in the
reference's contiguous layout is accepted too: its keys are copied into the
kernel layout for the call and the new positions written back.
"""
from __future__ import annotations

import ctypes
import itertools
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn as nn

from . import _lib, formats, synth
from .linear import PackedLinear


@dataclass
class ModelConfig:
    """TPU2BConfig's shape (configs/tpu.py:137-151) plus the constants the
    reference's modules fix: RMSNorm eps 1e-6 (generate_torch.py:30) and the
    RoPE base 10000 (generate_torch.py:41)."""
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


def model_config(config) -> ModelConfig:
    """A ModelConfig from any object carrying TPU2BConfig's attribute names
    (configs/tpu.py:137-151: vocab_size, n_layers, n_embd, n_head,
    ffn_hidden, context_len, block_size, n_codebook).  Attributes the
    reference's config lacks take the reference modules' defaults: norm_eps
    1e-6, rope_theta 10000, n_entries = n_codebook (else 8)."""
    if isinstance(config, ModelConfig):
        return config
    missing = [a for a in ("vocab_size", "n_layers", "n_embd", "n_head", "ffn_hidden",
                           "context_len") if not hasattr(config, a)]
    if missing:
        raise ValueError(f"config lacks {', '.join(missing)}")
    n_entries = getattr(config, "n_entries", None)
    if n_entries is None:
        n_entries = getattr(config, "n_codebook", 8)
    return ModelConfig(vocab_size=int(config.vocab_size), n_layers=int(config.n_layers),
                       n_embd=int(config.n_embd), n_head=int(config.n_head),
                       ffn_hidden=int(config.ffn_hidden), context_len=int(config.context_len),
                       block_size=int(getattr(config, "block_size", 128)),
                       n_entries=int(n_entries),
                       rope_theta=float(getattr(config, "rope_theta", 10000.0)),
                       norm_eps=float(getattr(config, "norm_eps", 1e-6)))


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
            _p(rows), None, None, None, 0, _p(w), _p(out), _lib.NB_F32, rows.shape[0], C,
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


def _cache_storage(k_buf, v_buf, B, H, D):
    """Kernel-layout tensors for a cache given in the reference's shapes
    (B, H, ctx, D): keys [B][H][D][ctx] and values [B][H][ctx][D], both
    contiguous fp32.  Returns (keys, values, keys copied?, values copied?);
    a copy is made only where the caller's tensor is not already in that
    layout (init_kv_cache's tensors never are copied)."""
    for name, t in (("keys", k_buf), ("values", v_buf)):
        if t.dim() != 4 or t.shape[0] != B or t.shape[1] != H or t.shape[3] != D:
            raise ValueError(f"cache {name} must be (batch {B}, heads {H}, ctx, head_dim {D}); "
                             f"got {tuple(t.shape)}")
        if t.dtype != torch.float32:
            raise ValueError(f"cache {name} must be float32, got {t.dtype}")
    if v_buf.shape[2] != k_buf.shape[2]:
        raise ValueError(f"cache keys hold {k_buf.shape[2]} positions, values {v_buf.shape[2]}")
    kt = k_buf.transpose(-1, -2)
    k_copy = not kt.is_contiguous()
    v_copy = not v_buf.is_contiguous()
    return (kt.contiguous() if k_copy else kt, v_buf.contiguous() if v_copy else v_buf,
            k_copy, v_copy)


class CausalAttention(nn.Module):
    """Causal self-attention (generate_torch.py:63-106): the packed q|k|v and
    output projections (built by ``make_linear(out, in)``) around
    nb_rope_kv_rows (RoPE, cache append) and nb_attention_rows (masked
    softmax over the cache).

    With a cache (keys, values, length) the tokens take positions length ..
    length + T - 1 and attend to the cache, which is extended (pos_offset is
    ignored, as in the reference); without one the T tokens attend causally
    to each other only, rotated at positions pos_offset .. pos_offset + T - 1
    (the reference's scaled_dot_product_attention branch)."""

    def __init__(self, n_embd, n_head, context_len, make_linear, rope_theta=10000.0):
        super().__init__()
        self.n_head = n_head
        self.head_dim = n_embd // n_head
        self.context_len = context_len
        self.qkv = make_linear(3 * n_embd, n_embd)
        # the reference passes a dummy in_features here (its loader replaces
        # the module); this one asks for the real shape
        self.out_proj = make_linear(n_embd, n_embd)
        cos, sin = precompute_rope(self.head_dim, context_len, rope_theta)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    def forward(self, x, kv_cache=None, pos_offset=0):
        B, T, C = x.shape
        H, D = self.n_head, self.head_dim
        dev = x.device
        qkv = self.qkv(x).reshape(B, T, 3 * C).to(torch.float32).contiguous()
        cos, sin = self.cos.to(dev).contiguous(), self.sin.to(dev).contiguous()
        if kv_cache is not None:
            k_buf, v_buf, pos0 = kv_cache
            pos0 = int(pos0)
            kt, vt, k_copy, v_copy = _cache_storage(k_buf, v_buf, B, H, D)
            ctx, first = k_buf.shape[2], pos0
            if pos0 < 0 or pos0 + T > ctx:
                raise ValueError(f"positions {pos0}..{pos0 + T - 1} outside a cache of {ctx}")
        else:
            # the T tokens alone: a scratch cache of T positions, RoPE tables
            # read from row pos_offset on
            kt = torch.zeros(B, H, D, T, device=dev)
            vt = torch.zeros(B, H, T, D, device=dev)
            pos0, ctx, first = 0, T, int(pos_offset)
        if first < 0 or first + T > cos.shape[0]:
            raise ValueError(f"positions up to {first + T} exceed the RoPE tables "
                             f"({cos.shape[0]})")
        cos_t, sin_t = cos[first - pos0:], sin[first - pos0:]
        q = torch.empty(T, C, device=dev)
        att = torch.empty(B, T, C, device=dev)
        lib, s = _lib.load(), _stream(dev)
        for b in range(B):
            _lib.check(lib.nb_rope_kv_rows(_p(qkv[b]), _p(kt[b]), _p(vt[b]), _p(cos_t),
                                           _p(sin_t), pos0, T, _p(q), H, D, ctx, s))
            _lib.check(lib.nb_attention_rows(_p(q), _p(kt[b]), _p(vt[b]), pos0, T,
                                             _p(att[b]), _lib.NB_F32, H, D, ctx, s))
        out = self.out_proj(att)
        if kv_cache is None:
            return out, None
        if k_copy:
            k_buf[:, :, pos0:pos0 + T] = kt[..., pos0:pos0 + T].transpose(-1, -2)
        if v_copy:
            v_buf[:, :, pos0:pos0 + T] = vt[:, :, pos0:pos0 + T]
        return out, (k_buf, v_buf, pos0 + T)


class SwiGLU(nn.Module):
    """down(silu(gate(x)) * up(x)) (generate_torch.py:109-117); the product is
    nb_silu_pairs_rows over the gate and up outputs side by side."""

    def __init__(self, n_embd, ffn_hidden, make_linear):
        super().__init__()
        self.gate = make_linear(ffn_hidden, n_embd)
        self.up = make_linear(ffn_hidden, n_embd)
        self.down = make_linear(n_embd, ffn_hidden)

    def forward(self, x):
        g, u = self.gate(x), self.up(x)
        F = g.shape[-1]
        pairs = torch.stack((g.float(), u.float()), dim=-1).reshape(-1, 2 * F).contiguous()
        act = torch.empty(pairs.shape[0], F, device=x.device)
        _lib.check(_lib.load().nb_silu_pairs_rows(_p(pairs), _p(act), _lib.NB_F32,
                                                  pairs.shape[0], F, _stream(x.device)))
        prod_dtype = torch.promote_types(g.dtype, u.dtype)
        return self.down(act.reshape(*g.shape[:-1], F).to(prod_dtype))


class TransformerBlock(nn.Module):
    """Pre-norm block (generate_torch.py:120-132): x + attn(ln1(x)), then
    + ffn(ln2(.)); the attention's residual add and the second norm are one
    nb_rmsnorm_rows (add form).  Sums take the promoted dtype of their
    operands, as torch's ``x + y`` does in the reference."""

    def __init__(self, n_embd, n_head, ffn_hidden, context_len, make_linear, *,
                 norm_eps=1e-6, rope_theta=10000.0):
        super().__init__()
        self.ln1 = RMSNorm(n_embd, norm_eps)
        self.attn = CausalAttention(n_embd, n_head, context_len, make_linear, rope_theta)
        self.ln2 = RMSNorm(n_embd, norm_eps)
        self.ffn = SwiGLU(n_embd, ffn_hidden, make_linear)

    def forward(self, x, kv_cache=None, pos_offset=0):
        C = x.shape[-1]
        a, new_cache = self.attn(self.ln1(x), kv_cache, pos_offset=pos_offset)
        x1_dtype = torch.promote_types(x.dtype, a.dtype)
        res = x.reshape(-1, C).to(torch.float32, copy=True)   # becomes x + a (a fresh copy)
        h = torch.empty_like(res)
        w2 = self.ln2.weight.detach().to(torch.float32).contiguous()
        _lib.check(_lib.load().nb_rmsnorm_rows(
            _p(res), _p(_rows(a, C)), None, None, 0, _p(w2), _p(h), _lib.NB_F32, res.shape[0], C,
            float(self.ln2.eps), _stream(x.device)))
        res = res.reshape(x.shape).to(x1_dtype)
        f = self.ffn(h.reshape(x.shape).to(x1_dtype))
        return res + f, new_cache


class PackedGPT(nn.Module):
    """The packed decoder (generate_torch.py:135-162): token embedding, the
    blocks, a final norm and the tied, soft-capped head 30 tanh(l / 30).

    The positional arguments are the reference's; ``make_linear(out, in)``
    builds every linear, in module order qkv, out_proj, gate, up, down per
    block.  Keyword extras: ``norm_eps``, ``rope_theta`` (the reference's
    fixed 1e-6 and 10000), ``block_size`` / ``n_entries`` (the packed
    format, recorded in ``cfg``) and ``device`` for the embedding and norms.
    Activations are fp32 through the packed linears (exact fp32 weights, the
    reference's module numerics); ``nativebit_amd.decode.DecodeEngine`` runs
    the same model on bf16 GEMV inputs for speed."""

    def __init__(self, vocab_size, n_layers, n_embd, n_head, ffn_hidden, context_len,
                 make_linear, *, norm_eps=1e-6, rope_theta=10000.0, block_size=128,
                 n_entries=8, device=None):
        super().__init__()
        self.cfg = ModelConfig(vocab_size=vocab_size, n_layers=n_layers, n_embd=n_embd,
                               n_head=n_head, ffn_hidden=ffn_hidden, context_len=context_len,
                               block_size=block_size, n_entries=n_entries,
                               rope_theta=rope_theta, norm_eps=norm_eps)
        self.n_layers = n_layers
        self.n_embd = n_embd
        self.n_head = n_head
        self.context_len = context_len
        self.embedding = nn.Embedding(vocab_size, n_embd, device=device)
        self.embedding.weight.requires_grad_(False)
        self.blocks = nn.ModuleList([
            TransformerBlock(n_embd, n_head, ffn_hidden, context_len, make_linear,
                             norm_eps=norm_eps, rope_theta=rope_theta)
            for _ in range(n_layers)])
        self.ln_f = RMSNorm(n_embd, norm_eps)
        if device is not None:
            self.blocks.to(device)
            self.ln_f.to(device)

    @classmethod
    def from_config(cls, config, make_linear, device=None) -> "PackedGPT":
        """Built from a ModelConfig or a TPU2BConfig-shaped object."""
        c = model_config(config)
        return cls(c.vocab_size, c.n_layers, c.n_embd, c.n_head, c.ffn_hidden, c.context_len,
                   make_linear, norm_eps=c.norm_eps, rope_theta=c.rope_theta,
                   block_size=c.block_size, n_entries=c.n_entries, device=device)

    @torch.no_grad()
    def forward(self, idx, kv_caches=None, pos_offset=0):
        """Logits (B, T, vocab) fp32 of tokens idx (B, T); with kv_caches
        (from init_kv_cache) the caches are read and extended and the new
        caches are returned too."""
        x = self.embedding(idx)
        caches = []
        for i, block in enumerate(self.blocks):
            x, c = block(x, kv_caches[i] if kv_caches is not None else None, pos_offset)
            caches.append(c)
        h = self.ln_f(x)
        emb = self.embedding.weight
        logits = 30.0 * torch.tanh((h.to(emb.dtype) @ emb.T).float() / 30.0)
        return (logits, caches) if kv_caches is not None else logits


def init_kv_cache(model: PackedGPT, batch_size=1, device="cuda", dtype=torch.float32):
    """Empty static caches, one (keys, values, length 0) per block, keys and
    values of the reference's shape (batch, heads, context_len, head_dim)
    fp32 (generate_torch.py:269-277).  The keys are a transposed view of
    (batch, heads, head_dim, context_len) storage, the attention kernels'
    layout, so the kernels read and extend them in place."""
    if dtype != torch.float32:
        raise ValueError("the caches are fp32")
    D = model.n_embd // model.n_head
    caches = []
    for _ in range(model.n_layers):
        k_store = torch.zeros(batch_size, model.n_head, D, model.context_len, device=device)
        v = torch.zeros(batch_size, model.n_head, model.context_len, D, device=device)
        caches.append((k_store.transpose(-1, -2), v, 0))
    return caches


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

# order of a block's quantized linears (module order of generate_torch.py:
# qkv, out_proj, gate, up, down -- replace_linears walks them in this order)
LINEAR_NAMES = ("qkv", "out_proj", "gate", "up", "down")


class UnloadedLinear(nn.Module):
    """Placeholder for a packed linear that a loader fills in (the reference
    builds nn.Linear placeholders, generate_torch.py:212-215; this one holds
    no weight)."""

    def __init__(self, out_features, in_features):
        super().__init__()
        self.out_features, self.in_features = int(out_features), int(in_features)

    def forward(self, x):
        raise RuntimeError("linear not loaded")

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}"


def _param(arr, device):
    """A file array as a device tensor of the file's dtype (the reference's
    ``torch.from_numpy(arr.copy()).to(device)``)."""
    return torch.from_numpy(np.array(arr, copy=True)).to(device)


def load_packed_model(packed_path: str, config=None, device="cuda") -> PackedGPT:
    """Build a PackedGPT from a .nbpack.npz (generate_torch.py:176-266).

    ``config`` is a TPU2BConfig (configs/tpu.py:137-151) or any object with
    its attribute names, or a ModelConfig (default: the 2.2B shape).  The
    model is built with placeholder linears, which are then replaced in
    module order (qkv, out_proj, gate, up, down per block) by the archive's
    quantized layers in natural-sorted key order (block_2 before block_10),
    as the reference's ``replace_linears`` does; each layer's shape is
    checked against its place.  The embedding and norm weights come from
    ``params/embedding``, ``params/block_<i>/RMSNorm_<j>/weight`` and
    ``params/ln_f/weight`` when present (ones otherwise, as the reference's
    freshly built modules), in the file's dtype.
    """
    cfg = model_config(config) if config is not None else ModelConfig()
    pack = formats.load_nbpack(packed_path)
    model = PackedGPT.from_config(cfg, UnloadedLinear, device=device)
    layers = iter(pack.layers)

    def replace_linears(module):
        for name, child in module.named_children():
            if isinstance(child, UnloadedLinear):
                entry = next(layers, None)
                if entry is None:
                    raise ValueError(f"{packed_path}: {len(pack.layers)} quantized layers, "
                                     f"{cfg.n_layers * len(LINEAR_NAMES)} needed")
                if tuple(entry.shape) != (child.out_features, child.in_features):
                    raise ValueError(f"{packed_path}: layer {entry.prefix} is {entry.shape}, "
                                     f"{name} needs ({child.out_features}, {child.in_features})")
                setattr(module, name, formats.packed_linear(entry, device))
            else:
                replace_linears(child)

    replace_linears(model)
    emb = pack.params.get("params/embedding")
    if emb is None:
        raise ValueError(f"{packed_path}: no params/embedding")
    model.embedding.weight = nn.Parameter(_param(emb, device), requires_grad=False)
    for i, blk in enumerate(model.blocks):
        for j, name in enumerate(("ln1", "ln2")):
            w = pack.params.get(f"params/block_{i}/RMSNorm_{j}/weight")
            if w is not None:
                getattr(blk, name).weight.data = _param(w, device)
    w = pack.params.get("params/ln_f/weight")
    if w is not None:
        model.ln_f.weight.data = _param(w, device)
    return model


def random_packed_model(cfg, seed: int = 0, device="cuda",
                        keep_indices: bool = False) -> PackedGPT:
    """Random-init packed model: every linear built as synth.make_layer
    (N(0, 0.02) latent weights, per-block quantile codebooks, nearest-entry
    indices; linear j of block l from seed * 1000 + l * 10 + j), embedding
    N(0, 0.02), norm weights one."""
    cfg = model_config(cfg)
    order = itertools.count()

    def make_linear(out_f, in_f):
        l, j = divmod(next(order), len(LINEAR_NAMES))
        lay = synth.make_layer(out_f, in_f, cfg.n_entries, cfg.block_size,
                               seed=seed * 1000 + l * 10 + j, device=device,
                               keep_indices=keep_indices)
        pl = PackedLinear(lay.packed, lay.codebook, out_f, in_f, block_size=cfg.block_size,
                          bits=lay.bits)
        if keep_indices:
            pl.indices = lay.indices
        return pl

    model = PackedGPT.from_config(cfg, make_linear, device=device)
    gen = torch.Generator(device=torch.device(device)).manual_seed(seed + 7)
    emb = torch.randn(cfg.vocab_size, cfg.n_embd, generator=gen, device=device) * 0.02
    model.embedding.weight = nn.Parameter(emb, requires_grad=False)
    return model


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
