"""CPU restatement of the reference's packed decoder -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and ``bench.py``'s ``cpu_baseline`` leg) may import this
module, as the checker.  It restates inference/generate_torch.py:29-162 and
269-320 in fp32 torch on the CPU, with every packed linear expanded to its
dense weight through the oracle's exact gather (``oracle.dequant``):

* ``PackedRef`` linears (packed stream, codebook): W[r, c] =
  cb[(r*K + c) // BS][index], the gather of triton_kernel.py:268-273,
  expanded when a forward pass uses them (``keep_dense`` keeps the expansion
  for small models), so a 2.2B-shaped model holds its packed bytes (1.3 GB)
  rather than 8.2 GB of fp32 weights;
* ``forward(idx, caches, pos)`` with the KV-cache path (generate_torch.py:
  80-98) or, without caches, causal attention over the whole sequence;
* ``greedy(prompt, n)``: the benchmark loop's greedy continuation
  (generate_torch.py:298-313).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import oracle as O


def dense_weight(packed, codebook, out_f, in_f, block_size=128, bits=3) -> torch.Tensor:
    """fp32 (out_f, in_f) weight by the exact gather."""
    p = np.asarray(packed, dtype=np.uint8)
    cb = np.asarray(codebook, dtype=np.float32)
    total = out_f * in_f
    idx = O.unpack(p, cb.shape[0] * block_size, bits)
    return torch.from_numpy(O.dequant(idx, cb, block_size, total).reshape(out_f, in_f))


class PackedRef:
    """A packed linear on the host: its stream and codebook, expanded to the
    dense fp32 weight by ``dense()`` (the reference's per-call gather,
    triton_kernel.py:258-273)."""

    def __init__(self, packed, codebook, out_f, in_f, block_size=128, bits=3, keep_dense=False):
        self.packed = np.ascontiguousarray(packed, dtype=np.uint8)
        self.codebook = np.ascontiguousarray(codebook, dtype=np.float32)
        self.out_f, self.in_f = int(out_f), int(in_f)
        self.block_size, self.bits = int(block_size), int(bits)
        self.keep_dense = keep_dense
        self._w = None

    def dense(self) -> torch.Tensor:
        if self._w is not None:
            return self._w
        w = dense_weight(self.packed, self.codebook, self.out_f, self.in_f, self.block_size,
                         self.bits)
        if self.keep_dense:
            self._w = w
        return w


def rmsnorm(x, w, eps):
    norm = torch.sqrt(x.float().pow(2).mean(-1, keepdim=True) + eps)
    return x.float() / norm * w.float()


def rope_tables(dim, max_len, theta=10000.0):
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    t = torch.arange(max_len, dtype=torch.float32)
    f = torch.outer(t, freqs)
    return torch.cos(f), torch.sin(f)


def rope(x, cos, sin, pos0):
    T = x.shape[2]
    c = cos[pos0:pos0 + T][None, None].repeat_interleave(2, dim=-1)
    s = sin[pos0:pos0 + T][None, None].repeat_interleave(2, dim=-1)
    x1, x2 = x[..., ::2], x[..., 1::2]
    rot = torch.stack((-x2, x1), dim=-1).reshape(x.shape)
    return x * c + rot * s


class DecoderRef:
    """The packed decoder on the CPU in fp32 (linears expanded per use)."""

    def __init__(self, cfg, layers, embedding, norms, ln_f):
        """layers: per block dict name -> (out, in) fp32 weight or PackedRef
        for qkv, out_proj, gate, up, down; norms: per block (ln1 w, ln2 w)."""
        self.cfg = cfg
        self.layers = layers
        self.emb = embedding.float()
        self.norms = norms
        self.ln_f = ln_f.float()
        self.D = cfg.n_embd // cfg.n_head
        self.cos, self.sin = rope_tables(self.D, cfg.context_len, cfg.rope_theta)

    @classmethod
    def from_model(cls, model, n_layers=None, keep_dense=None):
        """Host copy of a nativebit_amd.model.PackedGPT: packed streams and
        codebooks read back from its buffers (the first ``n_layers`` blocks
        when given).  ``keep_dense`` (default: models of <= 64M weights) keeps
        each expanded weight after its first use."""
        blocks = list(model.blocks)[:n_layers] if n_layers is not None else list(model.blocks)
        if keep_dense is None:
            n_w = sum(pl.out_features * pl.in_features for blk in blocks
                      for pl in (blk.attn.qkv, blk.attn.out_proj, blk.ffn.gate, blk.ffn.up,
                                 blk.ffn.down))
            keep_dense = n_w <= (64 << 20)
        layers, norms = [], []
        for blk in blocks:
            lin = {}
            for name, pl in (("qkv", blk.attn.qkv), ("out_proj", blk.attn.out_proj),
                             ("gate", blk.ffn.gate), ("up", blk.ffn.up), ("down", blk.ffn.down)):
                lin[name] = PackedRef(pl.packed_indices.cpu().numpy(), pl.codebook.cpu().numpy(),
                                      pl.out_features, pl.in_features, pl.block_size, pl.bits,
                                      keep_dense=keep_dense)
            layers.append(lin)
            norms.append((blk.ln1.weight.detach().cpu().float(), blk.ln2.weight.detach().cpu().float()))
        cfg = model.cfg
        if n_layers is not None:
            import dataclasses
            cfg = dataclasses.replace(cfg, n_layers=len(blocks))
        return cls(cfg, layers, model.embedding.weight.detach().cpu().float(), norms,
                   model.ln_f.weight.detach().cpu().float())

    def init_cache(self):
        c = self.cfg
        return [(torch.zeros(1, c.n_head, c.context_len, self.D),
                 torch.zeros(1, c.n_head, c.context_len, self.D)) for _ in range(c.n_layers)], 0

    @torch.no_grad()
    def forward(self, idx, cache=None, pos0=0, weight_dtype=None, act_dtype=None,
                head_dtype=None, accum_dtype=torch.float32):
        """Logits (B, T, V).  With ``cache`` = (per-layer (k, v), length) the
        cache path is used and updated in place; weight_dtype/act_dtype
        (e.g. torch.bfloat16) round linear weights / inputs, head_dtype the
        final hidden state and the tied embedding of the head, to emulate a
        reduced-precision path (products and sums stay fp32).
        ``accum_dtype`` = torch.float64 computes the linears' sums in fp64
        (rounded back to fp32): the spread between the two is the rounding
        noise a different fp32 summation order leaves in the logits."""
        c = self.cfg
        x = self.emb[idx]
        T = x.shape[1]

        def lin(v, w):
            if isinstance(w, PackedRef):
                w = w.dense()
            if weight_dtype is not None:
                w = w.to(weight_dtype).float()
            if act_dtype is not None:
                v = v.to(act_dtype).float()
            if accum_dtype != torch.float32:
                return (v.to(accum_dtype) @ w.to(accum_dtype).T).float()
            return v @ w.T

        p0 = pos0 if cache is None else cache[1]
        for l, L in enumerate(self.layers):
            kv = cache[0][l] if cache is not None else None
            x = self.block(l, x, lin, lambda h: self.attention(h, L, lin, kv, p0))
        if cache is not None:
            cache = (cache[0], cache[1] + T)
        x = rmsnorm(x, self.ln_f, c.norm_eps)
        e = self.emb
        if head_dtype is not None:
            x, e = x.to(head_dtype).float(), e.to(head_dtype).float()
        return self.head(x, e), cache

    # -- the pieces of a block, one method each (generate_torch.py:63-162) --

    def block(self, l, x, lin, attend):
        """x + attn(ln1(x)), then that + ffn(ln2(that))
        (TransformerBlock.forward, generate_torch.py:128-132)."""
        eps = self.cfg.norm_eps
        x = x + attend(rmsnorm(x, self.norms[l][0], eps))
        h2 = rmsnorm(x, self.norms[l][1], eps)
        return x + self.ffn(h2, self.layers[l], lin)

    def split_qkv(self, qkv):
        """q, k, v (B, H, T, D) from the fused projection's output (B, T, 3C):
        thirds in the order q | k | v, each split into heads
        (generate_torch.py:74-78)."""
        B, T, _ = qkv.shape
        H, D = self.cfg.n_head, self.D
        q, k, v = qkv.chunk(3, dim=-1)
        return tuple(t.reshape(B, T, H, D).transpose(1, 2) for t in (q, k, v))

    def rotate(self, x, p0):
        """RoPE at positions p0 .. p0 + T - 1 (generate_torch.py:48-60)."""
        return rope(x, self.cos, self.sin, p0)

    def attention(self, h, L, lin, kv, p0):
        """out_proj of causal softmax attention of the normed input h (B, T,
        C): with a cache kv = (keys, values) of (B, H, ctx, D) the rotated
        keys and the values are written at p0 .. p0 + T - 1 and every query
        sees the cache up to its own position (generate_torch.py:80-95);
        without one the T tokens attend to each other (the causal
        scaled_dot_product_attention branch, 97-101)."""
        B, T, C = h.shape
        D = self.D
        q, k, v = self.split_qkv(lin(h, L["qkv"]))
        q, k = self.rotate(q, p0), self.rotate(k, p0)
        if kv is not None:
            kb, vb = kv
            kb[:, :, p0:p0 + T] = k
            vb[:, :, p0:p0 + T] = v
            n = p0 + T
            att = (q * D ** -0.5) @ kb.transpose(-1, -2)
            qp = p0 + torch.arange(T)
            kp = torch.arange(kb.shape[2])
            mask = (kp[None, :] <= qp[:, None]) & (kp[None, :] < n)
            att = att.masked_fill(~mask[None, None], torch.finfo(att.dtype).min)
            o = F.softmax(att, dim=-1) @ vb
        else:
            att = (q * D ** -0.5) @ k.transpose(-1, -2)
            mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
            att = att.masked_fill(~mask[None, None], float("-inf"))
            o = F.softmax(att, dim=-1) @ v
        return lin(o.transpose(1, 2).reshape(B, T, C), L["out_proj"])

    def ffn(self, h2, L, lin):
        """down(silu(gate(h2)) * up(h2)) (SwiGLU.forward, generate_torch.py:
        116-117)."""
        return lin(F.silu(lin(h2, L["gate"])) * lin(h2, L["up"]), L["down"])

    def head(self, x, e):
        """Tied head with the soft cap: 30 tanh((x e^T) / 30)
        (generate_torch.py:158-160)."""
        return 30.0 * torch.tanh((x @ e.T) / 30.0)

    def dense_layer(self, l, weight_dtype=None):
        """Block l's linears as dense fp32 weights (rounded through
        weight_dtype when given)."""
        out = {}
        for name, w in self.layers[l].items():
            w = w.dense() if isinstance(w, PackedRef) else w
            out[name] = w.to(weight_dtype).float() if weight_dtype is not None else w
        return out

    @torch.no_grad()
    def layer_step(self, l, x, k_hist, v_hist, pos, weights=None, act_dtype=None):
        """One token through block l at position ``pos`` with the cache path
        (generate_torch.py:72-106, 120-132): x (C,) the fp32 residual stream
        in, k_hist / v_hist (H, pos, D) the rotated keys and the values of
        positions < pos, ``weights`` from dense_layer (rounded as wanted),
        act_dtype rounds the linears' inputs.  Returns (x out (C,), rotated
        key (H, D), value (H, D))."""
        c = self.cfg
        H, D = c.n_head, self.D
        W = weights if weights is not None else self.dense_layer(l)

        def lin(v, w):
            if act_dtype is not None:
                v = v.to(act_dtype).float()
            return v @ w.T

        ln1, ln2 = self.norms[l]
        h = rmsnorm(x, ln1, c.norm_eps)
        q, k, v = lin(h, W["qkv"]).reshape(3, 1, H, 1, D)
        q = rope(q, self.cos, self.sin, pos)[0]
        k = rope(k, self.cos, self.sin, pos)[0]
        v = v[0]
        keys = torch.cat([k_hist, k], dim=1)            # (H, pos + 1, D)
        vals = torch.cat([v_hist, v], dim=1)
        att = (q * D ** -0.5) @ keys.transpose(-1, -2)  # (H, 1, pos + 1)
        o = (F.softmax(att, dim=-1) @ vals).reshape(H * D)
        x1 = x + lin(o, W["out_proj"])
        h2 = rmsnorm(x1, ln2, c.norm_eps)
        x2 = x1 + self.ffn(h2, W, lin)
        return x2, k[:, 0], v[:, 0]

    @torch.no_grad()
    def greedy(self, prompt, n_generate):
        """Greedy continuation (generate_torch.py:298-313)."""
        cache = self.init_cache()
        logits, cache = self.forward(torch.tensor([list(prompt)]), cache)
        tok = int(logits[0, -1].argmax())
        out = []
        for _ in range(n_generate):
            out.append(tok)
            logits, cache = self.forward(torch.tensor([[tok]]), cache)
            tok = int(logits[0, -1].argmax())
        return out
