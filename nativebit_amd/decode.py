"""Greedy decode of a packed NativeBit model on the GPU, two ways.

Both run the model of ``nativebit_amd.model.PackedGPT`` (inference/
generate_torch.py:135-162) with the position and the current token in
device memory, so no token needs a host round trip (the reference
synchronises on ``int(logits.argmax())`` every token, generate_torch.py:311).

* ``DecodeEngine``: a token is a fixed sequence of gfx950 launches -- per
  layer q|k|v GEMV (RMSNorm formed in its prologue) -> nb_attention_step ->
  o GEMV (residual add in its epilogue) -> gate|up GEMV (RMSNorm prologue,
  silu(gate) * up of its row pairs in its epilogue) -> down GEMV (residual
  add epilogue), after the embedding lookup and before the final norm,
  head and greedy choice (nb_rmsnorm_lm_head_argmax, one launch) --
  captured once in a HIP graph and replayed.
* ``PersistentDecodeEngine``: nb_decode_persistent runs many tokens in one
  cooperative launch, the phases of a token separated by grid barriers and
  the packed weights of the next phases streamed during each barrier.

Numerics: the residual stream, norms, attention and KV cache are fp32 as in
the reference; the activations handed to the packed GEMVs are rounded to
bf16 (the bf16 path of inference/eval_ppl.py:149-174, with bf16-rounded
codebook entries and fp32 accumulation); the tied head reads a bf16 copy of
the embedding.  The prompt is fed through the same step with teacher
forcing.
"""
from __future__ import annotations

import ctypes
import time

import torch

from . import _lib, ops
from .model import PackedGPT, precompute_rope


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _interleave_rows(a, b):
    """One packed layer whose rows alternate a's row i and b's row i (same
    shape, K % 128 == 0 so a row is whole blocks): row 2i = a row i, row
    2i + 1 = b row i."""
    N, K = a.out_features, a.in_features
    rb = K // 128
    pa = a.packed_indices[: N * rb * 48].view(N, 1, rb * 48)
    pb = b.packed_indices[: N * rb * 48].view(N, 1, rb * 48)
    ca, cb = a.codebook.view(N, 1, rb, -1), b.codebook.view(N, 1, rb, -1)
    packed = torch.cat([pa, pb], dim=1).reshape(-1).contiguous()
    cbk = torch.cat([ca, cb], dim=1).reshape(2 * N * rb, -1).contiguous()
    return packed, cbk


def _fuse_rows(layers):
    """One packed layer holding the rows of several (same in_features, rows
    never share a block): streams and codebooks concatenated."""
    packed = torch.cat([l.packed_indices for l in layers]).contiguous()
    cb = torch.cat([l.codebook for l in layers]).contiguous()
    return packed, cb, sum(l.out_features for l in layers), layers[0].in_features


class _DecoderBase:
    """Device-resident state shared by the decode engines: fused weights,
    norms, caches, embedding copies, the decode state, forced and chosen
    tokens, and the whole-sequence API."""

    # row order of the fused gate|up layer: "stacked" (all gate rows, then
    # all up rows) or "interleaved" (gate row i, up row i, ...)
    _gu_rows = "stacked"

    def __init__(self, model: PackedGPT, max_steps: int | None = None):
        cfg = model.cfg
        dev = model.embedding.weight.device
        if dev.type != "cuda":
            raise ValueError(f"{type(self).__name__} runs on a ROCm GPU")
        self.model, self.cfg, self.dev = model, cfg, dev
        C, F, H = cfg.n_embd, cfg.ffn_hidden, cfg.n_head
        D = C // H
        self.C, self.F, self.H, self.D = C, F, H, D
        self.V = model.embedding.weight.shape[0]
        self.ctx = cfg.context_len
        self.max_steps = max_steps or cfg.context_len
        f32, bf16 = torch.float32, torch.bfloat16
        self._z = lambda *s, dt=f32: torch.zeros(*s, dtype=dt, device=dev)  # noqa: E731
        z = self._z
        self.logits = z(self.V)
        self.emb_f32 = model.embedding.weight.detach().to(f32).contiguous()
        self.emb_bf16 = self.emb_f32.to(bf16).contiguous()
        cos, sin = precompute_rope(D, self.ctx, cfg.rope_theta)
        self.cos, self.sin = cos.to(dev).contiguous(), sin.to(dev).contiguous()
        self.kc = z(cfg.n_layers, H, D, self.ctx)   # keys transposed: [layer][head][dim][pos]
        self.vc = z(cfg.n_layers, H, self.ctx, D)
        self.state_t = z(32, dt=torch.uint8)
        self.tokens = z(self.max_steps, dt=torch.int32)
        self.force = z(self.max_steps, dt=torch.int32)
        self.n_force = 0
        # per layer: fused q|k|v and gate|up streams (rows never share a
        # block, so the fused stream is the layers' streams concatenated)
        self.fused = []
        self.norms = []
        for blk in model.blocks:
            qkv_p, qkv_c, _, _ = _fuse_rows([blk.attn.qkv])
            if self._gu_rows == "interleaved":
                gu_p, gu_c = _interleave_rows(blk.ffn.gate, blk.ffn.up)
            else:
                gu_p, gu_c, _, _ = _fuse_rows([blk.ffn.gate, blk.ffn.up])
            o, dn = blk.attn.out_proj, blk.ffn.down
            self.fused.append(((qkv_p, qkv_c), (o.packed_indices, o.codebook), (gu_p, gu_c),
                               (dn.packed_indices, dn.codebook)))
            self.norms.append((blk.ln1.weight.detach().float().contiguous(),
                               blk.ln2.weight.detach().float().contiguous()))
        self.ln_f = model.ln_f.weight.detach().float().contiguous()
        self.eps = float(cfg.norm_eps)
        self.fed = 0

    # -- state ------------------------------------------------------------
    def reset(self, prompt_tokens):
        """Start a sequence: position 0, first prompt token fed, the rest
        forced."""
        prompt = [int(t) for t in prompt_tokens]
        if not prompt:
            raise ValueError("empty prompt")
        if min(prompt) < 0 or max(prompt) >= self.V:
            raise ValueError(f"prompt token outside 0..{self.V - 1}")
        if len(prompt) > self.max_steps:
            raise ValueError("prompt longer than max_steps")
        st = _lib.DecodeState(0, 0, prompt[0], 0, 0)
        host = torch.frombuffer(bytearray(bytes(st)), dtype=torch.uint8)
        self.state_t[: ctypes.sizeof(st)].copy_(host)
        self.n_force = len(prompt) - 1
        if self.n_force:
            self.force[: self.n_force].copy_(torch.tensor(prompt[1:], dtype=torch.int32))
        self.kc.zero_()
        self.vc.zero_()
        self.fed = 0

    def _advance(self, n):
        if self.fed + n > min(self.ctx, self.max_steps):
            raise ValueError(f"{self.fed} + {n} steps exceed the context ({self.ctx}) or "
                             f"max_steps ({self.max_steps})")
        self.fed += n

    def state(self) -> dict:
        st = _lib.DecodeState.from_buffer_copy(bytes(self.state_t[:24].cpu().numpy()))
        return {"pos": st.pos, "token": st.token, "step": st.step, "key": st.key, "done": st.done}

    def run(self, n_steps: int):
        raise NotImplementedError

    def _prepare_timing(self):
        """Work done once per timed run before the clock starts."""

    # -- whole sequences ----------------------------------------------------
    @torch.no_grad()
    def generate(self, prompt_tokens, n_generate: int) -> list:
        """Greedy continuation: the n_generate tokens the reference's loop
        produces (generate_torch.py:298-313)."""
        n_prompt = len(prompt_tokens)
        if n_prompt + n_generate > min(self.ctx, self.max_steps):
            raise ValueError("prompt + generated tokens exceed the context")
        self.reset(prompt_tokens)
        self.run(n_prompt + n_generate - 1)
        torch.cuda.synchronize()
        return self.tokens[n_prompt - 1: n_prompt - 1 + n_generate].cpu().tolist()

    @torch.no_grad()
    def benchmark(self, prompt_tokens, n_generate: int, n_runs: int = 3) -> dict:
        """Decode tokens/s after the prompt (timed like generate_torch.py:
        280-320: the prompt is fed first, then the continuation is timed)."""
        n_prompt = len(prompt_tokens)
        times = []
        for _ in range(n_runs):
            self.reset(prompt_tokens)
            self._prepare_timing()
            self.run(n_prompt)          # prompt (teacher forced) + first token chosen
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            self.run(n_generate - 1)    # the rest of the continuation
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        t = sorted(times)[len(times) // 2]
        return {"generate_tps": (n_generate - 1) / t, "per_token_ms": t / (n_generate - 1) * 1e3,
                "runs": len(times)}


class DecodeEngine(_DecoderBase):
    """Device-resident greedy decoder for one sequence (batch 1): one HIP
    graph of launches per token."""

    _gu_rows = "interleaved"   # the gate|up GEMV hands silu(gate) * up to down

    def __init__(self, model: PackedGPT, max_steps: int | None = None,
                 record_layers: bool = False, sel_layout: bool = True):
        """``record_layers``: after every layer the step also copies the
        residual stream into ``self.layer_x[l]`` (for layer-by-layer
        comparisons; one extra copy launch per layer).  ``sel_layout``: the
        step's GEMVs read copies of the index streams re-ordered into the
        selector-ordered unit layout (nb_stream_layout; less dequantization
        work, bit-identical outputs); the prompt pass keeps the originals."""
        super().__init__(model, max_steps)
        C, F, H = self.C, self.F, self.H
        self.layer_x = self._z(model.cfg.n_layers, C) if record_layers else None
        z, bf16 = self._z, torch.bfloat16
        self.x = z(C)                # residual stream (fp32)
        self.h = z(C, dt=bf16)       # normalised embedding row (layer 0's q|k|v input)
        self.qkv = z(3 * C)
        self.att = z(C, dt=bf16)
        self.act = z(F, dt=bf16)     # silu(gate) * up, the down projection's input
        self.work = z(int(_lib.load().nb_attention_work_floats(H)))
        self.done = z(H, dt=torch.int32)
        # Fused forms of the packed GEMVs (nb_batch_item x_mode / y_mode):
        # the norms, silu(gate) * up and the residual adds of the reference's
        # block (generate_torch.py:126-132) happen inside the GEMV launches.
        # Layer 0's q|k|v reads h, the normalised embedding row.
        eps = self.eps
        add = {"y": "add"}
        self.gemvs = []
        lay = "sel" if sel_layout else "rows"
        for l, ((qkv_p, qkv_c), (o_p, o_c), (gu_p, gu_c), (d_p, d_c)) in enumerate(self.fused):
            ln1, ln2 = self.norms[l]
            if sel_layout:
                qkv_p = ops.stream_layout(qkv_p, 3 * C, C)
                o_p = ops.stream_layout(o_p, C, C)
                gu_p = ops.stream_layout(gu_p, 2 * F, C)
                d_p = ops.stream_layout(d_p, C, F)
            qkv_item = ((self.h, qkv_p, qkv_c, self.qkv, 3 * C, C) if l == 0 else
                        (self.x, qkv_p, qkv_c, self.qkv, 3 * C, C, {"x": ("rmsnorm", ln1, eps)}))
            self.gemvs.append((
                ops.GemvBatch([qkv_item], layout=lay),
                ops.GemvBatch([(self.att, o_p, o_c, self.x, C, C, add)], layout=lay),
                ops.GemvBatch([(self.x, gu_p, gu_c, self.act, 2 * F, C,
                                {"x": ("rmsnorm", ln2, eps), "y": "silu_pairs"})], layout=lay),
                ops.GemvBatch([(self.act, d_p, d_c, self.x, C, F, add)], layout=lay),
            ))
        self.graph = None
        self._prompt_graphs = {}   # prompt length -> (graph, buffers) of the prompt pass

    def reset(self, prompt_tokens):
        super().reset(prompt_tokens)
        self.done.zero_()
        self.graph = None  # n_force is baked into the launch

    def _launch(self):
        lib = _lib.load()
        s = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        ck = _lib.check
        st = _ptr(self.state_t)
        C = self.C
        BF = _lib.NB_BF16
        # x = embedding[token], h = rmsnorm(x) * ln1 of layer 0
        ck(lib.nb_add_rmsnorm(_ptr(self.x), None, _ptr(self.emb_f32), st, _ptr(self.norms[0][0]),
                              _ptr(self.h), BF, C, self.eps, s))
        for l, (g_qkv, g_o, g_gu, g_d) in enumerate(self.gemvs):
            g_qkv.run()                      # qkv = W_qkv rmsnorm(x)
            ck(lib.nb_attention_step(_ptr(self.qkv), _ptr(self.kc[l]), _ptr(self.vc[l]),
                                     _ptr(self.cos), _ptr(self.sin), st, _ptr(self.work),
                                     _ptr(self.done), _ptr(self.att), BF, self.H, self.D,
                                     self.ctx, s))
            g_o.run()                        # x += W_o att
            g_gu.run()                       # act = silu(gate) * up of rmsnorm(x)
            g_d.run()                        # x += W_down act
            if self.layer_x is not None:
                self.layer_x[l].copy_(self.x)
        # the final norm, the tied head and the greedy choice in one launch
        ck(lib.nb_rmsnorm_lm_head_argmax(_ptr(self.x), _ptr(self.ln_f), self.eps,
                                         _ptr(self.emb_bf16), _ptr(self.logits), st,
                                         _ptr(self.tokens), self.max_steps, _ptr(self.force),
                                         self.n_force, self.V, C, s))

    def step(self):
        """Feed the current token (eagerly, no graph)."""
        self._advance(1)
        self._launch()

    @torch.no_grad()
    def prefill(self, prompt_tokens, graph: bool = True):
        """Feed the whole prompt as one batched pass -- the reference's
        prompt forward over T tokens (generate_torch.py:299-302) -- and choose
        the first generated token: per layer the q|k|v, o, gate|up and down
        matmuls are packed MFMA contractions over the T rows
        (nb_gemm_prefill_split: at T = 128 each layer's tile grid is small,
        so the kernel runs over K ranges with fp32 partials in a workspace),
        RoPE and the cache appends are nb_rope_kv_rows, causal attention is
        nb_attention_rows, and the norms with their residual adds are
        nb_rmsnorm_rows; the last row's final norm feeds nb_lm_head_argmax.
        Afterwards the state is that of the per-token path after the last
        prompt token, so run() continues the sequence.

        ``graph``: the pass's launches are captured once per prompt length
        (with buffers kept for that length) and replayed, so a prompt costs
        one graph launch instead of ~9 host launches per layer; False runs
        them eagerly."""
        prompt = [int(t) for t in prompt_tokens]
        self.reset(prompt)
        T = len(prompt)
        # the last prompt token's head writes tokens_out[T - 1] and leaves
        # position T, as the per-token path would; no layer reads the state
        st = _lib.DecodeState(0, T - 1, prompt[-1], T - 1, 0)
        self.state_t[: ctypes.sizeof(st)].copy_(torch.frombuffer(bytearray(bytes(st)),
                                                                  dtype=torch.uint8))
        toks = torch.tensor(prompt, dtype=torch.int32)
        if not graph:
            bufs = self._prompt_buffers(T)
            bufs["toks"].copy_(toks)
            self._prompt_launches(T, bufs)
        else:
            cached = self._prompt_graphs.get(T)
            if cached is None:
                if len(self._prompt_graphs) >= 4:   # keep the buffers of a few lengths
                    self._prompt_graphs.clear()
                bufs = self._prompt_buffers(T)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self._prompt_launches(T, bufs)
                cached = self._prompt_graphs[T] = (g, bufs)
            g, bufs = cached
            bufs["toks"].copy_(toks)
            g.replay()
        self.fed = T

    def _prompt_buffers(self, T):
        z, bf16, C, F = self._z, torch.bfloat16, self.C, self.F
        return {"toks": torch.zeros(T, dtype=torch.int32, device=self.dev),
                "x": z(T, C), "h": z(T, C, dt=bf16), "qkv": z(T, 3 * C), "q": z(T, C),
                "att": z(T, C, dt=bf16), "o": z(T, C), "gu": z(T, 2 * F),
                "act": z(T, F, dt=bf16), "dn": z(T, C)}

    def _prompt_launches(self, T, b):
        C, F, H, D = self.C, self.F, self.H, self.D
        lib, ck = _lib.load(), _lib.check
        s = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        BF = _lib.NB_BF16
        x, h, qkv, q, att, o, gu, act, dn = (b[k] for k in ("x", "h", "qkv", "q", "att", "o",
                                                              "gu", "act", "dn"))
        ln1 = [n[0] for n in self.norms]
        ck(lib.nb_rmsnorm_rows(_ptr(x), None, _ptr(self.emb_f32), _ptr(b["toks"]), self.V,
                               _ptr(ln1[0]), _ptr(h), BF, T, C, self.eps, s))
        for l, ((qkv_p, qkv_c), (o_p, o_c), (gu_p, gu_c), (d_p, d_c)) in enumerate(self.fused):
            ops.gemm_prefill(h, qkv_p, qkv_c, 3 * C, C, out=qkv)
            ck(lib.nb_rope_kv_rows(_ptr(qkv), _ptr(self.kc[l]), _ptr(self.vc[l]), _ptr(self.cos),
                                   _ptr(self.sin), 0, T, _ptr(q), H, D, self.ctx, s))
            ck(lib.nb_attention_rows(_ptr(q), _ptr(self.kc[l]), _ptr(self.vc[l]), 0, T, _ptr(att),
                                     BF, H, D, self.ctx, s))
            ops.gemm_prefill(att, o_p, o_c, C, C, out=o)
            ck(lib.nb_rmsnorm_rows(_ptr(x), _ptr(o), None, None, 0, _ptr(self.norms[l][1]),
                                   _ptr(h), BF, T, C, self.eps, s))
            ops.gemm_prefill(h, gu_p, gu_c, 2 * F, C, out=gu)  # gate, up columns interleaved
            ck(lib.nb_silu_pairs_rows(_ptr(gu), _ptr(act), BF, T, F, s))
            ops.gemm_prefill(act, d_p, d_c, C, F, out=dn)
            w_next = ln1[l + 1] if l + 1 < len(self.fused) else self.ln_f
            ck(lib.nb_rmsnorm_rows(_ptr(x), _ptr(dn), None, None, 0, _ptr(w_next), _ptr(h), BF,
                                   T, C, self.eps, s))
        ck(lib.nb_lm_head_argmax(_ptr(h[T - 1]), _ptr(self.emb_bf16), _ptr(self.logits),
                                 _ptr(self.state_t), _ptr(self.tokens), self.max_steps,
                                 _ptr(self.force), self.n_force, self.V, C, s))
        self.x.copy_(x[T - 1])

    @torch.no_grad()
    def generate(self, prompt_tokens, n_generate: int, batched_prompt: bool = True) -> list:
        """Greedy continuation (generate_torch.py:298-313): the prompt as one
        batched pass (or, with batched_prompt=False, fed token by token
        through the decode step), then one graph replay per token."""
        if not batched_prompt:
            return super().generate(prompt_tokens, n_generate)
        n_prompt = len(prompt_tokens)
        if n_prompt + n_generate > min(self.ctx, self.max_steps):
            raise ValueError("prompt + generated tokens exceed the context")
        self.prefill(prompt_tokens)
        self.run(n_generate - 1)
        torch.cuda.synchronize()
        return self.tokens[n_prompt - 1: n_prompt - 1 + n_generate].cpu().tolist()

    @torch.no_grad()
    def benchmark(self, prompt_tokens, n_generate: int, n_runs: int = 3) -> dict:
        """Decode tokens/s after the prompt (timed like generate_torch.py:
        280-320: the prompt pass first, then the continuation is timed), and
        the prompt pass's own time."""
        times, prompt_times = [], []
        for _ in range(n_runs):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            self.prefill(prompt_tokens)   # the prompt, batched; first token chosen
            torch.cuda.synchronize()
            prompt_times.append(time.perf_counter() - t0)
            if self.graph is None:
                self.capture()
            t0 = time.perf_counter()
            self.run(n_generate - 1)      # the rest of the continuation
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        t = sorted(times)[len(times) // 2]
        tp = sorted(prompt_times)[len(prompt_times) // 2]
        return {"generate_tps": (n_generate - 1) / t, "per_token_ms": t / (n_generate - 1) * 1e3,
                "prompt_ms": tp * 1e3, "prompt_tps": len(prompt_tokens) / tp,
                "runs": len(times)}

    def capture(self):
        """Capture one step in a HIP graph (replayed by run())."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._launch()
        self.graph = g

    def _prepare_timing(self):
        self.capture()

    def run(self, n_steps: int):
        self._advance(n_steps)
        if self.graph is None:
            self.capture()
        for _ in range(n_steps):
            self.graph.replay()


class PersistentDecodeEngine(_DecoderBase):
    """Device-resident greedy decoder for one sequence (batch 1): any number
    of tokens per launch of nb_decode_persistent."""

    def __init__(self, model: PackedGPT, max_steps: int | None = None, spin_limit: int = 0):
        raise _lib.NativeBitError(
            _lib.NB_EUNSUPPORTED,
            "PersistentDecodeEngine is switched off: nb_decode_persistent made an illegal "
            "memory access on a 26-layer model whose cause is not yet shown; use DecodeEngine")
        super().__init__(model, max_steps)
        self.spin_limit = int(spin_limit)
        rows = []
        for l, ((qkv_p, qkv_c), (o_p, o_c), (gu_p, gu_c), (d_p, d_c)) in enumerate(self.fused):
            ln1, ln2 = self.norms[l]
            rows.append([t.data_ptr() for t in (qkv_p, qkv_c, o_p, o_c, gu_p, gu_c, d_p, d_c,
                                                ln1, ln2, self.kc[l], self.vc[l])])
        # the device table of struct nb_decode_layer (12 pointers per layer)
        self.layer_table = torch.tensor(rows, dtype=torch.int64).to(self.dev)
        self.desc = _lib.DecodeModel(
            self.cfg.n_layers, self.C, self.H, self.D, self.F, self.V, self.ctx, self.eps,
            self.layer_table.data_ptr(), self.ln_f.data_ptr(), self.emb_f32.data_ptr(),
            self.emb_bf16.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr())
        lib = _lib.load()
        nbytes = int(lib.nb_decode_workspace_bytes(ctypes.byref(self.desc)))
        if nbytes <= 0:
            raise _lib.NativeBitError(_lib.NB_EUNSUPPORTED, _lib.last_error())
        self.workspace = self._z(nbytes, dt=torch.uint8)

    def run(self, n_steps: int):
        """Feed n_steps tokens in one launch (no synchronisation)."""
        if n_steps <= 0:
            return
        self._advance(n_steps)
        s = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        _lib.check(_lib.load().nb_decode_persistent(
            ctypes.byref(self.desc), _ptr(self.workspace), self.workspace.numel(),
            _ptr(self.state_t), _ptr(self.logits), _ptr(self.tokens), self.max_steps,
            _ptr(self.force), self.n_force, n_steps, self.spin_limit, s))

    def step(self):
        self.run(1)

    def error(self) -> int:
        """The launch's error word (synchronises): 0, or 1 when a grid
        barrier wait ran past the spin limit."""
        off = _lib.NB_DECODE_ERR_OFFSET
        return int(self.workspace[off: off + 4].view(torch.int32).item())

    @torch.no_grad()
    def generate(self, prompt_tokens, n_generate: int) -> list:
        toks = super().generate(prompt_tokens, n_generate)
        if self.error():
            raise _lib.NativeBitError(_lib.NB_ELAUNCH, "nb_decode_persistent: a grid barrier "
                                      "wait ran past its spin limit")
        return toks
