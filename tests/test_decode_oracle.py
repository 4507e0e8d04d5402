"""The CPU decode oracle (oracle/decode_ref.py) pinned by invariants.

* RoPE: identity at position 0, each (2i, 2i+1) pair keeps its norm, and
  the rotation angle is pos * theta^(-2i/D) (closed form).
* RMSNorm: a hand-computed example.
* The KV-cache path (token by token) equals attention over the whole
  sequence at once -- the reference's two paths (generate_torch.py:80-101).
* Greedy decoding is the argmax of the cached forward at each step.
* Block composition: the oracle's logits equal a scalar closed form of the
  reference's decoder on tiny hand-built models (and two values worked out
  by hand), through both the whole-sequence and the cache path; each of 14
  planted slips (gate/up swapped, a residual dropped or misplaced, norm
  weights swapped, cap constant changed or dropped, head untied, RoPE sign
  or pair layout, k/v swapped, heads transposed, scale, causal mask) fails
  at least one of those checks.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nativebit_amd.model import ModelConfig
from oracle import decode_ref as R


def tiny_ref(seed=0, n_layers=2, C=64, H=4, F=128, V=50, ctx=32):
    cfg = ModelConfig(vocab_size=V, n_layers=n_layers, n_embd=C, n_head=H, ffn_hidden=F,
                      context_len=ctx)
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.2  # noqa: E731
    layers = [{"qkv": r(3 * C, C), "out_proj": r(C, C), "gate": r(F, C), "up": r(F, C),
               "down": r(C, F)} for _ in range(n_layers)]
    norms = [(1 + r(C), 1 + r(C)) for _ in range(n_layers)]
    return R.DecoderRef(cfg, layers, r(V, C) * 5, norms, 1 + r(C))


def test_rope_closed_form():
    D, T = 16, 10
    cos, sin = R.rope_tables(D, T)
    x = torch.randn(1, 1, T, D, dtype=torch.float64).float()
    y = R.rope(x, cos, sin, 0)
    assert torch.allclose(y[0, 0, 0], x[0, 0, 0])
    pairs_x = x.reshape(1, 1, T, D // 2, 2).norm(dim=-1)
    pairs_y = y.reshape(1, 1, T, D // 2, 2).norm(dim=-1)
    assert torch.allclose(pairs_x, pairs_y, rtol=1e-5, atol=1e-6)
    pos, i = 7, 3
    ang = pos * 10000.0 ** (-2 * i / D)
    a, b = float(x[0, 0, pos, 2 * i]), float(x[0, 0, pos, 2 * i + 1])
    assert math.isclose(float(y[0, 0, pos, 2 * i]), a * math.cos(ang) - b * math.sin(ang),
                        rel_tol=1e-5, abs_tol=1e-6)
    assert math.isclose(float(y[0, 0, pos, 2 * i + 1]), b * math.cos(ang) + a * math.sin(ang),
                        rel_tol=1e-5, abs_tol=1e-6)


def test_rmsnorm_hand_example():
    x = torch.tensor([[3.0, 4.0]])
    w = torch.tensor([1.0, 2.0])
    # mean(x^2) = 12.5, norm = sqrt(12.5 + 1e-6)
    n = math.sqrt(12.5 + 1e-6)
    assert torch.allclose(R.rmsnorm(x, w, 1e-6), torch.tensor([[3 / n, 8 / n]]))


def test_cache_path_equals_full_sequence():
    ref = tiny_ref()
    toks = torch.tensor([[3, 17, 5, 42, 8, 11, 0, 29]])
    full, _ = ref.forward(toks)
    cache = ref.init_cache()
    steps = []
    for t in range(toks.shape[1]):
        lg, cache = ref.forward(toks[:, t:t + 1], cache)
        steps.append(lg[0, 0])
    inc = torch.stack(steps)
    assert torch.allclose(inc, full[0], rtol=1e-4, atol=1e-5)
    # a prefill of 5 then single steps agrees too
    cache = ref.init_cache()
    lg5, cache = ref.forward(toks[:, :5], cache)
    assert torch.allclose(lg5[0], full[0, :5], rtol=1e-4, atol=1e-5)
    lg6, cache = ref.forward(toks[:, 5:6], cache)
    assert torch.allclose(lg6[0, 0], full[0, 5], rtol=1e-4, atol=1e-5)


def test_greedy_is_argmax_chain():
    ref = tiny_ref(seed=1)
    prompt = [1, 2, 3]
    out = ref.greedy(prompt, 5)
    seq = list(prompt)
    for tok in out:
        lg, _ = ref.forward(torch.tensor([seq]))
        assert int(lg[0, -1].argmax()) == tok
        seq.append(tok)


# ---------------------------------------------------------------------------
# Block composition pinned by closed forms on tiny hand-built models.
#
# ``scalar_logits`` evaluates the decoder of generate_torch.py:29-162 with
# plain Python floats, one scalar at a time (matrix-vector products as
# sums, the 2x2 rotation of each (2i, 2i+1) pair written out, the softmax
# as exp / sum), so it shares no code with the torch oracle.  The models
# are chosen so that each piece shows: zero attention weights isolate the
# SwiGLU path, distinct diagonal / permutation gate, up and down weights
# tell gate from up and W from W^T, distinct norm weights tell ln1 / ln2 /
# ln_f apart, embeddings of norm ~7 push the head into tanh's curved part
# (so the 30 of the soft cap matters), and two positions with non-trivial
# rotations give hand-checkable softmax weights.  The planted-mistake
# variants below (subclasses of the oracle with one plausible slip each)
# must fail at least one of these checks.
# ---------------------------------------------------------------------------

def _mv(W, x):
    return [sum(w * v for w, v in zip(row, x)) for row in W]


def _rms(x, w, eps=1e-6):
    r = math.sqrt(sum(v * v for v in x) / len(x) + eps)
    return [v / r * g for v, g in zip(x, w)]


def _silu(z):
    return z / (1.0 + math.exp(-z))


def _rot(vec, pos, theta=10000.0):
    D = len(vec)
    out = []
    for i in range(D // 2):
        a = pos * theta ** (-2.0 * i / D)
        x0, x1 = vec[2 * i], vec[2 * i + 1]
        out += [x0 * math.cos(a) - x1 * math.sin(a), x1 * math.cos(a) + x0 * math.sin(a)]
    return out


def scalar_logits(m, tokens, pos0=0):
    """Logits [t][v] of ``tokens`` as one causal sequence at positions pos0..
    (dict model m: C, H, emb, layers of lists, ln1/ln2 per layer, lnf)."""
    C, H = m["C"], m["H"]
    D = C // H
    xs = [list(m["emb"][t]) for t in tokens]
    for L, (g1, g2) in zip(m["layers"], m["norms"]):
        hs = [_rms(x, g1) for x in xs]
        qkv = [_mv(L["qkv"], h) for h in hs]
        q = [_rot_heads(r[:C], pos0 + t, H) for t, r in enumerate(qkv)]
        k = [_rot_heads(r[C:2 * C], pos0 + t, H) for t, r in enumerate(qkv)]
        v = [r[2 * C:] for r in qkv]
        outs = []
        for t in range(len(tokens)):
            o = []
            for hd in range(H):
                sl = slice(hd * D, (hd + 1) * D)
                s = [sum(a * b for a, b in zip(q[t][sl], k[j][sl])) / math.sqrt(D)
                     for j in range(t + 1)]
                mx = max(s)
                e = [math.exp(z - mx) for z in s]
                w = [z / sum(e) for z in e]
                o += [sum(w[j] * v[j][sl][d] for j in range(t + 1)) for d in range(D)]
            outs.append(o)
        xs = [[a + b for a, b in zip(x, _mv(L["out_proj"], o))] for x, o in zip(xs, outs)]
        h2s = [_rms(x, g2) for x in xs]
        acts = [[_silu(g) * u for g, u in zip(_mv(L["gate"], h), _mv(L["up"], h))] for h in h2s]
        xs = [[a + b for a, b in zip(x, _mv(L["down"], a_))] for x, a_ in zip(xs, acts)]
    hf = [_rms(x, m["lnf"]) for x in xs]
    return [[30.0 * math.tanh(sum(e * h for e, h in zip(row, hv)) / 30.0) for row in m["emb"]]
            for hv in hf]


def _rot_heads(vec, pos, H):
    D = len(vec) // H
    out = []
    for hd in range(H):
        out += _rot(vec[hd * D:(hd + 1) * D], pos)
    return out


def _as_ref(m, cls=R.DecoderRef, ctx=16):
    C, H = m["C"], m["H"]
    F = len(m["layers"][0]["gate"])
    cfg = ModelConfig(vocab_size=len(m["emb"]), n_layers=len(m["layers"]), n_embd=C, n_head=H,
                      ffn_hidden=F, context_len=ctx)
    t = lambda a: torch.tensor(a, dtype=torch.float32)  # noqa: E731
    layers = [{k: t(v) for k, v in L.items()} for L in m["layers"]]
    norms = [(t(a), t(b)) for a, b in m["norms"]]
    return cls(cfg, layers, t(m["emb"]), norms, t(m["lnf"]))


def _zeros(r, c):
    return [[0.0] * c for _ in range(r)]


def ffn_model():
    """One block, C = F = 2, one head: q|k|v and out_proj zero (attention adds
    nothing), gate / up diagonal with different entries, down a scaled
    permutation; embeddings of norm 5..7."""
    return {"C": 2, "H": 1,
            "emb": [[3.0, 4.0], [-5.0, 1.0], [2.0, -6.0], [0.5, 7.0]],
            "layers": [{"qkv": _zeros(6, 2), "out_proj": _zeros(2, 2),
                        "gate": [[1.5, 0.0], [0.0, -0.7]], "up": [[0.4, 0.0], [0.0, 2.0]],
                        "down": [[0.0, 3.0], [-2.0, 0.0]]}],
            "norms": [([1.0, 1.0], [0.8, 1.6])],
            "lnf": [1.25, 0.75]}


def attn_model():
    """One block, C = D = 4, one head: q, k, v, out_proj explicit; gate / up /
    down zero (SwiGLU adds nothing); distinct ln1 / ln_f weights."""
    qkv = [[1.0, 0.5, 0.0, -1.0], [0.0, 1.0, 2.0, 0.0], [0.5, 0.0, 1.0, 1.0], [-1.0, 1.0, 0.0, 0.5],
           [0.0, 2.0, -1.0, 0.0], [1.0, 0.0, 0.5, 0.5], [0.0, -1.0, 1.0, 2.0], [1.5, 0.0, 0.0, 1.0],
           [2.0, 0.0, 0.0, 0.0], [0.0, -3.0, 0.0, 0.0], [0.0, 0.0, 1.0, 0.0], [0.0, 0.0, 0.0, 4.0]]
    return {"C": 4, "H": 1,
            "emb": [[2.0, -1.0, 3.0, 0.5], [-1.5, 2.5, 0.0, 4.0], [3.0, 3.0, -2.0, -1.0]],
            "layers": [{"qkv": qkv, "out_proj": [[0.0, 1.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0],
                                                 [0.0, 0.0, 0.0, -1.0], [0.0, 0.0, 2.0, 0.0]],
                        "gate": _zeros(3, 4), "up": _zeros(3, 4), "down": _zeros(4, 3)}],
            "norms": [([1.0, 2.0, 0.5, 1.5], [1.0, 1.0, 1.0, 1.0])],
            "lnf": [2.0, 1.0, 1.5, 0.5]}


def random_model(seed, n_layers=2, C=4, H=2, F=6, V=5):
    """Small dense model with no structure, several layers and heads."""
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.normal(0, 0.6, s).tolist()  # noqa: E731
    return {"C": C, "H": H, "emb": (rng.normal(0, 2.5, (V, C))).tolist(),
            "layers": [{"qkv": r(3 * C, C), "out_proj": r(C, C), "gate": r(F, C),
                        "up": r(F, C), "down": r(C, F)} for _ in range(n_layers)],
            "norms": [((1 + rng.normal(0, 0.3, C)).tolist(), (1 + rng.normal(0, 0.3, C)).tolist())
                      for _ in range(n_layers)],
            "lnf": (1 + rng.normal(0, 0.3, C)).tolist()}


CASES = [("ffn", ffn_model, [0, 1, 2, 3], 0), ("attn", attn_model, [0, 1], 0),
         ("attn_pos", attn_model, [2, 0, 1], 3), ("random", lambda: random_model(4), [1, 3, 0, 4], 1),
         ("random1", lambda: random_model(9, n_layers=1, C=8, H=2, F=4), [2, 2, 1], 0)]


def _agree(ref_cls, name, build, toks, pos0, tol=2e-5):
    m = build()
    want = torch.tensor(scalar_logits(m, toks, pos0), dtype=torch.float64)
    ref = _as_ref(m, ref_cls)
    got, _ = ref.forward(torch.tensor([toks]), pos0=pos0)
    err = float((got[0].double() - want).abs().max())
    return err <= tol * max(1.0, float(want.abs().max())), err


def test_closed_form_hand_values():
    """Two entries worked out by hand from ffn_model (one token, position
    0; attention adds nothing): x = (3, 4) has rms sqrt(12.5), so ln2 gives
    (3, 4) / 3.53553 * (0.8, 1.6) = (0.67882, 1.81019); gate (1.01823,
    -1.26714), up (0.27153, 3.62039); silu(gate) * up = (0.20311, -1.00810);
    down swaps and scales: (3 * -1.00810, -2 * 0.20311) = (-3.02430,
    -0.40622); x2 = (-0.02430, 3.59378), rms 2.54124, ln_f gives (-0.01195,
    1.06064); the logit of token 0 is 30 tanh((3 * -0.01195 + 4 * 1.06064)
    / 30) = 30 tanh(4.20669 / 30) = 4.17934, of token 3 30 tanh(7.41848 /
    30) = 7.27087."""
    m = ffn_model()
    lg = scalar_logits(m, [0])[0]
    assert math.isclose(lg[0], 4.17934, abs_tol=2e-4), lg
    assert math.isclose(lg[3], 7.27087, abs_tol=2e-4), lg
    got, _ = _as_ref(m).forward(torch.tensor([[0]]))
    assert math.isclose(float(got[0, 0, 0]), 4.17934, abs_tol=2e-4)
    assert math.isclose(float(got[0, 0, 3]), 7.27087, abs_tol=2e-4)


def test_two_position_softmax_by_hand():
    """attn_model at positions 0 and 1: position 0 sees only itself, so its
    attention output is its own value vector; position 1's weights are the
    softmax of its two scores, which the scalar form computes -- checked here
    to sum to one and to differ from uniform (the rotation matters)."""
    m = attn_model()
    C = 4
    L = m["layers"][0]
    hs = [_rms(m["emb"][t], m["norms"][0][0]) for t in (0, 1)]
    qkv = [_mv(L["qkv"], h) for h in hs]
    q1 = _rot(qkv[1][:C], 1)
    ks = [_rot(qkv[0][C:2 * C], 0), _rot(qkv[1][C:2 * C], 1)]
    s = [sum(a * b for a, b in zip(q1, k)) / 2.0 for k in ks]
    w = [math.exp(z) / sum(math.exp(y) for y in s) for z in s]
    assert abs(sum(w) - 1) < 1e-12 and abs(w[0] - 0.5) > 0.05
    # without RoPE the scores would differ: the rotation by 1 radian moves them
    s_norot = [sum(a * b for a, b in zip(qkv[1][:C], qkv[j][C:2 * C])) / 2.0 for j in (0, 1)]
    assert abs(s_norot[0] - s[0]) > 1e-3
    full = scalar_logits(m, [0, 1])
    got, _ = _as_ref(m).forward(torch.tensor([[0, 1]]))
    assert torch.allclose(got[0].double(), torch.tensor(full, dtype=torch.float64), atol=1e-4)


@pytest.mark.parametrize("name,build,toks,pos0", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_closed_form(name, build, toks, pos0):
    ok, err = _agree(R.DecoderRef, name, build, toks, pos0)
    assert ok, (name, err)


@pytest.mark.parametrize("name,build,toks,pos0", CASES, ids=[c[0] for c in CASES])
def test_cache_path_matches_closed_form(name, build, toks, pos0):
    """The cache path, token by token from position 0, against the closed form."""
    m = build()
    want = torch.tensor(scalar_logits(m, toks, 0), dtype=torch.float64)
    ref = _as_ref(m)
    cache = ref.init_cache()
    rows = []
    for t in toks:
        lg, cache = ref.forward(torch.tensor([[t]]), cache)
        rows.append(lg[0, 0].double())
    assert torch.allclose(torch.stack(rows), want, atol=1e-4)


# -- planted mistakes: each variant must disagree with a closed form ---------

class SwapGateUp(R.DecoderRef):
    def ffn(self, h2, L, lin):
        return lin(F.silu(lin(h2, L["up"])) * lin(h2, L["gate"]), L["down"])


class DropAttnResidual(R.DecoderRef):
    def block(self, l, x, lin, attend):
        eps = self.cfg.norm_eps
        x = attend(R.rmsnorm(x, self.norms[l][0], eps))
        return x + self.ffn(R.rmsnorm(x, self.norms[l][1], eps), self.layers[l], lin)


class DropFfnResidual(R.DecoderRef):
    def block(self, l, x, lin, attend):
        eps = self.cfg.norm_eps
        x = x + attend(R.rmsnorm(x, self.norms[l][0], eps))
        return self.ffn(R.rmsnorm(x, self.norms[l][1], eps), self.layers[l], lin)


class FfnResidualFromBlockInput(R.DecoderRef):
    def block(self, l, x, lin, attend):
        eps = self.cfg.norm_eps
        x1 = x + attend(R.rmsnorm(x, self.norms[l][0], eps))
        return x + self.ffn(R.rmsnorm(x1, self.norms[l][1], eps), self.layers[l], lin)


class SwapNorms(R.DecoderRef):
    def block(self, l, x, lin, attend):
        eps = self.cfg.norm_eps
        x = x + attend(R.rmsnorm(x, self.norms[l][1], eps))
        return x + self.ffn(R.rmsnorm(x, self.norms[l][0], eps), self.layers[l], lin)


class CapConstant(R.DecoderRef):
    def head(self, x, e):
        return 50.0 * torch.tanh((x @ e.T) / 50.0)


class NoCap(R.DecoderRef):
    def head(self, x, e):
        return x @ e.T


class UntiedHead(R.DecoderRef):
    def head(self, x, e):
        return super().head(x, e.flip(0))


class RopeSignFlipped(R.DecoderRef):
    def rotate(self, x, p0):
        return R.rope(x, self.cos, -self.sin, p0)


class RopeHalfSplit(R.DecoderRef):
    def rotate(self, x, p0):
        T, D = x.shape[2], x.shape[-1]
        c = self.cos[p0:p0 + T][None, None].repeat(1, 1, 1, 2)
        s = self.sin[p0:p0 + T][None, None].repeat(1, 1, 1, 2)
        rot = torch.cat((-x[..., D // 2:], x[..., :D // 2]), dim=-1)
        return x * c + rot * s


class SwapKV(R.DecoderRef):
    def split_qkv(self, qkv):
        q, k, v = super().split_qkv(qkv)
        return q, v, k


class HeadsTransposed(R.DecoderRef):
    def split_qkv(self, qkv):
        B, T, _ = qkv.shape
        H, D = self.cfg.n_head, self.D
        q, k, v = qkv.chunk(3, dim=-1)
        return tuple(t.reshape(B, T, D, H).transpose(-1, -2).transpose(1, 2) for t in (q, k, v))


class NoScale(R.DecoderRef):
    def rotate(self, x, p0):
        # scores scaled by sqrt(D) on top of the 1/sqrt(D): the rotated q and k
        # each carry D^(1/4)
        return R.rope(x, self.cos, self.sin, p0) * self.D ** 0.25


class NoCausalMask(R.DecoderRef):
    def attention(self, h, L, lin, kv, p0):
        B, T, C = h.shape
        q, k, v = self.split_qkv(lin(h, L["qkv"]))
        q, k = self.rotate(q, p0), self.rotate(k, p0)
        o = F.softmax((q * self.D ** -0.5) @ k.transpose(-1, -2), dim=-1) @ v
        return lin(o.transpose(1, 2).reshape(B, T, C), L["out_proj"])


MUTANTS = [SwapGateUp, DropAttnResidual, DropFfnResidual, FfnResidualFromBlockInput, SwapNorms,
           CapConstant, NoCap, UntiedHead, RopeSignFlipped, RopeHalfSplit, SwapKV,
           HeadsTransposed, NoScale, NoCausalMask]


@pytest.mark.parametrize("cls", MUTANTS, ids=[c.__name__ for c in MUTANTS])
def test_planted_mistake_fails_closed_form(cls):
    failed = [name for name, build, toks, pos0 in CASES
              if not _agree(cls, name, build, toks, pos0)[0]]
    assert failed, f"{cls.__name__} passed every closed-form check"
