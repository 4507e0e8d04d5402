"""The CPU decode oracle (oracle/decode_ref.py) pinned by invariants.

* RoPE: identity at position 0, each (2i, 2i+1) pair keeps its norm, and
  the rotation angle is pos * theta^(-2i/D) (closed form).
* RMSNorm: a hand-computed example.
* The KV-cache path (token by token) equals attention over the whole
  sequence at once -- the reference's two paths (generate_torch.py:80-101).
* Greedy decoding is the argmax of the cached forward at each step.
"""
import math

import numpy as np
import torch

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
