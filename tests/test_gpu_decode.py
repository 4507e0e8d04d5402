"""GPU parity of the decode path (run with -m gpu).

* nb_add_rmsnorm, nb_attention_step, nb_silu_mul, nb_lm_head_argmax against
  torch fp32 restatements of the reference's ops (generate_torch.py:29-117,
  157-159) on the same inputs;
* greedy argmax tie-breaking (first index, as torch.argmax) and teacher
  forcing;
* PackedGPT on the GPU (fp32 activations, the reference's numerics) against
  the CPU oracle decoder with dense weights: logits and greedy tokens;
* DecodeEngine (bf16 GEMV inputs) against the oracle with the same bf16
  rounding, step by step under teacher forcing, and its HIP-graph replays
  against its eager steps;
* a model written to .nbpack.npz and loaded back gives the same logits.
"""
import ctypes

import numpy as np
import pytest
import torch

from nativebit_amd import _lib, formats
from nativebit_amd.decode import DecodeEngine
from nativebit_amd.model import ModelConfig, load_packed_model, precompute_rope, random_packed_model
from oracle import decode_ref as R

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = torch.as_tensor(a).double().reshape(-1).cpu()
    b = torch.as_tensor(b).double().reshape(-1).cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


def P(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def state_tensor(dev, pos=0, token=0, step=0):
    st = _lib.DecodeState(0, pos, token, step, 0)
    t = torch.zeros(32, dtype=torch.uint8, device=dev)
    t[:24].copy_(torch.frombuffer(bytearray(bytes(st)), dtype=torch.uint8))
    return t


def read_state(t):
    return _lib.DecodeState.from_buffer_copy(bytes(t[:24].cpu().numpy()))


TINY = ModelConfig(vocab_size=1000, n_layers=2, n_embd=256, n_head=4, ffn_hidden=512,
                   context_len=64)


@pytest.fixture(scope="module")
def tiny_model(dev):
    return random_packed_model(TINY, seed=5, device=dev)


@pytest.fixture(scope="module")
def tiny_ref(tiny_model):
    return R.DecoderRef.from_model(tiny_model)


@pytest.mark.parametrize("mode", ["plain", "residual", "embed"])
@pytest.mark.parametrize("hdt", [torch.float32, torch.bfloat16])
def test_add_rmsnorm(dev, mode, hdt):
    note(f"add_rmsnorm {mode} {hdt}")
    lib = _lib.load()
    n = 2560
    g = torch.Generator().manual_seed(1)
    x0 = torch.randn(n, generator=g)
    y = torch.randn(n, generator=g)
    w = torch.randn(n, generator=g)
    emb = torch.randn(7, n, generator=g)
    st = state_tensor(dev, token=4)
    x = x0.to(dev)
    h = torch.empty(n, dtype=hdt, device=dev)
    yd = y.to(dev) if mode == "residual" else None
    ed = emb.to(dev) if mode == "embed" else None
    wd = w.to(dev)  # (device copies held in names: a temporary could be freed before the launch)
    _lib.check(lib.nb_add_rmsnorm(P(x), P(yd), P(ed), P(st), P(wd), P(h),
                                  _lib.NB_BF16 if hdt == torch.bfloat16 else _lib.NB_F32, n, 1e-6,
                                  stream()))
    xr = {"plain": x0, "residual": x0 + y, "embed": emb[4]}[mode]
    hr = R.rmsnorm(xr, w, 1e-6)
    assert torch.equal(x.cpu(), xr)
    assert rel(h.float(), hr) <= (4e-3 if hdt == torch.bfloat16 else 1e-6)


def torch_attention(qkv, kc, vc, pos, H, D, ctx):
    """One-token attention with the cache, as generate_torch.py:72-98."""
    C = H * D
    cos, sin = precompute_rope(D, ctx)
    q = qkv[:C].reshape(1, H, 1, D)
    k = qkv[C:2 * C].reshape(1, H, 1, D)
    v = qkv[2 * C:].reshape(1, H, 1, D)
    q, k = R.rope(q, cos, sin, pos), R.rope(k, cos, sin, pos)
    kc = kc.clone()
    vc = vc.clone()
    kc[:, pos] = k[0, :, 0]
    vc[:, pos] = v[0, :, 0]
    qs = q[0, :, 0] * D ** -0.5                                   # (H, D)
    att = (kc[:, :pos + 1] @ qs.unsqueeze(-1)).squeeze(-1)        # (H, pos+1)
    p = torch.softmax(att, dim=-1)
    out = (p.unsqueeze(1) @ vc[:, :pos + 1]).reshape(C)
    return out, kc, vc


@pytest.mark.parametrize("H,D,ctx", [(20, 128, 80), (4, 64, 80), (2, 32, 80), (20, 128, 1024),
                                     (3, 128, 300), (2, 128, 82)])
def test_attention_step(dev, H, D, ctx):
    lib = _lib.load()
    g = torch.Generator().manual_seed(H * 100 + D)
    kc = torch.randn(H, ctx, D, generator=g)
    vc = torch.randn(H, ctx, D, generator=g)
    cos, sin = precompute_rope(D, ctx)
    work = torch.zeros(int(lib.nb_attention_work_floats(H)), device=dev)
    done = torch.zeros(H, dtype=torch.int32, device=dev)
    kd, vd = kc.transpose(1, 2).contiguous().to(dev), vc.to(dev)   # keys [H][D][ctx]
    cosd, sind = cos.to(dev), sin.to(dev)
    # (tile edges of the 128-position tile kernel and of the 16-split kernels)
    for pos in sorted(p for p in {0, 1, 15, 16, 17, 63, 127, 128, 129, 255, 256, 257, 383, 384,
                                  511, 767, 768, 895, 896, ctx // 2, ctx - 1} if p < ctx):
        note(f"attention H={H} D={D} pos={pos}")
        qkv = torch.randn(3 * H * D, generator=g)
        qkvd = qkv.to(dev)
        st = state_tensor(dev, pos=pos)
        out = torch.empty(H * D, device=dev)
        _lib.check(lib.nb_attention_step(P(qkvd), P(kd), P(vd), P(cosd), P(sind), P(st), P(work),
                                         P(done), P(out), _lib.NB_F32, H, D, ctx, stream()))
        ref, kc, vc = torch_attention(qkv, kc, vc, pos, H, D, ctx)
        assert rel(out, ref) <= 1e-5, (pos, rel(out, ref))
        assert torch.allclose(kd.cpu().transpose(1, 2), kc, rtol=1e-6, atol=1e-6)
        assert torch.equal(vd.cpu(), vc)
        assert int(done.abs().sum()) == 0


def test_silu_mul(dev):
    lib = _lib.load()
    n = 6912
    gu = torch.randn(2 * n, generator=torch.Generator().manual_seed(3)) * 4
    gud = gu.to(dev)
    out = torch.empty(n, device=dev)
    _lib.check(lib.nb_silu_mul(P(gud), P(out), _lib.NB_F32, n, stream()))
    ref = torch.nn.functional.silu(gu[:n]) * gu[n:]
    assert rel(out, ref) <= 1e-6


def run_head(dev, h, emb, st, force=None, n_force=0, tokens=None):
    lib = _lib.load()
    V, C = emb.shape
    logits = torch.empty(V, device=dev)
    cap = tokens.numel() if tokens is not None else 0
    _lib.check(lib.nb_lm_head_argmax(P(h), P(emb), P(logits), P(st), P(tokens), cap, P(force),
                                     n_force, V, C, stream()))
    return logits


@pytest.mark.parametrize("V,C", [(32000, 2560), (1000, 256), (50257, 2560)])
def test_lm_head_argmax(dev, V, C):
    note(f"lm_head V={V} C={C}")
    g = torch.Generator().manual_seed(V)
    h = torch.randn(C, generator=g).to(torch.bfloat16)
    emb = (torch.randn(V, C, generator=g) * 0.5).to(torch.bfloat16)
    st = state_tensor(dev, pos=3, token=9, step=2)
    tokens = torch.full((8,), -1, dtype=torch.int32, device=dev)
    hd, ed = h.to(dev), emb.to(dev)
    logits = run_head(dev, hd, ed, st, tokens=tokens)
    ref = 30.0 * torch.tanh((emb.float() @ h.float()) / 30.0)
    assert rel(logits, ref) <= 1e-5
    s = read_state(st)
    best = int(logits.cpu().argmax())
    assert s.token == best and s.pos == 4 and s.step == 3 and s.key == 0 and s.done == 0
    assert int(tokens[2]) == best
    assert int(ref.argmax()) == best or float(ref.max() - ref[best]) < 1e-4


@pytest.mark.parametrize("V,C", [(32000, 2560), (1000, 256)])
def test_rmsnorm_lm_head_equals_two_launches(dev, V, C):
    """nb_rmsnorm_lm_head_argmax (the final norm formed inside the head's
    launch) gives the logits, token and state of nb_add_rmsnorm followed by
    nb_lm_head_argmax, bit for bit, with forcing and tokens_out as well."""
    note(f"rmsnorm + lm_head fused V={V} C={C}")
    lib = _lib.load()
    g = torch.Generator().manual_seed(V + C)
    x = (torch.randn(C, generator=g) * 3).to(dev)
    w = torch.randn(C, generator=g).to(dev)
    emb = (torch.randn(V, C, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    force = torch.tensor([11, 12], dtype=torch.int32, device=dev)
    eps = 1e-6
    for step, n_force in ((0, 2), (2, 2)):   # a forced step, then a free one
        st_a = state_tensor(dev, pos=5, token=1, step=step)
        st_b = state_tensor(dev, pos=5, token=1, step=step)
        tok_a = torch.full((4,), -1, dtype=torch.int32, device=dev)
        tok_b = tok_a.clone()
        h = torch.empty(C, dtype=torch.bfloat16, device=dev)
        la = torch.empty(V, device=dev)
        lb = torch.empty(V, device=dev)
        _lib.check(lib.nb_add_rmsnorm(P(x), None, None, P(st_a), P(w), P(h), _lib.NB_BF16, C, eps,
                                      stream()))
        _lib.check(lib.nb_lm_head_argmax(P(h), P(emb), P(la), P(st_a), P(tok_a), 4, P(force),
                                         n_force, V, C, stream()))
        _lib.check(lib.nb_rmsnorm_lm_head_argmax(P(x), P(w), eps, P(emb), P(lb), P(st_b), P(tok_b),
                                                 4, P(force), n_force, V, C, stream()))
        torch.cuda.synchronize()
        assert torch.equal(la, lb)
        assert torch.equal(tok_a, tok_b)
        sa, sb = read_state(st_a), read_state(st_b)
        assert (sa.token, sa.pos, sa.step, sa.key, sa.done) == \
            (sb.token, sb.pos, sb.step, sb.key, sb.done)
        assert sb.token == (force[step].item() if step < n_force else int(lb.cpu().argmax()))


def test_lm_head_ties_and_forcing(dev):
    C, V = 256, 4096
    h = torch.ones(C, dtype=torch.bfloat16)
    emb = torch.zeros(V, C, dtype=torch.bfloat16)
    emb[[1234, 77, 3000]] = 1.0  # three equal maxima: the first index wins
    hd, ed = h.to(dev), emb.to(dev)
    st = state_tensor(dev)
    run_head(dev, hd, ed, st)
    assert read_state(st).token == 77
    force = torch.tensor([5, 6], dtype=torch.int32, device=dev)
    tokens = torch.zeros(4, dtype=torch.int32, device=dev)
    st = state_tensor(dev)
    for want_next in (5, 6, 77):
        run_head(dev, hd, ed, st, force=force, n_force=2, tokens=tokens)
        assert read_state(st).token == want_next
    assert tokens[:3].tolist() == [77, 77, 77]


def test_packed_gpt_matches_oracle(dev, tiny_model, tiny_ref):
    """fp32 activations end to end: the reference's numerics."""
    prompt = [5, 900, 17, 3, 250, 42]
    x = torch.tensor([prompt], device=dev)
    full = tiny_model(x)
    ref, _ = tiny_ref.forward(torch.tensor([prompt]))
    assert rel(full[0].cpu(), ref[0]) <= 1e-4
    from nativebit_amd.model import greedy_generate
    ours = greedy_generate(tiny_model, prompt, 8, device=dev)
    theirs = tiny_ref.greedy(prompt, 8)
    assert ours == theirs


def test_decode_engine_matches_oracle(dev, tiny_model, tiny_ref):
    """bf16 GEMV inputs: compare each teacher-forced step's logits with the
    oracle under the same bf16 rounding of weights and GEMV inputs."""
    eng = DecodeEngine(tiny_model, max_steps=32)
    seq = [5, 900, 17, 3, 250, 42, 7, 1, 999, 64, 12, 300]
    eng.reset(seq)           # every later token forced
    cache = tiny_ref.init_cache()
    for t in range(len(seq)):
        eng.step()
        lg, cache = tiny_ref.forward(torch.tensor([[seq[t]]]), cache,
                                     weight_dtype=torch.bfloat16, act_dtype=torch.bfloat16,
                                     head_dtype=torch.bfloat16)
        ours = eng.logits.cpu()
        assert rel(ours, lg[0, 0]) <= 5e-3, (t, rel(ours, lg[0, 0]))
        top2 = torch.topk(lg[0, 0], 2).values
        if float(top2[0] - top2[1]) > 1e-3:
            assert int(ours.argmax()) == int(lg[0, 0].argmax())
    s = eng.state()
    assert s["pos"] == len(seq) and s["step"] == len(seq)


def test_decode_engine_graph_replay(dev, tiny_model):
    eng = DecodeEngine(tiny_model, max_steps=40)
    prompt = [1, 2, 3, 4]
    eager = []
    eng.reset(prompt)
    for _ in range(10):
        eng.step()
        eager.append(eng.logits.clone())
    eng.reset(prompt)
    eng.capture()
    for i in range(10):
        eng._advance(1)
        eng.graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(eng.logits, eager[i]), i
    toks = eng.generate(prompt, 12)
    assert len(toks) == 12 and eng.state()["step"] == len(prompt) + 11


def test_nbpack_file_roundtrip(dev, tiny_model, tmp_path):
    from nativebit_amd.model import to_nbpack_params
    path = str(tmp_path / "tiny.nbpack.npz")
    np.savez_compressed(path, **to_nbpack_params(tiny_model))
    loaded = load_packed_model(path, TINY, device=dev)
    x = torch.tensor([[1, 2, 3, 999]], device=dev)
    assert torch.equal(loaded(x), tiny_model(x))
    pack = formats.load_nbpack(path)
    assert len(pack.layers) == 10
