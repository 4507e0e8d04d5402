"""GPU parity of the batched prompt pass (run with -m gpu).

* nb_rmsnorm_rows (plain, residual add, embedding lookup), nb_silu_pairs_rows,
  nb_rope_kv_rows and nb_attention_rows against the oracle's statements of
  the reference's ops (oracle/decode_ref.py: rmsnorm, rope, softmax
  attention over a cache with the causal mask) on the same inputs, at the
  2.2B model's head shape and smaller ones, with earlier cache positions
  present (pos0 > 0) and a pass that ends at the last cache position;
* apply_rope of the module API against the oracle's rope, bit for bit;
* PackedGPT's module forward with a cache fed in pieces against the same
  tokens as one sequence, and its caches against the oracle's;
* DecodeEngine.prefill (packed MFMA GEMMs plus the row kernels) against the
  oracle over the same tokens with the same bf16 rounding of weights and
  matmul inputs, and against the per-token decode path (teacher forced):
  logits of the last prompt token, every cached key and value, the decode
  state; the greedy tokens generated after it against the oracle's logits.
"""
import ctypes

import pytest
import torch
import torch.nn.functional as F

from nativebit_amd import _lib
from nativebit_amd.decode import DecodeEngine
from nativebit_amd.model import (ModelConfig, apply_rope, init_kv_cache, precompute_rope,
                                 random_packed_model)
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


DT = {torch.float32: _lib.NB_F32, torch.bfloat16: _lib.NB_BF16}
TOL = {torch.float32: 1e-6, torch.bfloat16: 4e-3}


@pytest.mark.parametrize("mode", ["plain", "residual", "embed"])
@pytest.mark.parametrize("hdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,C", [(5, 2560), (1, 256), (130, 512)])
def test_rmsnorm_rows(dev, mode, hdt, T, C):
    note(f"rmsnorm_rows {mode} {hdt} T={T} C={C}")
    lib = _lib.load()
    g = torch.Generator().manual_seed(T * 7 + C)
    x0 = torch.randn(T, C, generator=g)
    add = torch.randn(T, C, generator=g)
    w = torch.randn(C, generator=g)
    emb = torch.randn(11, C, generator=g)
    tokens = torch.randint(0, 11, (T,), generator=g, dtype=torch.int32)
    x = x0.to(dev)
    h = torch.empty(T, C, dtype=hdt, device=dev)
    ad = add.to(dev) if mode == "residual" else None
    ed = emb.to(dev) if mode == "embed" else None
    td = tokens.to(dev) if mode == "embed" else None
    wd = w.to(dev)
    _lib.check(lib.nb_rmsnorm_rows(P(x), P(ad), P(ed), P(td), 11, P(wd), P(h), DT[hdt], T, C,
                                   1e-6, stream()))
    xr = {"plain": x0, "residual": x0 + add, "embed": emb[tokens.long()]}[mode]
    assert torch.equal(x.cpu(), xr)
    hr = R.rmsnorm(xr, w, 1e-6)
    for t in range(T):
        assert rel(h[t].float(), hr[t]) <= TOL[hdt], t


def test_rmsnorm_rows_token_outside_table(dev):
    """Tokens outside [0, vocab) read nothing; their rows become NaN, the
    other rows are the lookup's."""
    note("rmsnorm_rows tokens outside the table")
    lib = _lib.load()
    C, V = 256, 11
    g = torch.Generator().manual_seed(5)
    emb = torch.randn(V, C, generator=g)
    w = torch.randn(C, generator=g)
    tokens = torch.tensor([3, -1, 10, 11, 1 << 30, 0], dtype=torch.int32)
    T = tokens.numel()
    x = torch.zeros(T, C, device=dev)
    h = torch.empty(T, C, device=dev)
    ed, td, wd = emb.to(dev), tokens.to(dev), w.to(dev)   # held until the kernel has run
    _lib.check(lib.nb_rmsnorm_rows(P(x), None, P(ed), P(td), V, P(wd), P(h), _lib.NB_F32, T, C,
                                   1e-6, stream()))
    xc, hc = x.cpu(), h.cpu()
    for t, tok in enumerate(tokens.tolist()):
        if 0 <= tok < V:
            assert torch.equal(xc[t], emb[tok]), t
            assert rel(hc[t], R.rmsnorm(emb[tok], w, 1e-6)) <= 1e-6, t
        else:
            assert torch.isnan(xc[t]).all() and torch.isnan(hc[t]).all(), t


@pytest.mark.parametrize("adt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,Fw", [(3, 6912), (128, 512), (1, 8)])
def test_silu_pairs_rows(dev, adt, T, Fw):
    note(f"silu_pairs_rows {adt} T={T} F={Fw}")
    g = torch.Generator().manual_seed(T + Fw)
    gu = torch.randn(T, 2 * Fw, generator=g) * 3
    gud = gu.to(dev)
    act = torch.empty(T, Fw, dtype=adt, device=dev)
    _lib.check(_lib.load().nb_silu_pairs_rows(P(gud), P(act), DT[adt], T, Fw, stream()))
    ref = F.silu(gu[:, 0::2]) * gu[:, 1::2]
    assert rel(act.float(), ref) <= TOL[adt]


# (n_head, head_dim, ctx, pos0, T): the 2.2B head shape from position 0, a
# pass that ends at the last cache position, ragged small shapes
CASES = [(20, 128, 1024, 0, 128), (20, 128, 1024, 900, 124), (20, 128, 1024, 37, 1),
         (4, 64, 80, 10, 37), (2, 32, 80, 0, 17), (3, 16, 40, 5, 35)]


def _qkv_heads(qkv, T, H, D):
    """(T, 3HD) -> q, k, v as (1, H, T, D)."""
    q, k, v = qkv.reshape(T, 3, H, D).permute(1, 2, 0, 3).unsqueeze(1)
    return q, k, v


@pytest.mark.parametrize("H,D,ctx,pos0,T", CASES)
def test_rope_kv_rows(dev, H, D, ctx, pos0, T):
    note(f"rope_kv_rows H={H} D={D} ctx={ctx} pos0={pos0} T={T}")
    lib = _lib.load()
    C = H * D
    g = torch.Generator().manual_seed(H * D + pos0 + T)
    qkv = torch.randn(T, 3 * C, generator=g)
    kc0 = torch.randn(H, D, ctx, generator=g)      # keys [H][D][ctx]
    vc0 = torch.randn(H, ctx, D, generator=g)      # values [H][ctx][D]
    cos, sin = precompute_rope(D, ctx)
    qkvd, kd, vd = qkv.to(dev), kc0.to(dev), vc0.to(dev)
    cosd, sind = cos.to(dev), sin.to(dev)
    q_out = torch.empty(T, C, device=dev)
    _lib.check(lib.nb_rope_kv_rows(P(qkvd), P(kd), P(vd), P(cosd), P(sind), pos0, T, P(q_out),
                                   H, D, ctx, stream()))
    q, k, v = _qkv_heads(qkv, T, H, D)
    qr = R.rope(q, cos, sin, pos0)[0]             # (H, T, D)
    kr = R.rope(k, cos, sin, pos0)[0]
    kc, vc = kd.cpu(), vd.cpu()
    span = slice(pos0, pos0 + T)
    assert torch.allclose(kc[:, :, span], kr.transpose(1, 2), rtol=1e-6, atol=1e-6)
    assert torch.equal(vc[:, span], v[0])
    outside = torch.ones(ctx, dtype=torch.bool)
    outside[span] = False
    assert torch.equal(kc[:, :, outside], kc0[:, :, outside])
    assert torch.equal(vc[:, outside], vc0[:, outside])
    q_ref = (qr * D ** -0.5).transpose(0, 1).reshape(T, C)
    assert rel(q_out, q_ref) <= 1e-6


def attention_ref(q, kc, vc, pos0, T, H, D):
    """out[t] = softmax(q[t] . k[0..pos0+t]) v[0..pos0+t], per head, in fp64
    (the masked cache attention of generate_torch.py:89-98)."""
    qh = q.double().reshape(T, H, D).transpose(0, 1)              # (H, T, D)
    n = pos0 + T
    keys = kc[:, :, :n].double()                                   # (H, D, n)
    att = qh @ keys                                                # (H, T, n)
    mask = torch.arange(n)[None, :] <= (pos0 + torch.arange(T))[:, None]
    att = att.masked_fill(~mask[None], float("-inf"))
    out = torch.softmax(att, dim=-1) @ vc[:, :n].double()          # (H, T, D)
    return out.transpose(0, 1).reshape(T, H * D)


@pytest.mark.parametrize("odt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H,D,ctx,pos0,T", CASES)
def test_attention_rows(dev, H, D, ctx, pos0, T, odt):
    note(f"attention_rows H={H} D={D} ctx={ctx} pos0={pos0} T={T} {odt}")
    lib = _lib.load()
    C = H * D
    g = torch.Generator().manual_seed(H + D + ctx + pos0 + T)
    q = torch.randn(T, C, generator=g) * D ** -0.5 * 2
    kc = torch.randn(H, D, ctx, generator=g)
    vc = torch.randn(H, ctx, D, generator=g)
    # past the pass: garbage the causal mask must hide
    kc[:, :, pos0 + T:] = 1e4
    vc[:, pos0 + T:] = float("nan")
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    out = torch.empty(T, C, dtype=odt, device=dev)
    _lib.check(lib.nb_attention_rows(P(qd), P(kd), P(vd), pos0, T, P(out), DT[odt], H, D, ctx,
                                     stream()))
    ref = attention_ref(q, kc, vc, pos0, T, H, D)
    o = out.float().cpu()
    assert torch.isfinite(o).all()
    for t in range(T):
        assert rel(o[t], ref[t]) <= (1e-5 if odt == torch.float32 else 4e-3), t


def test_apply_rope_matches_oracle():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 4, 9, 32, generator=g)
    k = torch.randn(1, 4, 9, 32, generator=g)
    cos, sin = precompute_rope(32, 64)
    c2, s2 = R.rope_tables(32, 64)
    assert torch.equal(cos, c2) and torch.equal(sin, s2)
    qr, kr = apply_rope(q, k, cos, sin, pos_offset=11)
    assert torch.equal(qr, R.rope(q, cos, sin, 11))
    assert torch.equal(kr, R.rope(k, cos, sin, 11))


TINY = ModelConfig(vocab_size=1000, n_layers=2, n_embd=256, n_head=4, ffn_hidden=512,
                   context_len=64)


@pytest.fixture(scope="module")
def tiny_model(dev):
    return random_packed_model(TINY, seed=5, device=dev)


@pytest.fixture(scope="module")
def tiny_ref(tiny_model):
    return R.DecoderRef.from_model(tiny_model)


def test_packed_gpt_cache_in_pieces(dev, tiny_model, tiny_ref):
    """The module forward over a cache fed 5 + 1 + 3 tokens equals the same
    9 tokens as one sequence without a cache; the caches hold the oracle's
    rotated keys and values."""
    seq = [5, 900, 17, 3, 250, 42, 7, 1, 999]
    whole = tiny_model(torch.tensor([seq], device=dev))
    caches = init_kv_cache(tiny_model, device=dev)
    parts = []
    for a, b in ((0, 5), (5, 6), (6, 9)):
        lg, caches = tiny_model(torch.tensor([seq[a:b]], device=dev), kv_caches=caches)
        parts.append(lg)
    assert all(c[2] == len(seq) for c in caches)
    assert rel(torch.cat(parts, dim=1), whole) <= 1e-5
    cache = tiny_ref.init_cache()
    ref, cache = tiny_ref.forward(torch.tensor([seq]), cache)
    assert rel(whole[0].cpu(), ref[0]) <= 1e-4
    n = len(seq)
    for l, (kb, vb, _) in enumerate(caches):
        ko, vo = cache[0][l]
        # the reference's cache shapes and indexing (positions on dim 2)
        assert kb.shape == vb.shape == ko.shape, l
        assert rel(kb[0, :, :n].cpu(), ko[0, :, :n]) <= 1e-5, l
        assert rel(vb[0, :, :n].cpu(), vo[0, :, :n]) <= 1e-5, l


BF16 = dict(weight_dtype=torch.bfloat16, act_dtype=torch.bfloat16, head_dtype=torch.bfloat16)


def _check_prefill(eng, ref, seq, bound):
    """eng has run prefill(seq): last logits and caches against the oracle
    over the same tokens (bf16 rounding of weights, matmul inputs, head)."""
    T = len(seq)
    cache = ref.init_cache()
    lg, cache = ref.forward(torch.tensor([seq]), cache, **BF16)
    e = rel(eng.logits.cpu(), lg[0, -1])
    note(f"prefill T={T}: logits rel vs oracle {e:.2e}")
    assert e <= bound, e
    for l in range(ref.cfg.n_layers):
        ko, vo = cache[0][l]
        ek = rel(eng.kc[l][:, :, :T].transpose(1, 2).cpu(), ko[0, :, :T])
        ev = rel(eng.vc[l][:, :T].cpu(), vo[0, :, :T])
        assert ek <= bound and ev <= bound, (l, ek, ev)
    s = eng.state()
    assert s["pos"] == T and s["step"] == T
    assert s["token"] == int(eng.logits.argmax())
    assert int(eng.tokens[T - 1]) == s["token"]
    return lg


@pytest.mark.parametrize("T", [1, 12, 40, 63])
def test_prefill_vs_oracle(dev, tiny_model, tiny_ref, T):
    g = torch.Generator().manual_seed(T)
    seq = torch.randint(0, TINY.vocab_size, (T,), generator=g).tolist()
    eng = DecodeEngine(tiny_model, max_steps=64)
    eng.prefill(seq)
    _check_prefill(eng, tiny_ref, seq, 5e-3)


def test_prefill_graph_equals_eager(dev, tiny_model):
    """The prompt pass replayed from its captured graph (buffers kept per
    prompt length) equals the eager launches bit for bit, also for a second
    prompt of the same length (new tokens into the same buffers) and after a
    prompt of another length."""
    eager = DecodeEngine(tiny_model, max_steps=64)
    cached = DecodeEngine(tiny_model, max_steps=64)
    g = torch.Generator().manual_seed(77)
    for T in (24, 24, 9, 24):
        seq = torch.randint(0, TINY.vocab_size, (T,), generator=g).tolist()
        note(f"prefill graph vs eager T={T}")
        eager.prefill(seq, graph=False)
        cached.prefill(seq)
        torch.cuda.synchronize()
        assert torch.equal(eager.logits, cached.logits)
        assert torch.equal(eager.x, cached.x)
        assert torch.equal(eager.kc, cached.kc) and torch.equal(eager.vc, cached.vc)
        assert eager.state() == cached.state()
        assert int(eager.tokens[T - 1]) == int(cached.tokens[T - 1])


def test_prefill_vs_teacher_forced(dev, tiny_model):
    """The batched prompt leaves the state, caches and logits the per-token
    path leaves after the same prompt, and nothing past the prompt in the
    caches; the next step from the same token then agrees too."""
    seq = [5, 900, 17, 3, 250, 42, 7, 1, 999, 64, 12, 300, 8, 8, 8, 1, 2, 3, 4, 5]
    T = len(seq)
    a = DecodeEngine(tiny_model, max_steps=40)
    a.prefill(seq)
    b = DecodeEngine(tiny_model, max_steps=40)
    b.reset(seq)
    for _ in range(T):
        b.step()
    sa, sb = a.state(), b.state()
    assert (sa["pos"], sa["step"]) == (sb["pos"], sb["step"]) == (T, T)
    assert rel(a.logits, b.logits) <= 5e-3
    top2 = torch.topk(b.logits.float(), 2).values
    if float(top2[0] - top2[1]) > 0.05:
        assert sa["token"] == sb["token"]
    assert rel(a.kc[:, :, :, :T], b.kc[:, :, :, :T]) <= 5e-3
    assert rel(a.vc[:, :, :T], b.vc[:, :, :T]) <= 5e-3
    assert float(a.kc[:, :, :, T:].abs().sum()) == 0 and float(a.vc[:, :, T:].abs().sum()) == 0
    if sa["token"] == sb["token"]:
        a.step()
        b.step()
        assert rel(a.logits, b.logits) <= 5e-3


def test_generate_batched_prompt_vs_oracle(dev, tiny_model, tiny_ref):
    """Every greedy token after the batched prompt is the oracle's argmax,
    or within 0.05 of its largest logit (a near tie), teacher forced over
    the same tokens."""
    prompt = [11, 22, 33, 44, 55, 66, 77, 88, 99, 111, 222, 333, 444, 555, 666, 777, 888, 999]
    eng = DecodeEngine(tiny_model, max_steps=48)
    toks = eng.generate(prompt, 12)
    again = eng.generate(prompt, 12)
    assert toks == again
    lg, _ = tiny_ref.forward(torch.tensor([prompt + toks[:-1]]), tiny_ref.init_cache(), **BF16)
    for i, tok in enumerate(toks):
        row = lg[0, len(prompt) - 1 + i]
        assert float(row[tok]) >= float(row.max()) - 0.05, (i, tok, int(row.argmax()))
