"""GPU parity of the persistent decode (nb_decode_persistent; run with -m gpu).

* teacher-forced logits against the CPU oracle decoder with the same bf16
  rounding of weights and GEMV inputs (the reference's model, generate_torch.
  py:135-162, in its bf16 form, eval_ppl.py:149-174);
* determinism: all steps in one launch give bit-identical logits and tokens
  to one launch per step (row sums, attention combine and argmax do not
  depend on scheduling);
* against DecodeEngine (one HIP graph of launches per token) at three
  shapes: the tiny model, a medium one with 128-wide heads and several
  attention splits, and two layers of the 2.2B shape (2560 / 6912, 20
  heads, vocab 32000) where a workgroup runs on every CU;
* a grid barrier that runs past a tiny spin limit (forced from the host)
  ends the launch with the error word set, and the next launch works.
"""
import pytest
import torch

from nativebit_amd import _lib
from nativebit_amd.decode import DecodeEngine, PersistentDecodeEngine
from nativebit_amd.model import ModelConfig, random_packed_model
from oracle import decode_ref as R

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="nb_decode_persistent faulted the GPU (illegal memory access) on the "
                            "26-layer 2.2B model in a 128-step launch; the cause is not yet shown, "
                            "so the persistent path stays off the GPU until it is"),
]

TINY = ModelConfig(vocab_size=1000, n_layers=2, n_embd=256, n_head=4, ffn_hidden=512,
                   context_len=64)
# 128-wide heads, R = 12 and R = 4 rows per chunk, up to 3 attention splits
MEDIUM = ModelConfig(vocab_size=2000, n_layers=2, n_embd=640, n_head=5, ffn_hidden=1792,
                     context_len=192)
# two layers of the 2.2B shape (configs/tpu.py), the vocabulary of config 4b
REAL2 = ModelConfig(vocab_size=32000, n_layers=2, n_embd=2560, n_head=20, ffn_hidden=6912,
                    context_len=256)


def note(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = torch.as_tensor(a).double().reshape(-1).cpu()
    b = torch.as_tensor(b).double().reshape(-1).cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


@pytest.fixture(scope="module")
def tiny_model(dev):
    return random_packed_model(TINY, seed=5, device=dev)


@pytest.fixture(scope="module")
def medium_model(dev):
    return random_packed_model(MEDIUM, seed=11, device=dev)


def seq_of(n, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (n,), generator=g).tolist()


def test_persistent_matches_oracle(dev, tiny_model):
    note("persistent vs oracle, tiny, teacher forced")
    ref = R.DecoderRef.from_model(tiny_model)
    eng = PersistentDecodeEngine(tiny_model, max_steps=32)
    seq = [5, 900, 17, 3, 250, 42, 7, 1, 999, 64, 12, 300]
    eng.reset(seq)
    cache = ref.init_cache()
    for t in range(len(seq)):
        eng.step()
        lg, cache = ref.forward(torch.tensor([[seq[t]]]), cache, weight_dtype=torch.bfloat16,
                                act_dtype=torch.bfloat16, head_dtype=torch.bfloat16)
        ours = eng.logits.cpu()
        assert eng.error() == 0
        assert rel(ours, lg[0, 0]) <= 5e-3, (t, rel(ours, lg[0, 0]))
        top2 = torch.topk(lg[0, 0], 2).values
        if float(top2[0] - top2[1]) > 1e-3:
            assert int(ours.argmax()) == int(lg[0, 0].argmax())
    s = eng.state()
    assert s["pos"] == len(seq) and s["step"] == len(seq) and s["key"] == 0


@pytest.mark.parametrize("which", ["tiny", "medium"])
def test_one_launch_equals_per_step(dev, which, tiny_model, medium_model):
    model = tiny_model if which == "tiny" else medium_model
    note(f"persistent one launch vs per step, {which}")
    V = model.cfg.vocab_size
    prompt = seq_of(9, V, 1)
    eng = PersistentDecodeEngine(model, max_steps=64)
    eng.reset(prompt)
    per_step = []
    for _ in range(len(prompt) + 15):
        eng.step()
        per_step.append(eng.logits.clone())
    toks_a = eng.tokens[: len(prompt) + 15].clone()
    eng.reset(prompt)
    eng.run(len(prompt) + 15)
    torch.cuda.synchronize()
    assert eng.error() == 0
    assert torch.equal(eng.tokens[: len(prompt) + 15], toks_a)
    assert torch.equal(eng.logits, per_step[-1])
    # split 7 + rest
    eng.reset(prompt)
    eng.run(7)
    eng.run(len(prompt) + 8)
    assert torch.equal(eng.tokens[: len(prompt) + 15], toks_a)
    assert torch.equal(eng.logits, per_step[-1])


def compare_engines(model, seq, tol=5e-3):
    """Both engines teacher-forced through seq: per-step logits within tol
    (both are bf16-input approximations of the fp32 model that sum in
    different orders; a one-ulp flip of a bf16-rounded GEMV input moves the
    logits by ~1e-4 relative), and the same argmax wherever the top-2 gap
    exceeds twice the largest elementwise difference (then it must agree)."""
    g = DecodeEngine(model, max_steps=len(seq))
    p = PersistentDecodeEngine(model, max_steps=len(seq))
    g.reset(seq)
    p.reset(seq)
    worst = 0.0
    for t in range(len(seq)):
        g.step()
        p.step()
        lg, lp = g.logits.cpu(), p.logits.cpu()
        r = rel(lp, lg)
        worst = max(worst, r)
        assert r <= tol, (t, r)
        delta = float((lp - lg).abs().max())
        top2 = torch.topk(lg, 2).values
        if float(top2[0] - top2[1]) > 2 * delta:
            assert int(lp.argmax()) == int(lg.argmax()), t
    assert p.error() == 0
    note(f"worst step rel {worst:.2e}")
    return g, p


def test_matches_graph_engine_tiny(dev, tiny_model):
    note("persistent vs graph engine, tiny")
    compare_engines(tiny_model, seq_of(26, 1000, 2))


def test_matches_graph_engine_medium(dev, medium_model):
    note("persistent vs graph engine, medium (D=128, several splits)")
    compare_engines(medium_model, seq_of(170, 2000, 3))


def test_matches_graph_engine_real_shape(dev):
    note("persistent vs graph engine, two 2.2B-shape layers, vocab 32000")
    model = random_packed_model(REAL2, seed=3, device=dev)
    compare_engines(model, seq_of(80, 32000, 4))
    # a whole continuation in one launch gives the per-step launches' tokens
    prompt = seq_of(40, 32000, 5)
    p = PersistentDecodeEngine(model, max_steps=80)
    whole = p.generate(prompt, 30)
    p.reset(prompt)
    for _ in range(len(prompt) + 29):
        p.step()
    assert p.tokens[len(prompt) - 1: len(prompt) + 29].cpu().tolist() == whole


def test_spin_limit_abort_and_recovery(dev, tiny_model):
    note("persistent: spin limit 1 (forced barrier time-out), then a normal launch")
    prompt = [3, 1, 4, 1, 5]
    good = PersistentDecodeEngine(tiny_model, max_steps=32).generate(prompt, 10)
    eng = PersistentDecodeEngine(tiny_model, max_steps=32, spin_limit=1)
    eng.reset(prompt)
    eng.run(14)
    torch.cuda.synchronize()
    err = eng.error()
    assert err in (0, 1)
    if err:
        with pytest.raises(_lib.NativeBitError):
            eng.generate(prompt, 10)
    eng.spin_limit = 0
    assert eng.generate(prompt, 10) == good
