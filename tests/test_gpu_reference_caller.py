"""The reference's own decode caller, unchanged, on the GPU (run with -m gpu).

inference/generate_torch.py:330-360 builds its model with
``load_packed_model(args.checkpoint, TPU2BConfig())`` and decodes with
``init_kv_cache(model)`` then ``model(x, kv_caches=caches)`` per token.  Here
that code runs as written against this library:

* an archive in the reference packer's key layout and key order
  (inference/pack.py:114-151; block_10's keys before block_2's) is loaded
  through an object with exactly TPU2BConfig's attribute names;
* the prompt and then one token at a time go through the module forward
  with the caches, and every step's logits are compared with the CPU
  decoder oracle built from the same archive by explicit key names (so a
  loader that put a layer in the wrong block would fail);
* without a cache and with pos_offset > 0 the tokens attend to each other
  only, rotated at pos_offset.. (the reference's SDPA branch), against the
  oracle's whole-sequence path at the same offset;
* a cache the caller builds in the reference's contiguous layout gives the
  logits and the keys of init_kv_cache's.
"""
import numpy as np
import pytest
import torch

from nativebit_amd.model import init_kv_cache, load_packed_model, model_config
from oracle import decode_ref as R
from refmodel import TPU2BLike, archive

pytestmark = pytest.mark.gpu

NAMES = [("qkv", "CausalSelfAttention_0.NativeBitDense_0"),
         ("out_proj", "CausalSelfAttention_0.NativeBitDense_1"),
         ("gate", "SwiGLU_0.NativeBitDense_0"), ("up", "SwiGLU_0.NativeBitDense_1"),
         ("down", "SwiGLU_0.NativeBitDense_2")]


def note(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = torch.as_tensor(a).double().reshape(-1).cpu()
    b = torch.as_tensor(b).double().reshape(-1).cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


@pytest.fixture(scope="module")
def packed_file(tmp_path_factory):
    cfg = model_config(TPU2BLike())
    save, _ = archive(cfg, seed=7)
    path = str(tmp_path_factory.mktemp("refcaller") / "tpu2b_small.nbpack.npz")
    np.savez_compressed(path, **save)
    return path, save, cfg


def oracle_from_archive(save, cfg):
    """The CPU decoder oracle over the archive's arrays, block i from the
    keys named block_i (no sorting involved)."""
    layers, norms = [], []
    for i in range(cfg.n_layers):
        lin = {}
        for name, key in NAMES:
            p = f"params.block_{i}.{key}"
            o, k = (int(v) for v in save[f"shape.{p}"])
            lin[name] = R.PackedRef(save[f"idx.{p}"], save[f"cb.{p}"], o, k, 128, 3,
                                    keep_dense=True)
        layers.append(lin)
        norms.append((torch.from_numpy(save[f"param.params.block_{i}.RMSNorm_0.weight"]),
                      torch.from_numpy(save[f"param.params.block_{i}.RMSNorm_1.weight"])))
    return R.DecoderRef(cfg, layers, torch.from_numpy(save["param.params.embedding"]), norms,
                        torch.from_numpy(save["param.params.ln_f.weight"]))


@pytest.fixture(scope="module")
def loaded(dev, packed_file):
    path, save, cfg = packed_file
    note("load_packed_model with a TPU2BConfig-shaped config")
    model = load_packed_model(path, TPU2BLike(), device=dev)
    return model, oracle_from_archive(save, cfg)


def test_reference_decode_loop(dev, loaded):
    """generate_torch.py:351-360 as written: prompt pass over fresh caches,
    then one token per forward; teacher forced by the oracle's greedy token
    so both see the same sequence."""
    model, ref = loaded
    prompt = [5, 200, 17, 3, 299, 42, 0, 128]
    note(f"reference loop: prompt of {len(prompt)}, 10 steps")
    caches = init_kv_cache(model)
    x = torch.tensor([prompt], dtype=torch.long, device="cuda")
    with torch.no_grad():
        logits, caches = model(x, kv_caches=caches)
    rcache = ref.init_cache()
    rl, rcache = ref.forward(torch.tensor([prompt]), rcache)
    assert logits.shape == (1, len(prompt), 300)
    assert rel(logits[0], rl[0]) <= 1e-4
    for step in range(10):
        want = int(rl[0, -1].argmax())
        top2 = torch.topk(rl[0, -1], 2).values
        if float(top2[0] - top2[1]) > 1e-3:
            assert int(logits[0, -1].argmax()) == want, step
        x1 = torch.tensor([[want]], dtype=torch.long, device="cuda")
        with torch.no_grad():
            logits, caches = model(x1, kv_caches=caches)
        rl, rcache = ref.forward(torch.tensor([[want]]), rcache)
        assert rel(logits[0, 0], rl[0, 0]) <= 1e-4, step
    assert all(c[2] == len(prompt) + 10 for c in caches)
    # the caches read as the reference's (positions on dim 2)
    n = len(prompt) + 10
    for l, (kb, vb, _) in enumerate(caches):
        ko, vo = rcache[0][l]
        assert rel(kb[0, :, :n], ko[0, :, :n]) <= 1e-5, l
        assert rel(vb[0, :, :n], vo[0, :, :n]) <= 1e-5, l


@pytest.mark.parametrize("pos_offset", [0, 5, 17])
def test_no_cache_with_pos_offset(dev, loaded, pos_offset):
    """No cache: the T tokens attend to each other only, rotated at
    pos_offset .. (generate_torch.py:97-101 with apply_rope at pos_offset).
    RoPE scores depend on position differences only, so every offset gives
    the offset-0 logits up to rounding; attending to pos_offset empty cache
    slots as well (zero keys: score 0, zero values) would not."""
    model, ref = loaded
    toks = [9, 1, 250, 33, 7]
    note(f"no cache, pos_offset {pos_offset}")
    x = torch.tensor([toks], device=dev)
    lg = model(x, pos_offset=pos_offset)
    want, _ = ref.forward(torch.tensor([toks]), pos0=pos_offset)
    assert rel(lg[0], want[0]) <= 1e-4
    assert rel(lg[0], model(x)[0]) <= 1e-5


def test_reference_layout_cache(dev, loaded):
    """Caches in the reference's own contiguous layout (generate_torch.py:
    269-277) give init_kv_cache's logits and keys."""
    model, _ = loaded
    H, D, ctx = model.n_head, model.n_embd // model.n_head, model.context_len
    note("reference-layout caches")
    own = init_kv_cache(model)
    theirs = [(torch.zeros(1, H, ctx, D, device=dev), torch.zeros(1, H, ctx, D, device=dev), 0)
              for _ in range(model.n_layers)]
    seq = [[4, 8, 15, 16], [23], [42, 2]]
    for part in seq:
        x = torch.tensor([part], device=dev)
        a, own = model(x, kv_caches=own)
        b, theirs = model(x, kv_caches=theirs)
        assert torch.equal(a, b)
    for (ka, va, na), (kb, vb, nb) in zip(own, theirs):
        assert na == nb == 7
        assert torch.equal(ka, kb) and torch.equal(va, vb)
