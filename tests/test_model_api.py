"""The reference's model API on the host (no GPU): constructor signatures,
TPU2BConfig-shaped configs, the loader's layer order and shape checks, and
the KV-cache layouts.

* ``PackedGPT``, ``TransformerBlock``, ``CausalAttention``, ``SwiGLU`` and
  ``RMSNorm`` take the positional arguments of inference/generate_torch.py:
  29-147, and build their linears through ``make_linear(out, in)`` in the
  reference's module order;
* ``load_packed_model(path, config)`` accepts an object with exactly
  TPU2BConfig's attribute names (configs/tpu.py:137-151) and fills block i
  with the archive's block-i layers although the reference's packer writes
  the keys in alphabetical order (block_10 before block_2,
  inference/pack.py:114);
* ``init_kv_cache`` returns the reference's shapes (generate_torch.py:
  269-277) over the kernels' key layout, and wrong caches raise.
"""
import inspect

import numpy as np
import pytest
import torch

from nativebit_amd import model as M
from refmodel import TPU2BLike, archive as _archive


def test_constructor_signatures_are_the_reference_ones():
    def positional(f):
        return [p.name for p in inspect.signature(f).parameters.values()
                if p.kind == p.POSITIONAL_OR_KEYWORD and p.name != "self"]
    assert positional(M.PackedGPT.__init__) == ["vocab_size", "n_layers", "n_embd", "n_head",
                                                "ffn_hidden", "context_len", "make_linear"]
    assert positional(M.TransformerBlock.__init__) == ["n_embd", "n_head", "ffn_hidden",
                                                       "context_len", "make_linear"]
    assert positional(M.CausalAttention.__init__)[:4] == ["n_embd", "n_head", "context_len",
                                                          "make_linear"]
    assert positional(M.SwiGLU.__init__) == ["n_embd", "ffn_hidden", "make_linear"]
    assert positional(M.RMSNorm.__init__) == ["dim", "eps"]
    assert positional(M.PackedGPT.forward) == ["idx", "kv_caches", "pos_offset"]
    assert positional(M.load_packed_model) == ["packed_path", "config", "device"]
    assert positional(M.init_kv_cache)[:3] == ["model", "batch_size", "device"]


def test_make_linear_order_and_shapes():
    calls = []

    def make_linear(out_f, in_f):
        calls.append((out_f, in_f))
        return M.UnloadedLinear(out_f, in_f)

    model = M.PackedGPT(100, 2, 64, 4, 96, 16, make_linear)
    C, F = 64, 96
    one = [(3 * C, C), (C, C), (F, C), (F, C), (C, F)]
    assert calls == one * 2
    names = [n for n, m in model.named_modules() if isinstance(m, M.UnloadedLinear)]
    assert names == [f"blocks.{i}.{p}" for i in range(2)
                     for p in ("attn.qkv", "attn.out_proj", "ffn.gate", "ffn.up", "ffn.down")]
    assert model.cfg.norm_eps == 1e-6 and model.cfg.rope_theta == 10000.0
    assert model.blocks[1].ln2.eps == 1e-6


def test_model_config_from_tpu2b_shape():
    c = M.model_config(TPU2BLike())
    assert (c.vocab_size, c.n_layers, c.n_embd, c.n_head, c.ffn_hidden, c.context_len) == \
        (300, 12, 256, 4, 384, 32)
    assert c.n_entries == 8 and c.block_size == 128
    assert c.norm_eps == 1e-6 and c.rope_theta == 10000.0

    class Partial:
        n_layers = 2
    with pytest.raises(ValueError, match="vocab_size"):
        M.model_config(Partial())


def test_loader_order_with_tpu2b_config(tmp_path):
    cfg = M.model_config(TPU2BLike())
    save, truth = _archive(cfg)
    keys = [k for k in save if k.startswith("idx.")]
    assert keys.index("idx.params.block_10.CausalSelfAttention_0.NativeBitDense_0") < \
        keys.index("idx.params.block_2.CausalSelfAttention_0.NativeBitDense_0")
    path = str(tmp_path / "m.nbpack.npz")
    np.savez_compressed(path, **save)
    model = M.load_packed_model(path, TPU2BLike(), device="cpu")
    for i, blk in enumerate(model.blocks):
        mods = (blk.attn.qkv, blk.attn.out_proj, blk.ffn.gate, blk.ffn.up, blk.ffn.down)
        for j, pl in enumerate(mods):
            lay = truth[(i, j)]
            assert torch.equal(pl.packed_indices, lay.packed), (i, j)
            assert torch.equal(pl.codebook, lay.codebook), (i, j)
        assert torch.equal(blk.ln1.weight, torch.from_numpy(
            save[f"param.params.block_{i}.RMSNorm_0.weight"]))
        assert torch.equal(blk.ln2.weight, torch.from_numpy(
            save[f"param.params.block_{i}.RMSNorm_1.weight"]))
    assert torch.equal(model.embedding.weight, torch.from_numpy(save["param.params.embedding"]))
    assert torch.equal(model.ln_f.weight, torch.from_numpy(save["param.params.ln_f.weight"]))


def test_loader_rejects_short_or_misshaped_archives(tmp_path):
    cfg = M.model_config(TPU2BLike())
    save, _ = _archive(cfg)
    short = {k: v for k, v in save.items() if "block_11." not in k}
    p1 = str(tmp_path / "short.nbpack.npz")
    np.savez_compressed(p1, **short)
    with pytest.raises(ValueError, match="quantized layers"):
        M.load_packed_model(p1, TPU2BLike(), device="cpu")

    class Wider(TPU2BLike):
        ffn_hidden = 512
    p2 = str(tmp_path / "full.nbpack.npz")
    np.savez_compressed(p2, **save)
    with pytest.raises(ValueError, match="needs"):
        M.load_packed_model(p2, Wider(), device="cpu")


def test_kv_cache_shapes_and_layout():
    model = M.PackedGPT(50, 3, 64, 4, 96, 16, M.UnloadedLinear)
    caches = M.init_kv_cache(model, batch_size=2, device="cpu")
    assert len(caches) == 3
    for k, v, n in caches:
        assert k.shape == v.shape == (2, 4, 16, 16) and n == 0
        assert k.transpose(-1, -2).is_contiguous() and v.is_contiguous()
    k, v, _ = caches[0]
    kt, vt, kc, vc = M._cache_storage(k, v, 2, 4, 16)
    assert not kc and not vc and kt.data_ptr() == k.data_ptr()
    # a contiguous cache of the reference's layout is accepted (copied)
    kr = torch.zeros(2, 4, 16, 16)
    kt, _, kc, _ = M._cache_storage(kr, v, 2, 4, 16)
    assert kc and kt.shape == (2, 4, 16, 16) and kt.is_contiguous()
    with pytest.raises(ValueError, match="head_dim"):
        M._cache_storage(torch.zeros(2, 4, 16, 8), v, 2, 4, 16)
    with pytest.raises(ValueError, match="float32"):
        M._cache_storage(k.half(), v, 2, 4, 16)
    with pytest.raises(ValueError, match="positions"):
        M._cache_storage(k, torch.zeros(2, 4, 12, 16), 2, 4, 16)
