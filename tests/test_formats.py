"""The reference's packed checkpoint formats (nativebit_amd.formats), on CPU.

.nbpack.npz (inference/pack.py:60-156, read as generate_torch.py:176-266)
and format v1 (nativebit/pack.py:202-415): byte-exact streams against the
oracle's packer of the oracle's nearest-entry indices, the archive's key
layout, natural-sort layer order, training-only keys dropped, and a loud
failure on corrupt or truncated files.
"""
import numpy as np
import pytest
import torch

from nativebit_amd import formats
from oracle import oracle as O


def jax_like_params(n_blocks=3, C=256, F=512, V=64, bs=128, seed=0):
    """A tiny training checkpoint in the '/'-joined layout of the JAX
    trainer: per block qkv/out_proj/gate/up/down NativeBitDense weights (out,
    in) with per-block codebooks, RMSNorm weights, embedding, ln_f, and
    training-only state that the packer must drop."""
    rng = np.random.default_rng(seed)
    p = {"params/embedding": rng.standard_normal((V, C)).astype(np.float32) * 0.02,
         "params/ln_f/weight": np.ones(C, np.float32)}
    shapes = {"CausalSelfAttention_0/NativeBitDense_0": (3 * C, C),
              "CausalSelfAttention_0/NativeBitDense_1": (C, C),
              "SwiGLU_0/NativeBitDense_0": (F, C), "SwiGLU_0/NativeBitDense_1": (F, C),
              "SwiGLU_0/NativeBitDense_2": (C, F)}
    for i in range(n_blocks):
        for name, (o, k) in shapes.items():
            pre = f"params/block_{i}/{name}"
            w = rng.standard_normal((o, k)).astype(np.float32) * 0.02
            nb = o * k // bs
            cb = np.sort(rng.standard_normal((nb, 8)).astype(np.float32) * 0.02, axis=1)
            p[pre + "/weight"] = w
            p[pre + "/codebook"] = cb
            p[pre + "/qw_delta"] = np.zeros_like(w)
            p[pre + "/ema_N"] = np.zeros((nb, 8), np.float32)
        p[f"params/block_{i}/RMSNorm_0/weight"] = rng.standard_normal(C).astype(np.float32)
        p[f"params/block_{i}/RMSNorm_1/weight"] = rng.standard_normal(C).astype(np.float32)
    return p


def test_natural_key_order():
    keys = ["params.block_10.x", "params.block_2.x", "params.block_1.x"]
    assert sorted(keys, key=formats.natural_key) == [
        "params.block_1.x", "params.block_2.x", "params.block_10.x"]


def test_pack_checkpoint_roundtrip(tmp_path):
    params = jax_like_params(n_blocks=11)  # block_10 sorts after block_9
    path = formats.pack_checkpoint(params, str(tmp_path / "m.nbpack"))
    assert path.endswith(".npz")
    with np.load(path, allow_pickle=False) as f:
        files = set(f.files)
        meta = f["__metadata__"]
    assert list(meta) == [128, 8, 55, 2 + 2 * 11]
    assert not any("qw_delta" in k or "ema_N" in k or k.endswith(".codebook") for k in files
                   if k.startswith("param."))
    pack = formats.load_nbpack(path)
    assert len(pack.layers) == 55
    order = [e.prefix for e in pack.layers]
    assert order == sorted(order, key=formats.natural_key)
    assert order[5].startswith("params.block_1.") and order[-1].startswith("params.block_10.")
    assert order[:5] == [f"params.block_0.{n}" for n in (
        "CausalSelfAttention_0.NativeBitDense_0", "CausalSelfAttention_0.NativeBitDense_1",
        "SwiGLU_0.NativeBitDense_0", "SwiGLU_0.NativeBitDense_1", "SwiGLU_0.NativeBitDense_2")]
    for e in pack.layers[:10]:
        key = e.prefix.replace(".", "/")
        w, cb = params[key + "/weight"], params[key + "/codebook"]
        idx = O.quantize(w, cb, 128)
        assert np.array_equal(e.packed, O.pack(idx, 3))
        assert np.array_equal(e.codebook, cb)
        assert e.shape == w.shape and e.idxshape == (cb.shape[0], 128)
        assert np.array_equal(e.indices().reshape(-1), idx)
    assert np.array_equal(pack.params["params/embedding"], params["params/embedding"])
    assert "params/block_3/RMSNorm_1/weight" in pack.params


@pytest.mark.parametrize("damage", ["drop_cb", "truncate", "bad_idxshape", "bad_meta"])
def test_corrupt_nbpack_raises(tmp_path, damage):
    path = formats.pack_checkpoint(jax_like_params(n_blocks=1), str(tmp_path / "m.nbpack.npz"))
    with np.load(path, allow_pickle=False) as f:
        d = {k: f[k] for k in f.files}
    victim = sorted(k for k in d if k.startswith("idx."))[0][4:]
    if damage == "drop_cb":
        del d["cb." + victim]
    elif damage == "truncate":
        d["idx." + victim] = d["idx." + victim][:-7]
    elif damage == "bad_idxshape":
        d["idxshape." + victim] = np.array([3, 128])
    else:
        d["__metadata__"] = np.array([128])
    bad = str(tmp_path / "bad.nbpack.npz")
    np.savez_compressed(bad, **d)
    with pytest.raises(ValueError):
        formats.load_nbpack(bad)


def test_v1_roundtrip(tmp_path):
    rng = np.random.default_rng(3)
    layers = {}
    for name, (o, k) in {"blocks.0.attn.qkv": (96, 32), "blocks.0.ffn.w_down": (32, 64)}.items():
        nb = -(-o * k // 64)
        layers[name] = {"indices": rng.integers(0, 8, nb * 64, dtype=np.uint8),
                        "codebook": rng.standard_normal((nb, 8)).astype(np.float32),
                        "shape": (o, k), "block_size": 64}
    fp = {"tok_emb.weight": torch.randn(10, 32)}
    path = str(tmp_path / "m.pt")
    formats.save_packed_v1(path, layers, fp, {"n_embd": 32}, n_entries=8)
    st = formats.load_packed_v1(path)
    assert st["format_version"] == 1 and st["bits"] == 3 and st["n_entries"] == 8
    for name, d in layers.items():
        e = st["quantized_layers"][name]
        assert e["shape"] == d["shape"] and e["block_size"] == 64
        assert e["num_blocks"] == d["codebook"].shape[0]
        assert e["total_weights"] == d["shape"][0] * d["shape"][1]
        assert np.array_equal(e["packed_indices"].numpy(), O.pack(d["indices"], 3))
        assert e["codebook"].dtype == torch.float16
        assert torch.equal(e["codebook_f32"], torch.from_numpy(d["codebook"]).half().float())
    assert st["float_params"]["tok_emb.weight"].dtype == torch.float16


def test_v1_rejects_other_versions(tmp_path):
    path = str(tmp_path / "x.pt")
    torch.save({"format_version": 2}, path)
    with pytest.raises(ValueError):
        formats.load_packed_v1(path)
