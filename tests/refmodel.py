"""Shared test fixtures for the reference-caller tests: a config object with
exactly TPU2BConfig's attribute names, and a .nbpack.npz archive in the
reference packer's key layout and key order."""
import numpy as np

from nativebit_amd import synth


class TPU2BLike:
    """TPU2BConfig's attribute names and nothing else (configs/tpu.py:137-151),
    at a small shape."""
    n_layers = 12
    n_embd = 256
    n_head = 4
    ffn_hidden = 384
    context_len = 32
    vocab_size = 300
    block_size = 128
    n_codebook = 8
    batch_size = 64
    lr = 3e-4
    codebook_lr = 3e-5
    max_steps = 20000
    warmup_steps = 1000
    grad_clip = 1.0
    codebook_grad_clip = 1.0
    log_every = 100


def archive(cfg, seed=3):
    """A .nbpack.npz dict in the reference packer's key layout and key order
    (sorted prefixes, inference/pack.py:114-124; params after), plus each
    layer's (packed, codebook) by block and name for checking."""
    C, F = cfg.n_embd, cfg.ffn_hidden
    names = [("CausalSelfAttention_0.NativeBitDense_0", (3 * C, C)),
             ("CausalSelfAttention_0.NativeBitDense_1", (C, C)),
             ("SwiGLU_0.NativeBitDense_0", (F, C)), ("SwiGLU_0.NativeBitDense_1", (F, C)),
             ("SwiGLU_0.NativeBitDense_2", (C, F))]
    layers, truth = {}, {}
    for i in range(cfg.n_layers):
        for j, (n, (o, k)) in enumerate(names):
            lay = synth.make_layer(o, k, 8, 128, seed=seed * 100 + i * 10 + j, device="cpu")
            layers[f"params.block_{i}.{n}"] = (lay.packed.numpy(), lay.codebook.numpy(), (o, k))
            truth[(i, j)] = lay
    save = {}
    for p in sorted(layers):            # alphabetical: block_10 before block_2
        packed, cb, shape = layers[p]
        save[f"idx.{p}"] = packed
        save[f"cb.{p}"] = cb
        save[f"shape.{p}"] = np.array(shape)
        save[f"idxshape.{p}"] = np.array([cb.shape[0], 128])
    rng = np.random.default_rng(seed)
    for i in range(cfg.n_layers):
        save[f"param.params.block_{i}.RMSNorm_0.weight"] = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
        save[f"param.params.block_{i}.RMSNorm_1.weight"] = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    save["param.params.embedding"] = (0.02 * rng.standard_normal((cfg.vocab_size, C))).astype(np.float32)
    save["param.params.ln_f.weight"] = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    save["__metadata__"] = np.array([128, 8, 5 * cfg.n_layers, 2 * cfg.n_layers + 2])
    return save, truth
