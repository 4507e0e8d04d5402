"""The reference's packed checkpoint formats, read and written on the host.

Two formats carry NativeBit models to inference:

* ``.nbpack.npz`` (inference/pack.py:60-156): a numpy archive with, per
  quantized layer ``<p>`` (the parameter path with '/' replaced by '.'),
  ``idx.<p>`` the 3-bit stream (uint8), ``cb.<p>`` the fp32 codebooks
  (num_blocks, n_entries), ``shape.<p>`` the weight shape (out, in) and
  ``idxshape.<p>`` the index array shape (num_blocks, block_size); every other
  parameter as ``param.<path>``; and ``__metadata__`` = [block_size,
  n_entries, n_quantized, n_other].  Written with ``np.savez_compressed``.
* format v1 (nativebit/pack.py:202-336): a ``torch.save`` dict
  ``{format_version, config, bits, n_entries, quantized_layers: {name:
  {packed_indices, codebook (fp16), shape, block_size, n_entries,
  num_blocks, total_weights[, bias]}}, float_params}``.

Readers validate what they read and raise ``ValueError`` on a corrupt or
truncated file; archives are opened without pickle (``allow_pickle=False``,
``torch.load(weights_only=True)``).  Packed streams are uploaded to the
device as they are: a stream is the device format byte for byte.
"""
from __future__ import annotations

import math
import os
import re
from dataclasses import dataclass, field

import numpy as np
import torch

from . import pack as host_pack

FORMAT_VERSION = host_pack.FORMAT_VERSION
_TRAINING_ONLY_TAGS = ("/qw_delta", "/ema_N", "/ema_s")  # inference/pack.py:91-94


def natural_key(s: str):
    """Sort key that orders block_2 before block_10 (generate_torch.py:226-228)."""
    return [int(c) if c.isdigit() else c for c in re.split(r"(\d+)", s)]


@dataclass
class PackedEntry:
    """One quantized layer of a .nbpack.npz archive."""
    prefix: str                 # '.'-joined parameter path of the layer
    packed: np.ndarray          # uint8 3-bit stream
    codebook: np.ndarray        # (num_blocks, n_entries) float32
    shape: tuple                # (out_features, in_features)
    idxshape: tuple             # (num_blocks, block_size)

    @property
    def block_size(self) -> int:
        return int(self.idxshape[1])

    def indices(self) -> np.ndarray:
        """Unpacked uint8 indices, (num_blocks, block_size)."""
        nb, bs = self.idxshape
        return host_pack.unpack_bits_np(self.packed, nb * bs, 3).reshape(nb, bs)


@dataclass
class NBPack:
    """Contents of a .nbpack.npz archive."""
    layers: list = field(default_factory=list)   # PackedEntry, natural-sorted by prefix
    params: dict = field(default_factory=dict)   # '/'-joined path -> ndarray
    block_size: int = 128
    n_entries: int = 8

    def layer(self, prefix: str) -> PackedEntry:
        for e in self.layers:
            if e.prefix == prefix:
                return e
        raise KeyError(prefix)


def _quantized_prefixes(keys):
    """Parameter paths that have both a weight and a codebook
    (inference/pack.py:68-77)."""
    keyset = set(keys)
    out = {}
    for k in keys:
        if k.endswith("/weight"):
            prefix = k.rsplit("/weight", 1)[0]
            if prefix + "/codebook" in keyset:
                out[prefix] = (k, prefix + "/codebook")
    return out


def pack_checkpoint(ckpt, out_path: str, block_size: int = 128, n_entries: int = 8) -> str:
    """Training parameters -> .nbpack.npz (inference/pack.py:60-156).

    ``ckpt`` is a path to an ``.npz`` of '/'-joined parameter paths (the
    JAX training checkpoint layout) or a dict of the same.  Each quantized
    layer's latent weight is assigned to its nearest codebook entry
    (squared distance, first index on ties) and 3-bit packed; other
    parameters are kept except training-only state.  Returns the path
    written (``.npz`` appended if missing, as numpy does).
    """
    if isinstance(ckpt, (str, os.PathLike)):
        with np.load(ckpt, allow_pickle=False) as f:
            ckpt = {k: f[k] for k in f.files}
    keys = list(ckpt.keys())
    quantized = _quantized_prefixes(keys)
    save = {}
    for prefix, (wk, ck) in sorted(quantized.items()):
        weight = np.asarray(ckpt[wk], dtype=np.float32)
        codebook = np.asarray(ckpt[ck], dtype=np.float32)
        if codebook.ndim != 2 or codebook.shape[1] > 8:
            raise ValueError(f"{ck}: expected (num_blocks, <=8) codebook, got {codebook.shape}")
        indices = host_pack.quantize_weight(weight, codebook)
        safe = prefix.replace("/", ".")
        save[f"idx.{safe}"] = host_pack.pack_bits_np(indices, 3)
        save[f"cb.{safe}"] = codebook
        save[f"shape.{safe}"] = np.array(weight.shape)
        save[f"idxshape.{safe}"] = np.array(indices.shape)
    other = []
    for k in keys:
        prefix = k.rsplit("/", 1)[0] if "/" in k else ""
        if prefix in quantized and k.endswith("/weight"):
            continue
        if k.endswith("/codebook") or any(t in k for t in _TRAINING_ONLY_TAGS):
            continue
        other.append(k)
    for k in other:
        arr = np.asarray(ckpt[k])
        if arr.dtype.kind == "V":  # bfloat16 stored as void: kept as 2-byte floats
            arr = np.frombuffer(arr.tobytes(), dtype=np.float16).reshape(arr.shape)
        save[f"param.{k.replace('/', '.')}"] = arr
    save["__metadata__"] = np.array([block_size, n_entries, len(quantized), len(other)])
    np.savez_compressed(out_path, **save)
    return out_path if str(out_path).endswith(".npz") else str(out_path) + ".npz"


def load_nbpack(path: str) -> NBPack:
    """Read and validate a .nbpack.npz (generate_torch.py:180-201)."""
    out = NBPack()
    with np.load(path, allow_pickle=False) as f:
        files = set(f.files)
        if "__metadata__" in files:
            meta = f["__metadata__"]
            if meta.size < 2:
                raise ValueError(f"{path}: __metadata__ has {meta.size} fields")
            out.block_size, out.n_entries = int(meta[0]), int(meta[1])
        for key in sorted((k for k in files if k.startswith("idx.")), key=natural_key):
            p = key[4:]
            missing = [f"{t}.{p}" for t in ("cb", "shape", "idxshape") if f"{t}.{p}" not in files]
            if missing:
                raise ValueError(f"{path}: layer {p} lacks {', '.join(missing)}")
            packed = np.ascontiguousarray(f[key], dtype=np.uint8).reshape(-1)
            cb = np.ascontiguousarray(f[f"cb.{p}"], dtype=np.float32)
            shape = tuple(int(v) for v in f[f"shape.{p}"])
            idxshape = tuple(int(v) for v in f[f"idxshape.{p}"])
            if len(shape) != 2 or len(idxshape) != 2:
                raise ValueError(f"{path}: layer {p} shape {shape} / idxshape {idxshape}")
            nb, bs = idxshape
            if cb.ndim != 2 or cb.shape[0] != nb:
                raise ValueError(f"{path}: layer {p} codebook {cb.shape} vs {nb} blocks")
            if nb != math.ceil(shape[0] * shape[1] / bs):
                raise ValueError(f"{path}: layer {p}: {nb} blocks of {bs} for shape {shape}")
            if packed.size < host_pack.packed_nbytes(nb * bs, 3):
                raise ValueError(f"{path}: layer {p} stream of {packed.size} bytes is truncated")
            out.layers.append(PackedEntry(p, packed, cb, shape, idxshape))
        for key in files:
            if key.startswith("param."):
                arr = f[key]
                if arr.dtype.kind == "V":
                    arr = np.frombuffer(arr.tobytes(), dtype=np.float16).reshape(arr.shape)
                out.params[key[6:].replace(".", "/")] = arr
    return out


# ---------------------------------------------------------------------------
# format v1 (torch.save)
# ---------------------------------------------------------------------------

def save_packed_v1(path: str, layers: dict, float_params: dict, config: dict,
                   n_entries: int = 8) -> None:
    """Write format v1 (nativebit/pack.py:256-320).

    ``layers``: name -> dict(indices=(uint8 flat or (num_blocks, bs)),
    codebook=(num_blocks, n_entries) float, shape=(out, in), block_size=int
    [, bias]).  Indices are packed at ceil(log2 n_entries) bits, codebooks
    and float parameters stored as fp16, as the reference does.
    """
    bits = host_pack.bits_for_entries(n_entries)
    state = {"format_version": FORMAT_VERSION, "config": dict(config), "bits": bits,
             "n_entries": n_entries, "quantized_layers": {}, "float_params": {}}
    for name, d in layers.items():
        cb = torch.as_tensor(d["codebook"], dtype=torch.float32)
        num_blocks = cb.shape[0]
        out_f, in_f = (int(v) for v in d["shape"])
        entry = {
            "packed_indices": host_pack.pack_nbits(torch.as_tensor(d["indices"]).reshape(-1), bits),
            "codebook": cb.half(),
            "shape": (out_f, in_f),
            "block_size": int(d["block_size"]),
            "n_entries": n_entries,
            "num_blocks": int(num_blocks),
            "total_weights": out_f * in_f,
        }
        if d.get("bias") is not None:
            entry["bias"] = torch.as_tensor(d["bias"]).half()
        state["quantized_layers"][name] = entry
    for name, t in float_params.items():
        state["float_params"][name] = torch.as_tensor(t).half()
    torch.save(state, path)


def load_packed_v1(path: str) -> dict:
    """Read and validate format v1 (nativebit/pack.py:343-415) without
    unpickling arbitrary objects.  Returns the state dict; each quantized
    layer gains ``codebook_f32`` (exact fp16 -> fp32 widening)."""
    state = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(state, dict) or state.get("format_version") != FORMAT_VERSION:
        raise ValueError(f"{path}: not a format v{FORMAT_VERSION} packed model")
    bits = int(state["bits"])
    for name, d in state["quantized_layers"].items():
        for k in ("packed_indices", "codebook", "shape", "block_size", "num_blocks", "total_weights"):
            if k not in d:
                raise ValueError(f"{path}: layer {name} lacks {k}")
        need = host_pack.packed_nbytes(int(d["num_blocks"]) * int(d["block_size"]), bits)
        if d["packed_indices"].numel() < need:
            raise ValueError(f"{path}: layer {name} stream is truncated")
        d["codebook_f32"] = d["codebook"].float()
    return state


def packed_linear(entry: PackedEntry, device="cuda", out_dtype=torch.float32):
    """A PackedLinear holding an archive layer (stream uploaded as is)."""
    from .linear import PackedLinear
    layer = PackedLinear.from_stream(entry.packed, entry.codebook, entry.shape, device=device,
                                     block_size=entry.block_size, bits=3)
    layer.out_dtype = out_dtype
    return layer
