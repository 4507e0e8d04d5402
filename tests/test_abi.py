"""The C ABI without a GPU: the library loads, exports exactly what
include/nativebit_amd.h declares, and rejects bad arguments on the host
before any launch (no compute call is made here).

Pointers passed below are never dereferenced: every call either fails
validation or has nothing to do (N == 0 / count == 0).
"""
import ctypes
import os
import re
import subprocess

import pytest

from nativebit_amd import _lib
from tests.conftest import ROOT, gpu_available

HEADER = os.path.join(ROOT, "include", "nativebit_amd.h")
FAKE = 0x100000  # aligned, never dereferenced


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(nb_[a-z_0-9]+)\s*\(", text))


def test_header_and_binding_agree():
    assert declared() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (nb_\w+)$", out, flags=re.M))
    assert declared() <= exported
    for name in declared():
        assert getattr(lib, name) is not None
    assert lib.nb_abi_version() == 2


def test_packed_nbytes(golden):
    lib = _lib.load()
    for e in golden["lengths"]:
        assert lib.nb_packed_nbytes(e["count"], e["bits"]) == e["nbytes"]
    assert lib.nb_packed_nbytes(10, 0) == 0 and lib.nb_packed_nbytes(10, 9) == 0


def gemv(**kw):
    a = dict(x=FAKE, x_dtype=_lib.NB_F32, ldx=0, packed=FAKE, codebook=FAKE, y=FAKE,
             y_dtype=_lib.NB_F32, ldy=0, M=1, N=8, K=256, bits=3, n_entries=8,
             block_size=128, stream=None)
    a.update(kw)
    return _lib.load().nb_gemv(*a.values())


@pytest.mark.parametrize("kw,status", [
    (dict(M=0), _lib.NB_EUNSUPPORTED),
    (dict(M=17), _lib.NB_EUNSUPPORTED),
    (dict(N=-1), _lib.NB_EINVAL),
    (dict(bits=0), _lib.NB_EUNSUPPORTED),
    (dict(bits=9), _lib.NB_EUNSUPPORTED),
    (dict(n_entries=9), _lib.NB_EINVAL),
    (dict(n_entries=0), _lib.NB_EINVAL),
    (dict(block_size=0), _lib.NB_EINVAL),
    (dict(x_dtype=7), _lib.NB_EINVAL),
    (dict(y_dtype=_lib.NB_U8), _lib.NB_EINVAL),
    (dict(M=2, ldx=100), _lib.NB_EINVAL),
    (dict(M=2, ldx=256, ldy=4), _lib.NB_EINVAL),
    (dict(y=None), _lib.NB_EINVAL),
    (dict(packed=None), _lib.NB_EINVAL),
    (dict(codebook=None), _lib.NB_EINVAL),
    (dict(y=FAKE + 2), _lib.NB_EALIGN),
    (dict(x=FAKE + 1, x_dtype=_lib.NB_BF16), _lib.NB_EALIGN),
    (dict(codebook=FAKE + 2), _lib.NB_EALIGN),
])
def test_gemv_validation(kw, status):
    assert gemv(**kw) == status
    assert _lib.last_error()  # a message for every failure


def test_gemv_empty_is_noop():
    assert gemv(N=0, y=None, x=None) == _lib.NB_OK


def test_codec_validation():
    lib = _lib.load()
    assert lib.nb_unpack(FAKE, FAKE, 10, 9, None) == _lib.NB_EUNSUPPORTED
    assert lib.nb_unpack(FAKE, FAKE, -1, 3, None) == _lib.NB_EINVAL
    assert lib.nb_unpack(None, FAKE, 10, 3, None) == _lib.NB_EINVAL
    assert lib.nb_unpack(None, None, 0, 3, None) == _lib.NB_OK
    assert lib.nb_pack(FAKE, None, 10, 3, None) == _lib.NB_EINVAL
    assert lib.nb_pack(FAKE, FAKE, 10, 0, None) == _lib.NB_EUNSUPPORTED
    dq = lib.nb_dequant
    assert dq(FAKE, FAKE, FAKE, _lib.NB_F32, 1000, 7, 3, 8, 128, None) == _lib.NB_EINVAL
    assert dq(FAKE, FAKE, FAKE, _lib.NB_U8, 100, 1, 3, 8, 128, None) == _lib.NB_EINVAL
    assert dq(FAKE, FAKE + 1, FAKE, _lib.NB_F32, 100, 1, 3, 8, 128, None) == _lib.NB_EALIGN
    assert dq(FAKE, FAKE, FAKE + 1, _lib.NB_BF16, 100, 1, 3, 8, 128, None) == _lib.NB_EALIGN
    assert dq(FAKE, FAKE, FAKE, _lib.NB_F32, 100, 1, 3, 9, 128, None) == _lib.NB_EINVAL
    assert dq(None, None, None, _lib.NB_F32, 0, 0, 3, 8, 128, None) == _lib.NB_OK


@pytest.mark.skipif(gpu_available(), reason="only meaningful without a GPU")
def test_valid_call_without_gpu_reports_nodev():
    # All arguments valid: validation passes and the device check refuses.
    assert gemv() == _lib.NB_ENODEV
    assert "gfx950" in _lib.last_error() or "hip" in _lib.last_error().lower()


def test_error_message_is_thread_local():
    import threading
    gemv(M=0)
    msgs = []
    t = threading.Thread(target=lambda: msgs.append(_lib.last_error()))
    t.start()
    t.join()
    assert msgs == [""]
    assert "M=0" in _lib.last_error()


def test_python_wrappers_refuse_cpu_tensors():
    import torch
    from nativebit_amd import ops
    with pytest.raises(ValueError, match="GPU"):
        ops.gemv(torch.zeros(256), torch.zeros(96, dtype=torch.uint8),
                 torch.zeros(2, 8), 1, 256)
    with pytest.raises(ValueError, match="GPU"):
        ops.pack(torch.zeros(8, dtype=torch.uint8), 3)


def test_ctypes_types():
    # the stream argument is a plain pointer in the ABI
    assert _lib.SIGNATURES["nb_gemv"][1][-1] is ctypes.c_void_p


def test_batch_validation():
    lib = _lib.load()
    Item = _lib.BatchItem
    good = Item(FAKE, FAKE, FAKE, FAKE, 32, 256)
    arr = (Item * 2)(good, good)
    nbytes = lib.nb_gemv_batch_table_bytes(2)
    assert nbytes > 0 and lib.nb_gemv_batch_table_bytes(0) == 0
    buf = ctypes.create_string_buffer(nbytes)
    assert lib.nb_gemv_batch_plan(arr, 2, buf, nbytes) == _lib.NB_OK
    assert lib.nb_gemv_batch_plan(arr, 2, buf, nbytes - 1) == _lib.NB_EINVAL
    assert lib.nb_gemv_batch_plan(arr, -1, buf, nbytes) == _lib.NB_EINVAL
    for bad, st in ((Item(FAKE, FAKE, FAKE, FAKE, 32, 200), _lib.NB_EUNSUPPORTED),
                    (Item(FAKE, FAKE, FAKE, FAKE, 32, 8320), _lib.NB_EUNSUPPORTED),
                    (Item(FAKE + 8, FAKE, FAKE, FAKE, 32, 256), _lib.NB_EALIGN),
                    (Item(FAKE, None, FAKE, FAKE, 32, 256), _lib.NB_EINVAL),
                    (Item(FAKE, FAKE, FAKE, FAKE, -1, 256), _lib.NB_EINVAL)):
        one = (Item * 1)(bad)
        assert lib.nb_gemv_batch_plan(one, 1, buf, nbytes) == st
        assert lib.nb_gemv_batched(one, FAKE, 1, _lib.NB_F32, None) == st
    assert lib.nb_gemv_batched(arr, None, 2, _lib.NB_F32, None) == _lib.NB_EINVAL
    assert lib.nb_gemv_batched(arr, FAKE, 2, 7, None) == _lib.NB_EINVAL
    empty = (Item * 1)(Item(None, None, None, None, 0, 256))
    assert lib.nb_gemv_batched(empty, None, 1, _lib.NB_F32, None) == _lib.NB_OK


def test_batch_fused_forms_validation():
    """x_mode / y_mode / norm_w / eps of nb_batch_item, checked on the host."""
    lib = _lib.load()
    Item = _lib.BatchItem
    nbytes = lib.nb_gemv_batch_table_bytes(1)
    buf = ctypes.create_string_buffer(nbytes)
    X, Y = _lib.NB_X_RMSNORM, _lib.NB_Y_ADD

    def plan(*a):
        one = (Item * 1)(Item(*a))
        return lib.nb_gemv_batch_plan(one, 1, buf, nbytes)

    def batched(y_dtype, *a):
        one = (Item * 1)(Item(*a))
        return lib.nb_gemv_batched(one, FAKE, 1, y_dtype, None)

    base = (FAKE, FAKE, FAKE, FAKE, 32, 256)
    assert plan(*base, X, Y, FAKE, 1e-5, 0) == _lib.NB_OK
    assert plan(*base, _lib.NB_X_SILU_MUL, 0, None, 0.0, 0) == _lib.NB_OK
    assert plan(*base, 3, 0, None, 0.0, 0) == _lib.NB_EINVAL           # unknown x_mode
    assert plan(*base, -1, 0, None, 0.0, 0) == _lib.NB_EINVAL
    assert plan(*base, 0, 3, None, 0.0, 0) == _lib.NB_EINVAL           # unknown y_mode
    P2 = _lib.NB_Y_SILU_PAIRS
    assert plan(*base, X, P2, FAKE, 1e-5, 0) == _lib.NB_OK             # gate|up pairs
    assert plan(FAKE, FAKE, FAKE, FAKE, 33, 256, 0, P2, None, 0.0, 0) == _lib.NB_EINVAL  # odd N
    two = (Item * 2)(Item(*base, 0, P2, None, 0.0, 0), Item(*base, 0, 0, None, 0.0, 0))
    assert lib.nb_gemv_batch_plan(two, 2, ctypes.create_string_buffer(
        lib.nb_gemv_batch_table_bytes(2)), lib.nb_gemv_batch_table_bytes(2)) == \
        _lib.NB_EUNSUPPORTED                                            # pairs not alone
    assert batched(_lib.NB_F32, *base, 0, P2, None, 0.0, 0) == _lib.NB_EUNSUPPORTED  # bf16 only
    assert plan(*base, X, 0, None, 1e-5, 0) == _lib.NB_EINVAL          # rmsnorm without weights
    assert plan(*base, X, 0, FAKE + 4, 1e-5, 0) == _lib.NB_EALIGN      # weights misaligned
    assert plan(*base, X, 0, FAKE, -1.0, 0) == _lib.NB_EINVAL          # negative eps
    assert plan(*base, X, 0, FAKE, float("nan"), 0) == _lib.NB_EINVAL
    assert plan(*base, 0, 0, None, 0.0, 1) == _lib.NB_EINVAL           # reserved not zero
    # y += result is fp32 only
    assert batched(_lib.NB_BF16, *base, 0, Y, None, 0.0, 0) == _lib.NB_EUNSUPPORTED


def test_linspace01_equals_torch():
    """The quantile fractions of nb_block_codebooks are torch.linspace's,
    bit for bit, for every entry count it takes."""
    import torch
    lib = _lib.load()
    for n in range(1, 257):
        buf = (ctypes.c_float * n)()
        assert lib.nb_linspace01(n, buf) == _lib.NB_OK
        assert torch.equal(torch.tensor(list(buf), dtype=torch.float32), torch.linspace(0, 1, n)), n
    assert lib.nb_linspace01(0, (ctypes.c_float * 1)()) == _lib.NB_EINVAL
    assert lib.nb_linspace01(257, (ctypes.c_float * 257)()) == _lib.NB_EINVAL


def test_block_codebooks_validation():
    c = _lib.load().nb_block_codebooks
    assert c(FAKE, 0, 128, 8, FAKE, None) == _lib.NB_OK
    assert c(FAKE, 100, 0, 8, FAKE, None) == _lib.NB_EUNSUPPORTED
    assert c(FAKE, 100, 1025, 8, FAKE, None) == _lib.NB_EUNSUPPORTED
    assert c(FAKE, 100, 128, 0, FAKE, None) == _lib.NB_EUNSUPPORTED
    assert c(FAKE, 100, 128, 257, FAKE, None) == _lib.NB_EUNSUPPORTED
    assert c(FAKE, -1, 128, 8, FAKE, None) == _lib.NB_EINVAL
    assert c(None, 100, 128, 8, FAKE, None) == _lib.NB_EINVAL
    assert c(FAKE + 2, 100, 128, 8, FAKE, None) == _lib.NB_EALIGN


def test_quantize_pack_validation():
    """nb_quantize_pack: format and tiling checks on the host."""
    q = _lib.load().nb_quantize_pack
    ok = (FAKE, 1000, FAKE, 8, 8, 125, 3, FAKE, None)
    assert q(*ok[:1], 0, FAKE, 0, 8, 125, 3, FAKE, None) == _lib.NB_OK      # nothing to do
    for i, bad, st in ((6, 0, _lib.NB_EUNSUPPORTED), (6, 9, _lib.NB_EUNSUPPORTED),   # bits
                       (4, 9, _lib.NB_EINVAL), (4, 0, _lib.NB_EINVAL),               # entries > 2^bits
                       (5, 0, _lib.NB_EINVAL),                                        # block size
                       (3, 7, _lib.NB_EINVAL), (3, 9, _lib.NB_EINVAL),               # blocks don't tile
                       (1, -1, _lib.NB_EINVAL),
                       (0, None, _lib.NB_EINVAL), (7, None, _lib.NB_EINVAL),
                       (0, FAKE + 2, _lib.NB_EALIGN)):
        a = list(ok)
        a[i] = bad
        assert q(*a) == st, (i, bad)


def test_skinny_batch_validation():
    """nb_gemm_skinny_batched: M range, bf16 activations only, the shared
    item checks and the y_dtype / NB_Y_ADD rules, all on the host."""
    lib = _lib.load()
    Item = _lib.BatchItem
    good = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 256))
    sk = lib.nb_gemm_skinny_batched
    for M in (0, -1, 17):
        assert sk(good, FAKE, 1, M, _lib.NB_F32, None) == _lib.NB_EINVAL
    assert sk(good, FAKE, 1, 4, 7, None) == _lib.NB_EINVAL
    assert sk(good, None, 1, 4, _lib.NB_F32, None) == _lib.NB_EINVAL
    assert sk(good, FAKE + 4, 1, 4, _lib.NB_F32, None) == _lib.NB_EALIGN
    norm = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 256, _lib.NB_X_RMSNORM, 0, FAKE, 1e-5, 0))
    assert sk(norm, FAKE, 1, 4, _lib.NB_F32, None) == _lib.NB_EUNSUPPORTED
    add16 = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 256, 0, _lib.NB_Y_ADD, None, 0.0, 0))
    assert sk(add16, FAKE, 1, 4, _lib.NB_BF16, None) == _lib.NB_EUNSUPPORTED
    for bad, st in ((Item(FAKE, FAKE, FAKE, FAKE, 32, 200), _lib.NB_EUNSUPPORTED),
                    (Item(FAKE + 8, FAKE, FAKE, FAKE, 32, 256), _lib.NB_EALIGN),
                    (Item(FAKE, FAKE, FAKE, FAKE, -1, 256), _lib.NB_EINVAL)):
        assert sk((Item * 1)(bad), FAKE, 1, 4, _lib.NB_F32, None) == st
    empty = (Item * 1)(Item(None, None, None, None, 0, 256))
    assert sk(empty, None, 1, 4, _lib.NB_F32, None) == _lib.NB_OK


def test_quad_batch_and_layout_validation():
    """nb_gemm_skinny_quad_batched: M <= 4, K >= 2048, plus the skinny
    checks; nb_quad_layout: shape, pointers and alignment; the layout's
    byte count (ceil(N / 4) * 4 rows of K / 128 blocks of 48 bytes)."""
    lib = _lib.load()
    Item = _lib.BatchItem
    good = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 2048))
    qs = lib.nb_gemm_skinny_quad_batched
    for M in (0, 5, 16):
        assert qs(good, FAKE, 1, M, _lib.NB_F32, None) == _lib.NB_EINVAL
    assert _lib.last_error().startswith("nb_gemm_skinny_quad_batched")
    short = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 1920))
    assert qs(short, FAKE, 1, 4, _lib.NB_F32, None) == _lib.NB_EUNSUPPORTED
    assert qs(good, None, 1, 4, _lib.NB_F32, None) == _lib.NB_EINVAL
    add16 = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 2048, 0, _lib.NB_Y_ADD, None, 0.0, 0))
    assert qs(add16, FAKE, 1, 2, _lib.NB_BF16, None) == _lib.NB_EUNSUPPORTED
    empty = (Item * 1)(Item(None, None, None, None, 0, 2048))
    assert qs(empty, None, 1, 4, _lib.NB_F32, None) == _lib.NB_OK
    assert lib.nb_quad_layout_bytes(8, 2048) == 8 * 16 * 48
    assert lib.nb_quad_layout_bytes(9, 256) == 12 * 2 * 48
    assert lib.nb_quad_layout_bytes(0, 256) == 0 and lib.nb_quad_layout_bytes(4, 200) == 0
    ql = lib.nb_quad_layout
    assert ql(FAKE, FAKE, 8, 200, FAKE, FAKE, None) == _lib.NB_EINVAL
    assert ql(FAKE, FAKE, 8, 8320, FAKE, FAKE, None) == _lib.NB_EINVAL
    assert ql(FAKE, FAKE, -1, 256, FAKE, FAKE, None) == _lib.NB_EINVAL
    assert ql(None, FAKE, 8, 256, FAKE, FAKE, None) == _lib.NB_EINVAL
    assert ql(FAKE, FAKE, 8, 256, FAKE + 8, FAKE, None) == _lib.NB_EALIGN
    assert _lib.last_error().startswith("nb_quad_layout")
    assert ql(None, None, 0, 256, None, None, None) == _lib.NB_OK


def test_tile_batch_and_layout_validation():
    """nb_gemm_skinny_tile_batched: the skinny checks (M 1..16) under its
    own name; nb_tile_layout: shape, pointers and alignment; the layout's
    byte count (ceil(N / 16) * ceil(K / 512) tiles of 3072 index bytes)."""
    lib = _lib.load()
    Item = _lib.BatchItem
    good = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 256))
    ts = lib.nb_gemm_skinny_tile_batched
    for M in (0, 17):
        assert ts(good, FAKE, 1, M, _lib.NB_F32, None) == _lib.NB_EINVAL
    assert _lib.last_error().startswith("nb_gemm_skinny_tile_batched")
    assert ts(good, None, 1, 8, _lib.NB_F32, None) == _lib.NB_EINVAL
    assert ts((Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 200)), FAKE, 1, 8, _lib.NB_F32,
              None) == _lib.NB_EUNSUPPORTED
    add16 = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 256, 0, _lib.NB_Y_ADD, None, 0.0, 0))
    assert ts(add16, FAKE, 1, 8, _lib.NB_BF16, None) == _lib.NB_EUNSUPPORTED
    empty = (Item * 1)(Item(None, None, None, None, 0, 256))
    assert ts(empty, None, 1, 8, _lib.NB_F32, None) == _lib.NB_OK
    assert lib.nb_tile_layout_bytes(16, 2048) == 4 * 3072
    assert lib.nb_tile_layout_bytes(17, 6912) == 2 * 14 * 3072
    assert lib.nb_tile_layout_bytes(0, 256) == 0 and lib.nb_tile_layout_bytes(4, 200) == 0
    tl = lib.nb_tile_layout
    for N, K in ((8, 200), (8, 0), (-1, 256)):
        assert tl(FAKE, FAKE, N, K, FAKE, FAKE, None) == _lib.NB_EINVAL
    assert _lib.last_error().startswith("nb_tile_layout")
    assert tl(None, FAKE, 8, 256, FAKE, FAKE, None) == _lib.NB_EINVAL
    assert tl(FAKE, FAKE, 8, 256, FAKE, None, None) == _lib.NB_EINVAL
    assert tl(FAKE + 8, FAKE, 8, 256, FAKE, FAKE, None) == _lib.NB_EALIGN
    assert tl(FAKE, FAKE, 8, 256, FAKE, FAKE + 4, None) == _lib.NB_EALIGN
    assert tl(None, None, 0, 256, None, None, None) == _lib.NB_OK


# --- prefill and decode-step entry points: host-side validation -------------

def prefill(**kw):
    a = dict(x=FAKE, ldx=256, packed=FAKE, codebook=FAKE, y=FAKE, y_dtype=_lib.NB_BF16, ldy=64,
             M=32, N=64, K=256, stream=None)
    a.update(kw)
    return _lib.load().nb_gemm_prefill(*a.values())


@pytest.mark.parametrize("kw,status", [
    (dict(K=200), _lib.NB_EUNSUPPORTED),
    (dict(M=-1), _lib.NB_EINVAL),
    (dict(ldx=128), _lib.NB_EINVAL),
    (dict(ldy=10), _lib.NB_EINVAL),
    (dict(y_dtype=7), _lib.NB_EINVAL),
    (dict(x=None), _lib.NB_EINVAL),
    (dict(x=FAKE + 8), _lib.NB_EALIGN),
    (dict(ldx=260), _lib.NB_EALIGN),
    (dict(codebook=FAKE + 4), _lib.NB_EALIGN),
])
def test_prefill_validation(kw, status):
    assert prefill(**kw) == status
    assert _lib.last_error().startswith("nb_gemm_prefill")


def test_prefill_empty_is_ok():
    assert prefill(M=0) == _lib.NB_OK and prefill(N=0) == _lib.NB_OK


def prefill_split(**kw):
    lib = _lib.load()
    a = dict(x=FAKE, ldx=2560, packed=FAKE, codebook=FAKE, y=FAKE, y_dtype=_lib.NB_BF16,
             ldy=2560, M=128, N=2560, K=2560, ws=FAKE,
             ws_bytes=int(lib.nb_gemm_prefill_split_ws_bytes(128, 2560, 2560)), stream=None)
    a.update(kw)
    return lib.nb_gemm_prefill_split(*a.values())


def test_prefill_split_ws_bytes():
    """K ranges (fp32 partial products M x N each) only where the tile grid
    would leave CUs idle: few tokens, narrow layers; at M = 2048 only the
    long-K down projection (three ranges of the 256 x 256 tile on a
    256-CU device: 80 tiles x 3 instead of 160 tiles of 256 x 128)."""
    lib = _lib.load()
    b = lib.nb_gemm_prefill_split_ws_bytes
    for N, K in ((7680, 2560), (2560, 2560), (13824, 2560), (2560, 6912)):
        assert b(1024, N, K) == 0
        assert b(2048, N, K) == (3 * 2048 * N * 4 if K == 6912 else 0)
        s = b(128, N, K)
        assert s > 0 and s % (128 * N * 4) == 0 and 2 <= s // (128 * N * 4) <= 8
        # partial products at most four times the packed weight's bytes
        assert s <= 4 * N * K // 128 * 80
    assert b(512, 7680, 2560) == 0 and b(512, 2560, 6912) > 0
    assert b(0, 64, 256) == 0 and b(32, 64, 200) == 0 and b(-1, 64, 256) == 0
    assert b(128, 8, 128) == 0          # one step of K: nothing to split


@pytest.mark.parametrize("kw,status", [
    (dict(K=200), _lib.NB_EUNSUPPORTED),
    (dict(M=-1), _lib.NB_EINVAL),
    (dict(ldy=100), _lib.NB_EINVAL),
    (dict(y_dtype=7), _lib.NB_EINVAL),
    (dict(ws=None), _lib.NB_EINVAL),
    (dict(ws=FAKE + 16), _lib.NB_EALIGN),
    (dict(ws_bytes=4096), _lib.NB_EINVAL),
    (dict(ws_bytes=-1), _lib.NB_EINVAL),
    (dict(x=FAKE + 8), _lib.NB_EALIGN),
])
def test_prefill_split_validation(kw, status):
    assert prefill_split(**kw) == status
    assert _lib.last_error().startswith("nb_gemm_prefill_split")


def test_prefill_split_empty_is_ok():
    assert prefill_split(M=0) == _lib.NB_OK and prefill_split(N=0) == _lib.NB_OK


@pytest.mark.parametrize("kw,status", [
    (dict(n=0), _lib.NB_EINVAL),
    (dict(h_dtype=5), _lib.NB_EINVAL),
    (dict(emb=FAKE, state=None), _lib.NB_EINVAL),
    (dict(x=None), _lib.NB_EINVAL),
    (dict(eps=-1.0), _lib.NB_EINVAL),
    (dict(w=FAKE + 2), _lib.NB_EALIGN),
])
def test_add_rmsnorm_validation(kw, status):
    a = dict(x=FAKE, y=None, emb=None, state=FAKE, w=FAKE, h=FAKE, h_dtype=_lib.NB_BF16, n=2560,
             eps=1e-6, stream=None)
    a.update(kw)
    assert _lib.load().nb_add_rmsnorm(*a.values()) == status


@pytest.mark.parametrize("kw,status", [
    (dict(head_dim=127), _lib.NB_EUNSUPPORTED),
    (dict(head_dim=512), _lib.NB_EUNSUPPORTED),
    (dict(ctx=2048), _lib.NB_EUNSUPPORTED),
    (dict(n_head=0), _lib.NB_EINVAL),
    (dict(work=None), _lib.NB_EINVAL),
    (dict(out_dtype=9), _lib.NB_EINVAL),
    (dict(k_cache=FAKE + 2), _lib.NB_EALIGN),
])
def test_attention_step_validation(kw, status):
    a = dict(qkv=FAKE, k_cache=FAKE, v_cache=FAKE, cos=FAKE, sin=FAKE, state=FAKE, work=FAKE,
             done=FAKE, out=FAKE, out_dtype=_lib.NB_BF16, n_head=20, head_dim=128, ctx=1024,
             stream=None)
    a.update(kw)
    assert _lib.load().nb_attention_step(*a.values()) == status
    assert _lib.load().nb_attention_work_floats(20) > 20 * 128


@pytest.mark.parametrize("kw,status", [
    (dict(n_head=65), _lib.NB_EUNSUPPORTED),       # beyond the static scratch
    (dict(head_dim=127), _lib.NB_EUNSUPPORTED),
    (dict(ctx=2048), _lib.NB_EUNSUPPORTED),
    (dict(n_head=0), _lib.NB_EINVAL),
    (dict(qkv=None), _lib.NB_EINVAL),
    (dict(out_dtype=9), _lib.NB_EINVAL),
    (dict(v_cache=FAKE + 2), _lib.NB_EALIGN),
])
def test_attention_step_static_validation(kw, status):
    a = dict(qkv=FAKE, k_cache=FAKE, v_cache=FAKE, cos=FAKE, sin=FAKE, state=FAKE, out=FAKE,
             out_dtype=_lib.NB_BF16, n_head=20, head_dim=128, ctx=1024, stream=None)
    a.update(kw)
    assert _lib.load().nb_attention_step_static(*a.values()) == status


def test_attention_static_scratch_size():
    lib = _lib.load()
    # 64 heads of split partials (nb_attention_work_floats) + 64 counters
    assert lib.nb_attention_static_scratch_bytes() == lib.nb_attention_work_floats(64) * 4 + 64 * 4
    if not gpu_available():
        a = dict(qkv=FAKE, k_cache=FAKE, v_cache=FAKE, cos=FAKE, sin=FAKE, state=FAKE, out=FAKE,
                 out_dtype=_lib.NB_BF16, n_head=20, head_dim=128, ctx=1024, stream=None)
        assert lib.nb_attention_step_static(*a.values()) == _lib.NB_ENODEV


@pytest.mark.parametrize("kw,status", [
    (dict(C=100), _lib.NB_EUNSUPPORTED),
    (dict(C=16384), _lib.NB_EUNSUPPORTED),
    (dict(V=0), _lib.NB_EUNSUPPORTED),
    (dict(n_force=3, force=None), _lib.NB_EINVAL),
    (dict(tokens_cap=4, tokens=None), _lib.NB_EINVAL),
    (dict(state=None), _lib.NB_EINVAL),
    (dict(emb=FAKE + 8), _lib.NB_EALIGN),
])
def test_lm_head_validation(kw, status):
    a = dict(h=FAKE, emb=FAKE, logits=None, state=FAKE, tokens=None, tokens_cap=0, force=None,
             n_force=0, V=32000, C=2560, stream=None)
    a.update(kw)
    assert _lib.load().nb_lm_head_argmax(*a.values()) == status


@pytest.mark.parametrize("kw,status", [
    (dict(C=100), _lib.NB_EUNSUPPORTED),
    (dict(V=0), _lib.NB_EUNSUPPORTED),
    (dict(x=None), _lib.NB_EINVAL),
    (dict(norm_w=None), _lib.NB_EINVAL),
    (dict(eps=-1.0), _lib.NB_EINVAL),
    (dict(eps=float("nan")), _lib.NB_EINVAL),
    (dict(n_force=3, force=None), _lib.NB_EINVAL),
    (dict(tokens_cap=4, tokens=None), _lib.NB_EINVAL),
    (dict(state=None), _lib.NB_EINVAL),
    (dict(x=FAKE + 2), _lib.NB_EALIGN),
    (dict(norm_w=FAKE + 2), _lib.NB_EALIGN),
    (dict(emb=FAKE + 8), _lib.NB_EALIGN),
])
def test_rmsnorm_lm_head_validation(kw, status):
    a = dict(x=FAKE, norm_w=FAKE, eps=1e-6, emb=FAKE, logits=None, state=FAKE, tokens=None,
             tokens_cap=0, force=None, n_force=0, V=32000, C=2560, stream=None)
    a.update(kw)
    assert _lib.load().nb_rmsnorm_lm_head_argmax(*a.values()) == status
    assert _lib.last_error().startswith("nb_rmsnorm_lm_head_argmax")


def test_silu_mul_validation():
    lib = _lib.load()
    assert lib.nb_silu_mul(FAKE, FAKE, _lib.NB_BF16, 0, None) == _lib.NB_EINVAL
    assert lib.nb_silu_mul(None, FAKE, _lib.NB_BF16, 8, None) == _lib.NB_EINVAL
    assert lib.nb_silu_mul(FAKE, FAKE, 3, 8, None) == _lib.NB_EINVAL


def decode_model(**kw):
    a = dict(n_layers=26, n_embd=2560, n_head=20, head_dim=128, ffn_hidden=6912, vocab=32000,
             ctx=1024, eps=1e-6, layers=FAKE, ln_f=FAKE, emb_f32=FAKE, emb_bf16=FAKE,
             rope_cos=FAKE, rope_sin=FAKE)
    a.update(kw)
    return _lib.DecodeModel(*a.values())


@pytest.mark.parametrize("kw,status", [
    (dict(n_layers=0), _lib.NB_EINVAL),
    (dict(n_layers=65), _lib.NB_EUNSUPPORTED),
    (dict(n_embd=2500, n_head=20, head_dim=125), _lib.NB_EUNSUPPORTED),
    (dict(n_embd=8192, n_head=64), _lib.NB_EUNSUPPORTED),
    (dict(ffn_hidden=8320), _lib.NB_EUNSUPPORTED),
    (dict(head_dim=64), _lib.NB_EUNSUPPORTED),           # n_head * head_dim != n_embd
    (dict(n_head=10, head_dim=256), _lib.NB_EUNSUPPORTED),
    (dict(ctx=1025), _lib.NB_EUNSUPPORTED),
    (dict(eps=-1.0), _lib.NB_EINVAL),
    (dict(layers=None), _lib.NB_EINVAL),
    (dict(emb_bf16=FAKE + 8), _lib.NB_EALIGN),
])
def test_decode_model_validation(kw, status):
    lib = _lib.load()
    m = decode_model(**kw)
    assert lib.nb_decode_workspace_bytes(ctypes.byref(m)) == 0
    st = lib.nb_decode_persistent(ctypes.byref(m), FAKE, 1 << 30, FAKE, None, None, 0, None, 0,
                                  4, 0, None)
    assert st == status, _lib.last_error()


def test_decode_persistent_validation():
    lib = _lib.load()
    m = decode_model()
    need = lib.nb_decode_workspace_bytes(ctypes.byref(m))
    # control block + residual, q|k|v, attention output, gate|up, attention partials
    assert need >= 4096 + 2560 * 4 + 3 * 2560 * 4 + 2560 * 2 + 2 * 6912 * 4
    assert need % 256 == 0

    def call(**kw):
        a = dict(model=ctypes.byref(m), ws=FAKE, ws_bytes=need, state=FAKE, logits=None,
                 tokens=None, tokens_cap=0, force=None, n_force=0, n_steps=4, spin_limit=0,
                 stream=None)
        a.update(kw)
        return lib.nb_decode_persistent(*a.values())

    assert call(ws_bytes=need - 1) == _lib.NB_EINVAL
    assert call(ws=None) == _lib.NB_EINVAL
    assert call(state=None) == _lib.NB_EINVAL
    assert call(n_steps=-1) == _lib.NB_EINVAL
    assert call(n_force=2) == _lib.NB_EINVAL
    assert call(tokens_cap=3) == _lib.NB_EINVAL
    assert call(ws=FAKE + 128) == _lib.NB_EALIGN
    assert call(model=None) == _lib.NB_EINVAL
    assert call(n_steps=0) == _lib.NB_OK          # nothing to do, nothing launched
    if not gpu_available():
        assert call() == _lib.NB_ENODEV


def test_decode_struct_layout():
    # the ctypes mirrors of struct nb_decode_layer / nb_decode_model
    assert ctypes.sizeof(_lib.DecodeLayer) == 12 * 8
    assert _lib.DecodeModel.layers.offset == 32 and ctypes.sizeof(_lib.DecodeModel) == 32 + 6 * 8


@pytest.mark.parametrize("kw,status", [
    (dict(vocab=0), _lib.NB_EINVAL),          # a lookup needs the table's row count
    (dict(vocab=-5), _lib.NB_EINVAL),
    (dict(tokens=None), _lib.NB_EINVAL),      # emb and tokens go together
    (dict(add=FAKE), _lib.NB_EINVAL),         # a lookup takes no add
    (dict(C=0), _lib.NB_EINVAL),
    (dict(h_dtype=9), _lib.NB_EINVAL),
    (dict(tokens=FAKE + 2), _lib.NB_EALIGN),
])
def test_rmsnorm_rows_validation(kw, status):
    a = dict(x=FAKE, add=None, emb=FAKE, tokens=FAKE, vocab=11, w=FAKE, h=FAKE,
             h_dtype=_lib.NB_F32, T=4, C=256, eps=1e-6, stream=None)
    a.update(kw)
    assert _lib.load().nb_rmsnorm_rows(*a.values()) == status
    assert _lib.last_error().startswith("nb_rmsnorm_rows")


def test_rmsnorm_rows_vocab_ignored_without_lookup():
    assert _lib.load().nb_rmsnorm_rows(FAKE, None, None, None, 0, FAKE, FAKE, _lib.NB_F32, 0,
                                       256, 1e-6, None) == _lib.NB_OK


def test_prefill_f32_ws_bytes():
    lib = _lib.load()
    # bf16 hi and lo parts of x (256-byte rounded), the residual codebook,
    # the split partials of the bf16 kernel
    for M, N, K in ((17, 128, 128), (2048, 2560, 2560), (128, 2560, 6912)):
        xb = -(-M * K * 2 // 256) * 256
        cb = -(-N * (K // 128) * 8 * 4 // 256) * 256
        split = int(lib.nb_gemm_prefill_split_ws_bytes(M, N, K))
        assert lib.nb_gemm_prefill_f32_ws_bytes(M, N, K) == 2 * xb + cb + split
    assert lib.nb_gemm_prefill_f32_ws_bytes(4, 4, 100) == 0


def prefill_f32(**kw):
    lib = _lib.load()
    a = dict(x=FAKE, ldx=256, packed=FAKE, codebook=FAKE, y=FAKE, ldy=64, M=32, N=64, K=256,
             ws=FAKE, ws_bytes=int(lib.nb_gemm_prefill_f32_ws_bytes(32, 64, 256)), stream=None)
    a.update(kw)
    return lib.nb_gemm_prefill_f32(*a.values())


@pytest.mark.parametrize("kw,status", [
    (dict(K=200), _lib.NB_EUNSUPPORTED),
    (dict(M=-1), _lib.NB_EINVAL),
    (dict(ldx=128), _lib.NB_EINVAL),
    (dict(ldy=10), _lib.NB_EINVAL),
    (dict(ws=None), _lib.NB_EINVAL),
    (dict(ws=FAKE + 16), _lib.NB_EALIGN),
    (dict(ws_bytes=1024), _lib.NB_EINVAL),
    (dict(x=FAKE + 2), _lib.NB_EALIGN),
    (dict(codebook=FAKE + 4), _lib.NB_EALIGN),
])
def test_prefill_f32_validation(kw, status):
    assert prefill_f32(**kw) == status
    assert _lib.last_error().startswith("nb_gemm_prefill_f32")


def test_prefill_f32_empty_is_ok():
    assert prefill_f32(M=0) == _lib.NB_OK and prefill_f32(N=0) == _lib.NB_OK
