"""The selector-ordered unit layout (nb_stream_layout) on the CPU: its
definition from the unpacked indices, the 17-op selector extraction the
batched kernels use on it, and the new entry points' host-side checks.

A 12-byte unit holds 32 3-bit indices.  The batched kernels feed one
v_perm_b32 lookup with a "selector": four indices, one per byte, namely
indices o(s) + 8k (k = 0..3) for selector s, o = (0, 1, 3, 4, 6, 7, 2, 5)
(nb_stream_common.h, unit_selectors).  The layout stores the same 96 bits
so that selectors 0-5 are one shift and one mask of a dword and selectors
6-7 combine two leftover fields.  These tests pin the layout by building it
from the indices and checking that the extraction returns, for every
selector, exactly the four indices it must (a swapped dword, shift or mask
fails them)."""
import numpy as np
import pytest

from nativebit_amd import _lib
from oracle import oracle as O
from tests.test_abi import FAKE

SEL_OFFSET = (0, 1, 3, 4, 6, 7, 2, 5)
M = 0x07070707


def sel_layout_np(idx: np.ndarray) -> np.ndarray:
    """The selector-ordered stream (uint8) of indices idx (length a multiple
    of 32), built field by field."""
    u = np.asarray(idx, np.uint32).reshape(-1, 32)
    sel = lambda s, k: u[:, SEL_OFFSET[s] + 8 * k]
    words = np.zeros((u.shape[0], 3), np.uint32)
    for k in range(4):
        b0 = sel(0, k) | (sel(1, k) << 3) | ((sel(6, k) & 3) << 6)
        b1 = sel(2, k) | (sel(3, k) << 3) | ((sel(7, k) & 3) << 6)
        b2 = sel(4, k) | (sel(5, k) << 3) | ((sel(6, k) >> 2) << 6) | ((sel(7, k) >> 2) << 7)
        words[:, 0] |= b0 << (8 * k)
        words[:, 1] |= b1 << (8 * k)
        words[:, 2] |= b2 << (8 * k)
    return words.astype("<u4").view(np.uint8).reshape(-1)


def extract_sel(stream: np.ndarray) -> np.ndarray:
    """The kernels' 17-op extraction (unit_selectors_sel) of every unit:
    (units, 8) selector dwords."""
    d = np.asarray(stream, np.uint8).reshape(-1, 12).view("<u4").astype(np.uint32)
    d0, d1, d2 = d[:, 0], d[:, 1], d[:, 2]
    return np.stack([d0 & M, (d0 >> 3) & M, d1 & M, (d1 >> 3) & M, d2 & M, (d2 >> 3) & M,
                     ((d0 >> 6) & 0x03030303) | ((d2 >> 4) & 0x04040404),
                     ((d1 >> 6) & 0x03030303) | ((d2 >> 5) & 0x04040404)], axis=1)


def expected_sel(idx: np.ndarray) -> np.ndarray:
    """Selector s of each unit as the reference-layout extraction yields it:
    byte k = index o(s) + 8k."""
    u = np.asarray(idx, np.uint32).reshape(-1, 32)
    out = np.zeros((u.shape[0], 8), np.uint32)
    for s in range(8):
        for k in range(4):
            out[:, s] |= u[:, SEL_OFFSET[s] + 8 * k] << (8 * k)
    return out


def test_extraction_recovers_every_selector():
    rng = np.random.default_rng(5)
    idx = rng.integers(0, 8, 32 * 4000, dtype=np.uint8)
    st = sel_layout_np(idx)
    assert st.size == idx.size * 3 // 8  # the same bytes
    assert np.array_equal(extract_sel(st), expected_sel(idx))


@pytest.mark.parametrize("pos", range(32))
@pytest.mark.parametrize("v", [1, 2, 4, 7])
def test_single_index_lands_in_its_selector_byte(pos, v):
    """One nonzero index: exactly one selector byte is nonzero, the one the
    index belongs to, and it holds the index's value."""
    idx = np.zeros(32, np.uint8)
    idx[pos] = v
    got = extract_sel(sel_layout_np(idx))[0]
    s = SEL_OFFSET.index(pos % 8)
    k = pos // 8
    want = np.zeros(8, np.uint32)
    want[s] = v << (8 * k)
    assert np.array_equal(got, want)


def test_layout_is_a_bit_permutation_of_the_stream():
    """Every bit of the reference stream appears exactly once: the layout of
    a one-bit stream has exactly one bit set, and distinct bits go to
    distinct places."""
    seen = set()
    for bit in range(96):
        ref = np.zeros(12, np.uint8)
        ref[bit // 8] = 1 << (bit % 8)
        idx = O.unpack(ref, 32, 3)
        st = sel_layout_np(idx)
        ones = np.flatnonzero(np.unpackbits(st, bitorder="little"))
        assert ones.size == 1
        seen.add(int(ones[0]))
    assert len(seen) == 96


def test_stream_layout_and_batched_sel_validation():
    lib = _lib.load()
    sl = lib.nb_stream_layout
    for N, K in ((8, 200), (8, 0), (-1, 256)):
        assert sl(FAKE, FAKE, N, K, None) == _lib.NB_EINVAL
    assert _lib.last_error().startswith("nb_stream_layout")
    assert sl(None, FAKE, 8, 256, None) == _lib.NB_EINVAL
    assert sl(FAKE, None, 8, 256, None) == _lib.NB_EINVAL
    assert sl(FAKE + 2, FAKE, 8, 256, None) == _lib.NB_EALIGN
    assert sl(FAKE, FAKE + 2, 8, 256, None) == _lib.NB_EALIGN
    assert sl(None, None, 0, 256, None) == _lib.NB_OK
    Item = _lib.BatchItem
    bs = lib.nb_gemv_batched_sel
    good = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 256))
    assert bs(good, None, 1, _lib.NB_F32, None) == _lib.NB_EINVAL
    assert _lib.last_error().startswith("nb_gemv_batched_sel")
    assert bs(good, FAKE, 1, 7, None) == _lib.NB_EINVAL
    bad_k = (Item * 1)(Item(FAKE, FAKE, FAKE, FAKE, 32, 200))
    assert bs(bad_k, FAKE, 1, _lib.NB_F32, None) == lib.nb_gemv_batched(bad_k, FAKE, 1,
                                                                        _lib.NB_F32, None)
    empty = (Item * 1)(Item(None, None, None, None, 0, 256))
    assert bs(empty, None, 1, _lib.NB_F32, None) == _lib.NB_OK
