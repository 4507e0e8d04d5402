"""CPU emulation of the persistent decode kernel's address arithmetic and
chunk scheduling (csrc/nb_decode_persistent.hip), at the configuration whose
GPU run made an illegal memory access: 26 layers, 20 heads of 128, F = 6912,
vocab 32000, context 1024, a 128-token prompt and 128 steps in one launch, on
256 workgroups.

Every global address the kernel forms from its tables and counters is
checked against the allocation it must stay in, and every LDS offset
against its region:

* the [layer][kind] pointer table in LDS and the chunk loads it drives
  (direct-to-LDS, 16 bytes per lane, clamped to the chunk's last piece);
* the KV-cache reads and appends of every layer at every position;
* the attention split ranges, partial-sum slots and split counters;
* the tied head's rows and the prologue / epilogue vectors;
* the chunk-counter protocol: 32 LDS counters reused modulo 32 over the
  104 GEMV phases of a token, driven by a randomised interleaving of the 11
  streaming waves' grabs, must hand every chunk of every phase to exactly
  one wave, inside its own phase.

The kernel's constants are read from its source, so the emulation follows
the file it checks.  The kernel is switched off at the C ABI; this test is
the record that its address arithmetic, as written, stays in bounds at the
faulting configuration (so the fault's cause is not there)."""
import os
import random
import re

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "..", "nativebit_amd", "csrc", "nb_decode_persistent.hip")


def _constants():
    text = open(SRC).read()
    env = {"kXColBytes": 17 * 16}
    for name, expr in re.findall(r"constexpr int (k\w+) = ([^;]+);", text):
        # integer expressions of the source; C++ "/" on ints is "//" here
        code = expr.split("//")[0].replace("/", "//")
        env[name] = eval(code, {}, dict(env))  # noqa: S307 (own source)
    return env


K = _constants()

# the faulting configuration
L, C, H, D, F, V, CTX = 26, 2560, 20, 128, 6912, 32000, 1024
PROMPT, STEPS, G = 128, 128, 256
KINDS = ("qkv", "o", "gu", "down")


def kind_shape(kind):
    N = {"qkv": 3 * C, "o": C, "gu": 2 * F, "down": C}[kind]
    Kd = F if kind == "down" else C
    return N, Kd


def geo(kind, g):
    N, Kd = kind_shape(kind)
    bpr = Kd >> 7
    R = K["kChunkMax"] // bpr
    nbk = R * bpr
    nch = (N + R - 1) // R
    return dict(N=N, bpr=bpr, R=R, nbk=nbk, c0=nch * g // G, c1=nch * (g + 1) // G, nch=nch)


def test_lds_layout_fits_and_regions_disjoint():
    assert K["kLdsBytes"] <= 160 * 1024
    regions = [("ring", K["kOffRing"], K["kSWaves"] * K["kDepth"] * K["kSlotBytes"]),
               ("x", K["kOffX"], K["kXStage"]), ("tmp", K["kOffTmp"], K["kTmpBytes"]),
               ("y", K["kOffY"], K["kYMax"] * 4), ("cnt", K["kOffCnt"], K["kCntWindow"] * 4),
               ("misc", K["kOffMisc"], 256), ("geo", K["kOffGeo"], 128),
               ("lane", K["kOffLane"], 512), ("ptab", K["kOffPtab"], K["kMaxLayers"] * 64),
               ("args", K["kOffArgs"], 256)]
    for (a, oa, na), (b, ob, nb) in zip(regions, regions[1:]):
        assert oa + na <= ob, (a, b)
    # the misc slots the kernel uses: argmax keys (16 x 8 bytes at +64), abort flag (+192)
    assert 64 + 16 * 8 <= 192 and 192 + 4 <= 256
    # four KGeo records of six ints; 4 x 64 lane-table bytes
    assert 4 * 6 * 4 <= 128 and 4 * 64 <= 512
    # attention scratch of the streaming waves may run from x into tmp only
    assert K["kSWaves"] * K["kAttScratch"] <= K["kXStage"] + K["kTmpBytes"]
    # per-wave row-sum scratch inside tmp
    assert K["kSWaves"] * 256 <= K["kTmpBytes"]
    assert L <= K["kMaxLayers"] and C <= K["kMaxC"] and F <= K["kMaxF"] and D <= K["kMaxD"]
    assert H <= K["kMaxHeads"] and CTX <= K["kMaxSplits"] * K["kSplitLen"]


def test_gemv_chunk_loads_and_epilogue_in_bounds():
    for kind in KINDS:
        g0 = geo(kind, 0)
        N, bpr, R, nbk = g0["N"], g0["bpr"], g0["R"], g0["nbk"]
        stream_bytes, cb_bytes = N * bpr * 48, N * bpr * 32
        assert R >= 1 and nbk <= K["kChunkMax"]
        for g in range(G):
            gg = geo(kind, g)
            assert gg["c1"] > gg["c0"], "every workgroup needs a chunk of every kind"
            nrows = min(N, gg["c1"] * R) - gg["c0"] * R
            assert 0 < nrows <= K["kYMax"]
            for c in range(gg["c0"], gg["c1"]):
                rows = min(R, N - c * R)
                nb = rows * bpr
                b0 = c * nbk
                ilast, clast = nb * 48 - 16, nb * 32 - 16
                for off in (0, 1024, 2048):
                    for lane in (0, 63):
                        a = b0 * 48 + min(16 * lane + off, ilast)
                        assert 0 <= a and a + 16 <= stream_bytes
                for off in (0, 1024):
                    for lane in (0, 63):
                        a = b0 * 32 + min(16 * lane + off, clast)
                        assert 0 <= a and a + 16 <= cb_bytes
                # LDS result slot of the chunk's rows
                for lane in range(rows):
                    assert 0 <= (c - gg["c0"]) * R + lane < K["kYMax"]
                # lanes past the chunk's blocks: column table entry and x stage
                for lane in range(64):
                    col = lane % bpr if lane < R * bpr else 0
                    assert (col + 1) * K["kXColBytes"] <= K["kXStage"]
    # pointer table: slot (layer * 4 + kind) * 2 + 1 of the kMaxLayers * 8 pointers
    assert ((L - 1) * 4 + 3) * 2 + 1 < K["kMaxLayers"] * 8


def test_attention_and_cache_addresses_in_bounds():
    kc_len = vc_len = H * D * CTX          # floats per layer
    awork_len = H * K["kMaxSplits"] * (K["kMaxD"] + 2)
    half, dq = D // 2, D // 4
    for pos in range(0, PROMPT + STEPS):
        n = pos + 1
        S = (n + K["kSplitLen"] - 1) // K["kSplitLen"]
        assert S <= K["kMaxSplits"] and S <= 64
        for h in (0, H - 1):
            kt, vc = h * D * CTX, h * CTX * D
            # append of the new key (transposed) and value
            for lane in (0, half - 1):
                for d in (2 * lane, 2 * lane + 1):
                    assert 0 <= kt + d * CTX + pos < kc_len
                    assert 0 <= vc + pos * D + d < vc_len
            for s in (0, S - 1):
                t0, t1 = s * K["kSplitLen"], min(n, s * K["kSplitLen"] + K["kSplitLen"])
                for lane in (0, 63):
                    qd, p = lane >> 4, lane & 15
                    t = t0 + p
                    if t < t1:
                        for j in (0, dq - 1):
                            assert kt + (qd * dq + j) * CTX + t < kc_len
                for i in range(K["kSplitLen"]):
                    tt = t0 + i
                    if tt < t1:
                        assert vc + tt * D + 2 * (half - 1) + 1 < vc_len
                wk = (h * K["kMaxSplits"] + s) * (K["kMaxD"] + 2)
                assert wk + 3 + 2 * (half - 1) < awork_len
            # combine reads of split j < S and the split counter
            base = h * K["kMaxSplits"] * (K["kMaxD"] + 2)
            assert base + (S - 1) * (K["kMaxD"] + 2) + 3 + 2 * (half - 1) < awork_len
            assert K["kCtlDone"] + h < K["kCtlBytes"] // 4
            # bf16 pair output
            assert ((h * D) >> 1) + half - 1 < C // 2
        # RoPE table row
        assert pos * half + half - 1 < CTX * half


def test_head_and_vectors_in_bounds():
    NW = G * K["kSWaves"]
    for wave in (0, K["kSWaves"] - 1):
        for g in (0, G - 1):
            r = g * K["kSWaves"] + wave
            while r < V:
                for r_ in (r, r + NW):
                    if r_ < V:
                        for i in range(K["kHeadPieces"]):
                            for lane in (0, 63):
                                c = lane * 8 + 512 * i
                                if c < C:
                                    assert r_ * C + c + 8 <= V * C
                r += 2 * NW
    # residual-stream slice written from the embedding row, per workgroup
    for g in (0, G - 1):
        i0, i1 = C * g // G, C * (g + 1) // G
        assert 0 <= i0 <= i1 <= C
    # prologue element loops: kThreads x kPerThread* covers C, F, C / 2 pairs
    assert K["kThreads"] * K["kPerThreadC"] >= C and K["kThreads"] * K["kPerThreadF"] >= F


def test_chunk_counter_protocol_one_workgroup():
    """The counter window at 104 GEMV phases a token: each chunk of each
    phase is grabbed exactly once and computed inside its phase, whatever
    the interleaving of the 11 waves, over two tokens of the 26 layers."""
    rng = random.Random(7)
    W, window, depth = K["kSWaves"], K["kCntWindow"], K["kDepth"]
    for g in (0, 1, 127, G - 1):
        geos = [geo(k, g) for k in KINDS]
        n_tok = 2
        GP = n_tok * 4 * L
        cnt = [geos[i & 3]["c0"] for i in range(window)]
        waves = [dict(cq=0, ck=0, cl=0, cv=GP > 0, slots=[None, None], hs=0) for _ in range(W)]
        computed = {}

        def grab(w, s):
            while w["cv"]:
                i = w["cq"] & (window - 1)
                t = cnt[i]
                cnt[i] += 1
                if t < geos[w["ck"]]["c1"]:
                    w["slots"][s] = (w["cq"], t)
                    return
                w["cq"] += 1
                w["ck"] += 1
                if w["ck"] == 4:
                    w["ck"] = 0
                    w["cl"] = (w["cl"] + 1) % L
                if w["cq"] >= GP:
                    w["cv"] = False
            w["slots"][s] = None

        for w in waves:
            for s in range(depth):
                grab(w, s)
        for gq in range(GP):
            kind = gq & 3
            busy = list(range(W))
            while busy:
                wi = rng.choice(busy)
                w = waves[wi]
                head = w["slots"][w["hs"]]
                if head is None or head[0] != gq:
                    busy.remove(wi)
                    continue
                key = (gq, head[1])
                assert key not in computed, ("chunk computed twice", key)
                computed[key] = wi
                grab(w, w["hs"])
                w["hs"] ^= 1
            # phase end: no wave holds a chunk of this or an earlier phase
            for w in waves:
                for sl in w["slots"]:
                    assert sl is None or sl[0] > gq, ("stale slot", gq, sl)
            cnt[gq & (window - 1)] = geos[kind]["c0"]
            got = sorted(c for (q, c) in computed if q == gq)
            assert got == list(range(geos[kind]["c0"], geos[kind]["c1"])), (g, gq)
        assert len(computed) == sum(n_tok * L * (gg["c1"] - gg["c0"]) for gg in geos)


@pytest.mark.parametrize("kind", KINDS)
def test_workgroup_count_fits_every_kind(kind):
    # the launcher's grid: one workgroup per CU, fewer when a kind has fewer
    # chunks; at the 2.2B shape every kind has at least 256 chunks
    assert geo(kind, 0)["nch"] >= G


# -- the argmax key hand-over and the embedding address it drives ------------
#
# After the head phase every workgroup reads st->key, forms the chosen token
# am = 0xffffffff - low32(key) and, at the next token's layer 0, reads the
# embedding row emb_f32 + tok * C.  A key that holds no maximum (cleared, or
# read before the max) gives am = 0xffffffff, i.e. token -1 as an int: the
# row 10 KB before the table.  The kernel's checked_token maps any token
# outside [0, V) to row 0 and sets bit 1 of the error word, so the address
# stays inside the table and the launch ends at its next grid barrier.

def _key(logit, row):
    """The head's 64-bit key: order-preserving logit bits << 32 | ~row."""
    import struct
    b = struct.unpack("<I", struct.pack("<f", logit))[0]
    ob = (b ^ 0xFFFFFFFF) if b & 0x80000000 else (b | 0x80000000)
    return (ob << 32) | (0xFFFFFFFF - row)


def _am(key):
    v = 0xFFFFFFFF - (key & 0xFFFFFFFF)
    return v - (1 << 32) if v & 0x80000000 else v   # the kernel's (int) cast


def _checked(t, err):
    if 0 <= t < V:
        return t, err
    return 0, err | 2


def test_key_handover_model_and_token_guard():
    src = open(SRC).read()
    # the expressions modelled here are the kernel's
    assert "(int)(0xffffffffu - (uint32_t)(key & 0xffffffffull))" in src
    assert "if ((unsigned)t < (unsigned)args.V) return t;" in src
    assert "tok = checked_token(" in src and "tok = checked_token(tok);" in src
    emb_bytes = V * C * 4
    # a merged key: the first row with the largest logit, in range
    keys = [_key(1.5, 7), _key(3.25, 31999), _key(3.25, 40), _key(-2.0, 0)]
    best = max(keys)
    assert _am(best) == 40
    # a key with no maximum in it: token -1, an address before the table
    assert _am(0) == -1
    assert -1 * C * 4 < 0
    tok, err = _checked(_am(0), 0)
    assert (tok, err) == (0, 2) and 0 <= tok * C * 4 and tok * C * 4 + C * 4 <= emb_bytes
    # every valid token passes unchanged; every other int is caught
    for t in (0, 1, V - 1):
        assert _checked(t, 0) == (t, 0)
    for t in (-1, V, V + 5, -(1 << 31), (1 << 31) - 1):
        tt, e = _checked(t, 0)
        assert tt == 0 and e == 2
