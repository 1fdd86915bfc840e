"""Closed-form probes of the oracle's decoders for the types outside the
reference's quant_ref.h fixtures: Q5_0, Q2_K, Q3_K, Q5_K.

Each probe decodes a block element by element, straight from the block
structs (src/kernels.h:21-79) and the element order of the reference's
scalar loops (src/matmul.cpp:102-121, :200-314; dequantize :504-675):
for element e it names the byte and bits that hold e's code, high bit,
sub-block scale and min. That per-element addressing is written here on
its own, not shared with the oracle's block loops (oracle/lp_oracle.c), so
a swapped sub-block, a wrong hmask/qh bit, a wrong scale nibble or a
mis-placed d/dmin field fails. Scales d, dmin are powers of two and every
code is a small integer, so every expected value is exact in fp32 and the
comparisons are bit-exact.

Three checks per type:
  * random blocks (every field random): or_dequantize == the element-wise
    decode, all 256 (32) elements of several blocks;
  * one-hot activations: the scalar dot of e_i with the row
    (gemm_scalar, the reference's fp32 path) == element i's value;
  * single-field probes: changing one field changes exactly the elements
    the format says it controls, by the closed-form amount.
"""
import numpy as np
import pytest

from oracle.oracle import Q2_K, Q3_K, Q5_0, Q5_K

POW2_F16 = {0.25: 0x3400, 0.5: 0x3800, 1.0: 0x3C00, 2.0: 0x4000}


def _f16(v):
    return np.frombuffer(np.uint16(POW2_F16[v]).tobytes(), np.uint8)


def _get_scale_min(q, j):
    """The 6-bit (scale, min) pair j of a 12-byte K-quant scale array: pairs
    0..3 are the low six bits of bytes j and j+4; pairs 4..7 take their low
    four bits from byte j+4 (scale: low nibble, min: high nibble) and their
    top two bits from the top of bytes j-4 (scale) and j (min)."""
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4)
    mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4)
    return sc, mn


def _q3k_scale(sc12, i):
    """Signed 6-bit scale i (0..15) of Q3_K: low four bits from byte i (low
    nibble, i < 8) or byte i-8 (high nibble); top two bits from byte 8 + i%4,
    bit pair i//4; stored with an offset of 32."""
    low = (sc12[i] & 0xF) if i < 8 else (sc12[i - 8] >> 4)
    high = (sc12[8 + i % 4] >> (2 * (i // 4))) & 3
    return (low | (high << 4)) - 32


def decode_q5_0(b, d):
    qh = int.from_bytes(bytes(b[2:6]), "little")
    qs = b[6:22]
    out = np.zeros(32)
    for e in range(32):
        nib = (qs[e] & 0xF) if e < 16 else (qs[e - 16] >> 4)
        q = nib | (((qh >> e) & 1) << 4)
        out[e] = d * (q - 16)
    return out


def decode_q2_k(b, d, dmin):
    sc, qs = b[0:16], b[16:80]
    out = np.zeros(256)
    for e in range(256):
        half, r = divmod(e, 128)
        j, l = divmod(r, 32)
        code = (qs[32 * half + l] >> (2 * j)) & 3
        i = 8 * half + 2 * j + (l >= 16)
        out[e] = d * (sc[i] & 0xF) * code - dmin * (sc[i] >> 4)
    return out


def decode_q3_k(b, d):
    hm, qs, sc = b[0:32], b[32:96], b[96:108]
    out = np.zeros(256)
    for e in range(256):
        half, r = divmod(e, 128)
        s, l = divmod(r, 32)
        code = (qs[32 * half + l] >> (2 * s)) & 3
        hbit = (hm[l] >> (4 * half + s)) & 1
        i = 8 * half + 2 * s + (l >= 16)
        out[e] = d * _q3k_scale(sc, i) * (code - (0 if hbit else 4))
    return out


def decode_q5_k(b, d, dmin):
    sc, qh, qs = b[4:16], b[16:48], b[48:176]
    out = np.zeros(256)
    for e in range(256):
        c, r = divmod(e, 64)
        l = r % 32
        if r < 32:
            v = (qs[32 * c + l] & 0xF) + 16 * ((qh[l] >> (2 * c)) & 1)
            s, m = _get_scale_min(sc, 2 * c)
        else:
            v = (qs[32 * c + l] >> 4) + 16 * ((qh[l] >> (2 * c + 1)) & 1)
            s, m = _get_scale_min(sc, 2 * c + 1)
        out[e] = d * s * v - dmin * m
    return out


# (bytes per block, elements, byte offsets of d and dmin, decoder)
FMT = {
    Q5_0: (22, 32, 0, None, lambda b, d, dm: decode_q5_0(b, d)),
    Q2_K: (84, 256, 80, 82, decode_q2_k),
    Q3_K: (110, 256, 108, None, lambda b, d, dm: decode_q3_k(b, d)),
    Q5_K: (176, 256, 0, 2, decode_q5_k),
}
NAMES = {Q5_0: "Q5_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q5_K: "Q5_K"}
TYPES = list(FMT)


def _block(t, rng, d, dmin):
    nb, ne, od, om, _ = FMT[t]
    b = rng.integers(0, 256, nb, dtype=np.uint8)
    b[od:od + 2] = _f16(d)
    if om is not None:
        b[om:om + 2] = _f16(dmin)
    return b


def _expected(t, b, d, dmin):
    return FMT[t][4]([int(v) for v in b], d, dmin)


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_random_blocks_dequantize(orc, t):
    rng = np.random.default_rng(900 + t)
    nb, ne = FMT[t][0], FMT[t][1]
    for d, dmin in [(1.0, 1.0), (0.5, 2.0), (2.0, 0.25), (0.25, 0.5)]:
        blocks = [_block(t, rng, d, dmin) for _ in range(6)]
        w = np.concatenate(blocks)
        got = orc.dequantize(t, w, ne * len(blocks))
        want = np.concatenate([_expected(t, b, d, dmin) for b in blocks]).astype(np.float32)
        assert np.array_equal(got, want), (NAMES[t], d, dmin, np.flatnonzero(got != want)[:8])


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_one_hot_scalar_dot(orc, t):
    """The reference's fp32 scalar dot (gemm_scalar) against e_i returns
    element i of the decode, for every i of a random block."""
    rng = np.random.default_rng(950 + t)
    ne = FMT[t][1]
    b = _block(t, rng, 0.5, 2.0)
    want = _expected(t, b, 0.5, 2.0).astype(np.float32)
    X = np.eye(ne, dtype=np.float32)
    y = orc.gemm_scalar(t, X, b, 1, nthreads=1)[:, 0]
    assert np.array_equal(y, want), np.flatnonzero(y != want)[:8]


def _diff(orc, t, b0, b1):
    ne = FMT[t][1]
    return orc.dequantize(t, b1, ne) - orc.dequantize(t, b0, ne)


def test_q5_0_high_bit_probe(orc):
    """Setting bit e of qh raises element e (and only e) by 16*d."""
    t = Q5_0
    b0 = np.zeros(22, np.uint8)
    b0[0:2] = _f16(0.5)
    for e in range(32):
        b1 = b0.copy()
        b1[2 + e // 8] |= 1 << (e % 8)
        delta = _diff(orc, t, b0, b1)
        assert np.array_equal(np.flatnonzero(delta), [e]) and delta[e] == 8.0


def test_q2_k_scale_and_min_probe(orc):
    """With every code 1: scale nibble i scales exactly sub-block i
    (elements 16i .. 16i+15, the reference's order), min nibble i shifts
    exactly sub-block i down by dmin*m."""
    t = Q2_K
    b0 = np.zeros(84, np.uint8)
    b0[16:80] = 0x55                       # every 2-bit code = 1
    b0[80:82], b0[82:84] = _f16(1.0), _f16(2.0)
    for i in range(16):
        b1 = b0.copy()
        b1[i] = 0x03                       # scale 3, min 0
        delta = _diff(orc, t, b0, b1)
        assert np.array_equal(np.flatnonzero(delta), np.arange(16 * i, 16 * i + 16))
        assert np.all(delta[16 * i:16 * i + 16] == 3.0)
        b1[i] = 0x50                       # scale 0, min 5
        delta = _diff(orc, t, b0, b1)
        assert np.all(delta[16 * i:16 * i + 16] == -10.0) and np.count_nonzero(delta) == 16


def test_q3_k_hmask_and_scale_probe(orc):
    """Q3_K: one hmask bit lifts one element by 4*d*scale; each of the 16
    signed 6-bit scales (low nibble, high bit pair) scales exactly its
    16-element sub-block."""
    t = Q3_K
    b0 = np.zeros(110, np.uint8)
    b0[108:110] = _f16(1.0)
    b0[96:104] = 0x11                      # every low nibble 1
    b0[104:108] = 0xAA                     # every high pair 2: scale = 33 - 32 = 1
    base = orc.dequantize(t, b0, 256)
    assert np.all(base == -4.0)            # code 0, no high bit: (0 - 4) * 1
    for e in range(0, 256, 7):
        b1 = b0.copy()
        half, r = divmod(e, 128)
        s, l = divmod(r, 32)
        b1[l] |= 1 << (4 * half + s)       # hmask byte l, bit 4*half + s
        delta = _diff(orc, t, b0, b1)
        assert np.array_equal(np.flatnonzero(delta), [e]) and delta[e] == 4.0
    for i in range(16):
        b1 = b0.copy()
        # scale i -> 40 - 32 = 8: low nibble 8, high pair 2 (unchanged)
        if i < 8:
            b1[96 + i] = (b1[96 + i] & 0xF0) | 0x8
        else:
            b1[96 + i - 8] = (b1[96 + i - 8] & 0x0F) | 0x80
        delta = _diff(orc, t, b0, b1)
        assert np.array_equal(np.flatnonzero(delta), np.arange(16 * i, 16 * i + 16))
        assert np.all(delta[16 * i:16 * i + 16] == -28.0)     # (8 - 1) * -4
        b2 = b0.copy()
        # high pair of scale i from 2 to 3: scale 49 - 32 = 17
        pos, sh = 104 + i % 4, 2 * (i // 4)
        b2[pos] = (b2[pos] & ~np.uint8(3 << sh)) | np.uint8(3 << sh)
        delta = _diff(orc, t, b0, b2)
        assert np.array_equal(np.flatnonzero(delta), np.arange(16 * i, 16 * i + 16))
        assert np.all(delta[16 * i:16 * i + 16] == -64.0)     # (17 - 1) * -4


def test_q5_k_high_bit_and_scale_probe(orc):
    """Q5_K: qh bit 2c (low nibbles) / 2c+1 (high nibbles) of byte l lifts
    element 64c + l / 64c + 32 + l by 16*d*sc; scale pair j scales exactly
    elements 32j .. 32j+31."""
    t = Q5_K
    b0 = np.zeros(176, np.uint8)
    b0[0:2], b0[2:4] = _f16(1.0), _f16(0.5)
    b0[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]    # every scale 1, every min 0
    base = orc.dequantize(t, b0, 256)
    assert np.all(base == 0.0)
    for c in range(4):
        for l in range(0, 32, 5):
            for hi in (0, 1):
                b1 = b0.copy()
                b1[16 + l] |= 1 << (2 * c + hi)
                delta = _diff(orc, t, b0, b1)
                e = 64 * c + 32 * hi + l
                assert np.array_equal(np.flatnonzero(delta), [e]) and delta[e] == 16.0
    b0[48:176] = 0x11                      # every code 1
    for j in range(8):
        b1 = b0.copy()
        if j < 4:
            b1[4 + j] = 7                  # scale 7
            b1[8 + j] = 3                  # min 3
        else:
            b1[8 + j] = 0x37               # scale low 7, min low 3 (top bits 0)
        delta = _diff(orc, t, b0, b1)
        assert np.array_equal(np.flatnonzero(delta), np.arange(32 * j, 32 * j + 32)), j
        assert np.all(delta[32 * j:32 * j + 32] == (7 - 1) - 0.5 * 3)
