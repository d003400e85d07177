"""Packers for GGUF weight blocks, written from the format definitions
(ggml's block_q8_0, block_q4_K, block_q6_K layouts, quantize direction):
given chosen scales, mins and quants they produce the block bytes, so tests
can check a dequantiser against values known from the format formula."""
import numpy as np


def f16_bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def pack_q8_0(d, q):
    """d: fp16 scale per block [nb]; q: int8 [nb, 32] -> bytes [nb * 34]."""
    nb = q.shape[0]
    out = np.zeros((nb, 34), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def pack_q4_k(d, dmin, sc, mn, q):
    """d, dmin: [nb]; sc, mn: 6-bit [nb, 8]; q: nibbles [nb, 256] -> bytes [nb * 144].
    Scales: j < 4 in the low 6 bits of bytes j (scale) and j + 4 (min); j >= 4
    split into a low nibble (byte j + 4: scale low, min high) and 2 high bits
    (the top bits of bytes j - 4 and j)."""
    nb = q.shape[0]
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = f16_bits(dmin).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    s = np.zeros((nb, 12), np.int64)
    for j in range(4):
        s[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        s[:, j + 4] = (mn[:, j] & 63) | ((mn[:, j + 4] >> 4) << 6)
        s[:, j + 8] = (sc[:, j + 4] & 15) | ((mn[:, j + 4] & 15) << 4)
    out[:, 4:16] = s.astype(np.uint8)
    qs = np.zeros((nb, 128), np.int64)
    for c in range(4):
        qs[:, 32 * c:32 * c + 32] = q[:, 64 * c:64 * c + 32] | (q[:, 64 * c + 32:64 * c + 64] << 4)
    out[:, 16:] = qs.astype(np.uint8)
    return out.reshape(-1)


def q4_k_values(d, dmin, sc, mn, q):
    """The format's values: element 32j + l of a block is d*sc[j]*q - dmin*mn[j]."""
    d = np.asarray(d, np.float16).astype(np.float64)[:, None]
    dmin = np.asarray(dmin, np.float16).astype(np.float64)[:, None]
    j = np.arange(256) // 32
    return d * sc[:, j] * q - dmin * mn[:, j]


def pack_q6_k(d, sc, q):
    """d: [nb]; sc: int8 [nb, 16]; q: [nb, 256] in [-32, 31] -> bytes [nb * 210].
    Half n of 128 elements, l < 32: the four 32-element groups' low nibbles go
    to ql[64n + l] (groups 0 | 2 << 4) and ql[64n + 32 + l] (groups 1 | 3 << 4),
    their high 2 bits to qh[32n + l] (group g at bits 2g)."""
    nb = q.shape[0]
    u = (q + 32).astype(np.int64)
    ql = np.zeros((nb, 128), np.int64)
    qh = np.zeros((nb, 64), np.int64)
    for n in range(2):
        g = [u[:, 128 * n + 32 * t:128 * n + 32 * t + 32] for t in range(4)]
        ql[:, 64 * n:64 * n + 32] = (g[0] & 15) | ((g[2] & 15) << 4)
        ql[:, 64 * n + 32:64 * n + 64] = (g[1] & 15) | ((g[3] & 15) << 4)
        qh[:, 32 * n:32 * n + 32] = (g[0] >> 4) | ((g[1] >> 4) << 2) | ((g[2] >> 4) << 4) | ((g[3] >> 4) << 6)
    out = np.zeros((nb, 210), np.uint8)
    out[:, :128] = ql.astype(np.uint8)
    out[:, 128:192] = qh.astype(np.uint8)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def q6_k_values(d, sc, q):
    """Element 128n + 32t + l of a block is d * sc[8n + 2t + l // 16] * q."""
    d = np.asarray(d, np.float16).astype(np.float64)[:, None]
    e = np.arange(256)
    n, t, l = e // 128, (e % 128) // 32, e % 32
    return d * sc[:, 8 * n + 2 * t + l // 16] * q


def _k4_scales(sc, mn):
    """The 12 scale bytes of Q4_K / Q5_K from 6-bit scales and mins [nb, 8]."""
    s = np.zeros((sc.shape[0], 12), np.int64)
    for j in range(4):
        s[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        s[:, j + 4] = (mn[:, j] & 63) | ((mn[:, j + 4] >> 4) << 6)
        s[:, j + 8] = (sc[:, j + 4] & 15) | ((mn[:, j + 4] & 15) << 4)
    return s.astype(np.uint8)


def _nibbles32(q):
    """16 bytes holding 32 4-bit values: element j < 16 low nibble of byte j,
    element 16 + j high nibble of byte j."""
    return ((q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)).astype(np.uint8)


def _bits32(q):
    """Bit 4 of each of 32 values as a little-endian 32-bit word, 4 bytes."""
    w = ((q >> 4) & 1).astype(np.uint64) << np.arange(32, dtype=np.uint64)
    return w.sum(axis=1).astype(np.uint32).reshape(-1, 1).view(np.uint8)


def pack_q5_0(d, q):
    """d: [nb]; q: [nb, 32] in [0, 31] (value d * (q - 16)) -> bytes [nb * 22]."""
    nb = q.shape[0]
    out = np.zeros((nb, 22), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:6] = _bits32(q)
    out[:, 6:] = _nibbles32(q)
    return out.reshape(-1)


def pack_q5_1(d, m, q):
    """d, m: [nb]; q: [nb, 32] in [0, 31] (value d * q + m) -> bytes [nb * 24]."""
    nb = q.shape[0]
    out = np.zeros((nb, 24), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = f16_bits(m).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 4:8] = _bits32(q)
    out[:, 8:] = _nibbles32(q)
    return out.reshape(-1)


# The IQ4_NL format's fixed table of 16 non-linear levels.
IQ4NL_LEVELS = np.array([-127, -104, -83, -65, -49, -35, -22, -10,
                         1, 13, 25, 38, 53, 69, 89, 113], np.int64)


def pack_iq4nl(d, idx):
    """d: [nb]; idx: [nb, 32] in [0, 15] (value d * level[idx]) -> bytes [nb * 18]."""
    nb = idx.shape[0]
    out = np.zeros((nb, 18), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = _nibbles32(idx)
    return out.reshape(-1)


def pack_q2_k(d, dmin, sc, mn, q):
    """d, dmin: [nb]; sc, mn: 4-bit [nb, 16]; q: [nb, 256] in [0, 3]
    (element e: d*sc[e//16]*q - dmin*mn[e//16]) -> bytes [nb * 84].
    Element 128n + 32j + 16g + l sits in bits 2j of qs byte 32n + 16g + l."""
    nb = q.shape[0]
    out = np.zeros((nb, 84), np.uint8)
    out[:, :16] = ((sc & 15) | ((mn & 15) << 4)).astype(np.uint8)
    qs = np.zeros((nb, 64), np.int64)
    for n in range(2):
        for j in range(4):
            qs[:, 32 * n:32 * n + 32] |= q[:, 128 * n + 32 * j:128 * n + 32 * j + 32] << (2 * j)
    out[:, 16:80] = qs.astype(np.uint8)
    out[:, 80:82] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 82:84] = f16_bits(dmin).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def pack_q3_k(d, sc, q):
    """d: [nb]; sc: 6-bit [nb, 16]; q: [nb, 256] in [-4, 3]
    (element e: d * (sc[e//16] - 32) * q) -> bytes [nb * 110].  q is stored
    as q mod 4 in qs (as Q2_K) plus a hmask bit 4n + j that is set when q >= 0;
    scale i keeps 4 low bits in byte i (i < 8) or the high nibble of byte
    i - 8, and 2 high bits at bit 2(i // 4) of byte 8 + i % 4."""
    nb = q.shape[0]
    out = np.zeros((nb, 110), np.uint8)
    hm = np.zeros((nb, 32), np.int64)
    qs = np.zeros((nb, 64), np.int64)
    for n in range(2):
        for j in range(4):
            blk = q[:, 128 * n + 32 * j:128 * n + 32 * j + 32]
            qs[:, 32 * n:32 * n + 32] |= (blk & 3) << (2 * j)
            hm |= (blk >= 0).astype(np.int64) << (4 * n + j)
    out[:, :32] = hm.astype(np.uint8)
    out[:, 32:96] = qs.astype(np.uint8)
    s = np.zeros((nb, 12), np.int64)
    for i in range(16):
        lo, hi = sc[:, i] & 15, (sc[:, i] >> 4) & 3
        if i < 8:
            s[:, i] |= lo
        else:
            s[:, i - 8] |= lo << 4
        s[:, 8 + i % 4] |= hi << (2 * (i // 4))
    out[:, 96:108] = s.astype(np.uint8)
    out[:, 108:110] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def pack_q5_k(d, dmin, sc, mn, q):
    """d, dmin: [nb]; sc, mn: 6-bit [nb, 8]; q: [nb, 256] in [0, 31]
    (element e: d*sc[e//32]*q - dmin*mn[e//32]) -> bytes [nb * 176]:
    Q4_K's header and nibble layout plus qh[32], bit s of qh[l] = bit 4 of
    element 32s + l."""
    nb = q.shape[0]
    out = np.zeros((nb, 176), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = f16_bits(dmin).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 4:16] = _k4_scales(sc, mn)
    qh = np.zeros((nb, 32), np.int64)
    for s_ in range(8):
        qh |= ((q[:, 32 * s_:32 * s_ + 32] >> 4) & 1) << s_
    out[:, 16:48] = qh.astype(np.uint8)
    qs = np.zeros((nb, 128), np.int64)
    for c in range(4):
        qs[:, 32 * c:32 * c + 32] = (q[:, 64 * c:64 * c + 32] & 15) | ((q[:, 64 * c + 32:64 * c + 64] & 15) << 4)
    out[:, 48:] = qs.astype(np.uint8)
    return out.reshape(-1)


def scaled_values(d, scale, q, group, dmin=None, mins=None):
    """Element e of a block: d * scale[e // group] * q[e] (- dmin * mins[e // group])."""
    d = np.asarray(d, np.float16).astype(np.float64)[:, None]
    g = np.arange(q.shape[1]) // group
    v = d * scale[:, g] * q
    if dmin is not None:
        v = v - np.asarray(dmin, np.float16).astype(np.float64)[:, None] * mins[:, g]
    return v


def random_rows(rng, qtype, rows, k):
    """Random GGUF rows of type qtype (sane scales) -> raw bytes."""
    if qtype == 1:
        return np.asarray(rng.standard_normal(rows * k), np.float16).view(np.uint8)
    if qtype == 8:
        nb = rows * k // 32
        return pack_q8_0(rng.uniform(0.001, 0.02, nb), rng.integers(-128, 128, (nb, 32)))
    nb = rows * k // 256
    if qtype in (6, 7, 20):
        nb = rows * k // 32
        d = rng.uniform(0.001, 0.02, nb)
        if qtype == 6:
            return pack_q5_0(d, rng.integers(0, 32, (nb, 32)))
        if qtype == 7:
            return pack_q5_1(d, rng.uniform(-0.05, 0.05, nb), rng.integers(0, 32, (nb, 32)))
        return pack_iq4nl(d, rng.integers(0, 16, (nb, 32)))
    if qtype == 10:
        return pack_q2_k(rng.uniform(0.001, 0.02, nb), rng.uniform(0.0, 0.02, nb),
                         rng.integers(0, 16, (nb, 16)), rng.integers(0, 16, (nb, 16)),
                         rng.integers(0, 4, (nb, 256)))
    if qtype == 11:
        return pack_q3_k(rng.uniform(0.001, 0.02, nb), rng.integers(0, 64, (nb, 16)),
                         rng.integers(-4, 4, (nb, 256)))
    if qtype == 13:
        return pack_q5_k(rng.uniform(0.001, 0.02, nb), rng.uniform(0.0, 0.02, nb),
                         rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8)),
                         rng.integers(0, 32, (nb, 256)))
    if qtype == 12:
        return pack_q4_k(rng.uniform(0.001, 0.02, nb), rng.uniform(0.0, 0.02, nb),
                         rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8)),
                         rng.integers(0, 16, (nb, 256)))
    return pack_q6_k(rng.uniform(0.001, 0.02, nb), rng.integers(-128, 128, (nb, 16)),
                     rng.integers(-32, 32, (nb, 256)))
