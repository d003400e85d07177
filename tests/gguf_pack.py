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


def random_rows(rng, qtype, rows, k):
    """Random GGUF rows of type qtype (sane scales) -> raw bytes."""
    if qtype == 1:
        return np.asarray(rng.standard_normal(rows * k), np.float16).view(np.uint8)
    if qtype == 8:
        nb = rows * k // 32
        return pack_q8_0(rng.uniform(0.001, 0.02, nb), rng.integers(-128, 128, (nb, 32)))
    nb = rows * k // 256
    if qtype == 12:
        return pack_q4_k(rng.uniform(0.001, 0.02, nb), rng.uniform(0.0, 0.02, nb),
                         rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8)),
                         rng.integers(0, 16, (nb, 256)))
    return pack_q6_k(rng.uniform(0.001, 0.02, nb), rng.integers(-128, 128, (nb, 16)),
                     rng.integers(-32, 32, (nb, 256)))
