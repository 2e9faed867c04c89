"""Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011) and the
Box-Muller transform, in Python integers and float64: the checker for psgdk_fill_normal."""
import math

M0, M1 = 0xD2511F53, 0xCD9E8D57  # round multipliers
W0, W1 = 0x9E3779B9, 0xBB67AE85  # key increments between rounds
MASK = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """Four 32-bit words of the block at counter ctr (4 words) under key (2 words)."""
    c = list(ctr)
    k0, k1 = key
    for _ in range(10):
        p0, p1 = M0 * c[0], M1 * c[2]
        c = [((p1 >> 32) ^ c[1] ^ k0) & MASK, p1 & MASK, ((p0 >> 32) ^ c[3] ^ k1) & MASK, p0 & MASK]
        k0, k1 = (k0 + W0) & MASK, (k1 + W1) & MASK
    return c


def normals(n, seed, stream_id):
    """Elements 0 .. n - 1 of psgdk_fill_normal(seed, stream_id): block b (elements 4 b .. 4 b + 3) from the counter
    (b low, b high, stream low, stream high) under key (seed low, seed high); u = (floor(x / 256) + 1/2) 2^-24;
    pairs (u0, u1) give sqrt(-2 ln u0) (cos 2 pi u1, sin 2 pi u1)."""
    out = []
    key = (seed & MASK, (seed >> 32) & MASK)
    for b in range((n + 3) // 4):
        w = philox4x32_10((b & MASK, b >> 32, stream_id & MASK, (stream_id >> 32) & MASK), key)
        for h in range(2):
            u0, u1 = ((w[2 * h] >> 8) + 0.5) * 2.0 ** -24, ((w[2 * h + 1] >> 8) + 0.5) * 2.0 ** -24
            r = math.sqrt(-2.0 * math.log(u0))
            out += [r * math.cos(2 * math.pi * u1), r * math.sin(2 * math.pi * u1)]
    return out[:n]
