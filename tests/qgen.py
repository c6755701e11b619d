"""Independent GGUF block *encoders* and seeded synthetic data for the tests.

The encoders are written from the storage formats (ggml ``block_q4_0`` / ``block_q5_0`` /
``block_q8_0`` / ``block_q4_K`` / ``block_q6_K``), in the encoding direction, in numpy.  They share
no code with the oracle's decoders, so "encode known integers, decode with the oracle, compare with
the closed form" pins the decoders: a swapped nibble, a wrong scale index or a wrong bit of qh
fails.  Random data uses numpy's PCG64 generator with explicit seeds.
"""
from __future__ import annotations

import numpy as np

Q4_0, Q5_0, Q8_0, Q8_1, Q4_K, Q6_K = 2, 6, 8, 9, 12, 14
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q8_1: (32, 36), Q4_K: (256, 144), Q6_K: (256, 210)}


def f16_bits(v) -> np.ndarray:
    """Binary16 bit patterns of float values (numpy rounds to nearest, ties to even)."""
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_val(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---- encoders: logical values -> bytes ----------------------------------------------------
# Each takes arrays over nb blocks and returns a uint8 array of nb * block_bytes.

def pack_q8_0(d_bits: np.ndarray, q: np.ndarray) -> np.ndarray:
    """d_bits [nb] f16 bits, q [nb, 32] int8 values."""
    nb = q.shape[0]
    out = np.zeros((nb, 34), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nb, 1).view(np.uint8)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def pack_q4_0(d_bits: np.ndarray, q: np.ndarray) -> np.ndarray:
    """q [nb, 32] in 0..15; value = d*(q-8).  Byte i holds element i (low) and i+16 (high)."""
    nb = q.shape[0]
    q = q.astype(np.uint8)
    out = np.zeros((nb, 18), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nb, 1).view(np.uint8)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(-1)


def pack_q5_0(d_bits: np.ndarray, q: np.ndarray) -> np.ndarray:
    """q [nb, 32] in 0..31; value = d*(q-16).  Bit e of the 32-bit qh is bit 4 of element e."""
    nb = q.shape[0]
    q = q.astype(np.uint32)
    out = np.zeros((nb, 22), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nb, 1).view(np.uint8)
    qh = np.zeros(nb, np.uint32)
    for e in range(32):
        qh |= ((q[:, e] >> 4) & 1) << e
    out[:, 2:6] = qh.astype("<u4").reshape(nb, 1).view(np.uint8)
    lo = (q & 15).astype(np.uint8)
    out[:, 6:] = lo[:, :16] | (lo[:, 16:] << 4)
    return out.reshape(-1)


def pack_q4_k(d_bits, dmin_bits, sc, mn, q) -> np.ndarray:
    """sc, mn [nb, 8] in 0..63; q [nb, 256] in 0..15; value = d*sc[j]*q - dmin*mn[j], j = e//32.

    The 12 scale bytes: bytes 0-3 hold sc[0..3] (low 6 bits) and the top 2 bits of sc[4..7];
    bytes 4-7 hold mn[0..3] and the top 2 bits of mn[4..7]; bytes 8-11 hold the low nibbles of
    sc[4..7] (low half) and mn[4..7] (high half).  The 128 qs bytes hold sub-block pairs
    (2p, 2p+1) as the low / high nibbles of bytes 32p .. 32p+31.
    """
    nb = q.shape[0]
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    q = q.astype(np.uint8)
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nb, 1).view(np.uint8)
    out[:, 2:4] = dmin_bits.astype("<u2").reshape(nb, 1).view(np.uint8)
    s = np.zeros((nb, 12), np.uint8)
    for j in range(4):
        s[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        s[:, j + 4] = (mn[:, j] & 63) | ((mn[:, j + 4] >> 4) << 6)
        s[:, j + 8] = (sc[:, j + 4] & 15) | ((mn[:, j + 4] & 15) << 4)
    out[:, 4:16] = s
    for p in range(4):
        out[:, 16 + 32 * p:16 + 32 * p + 32] = q[:, 64 * p:64 * p + 32] | (q[:, 64 * p + 32:64 * p + 64] << 4)
    return out.reshape(-1)


def pack_q6_k(d_bits, sc, q) -> np.ndarray:
    """sc [nb, 16] int8 (sc[i] scales elements 16i..16i+15); q [nb, 256] in -32..31;
    value = d*sc[e//16]*q[e].

    Each 128-element half h stores its 6-bit values u = q + 32 as: ql[64h + l] = u[l] | u[l+64]<<4,
    ql[64h + 32 + l] = u[l+32] | u[l+96]<<4 (low nibbles), and
    qh[32h + l] = u[l]>>4 | (u[l+32]>>4)<<2 | (u[l+64]>>4)<<4 | (u[l+96]>>4)<<6,
    with l in 0..31 and u indexed within the half.
    """
    nb = q.shape[0]
    u = (q.astype(np.int16) + 32).astype(np.uint8)
    out = np.zeros((nb, 210), np.uint8)
    for h in range(2):
        uh = u[:, 128 * h:128 * h + 128]
        l = np.arange(32)
        out[:, 64 * h + l] = (uh[:, l] & 15) | ((uh[:, l + 64] & 15) << 4)
        out[:, 64 * h + 32 + l] = (uh[:, l + 32] & 15) | ((uh[:, l + 96] & 15) << 4)
        out[:, 128 + 32 * h + l] = ((uh[:, l] >> 4) | ((uh[:, l + 32] >> 4) << 2)
                                    | ((uh[:, l + 64] >> 4) << 4) | ((uh[:, l + 96] >> 4) << 6))
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d_bits.astype("<u2").reshape(nb, 1).view(np.uint8)
    return out.reshape(-1)


# ---- closed-form values of the logical contents (float32, operations in written order) ------

def value_q8_0(d_bits, q):
    return f16_val(d_bits)[:, None] * q.astype(np.float32)


def value_q4_0(d_bits, q):
    return f16_val(d_bits)[:, None] * (q.astype(np.float32) - np.float32(8))


def value_q5_0(d_bits, q):
    return f16_val(d_bits)[:, None] * (q.astype(np.float32) - np.float32(16))


def value_q4_k(d_bits, dmin_bits, sc, mn, q):
    d = f16_val(d_bits)[:, None]
    dmin = f16_val(dmin_bits)[:, None]
    scr = np.repeat(sc.astype(np.float32), 32, axis=1)
    mnr = np.repeat(mn.astype(np.float32), 32, axis=1)
    return (d * scr) * q.astype(np.float32) - dmin * mnr


def value_q6_k(d_bits, sc, q):
    d = f16_val(d_bits)[:, None]
    scr = np.repeat(sc.astype(np.float32), 16, axis=1)
    return (d * scr) * q.astype(np.float32)


# ---- random logical blocks + their bytes ----------------------------------------------------

def random_blocks(qtype: int, nb: int, rng: np.random.Generator, scale: float = 0.01):
    """Returns (packed bytes, float32 values [nb*block_elems]) for nb random blocks."""
    d = f16_bits(np.abs(rng.standard_normal(nb)) * scale)
    if qtype == Q8_0:
        q = rng.integers(-127, 128, size=(nb, 32))
        return pack_q8_0(d, q), value_q8_0(d, q).reshape(-1)
    if qtype == Q4_0:
        q = rng.integers(0, 16, size=(nb, 32))
        return pack_q4_0(d, q), value_q4_0(d, q).reshape(-1)
    if qtype == Q5_0:
        q = rng.integers(0, 32, size=(nb, 32))
        return pack_q5_0(d, q), value_q5_0(d, q).reshape(-1)
    if qtype == Q4_K:
        dmin = f16_bits(np.abs(rng.standard_normal(nb)) * scale)
        sc = rng.integers(0, 64, size=(nb, 8))
        mn = rng.integers(0, 64, size=(nb, 8))
        q = rng.integers(0, 16, size=(nb, 256))
        return pack_q4_k(d, dmin, sc, mn, q), value_q4_k(d, dmin, sc, mn, q).reshape(-1)
    if qtype == Q6_K:
        sc = rng.integers(-128, 128, size=(nb, 16))
        q = rng.integers(-32, 32, size=(nb, 256))
        return pack_q6_k(d, sc, q), value_q6_k(d, sc, q).reshape(-1)
    raise ValueError(qtype)


def random_matrix(qtype: int, out_dim: int, in_dim: int, seed: int, scale: float = 0.01):
    """Row-major [out_dim, in_dim] quantized matrix: (bytes, row_bytes, float32 values)."""
    be, bb = BLOCK[qtype]
    assert in_dim % be == 0
    rng = np.random.default_rng(seed)
    nb = out_dim * in_dim // be
    w, vals = random_blocks(qtype, nb, rng, scale)
    return w, in_dim // be * bb, vals.reshape(out_dim, in_dim)


def random_x(m: int, in_dim: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((m, in_dim)).astype(np.float32)


def normwise_rel_err(y, ref) -> float:
    """max_i |y_i - ref_i| / max_j |ref_j|: the parity metric (1e-3 gate)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))
