"""Shared test helpers: GGUF block builders, seeded inputs, tolerance rule."""
from __future__ import annotations

import struct

import numpy as np

F32, F16, Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 0, 1, 2, 6, 8, 10, 11, 12, 13, 14, 15, 30
QUANT_TYPES = [Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K]
NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 6: "Q5_0", 8: "Q8_0", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K",
         14: "Q6_K", 15: "Q8_K", 30: "BF16"}
GEOM = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144),
        Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292), F32: (1, 4)}


def h16(v: int) -> bytes:
    return struct.pack("<H", v)


def q4_0_block(d: int, qs) -> bytes:
    return h16(d) + bytes(qs)


def q5_0_block(d: int, qh: int, qs) -> bytes:
    return h16(d) + struct.pack("<I", qh) + bytes(qs)


def q8_0_block(d: int, q) -> bytes:
    return h16(d) + bytes((v & 0xFF) for v in q)


def row_bytes(t: int, in_dim: int) -> int:
    qk, bs = GEOM[t]
    return in_dim // qk * bs


def random_blocks(t: int, n_blocks: int, rng: np.random.Generator, sigma: float = 0.02) -> np.ndarray:
    """Random payload with |N(0, sigma)| f16 scales in every scale field."""
    qk, bs = GEOM[t]
    raw = rng.integers(0, 256, size=(n_blocks, bs), dtype=np.uint8)

    def f16(v):
        return np.abs(v).astype(np.float16).view(np.uint16)

    if t == Q8_0:
        raw[:, 0:2] = f16(rng.normal(0, sigma, n_blocks) / 127).view(np.uint8).reshape(-1, 2)
        q = rng.integers(-127, 128, size=(n_blocks, 32)).astype(np.int8)
        raw[:, 2:] = q.view(np.uint8)
    elif t in (Q4_0, Q5_0):
        raw[:, 0:2] = f16(rng.normal(0, sigma, n_blocks)).view(np.uint8).reshape(-1, 2)
    elif t in (Q4_K, Q5_K):
        raw[:, 0:4] = f16(rng.normal(0, sigma, (n_blocks, 2))).view(np.uint8).reshape(-1, 4)
    elif t == Q6_K:
        raw[:, 208:210] = f16(rng.normal(0, sigma, n_blocks)).view(np.uint8).reshape(-1, 2)
    elif t == Q2_K:
        raw[:, 80:84] = f16(rng.normal(0, sigma, (n_blocks, 2))).view(np.uint8).reshape(-1, 4)
    elif t == Q3_K:
        raw[:, 108:110] = f16(rng.normal(0, sigma, n_blocks)).view(np.uint8).reshape(-1, 2)
    elif t == Q8_K:
        raw[:, 0:4] = np.abs(rng.normal(0, sigma, n_blocks)).astype(np.float32).view(np.uint8).reshape(-1, 4)
    elif t == F32:
        raw = rng.normal(0, 1, n_blocks).astype(np.float32).view(np.uint8).reshape(-1, 4)
    return raw.reshape(-1)


def random_matrix(t: int, out_dim: int, in_dim: int, rng: np.random.Generator, sigma: float = 0.02) -> np.ndarray:
    qk, _ = GEOM[t]
    if t == F32:
        return rng.normal(0, 1, (out_dim, in_dim)).astype(np.float32).view(np.uint8).reshape(-1)
    return random_blocks(t, out_dim * in_dim // qk, rng, sigma)


def rel_err(y: np.ndarray, ref: np.ndarray, floor_frac: float = 1e-3) -> float:
    """Max per-element relative error |y - ref| / max(|ref|, floor_frac * max|ref|).

    The floor keeps elements that cancel to ~0 (random dot products) from
    turning summation-order noise into huge relative errors."""
    ref = ref.astype(np.float64)
    d = np.abs(y.astype(np.float64) - ref)
    floor = floor_frac * max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(d / np.maximum(np.abs(ref), floor))) if ref.size else 0.0


def assert_close(y, ref, tol: float = 1e-4, floor_frac: float = 1e-3, what: str = ""):
    e = rel_err(np.asarray(y), np.asarray(ref), floor_frac)
    assert e <= tol, f"{what}: max relative error {e:.3e} > {tol:.1e}"
    return e


def scaled_err(y, ref, scale, floor: float = 1e-2) -> float:
    """Max per-element error |y - ref| / max(|ref|, floor * scale).

    ``scale`` is each element's term magnitude (sum_j |w_ij x_j| for a matvec,
    sum_p p_p |v_p| for attention).  Well-conditioned elements get the plain
    relative error; an element that cancels to near zero is measured against
    1% of its terms, which is where any two f32 summation orders (the
    reference's sequential one included) legitimately differ."""
    ref = np.asarray(ref, np.float64)
    d = np.abs(np.asarray(y, np.float64) - ref)
    den = np.maximum(np.abs(ref), floor * np.asarray(scale, np.float64))
    return float(np.max(d / np.maximum(den, 1e-30))) if ref.size else 0.0


def assert_close_scaled(y, ref, scale, tol: float = 1e-4, what: str = ""):
    e = scaled_err(y, ref, scale)
    assert e <= tol, f"{what}: max scaled relative error {e:.3e} > {tol:.1e}"
    return e


# Byte ranges of a GGUF block that form the packed layout's regions, in region
# order (the layout documented in include/ramforge_hip.h).
PACK_REGIONS = {Q8_0: [(2, 34), (0, 2)], Q4_0: [(2, 18), (0, 2)], Q4_K: [(16, 144), (0, 16)],
                Q6_K: [(0, 128), (128, 192), (192, 208), (208, 210)]}


def pack_host(t: int, raw: np.ndarray, rows: int, in_dim: int) -> np.ndarray:
    """Packed layout built on the host from the GGUF bytes: each region (a
    byte range of every block) for all blocks of all rows, one after another."""
    qk, bs = GEOM[t]
    blocks = raw.reshape(rows * in_dim // qk, bs)
    return np.concatenate([blocks[:, a:b].reshape(-1) for a, b in PACK_REGIONS[t]])


def zero_code_patch(t: int, raw: np.ndarray, elems) -> np.ndarray:
    """Sets the codes of block elements `elems` (indices within a block) to
    the format's zero weight in every block of a GGUF payload (block layouts
    of quant.rs as the oracle decodes them)."""
    qk, bs = GEOM[t]
    b = raw.reshape(-1, bs)
    for e in elems:
        if t == Q8_0:
            b[:, 2 + e] = 0
        elif t == Q8_K:
            b[:, 4 + e] = 0
        elif t in (Q4_0, Q5_0):
            base = 2 if t == Q4_0 else 6
            j, hi = e % 16, e >= 16
            col = b[:, base + j]
            nib0 = 8 if t == Q4_0 else 0
            b[:, base + j] = (col & 0x0F) | (nib0 << 4) if hi else (col & 0xF0) | nib0
            if t == Q5_0:  # high bit of element e: bit e of qh (value 16 - 16 = 0)
                qh = b[:, 2:6].copy().view(np.uint32).reshape(-1)
                qh |= np.uint32(1 << e)
                b[:, 2:6] = qh.view(np.uint8).reshape(-1, 4)
        elif t == Q6_K:  # element 128 hf + 32 k + l: low nibble 0, high bits 2 (q = 32)
            hf, k, l = e // 128, (e % 128) // 32, e % 32
            ql = 64 * hf + 32 * (k & 1) + l
            b[:, ql] = (b[:, ql] & 0x0F) if (k >> 1) else (b[:, ql] & 0xF0)
            qh = 128 + 32 * hf + l
            b[:, qh] = (b[:, qh] & ~np.uint8(3 << (2 * k))) | np.uint8(2 << (2 * k))
        elif t == Q3_K:  # element 128 n + 32 j + l: low bits 0, hmask bit set (q = 4 - 4)
            n, j, l = e // 128, (e % 128) // 32, e % 32
            b[:, 32 + 32 * n + l] &= ~np.uint8(3 << (2 * j))
            b[:, l] |= np.uint8(1 << (4 * n + j))
        else:
            raise ValueError(f"no zero code for type {t}")
    return raw
