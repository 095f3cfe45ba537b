"""IQ4_XS oracle: llama.cpp IQ4_XS blocks, the reference's planar tables and their dequant (test infrastructure only).

Block (136 bytes per 256 weights, iqquant.py:5-6,15): d f16 [0:2] | sh u16 [2:4] (two high scale bits per 32-weight
sub-block) | sl [4:8] (eight low 4-bit scale parts, low nibble first) | qs [8:136] (4-bit indices into the 16-entry
non-linear table kvalues_iq4nl; sub-block i = bytes 16i .. 16i+15: weight j < 16 in the low nibble of byte j,
weight 16 + j in the high nibble).
Weight = f16(d) * ((sl_i | sh_i << 4) - 32) * kvalues[nibble]        (iqquant.py:137-148)
Every factor is exact in f32 (<= 11 + 6 + 7 significant bits), so any evaluation order gives the same bits.

Planar tables (planes.py:26-28,136-170; one expert matrix = R rows, nblk blocks per row, W = 32 nblk words):
  qs u32 [W, R]       word w = qs bytes 4w .. 4w+3 of the row                     (GGUF bytes 8..135)
  sl u32 [nblk, R]    u32 b: nibble i = low scale bits of sub-block i            (GGUF 4..7)
  sh u32 [nblk, R]    u32 b: bits 2i, 2i+1 = high scale bits of sub-block i      (GGUF 2..3, zero-extended)
  d  u32 [ceil(nblk/2), R]  u32 b//2, half b%2 = f16 bits of block b           (GGUF 0..1)
Word w, byte j: low nibble = input 32 (w // 4) + 4 (w % 4) + j, high nibble = that + 16 (planes.py:78-82).
"""
import os

import numpy as np

from .bf16 import f16_bits_to_f32

QK = 256
BLOCK_BYTES = 136
PLANE_KEYS = ("qs", "sl", "sh", "d")                  # planes.py:46
_KV = None


def kvalues():
    """int8 [16] the non-linear IQ4 table, as vendored by the reference (iqquant.py:20)."""
    global _KV
    if _KV is None:
        _KV = np.load(os.path.join(os.path.dirname(__file__), "data", "iq4nl_kvalues.npy"))
        assert _KV.shape == (16,) and _KV.dtype == np.int8
    return _KV


def plane_rows(nblk):
    """Rows per expert of every plane (planes.py:64-65)."""
    return {"qs": 32 * nblk, "sl": nblk, "sh": nblk, "d": (nblk + 1) // 2}


# ------------------------------------------------------------------------------------------------ block form
def dequant_blocks(blk):
    """uint8 [..., nblk, 136] -> f32 [..., nblk, 256]: restates iqquant.dequant_iq4_xs (iqquant.py:137-148)."""
    blk = np.asarray(blk, dtype=np.uint8)
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))       # [...]
    sh = blk[..., 2].astype(np.int32) | (blk[..., 3].astype(np.int32) << 8)                       # 16 bits
    sl = blk[..., 4:8]
    lo = np.stack([sl & 15, sl >> 4], axis=-1).reshape(blk.shape[:-1] + (8,)).astype(np.int32)  # sub-block i
    hi = np.stack([(sh >> (2 * i)) & 3 for i in range(8)], axis=-1)
    scale = ((lo | (hi << 4)) - 32).astype(np.float32)                                          # [..., 8]
    qs = blk[..., 8:136].reshape(blk.shape[:-1] + (8, 16))
    nib = np.concatenate([qs & 15, qs >> 4], axis=-1).astype(np.int64)                          # [..., 8, 32]
    v = kvalues().astype(np.float32)[nib]
    w = d[..., None, None] * scale[..., None] * v
    return w.reshape(blk.shape[:-1] + (QK,)).astype(np.float32)


def random_blocks(rng, E, R, nblk, scale=0.02):
    """Uniform random block bytes with a finite f16 d in [scale/2, scale] (every other byte pattern is valid)."""
    t = rng.integers(0, 256, (E, R, nblk, BLOCK_BYTES), dtype=np.uint8)
    d = rng.uniform(0.5 * scale, scale, (E, R, nblk)).astype(np.float16)
    t[..., 0:2] = np.frombuffer(d.tobytes(), np.uint8).reshape(E, R, nblk, 2)
    return t


# ------------------------------------------------------------------------------------------------ planar form
def _u32(a):
    E, R = a.shape[:2]
    return np.ascontiguousarray(a.reshape(E, R, -1)).view("<u4")


def _merge(a):
    E, R, P = a.shape
    return np.ascontiguousarray(a.transpose(0, 2, 1)).reshape(E * P, R)


def pack_planes(t):
    """uint8 [E, R, nblk, 136] -> {plane: u32 [E*rows_p, R]} (planes.py:136-170, IQ4_XS branch)."""
    E, R, nblk, bb = t.shape
    assert bb == BLOCK_BYTES
    d = t[..., 0:2].reshape(E, R, nblk * 2)
    if nblk % 2:
        d = np.concatenate([d, np.zeros((E, R, 2), np.uint8)], -1)
    sh = np.concatenate([t[..., 2:4], np.zeros((E, R, nblk, 2), np.uint8)], -1)
    out = {"d": np.ascontiguousarray(d).view("<u4"), "sh": _u32(sh), "sl": _u32(t[..., 4:8]),
           "qs": _u32(t[..., 8:136])}
    rows = plane_rows(nblk)
    res = {k: _merge(out[k]) for k in PLANE_KEYS}
    for k, a in res.items():
        assert a.shape == (E * rows[k], R), (k, a.shape)
    return res


def dequant_planes_natural(planes, nblk):
    """{plane: u32 [E*rows_p, R]} -> f32 [E, R, 256*nblk] in natural input order, read straight from the planar bit
    map (the module docstring).  An independent restatement of planes._deq_iq4_xs + dequant_natural
    (planes.py:230-243,294-300): block form and planar form agreeing bit for bit pins the packer."""
    rows = plane_rows(nblk)
    R = planes["qs"].shape[-1]
    E = planes["qs"].shape[0] // rows["qs"]
    p = {k: np.asarray(planes[k], dtype=np.uint32).reshape(E, rows[k], R) for k in PLANE_KEYS}
    W = 32 * nblk
    w = np.arange(W)
    sub = w // 4                                                        # sub-block of the word (8 per block)
    b, i = sub // 8, sub % 8
    lo = (p["sl"][:, b, :] >> (4 * i)[None, :, None]) & 15
    hi = (p["sh"][:, b, :] >> (2 * i)[None, :, None]) & 3
    dbits = (p["d"][:, b // 2, :] >> ((b % 2) * 16)[None, :, None]) & 0xFFFF
    scale = f16_bits_to_f32(dbits) * ((lo | (hi << 4)).astype(np.int32) - 32).astype(np.float32)   # [E, W, R]
    kv = kvalues().astype(np.float32)
    out = np.zeros((E, nblk * QK, R), np.float32)
    qs = p["qs"]
    base = 32 * sub + 4 * (w % 4)                                       # input of byte 0's low nibble
    for j in range(4):
        for pos in range(2):
            nib = (qs >> (8 * j + 4 * pos)) & 15
            out[:, base + 16 * pos + j, :] = scale * kv[nib]
    return out.transpose(0, 2, 1).copy()


def hbm_bytes(R, K):
    """Stored bytes of one R x K IQ4_XS matrix: R * K/256 * 136 (4.25 bits per weight)."""
    return R * (K // QK) * BLOCK_BYTES
