"""IQ2_S oracle: llama.cpp IQ2_S blocks, the reference's planar tables and their dequant (test infrastructure only).

Block (82 bytes per 256 weights, iqquant.py:5-6,15):  d f16 [0:2] | qs [2:34] (low 8 bits of 32 grid indices, one
per group of 8 weights) | signs [34:66] (one bit per weight, byte g = group g, bit k = position k) | qh [66:74] (two
high index bits per group, 4 groups per byte, low bits first) | scales [74:82] (sixteen 4-bit scales, low nibble
first, one per 16 weights = 2 groups).
Weight = f16(d) * (0.5 + scale) * 0.25 * grid[idx][pos] * (+-1)      (iqquant.py:110-120)
Every factor is exact in f32 (d: 11 significant bits, (0.5 + s) * 0.25 = (2s + 1) / 8: 5 bits, grid levels 8, 25, 43:
6 bits), so any evaluation order gives the same bits.

Planar tables (planes.py:17-21,136-170; one expert matrix = R rows, nblk blocks per row, W = 8 nblk words):
  qs u32 [W, R]       word w: byte j = low index bits of group 4w+j                 (GGUF bytes 2..33)
  sg u32 [W, R]       word w: byte j = signs of group 4w+j                          (GGUF 34..65)
  qh u32 [W/4, R]     u32 w//4, byte w%4: bits 2j, 2j+1 = high index bits of group 4w+j   (GGUF 66..73)
  sc u32 [W/4, R]     u32 w//4, byte w%4: nibble h = scale of groups 4w+2h, 4w+2h+1       (GGUF 74..81)
  d  u32 [ceil(nblk/2), R]  u32 b//2, half b%2 = f16 bits of block b                (GGUF 0..1)
Experts are merged along axis 0: [E * rows_p, R].  Word w covers inputs 32w .. 32w+31 (planes.py:76-77).
"""
import os

import numpy as np

from .bf16 import f16_bits_to_f32

QK = 256
BLOCK_BYTES = 82
PLANE_KEYS = ("qs", "sg", "qh", "sc", "d")          # planes.py:45
LEVELS = (8, 25, 43)                                # iqquant.py:48
_GRID = None


def grid():
    """int8 [1024, 8] IQ2_S codebook (levels 8, 25, 43), the table vendored by the reference (iqquant.py:18)."""
    global _GRID
    if _GRID is None:
        _GRID = np.load(os.path.join(os.path.dirname(__file__), "data", "iq2s_grid.npy"))
        assert _GRID.shape == (1024, 8) and _GRID.dtype == np.int8
    return _GRID


def plane_rows(nblk):
    """Rows per expert of every plane (planes.py:56-62)."""
    W = 8 * nblk
    return {"qs": W, "sg": W, "qh": W // 4, "sc": W // 4, "d": (nblk + 1) // 2}


# ------------------------------------------------------------------------------------------------ block form
_CHUNK_BLOCKS = 8192


def dequant_blocks(blk):
    """uint8 [..., nblk, 82] -> f32 [..., nblk, 256]: restates iqquant.dequant_iq2_s (iqquant.py:110-120).
    Every block decodes on its own, so large inputs are decoded in chunks of blocks (smaller temporaries)."""
    blk = np.asarray(blk, dtype=np.uint8)
    n = blk.size // BLOCK_BYTES
    if n > _CHUNK_BLOCKS:
        flat = blk.reshape(n, BLOCK_BYTES)
        out = np.empty((n, QK), np.float32)
        for i in range(0, n, _CHUNK_BLOCKS):
            out[i:i + _CHUNK_BLOCKS] = _dequant_blocks(flat[i:i + _CHUNK_BLOCKS])
        return out.reshape(blk.shape[:-1] + (QK,))
    return _dequant_blocks(blk)


def _dequant_blocks(blk):
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))      # [...]
    qs = blk[..., 2:34].astype(np.int64)                                                            # [..., 32]
    signs = np.unpackbits(blk[..., 34:66], axis=-1, bitorder="little").astype(np.float32)          # [..., 256]
    qh = blk[..., 66:74].astype(np.int64)                                                           # [..., 8]
    hi = np.stack([(qh >> (2 * k)) & 3 for k in range(4)], axis=-1).reshape(blk.shape[:-1] + (32,))
    sc_b = blk[..., 74:82]
    sc = np.stack([sc_b & 15, sc_b >> 4], axis=-1).reshape(blk.shape[:-1] + (16,)).astype(np.float32)
    idx = qs | (hi << 8)                                                                            # [..., 32]
    g = grid()[idx].astype(np.float32).reshape(blk.shape[:-1] + (16, 16))                          # 2 groups / scale
    db = d[..., None, None] * (0.5 + sc)[..., None] * 0.25
    w = (db * g).reshape(blk.shape[:-1] + (QK,)) * (1.0 - 2.0 * signs)
    return w.astype(np.float32)


def dequant_rows(raw, ne0):
    """raw GGUF bytes of whole rows -> f32 [rows, ne0] (iqquant.py:236-240)."""
    blk = np.frombuffer(bytes(raw), np.uint8).reshape(-1, ne0 // QK, BLOCK_BYTES)
    return dequant_blocks(blk).reshape(blk.shape[0], ne0)


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
    """uint8 [E, R, nblk, 82] -> {plane: u32 [E*rows_p, R]} (planes.py:136-170, IQ2_S branch)."""
    E, R, nblk, bb = t.shape
    assert bb == BLOCK_BYTES
    d = t[..., 0:2].reshape(E, R, nblk * 2)
    if nblk % 2:
        d = np.concatenate([d, np.zeros((E, R, 2), np.uint8)], -1)
    out = {"d": np.ascontiguousarray(d).view("<u4"), "qs": _u32(t[..., 2:34]), "sg": _u32(t[..., 34:66]),
           "qh": _u32(t[..., 66:74]), "sc": _u32(t[..., 74:82])}
    rows = plane_rows(nblk)
    res = {k: _merge(out[k]) for k in PLANE_KEYS}
    for k, a in res.items():
        assert a.shape == (E * rows[k], R), (k, a.shape)
    return res


def dequant_planes_natural(planes, nblk):
    """{plane: u32 [E*rows_p, R]} -> f32 [E, R, 256*nblk] in natural input order, read straight from the planar bit
    map (the module docstring).  An independent restatement of planes._deq_iq2_s + dequant_natural
    (planes.py:246-259,294-300): block form and planar form agreeing bit for bit pins the packer."""
    rows = plane_rows(nblk)
    R = planes["qs"].shape[-1]
    E = planes["qs"].shape[0] // rows["qs"]
    p = {k: np.asarray(planes[k], dtype=np.uint32).reshape(E, rows[k], R) for k in PLANE_KEYS}
    W = 8 * nblk
    w = np.arange(W)
    qs, sg = p["qs"], p["sg"]                                           # [E, W, R]
    qhb = (p["qh"][:, w // 4, :] >> ((w % 4) * 8)[None, :, None]) & 255
    scb = (p["sc"][:, w // 4, :] >> ((w % 4) * 8)[None, :, None]) & 255
    b = w // 8
    dbits = (p["d"][:, b // 2, :] >> ((b % 2) * 16)[None, :, None]) & 0xFFFF
    d = f16_bits_to_f32(dbits)
    out = np.zeros((E, W, 32, R), np.float32)
    g = grid().astype(np.float32)
    for j in range(4):
        idx = ((qs >> (8 * j)) & 255) | (((qhb >> (2 * j)) & 3) << 8)
        lv = g[idx]                                                      # [E, W, R, 8]
        s_nib = ((scb >> (4 * (j // 2))) & 15).astype(np.float32)
        scale = d * (0.5 + s_nib) * 0.25
        for k in range(8):
            s = ((sg >> (8 * j + k)) & 1).astype(np.float32)
            out[:, :, 8 * j + k, :] = scale * lv[..., k] * (1.0 - 2.0 * s)
    return out.reshape(E, W * 32, R).transpose(0, 2, 1).copy()          # input = 32 w + 8 j + k


def hbm_bytes(R, K):
    """Stored bytes of one R x K IQ2_S matrix: R * K/256 * 82 (2.5625 bits per weight)."""
    return R * (K // QK) * BLOCK_BYTES
