"""IQ3_S oracle: llama.cpp IQ3_S blocks, the reference's planar tables and their dequant (test infrastructure only).

Block (110 bytes per 256 weights, iqquant.py:5-6,15):  d f16 [0:2] | qs [2:66] (low 8 bits of 64 grid indices) |
qh [66:74] (bit 8 of each index) | signs [74:106] (one bit per weight) | scales [106:110] (eight 4-bit scales,
low nibble first, one per 32 weights).
Weight = f16(d) * (1 + 2 * scale) * grid[idx][pos] * (+-1)        (iqquant.py:123-132)
Every factor is exact in f32 (<= 11 + 5 + 4 significant bits), so any evaluation order gives the same bits.

Planar tables (planes.py:22-25,136-170; one expert matrix = R rows, nblk blocks per row, W = 16 nblk words):
  qs u32 [W, R]       word w: byte j = low index bits of group 4w+j                 (GGUF bytes 2..65)
  sg u32 [W/2, R]     u32 w//2, half w%2: nibble j = signs of group 4w+j            (GGUF 74..105)
  qh u32 [W/8, R]     u32 w//8: bit 4(w%8)+j = bit 8 of group 4w+j's index          (GGUF 66..73)
  sc u32 [W/16, R]    u32 w//16: nibble (w//2)%8 = scale of words 2n, 2n+1          (GGUF 106..109)
  d  u32 [ceil(nblk/2), R]  u32 b//2, half b%2 = f16 bits of block b                (GGUF 0..1)
Experts are merged along axis 0: [E * rows_p, R].  Word w covers inputs 16w .. 16w+15 (planes.py:78).
"""
import os

import numpy as np

from .bf16 import f16_bits_to_f32

QK = 256
BLOCK_BYTES = 110
PLANE_KEYS = ("qs", "sg", "qh", "sc", "d")          # planes.py:45
_GRID = None


def grid():
    """int8 [512, 4] IQ3_S codebook (odd levels 1..15), the table vendored by the reference (iqquant.py:18)."""
    global _GRID
    if _GRID is None:
        _GRID = np.load(os.path.join(os.path.dirname(__file__), "data", "iq3s_grid.npy"))
        assert _GRID.shape == (512, 4) and _GRID.dtype == np.int8
    return _GRID


def plane_rows(nblk):
    """Rows per expert of every plane (planes.py:56-63)."""
    W = 16 * nblk
    return {"qs": W, "sg": W // 2, "qh": W // 8, "sc": W // 16, "d": (nblk + 1) // 2}


# ------------------------------------------------------------------------------------------------ block form
def dequant_blocks(blk):
    """uint8 [..., nblk, 110] -> f32 [..., nblk, 256]: restates iqquant.dequant_iq3_s (iqquant.py:123-132).
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


_CHUNK_BLOCKS = 8192


def _dequant_blocks(blk):
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))      # [...]
    qs = blk[..., 2:66].astype(np.int64)                                                            # [..., 64]
    qh = np.unpackbits(blk[..., 66:74], axis=-1, bitorder="little").astype(np.int64)               # [..., 64]
    signs = np.unpackbits(blk[..., 74:106], axis=-1, bitorder="little").astype(np.float32)         # [..., 256]
    sc_b = blk[..., 106:110]
    sc = np.stack([sc_b & 15, sc_b >> 4], axis=-1).reshape(blk.shape[:-1] + (8,)).astype(np.float32)
    idx = qs | (qh << 8)                                                                            # [..., 64]
    g = grid()[idx].astype(np.float32).reshape(blk.shape[:-1] + (8, 32))                           # 8 groups of 4 / scale
    db = d[..., None, None] * (1.0 + 2.0 * sc)[..., None]
    w = (db * g).reshape(blk.shape[:-1] + (QK,)) * (1.0 - 2.0 * signs)
    return w.astype(np.float32)


def dequant_rows(raw, ne0):
    """raw GGUF bytes of whole rows -> f32 [rows, ne0] (iqquant.py:236-240)."""
    blk = np.frombuffer(bytes(raw), np.uint8).reshape(-1, ne0 // QK, BLOCK_BYTES)
    return dequant_blocks(blk).reshape(blk.shape[0], ne0)


def random_blocks(rng, E, R, nblk, scale=0.02):
    """Uniform random block bytes with a finite f16 d in [scale/2, scale] (test_planes.py:17-26)."""
    t = rng.integers(0, 256, (E, R, nblk, BLOCK_BYTES), dtype=np.uint8)
    d = rng.uniform(0.5 * scale, scale, (E, R, nblk)).astype(np.float16)
    t[..., 0:2] = np.frombuffer(d.tobytes(), np.uint8).reshape(E, R, nblk, 2)
    return t


# ------------------------------------------------------------------------------------------------ planar form
def _u32(a):
    """[E, R, nblk, n] u8 -> [E, R, nblk*n/4] u32 little-endian (planes.py:122-127)."""
    E, R = a.shape[:2]
    a = np.ascontiguousarray(a.reshape(E, R, -1))
    return a.view("<u4")


def _merge(a):
    """[E, R, P] -> [E*P, R] (planes.py:130-133)."""
    E, R, P = a.shape
    return np.ascontiguousarray(a.transpose(0, 2, 1)).reshape(E * P, R)


def pack_planes(t):
    """uint8 [E, R, nblk, 110] -> {plane: u32 [E*rows_p, R]} (planes.py:136-170, IQ3_S branch)."""
    E, R, nblk, bb = t.shape
    assert bb == BLOCK_BYTES
    d = t[..., 0:2].reshape(E, R, nblk * 2)
    if nblk % 2:
        d = np.concatenate([d, np.zeros((E, R, 2), np.uint8)], -1)
    out = {"d": np.ascontiguousarray(d).view("<u4"),
           "qs": _u32(t[..., 2:66]), "qh": _u32(t[..., 66:74]), "sg": _u32(t[..., 74:106]),
           "sc": _u32(t[..., 106:110])}
    rows = plane_rows(nblk)
    res = {k: _merge(out[k]) for k in PLANE_KEYS}
    for k, a in res.items():
        assert a.shape == (E * rows[k], R), (k, a.shape)
    return res


def dequant_planes_natural(planes, nblk):
    """{plane: u32 [E*rows_p, R]} -> f32 [E, R, 256*nblk] in natural input order, read straight from the planar bit
    map (the module docstring).  An independent restatement of planes._deq_iq3_s + dequant_natural
    (planes.py:262-276,294-300): block form and planar form agreeing bit for bit pins the packer."""
    rows = plane_rows(nblk)
    R = planes["qs"].shape[-1]
    E = planes["qs"].shape[0] // rows["qs"]
    p = {k: np.asarray(planes[k], dtype=np.uint32).reshape(E, rows[k], R) for k in PLANE_KEYS}
    W = 16 * nblk
    w = np.arange(W)
    qs = p["qs"]                                                        # [E, W, R]
    sgh = (p["sg"][:, w // 2, :] >> ((w % 2) * 16)[None, :, None]) & 0xFFFF
    qhn = (p["qh"][:, w // 8, :] >> ((w % 8) * 4)[None, :, None]) & 15
    scn = (p["sc"][:, w // 16, :] >> (((w // 2) % 8) * 4)[None, :, None]) & 15
    b = w // 16
    dbits = (p["d"][:, b // 2, :] >> ((b % 2) * 16)[None, :, None]) & 0xFFFF
    scale = f16_bits_to_f32(dbits) * (1.0 + 2.0 * scn.astype(np.float32))      # [E, W, R]
    out = np.zeros((E, W, 16, R), np.float32)
    g = grid().astype(np.float32)
    for j in range(4):
        idx = ((qs >> (8 * j)) & 255) | (((qhn >> j) & 1) << 8)
        lv = g[idx]                                                      # [E, W, R, 4]
        for k in range(4):
            s = ((sgh >> (4 * j + k)) & 1).astype(np.float32)
            out[:, :, 4 * j + k, :] = scale * lv[..., k] * (1.0 - 2.0 * s)
    return out.reshape(E, W * 16, R).transpose(0, 2, 1).copy()          # input = 16 w + 4 j + k


def hbm_bytes(R, K):
    """Stored bytes of one R x K IQ3_S matrix: R * K/256 * 110 (3.4375 bits per weight)."""
    return R * (K // QK) * BLOCK_BYTES
