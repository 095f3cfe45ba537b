"""Q2_K / Q3_K oracle (the MTP layer's experts): ggml's K-quant blocks, the reference's planar tables and their
dequant (test infrastructure only).

Q2_K block (84 bytes per 256 weights, iqquant.py:15): scales [0:16] (per 16 weights: low nibble scale, high nibble
min) | qs [16:80] (2-bit values) | d f16 [80:82] | dmin f16 [82:84].
Q3_K block (110 bytes): hmask [0:32] (high bits) | qs [32:96] (2-bit low parts) | scales [96:108] (sixteen 6-bit
scales, packed) | d f16 [108:110].
Weight position p = 128 n + 32 s + l of a block (half n, shift s, l = 0..31) takes bits 2s, 2s+1 of qs byte 32 n + l,
scale byte is = 8 n + 2 s + (l >= 16) and, for Q3_K, hmask bit 4 n + s of byte l (ggml dequantize_row_q2_K /
dequantize_row_q3_K, restated by iqquant.py:204-229):
  Q2_K: w = (d * (sc & 15)) * v - dmin * (sc >> 4)     one f32 rounding (the product d * sc * v is exact)
  Q3_K: w = d * (sc6 - 32) * (v - (hbit ? 0 : 4))      exact in f32
Q3_K's 12 scale bytes unpack to 16 six-bit values (iqquant.py:190-201): index i < 8: low nibble of byte i % 8 ... as
_q3k_scale below states per index.

Planar tables (planes.py:34-41,136-170; W = 16 nblk words of qs per row): qs u32 [W, R] (word w = qs bytes
4w .. 4w+3 of the row); Q2_K sc u32 [4 nblk, R] (the block's 16 scale bytes), d u32 [nblk, R] (d | dmin << 16);
Q3_K hm u32 [8 nblk, R] (the hmask bytes), sc u32 [4 nblk, R] (the 16 unpacked scales as bytes), d u32 [nblk, R]
(f16 d in the low half).  Word w, byte j holds input 256 (w // 16) + 128 ((w % 16) // 8) + 32 s + 4 (w % 8) + j at
shift s.
"""
import numpy as np

from .bf16 import f16_bits_to_f32

QK = 256
BLOCK_BYTES = {"Q2_K": 84, "Q3_K": 110}
PLANE_KEYS = {"Q2_K": ("qs", "sc", "d"), "Q3_K": ("qs", "hm", "sc", "d")}      # planes.py:45-46


def plane_rows(qtype, nblk):
    """Rows per expert of every plane (planes.py:66-69)."""
    if qtype == "Q2_K":
        return {"qs": 16 * nblk, "sc": 4 * nblk, "d": nblk}
    return {"qs": 16 * nblk, "hm": 8 * nblk, "sc": 4 * nblk, "d": nblk}


def _f16(b, o):
    return f16_bits_to_f32(b[..., o].astype(np.uint32) | (b[..., o + 1].astype(np.uint32) << 8))


def _q3k_scale(sc12, i):
    """Six-bit scale i (0..15) of Q3_K's 12 packed bytes: low 4 bits from byte i % 8 (low nibble for i < 8, high
    nibble for i >= 8), high 2 bits from byte 8 + i % 4 at bit 2 (i // 4)."""
    lo = (sc12[..., i % 8] >> (0 if i < 8 else 4)) & 15
    hi = (sc12[..., 8 + i % 4] >> (2 * (i // 4))) & 3
    return (lo | (hi << 4)).astype(np.uint8)


def q3k_scales(sc12):
    """uint8 [..., 12] -> uint8 [..., 16] (the unpacked scales in `is` order)."""
    sc12 = np.asarray(sc12, np.uint8)
    return np.stack([_q3k_scale(sc12, i) for i in range(16)], axis=-1)


def dequant_blocks(blk, qtype):
    """uint8 [..., nblk, bb] -> f32 [..., nblk, 256] in natural order."""
    blk = np.asarray(blk, np.uint8)
    if qtype == "Q2_K":
        sc, qs = blk[..., 0:16], blk[..., 16:80]
        d, dmin = _f16(blk, 80), _f16(blk, 82)
    else:
        hm, qs, sc = blk[..., 0:32], blk[..., 32:96], q3k_scales(blk[..., 96:108])
        d = _f16(blk, 108)
    out = np.empty(blk.shape[:-1] + (QK,), np.float32)
    for n in range(2):
        for s in range(4):
            v = ((qs[..., 32 * n:32 * n + 32] >> (2 * s)) & 3).astype(np.float32)              # [..., 32]
            for h in range(2):
                b = sc[..., 8 * n + 2 * s + h].astype(np.float32)[..., None]
                vv = v[..., 16 * h:16 * h + 16]
                if qtype == "Q2_K":
                    bi = sc[..., 8 * n + 2 * s + h]
                    dl = (d * (bi & 15).astype(np.float32))[..., None]
                    ml = (np.asarray(dmin) * (bi >> 4).astype(np.float32))[..., None]
                    w = (dl * vv).astype(np.float32) - ml                                          # one rounding
                else:
                    hb = ((hm[..., 16 * h:16 * h + 16] >> (4 * n + s)) & 1).astype(np.float32)
                    w = d[..., None] * (b - 32.0) * (vv - 4.0 * (1.0 - hb))
                o = 128 * n + 32 * s + 16 * h
                out[..., o:o + 16] = w.astype(np.float32)
    return out


def random_blocks(rng, qtype, E, R, nblk, scale=0.02):
    """Uniform random block bytes with finite f16 d (and dmin) in [scale/2, scale]."""
    bb = BLOCK_BYTES[qtype]
    t = rng.integers(0, 256, (E, R, nblk, bb), dtype=np.uint8)
    offs = (80, 82) if qtype == "Q2_K" else (108,)
    for o in offs:
        d = rng.uniform(0.5 * scale, scale, (E, R, nblk)).astype(np.float16)
        t[..., o:o + 2] = np.frombuffer(d.tobytes(), np.uint8).reshape(E, R, nblk, 2)
    return t


def _u32(a):
    E, R = a.shape[:2]
    return np.ascontiguousarray(a.reshape(E, R, -1)).view("<u4")


def _merge(a):
    E, R, P = a.shape
    return np.ascontiguousarray(a.transpose(0, 2, 1)).reshape(E * P, R)


def pack_planes(t, qtype):
    """uint8 [E, R, nblk, bb] -> {plane: u32 [E*rows_p, R]} (planes.py:140-150, the K-quant branch)."""
    E, R, nblk, bb = t.shape
    assert bb == BLOCK_BYTES[qtype]
    if qtype == "Q2_K":
        out = {"qs": _u32(t[..., 16:80]), "sc": _u32(t[..., 0:16]), "d": _u32(t[..., 80:84])}
    else:
        d = np.concatenate([t[..., 108:110], np.zeros((E, R, nblk, 2), np.uint8)], -1)
        out = {"qs": _u32(t[..., 32:96]), "hm": _u32(t[..., 0:32]), "sc": _u32(q3k_scales(t[..., 96:108])),
               "d": _u32(d)}
    rows = plane_rows(qtype, nblk)
    res = {k: _merge(out[k]) for k in PLANE_KEYS[qtype]}
    for k, a in res.items():
        assert a.shape == (E * rows[k], R), (k, a.shape)
    return res


def dequant_planes_natural(planes, qtype, nblk):
    """{plane: u32 [E*rows_p, R]} -> f32 [E, R, 256*nblk], read straight from the planar bit map (the module
    docstring; planes.py:209-243): block form == planar form pins the packer."""
    rows = plane_rows(qtype, nblk)
    R = planes["qs"].shape[-1]
    E = planes["qs"].shape[0] // rows["qs"]
    p = {k: np.asarray(planes[k], np.uint32).reshape(E, rows[k], R) for k in PLANE_KEYS[qtype]}
    out = np.zeros((E, nblk * QK, R), np.float32)
    for w in range(16 * nblk):
        b, n, q = w // 16, (w % 16) // 8, w % 8
        word = p["qs"][:, w, :]
        dw = p["d"][:, b, :]
        d = f16_bits_to_f32(dw & 0xFFFF)
        for s in range(4):
            for j in range(4):
                v = ((word >> (8 * j + 2 * s)) & 3).astype(np.float32)
                i_s = 8 * n + 2 * s + (q >= 4)
                scb = (p["sc"][:, 4 * b + i_s // 4, :] >> (8 * (i_s % 4))) & 255
                if qtype == "Q2_K":
                    dl = d * (scb & 15).astype(np.float32)
                    ml = f16_bits_to_f32(dw >> 16) * (scb >> 4).astype(np.float32)
                    val = (dl * v).astype(np.float32) - ml
                else:
                    l = 4 * q + j
                    hmb = (p["hm"][:, 8 * b + l // 4, :] >> (8 * (l % 4))) & 255
                    hb = ((hmb >> (4 * n + s)) & 1).astype(np.float32)
                    val = d * (scb.astype(np.float32) - 32.0) * (v - 4.0 * (1.0 - hb))
                out[:, 256 * b + 128 * n + 32 * s + 4 * q + j, :] = val
    return out.transpose(0, 2, 1).copy()


def hbm_bytes(qtype, R, K):
    return R * (K // QK) * BLOCK_BYTES[qtype]
