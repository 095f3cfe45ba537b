"""Host-side packers that turn stored weights into the device tables the HIP kernels read (load-time work, NumPy).

* IQ3_S, IQ4_XS: GGUF blocks -> the reference's planar tables, unchanged (planes.py:136-170); the kernels read those
  planes directly, so tables packed by the reference's own ``pack_planes`` drop in as they are.
* CB3 (the benchmark's 3-bit codebook format): canonical rows (10 codes per u32, 8 bf16 centroids per 128-column
  group) -> 16-row x 160-column code tiles in the lane order of the matrix-core kernels (cb3_tile_words) and a
  [group][row] codebook plane.  Same bytes per row as the canonical form plus the zero padding of the last tile.
* int8 (quant8.py:17-18): {"q": int8 [in, out], "s": f32 [1, out]} -> qT int8 [out, in] + s f32 [out].
"""
import numpy as np

QK = 256
IQ3S_BLOCK_BYTES = 110
CB3_GROUP = 128


# ------------------------------------------------------------------------------------------------ IQ3_S
def iq3s_plane_rows(nblk):
    """rows_p per expert (planes.py:62-63)."""
    W = 16 * nblk
    return {"qs": W, "sg": W // 2, "qh": W // 8, "sc": W // 16, "d": (nblk + 1) // 2}


def _le_words(a):
    E, R = a.shape[:2]
    return np.ascontiguousarray(a.reshape(E, R, -1)).view("<u4")


def _expert_major(a):
    """[E, R, P] -> [E*P, R]: experts stacked, rows on the minor axis."""
    E, R, P = a.shape
    return np.ascontiguousarray(a.transpose(0, 2, 1)).reshape(E * P, R)


def iq3s_pack_planes(blocks):
    """uint8 [E, R, nblk, 110] GGUF IQ3_S blocks -> {plane: u32 [E*rows_p, R]} in the reference's planar layout
    (field split of planes.py:153-160: d | qs | qh | sg | sc)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    E, R, nblk, bb = blocks.shape
    if bb != IQ3S_BLOCK_BYTES:
        raise ValueError("IQ3_S blocks are %d bytes, got %d" % (IQ3S_BLOCK_BYTES, bb))
    d = blocks[..., 0:2].reshape(E, R, 2 * nblk)
    if nblk % 2:
        d = np.concatenate([d, np.zeros((E, R, 2), np.uint8)], axis=-1)
    raw = {"qs": blocks[..., 2:66], "qh": blocks[..., 66:74], "sg": blocks[..., 74:106], "sc": blocks[..., 106:110]}
    out = {k: _expert_major(_le_words(v)) for k, v in raw.items()}
    out["d"] = _expert_major(np.ascontiguousarray(d).view("<u4"))
    return {k: out[k] for k in ("qs", "sg", "qh", "sc", "d")}


def iq3s_hbm_bytes(R, K):
    return R * (K // QK) * IQ3S_BLOCK_BYTES


# ------------------------------------------------------------------------------------------------ IQ2_S
IQ2S_BLOCK_BYTES = 82


def iq2s_plane_rows(nblk):
    """rows_p per expert (planes.py:60-61)."""
    W = 8 * nblk
    return {"qs": W, "sg": W, "qh": W // 4, "sc": W // 4, "d": (nblk + 1) // 2}


def iq2s_pack_planes(blocks):
    """uint8 [E, R, nblk, 82] GGUF IQ2_S blocks -> {plane: u32 [E*rows_p, R]} in the reference's planar layout
    (field split of planes.py:157-158: d | qs | sg | qh | sc)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    E, R, nblk, bb = blocks.shape
    if bb != IQ2S_BLOCK_BYTES:
        raise ValueError("IQ2_S blocks are %d bytes, got %d" % (IQ2S_BLOCK_BYTES, bb))
    d = blocks[..., 0:2].reshape(E, R, 2 * nblk)
    if nblk % 2:
        d = np.concatenate([d, np.zeros((E, R, 2), np.uint8)], axis=-1)
    raw = {"qs": blocks[..., 2:34], "sg": blocks[..., 34:66], "qh": blocks[..., 66:74], "sc": blocks[..., 74:82]}
    out = {k: _expert_major(_le_words(v)) for k, v in raw.items()}
    out["d"] = _expert_major(np.ascontiguousarray(d).view("<u4"))
    return {k: out[k] for k in ("qs", "sg", "qh", "sc", "d")}


def iq2s_hbm_bytes(R, K):
    return R * (K // QK) * IQ2S_BLOCK_BYTES


# ------------------------------------------------------------------------------------------------ Q2_K, Q3_K
KQ_BLOCK_BYTES = {"Q2_K": 84, "Q3_K": 110}


def q3k_unpack_scales(sc12):
    """Q3_K's 12 packed scale bytes -> the 16 six-bit scales as bytes (iqquant.py:190-201): scale i takes its low 4 bits
    from byte i % 8 (low nibble for i < 8, high nibble above) and its high 2 bits from byte 8 + i % 4, bits 2 (i // 4)."""
    sc12 = np.asarray(sc12, np.uint8)
    out = [((sc12[..., i % 8] >> (0 if i < 8 else 4)) & 15) | (((sc12[..., 8 + i % 4] >> (2 * (i // 4))) & 3) << 4)
           for i in range(16)]
    return np.stack(out, axis=-1).astype(np.uint8)


def kq_pack_planes(blocks, qtype):
    """uint8 [E, R, nblk, bb] GGUF Q2_K / Q3_K blocks -> {plane: u32 [E*rows_p, R]} in the reference's planar layout
    (planes.py:140-150: Q2_K qs | sc | d+dmin; Q3_K qs | hm | unpacked sc | d zero-extended)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    E, R, nblk, bb = blocks.shape
    if bb != KQ_BLOCK_BYTES[qtype]:
        raise ValueError("%s blocks are %d bytes, got %d" % (qtype, KQ_BLOCK_BYTES[qtype], bb))
    if qtype == "Q2_K":
        raw = {"qs": blocks[..., 16:80], "sc": blocks[..., 0:16], "d": blocks[..., 80:84]}
        keys = ("qs", "sc", "d")
    else:
        d = np.concatenate([blocks[..., 108:110], np.zeros((E, R, nblk, 2), np.uint8)], axis=-1)
        raw = {"qs": blocks[..., 32:96], "hm": blocks[..., 0:32], "sc": q3k_unpack_scales(blocks[..., 96:108]),
               "d": d}
        keys = ("qs", "hm", "sc", "d")
    out = {k: _expert_major(_le_words(v)) for k, v in raw.items()}
    return {k: out[k] for k in keys}


# ------------------------------------------------------------------------------------------------ IQ4_XS
IQ4XS_BLOCK_BYTES = 136


def iq4xs_plane_rows(nblk):
    """rows_p per expert (planes.py:64-65)."""
    return {"qs": 32 * nblk, "sl": nblk, "sh": nblk, "d": (nblk + 1) // 2}


def iq4xs_pack_planes(blocks):
    """uint8 [E, R, nblk, 136] GGUF IQ4_XS blocks -> {plane: u32 [E*rows_p, R]} in the reference's planar layout
    (field split of planes.py:161-163: d | sh (zero-extended to 32 bits) | sl | qs)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    E, R, nblk, bb = blocks.shape
    if bb != IQ4XS_BLOCK_BYTES:
        raise ValueError("IQ4_XS blocks are %d bytes, got %d" % (IQ4XS_BLOCK_BYTES, bb))
    d = blocks[..., 0:2].reshape(E, R, 2 * nblk)
    if nblk % 2:
        d = np.concatenate([d, np.zeros((E, R, 2), np.uint8)], axis=-1)
    sh = np.concatenate([blocks[..., 2:4], np.zeros((E, R, nblk, 2), np.uint8)], axis=-1)
    raw = {"qs": blocks[..., 8:136], "sl": blocks[..., 4:8], "sh": sh}
    out = {k: _expert_major(_le_words(v)) for k, v in raw.items()}
    out["d"] = _expert_major(np.ascontiguousarray(d).view("<u4"))
    return {k: out[k] for k in ("qs", "sl", "sh", "d")}


def iq4xs_hbm_bytes(R, K):
    return R * (K // QK) * IQ4XS_BLOCK_BYTES


# ------------------------------------------------------------------------------------------------ CB3
def cb3_words_per_row(K):
    return -(-K // 10)


def cb3_unpack_canonical(words, K):
    """u32 [..., Wd] canonical words (code j of word w at bits 3j) -> u8 [..., K] codes."""
    words = np.asarray(words, dtype=np.uint32)
    c = (words[..., None] >> (3 * np.arange(10, dtype=np.uint32))) & 7
    return c.reshape(words.shape[:-1] + (words.shape[-1] * 10,))[..., :K].astype(np.uint8)


CB3_TILE_ROWS = 16
CB3_TILE_COLS = 160


def cb3_tile_count(K):
    """Column tiles per row (the last one zero-padded past K)."""
    return -(-K // CB3_TILE_COLS)


def cb3_tile_words(codes):
    """u8 codes [E, R, K] -> u32 [E, CT*RT*256]: the matrix-core tile layout of the CB3 kernels.
    Tile (ct, rt) = rows 16rt..16rt+15 x columns 160ct..160ct+159, 1 KB, tiles ordered [ct][rt].  Lane l = 16q + i
    of a tile holds row 16rt + i at columns 160ct + 32m + 8q + j (m = 0..4, j = 0..7) as code n = 8m + j, in 4 words;
    word pair p (words 2p, 2p+1) holds n = 20p + c, c = 0..19:
        word 2p   byte b = code[c=b] | code[c=4+b] << 3 | (code[c=16+b] & 3) << 6
        word 2p+1 byte b = code[c=8+b] | code[c=12+b] << 3 | (code[c=16+b] >> 2) << 6
    Columns past K hold code 0."""
    codes = np.asarray(codes, dtype=np.uint32)
    E, R, K = codes.shape
    if R % CB3_TILE_ROWS:
        raise ValueError("CB3 tiles need rows in multiples of 16, got %d" % R)
    CT, RT = cb3_tile_count(K), R // CB3_TILE_ROWS
    c = np.zeros((E, R, CT * CB3_TILE_COLS), np.uint32)
    c[..., :K] = codes
    c = c.reshape(E, RT, 16, CT, 5, 4, 8).transpose(0, 3, 1, 5, 2, 4, 6)    # e, ct, rt, q, i, m, j
    c = c.reshape(E, CT, RT, 64, 2, 20)                                      # lane = 16q + i; n = 8m + j = 20p + c
    j = np.arange(4)
    a = c[..., j] | (c[..., 4 + j] << 3) | ((c[..., 16 + j] & 3) << 6)
    b = c[..., 8 + j] | (c[..., 12 + j] << 3) | ((c[..., 16 + j] >> 2) << 6)
    sh = (8 * j).astype(np.uint32)
    wa = (a << sh).sum(-1, dtype=np.uint64).astype(np.uint32)
    wb = (b << sh).sum(-1, dtype=np.uint64).astype(np.uint32)
    return np.stack([wa, wb], axis=-1).reshape(E, CT * RT * 256)


def cb3_codebook_words(cb):
    """bf16 bits u16 [..., G, 8] -> u32 [..., G, 4]: lo bytes of centroids 0-3, 4-7, hi bytes 0-3, 4-7."""
    cb = np.asarray(cb, dtype=np.uint16)
    lo = (cb & 0xFF).astype(np.uint32)
    hi = (cb >> 8).astype(np.uint32)
    sh = (8 * np.arange(4)).astype(np.uint32)
    pack = lambda a: (a << sh).sum(-1, dtype=np.uint64).astype(np.uint32)
    return np.stack([pack(lo[..., 0:4]), pack(lo[..., 4:8]), pack(hi[..., 0:4]), pack(hi[..., 4:8])], axis=-1)


def cb3_pack_planes(words, cb, K):
    """Canonical CB3 experts -> device planes.
    words u32 [E, R, ceil(K/10)] (canonical), cb u16 [E, R, K/128, 8] (bf16 bits) ->
    {"qs": u32 [E, CT*RT*256] (cb3_tile_words), "cb": u32 [E, G*R*4] ([group][row][4 dwords])}."""
    words = np.asarray(words, dtype=np.uint32)
    E, R, Wd = words.shape
    if K % CB3_GROUP or Wd != cb3_words_per_row(K):
        raise ValueError("CB3: K must be a multiple of 128 with ceil(K/10) words per row")
    G = K // CB3_GROUP
    cb = np.asarray(cb, dtype=np.uint16)
    if cb.shape != (E, R, G, 8):
        raise ValueError("CB3 codebook must be [E, R, K/128, 8], got %s" % (cb.shape,))
    qs = cb3_tile_words(cb3_unpack_canonical(words, K))
    cbw = np.ascontiguousarray(cb3_codebook_words(cb).transpose(0, 2, 1, 3)).reshape(E, G * R * 4)
    return {"qs": qs, "cb": cbw}


def cb3_plane_words(R, K):
    """u32 words per expert of each CB3 device plane."""
    return {"qs": cb3_tile_count(K) * (R // CB3_TILE_ROWS) * 256, "cb": (K // CB3_GROUP) * R * 4}


def cb3_hbm_bytes(R, K):
    return R * (4 * cb3_words_per_row(K) + 16 * (K // CB3_GROUP))


# ------------------------------------------------------------------------------------------------ int8
def int8_pack(q, s):
    """Reference leaf {"q": int8 [in, out], "s": f32 [1, out] or [in, 1]} (quant8.py:17-18,26-32) ->
    (qT int8 [out, in], s flat f32, axis): axis 1 for per-column scales [1, out] (s [out]), 0 for per-row scales
    [in, 1] (s [in]), as quantize_array's ``axis``."""
    q = np.asarray(q, dtype=np.int8)
    s = np.asarray(s, dtype=np.float32)
    if q.ndim != 2:
        raise ValueError("int8_pack expects q [in, out]")
    if s.shape == (1, q.shape[1]):
        axis = 1
    elif s.shape == (q.shape[0], 1):
        axis = 0
    else:
        raise ValueError("int8_pack expects scales [1, out] or [in, 1], got %s for q %s" % (s.shape, q.shape))
    return np.ascontiguousarray(q.T), np.ascontiguousarray(s.reshape(-1)), axis
