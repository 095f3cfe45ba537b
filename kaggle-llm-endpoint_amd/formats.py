"""Host-side packers that turn stored weights into the device tables the HIP kernels read (load-time work, NumPy).

* IQ3_S: GGUF blocks -> the reference's planar tables, unchanged (planes.py:136-170); the kernels read those
  planes directly, so tables packed by the reference's own ``pack_planes`` drop in as they are.
* CB3 (the benchmark's 3-bit codebook format): canonical rows (10 codes per u32, 8 bf16 centroids per 128-column
  group) -> planes in the same "matrix row = minor axis" convention, with the code bits rearranged inside each word
  pair so that the kernel gets byte-sized codebook selectors from one AND.  Same byte count as the canonical form.
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


# ------------------------------------------------------------------------------------------------ CB3
def cb3_words_per_row(K):
    return -(-K // 10)


def cb3_unpack_canonical(words, K):
    """u32 [..., Wd] canonical words (code j of word w at bits 3j) -> u8 [..., K] codes."""
    words = np.asarray(words, dtype=np.uint32)
    c = (words[..., None] >> (3 * np.arange(10, dtype=np.uint32))) & 7
    return c.reshape(words.shape[:-1] + (words.shape[-1] * 10,))[..., :K].astype(np.uint8)


def cb3_device_words(codes):
    """u8 codes [..., K] -> u32 [..., ceil(K/10)] in the kernel's word layout:
    pair P (columns c = 20P..20P+19):  word 2P   byte j = code[c+j] | code[c+4+j] << 3 | (code[c+16+j] & 3) << 6
                                       word 2P+1 byte j = code[c+8+j] | code[c+12+j] << 3 | (code[c+16+j] >> 2) << 6
    trailing single word (odd count):  byte j = code[c+j] | code[c+4+j] << 3; code[c+8], code[c+9] low 2 bits in
                                       bits 6-7 of bytes 0, 1 and high bits in bit 6 of bytes 2, 3."""
    codes = np.asarray(codes, dtype=np.uint32)
    lead, K = codes.shape[:-1], codes.shape[-1]
    Wd = cb3_words_per_row(K)
    npair, tail = Wd // 2, Wd % 2
    c = np.zeros(lead + (20 * npair + 10 * tail,), np.uint32)
    c[..., :K] = codes
    out = np.zeros(lead + (Wd,), np.uint32)
    if npair:
        p = c[..., :20 * npair].reshape(lead + (npair, 20))
        j = np.arange(4)
        b0 = p[..., j] | (p[..., 4 + j] << 3) | ((p[..., 16 + j] & 3) << 6)            # [..., npair, 4]
        b1 = p[..., 8 + j] | (p[..., 12 + j] << 3) | ((p[..., 16 + j] >> 2) << 6)
        sh = (8 * j).astype(np.uint32)
        out[..., 0:2 * npair:2] = (b0 << sh).sum(-1, dtype=np.uint64).astype(np.uint32)
        out[..., 1:2 * npair:2] = (b1 << sh).sum(-1, dtype=np.uint64).astype(np.uint32)
    if tail:
        t = c[..., 20 * npair:]
        j = np.arange(4)
        b = t[..., j] | (t[..., 4 + j] << 3)
        c8, c9 = t[..., 8], t[..., 9]
        b[..., 0] |= (c8 & 3) << 6
        b[..., 1] |= (c9 & 3) << 6
        b[..., 2] |= (c8 >> 2) << 6
        b[..., 3] |= (c9 >> 2) << 6
        out[..., Wd - 1] = (b << (8 * j).astype(np.uint32)).sum(-1, dtype=np.uint64).astype(np.uint32)
    return out


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
    {"qs": u32 [E*Wd, R], "cb": u32 [E*G*4, R]}."""
    words = np.asarray(words, dtype=np.uint32)
    E, R, Wd = words.shape
    if K % CB3_GROUP or Wd != cb3_words_per_row(K):
        raise ValueError("CB3: K must be a multiple of 128 with ceil(K/10) words per row")
    G = K // CB3_GROUP
    cb = np.asarray(cb, dtype=np.uint16)
    if cb.shape != (E, R, G, 8):
        raise ValueError("CB3 codebook must be [E, R, K/128, 8], got %s" % (cb.shape,))
    dev = cb3_device_words(cb3_unpack_canonical(words, K))                   # [E, R, Wd]
    cbw = cb3_codebook_words(cb).reshape(E, R, G * 4)                        # [E, R, G*4]
    return {"qs": _expert_major(dev), "cb": _expert_major(cbw)}


def cb3_hbm_bytes(R, K):
    return R * (4 * cb3_words_per_row(K) + 16 * (K // CB3_GROUP))


# ------------------------------------------------------------------------------------------------ int8
def int8_pack(q, s):
    """Reference leaf {"q": int8 [in, out], "s": f32 [1, out]} (per-column scales) -> (qT int8 [out, in], s [out])."""
    q = np.asarray(q, dtype=np.int8)
    s = np.asarray(s, dtype=np.float32)
    if s.shape != (1, q.shape[1]):
        raise ValueError("int8_pack expects per-output-channel scales [1, out], got %s" % (s.shape,))
    return np.ascontiguousarray(q.T), np.ascontiguousarray(s.reshape(-1))
