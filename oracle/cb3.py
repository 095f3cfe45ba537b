"""CB3 oracle -- the benchmark's synthetic 3-bit codebook format (test infrastructure only).

No reference function implements CB3; it is defined by the benchmark configuration text and pinned by closed form:
  code[r, k] in [0, 8), codebook C[r, g, 0..7] bf16 sorted ascending (g = k // 128),
  w[r, k] = C[r, k // 128, code[r, k]]  (exact bf16 -> f32),
  canonical packing: word[r, w] = sum_{j<10} code[r, 10w + j] << 3j, bits 30-31 zero, ceil(K/10) words per row.
Stored bytes of an R x K matrix: R * (4 * ceil(K/10) + 16 * K/128)  (4.203 bits per weight at K = 2048, 6144).
"""
import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

GROUP = 128


def words_per_row(K):
    return -(-K // 10)


def generate(rng, N, K, sigma=0.02):
    """(codes u8 [N, K] uniform in [0,8), codebook bf16 bits u16 [N, K/128, 8] sorted ascending)."""
    assert K % GROUP == 0
    codes = rng.integers(0, 8, (N, K), dtype=np.uint8)
    c = np.sort(rng.normal(0.0, sigma, (N, K // GROUP, 8)).astype(np.float32), axis=-1)
    cb = f32_to_bf16_bits(c)
    # rounding can reorder only equal neighbours; keep the sorted invariant on the stored bits
    cbf = bf16_bits_to_f32(cb)
    cb = f32_to_bf16_bits(np.sort(cbf, axis=-1))
    return codes, cb


def bf16_normal(rng, shape):
    """bf16-representable N(0,1) activations as f32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal(shape).astype(np.float32)))


def pack_canonical(codes):
    """codes u8 [N, K] -> words u32 [N, ceil(K/10)] with word = sum_j code[10w+j] << 3j."""
    N, K = codes.shape
    Wd = words_per_row(K)
    c = np.zeros((N, Wd * 10), np.uint32)
    c[:, :K] = codes
    c = c.reshape(N, Wd, 10)
    return (c << (3 * np.arange(10, dtype=np.uint32))).sum(-1, dtype=np.uint64).astype(np.uint32)


def unpack_canonical(words, K):
    """words u32 [N, Wd] -> codes u8 [N, K]."""
    words = np.asarray(words, dtype=np.uint32)
    N, Wd = words.shape
    c = (words[:, :, None] >> (3 * np.arange(10, dtype=np.uint32))) & 7
    return c.reshape(N, Wd * 10)[:, :K].astype(np.uint8)


def dequant(codes, cb):
    """codes u8 [N, K], cb u16 [N, G, 8] -> f32 [N, K]: w = C[r, k//128, code]."""
    N, K = codes.shape
    g = np.arange(K) // GROUP
    bits = cb[np.arange(N)[:, None], g[None, :], codes.astype(np.int64)]
    return bf16_bits_to_f32(bits)


def hbm_bytes(R, K):
    return R * (4 * words_per_row(K) + 16 * (K // GROUP))


def decode_device_words(dev, K):
    """Codes from the kernel's word layout (an independent per-column restatement used to pin the packer):
    column c = 20P + o of a word pair (words 2P, 2P+1 = a, b):
      o < 4: a byte o bits 0-2;  o < 8: a byte o-4 bits 3-5;  o < 12: b byte o-8 bits 0-2;  o < 16: b byte o-12 bits 3-5;
      o >= 16 (j = o-16): (a byte j bits 6-7) | (b byte j bit 6) << 2.
    A trailing single word a (odd word count): o < 8 as above, o = 8: a bits 6-7 | a bit 22 << 2, o = 9: a bits
    14-15 | a bit 30 << 2."""
    dev = np.asarray(dev, dtype=np.uint32)
    N, Wd = dev.shape
    out = np.zeros((N, K), np.uint8)
    for c in range(K):
        P, o = divmod(c, 20)
        a = dev[:, 2 * P]
        single = 2 * P + 1 >= Wd
        b = dev[:, 2 * P + 1] if not single else None
        byte = lambda v, j: (v >> (8 * j)) & 255
        if o < 4:
            v = byte(a, o) & 7
        elif o < 8:
            v = (byte(a, o - 4) >> 3) & 7
        elif single:
            if o == 8:
                v = ((a >> 6) & 3) | (((a >> 22) & 1) << 2)
            elif o == 9:
                v = ((a >> 14) & 3) | (((a >> 30) & 1) << 2)
            else:
                raise ValueError("column beyond the last word")
        elif o < 12:
            v = byte(b, o - 8) & 7
        elif o < 16:
            v = (byte(b, o - 12) >> 3) & 7
        else:
            j = o - 16
            v = ((byte(a, j) >> 6) & 3) | (((byte(b, j) >> 6) & 1) << 2)
        out[:, c] = v
    return out
