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
