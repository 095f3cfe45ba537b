"""CPU: pins the CB3 oracle (the benchmark's 3-bit codebook format; no reference function exists).

Closed form: w[r, k] = C[r, k // 128, code[r, k]] (bf16 exact), canonical words hold 10 codes of 3 bits each.
Pinned by single-code perturbations, the byte counts the benchmark configuration quotes, and the generator's
distribution invariants.
"""
import numpy as np

from oracle import cb3
from oracle.bf16 import bf16_bits_to_f32


def test_canonical_pack_roundtrip_and_bits():
    rng = np.random.default_rng(1)
    for K in (128, 640, 2048, 6144):
        codes = rng.integers(0, 8, (5, K), dtype=np.uint8)
        words = cb3.pack_canonical(codes)
        assert words.shape == (5, -(-K // 10)) and words.dtype == np.uint32
        assert not (words >> 30).any()                                   # bits 30-31 unused
        assert np.array_equal(cb3.unpack_canonical(words, K), codes)


def test_canonical_single_code_positions():
    K = 128
    for c, v in [(0, 1), (9, 7), (10, 5), (127, 3)]:
        codes = np.zeros((1, K), np.uint8)
        codes[0, c] = v
        words = cb3.pack_canonical(codes)[0]
        want = np.zeros_like(words)
        want[c // 10] = v << (3 * (c % 10))
        assert np.array_equal(words, want)


def test_dequant_single_code_and_group():
    rng = np.random.default_rng(2)
    codes, cb = cb3.generate(rng, 4, 384)
    base = cb3.dequant(codes, cb)
    assert np.array_equal(base[2, 130].view(np.uint32), bf16_bits_to_f32(cb[2, 1, codes[2, 130]]).view(np.uint32))
    c2 = codes.copy()
    c2[2, 300] = (c2[2, 300] + 3) % 8
    w = cb3.dequant(c2, cb)
    diff = np.argwhere(w != base)
    assert diff.tolist() == [[2, 300]] and w[2, 300] == bf16_bits_to_f32(cb[2, 2, c2[2, 300]])


def test_generator_invariants():
    rng = np.random.default_rng(3)
    codes, cb = cb3.generate(rng, 64, 2048)
    assert codes.min() >= 0 and codes.max() <= 7
    c = bf16_bits_to_f32(cb)
    assert c.shape == (64, 16, 8) and (np.diff(c, axis=-1) >= 0).all()          # sorted centroids
    assert 0.01 < c.std() < 0.03                                              # N(0, 0.02)


def test_byte_counts_of_the_benchmark():
    assert cb3.hbm_bytes(1024, 2048) == 1101824                 # config 0: codes 1024 x 205 u32 + C [1024,16,8] bf16
    per_expert = 2 * cb3.hbm_bytes(2048, 6144) + cb3.hbm_bytes(6144, 2048)
    assert per_expert == 19832832
    assert 9 * per_expert == 178495488                          # config 1: 8 routed + 1 shared expert
