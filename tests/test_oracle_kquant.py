"""CPU: pins the Q2_K / Q3_K oracle (block dequant, scale unpacking, planar packer, planar dequant).

The reference holds no K-quant vectors (its tests build layouts at run time, T/test_spec_decode.py:27-43), so the
oracle is pinned by: the Q3_K scale unpacking checked against a second, word-parallel restatement (ggml's mask
form), single-field perturbations with exact expected weights, Q2_K's single f32 rounding against an f64 closed
form, and block form == planar form bit for bit."""
import numpy as np
import pytest

from oracle import kquant as kq
from oracle.bf16 import f16_bits_to_f32


def _q3k_scales_words(sc12):
    """The same unpacking on 32-bit words (ggml's kmask form): 3 words in, 4 words of 4 scales out."""
    sc12 = np.asarray(sc12, np.uint8)
    a = [sc12[..., 4 * i:4 * i + 4].copy().view("<u4")[..., 0] for i in range(3)]
    m1, m2 = np.uint32(0x03030303), np.uint32(0x0F0F0F0F)
    words = [(a[0] & m2) | (((a[2] >> 0) & m1) << 4), (a[1] & m2) | (((a[2] >> 2) & m1) << 4),
             ((a[0] >> 4) & m2) | (((a[2] >> 4) & m1) << 4), ((a[1] >> 4) & m2) | (((a[2] >> 6) & m1) << 4)]
    return np.stack(words, -1).astype("<u4").view(np.uint8)


def test_q3k_scales_two_restatements_and_known_answers():
    rng = np.random.default_rng(1)
    sc = rng.integers(0, 256, (500, 12), dtype=np.uint8)
    assert np.array_equal(kq.q3k_scales(sc), _q3k_scales_words(sc))
    one = np.zeros(12, np.uint8)
    one[1], one[9] = 0xA5, 0x30                                  # scale 1 = 5, scale 9 = 10 | 3 << 4
    s = kq.q3k_scales(one)
    want = np.zeros(16, np.uint8)
    want[1], want[9] = 5, 58
    assert np.array_equal(s, want)


def _blk(qtype, **fields):
    b = np.zeros(kq.BLOCK_BYTES[qtype], np.uint8)
    for o, v in fields.get("f16", []):
        b[o:o + 2] = np.frombuffer(np.float16(v).tobytes(), np.uint8)
    for o, v in fields.get("bytes", []):
        b[o] = v
    return b


def test_q2k_known_answers():
    # d = 1, dmin = 0.5; scale byte is = 5 (half 0, shift 2, second 16) = scale 2 | min 3 << 4;
    # qs byte 16 + 3 (l = 19) bits 4-5 = 2 -> weight 32*2 + 19 = 83 = 1*2*2 - 0.5*3
    b = _blk("Q2_K", f16=[(80, 1.0), (82, 0.5)], bytes=[(5, 0x32), (16 + 19, 2 << 4)])
    w = kq.dequant_blocks(b[None], "Q2_K")[0]
    want = np.zeros(256, np.float32)
    want[80:96] = -1.5
    want[83] = 2.5
    assert np.array_equal(w, want)


def test_q3k_known_answers():
    # all zero: scale 0 - 32, value 0 - 4 (high bit clear) -> d * 128 everywhere
    b = _blk("Q3_K", f16=[(108, 0.25)])
    w = kq.dequant_blocks(b[None], "Q3_K")[0]
    assert np.array_equal(w, np.full(256, 32.0, np.float32))
    # hmask byte 5 bit 6 (half 1, shift 2): weight 128 + 64 + 5 -> value 0 -> 0
    b = _blk("Q3_K", f16=[(108, 0.25)], bytes=[(5, 1 << 6)])
    w = kq.dequant_blocks(b[None], "Q3_K")[0]
    assert w[197] == 0.0 and np.array_equal(np.delete(w, 197), np.full(255, 32.0, np.float32))
    # qs byte 32 + 32 + 7 (half 1, l = 7) = 3 at shift 0: weight 128 + 7 -> 0.25 * -32 * (3 - 4) = 8
    b = _blk("Q3_K", f16=[(108, 0.25)], bytes=[(32 + 32 + 7, 3)])
    w = kq.dequant_blocks(b[None], "Q3_K")[0]
    assert w[135] == 8.0


def test_q2k_single_rounding_closed_form():
    rng = np.random.default_rng(2)
    t = kq.random_blocks(rng, "Q2_K", 1, 16, 3)[0]
    w = kq.dequant_blocks(t, "Q2_K")
    d = f16_bits_to_f32(t[..., 80].astype(np.uint32) | (t[..., 81].astype(np.uint32) << 8)).astype(np.float64)
    dm = f16_bits_to_f32(t[..., 82].astype(np.uint32) | (t[..., 83].astype(np.uint32) << 8)).astype(np.float64)
    for p in range(256):
        n, s, l = p // 128, (p // 32) % 4, p % 32
        sc = t[..., 8 * n + 2 * s + (l >= 16)].astype(np.float64)
        v = ((t[..., 16 + 32 * n + l] >> (2 * s)) & 3).astype(np.float64)
        exact = d * np.floor(sc % 16) * v - dm * np.floor(sc / 16)
        assert np.array_equal(w[..., p], exact.astype(np.float32))


@pytest.mark.parametrize("qtype", ["Q2_K", "Q3_K"])
def test_block_form_equals_planar_form(qtype):
    rng = np.random.default_rng(5)
    for nblk in (1, 2, 3):
        t = kq.random_blocks(rng, qtype, 2, 12, nblk)
        planes = kq.pack_planes(t, qtype)
        for k, rows in kq.plane_rows(qtype, nblk).items():
            assert planes[k].shape == (2 * rows, 12)
        got = kq.dequant_planes_natural(planes, qtype, nblk)
        want = kq.dequant_blocks(t, qtype).reshape(2, 12, nblk * 256)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_planar_bytes():
    rng = np.random.default_rng(6)
    t = kq.random_blocks(rng, "Q2_K", 1, 8, 2)
    assert sum(a.nbytes for a in kq.pack_planes(t, "Q2_K").values()) == t.nbytes
    t = kq.random_blocks(rng, "Q3_K", 1, 8, 2)
    assert sum(a.nbytes for a in kq.pack_planes(t, "Q3_K").values()) == 8 * 2 * (64 + 32 + 16 + 4)


@pytest.mark.parametrize("qtype", ["Q2_K", "Q3_K"])
def test_host_packer_equals_oracle(pkg, qtype):
    rng = np.random.default_rng(9)
    t = kq.random_blocks(rng, qtype, 3, 20, 3)
    a, b = pkg.formats.kq_pack_planes(t, qtype), kq.pack_planes(t, qtype)
    assert set(a) == set(b) and all(np.array_equal(a[k], b[k]) for k in b)
