"""CPU: the product's load-time packers agree with the oracle's independent restatements."""
import numpy as np
import pytest

from oracle import cb3 as ocb3, iq3s as oiq3


@pytest.mark.parametrize("R,nblk", [(16, 1), (16, 3), (8, 16), (24, 2)])
def test_iq3s_planes_match_oracle_packer(pkg, R, nblk):
    rng = np.random.default_rng(R * 31 + nblk)
    t = oiq3.random_blocks(rng, 3, R, nblk)
    ours = pkg.formats.iq3s_pack_planes(t)
    ref = oiq3.pack_planes(t)
    assert set(ours) == set(ref)
    for k in ref:
        assert ours[k].dtype == np.uint32 and np.array_equal(ours[k], ref[k]), k


@pytest.mark.parametrize("K", [128, 256, 384, 512, 640, 1280, 2048, 6144])
def test_cb3_device_words_roundtrip(pkg, K):
    rng = np.random.default_rng(K)
    codes = rng.integers(0, 8, (5, K), dtype=np.uint8)
    dev = pkg.formats.cb3_device_words(codes)
    assert dev.shape == (5, ocb3.words_per_row(K))
    assert np.array_equal(ocb3.decode_device_words(dev, K), codes)
    # bits 6-7 hold only C-field bits: no code bit is lost and the byte count equals the canonical packing
    assert dev.nbytes == ocb3.pack_canonical(codes).nbytes


def test_cb3_pack_planes_layout(pkg):
    rng = np.random.default_rng(1)
    E, R, K = 2, 8, 1280
    codes, cb = zip(*[ocb3.generate(rng, R, K) for _ in range(E)])
    codes, cb = np.stack(codes), np.stack(cb)
    words = np.stack([ocb3.pack_canonical(c) for c in codes])
    pl = pkg.formats.cb3_pack_planes(words, cb, K)
    Wd, G = ocb3.words_per_row(K), K // 128
    assert pl["qs"].shape == (E * Wd, R) and pl["cb"].shape == (E * G * 4, R)
    for e in range(E):
        dev = pl["qs"][e * Wd:(e + 1) * Wd].T
        assert np.array_equal(ocb3.decode_device_words(dev, K), codes[e])
        cbw = pl["cb"][e * G * 4:(e + 1) * G * 4].T.reshape(R, G, 4)
        lo = np.concatenate([(cbw[..., 0:1] >> (8 * np.arange(4))) & 255, (cbw[..., 1:2] >> (8 * np.arange(4))) & 255], -1)
        hi = np.concatenate([(cbw[..., 2:3] >> (8 * np.arange(4))) & 255, (cbw[..., 3:4] >> (8 * np.arange(4))) & 255], -1)
        assert np.array_equal((lo | (hi << 8)).astype(np.uint16), cb[e])
    assert sum(a.nbytes for a in pl.values()) == E * ocb3.hbm_bytes(R, K)


def test_int8_pack(pkg):
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (64, 32), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (1, 32)).astype(np.float32)
    qT, sv = pkg.formats.int8_pack(q, s)
    assert qT.shape == (32, 64) and np.array_equal(qT.T, q) and np.array_equal(sv, s[0])
    with pytest.raises(ValueError):
        pkg.formats.int8_pack(q, np.ones((64, 1), np.float32))          # per-row scales are not this layout
