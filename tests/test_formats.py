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


def decode_tile_words(qs, R, K):
    """Codes [R, K] from one expert's tile plane, restated per column from the layout's definition:
    column c -> tile ct = c // 160, k-step m, k-chunk q, position j inside the tile (o = c % 160 = 32m + 8q + j);
    row r -> row tile r // 16, lane 16q + r % 16; code n = 8m + j sits in word pair p = n // 20 at c' = n % 20:
    c' < 4: word 2p byte c' bits 0-2;  c' < 8: word 2p byte c'-4 bits 3-5;  c' < 12: word 2p+1 byte c'-8 bits 0-2;
    c' < 16: word 2p+1 byte c'-12 bits 3-5;  else: word 2p byte c'-16 bits 6-7 | word 2p+1 byte c'-16 bit 6 << 2."""
    qs = np.asarray(qs, dtype=np.uint32).reshape(-1)
    RT = R // 16
    r = np.arange(R)[:, None]
    c = np.arange(K)[None, :]
    ct, o = c // 160, c % 160
    m, q, j = o // 32, (o % 32) // 8, o % 8
    n = 8 * m + j
    p, cc = n // 20, n % 20
    base = ((ct * RT + r // 16) * 64 + 16 * q + r % 16) * 4
    a = qs[base + 2 * p]
    b = qs[base + 2 * p + 1]
    byte = lambda w, k: (w >> (8 * k).astype(np.uint32)) & 255
    out = np.where(cc < 4, byte(a, cc % 4) & 7,
          np.where(cc < 8, (byte(a, (cc - 4) % 4) >> 3) & 7,
          np.where(cc < 12, byte(b, (cc - 8) % 4) & 7,
          np.where(cc < 16, (byte(b, (cc - 12) % 4) >> 3) & 7,
                   (byte(a, (cc - 16) % 4) >> 6) | (((byte(b, (cc - 16) % 4) >> 6) & 1) << 2)))))
    return out.astype(np.uint8)


@pytest.mark.parametrize("R,K", [(16, 128), (32, 256), (16, 640), (48, 1280), (64, 2048), (16, 6144)])
def test_cb3_tile_words_roundtrip(pkg, R, K):
    rng = np.random.default_rng(R * 7 + K)
    codes = rng.integers(0, 8, (3, R, K), dtype=np.uint8)
    qs = pkg.formats.cb3_tile_words(codes)
    CT = -(-K // 160)
    assert qs.shape == (3, CT * (R // 16) * 256)
    for e in range(3):
        assert np.array_equal(decode_tile_words(qs[e], R, K), codes[e])
    # padding columns of the last tile decode to code 0
    full = decode_tile_words(qs[0], R, CT * 160)
    assert not full[:, K:].any()
    # every bit of a tile word carries a code bit: 40 codes in 4 words, padding only in the last column tile
    assert 4 * 32 == 40 * 3 + 8 and qs.nbytes == 3 * R * CT * 160 * 4 // 10


def test_cb3_tile_words_single_codes(pkg):
    """One nonzero code at a time lands exactly where the layout puts it (catches transposed or shifted indices)."""
    R, K = 32, 320
    for (r, c, v) in [(0, 0, 1), (5, 7, 7), (17, 8, 3), (31, 159, 5), (3, 160, 6), (20, 183, 2), (9, 319, 4)]:
        codes = np.zeros((1, R, K), np.uint8)
        codes[0, r, c] = v
        qs = pkg.formats.cb3_tile_words(codes)[0]
        ct, o = divmod(c, 160)
        m, rem = divmod(o, 32)
        q, j = divmod(rem, 8)
        p, cc = divmod(8 * m + j, 20)
        w0 = ((ct * (R // 16) + r // 16) * 64 + 16 * q + r % 16) * 4 + 2 * p
        if cc < 8:
            want = {w0}
        elif cc < 16:
            want = {w0 + 1}
        else:          # split: low 2 bits in word 2p, high bit in word 2p+1
            want = ({w0} if v & 3 else set()) | ({w0 + 1} if v & 4 else set())
        assert set(np.flatnonzero(qs).tolist()) == want, (r, c)
        assert np.array_equal(decode_tile_words(qs, R, K), codes[0])


def test_cb3_pack_planes_layout(pkg):
    rng = np.random.default_rng(1)
    E, R, K = 2, 32, 1280
    codes, cb = zip(*[ocb3.generate(rng, R, K) for _ in range(E)])
    codes, cb = np.stack(codes), np.stack(cb)
    words = np.stack([ocb3.pack_canonical(c) for c in codes])
    pl = pkg.formats.cb3_pack_planes(words, cb, K)
    G, CT = K // 128, -(-K // 160)
    assert pl["qs"].shape == (E, CT * (R // 16) * 256) and pl["cb"].shape == (E, G * R * 4)
    for e in range(E):
        assert np.array_equal(decode_tile_words(pl["qs"][e], R, K), codes[e])
        cbw = pl["cb"][e].reshape(G, R, 4).transpose(1, 0, 2)          # [R, G, 4]
        lo = np.concatenate([(cbw[..., 0:1] >> (8 * np.arange(4))) & 255, (cbw[..., 1:2] >> (8 * np.arange(4))) & 255], -1)
        hi = np.concatenate([(cbw[..., 2:3] >> (8 * np.arange(4))) & 255, (cbw[..., 3:4] >> (8 * np.arange(4))) & 255], -1)
        assert np.array_equal((lo | (hi << 8)).astype(np.uint16), cb[e])
    # K = 1280 is a whole number of tiles: the device planes hold exactly the canonical bytes
    assert sum(a.nbytes for a in pl.values()) == E * ocb3.hbm_bytes(R, K)


def test_int8_pack(pkg):
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (64, 32), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (1, 32)).astype(np.float32)
    qT, sv, axis = pkg.formats.int8_pack(q, s)
    assert qT.shape == (32, 64) and np.array_equal(qT.T, q) and np.array_equal(sv, s[0]) and axis == 1
    sr = rng.uniform(0.5e-3, 2e-3, (64, 1)).astype(np.float32)        # per-row scales [in, 1] (quant8.py:26-32)
    qT, sv, axis = pkg.formats.int8_pack(q, sr)
    assert np.array_equal(qT.T, q) and np.array_equal(sv, sr[:, 0]) and axis == 0
    with pytest.raises(ValueError):
        pkg.formats.int8_pack(q, np.ones((64, 32), np.float32))
    L = pkg._lib.lib()
    assert L.mi_int8_project_workspace(8, 6144, 6144, 0) > 0 and L.mi_int8_project_workspace(8, 6144, 6144, 2) > 0
    assert L.mi_int8_project_workspace(8, 6144, 6144, 3) == 0
