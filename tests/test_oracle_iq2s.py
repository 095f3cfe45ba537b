"""CPU: pins the IQ2_S oracle (block dequant, planar packer, planar dequant) without the reference's code.

As for IQ3_S and IQ4_XS, the reference holds no expected outputs (its tests compute them at run time from gguf-py,
absent here).  The oracle is pinned by: the grid's source data file and published entries, single-field
perturbations whose effect the block definition fixes exactly (iqquant.py:110-120), agreement of two independent
restatements (block form vs planar form, planes.py:136-170 and the planar bit map of planes.py:17-21), and the real
GGUF block bytes the reference's tests use as inputs (test_planes.py:67-76).
"""
import json
import os

import numpy as np
import pytest

from oracle import iq2s
from oracle.bf16 import f16_bits_to_f32

GG = os.path.join(os.path.dirname(__file__), "golden", "gguf")
REF_GRIDS = "/root/reference/launcher/glm53-flash/engine/glm53/data/iq_grids.npz"


def test_grid():
    g = iq2s.grid()
    assert g.dtype == np.int8 and g.shape == (1024, 8)
    assert set(np.unique(g).tolist()) == {8, 25, 43}
    assert len({tuple(r) for r in g.tolist()}) == 1024                 # distinct codewords
    # llama.cpp's published iq2s_grid, entries 0..3 and 1023, as little-endian uint64 (byte k = position k)
    u = np.ascontiguousarray(g.astype(np.uint8)).view("<u8")[:, 0]
    assert [int(v) for v in u[:4]] == [0x0808080808080808, 0x080808080808082b, 0x0808080808081919,
                                       0x0808080808082b08]


@pytest.mark.skipif(not os.path.exists(REF_GRIDS), reason="reference data file not present on this machine")
def test_grid_matches_reference_data_file():
    z = np.load(REF_GRIDS)
    assert np.array_equal(np.asarray(z["IQ2_S"], np.int8), iq2s.grid())


def _block(d=1.0, qs=0, signs=0, qh=0, sc=0):
    b = np.zeros(82, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:34] = qs
    b[34:66] = signs
    b[66:74] = qh
    b[74:82] = sc
    return b


def test_block_known_answers():
    g = iq2s.grid().astype(np.float32)
    # all-zero fields: scale (0.5 + 0) * 0.25 = 1/8, index 0 (all eights), no signs -> d * 1/8 * 8 = d
    base = iq2s.dequant_blocks(_block(d=0.5)[None])[0]
    assert np.array_equal(base, np.full(256, 0.5, np.float32))
    # group 13 (weights 104..111): qs byte 13 = 7, qh byte 3 bits 2..3 (group 13 = 4*3 + 1) = 2 -> index 2*256 + 7
    b = _block(d=0.5)
    b[2 + 13] = 7
    b[66 + 3] = 2 << 2
    w = iq2s.dequant_blocks(b[None])[0]
    assert np.array_equal(w[104:112], 0.5 * 0.125 * g[512 + 7])
    assert np.array_equal(np.delete(w, range(104, 112)), np.delete(base, range(104, 112)))
    # sign byte 21 bit 6 -> weight 8*21 + 6 negated
    b = _block(d=0.5)
    b[34 + 21] = 1 << 6
    w = iq2s.dequant_blocks(b[None])[0]
    assert w[174] == -0.5 and np.array_equal(np.delete(w, 174), np.delete(base, 174))
    # scale byte 5, high nibble = 9 -> scale of groups 22, 23 (weights 176..191) = (0.5 + 9) * 0.25
    b = _block(d=0.5)
    b[74 + 5] = 9 << 4
    w = iq2s.dequant_blocks(b[None])[0]
    assert np.array_equal(w[176:192], np.full(16, 0.5 * 9.5 * 0.25 * 8, np.float32))
    assert np.array_equal(np.delete(w, range(176, 192)), np.delete(base, range(176, 192)))


def test_block_values_have_the_closed_form():
    """Every weight is f16(d) * (2s + 1) / 8 * (+-level) for a 4-bit s and a level in {8, 25, 43}, exactly."""
    rng = np.random.default_rng(3)
    blk = iq2s.random_blocks(rng, 1, 4, 3)[0]
    w = iq2s.dequant_blocks(blk)
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))
    ratio = w.astype(np.float64) / d[..., None]
    cands = np.array(sorted({sg * (2 * s + 1) * v / 8 for s in range(16) for v in (8, 25, 43) for sg in (1, -1)}))
    assert np.isin(ratio, cands).all()


def test_block_form_equals_planar_form():
    rng = np.random.default_rng(5)
    for nblk in (1, 2, 3, 8):
        t = iq2s.random_blocks(rng, 2, 24, nblk)
        planes = iq2s.pack_planes(t)
        for k, rows in iq2s.plane_rows(nblk).items():
            assert planes[k].shape == (2 * rows, 24)
        got = iq2s.dequant_planes_natural(planes, nblk)
        want = iq2s.dequant_blocks(t).reshape(2, 24, nblk * 256)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_planar_bytes():
    """The planes hold exactly the block bytes (d padded for odd nblk); hbm_bytes = R*K/256*82."""
    rng = np.random.default_rng(6)
    t = iq2s.random_blocks(rng, 1, 8, 2)
    planes = iq2s.pack_planes(t)
    assert sum(a.nbytes for a in planes.values()) == t.nbytes
    assert iq2s.hbm_bytes(2048, 6144) == 2048 * 24 * 82


def test_real_gguf_iq2s_rows():
    s = json.load(open(os.path.join(GG, "gguf_samples.json")))["IQ2_S"]
    raw = open(os.path.join(GG, s["file"]), "rb").read()
    assert len(raw) == s["nbytes"] == s["rows"] * s["ne0"] // 256 * 82
    w = iq2s.dequant_rows(raw, s["ne0"])
    assert w.shape == (s["rows"], s["ne0"]) and np.isfinite(w).all()
    blk = np.frombuffer(raw, np.uint8).reshape(s["rows"], -1, 82)
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))
    assert (np.abs(w).reshape(s["rows"], -1, 256) <= 43 * 31 / 8 * np.abs(d)[..., None]).all()
    planes = iq2s.pack_planes(blk[None])
    got = iq2s.dequant_planes_natural(planes, blk.shape[1])[0]
    assert np.array_equal(got.view(np.uint32), w.view(np.uint32))
