"""CPU: pins the IQ3_S oracle (block dequant, planar packer, planar dequant) without the reference's code.

The reference holds no expected outputs for this path (its tests compute them at run time from gguf-py, which is
absent here), so the oracle is pinned by: the codebook grid's published invariants and its source data file, single
bit / single field perturbations whose effect the block definition fixes exactly (iqquant.py:123-132), agreement of
two independent restatements (block form vs planar form, planes.py:136-170,262-276), and the real GGUF block bytes
the reference's tests use as inputs (test_planes.py:67-76).
"""
import json
import os

import numpy as np
import pytest

from oracle import iq3s
from oracle.bf16 import f16_bits_to_f32

GG = os.path.join(os.path.dirname(__file__), "golden", "gguf")
REF_GRIDS = "/root/reference/launcher/glm53-flash/engine/glm53/data/iq_grids.npz"


def test_grid_invariants():
    g = iq3s.grid()
    assert g.shape == (512, 4) and g.dtype == np.int8
    assert set(np.unique(g).tolist()) <= {1, 3, 5, 7, 9, 11, 13, 15}       # odd levels 1..15
    assert len({tuple(r) for r in g.tolist()}) == 512                      # 512 distinct 4-vectors


@pytest.mark.skipif(not os.path.exists(REF_GRIDS), reason="reference data file not present on this machine")
def test_grid_matches_reference_data_file():
    z = np.load(REF_GRIDS)                                                 # numpy loader, no pickle
    assert np.array_equal(np.asarray(z["IQ3_S"], np.int8), iq3s.grid())


def _block(d=1.0, scales=0, qs=0, qh=0, signs=0):
    b = np.zeros(110, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:66] = qs
    b[66:74] = qh
    b[74:106] = signs
    b[106:110] = scales
    return b


def test_block_known_answers():
    """All-zero fields: every weight is d * 1 * grid[0][pos]; then one field at a time moves exactly what the block
    layout says it moves."""
    g = iq3s.grid().astype(np.float32)
    base = iq3s.dequant_blocks(_block(d=0.5)[None])[0]
    assert np.array_equal(base, 0.5 * np.tile(g[0], 64))
    # one sign bit (weight 77 = byte 74 + 9, bit 5)
    b = _block(d=0.5)
    b[74 + 77 // 8] = 1 << (77 % 8)
    w = iq3s.dequant_blocks(b[None])[0]
    assert np.array_equal(np.flatnonzero(w != base), [77]) and w[77] == -base[77]
    # one qs byte: group 10 (weights 40..43) takes grid[200]
    b = _block(d=0.5)
    b[2 + 10] = 200
    w = iq3s.dequant_blocks(b[None])[0]
    assert np.array_equal(w[40:44], 0.5 * g[200]) and np.array_equal(np.delete(w, range(40, 44)),
                                                                       np.delete(base, range(40, 44)))
    # the matching qh bit adds 256 to group 10's index
    b[66 + 10 // 8] = 1 << (10 % 8)
    w = iq3s.dequant_blocks(b[None])[0]
    assert np.array_equal(w[40:44], 0.5 * g[456])
    # scale nibble 3 (high nibble of byte 107) = 7 scales weights 96..127 by 1 + 2*7 = 15
    b = _block(d=0.5)
    b[106 + 1] = 7 << 4
    w = iq3s.dequant_blocks(b[None])[0]
    assert np.array_equal(w[96:128], 15 * base[96:128])
    assert np.array_equal(np.delete(w, range(96, 128)), np.delete(base, range(96, 128)))


def test_block_values_have_the_closed_form():
    """Every weight is f16(d) * (2 sc + 1) * odd level * +-1, exactly, for random blocks."""
    rng = np.random.default_rng(3)
    blk = iq3s.random_blocks(rng, 1, 4, 3)[0]
    w = iq3s.dequant_blocks(blk)                                              # [4, 3, 256]
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))
    ratio = np.abs(w) / d[..., None]
    ok = np.zeros_like(ratio, bool)
    for sc in range(16):
        for lv in (1, 3, 5, 7, 9, 11, 13, 15):
            ok |= ratio == (2 * sc + 1) * lv
    assert ok.all()


def test_block_form_equals_planar_form():
    rng = np.random.default_rng(5)
    for nblk in (1, 2, 3, 8):
        t = iq3s.random_blocks(rng, 2, 24, nblk)
        planes = iq3s.pack_planes(t)
        for k, rows in iq3s.plane_rows(nblk).items():
            assert planes[k].shape == (2 * rows, 24)
        got = iq3s.dequant_planes_natural(planes, nblk)                        # [E, R, K]
        want = iq3s.dequant_blocks(t).reshape(2, 24, nblk * 256)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_planar_bytes_are_the_block_bytes():
    """The planar tables hold the block bytes and nothing else (planes.py:12-14): same total byte count per expert
    (d padded to whole u32 for odd nblk), hbm_bytes = R * K/256 * 110."""
    rng = np.random.default_rng(6)
    t = iq3s.random_blocks(rng, 1, 8, 2)
    planes = iq3s.pack_planes(t)
    assert sum(a.nbytes for a in planes.values()) == t.nbytes
    assert iq3s.hbm_bytes(2048, 6144) == 2048 * 24 * 110
    # per expert at the benchmark shapes (gate + up + down)
    assert 2 * iq3s.hbm_bytes(2048, 6144) + iq3s.hbm_bytes(6144, 2048) == 16220160


def test_real_gguf_iq3s_rows():
    s = json.load(open(os.path.join(GG, "gguf_samples.json")))["IQ3_S"]
    raw = open(os.path.join(GG, s["file"]), "rb").read()
    assert len(raw) == s["nbytes"] == s["rows"] * s["ne0"] // 256 * 110
    w = iq3s.dequant_rows(raw, s["ne0"])
    assert w.shape == (s["rows"], s["ne0"]) and np.isfinite(w).all()
    blk = np.frombuffer(raw, np.uint8).reshape(s["rows"], -1, 110)
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))
    assert (np.abs(w).reshape(s["rows"], -1, 256) <= 31 * 15 * np.abs(d)[..., None]).all()
    # block form == planar form on real bytes too
    planes = iq3s.pack_planes(blk[None])
    got = iq3s.dequant_planes_natural(planes, blk.shape[1])[0]
    assert np.array_equal(got.view(np.uint32), w.view(np.uint32))
