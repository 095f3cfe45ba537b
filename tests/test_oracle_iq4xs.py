"""CPU: pins the IQ4_XS oracle (block dequant, planar packer, planar dequant) without the reference's code.

As for IQ3_S, the reference holds no expected outputs (its tests compute them at run time from gguf-py, absent
here).  The oracle is pinned by: the level table's source data file and published values, single-field
perturbations whose effect the block definition fixes exactly (iqquant.py:137-148), agreement of two independent
restatements (block form vs planar form, planes.py:136-170 and the planar bit map of planes.py:26-28), and the real
GGUF block bytes the reference's tests use as inputs (test_planes.py:67-76).
"""
import json
import os

import numpy as np
import pytest

from oracle import iq4xs
from oracle.bf16 import f16_bits_to_f32

GG = os.path.join(os.path.dirname(__file__), "golden", "gguf")
REF_GRIDS = "/root/reference/launcher/glm53-flash/engine/glm53/data/iq_grids.npz"


def test_kvalues():
    kv = iq4xs.kvalues()
    # llama.cpp's published kvalues_iq4nl: 16 sorted, distinct int8 levels spanning -127 .. 113
    assert kv.dtype == np.int8 and kv.shape == (16,)
    assert (np.diff(kv.astype(int)) > 0).all() and kv[0] == -127 and kv[-1] == 113


@pytest.mark.skipif(not os.path.exists(REF_GRIDS), reason="reference data file not present on this machine")
def test_kvalues_match_reference_data_file():
    z = np.load(REF_GRIDS)
    assert np.array_equal(np.asarray(z["kvalues_iq4nl"], np.int8), iq4xs.kvalues())


def _block(d=1.0, sh=0, sl=0, qs=0):
    b = np.zeros(136, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(sh).tobytes(), np.uint8)
    b[4:8] = sl
    b[8:136] = qs
    return b


def test_block_known_answers():
    kv = iq4xs.kvalues().astype(np.float32)
    # all-zero fields: scale = 0 - 32 = -32, every index 0 -> d * -32 * kv[0]
    base = iq4xs.dequant_blocks(_block(d=0.25)[None])[0]
    assert np.array_equal(base, np.full(256, 0.25 * -32 * kv[0], np.float32))
    # byte 8 + 16*3 + 5 (sub-block 3, byte 5): low nibble = weight 96 + 5, high nibble = weight 96 + 21
    b = _block(d=0.25)
    b[8 + 16 * 3 + 5] = 0x9C                                   # low 12, high 9
    w = iq4xs.dequant_blocks(b[None])[0]
    assert w[101] == 0.25 * -32 * kv[12] and w[117] == 0.25 * -32 * kv[9]
    assert np.array_equal(np.delete(w, [101, 117]), np.delete(base, [101, 117]))
    # scale of sub-block 6: low nibble (sl byte 3, low half) = 5, high bits (sh bits 12, 13) = 2 -> 5 + 32 - 32 = 5
    b = _block(d=0.25)
    b[4 + 3] = 5
    b[2:4] = np.frombuffer(np.uint16(2 << 12).tobytes(), np.uint8)
    w = iq4xs.dequant_blocks(b[None])[0]
    assert np.array_equal(w[192:224], np.full(32, 0.25 * 5 * kv[0], np.float32))
    assert np.array_equal(np.delete(w, range(192, 224)), np.delete(base, range(192, 224)))
    # sl byte 0 high nibble = scale low bits of sub-block 1 (weights 32..63)
    b = _block(d=0.25)
    b[4] = 0xF0
    w = iq4xs.dequant_blocks(b[None])[0]
    assert np.array_equal(w[32:64], np.full(32, 0.25 * (15 - 32) * kv[0], np.float32))


def test_block_values_have_the_closed_form():
    """Every weight is f16(d) * (s - 32) * kvalue for some 6-bit s and table entry, exactly."""
    rng = np.random.default_rng(3)
    blk = iq4xs.random_blocks(rng, 1, 4, 3)[0]
    w = iq4xs.dequant_blocks(blk)
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))
    ratio = w / d[..., None]
    cands = np.array(sorted({(s - 32) * int(v) for s in range(64) for v in iq4xs.kvalues()}), np.float64)
    assert np.isin(ratio.astype(np.float64), cands).all()


def test_block_form_equals_planar_form():
    rng = np.random.default_rng(5)
    for nblk in (1, 2, 3, 8):
        t = iq4xs.random_blocks(rng, 2, 24, nblk)
        planes = iq4xs.pack_planes(t)
        for k, rows in iq4xs.plane_rows(nblk).items():
            assert planes[k].shape == (2 * rows, 24)
        got = iq4xs.dequant_planes_natural(planes, nblk)
        want = iq4xs.dequant_blocks(t).reshape(2, 24, nblk * 256)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_planar_bytes():
    """The planes hold the block bytes (sh zero-extended to 32 bits, d padded for odd nblk); hbm_bytes = R*K/256*136."""
    rng = np.random.default_rng(6)
    t = iq4xs.random_blocks(rng, 1, 8, 2)
    planes = iq4xs.pack_planes(t)
    assert sum(a.nbytes for a in planes.values()) == t.nbytes + 8 * 2 * 2
    assert iq4xs.hbm_bytes(6144, 2048) == 6144 * 8 * 136


def test_real_gguf_iq4xs_rows():
    s = json.load(open(os.path.join(GG, "gguf_samples.json")))["IQ4_XS"]
    raw = open(os.path.join(GG, s["file"]), "rb").read()
    assert len(raw) == s["nbytes"] == s["rows"] * s["ne0"] // 256 * 136
    blk = np.frombuffer(raw, np.uint8).reshape(s["rows"], -1, 136)
    w = iq4xs.dequant_blocks(blk).reshape(s["rows"], s["ne0"])
    assert np.isfinite(w).all()
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint32) | (blk[..., 1].astype(np.uint32) << 8))
    assert (np.abs(w).reshape(s["rows"], -1, 256) <= 32 * 127 * np.abs(d)[..., None]).all()
    planes = iq4xs.pack_planes(blk[None])
    got = iq4xs.dequant_planes_natural(planes, blk.shape[1])[0]
    assert np.array_equal(got.view(np.uint32), w.view(np.uint32))
