"""CPU: the committed fixtures agree with each other and with the oracle.

* the IQ3_S and IQ2_S grids are each committed twice (oracle/data/iq3s_grid.npy, iq2s_grid.npy for the oracle,
  csrc/iq3s_grid.inc, iq2s_grid.inc for the HIP library); both copies come from the reference's data file and must
  be the same table;
* the regression vectors under tests/golden/ (inputs + expected outputs, written by make_fixtures.py) still match
  what the oracle computes, so a drifting oracle or a corrupted fixture fails here, on the CPU.
"""
import os
import re

import numpy as np

from oracle import cb3, int8 as oi8, iq2s, iq3s, moe

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


def test_grid_inc_equals_oracle_grid():
    text = open(os.path.join(REPO, "kaggle-llm-endpoint_amd", "csrc", "iq3s_grid.inc")).read()
    words = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", text)], np.uint32)
    assert words.shape == (512,)
    g = np.stack([(words >> (8 * k)) & 255 for k in range(4)], -1).astype(np.int8)
    assert np.array_equal(g, iq3s.grid())


def test_iq2s_grid_inc_equals_oracle_grid():
    text = open(os.path.join(REPO, "kaggle-llm-endpoint_amd", "csrc", "iq2s_grid.inc")).read()
    words = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", text)], np.uint32)
    assert words.shape == (2048,)
    w = words.reshape(1024, 2)
    g = np.concatenate([np.stack([(w[:, h] >> (8 * k)) & 255 for k in range(4)], -1) for h in range(2)], -1)
    assert np.array_equal(g.astype(np.int8), iq2s.grid())


def _load(name):
    return np.load(os.path.join(HERE, "golden", name + ".npz"))


def test_cb3_vector():
    z = _load("cb3_mv")
    codes = cb3.unpack_canonical(z["words"], z["x"].shape[1])
    y = moe.matvec_f64(cb3.dequant(codes, z["cb"]), z["x"]).astype(np.float32)
    assert np.array_equal(y, z["y"])


def test_iq3s_vector():
    z = _load("iq3s_mv")
    blk = z["blocks"][0]
    w = iq3s.dequant_blocks(blk).reshape(blk.shape[0], -1)
    y = moe.matvec_f64(w, z["x"]).astype(np.float32)
    assert np.array_equal(y, z["y"])


def test_int8_vector():
    z = _load("int8")
    assert np.array_equal(oi8.project_bf16(z["x"], z["q"], z["s"]), z["y"])
