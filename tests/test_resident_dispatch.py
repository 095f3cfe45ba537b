"""CPU: ResidentFetch picks the reference's branch for each call (resident.py:100-108,137-143) and keeps its
constructor's attributes; bad modes are rejected at construction."""
import pytest
import torch


def test_branches_follow_the_reference(pkg):
    f = pkg.ResidentFetch({0: {}}, 256, 256, gather_max_rows=64)
    assert f.branch(8, 8) == "kernel" and f.branch(9, 8) == "ragged" and f.branch(1, 64) == "kernel"
    assert pkg.ResidentFetch({}, 256, 256, use_pallas=False).branch(8, 8) == "gather"
    assert pkg.ResidentFetch({}, 256, 256, use_pallas=False).branch(9, 8) == "sweep_xla"
    assert pkg.ResidentFetch({}, 256, 256, sweep_mode="dense").branch(9, 8) == "sweep"
    assert pkg.ResidentFetch({}, 256, 256, gather_max_rows=1000).branch(20, 2) == "kernel"


def test_constructor_attributes(pkg):
    f = pkg.ResidentFetch({1: {"gate_q": "IQ2_S"}}, 6144, 256, out_dtype=torch.float32, gather_max_rows=8, chunk=4,
                          interpret=True, tm=16, combine="gather")
    assert f.rows == {"gate_q": 256, "up_q": 256, "down_q": 6144}
    assert f.nblk == {"gate_q": 24, "up_q": 24, "down_q": 1}
    assert (f.gather_max_rows, f.chunk, f.interpret, f.tm, f.combine) == (8, 4, True, 16, "gather")
    assert pkg.resident._is_f32(f.out_dtype) and not pkg.resident._is_f32(torch.bfloat16)
    assert pkg.resident._is_f32("float32")


def test_bad_modes_rejected(pkg):
    with pytest.raises(ValueError):
        pkg.ResidentFetch({}, 256, 256, sweep_mode="masked")
    with pytest.raises(ValueError):
        pkg.ResidentFetch({}, 256, 256, combine="scatter")
