"""The tiled int8 weight layout (mi_int8_tile): the repack equals its definition, and every int8 entry point gives
bit-identical outputs with tiled weights (the kernels' arithmetic is the same; only the weights' addresses
differ)."""
import numpy as np
import pytest
import torch

from oracle import int8 as oi8
from oracle.bf16 import rel_l2, round_bf16

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int32 if t.dtype == torch.float32 else torch.int16).cpu().numpy()


@pytest.mark.parametrize("n_out,n_in", [(16, 256), (48, 512), (2048, 6144)])
def test_int8_tile_layout(pkg, gpu, n_out, n_in):
    """tiled[b, t, h * 1024 + l * 16 + j] = qT[16 t + l % 16, 128 b + 32 (l // 16) + 16 h + j]."""
    rng = np.random.default_rng(n_out + n_in)
    qT = rng.integers(-128, 128, (n_out, n_in), dtype=np.int8)
    got = pkg.int8_tile(torch.from_numpy(qT).cuda()).cpu().numpy()
    assert got.shape == (n_in // 128, n_out // 16, 2048)
    t, i, b, q, h, j = np.meshgrid(np.arange(n_out // 16), np.arange(16), np.arange(n_in // 128), np.arange(4),
                                   np.arange(2), np.arange(16), indexing="ij")
    want = np.zeros_like(got)
    want[b, t, h * 1024 + (i + 16 * q) * 16 + j] = qT[16 * t + i, 128 * b + 32 * q + 16 * h + j]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("B,n_in,n_out,axis", [(8, 6144, 6144, 1), (1, 256, 16, 1), (20, 1024, 512, 1),
                                               (8, 2048, 6144, 0), (3, 6144, 2048, 2), (32, 512, 512, 0)])
def test_int8_project_tiled_identical(pkg, gpu, B, n_in, n_out, axis):
    rng = np.random.default_rng(B + n_in + n_out + axis)
    q, s = oi8.generate(rng, n_in, n_out)
    if axis == 0:
        s = (rng.random((n_in, 1)) * 1.5e-3 + 0.5e-3).astype(np.float32)
    qT, sv, _ = pkg.formats.int8_pack(q, s)
    x = torch.from_numpy(round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))).cuda().to(torch.bfloat16)
    qd, sd = torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda()
    rows = pkg.int8_project(x, qd, sd, want_f32=True, scale_axis=axis)
    tiled = pkg.int8_project(x, pkg.int8_tile(qd), sd, want_f32=True, scale_axis=axis)
    assert np.array_equal(_bits(rows[0]), _bits(tiled[0]))
    assert np.array_equal(_bits(rows[1]), _bits(tiled[1]))
    if axis == 1:
        assert rel_l2(tiled[1].cpu().numpy(), oi8.project_f32(x.float().cpu().numpy(), q, s)) < 1e-5


def test_int8_many_and_mlp_tiled_identical(pkg, gpu):
    rng = np.random.default_rng(77)
    B, D, I = 8, 1024, 512
    x = torch.from_numpy(round_bf16(rng.standard_normal((B, D)).astype(np.float32))).cuda().to(torch.bfloat16)
    projs = []
    for n in (512, 256, 768):
        q, s = oi8.generate(rng, D, n)
        qT, sv, _ = pkg.formats.int8_pack(q, s)
        projs.append((torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda()))
    rows = pkg.int8_project_many(x, projs, want_f32=True)
    tiled = pkg.int8_project_many(x, [(pkg.int8_tile(qT), sv) for qT, sv in projs], want_f32=True)
    for a, b in zip(rows, tiled):
        assert np.array_equal(_bits(a[1]), _bits(b[1]))
    leaves = []
    for n_in, n_out, col in ((D, I, True), (D, I, True), (I, D, False)):
        q, s = oi8.generate(rng, n_in, n_out)
        if not col:
            s = (rng.random((n_in, 1)) * 1.5e-3 + 0.5e-3).astype(np.float32)
        qT, sv, ax = pkg.formats.int8_pack(q, s)
        leaves.append((torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda(), ax))
    y_rows = pkg.int8_mlp(x, *leaves, 7.0, want_f32=True)
    y_tiled = pkg.int8_mlp(x, *[(pkg.int8_tile(qT), sv, ax) for qT, sv, ax in leaves], 7.0, want_f32=True)
    assert np.array_equal(_bits(y_rows[0]), _bits(y_tiled[0]))
    assert np.array_equal(_bits(y_rows[1]), _bits(y_tiled[1]))
