"""GPU parity of the router (mi_moe_route, the reference's moe_route, model.py:798-808) against the CPU oracle.

Bar: the expert ids equal the oracle's wherever the oracle's choice values are separated by more than the f32
rounding of the logits (1e-5); where two choices lie closer, the selected choice values must agree within that
margin instead (f32 dot products against the oracle's f64).  Weights within rel 1e-5.  Equal choices (exact ties)
must come out lower id first, as lax.top_k orders them.
"""
import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.bf16 import round_bf16

pytestmark = pytest.mark.gpu
MARGIN = 1e-5


def _check(idx, w, x, rw, bias, k, norm, scaling):
    oi, ow, choice = omoe.route(x, rw, bias, k, norm, scaling)
    srt = -np.sort(-choice, axis=-1)
    for n in range(x.shape[0]):
        gaps = np.abs(np.diff(srt[n, :k + 1])) if k < choice.shape[1] else np.abs(np.diff(srt[n, :k]))
        if gaps.size == 0 or gaps.min() > MARGIN:
            assert idx[n].tolist() == oi[n].tolist(), n
            np.testing.assert_allclose(w[n], ow[n], rtol=1e-5, atol=1e-7)
        else:
            np.testing.assert_allclose(np.sort(choice[n, idx[n]]), np.sort(choice[n, oi[n]]), atol=MARGIN)
    assert (idx >= 0).all() and (idx < rw.shape[1]).all()
    assert all(len(set(r)) == k for r in idx.tolist())           # k distinct experts per token


@pytest.mark.parametrize("N,D,E,k", [(1, 6144, 64, 8), (8, 6144, 64, 8), (16, 6144, 256, 8), (512, 6144, 64, 8),
                                     (37, 258, 100, 5), (3, 512, 1024, 32), (5, 1000, 64, 1), (2, 64, 8, 8)])
@pytest.mark.parametrize("norm", [True, False])
def test_route(pkg, gpu, N, D, E, k, norm):
    rng = np.random.default_rng(N * 131 + E + k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    rw = (rng.standard_normal((D, E)) / np.sqrt(D)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    idx, w = pkg.route(torch.from_numpy(x).cuda().to(torch.bfloat16), torch.from_numpy(rw).cuda(),
                       torch.from_numpy(bias).cuda(), k, norm, 2.5)
    _check(idx.cpu().numpy(), w.cpu().numpy(), x, rw, bias, k, norm, 2.5)


def test_route_ties_and_bias(pkg, gpu):
    """All logits 0: every score 0.5; equal bias -> ids 0..k-1; a bias on chosen ids moves the selection only."""
    N, D, E, k = 3, 256, 64, 4
    x = torch.zeros((N, D), dtype=torch.bfloat16, device="cuda")
    rw = torch.zeros((D, E), dtype=torch.float32, device="cuda")
    idx, w = pkg.route(x, rw, None, k, True, 1.0)
    assert idx.cpu().tolist() == [[0, 1, 2, 3]] * N
    assert torch.allclose(w.cpu(), torch.full((N, k), 0.25))
    bias = torch.zeros(E, dtype=torch.float32)
    bias[[63, 5, 40, 17]] = torch.tensor([4.0, 3.0, 2.0, 1.0])
    idx, w = pkg.route(x, rw, bias.cuda(), k, False, 2.0)
    assert idx.cpu().tolist() == [[63, 5, 40, 17]] * N
    assert torch.equal(w.cpu(), torch.full((N, k), 1.0))


def test_moe_route_signature(pkg, gpu):
    """The reference's call form moe_route(p, x, cfg) (model.py:798, 843) and a second call reusing the outputs'
    device: deterministic, bit-identical."""
    class Cfg:
        topk, norm_topk, scaling = 8, True, 2.5
    rng = np.random.default_rng(4)
    D, E = 6144, 64
    p = {"router_w": torch.from_numpy((rng.standard_normal((D, E)) / np.sqrt(D)).astype(np.float32)).cuda(),
         "router_bias": torch.from_numpy((rng.standard_normal(E) * 0.05).astype(np.float32)).cuda()}
    x = torch.from_numpy(round_bf16(rng.standard_normal((4, D)).astype(np.float32))).cuda().to(torch.bfloat16)
    i1, w1 = pkg.moe_route(p, x, Cfg)
    i2, w2 = pkg.moe_route(p, x, Cfg)
    assert torch.equal(i1, i2) and torch.equal(w1, w2)
    _check(i1.cpu().numpy(), w1.cpu().numpy(), x.float().cpu().numpy(), p["router_w"].cpu().numpy(),
           p["router_bias"].cpu().numpy(), 8, True, 2.5)
