"""mi_moe_decode_noalloc (the decode layer with its partials and h in the library's static scratch array, no workspace
argument) against mi_moe_decode through the C ABI: identical outputs on two calls in a row, the second with fewer
tokens, at a small shape (also against the f64 oracle, rel-L2 <= 1e-5 as the decode's own tests) and at the
benchmark layer's shape; a layer whose data region exceeds the scratch array is rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.util import Layer, zipf_routing

pytestmark = pytest.mark.gpu


def _noalloc(pkg, tbs, x, idx, w, shared, limit, out_f32, out_bf16):
    L = pkg._lib.lib()
    N, k = idx.shape
    st = L.mi_moe_decode_noalloc(tbs["gate"].c, tbs["up"].c, tbs["down"].c, ctypes.c_void_p(x.data_ptr()), N, k,
                                 ctypes.c_void_p(idx.data_ptr()), ctypes.c_void_p(w.data_ptr()), shared, limit,
                                 ctypes.c_void_p(out_f32.data_ptr()), ctypes.c_void_p(out_bf16.data_ptr()),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    pkg._lib.check("mi_moe_decode_noalloc", st)


def _both(pkg, tbs, x, idx, w, shared, limit):
    N, D = x.shape[0], tbs["down"].rows
    of = torch.full((N, D), float("nan"), dtype=torch.float32, device="cuda")
    ob = torch.zeros((N, D), dtype=torch.bfloat16, device="cuda")
    _noalloc(pkg, tbs, x, idx, w, shared, limit, of, ob)
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, idx.shape[1], shared),
                     dtype=torch.uint8, device="cuda")
    rf, rb = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, idx, w, limit, shared_expert=shared,
                            want_bf16=True, workspace=ws)
    torch.cuda.synchronize()
    return of, ob, rf, rb


def test_noalloc_matches_decode_small(pkg, gpu):
    rng = np.random.default_rng(4242)
    E, D, I, limit = 10, 1280, 512, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    for N, k in ((8, 6), (3, 4)):                       # the second call is smaller
        idx, w = zipf_routing(rng, N, E, k)
        x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
        xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
        it, wt = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
        of, ob, rf, rb = _both(pkg, tbs, xt, it, wt, E, limit)
        assert torch.equal(of, rf) and torch.equal(ob, rb)
        want = omoe.decode_apply(L.deq, x, idx, w, limit) + omoe.shared_apply(lambda m: L.deq(m, E), x, limit)
        assert rel_l2(of.cpu().numpy(), want) < 1e-5


def test_noalloc_matches_decode_full_shape(pkg, gpu):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    E, D, I, k, limit = 65, 6144, 2048, 8, 10.0
    tbs = {name: pkg.random_cb3_table(E, R, K, gen) for name, (R, K) in
           (("gate", (I, D)), ("up", (I, D)), ("down", (D, I)))}
    rng = np.random.default_rng(9)
    for N in (16, 1):
        idx, w = zipf_routing(rng, N, E - 1, k)
        x = torch.randn((N, D), device="cuda", generator=gen).to(torch.bfloat16)
        of, ob, rf, rb = _both(pkg, tbs, x, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), E - 1, limit)
        assert torch.isfinite(of).all()
        assert torch.equal(of, rf) and torch.equal(ob, rb)
