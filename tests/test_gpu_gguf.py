"""GPU: the on-device planar packer (mi_pack_planes) equals the host packer (formats.*_pack_planes, itself pinned
against the oracle's restatement of planes.pack_planes) bit for bit, and a layer read from a GGUF file and packed on
the device decodes to the oracle's result (the reference's load path, resident.py:29-60, then apply)."""
import numpy as np
import pytest
import torch

from oracle import iq2s, iq3s, iq4xs, kquant, moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.gguf_write import expert_tensor, write_gguf
from tests.util import zipf_routing

pytestmark = pytest.mark.gpu
BB = {"IQ2_S": 82, "IQ3_S": 110, "IQ4_XS": 136, "Q2_K": 84, "Q3_K": 110}
ORACLE = {"IQ2_S": iq2s, "IQ3_S": iq3s, "IQ4_XS": iq4xs}


@pytest.mark.parametrize("qtype", ["IQ2_S", "IQ3_S", "IQ4_XS"])
@pytest.mark.parametrize("E,R,K", [(3, 80, 768), (2, 64, 1024), (1, 200, 256), (4, 128, 2560)])
def test_pack_planes_device(pkg, gpu, qtype, E, R, K):
    rng = np.random.default_rng(E * 7 + R + K)
    raw, _ = expert_tensor(rng, qtype, E, R, K, BB[qtype])
    got = pkg.pack_planes_device(torch.from_numpy(raw.reshape(-1)).cuda(), qtype, E, R, K)
    want = ORACLE[qtype].pack_planes(raw)
    for k in ORACLE[qtype].PLANE_KEYS:
        g = got[k].cpu().numpy().view(np.uint32)
        assert g.shape == want[k].shape, k
        assert np.array_equal(g, want[k]), k


@pytest.mark.parametrize("gu,dn", [("IQ2_S", "IQ4_XS"), ("Q2_K", "Q3_K")])
def test_load_layer_from_gguf_and_decode(pkg, gpu, tmp_path, gu, dn):
    """A layer written to a GGUF file (the real GGUF's IQ2_S/IQ4_XS mix; a K-quant MTP-style layer), read, packed
    and run through the decode against the oracle."""
    rng = np.random.default_rng(12)
    E, D, I, N, k, limit = 6, 512, 256, 4, 3, 10.0
    fmts = {"gate": gu, "up": gu, "down": dn}
    raws, tensors = {}, []
    for name, (R, K) in (("gate", (I, D)), ("up", (I, D)), ("down", (D, I))):
        raws[name], dims = expert_tensor(rng, fmts[name], E, R, K, BB[fmts[name]])
        tensors.append(("blk.5.ffn_%s_exps.weight" % name, dims, fmts[name], raws[name].tobytes()))
    write_gguf(tmp_path / "layer.gguf", {"general.architecture": "glm5next"}, tensors)
    gm = pkg.gguf.GGUFModel(pkg.gguf.open_mirror([str(tmp_path)]))
    tables, qtypes = pkg.gguf.load_layer(gm, 5, threads=2)
    assert qtypes == {"gate_q": gu, "up_q": gu, "down_q": dn}

    def deq(name, e):
        R, K = (D, I) if name == "down" else (I, D)
        qt = fmts[name]
        if qt in ("Q2_K", "Q3_K"):
            return kquant.dequant_blocks(raws[name][e], qt).reshape(R, K)
        return ORACLE[qt].dequant_blocks(raws[name][e]).reshape(R, K)

    idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    of, _ = pkg.moe_decode(tables["gate_q"], tables["up_q"], tables["down_q"], xt, torch.from_numpy(idx).cuda(),
                           torch.from_numpy(w).cuda(), limit)
    assert rel_l2(of.cpu().numpy(), omoe.decode_apply(deq, x, idx, w, limit)) < 1e-5
