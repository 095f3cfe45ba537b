"""The streaming-read probe (mi_read_probe, measurement only) reads every byte it is given: the XOR of the words it
writes equals the XOR of the source's words, for sizes that leave partial grid strides."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n16,wg", [(1, 1), (4096, 4), (1 << 16, 64), (1000003, 1024)])
def test_read_probe_reads_everything(pkg, gpu, n16, wg):
    rng = np.random.default_rng(n16)
    data = rng.integers(0, 1 << 32, 4 * n16, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(data.view(np.int32)).cuda()
    sink = torch.zeros(wg * 4, dtype=torch.int32, device="cuda")
    R, P = pkg.resident, pkg._lib
    P.check("mi_read_probe", P.probe_lib().mi_read_probe(R._ptr(src), 16 * n16, R._ptr(sink), wg, R._stream()))
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert int(got) == int(np.bitwise_xor.reduce(data))
