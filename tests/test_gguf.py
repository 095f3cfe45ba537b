"""CPU: the GGUF reader (the reference's gguf_reader interface, gguf_reader.py:78-165) on whole files and on
byte-range pieces with a manifest, as the reference's own test does (T/test_gguf_reader.py:21-47), plus its error
handling.  Files are written by tests/gguf_write.py from the published format."""
import json

import numpy as np
import pytest

from tests.gguf_write import expert_tensor, write_gguf


def _model(tmp_path, alignment=32):
    rng = np.random.default_rng(0)
    raw, dims = expert_tensor(rng, "IQ2_S", 4, 8, 512, 82)
    small = np.arange(64, dtype=np.float32).reshape(8, 8)
    kv = {"general.architecture": "glm5next", "glm5next.expert_count": 4, "glm5next.rope_theta": 1.5,
          "tokenizer.ggml.token_type": list(range(100)), "short.list": [1, 2, 3]}
    write_gguf(tmp_path / "m.gguf", kv, [("blk.3.ffn_gate_exps.weight", dims, "IQ2_S", raw.tobytes()),
                                         ("blk.0.attn_norm.weight", [8, 8], "F32", small.tobytes())], alignment)
    return raw, small


def _pieces(tmp_path, size=1000):
    data = (tmp_path / "m.gguf").read_bytes()
    pd = tmp_path / "pieces"
    pd.mkdir()
    pieces = []
    for i, s in enumerate(range(0, len(data), size)):
        (pd / ("m.gguf.p%02d" % i)).write_bytes(data[s:s + size])
        pieces.append({"name": "m.gguf.p%02d" % i, "start": s, "length": len(data[s:s + size])})
    (pd / "manifest.json").write_text(json.dumps({"files": {"m.gguf": {"size": len(data), "pieces": pieces}}}))
    return pd


@pytest.mark.parametrize("alignment", [32, 64])
def test_single_file_and_pieces(tmp_path, pkg, alignment):
    raw, small = _model(tmp_path, alignment)
    pd = _pieces(tmp_path)
    g = pkg.gguf
    for files in (g.open_mirror([str(tmp_path)]), g.open_mirror([str(pd)])):
        m = g.GGUFModel(files)
        assert m.kv["glm5next.expert_count"] == 4 and m.kv["general.architecture"] == "glm5next"
        assert m.kv["glm5next.rope_theta"] == 1.5 and m.kv["short.list"] == [1, 2, 3]
        assert "tokenizer.ggml.token_type" not in m.kv                  # long arrays are skipped
        t = m.info("blk.3.ffn_gate_exps.weight")
        assert t["type"] == "IQ2_S" and t["dims"] == [512, 8, 4]
        assert m.expert_bytes("blk.3.ffn_gate_exps.weight") == 8 * 2 * 82
        for e in range(4):
            got = np.frombuffer(m.read_expert("blk.3.ffn_gate_exps.weight", e), np.uint8)
            assert np.array_equal(got, raw[e].reshape(-1))
        got = m.read_experts("blk.3.ffn_gate_exps.weight", [3, 1], threads=2)
        assert np.array_equal(np.frombuffer(got[0], np.uint8), raw[3].reshape(-1))
        assert np.array_equal(np.frombuffer(got[1], np.uint8), raw[1].reshape(-1))
        sm = np.frombuffer(m.read("blk.0.attn_norm.weight"), np.float32).reshape(8, 8)
        assert np.array_equal(sm, small)
        # read blocks -> the reference's planes, host packer and oracle agree
        from oracle import iq2s
        blk = np.frombuffer(m.read_expert("blk.3.ffn_gate_exps.weight", 2), np.uint8).reshape(1, 8, 2, 82)
        a, b = pkg.formats.iq2s_pack_planes(blk), iq2s.pack_planes(blk)
        assert all(np.array_equal(a[k], b[k]) for k in iq2s.PLANE_KEYS)


def test_reader_errors(tmp_path, pkg):
    g = pkg.gguf
    _model(tmp_path)
    data = (tmp_path / "m.gguf").read_bytes()
    (tmp_path / "bad.bin").write_bytes(b"GGUX" + data[4:])
    with pytest.raises(ValueError, match="not a GGUF"):
        g.GGUFShard(g.PiecewiseFile.single(str(tmp_path / "bad.bin")))
    (tmp_path / "cut.bin").write_bytes(data[:len(data) - 600])
    with pytest.raises(ValueError, match="past the end"):
        g.GGUFShard(g.PiecewiseFile.single(str(tmp_path / "cut.bin")))
    with pytest.raises(ValueError, match="gap"):
        g.PiecewiseFile([(str(tmp_path / "m.gguf"), 0, 100), (str(tmp_path / "m.gguf"), 200, 100)])
    m = g.GGUFModel({"m.gguf": g.PiecewiseFile.single(str(tmp_path / "m.gguf"))})
    with pytest.raises(ValueError, match="outside tensor"):
        m.read("blk.0.attn_norm.weight", 200, 100)
