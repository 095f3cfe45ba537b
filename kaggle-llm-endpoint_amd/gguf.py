"""GGUF reading for the resident expert tables: the reference's reader interface (gguf_reader.py:78-165) over
positional reads (os.pread: no mmap, no page-cache pressure), on whole .gguf files or on byte-range pieces listed in
a manifest.json (the reference's 4 GB mirror pieces), plus the layer loader (resident.py:29-46) that turns one
layer's expert tensors into device ExpertTables through the on-device planar packer (mi_pack_planes).

GGUF layout (the published format, version 2 and 3): magic "GGUF", u32 version, u64 tensor count, u64 key/value
count; key/value pairs (u64-length string key, u32 value type, value); tensor infos (name, u32 n_dims, u64 dims,
u32 ggml type, u64 offset from the data section); the data section starts at the next multiple of
general.alignment (default 32).  Expert tensors blk.{L}.ffn_{gate,up,down}_exps.weight have dims
[ne0 = inputs, ne1 = rows, ne2 = experts]: numpy order (E, rows, inputs), quant blocks along the inputs.
"""
import json
import os
import struct
from concurrent.futures import ThreadPoolExecutor

# ggml type id -> (name, weights per block, bytes per block)
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2),
}
GGML_IDS = {name: tid for tid, (name, _, _) in GGML_TYPES.items()}

# value type id -> struct format of a scalar (8: string, 9: array are handled separately)
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_ARRAY_KEEP = 64          # arrays longer than this (tokenizer vocabularies) are skipped, as the reference does


class PiecewiseFile:
    """One logical file over one real file or over ordered (path, start, length) byte-range pieces."""

    def __init__(self, pieces):
        self.pieces = sorted(pieces, key=lambda p: p[1])
        pos = 0
        for path, start, length in self.pieces:
            if start != pos:
                raise ValueError("pieces leave a gap or overlap at byte %d (%s starts at %d)" % (pos, path, start))
            pos += length
        self.size = pos
        self._fds = {}

    @classmethod
    def single(cls, path):
        return cls([(path, 0, os.path.getsize(path))])

    def _fd(self, path):
        fd = self._fds.get(path)
        if fd is None:
            fd = self._fds[path] = os.open(path, os.O_RDONLY)
        return fd

    def pread(self, offset, length):
        if offset < 0 or length < 0 or offset + length > self.size:
            raise ValueError("read [%d, %d) outside the file's %d bytes" % (offset, offset + length, self.size))
        out = bytearray(length)
        mv = memoryview(out)
        for path, start, plen in self.pieces:
            lo, hi = max(offset, start), min(offset + length, start + plen)
            if hi <= lo:
                continue
            got, want, pos = 0, hi - lo, lo
            while got < want:                                  # pread may return short counts
                chunk = os.pread(self._fd(path), want - got, pos - start)
                if not chunk:
                    raise IOError("short read in %s at %d" % (path, pos - start))
                mv[pos - offset:pos - offset + len(chunk)] = chunk
                got += len(chunk)
                pos += len(chunk)
        return out

    def close(self):
        for fd in self._fds.values():
            os.close(fd)
        self._fds.clear()


def open_mirror(dirs):
    """dirs containing .gguf files and/or a manifest.json of byte-range pieces -> {file name: PiecewiseFile}."""
    files = {}
    for d in dirs:
        man = os.path.join(d, "manifest.json")
        if os.path.exists(man):
            with open(man) as f:
                m = json.load(f)
            for name, info in m["files"].items():
                files[name] = PiecewiseFile([(os.path.join(d, p["name"]), p["start"], p["length"])
                                             for p in info["pieces"]])
        for fn in sorted(os.listdir(d)):
            if fn.endswith(".gguf"):
                files[fn] = PiecewiseFile.single(os.path.join(d, fn))
    return files


class _Cursor:
    """Sequential little-endian reads over a PiecewiseFile, fetched in growing windows."""

    def __init__(self, pf, window=1 << 20):
        self.pf, self.pos, self.base, self.buf, self.window = pf, 0, 0, b"", window

    def take(self, n):
        if self.pos + n > self.base + len(self.buf):
            want = max(n, self.window)
            self.base = self.pos
            self.buf = bytes(self.pf.pread(self.pos, min(want, self.pf.size - self.pos)))
            if len(self.buf) < n:
                raise ValueError("GGUF header runs past the end of the file")
        off = self.pos - self.base
        self.pos += n
        return self.buf[off:off + n]

    def scalar(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        return self.take(self.scalar("<Q")).decode("utf-8", errors="replace")

    def value(self, vt):
        if vt in _SCALARS:
            return self.scalar(_SCALARS[vt])
        if vt == 8:
            return self.string()
        if vt == 9:
            et, n = self.scalar("<I"), self.scalar("<Q")
            return [self.value(et) for _ in range(n)]
        raise ValueError("unknown GGUF value type %d" % vt)


class GGUFShard:
    """One GGUF file: kv (metadata), tensors ({name: {"dims", "type", "offset", "nbytes"}}), data0 (data section)."""

    def __init__(self, pf):
        self.pf = pf
        c = _Cursor(pf)
        if c.take(4) != b"GGUF":
            raise ValueError("not a GGUF file")
        version = c.scalar("<I")
        if version not in (2, 3):
            raise ValueError("GGUF version %d is not supported (2 and 3 are)" % version)
        n_tensors, n_kv = c.scalar("<Q"), c.scalar("<Q")
        self.kv = {}
        for _ in range(n_kv):
            key, vt = c.string(), c.scalar("<I")
            v = c.value(vt)
            if not (isinstance(v, list) and len(v) > _ARRAY_KEEP):
                self.kv[key] = v
        align = int(self.kv.get("general.alignment", 32))
        self.tensors = {}
        for _ in range(n_tensors):
            name = c.string()
            dims = [c.scalar("<Q") for _ in range(c.scalar("<I"))]
            tid, off = c.scalar("<I"), c.scalar("<Q")
            if tid not in GGML_TYPES:
                raise ValueError("tensor %s: unknown ggml type %d" % (name, tid))
            tname, bs, tb = GGML_TYPES[tid]
            n = 1
            for d in dims:
                n *= d
            if n % bs:
                raise ValueError("tensor %s: %d values are not whole %s blocks" % (name, n, tname))
            self.tensors[name] = {"dims": dims, "type": tname, "offset": off, "nbytes": n // bs * tb}
        self.data0 = (c.pos + align - 1) // align * align
        for name, t in self.tensors.items():
            if self.data0 + t["offset"] + t["nbytes"] > pf.size:
                raise ValueError("tensor %s runs past the end of the file" % name)

    def read_tensor(self, name, offset=0, length=None):
        t = self.tensors[name]
        length = t["nbytes"] - offset if length is None else length
        if offset < 0 or offset + length > t["nbytes"]:
            raise ValueError("read outside tensor %s" % name)
        return self.pf.pread(self.data0 + t["offset"] + offset, length)


class GGUFModel:
    """Every shard of a split GGUF behind one tensor map (the reference's GGUFModel interface)."""

    def __init__(self, files):
        self.shards = {n: GGUFShard(pf) for n, pf in sorted(files.items())}
        self.where, self.kv = {}, {}
        for n, s in self.shards.items():
            self.kv.update(s.kv)
            for t in s.tensors:
                self.where[t] = n

    def info(self, name):
        return self.shards[self.where[name]].tensors[name]

    def read(self, name, offset=0, length=None):
        return self.shards[self.where[name]].read_tensor(name, offset, length)

    def expert_bytes(self, name):
        """Bytes of one expert of a [in, out, E] tensor."""
        t = self.info(name)
        return t["nbytes"] // t["dims"][2]

    def read_expert(self, name, e):
        n = self.expert_bytes(name)
        return self.read(name, e * n, n)

    def read_experts(self, name, es, threads=8):
        with ThreadPoolExecutor(max(1, threads)) as pool:
            return list(pool.map(lambda e: self.read_expert(name, e), es))


def load_layer(gm, layer, threads=8, device="cuda"):
    """One layer's routed experts -> ({"gate_q" | "up_q" | "down_q": ExpertTable}, {key: qtype}) for one GPU
    (resident.py:29-46 with one chip): the raw GGUF blocks are read, copied to the device once, and split into the
    reference's planar tables there (mi_pack_planes); Q2_K / Q3_K tensors (the MTP layer's experts, whose Q3_K scales
    are unpacked) are split on the host (formats.kq_pack_planes)."""
    import numpy as np
    import torch

    from . import formats
    from .resident import ExpertTable, pack_planes_device, to_device_planes

    tables, qtypes = {}, {}
    for key, tname in (("gate_q", "gate"), ("up_q", "up"), ("down_q", "down")):
        name = "blk.%d.ffn_%s_exps.weight" % (layer, tname)
        info = gm.info(name)
        ne0, ne1, E = info["dims"]
        qt = info["type"]
        raws = gm.read_experts(name, range(E), threads=threads)
        flat = np.frombuffer(b"".join(bytes(r) for r in raws), np.uint8)
        if qt in formats.KQ_BLOCK_BYTES:
            blk = flat.reshape(E, ne1, ne0 // 256, formats.KQ_BLOCK_BYTES[qt])
            planes = to_device_planes(formats.kq_pack_planes(blk, qt), device)
        else:
            planes = pack_planes_device(torch.from_numpy(flat.copy()).to(device), qt, E, ne1, ne0)
        tables[key] = ExpertTable(qt, planes, ne1, ne0)
        qtypes[key] = qt
    return tables, qtypes
