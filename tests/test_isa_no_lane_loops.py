"""CPU: no kernel of the library builds a buffer descriptor from a per-lane pointer.  Such a descriptor makes the
compiler loop over the lanes' distinct values (read the first lane's value, compare it with every lane's, run the
instruction for the lanes that match, repeat); besides costing a pass per distinct value, one such loop was seen
reusing its address registers for a spilled operand and writing out of bounds.  Every source is compiled to gfx950
assembly with the build's flags (one instantiation unit per k_*.hip), and the loop's signature -- a 64-bit compare of scalar
registers (the read-first-lane value) with vector registers -- must not appear."""
import os
import re
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest


def _build_module():
    import importlib.util
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("_mi355moe_build_isa",
                                                  os.path.join(repo, "kaggle-llm-endpoint_amd", "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    return b

SIGNATURE = re.compile(r"v_cmp_eq_u64_e(32|64) (vcc|s\[\d+:\d+\]), s\[\d+:\d+\], v\[\d+:\d+\]")


@pytest.mark.skipif(shutil.which(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")) is None, reason="no hipcc")
def test_no_per_lane_descriptor_loops():
    build = _build_module()
    # every source once: the first instantiation unit of each k_*.hip (the others compile the same code with other
    # template arguments), every other unit as it is
    seen, units = set(), []
    for u in build.UNITS + [build.PROBE_UNIT]:
        if u[0].startswith("k_") and u[0] in seen:
            continue
        seen.add(u[0])
        units.append(u)
    with tempfile.TemporaryDirectory() as tmp:
        def asm(u):
            src, defs, name = u
            out = os.path.join(tmp, name + ".s")
            cmd = [build.HIPCC] + build.FLAGS + defs + ["-I", build.INCLUDE, "--cuda-device-only", "-S",
                                                        os.path.join(build.CSRC, src), "-o", out]
            res = subprocess.run(cmd, capture_output=True, text=True)
            assert res.returncode == 0, (name, res.stderr[-2000:])
            with open(out) as f:
                return name, [l.strip() for l in f if SIGNATURE.search(l)]
        with ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
            found = {name: hits for name, hits in ex.map(asm, units) if hits}
    assert not found, found
