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


def _loops(asm_text):
    """(kernel, loop body lines) of every loop (a backward branch) in every kernel of an assembly file."""
    out = []
    for m in re.finditer(r"^(_ZN2mi\S+):", asm_text, re.M):
        name = m.group(1)
        end = asm_text.find(".Lfunc_end", m.end())
        body = [l.strip() for l in asm_text[m.end():end].split("\n")]
        body = [l for l in body if l and not l.startswith(";")]
        pos = {}
        for i, l in enumerate(body):
            lm = re.match(r"^(\.LBB\d+_\d+):", l)
            if lm:
                pos[lm.group(1)] = i
        for i, l in enumerate(body):
            bm = re.match(r"^s_c?branch\S*\s+(\.LBB\d+_\d+)", l)
            if bm and bm.group(1) in pos and pos[bm.group(1)] < i:
                out.append((name, body[pos[bm.group(1)]:i + 1]))
    return out


# decode launches whose weight loops keep their prefetched loads in flight: (source, defines, kernel name part)
STREAMING = [
    ("k_custream.hip", ["-DMI_CMODE=0"], "custream_kernel"),
    ("k_custream.hip", ["-DMI_CMODE=1"], "custream_kernel"),
    ("k_cumulti.hip", ["-DMI_UMODE=0"], "cumulti_kernel"),
    ("k_cumulti.hip", ["-DMI_UMODE=1"], "cumulti_kernel"),
    ("k_grouped.hip", ["-DMI_KMODE=0", "-DMI_KQT=2"], "grouped_kernel"),   # IQ3_S
    ("k_grouped.hip", ["-DMI_KMODE=1", "-DMI_KQT=2"], "grouped_kernel"),
    ("k_grouped.hip", ["-DMI_KMODE=0", "-DMI_KQT=4"], "grouped_kernel"),   # IQ2_S
    ("k_grouped.hip", ["-DMI_KMODE=0", "-DMI_KQT=3"], "grouped_kernel"),   # IQ4_XS (register ring)
]


@pytest.mark.skipif(shutil.which(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")) is None, reason="no hipcc")
def test_weight_loops_never_wait_for_every_load():
    """CPU: inside the decode launches' weight loops (a loop with matrix-core work and vector memory loads, and no
    workgroup barrier) no instruction waits for every vector memory load in flight (s_waitcnt vmcnt(0)): that would
    drain the loads prefetched for the next tiles.  Loads under a branch make the compiler emit exactly that where the
    branch rejoins, so the loops load branch-free (empty-range buffer descriptors past a split's end).  Left out: the
    IQ4_XS down launch at one token (its ring is loaded by instructions the compiler does not count) and the
    single-token down launch with 4 row tiles per unit (a tuning option, not a default: at its 128-register bound it
    spills, and waits for the spill reloads)."""
    build = _build_module()
    with tempfile.TemporaryDirectory() as tmp:
        def check(k):
            src, defs, part = STREAMING[k]
            out = os.path.join(tmp, "u%d.s" % k)
            cmd = [build.HIPCC] + build.FLAGS + defs + ["-I", build.INCLUDE, "--cuda-device-only", "-S",
                                                        os.path.join(build.CSRC, src), "-o", out]
            res = subprocess.run(cmd, capture_output=True, text=True)
            assert res.returncode == 0, (src, defs, res.stderr[-2000:])
            with open(out) as f:
                text = f.read()
            bad = []
            for name, body in _loops(text):
                if part not in name:
                    continue
                if "_ZN2mi14grouped_kernelILi1ELi3ELi1E" in name:     # IQ4_XS down at one token (LDS ring)
                    continue
                if "_ZN2mi15custream_kernelILi1ELi4E" in name:        # 4 row tiles in the down launch (not a
                    continue                                          # default): spills at 128 registers
                if not any(l.startswith("v_mfma") for l in body):
                    continue
                if not any(l.startswith(("global_load", "buffer_load")) for l in body):
                    continue
                if any(l.startswith("s_barrier") for l in body):
                    continue
                waits = [l for l in body if l.startswith("s_waitcnt") and "vmcnt(0)" in l]
                if waits:
                    bad.append((name[:80], len(body), len(waits)))
            return src, defs, bad
        with ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
            found = [(s, d, b) for s, d, b in ex.map(check, range(len(STREAMING))) if b]
    assert not found, found
