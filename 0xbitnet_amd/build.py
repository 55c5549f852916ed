"""Build liboxbitnet.so (HIP for gfx950 + host C++) in-tree with hipcc.

    python 0xbitnet_amd/build.py [--force] [-j N]

Objects go to 0xbitnet_amd/_build/, the library to 0xbitnet_amd/liboxbitnet.so
(rpath /opt/rocm/lib so the process uses the system ROCm runtime).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liboxbitnet.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    # every f32 op separately rounded (the oracle's convention); IEEE div/sqrt
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-I", os.path.join(HERE, "..", "include"),
]
# Device code: gfx950 only; packed-fp32 instructions are disabled.
DEVICE = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _check_resources(src: str, stderr: str) -> str:
    """Parse the compiler's kernel-resource-usage remarks for one source.

    Every kernel must run without a private segment: no scratch bytes per lane,
    no VGPR spills and no dynamic stack (a spill to scratch turns register
    traffic into memory traffic on the hot path).  SGPR spills land in VGPR
    lanes and are allowed.  Returns the remarks, one kernel per line, and raises
    when a kernel breaks the rule.
    """
    rows, bad, name = [], [], None
    for line in stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            rows.append([name])
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?(?: \[[^]]+\])?): (\S+) \[-Rpass", line)
        if m and name is not None:
            key, val = m.group(1), m.group(2)
            rows[-1].append(f"{key}={val}")
            if key.startswith(("ScratchSize", "VGPRs Spill", "Dynamic Stack")) and val not in ("0", "False"):
                bad.append(f"{name}: {key} = {val}")
    if bad:
        raise RuntimeError(f"{os.path.basename(src)}: kernels use scratch memory:\n  " + "\n  ".join(bad))
    return "\n".join(" ".join(r) for r in rows) + "\n"


def _diagnostics(stderr: str) -> list[str]:
    """Compiler output minus the resource remarks (and their source excerpts) and
    the host pass's note that it does not know the packed-fp32 feature."""
    keep, in_remark = [], False
    for line in stderr.splitlines():
        if "kernel-resource-usage" in line:
            in_remark = True
            continue
        if in_remark and re.match(r"^\s*\d*\s*\|", line):
            continue
        in_remark = False
        if "packed-fp32-ops" not in line:
            keep.append(line)
    return keep


def _deps() -> list[str]:
    return glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(HERE, "..", "include", "*.h"))


def _compile(src: str, force: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if not force and os.path.exists(obj):
        t = os.path.getmtime(obj)
        if all(os.path.getmtime(d) <= t for d in [src] + _deps()):
            return obj
    cmd = [HIPCC] + COMMON
    if src.endswith(".hip"):
        cmd += DEVICE + ["-Rpass-analysis=kernel-resource-usage", "-x", "hip"]
    else:
        cmd += ["-D__HIP_PLATFORM_AMD__"]
    cmd += ["-c", src, "-o", obj + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"compile failed: {os.path.basename(src)}")
    if src.endswith(".hip"):
        with open(obj + ".resources.txt", "w") as f:
            f.write(_check_resources(src, r.stderr))
    err = "\n".join(_diagnostics(r.stderr))
    if err.strip():
        sys.stderr.write(err + "\n")
    os.replace(obj + ".tmp", obj)
    return obj


def build(force: bool = False, jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    if force or not os.path.exists(LIB) or any(os.path.getmtime(o) > os.path.getmtime(LIB) for o in objs):
        cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB + ".tmp"] + objs + [
            f"-Wl,-rpath,{ROCM}/lib", "-lpthread"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
            raise RuntimeError("link failed")
        os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 1))
    a = ap.parse_args()
    print(build(a.force, a.j))
