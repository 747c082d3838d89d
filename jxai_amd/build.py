"""Build libjxmoe.so (HIP, gfx950) in-tree.

    python -m jxai_amd.build

Compiles every .hip source under jxai_amd/csrc with hipcc for gfx950 and
links jxai_amd/libjxmoe.so.  Flags that matter for parity:
  -ffp-contract=off                          every fused multiply-add is written
                                             explicitly (the router must follow
                                             the reference's exact fp32 order)
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE a/b for the Q8_0 scale amax/127
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                             no packed fp32 VALU instructions
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libjxmoe.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "jxmoe.h")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else "hipcc")

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Werror=return-type",
]


CXX = os.environ.get("CXX", "g++")
HOST_CFLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Werror=return-type"]


def sources() -> list[str]:
    """Device sources (.hip, hipcc for gfx950) and host-only sources (.cpp, the host compiler)."""
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def source_id() -> str:
    """First 16 hex digits of the SHA-256 over every source under csrc and include/jxmoe.h (names and
    bytes): compiled in as jx_build_id(), so a measurement recorded with one build can be told apart
    from another."""
    h = hashlib.sha256()
    for path in sources() + sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")) + [HEADER]:
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def _compile(src: str, sid: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src).rsplit(".", 1)[0] + ".o")
    define = f'-DJX_SOURCE_SHA="{sid}"'
    if src.endswith(".cpp"):
        cmd = [CXX, *HOST_CFLAGS, define, "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *CFLAGS, define, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError("hipcc not found: the MoE path needs ROCm's hipcc to build")
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    sid = source_id()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda src: _compile(src, sid), srcs))
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs], check=True)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} (source id {sid})")
    return LIB


if __name__ == "__main__":
    build()
