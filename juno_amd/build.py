"""Build libjunohip.so in-tree for gfx950 with hipcc.

    python -m juno_amd.build

Flags: -O3, C++17, and -Xclang -target-feature -Xclang -packed-fp32-ops, which keeps
the compiler from emitting packed-fp32 VALU instructions.
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
# JUNO_LIB_OUT: another output path (juno_amd/timeline.py builds its instrumented variant there)
OUT = os.environ.get("JUNO_LIB_OUT", os.path.join(HERE, "libjunohip.so"))
SOURCES = ["jh_api.cpp", "jh_gemv.hip", "jh_gemv_staged.hip", "jh_quant.hip", "jh_mfma.hip", "jh_decode.hip", "jh_gguf.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [*os.environ.get("JH_EXTRA_FLAGS", "").split(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


INCLUDE = os.path.join(os.path.dirname(HERE), "include")


def source_hash() -> str:
    """SHA-256 (first 16 hex digits) over the library's sources: every file in
    csrc/ and include/ by name and content, plus the compile flags.  Built into
    the library (jh_version) and checked by _lib.load(), so that a libjunohip.so
    left from other sources is refused rather than run."""
    h = hashlib.sha256()
    for d in (CSRC, INCLUDE):
        for name in sorted(os.listdir(d)):
            if name.endswith((".hip", ".cpp", ".hpp", ".h")):
                h.update(name.encode() + b"\0")
                with open(os.path.join(d, name), "rb") as f:
                    h.update(f.read() + b"\0")
    h.update(" ".join(FLAGS).encode())
    return h.hexdigest()[:16]


def build(verbose: bool = False) -> str:
    cmd = [HIPCC, *FLAGS, f'-DJH_SRC_HASH="{source_hash()}"', *[os.path.join(CSRC, s) for s in SOURCES],
           "-o", OUT + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops",)
    errs = "\n".join(l for l in r.stderr.splitlines() if l.strip() and not any(n in l for n in noise))
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{errs}")
    if errs and verbose:
        print(errs, file=sys.stderr)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
