"""Builds libmegaqwen_hip.so for gfx950 with hipcc (in-tree, next to this file).

    python -m megaqwen_amd.build            # or megaqwen_amd.build.build()

The library is plain HIP C++ behind the C ABI of include/megaqwen_hip.h; no torch headers.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmegaqwen_hip.so")
SOURCES = ["decode.hip", "prefill.hip", "flash_attn.hip", "capi.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # packed fp32 (v_pk_*_f32) stays off: the compiler must not form it on its own
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
]


# decode.hip's kernels hold up to 256 VGPRs (two waves per SIMD); a spill there is silent and
# costs ~15% of a decode step, so every compile reports per-kernel resource usage to
# _build/<source>_resources.txt (decode.hip's is RESOURCE_REPORT) and warns on a spill
RESOURCE_REPORT = os.path.join(HERE, "_build", "decode_resources.txt")


def resource_report(src: str) -> str:
    return os.path.join(HERE, "_build", src.replace(".hip", "_resources.txt"))


def parse_resource_usage(text: str) -> dict:
    """{kernel: {"VGPRs": n, "VGPRs Spill": n, "ScratchSize": n, ...}} from the compiler's
    kernel-resource-usage remarks."""
    out, cur = {}, None
    for line in text.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].split("[-Rpass")[0].strip()
        if body.startswith("Function Name:"):
            cur = body.split(":", 1)[1].strip()
            out[cur] = {}
        elif cur is not None and ":" in body:
            key, val = body.split(":", 1)
            key = key.split("[")[0].strip()
            try:
                out[cur][key] = int(val.strip())
            except ValueError:
                pass
    return out


def build(verbose: bool = False) -> str:
    objs = []
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    for src in SOURCES:
        obj = os.path.join(HERE, "_build", src.replace(".hip", ".o"))
        cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj,
               "-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics"]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, stderr=subprocess.PIPE, text=True)
        remarks = [ln for ln in r.stderr.splitlines() if "kernel-resource-usage" in ln]
        rest = [ln for ln in r.stderr.splitlines() if "kernel-resource-usage" not in ln]
        if rest:
            print("\n".join(rest), file=sys.stderr, flush=True)
        if r.returncode != 0:
            raise subprocess.CalledProcessError(r.returncode, cmd)
        with open(resource_report(src), "w") as f:
            f.write("\n".join(remarks) + "\n")
        for name, u in parse_resource_usage("\n".join(remarks)).items():
            if u.get("VGPRs Spill", 0) or u.get("ScratchSize", 0):
                print(f"warning: {name} spills ({u.get('VGPRs Spill', 0)} VGPRs, "
                      f"{u.get('ScratchSize', 0)} B scratch per lane)", file=sys.stderr)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
