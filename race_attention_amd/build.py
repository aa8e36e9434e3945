"""Build the gfx950 HIP library race_attention_amd/librace_attention.so.

One translation unit (csrc/race_capi.hip, which includes the kernel sources)
compiled with hipcc for gfx950 only.  Packed-fp32 instruction selection is
disabled (-packed-fp32-ops) for all device code.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc", "race_capi.hip")
OUT = os.path.join(HERE, "librace_attention.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-shared", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


# host-side sanitizer build (device code unchanged): -fsanitize applies to the
# host compilation only, through -Xarch_host
SAN_OUT = os.path.join(HERE, "_san", "librace_attention_asan.so")
SAN_FLAGS = ["-g", "-fno-omit-frame-pointer", "-Xarch_host", "-fsanitize=address",
             "-Xarch_host", "-fsanitize=undefined"]


def build(verbose: bool = True, sanitize: bool = False) -> str:
    out = SAN_OUT if sanitize else OUT
    if sanitize:
        os.makedirs(os.path.dirname(out), exist_ok=True)
    cmd = [HIPCC] + FLAGS + (SAN_FLAGS if sanitize else []) + [SRC, "-o", out + ".tmp"]
    if verbose:
        print("build:", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    msgs = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        print("\n".join(msgs), file=sys.stderr)
        raise RuntimeError("hipcc failed building librace_attention.so")
    if verbose and msgs:
        print("\n".join(msgs))
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    build(sanitize="--sanitize" in sys.argv)
