"""Compile the reference CPU kernel (kernels/cpu/race_pref.cpp) from its own
source under /root/reference into oracle/_ref/, with g++ and the installed
torch headers.  TEST INFRASTRUCTURE ONLY: the product never loads it.

This does not run the reference's build system (its race_ext.py / setup.py
loaders are broken as shipped: empty source list, hard-coded macOS path); it is
a one-file g++ compile of the unmodified source.  Output goes to oracle/_ref/
only, which is git-ignored.
"""
import os
import subprocess
import sys
import sysconfig

REF_SRC = "/root/reference/kernels/cpu/race_pref.cpp"
HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_ref")


def main() -> int:
    if not os.path.exists(REF_SRC):
        print(f"build_ref: {REF_SRC} absent; reference checker not built")
        return 0
    import torch
    import torch.utils.cpp_extension as ce

    os.makedirs(OUT_DIR, exist_ok=True)
    out = os.path.join(OUT_DIR, "race_pref" + sysconfig.get_config_var("EXT_SUFFIX"))
    if os.path.exists(out) and os.path.getmtime(out) >= os.path.getmtime(REF_SRC):
        print(f"build_ref: {out} up to date")
        return 0
    inc = []
    for p in ce.include_paths():
        inc += ["-isystem", p]
    inc += ["-isystem", sysconfig.get_paths()["include"]]
    libdir = ce.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = (["g++", "-O3", "-fopenmp", "-shared", "-fPIC", "-std=c++17", "-w",
            "-DTORCH_EXTENSION_NAME=race_pref", "-DTORCH_API_INCLUDE_EXTENSION_H",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}"] + inc +
           [REF_SRC, "-o", out + ".tmp", f"-L{libdir}", f"-Wl,-rpath,{libdir}",
            "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"])
    print("build_ref:", " ".join(cmd[:8]), "...", REF_SRC)
    subprocess.check_call(cmd)
    os.replace(out + ".tmp", out)
    print(f"build_ref: built {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
