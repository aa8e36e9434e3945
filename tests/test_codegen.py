"""Code-generation checks on the gfx950 assembly of the operator library (CPU).

The compiler issues a 16x16x16 bf16 MFMA and a following 16x16x32 bf16 MFMA
that reads the first one's accumulator as SrcC back to back, with no wait
states; on gfx950 the second product then reads a stale accumulator (measured
on MI355X: 0.74 relative error back to back, exact with s_nop padding between
the two).  The kernels therefore run 16-deep bf16 products as zero-padded
16x16x32 products; this test fails if any kernel in the built assembly
contains the 16x16x16 form or chains two different depths through SrcC.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

_MFMA = re.compile(r"^\s*(v_mfma_f32_16x16x(16|32)_bf16)\s+(v\[\d+:\d+\]|a\[\d+:\d+\]),\s*\S+,\s*\S+,\s*(\S+)")


def mixed_srcc_chains(asm: str):
    """(kernel, line) of every MFMA whose SrcC is the destination of the most
    recent MFMA of the other depth writing that register range."""
    found = []
    kernel = None
    last_writer = {}  # register range -> depth of the MFMA that last wrote it
    for ln in asm.splitlines():
        m = re.match(r"^(_ZN4race\S+):\s*$", ln)
        if m:
            kernel, last_writer = m.group(1), {}
            continue
        mm = _MFMA.match(ln)
        if kernel is None:
            continue
        if mm:
            depth, dst, srcc = mm.group(2), mm.group(3), mm.group(4).rstrip(",")
            if srcc in last_writer and last_writer[srcc] != depth:
                found.append((kernel, ln.strip()))
            last_writer[dst] = depth
        else:
            w = re.match(r"^\s*v_\S+\s+(v\[\d+:\d+\]|v\d+)", ln)
            if w:
                last_writer.pop(w.group(1), None)
    return found


def test_scanner_flags_a_mixed_chain():
    asm = "\n".join([
        "_ZN4race1kE:",
        "\tv_mfma_f32_16x16x16_bf16 v[4:7], v[4:5], v[6:7], 0",
        "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[0:3], v[8:11], v[4:7]",
        "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[12:15], v[8:11], v[0:3]",
    ])
    assert len(mixed_srcc_chains(asm)) == 1


@pytest.mark.skipif(shutil.which(HIPCC) is None and not os.path.exists(HIPCC), reason="hipcc not available")
def test_no_mixed_depth_srcc_chain(tmp_path):
    from race_attention_amd.build import FLAGS
    flags = [f for f in FLAGS if f not in ("-shared", "-fPIC")]
    out = tmp_path / "race_capi.s"
    subprocess.check_call([HIPCC] + flags + ["--cuda-device-only", "-S",
                           os.path.join(ROOT, "race_attention_amd", "csrc", "race_capi.hip"), "-o", str(out)],
                          stderr=subprocess.DEVNULL)
    asm = out.read_text()
    assert "v_mfma_f32_16x16x32_bf16" in asm
    assert "v_mfma_f32_16x16x16_bf16" not in asm
    bad = mixed_srcc_chains(asm)
    assert not bad, bad[:5]
