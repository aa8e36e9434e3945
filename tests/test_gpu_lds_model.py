"""The gfx950 LDS bank model (tests/lds_model.py) measured on the GPU with
tests/hip/lds_probe.hip: 16 waves issue one access shape with given per-lane
byte offsets; cost is clock cycles per access relative to a broadcast (every
lane one address) of the same shape.

  * lane passes: lanes a and b share a pass iff putting b on a's banks at
    another address (every other lane broadcasting elsewhere) slows the access;
  * the kernels' access patterns (tests/lds_layouts.py, from race_layout.h)
    measure conflict-free where the model says so, and the padded layouts they
    replaced measure conflicted."""
import ctypes
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import lds_layouts as L  # noqa: E402
from lds_model import R128_PASSES, ways  # noqa: E402

# cycle-ratio thresholds: collected after every parity test (tests/conftest.py),
# so that a timing outlier under pytest -x cannot leave a parity test unrun
pytestmark = [pytest.mark.gpu, pytest.mark.timing]

HERE = os.path.dirname(os.path.abspath(__file__))
OPS = {"r32": 0, "r64": 1, "r128": 2, "w32": 3, "w64": 4, "w128": 5, "rpi": 6, "rtr": 7}
SIZE = {"r32": 4, "r64": 8, "r128": 16, "w32": 4, "w64": 8, "w128": 16, "rpi": 8, "rtr": 8}


class Probe:
    def __init__(self, dev):
        self.lib = ctypes.CDLL(os.path.join(HERE, "hip", "liblds_probe.so"))
        self.lib.lds_probe.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        self.dev = dev
        self.cyc = torch.zeros(1, dtype=torch.int64, device=dev)
        self.sink = torch.zeros(1024, dtype=torch.int32, device=dev)
        self.base = {}

    def raw(self, op, offs, iters=200):
        assert len(offs) == 64
        for o in offs:  # in bounds of the probe's 8 KiB slot, aligned to the access
            assert 0 <= o and o + (40 if op == "rpi" else SIZE[op]) <= 8192 and o % SIZE[op] == 0, (op, o)
        t = torch.tensor(offs, dtype=torch.int32, device=self.dev)
        assert self.lib.lds_probe(OPS[op], t.data_ptr(), iters, self.cyc.data_ptr(), self.sink.data_ptr()) == 0
        return int(self.cyc.item()) / (iters * 8 * 16)

    def ratio(self, op, offs):
        if op not in self.base:
            self.base[op] = self.raw(op, [0] * 64)
        return self.raw(op, offs) / self.base[op]


@pytest.fixture(scope="module")
def probe(dev):
    p = Probe(dev)
    p.raw("r128", [16 * l for l in range(64)])  # warm-up
    return p


def _same_pass(probe, op, a):
    other = 64 if op == "rpi" else SIZE[op]
    base = [other] * 64
    base[a] = 0
    ref = probe.raw(op, base)
    found = []
    for b in range(64):
        if b == a:
            continue
        offs = list(base)
        offs[b] = 4096  # same banks as lane a, another address
        if probe.raw(op, offs) / ref > 1.05:
            found.append(b)
    return found


@pytest.mark.parametrize("a", [0, 5, 40])
def test_read_b128_lane_passes(probe, a):
    expect = sorted(next(p for p in R128_PASSES if a in p))
    expect.remove(a)
    got = _same_pass(probe, "r128", a)
    print(f"[lds] ds_read_b128 lanes sharing a pass with lane {a}: {got}", flush=True)
    assert got == expect


def test_read_b64_lane_passes(probe):
    got = _same_pass(probe, "rpi", 0)
    print(f"[lds] ds_read2_b64 lanes sharing a pass with lane 0: {got}", flush=True)
    assert got == list(range(1, 16))


def test_kernel_patterns_measured(probe):
    cases = [
        ("bucket rows SP=128, operand read", "r128", L.operand_read(128, 0, 1)),
        ("bucket rows SP=64, operand read", "r128", L.operand_read(64, 0, 1)),
        ("natural tiles, operand read", "r128", L.nat_read(0, 1)),
        ("planes^T / dproj rows, operand read", "r128", L.operand_read(32, 0, 0)),
        ("pi rows, pi-pair read", "rpi", L.pi_read(0)),
        ("pi rows, 8-byte store", "w64", L.pi_row_store(0, 1)),
    ]
    old = [
        ("padded [t][D+8], operand read", "r128", L.lanes(lambda g, i: i * 144 + 16 * g)),
        ("padded [t][D+8], pi-pair read", "rpi", L.lanes(lambda g, i: i * 144 + 8 * g)),
        ("padded [t][SP+8] SP=128, operand read", "r128", L.lanes(lambda g, i: i * 272 + 16 * g)),
        ("padded [.][32+8], pi-pair read", "rpi", L.lanes(lambda g, i: i * 80 + 8 * g)),
    ]
    for name, op, offs in cases + old:
        r = probe.ratio(op, offs)
        print(f"[lds] {name:40s} model ways {ways(op, offs)}  measured cost x{r:.2f}", flush=True)
    for name, op, offs in cases:
        assert ways(op, offs) == 1
        assert probe.ratio(op, offs) < 1.08, name
    for name, op, offs in old:
        assert ways(op, offs) >= 2
        assert probe.ratio(op, offs) > 1.3, name


def test_transpose_load_patterns(probe):
    """ds_read_b64_tr_b16 serves 32 lanes per pass (measured: lanes 0-31 share
    one).  The kernels' two transpose-load operands -- col_operand over the
    natural token rows (pitch D + 16) and ts_operand_tr over the swizzled
    [t][s] bucket rows -- measure conflict-free; the token rows at an unpadded
    pitch (D) and at D + 4 measure conflicted."""
    got = _same_pass(probe, "rtr", 0)
    print(f"[lds] ds_read_b64_tr_b16 lanes sharing a pass with lane 0: {got}", flush=True)
    assert got == list(range(1, 32))
    good = [(f"col_operand md={md} half={h}", L.tr_col_read(md, h)) for md in range(4) for h in (0, 16)]
    good += [(f"ts_operand_tr SP=128 wave {w} half={h}", L.rebased(L.tr_ts_read(128, 16 * w, h)))
             for w in (0, 3, 5) for h in (0, 16)]
    bad = [(f"col_operand pitch {pe} md=0", L.tr_col_read(0, 0, pe)) for pe in (L.D, L.D + 4)]
    for name, offs in good + bad:
        print(f"[lds] {name:40s} measured cost x{probe.ratio('rtr', offs):.2f}", flush=True)
    for name, offs in good:
        assert probe.ratio("rtr", offs) < 1.08, name
    for name, offs in bad:
        assert probe.ratio("rtr", offs) > 1.3, name
