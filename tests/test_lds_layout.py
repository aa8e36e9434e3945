"""CPU checks of the tile kernels' LDS layouts (race_layout.h) against the
gfx950 bank model (tests/lds_model.py, re-measured on the GPU by
tests/test_gpu_lds_model.py):

  * every 16-byte operand read of 16 rows and every pi-order pair read is
    conflict-free; 8-byte stores are at most 2-way;
  * the swizzle keeps each lane's k slots on the same logical k in every row
    (a product of two operands must pair equal k in all 16 x 16 lane pairs),
    and the pointer-plus-step addresses the kernels use equal the layout's;
  * the pi order makes the k of a pi-order operand one contiguous run;
  * the padded layouts the swizzle replaced were conflicted (the checks are
    sensitive)."""
import os
import shutil
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import lds_layouts as L  # noqa: E402
from lds_model import ways  # noqa: E402

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ needed to build the layout export")


@pytest.mark.parametrize("n", [32, 64, 128])
def test_swizzled_rows_keep_logical_k_per_slot(n):
    for r in range(64):
        for g in range(4):
            for kp in range(n // 32):
                # the kernels read at elem(r, 8g) + 32 kp: that must be logical k = 32 kp + 8g in every row
                assert L.elem(n, r, 8 * g) + 32 * kp == L.elem(n, r, 32 * kp + 8 * g)
        # rows 16 apart share the swizzle (one lane pointer, constant steps)
        for e in range(0, n, 4):
            assert L.elem(n, r + 16, e) - L.elem(n, r, e) == 16 * L.pitch(n)
        # a permutation of the row's 16-byte granules, inside each 32-element chunk
        assert sorted(L.elem(n, r, e) - r * L.pitch(n) for e in range(n)) == list(range(n))
        assert all((L.elem(n, r, e) - r * L.pitch(n)) // 32 == e // 32 for e in range(n))


def test_pi_order_runs():
    for h in range(2):
        for g in range(4):
            run = [L.pi_pos(32 * h + 4 * g + j) for j in range(4)] + [L.pi_pos(32 * h + 16 + 4 * g + j) for j in range(4)]
            assert run == list(range(32 * h + 8 * g, 32 * h + 8 * g + 8))
    assert sorted(L.pi_pos(k) for k in range(64)) == list(range(64))
    for m in range(16):  # aligned runs of 4 stay contiguous
        assert [L.pi_pos(4 * m + j) for j in range(4)] == [L.pi_pos(4 * m) + j for j in range(4)]


@pytest.mark.parametrize("n", [32, 64, 128])
def test_bucket_rows(n):
    for m in range(4):
        for kp in range(n // 32):
            assert ways("r128", L.operand_read(n, m, kp)) == 1
    for nt in range(4):
        for sw in range(0, n, 16):
            assert ways("w64", L.row_store(n, nt, sw)) <= 2


def test_natural_tiles():
    for m in range(2):
        for kp in range(2):
            assert ways("r128", L.nat_read(m, kp)) == 1
    for j in range(4):
        for half in range(2):
            assert ways("w64", L.nat_prefetch_store(j, half)) <= 2
    for cw in range(4):
        for e in range(2):
            assert ways("w64", L.nat_prefetcht_store(cw, e)) <= 2


def test_pi_rows():
    for n in range(4):
        assert ways("rpi", L.pi_read(n)) == 1
    for nt in range(2):
        for mt in range(2):
            assert ways("w64", L.pi_row_store(nt, mt)) == 1
    for cw in range(4):
        for q in range(4):
            assert ways("w32", L.transposed_word_store(cw, q)) == 1


def test_replaced_padded_layouts_were_conflicted():
    lanes = L.lanes
    # [t][D + 8] token tiles: 16-byte operand and pi-pair reads
    assert ways("r128", lanes(lambda g, i: i * 144 + 16 * g)) >= 2
    assert ways("rpi", lanes(lambda g, i: i * 144 + 8 * g)) >= 2
    # [t][SP + 8] bucket rows at SP = 128
    assert ways("r128", lanes(lambda g, i: i * 272 + 16 * g)) >= 2
    # [.][32 + 8] pi rows
    assert ways("rpi", lanes(lambda g, i: i * 80 + 8 * g)) >= 2
