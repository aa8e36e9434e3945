"""Lane byte-offset patterns of the tile kernels' LDS accesses (bf16, C4
tile shapes), built from the exported layout functions of
race_attention_amd/csrc/race_layout.h (tests/hip/layout_dump.cpp) the way the
kernels form their addresses: a per-lane pointer plus compile-time steps."""
import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "hip", "layout_dump.cpp")
SO = os.path.join(HERE, "hip", "liblayout_dump.so")
TT, D, NCOL = 32, 64, 32
PI_PITCH = TT + 4          # rows read only as pi-order pairs (ldp_of)

_lib = None


def build_dump():
    subprocess.check_call(["g++", "-std=c++17", "-O1", "-shared", "-fPIC", "-D__host__=", "-D__device__=",
                           SRC, "-o", SO])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(SO) or os.path.getmtime(SO) < os.path.getmtime(SRC):
            build_dump()
        _lib = ctypes.CDLL(SO)
    return _lib


def pitch(n):
    return lib().race_sw_pitch(n)


def elem(n, r, e):
    return lib().race_sw_elem(n, r, e)


def pi_pos(k):
    return lib().race_pi_pos(k)


def lanes(f):
    """f(g, i) for lane 16g + i"""
    return [f(l >> 4, l & 15) for l in range(64)]


# ---- swizzled rows of n elements (bucket arrays n = SP, planes^T / dproj n = NCOL)
def operand_read(n, m, kp):
    """16-byte operand of rows 16m + i: pointer elem(n, 16m + i, 8g), step 32 per chunk"""
    return lanes(lambda g, i: 2 * (elem(n, 16 * m + i, 8 * g) + 32 * kp))


def row_store(n, nt, sw):
    """8-byte store of elements sw + 4g of rows 16nt + i: pointer of row i, step 16 rows"""
    return lanes(lambda g, i: 2 * (elem(n, i, sw + 4 * g) + 16 * pitch(n) * nt))


# ---- natural token tiles and planes (n = D, k in pi order)
def nat_read(m, kp):
    return operand_read(D, m, kp)


def nat_prefetch_store(j, half, nth=512):
    """16-byte chunk idx = lane + 64 j (row idx / 8, logical k 8(idx % 8)) stored as two runs of 4"""
    return [2 * elem(D, (l + 64 * j) // 8, pi_pos(8 * ((l + 64 * j) % 8) + 4 * half)) for l in range(64)]


def nat_prefetcht_store(cw, e):
    """token-pair task of lane l: pair tp = (l >> 2) & 15, 8-byte chunk c = (l & 3) + 4 cw, row 2 tp + e"""
    return [2 * elem(D, 2 * ((l >> 2) & 15) + e, pi_pos(4 * ((l & 3) + 4 * cw))) for l in range(64)]


# ---- rows read only as pi-order pairs (pitch TT + 4)
def pi_read(n):
    return lanes(lambda g, i: 2 * ((16 * n + i) * PI_PITCH + 4 * g))


def pi_row_store(nt, mt):
    return lanes(lambda g, i: 2 * ((16 * nt + i) * PI_PITCH + 16 * mt + 4 * g))


def transposed_word_store(cw, q):
    """PrefetchT transposed commit: row 4c + q (c = (l & 3) + 4 cw), word tp = (l >> 2) & 15"""
    return [2 * ((4 * ((l & 3) + 4 * cw) + q) * PI_PITCH) + 4 * ((l >> 2) & 15) for l in range(64)]


# ---- LDS transpose loads (ds_read_b64_tr_b16): lane (g, p) reads 4 elements,
# columns c0 + 4(p & 3) of row 4g + (p >> 2), and row 16 + ... for the
# operand's second half (race_kernels.hip col_operand, ts_operand_tr)
TR_PITCH = D + 16  # natural token rows read only by transpose loads (race_kernels.hip TrL::LD)


def tr_col_read(md, half, pitch_elems=TR_PITCH):
    """col_operand: natural token rows, columns 16 md + 4(p & 3)"""
    return lanes(lambda g, p: 2 * ((4 * g + (p >> 2) + half) * pitch_elems + 16 * md + 4 * (p & 3)))


def tr_ts_read(n, sw, half):
    """ts_operand_tr: swizzled [t][s] rows of n buckets, columns sw + 4(p & 3)"""
    return lanes(lambda g, p: 2 * elem(n, 4 * g + (p >> 2) + half, sw + 4 * (p & 3)))


def rebased(offs):
    """the same banks inside the probe's 8 KiB slot (banks repeat every 256 bytes)"""
    m = min(offs) // 256 * 256
    return [o - m for o in offs]
