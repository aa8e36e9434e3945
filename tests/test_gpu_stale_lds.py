"""No kernel takes a value from LDS, or from a workspace, state or output
buffer, that it has not written.

LDS keeps what the previous workgroup on a CU left there.  A bucket slice
(bf16 with K >= 5: 128 of the L * 2^K buckets; fp32: 32) projects only the
column blocks of its own tables, so the rest of its sigmoid rows is such a
leftover; its padding buckets (s >= S, the last slice's tail) must not derive
their zero probabilities from those rows by a product (0 * NaN = NaN).
tests/hip/lds_fill.hip writes all-ones bytes -- NaN as fp32 and as bf16 --
over every CU's LDS.  Here every entry point's call runs one kernel phase at a
time (race_desc.phases), with the fill ahead of each phase (the probability
entry points: ahead of the call), and every output must be the one of a call
without it, bit for bit.

The first cases are slice plans whose padded last slice does not project the
first column block (bf16 K=5 L=5 and K=6 L=5, fp32 K=4 L=5 and K=2 L=9),
through the F1 operator, the key-weight / den form, the global normalisation
and the probability outputs (before the padding rows were read from a
projected table, 8 of those 10 gave NaN); the rest cover the other
instantiation families.

The same cases run once more with every buffer the wrappers allocate
(outputs, state, workspaces) filled with all-ones bytes before use: every
output element must still be the one of a call with fresh buffers."""
import ctypes
import os

import pytest
import torch

from helpers import make_case

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PHASED = ("race_fwd", "race_bwd", "race_fwd_ex", "race_bwd_ex", "race_fwd_global", "race_bwd_global")
WHOLE = ("race_probs", "race_probs_bwd")


class _Filled:
    """The operator library with the LDS filled ahead of each kernel phase."""

    def __init__(self, lib, dev):
        self.lib = lib
        self.fl = ctypes.CDLL(os.path.join(HERE, "hip", "liblds_fill.so"))
        self.fl.lds_fill.argtypes = [ctypes.c_uint, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        self.blocks = 8 * torch.cuda.get_device_properties(dev).multi_processor_count
        self.sink = torch.empty(self.blocks, dtype=torch.int32, device=dev)
        self.fills = 0

    def fill(self):
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert self.fl.lds_fill(0xFFFFFFFF, self.blocks, self.sink.data_ptr(), stream) == 0
        self.fills += 1

    def __getattr__(self, name):
        f = getattr(self.lib, name)
        if name in WHOLE:
            def whole(*args):
                self.fill()
                return f(*args)
            return whole
        if name in PHASED:
            def phased(*args):
                d = args[0]._obj
                for ph in (1, 2, 4):  # RACE_PHASE_REDUCE, _SCAN, _OUT
                    d.phases = ph
                    self.fill()
                    rc = f(*args)
                    if rc:
                        return rc
                d.phases = 0
                return 0
            return phased
        return f


def _calls(mode, q, k, v, do, planes, kw, it, seg, g):
    from race_attention_amd import functional as F
    L, K = kw["L"], kw["K"]
    if mode in ("causal", "noncausal"):
        out, st = F.race_fwd_raw(q, k, v, planes, L=L, K=K, causal=mode == "causal", inv_temp=it, seg_tiles=seg)
        return (out,) + tuple(F.race_bwd_raw(q, k, v, planes, do, st, L=L, K=K, causal=mode == "causal",
                                             inv_temp=it, seg_tiles=seg))
    if mode == "ex":
        B, T = q.shape[1], q.shape[2]
        km = (torch.rand(B, T, generator=g) * 1.5 + 0.1).to(q.device)
        dden = torch.randn(q.shape[0], B, q.shape[3], T, generator=g).to(q.device)
        out, den, st = F.race_fwd_ex_raw(q, k, v, planes, L=L, K=K, inv_temp=it, kmask=km, want_den=True,
                                         seg_tiles=seg)
        return (out, den) + tuple(F.race_bwd_ex_raw(q, k, v, planes, do, dden, st, L=L, K=K, inv_temp=it,
                                                    kmask=km, seg_tiles=seg))
    if mode == "global":
        out, den, st = F.race_global_fwd_raw(q, k, v, planes, L=L, K=K, beta=it, seg_tiles=seg)
        return (out, den) + tuple(F.race_global_bwd_raw(q, k, v, planes, out, den, do, None, st, L=L, K=K,
                                                        beta=it, seg_tiles=seg))
    P = F.race_probs_raw(q, planes, L=L, K=K, inv_temp=it)
    dP = torch.randn(P.shape, generator=g).to(q.device)
    return (P,) + tuple(F.race_probs_bwd_raw(q, planes, dP, L=L, K=K, inv_temp=it))


BF16_K5 = dict(B=2, T=200, H=2, L=5, K=5)
BF16_K6 = dict(B=2, T=224, H=3, L=5, K=6, v_shift=0.5)
F32_K4 = dict(B=1, T=150, H=2, L=5, K=4, dtype=torch.float32, unit=False)
F32_K2 = dict(B=1, T=100, H=2, L=9, K=2, dtype=torch.float32, unit=False)
CASES = [
    # name, mode, make_case kwargs, inv_temp (global: beta), seg_tiles
    ("bf16_K5L5_causal", "causal", BF16_K5, 0.125, 3),
    ("bf16_K6L5_noncausal", "noncausal", BF16_K6, 0.125, 2),
    ("fp32_K4L5_causal", "causal", F32_K4, 0.5, 2),
    ("fp32_K2L9_noncausal", "noncausal", F32_K2, 1.0, 0),
    ("bf16_K6L5_ex", "ex", BF16_K6, 1.0, 2),
    ("fp32_K4L5_ex", "ex", F32_K4, 0.7, 0),
    ("bf16_K5L5_global", "global", BF16_K5, 1.0, 3),
    ("fp32_K2L9_global", "global", F32_K2, 0.7, 2),
    ("bf16_K6L5_probs", "probs", BF16_K6, 0.125, 0),
    ("fp32_K4L5_probs", "probs", F32_K4, 0.5, 0),
    # the other instantiation families: whole 4- and 8-bit tiles, unsliced small tables, 8-bit slices
    ("bf16_K4L8_whole_causal", "causal", dict(B=1, T=1024, H=2, L=8, K=4), 0.125, 3),
    ("bf16_K8L4_whole_causal", "causal", dict(B=1, T=1056, H=2, L=4, K=8), 0.125, 4),
    ("bf16_K8L3_ragged_causal", "causal", dict(B=1, T=333, H=2, L=3, K=8), 0.125, 3),
    ("bf16_K2L5_noncausal", "noncausal", dict(B=2, T=300, H=2, L=5, K=2), 1.0, 0),
    ("bf16_K3L8_causal", "causal", dict(B=1, T=250, H=2, L=8, K=3), 0.125, 2),
    ("bf16_K4L8_global_whole", "global", dict(B=1, T=512, H=2, L=8, K=4), 1.0, 3),
]


@pytest.mark.parametrize("name,mode,kw,it,seg", CASES, ids=[c[0] for c in CASES])
def test_outputs_ignore_lds_leftovers(dev, monkeypatch, name, mode, kw, it, seg):
    from race_attention_amd import _lib
    q, k, v, do, planes = [x.to(dev) for x in make_case(seed=11, **kw)]
    clean = _calls(mode, q, k, v, do, planes, kw, it, seg, torch.Generator().manual_seed(5))
    filled_lib = _Filled(_lib.load(), dev)
    monkeypatch.setattr(_lib, "_lib", filled_lib)
    filled = _calls(mode, q, k, v, do, planes, kw, it, seg, torch.Generator().manual_seed(5))
    torch.cuda.synchronize()
    assert filled_lib.fills >= 2
    for j, (a, b) in enumerate(zip(clean, filled)):
        nan = int(torch.isnan(b).sum())
        print(f"[{name} output {j}] NaN after LDS fills {nan}; bit-identical {torch.equal(a, b)}", flush=True)
        assert torch.isfinite(a).all(), f"{name} output {j}: non-finite without the fill"
        assert torch.equal(a, b), f"{name} output {j}: {nan} NaN, differs after the LDS fills"


def _poisoned_empty(real_empty):
    def empty(*args, **kw):
        x = real_empty(*args, **kw)
        if x.numel():
            x.reshape(-1).view(torch.uint8).fill_(255)
        return x
    return empty


@pytest.mark.parametrize("name,mode,kw,it,seg", CASES, ids=[c[0] for c in CASES])
def test_outputs_ignore_buffer_contents(dev, monkeypatch, name, mode, kw, it, seg):
    import types

    from race_attention_amd import functional as F
    q, k, v, do, planes = [x.to(dev) for x in make_case(seed=11, **kw)]
    clean = _calls(mode, q, k, v, do, planes, kw, it, seg, torch.Generator().manual_seed(5))
    fake = types.SimpleNamespace(**{a: getattr(torch, a) for a in dir(torch) if not a.startswith("__")})
    fake.empty = _poisoned_empty(torch.empty)
    fake.empty_like = lambda t, **kw_: fake.empty(t.shape, dtype=kw_.get("dtype", t.dtype),
                                                  device=kw_.get("device", t.device))
    monkeypatch.setattr(F, "torch", fake)
    poisoned = _calls(mode, q, k, v, do, planes, kw, it, seg, torch.Generator().manual_seed(5))
    torch.cuda.synchronize()
    for j, (a, b) in enumerate(zip(clean, poisoned)):
        print(f"[{name} output {j}] bit-identical with poisoned buffers {torch.equal(a, b)}", flush=True)
        assert torch.equal(a, b), f"{name} output {j}: differs when the buffers start as all-ones bytes"
