"""CPU-side host logic of the module mirrors (no kernel launches)."""
import itertools

import numpy as np
import pytest
import torch

from race_attention_amd import race as rrace
from race_attention_amd import vit as rvit
from race_attention_amd.functional import make_desc


def test_causal_module_buffers_match_reference_shapes():
    torch.manual_seed(0)
    ace = rrace.BatchedACE(64, 4, 8, 1)
    assert ace.planes_T.shape == (64, 32)                      # misc/race.py:41-45
    assert ace.protos_T.shape == (4, 16)                       # misc/race.py:54-58
    ref = torch.tensor(list(itertools.product([-1., +1.], repeat=4))).T
    assert torch.equal(ace.protos_T, ref)
    ace2 = rrace.BatchedACE(64, 4, 8, 2, share_planes=False)
    assert ace2.planes_T.shape == (2, 64, 32)                   # misc/race.py:47-50
    assert set(dict(ace.named_buffers())) == {"planes_T", "protos_T"}


def test_noncausal_module_param_and_buffers():
    ace = rvit.BatchedACE(64, 2, 5, 1)
    assert ace.planes_T.shape == (1, 64, 10)                    # misc/vit.py:904-908 (share_planes=False)
    assert [n for n, _ in ace.named_parameters()] == ["logit_temp"]
    assert float(ace.logit_temp) == 0.0                        # log(1.0), misc/vit.py:915
    with torch.no_grad():
        ace.logit_temp.fill_(10.0)
    assert float(ace.scale()) == 20.0                          # clamp(1e-2, 20), misc/vit.py:923


def test_planes_from_T_column_order():
    """planes_T column j = l*K + k holds plane (l, k) (misc/race.py:41-45)."""
    L, K, d = 3, 2, 8
    planes = torch.randn(L, K, d)
    planes_T = planes.view(L * K, d).T
    assert torch.equal(rrace.planes_from_T(planes_T, L, K), planes)
    Mp = torch.randn(2, L, K, d)
    assert torch.equal(rrace.planes_from_T(Mp.view(2, L * K, d).transpose(1, 2), L, K), Mp)


def test_reference_head_merge_reproduces_reference_reinterpretation():
    """merge_heads(reference=True) == out.mean(0).permute(0,2,1,3).contiguous().view(B,T,-1)."""
    M, B, T, H, d = 2, 2, 6, 3, 4
    out_h = torch.randn(M, B, T, H, d)
    ref = out_h.mean(0).permute(0, 2, 1, 3).contiguous().view(B, T, -1)
    assert torch.equal(rrace.merge_heads(out_h, True), ref)
    plain = rrace.merge_heads(out_h, False)
    assert torch.equal(plain, out_h.mean(0).reshape(B, T, H * d))
    # the reference merge mixes tokens: row 0 holds head 0 of tokens 0..H-1
    one = torch.arange(T, dtype=torch.float32).view(1, 1, T, 1, 1).expand(1, 1, T, H, d)
    assert rrace.merge_heads(one, True)[0, 0, :d].tolist() == [0.0] * d
    assert rrace.merge_heads(one, True)[0, 0, d:2 * d].tolist() == [1.0] * d


def test_cpu_tensors_are_rejected_not_computed():
    ace = rrace.BatchedACE(64, 4, 8, 1)
    x = torch.randn(1, 1, 8, 2, 64)
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        ace(x, x, x)


def test_desc_from_expanded_inputs():
    q = torch.randn(1, 2, 10, 3, 64).expand(4, -1, -1, -1, -1)
    planes = torch.randn(1, 8, 4, 64)
    d = make_desc(q, q, q, planes, L=8, K=4, causal=True, eps=1e-6, inv_temp=0.125)
    assert list(d.q_stride) == [0, 10 * 3 * 64, 3 * 64, 64]
    assert (d.M, d.B, d.T, d.H, d.D) == (4, 2, 10, 3, 64)
    assert d.planes_m_stride == 0
    d2 = make_desc(q, q, q, torch.randn(4, 8, 4, 64), L=8, K=4, causal=False, eps=1e-6, inv_temp=1.0)
    assert d2.planes_m_stride == 8 * 4 * 64
    with pytest.raises(ValueError):
        make_desc(q, q, q, torch.randn(3, 8, 4, 64), L=8, K=4, causal=False, eps=1e-6, inv_temp=1.0)
    assert np.isclose(d.inv_temp, 0.125)


def test_global_module_matches_reference_construction():
    """CausalRACEAttention (misc/elsaa_causal_complete.py:438-481): buffer
    names and shapes, non-persistent buffers, log_beta parameter, clamp."""
    from race_attention_amd.causal import CausalRACEAttention
    m = CausalRACEAttention(256, 4, 0.1, num_bits=3, num_tables=5, beta_init=2.0)
    assert (m.h, m.dk, m.num_bits, m.num_tables, m.R, m.C, m.chunk_group_size) == (4, 64, 3, 5, 8, 256, 64)
    assert m.planes.shape == (5, 3, 64)
    assert torch.equal(m.corners, torch.tensor(list(itertools.product([-1.0, 1.0], repeat=3))))
    assert "planes" not in m.state_dict() and "corners" not in m.state_dict()
    assert abs(float(m.log_beta) - np.log(2.0)) < 1e-7
    with torch.no_grad():
        m.log_beta.fill_(10.0)
    assert float(m.beta()) == 20.0
    assert m.last_den is None
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        m(torch.randn(1, 8, 256))
