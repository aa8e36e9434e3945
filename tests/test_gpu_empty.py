"""Empty batches and sequences (B = 0 or T = 0) through the autograd
Functions: the outputs and gradients come back empty with the input's shape,
a tensor temperature's gradient is zero (the derivative of an empty sum), and
nothing is launched.  The reference's modules return empty outputs for such
inputs (torch ops on empty tensors; race_pref.cpp allocates its empty result,
kernels/cpu/race_pref.cpp:51,129-130).  The C ABI itself still rejects a
descriptor with T = 0 (tests/test_capi.py)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

D, L, K = 64, 4, 3


def _planes(dev):
    g = torch.Generator().manual_seed(7)
    return torch.randn(L, K, D, generator=g).to(dev)


@pytest.mark.parametrize("shape", [(1, 0, 16, 2, D), (1, 2, 0, 2, D), (2, 1, 0, 3, D)])
@pytest.mark.parametrize("causal", [True, False])
def test_empty_race_attention(dev, shape, causal):
    from race_attention_amd.functional import race_attention
    q, k, v = [torch.zeros(shape, dtype=torch.bfloat16, device=dev, requires_grad=True) for _ in range(3)]
    temp = torch.tensor(0.7, device=dev, requires_grad=True)
    print(f"[empty] race_attention shape={shape} causal={causal}", flush=True)
    out = race_attention(q, k, v, _planes(dev), L=L, K=K, causal=causal, inv_temp=temp)
    assert out.shape == shape and out.dtype == torch.bfloat16
    out.float().sum().backward()
    for x in (q, k, v):
        assert x.grad is not None and x.grad.shape == shape
    assert temp.grad is not None and float(temp.grad) == 0.0


def test_empty_global_ex_probs(dev):
    from race_attention_amd.functional import race_attention_ex, race_attention_global, race_bucket_probs
    shape = (1, 2, 0, 2, D)
    q, k, v = [torch.zeros(shape, dtype=torch.float32, device=dev, requires_grad=True) for _ in range(3)]
    beta = torch.tensor(1.0, device=dev, requires_grad=True)
    print("[empty] global / ex / probs, T = 0", flush=True)
    out, den = race_attention_global(q, k, v, _planes(dev), L=L, K=K, beta=beta)
    assert out.shape == shape and den.shape == (1, 2, 2, 0)
    (out.sum() + den.sum()).backward()
    assert q.grad.shape == shape and float(beta.grad) == 0.0

    q.grad = None
    out, den = race_attention_ex(q, k, v, _planes(dev), L=L, K=K, inv_temp=0.5,
                                 kmask=torch.ones(2, 0, device=dev), with_den=True)
    assert out.shape == shape and den.shape == (1, 2, 2, 0)
    (out.sum() + den.sum()).backward()
    assert q.grad.shape == shape

    x = torch.zeros(shape, dtype=torch.float32, device=dev, requires_grad=True)
    P = race_bucket_probs(x, _planes(dev), L=L, K=K, inv_temp=1.0)
    assert P.shape == (1, 2, 2, 0, L, 1 << K)
    P.sum().backward()
    assert x.grad.shape == shape


def test_empty_prefix_mean(dev):
    from race_attention_amd.functional import RACEPrefixMeanFlatFn
    w = torch.zeros(3, 0, device=dev, requires_grad=True)
    v = torch.zeros(3, 0, 5, device=dev, requires_grad=True)
    print("[empty] prefix mean, T = 0", flush=True)
    E = RACEPrefixMeanFlatFn.apply(w, v, 1e-6)
    assert E.shape == (3, 0, 5)
    E.sum().backward()
    assert w.grad.shape == (3, 0) and v.grad.shape == (3, 0, 5)
