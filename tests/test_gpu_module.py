"""Module-level GPU tests: the drop-in modules (race_attention_amd.race /
.vit, mirrors of misc/race.py:26-206 and misc/vit.py:888-1068) run on the GPU
in fp32 and are compared with a CPU fp64 copy of the same module whose
attention core is the fp64 oracle wrapped as an autograd Function.  Outputs
and every gradient (input, Linear weights, logit_temp) are compared with the
fp32 bar, max|a-b|/max|b| <= 1e-4."""
import copy

import pytest
import torch

from helpers import TOL, make_case, relerr

pytestmark = pytest.mark.gpu


def _planes4(planes):
    """[L,K,D] (shared) or [M,L,K,D] -> the oracle's [NP,L,K,D] fp64."""
    p = planes.detach().double()
    return (p.unsqueeze(0) if p.dim() == 3 else p).numpy()


class OracleRACE(torch.autograd.Function):
    """race_attention's contract on CPU fp64, computed by the oracle."""

    @staticmethod
    def forward(ctx, Q, K, V, planes, inv_temp, L, Kb, causal, eps):
        from oracle import race_oracle as ro
        it = float(inv_temp)
        arr = [x.detach().double().contiguous().numpy() for x in (Q, K, V)]
        pl = _planes4(planes)
        out = ro.race_forward(*arr, pl, causal=causal, eps=eps, inv_temp=it)
        ctx.save_for_backward(Q, K, V, planes)
        ctx.cfg = (causal, eps, it, torch.is_tensor(inv_temp))
        return torch.from_numpy(out)

    @staticmethod
    def backward(ctx, g):
        from oracle import race_oracle as ro
        Q, K, V, planes = ctx.saved_tensors
        causal, eps, it, temp_tensor = ctx.cfg
        arr = [x.detach().double().contiguous().numpy() for x in (Q, K, V, g)]
        dq, dk, dv, git = ro.race_backward(*arr, _planes4(planes), causal=causal, eps=eps, inv_temp=it)
        gt = torch.tensor(git, dtype=torch.float64) if temp_tensor else None
        return (torch.from_numpy(dq), torch.from_numpy(dk), torch.from_numpy(dv), None, gt,
                None, None, None, None)


def _oracle_attention(Qhf, Khf, Vhf, planes, *, L, K, causal, inv_temp, eps=1e-6):
    return OracleRACE.apply(Qhf, Khf, Vhf, planes, inv_temp, L, K, causal, eps)


def _run_pair(monkeypatch, mod_name, make, x_shape, seed):
    """Run make() on the GPU (fp32) and its fp64 CPU copy through the oracle."""
    import importlib
    mod = importlib.import_module(mod_name)
    torch.manual_seed(seed)
    m_cpu = make(mod)
    m_ref = copy.deepcopy(m_cpu).double()
    m_gpu = m_cpu.to("cuda")
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(*x_shape, generator=g)
    gy = torch.randn(*x_shape, generator=g)  # d_out == d_in in every case here

    xg = x.to("cuda").requires_grad_(True)
    y = m_gpu(xg)
    y.backward(gy.to("cuda"))
    torch.cuda.synchronize()

    monkeypatch.setattr(mod, "race_attention", _oracle_attention)
    xr = x.double().requires_grad_(True)
    yr = m_ref(xr)
    yr.backward(gy.double())
    monkeypatch.undo()

    pairs = [("y", y, yr), ("dx", xg.grad, xr.grad)]
    ref_params = dict(m_ref.named_parameters())
    for name, p in m_gpu.named_parameters():
        if p.grad is not None:
            pairs.append(("d" + name, p.grad, ref_params[name].grad))
    return pairs


def _check(tag, pairs, tol):
    errs = {n: relerr(a.detach().double().cpu(), b.detach()) for n, a, b in pairs}
    print(f"[{tag}] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for n, e in errs.items():
        assert e <= tol, f"{tag}: {n} relerr {e:.3e} > {tol:.1e}"


@pytest.mark.parametrize("merge", [True, False])
def test_causal_race_attention_module(dev, monkeypatch, merge):
    make = lambda mod: mod.RACEAttention(d=128, h=2, K=2, L=5, M=1, drop=0.0, qkv_bias=True,  # noqa: E731
                                         reference_head_merge=merge)
    _check(f"race.RACEAttention merge={merge}", _run_pair(monkeypatch, "race_attention_amd.race", make,
                                                          (2, 70, 128), seed=3), TOL[torch.float32])


def test_causal_race_attention_independent_planes(dev, monkeypatch):
    """M=2 estimators with independent sketches through BatchedACE directly."""
    import race_attention_amd.race as rr

    torch.manual_seed(5)
    ace = rr.BatchedACE(64, K=2, L=4, M=2, share_planes=False)
    g = torch.Generator().manual_seed(6)
    Khf, Vhf, Qhf = [torch.randn(2, 1, 40, 3, 64, generator=g) for _ in range(3)]
    gy = torch.randn(2, 1, 40, 3, 64, generator=g)
    ins = [t.to(dev).requires_grad_(True) for t in (Khf, Vhf, Qhf)]
    y = ace.to(dev)(*ins)
    y.backward(gy.to(dev))
    monkeypatch.setattr(rr, "race_attention", _oracle_attention)
    ref_ins = [t.double().requires_grad_(True) for t in (Khf, Vhf, Qhf)]
    yr = copy.deepcopy(ace).cpu().double()(*ref_ins)
    yr.backward(gy.double())
    pairs = [("y", y, yr)] + [(n, a.grad, b.grad) for n, a, b in zip(("dK", "dV", "dQ"), ins, ref_ins)]
    _check("race.BatchedACE M=2 independent", pairs, TOL[torch.float32])


def test_noncausal_vit_attention_module(dev, monkeypatch):
    """misc/vit.py RACEAttention: non-causal, M=2 independent sketches,
    learnable temperature (logit_temp receives its gradient)."""
    make = lambda mod: mod.RACEAttention(d_in=128, d_out=128, dropout=0.0, num_heads=2, L=5, K=2,  # noqa: E731
                                         N_M=2, qkv_bias=True)
    pairs = _run_pair(monkeypatch, "race_attention_amd.vit", make, (2, 50, 128), seed=8)
    assert any(n == "dace.logit_temp" for n, _, _ in pairs)
    _check("vit.RACEAttention M=2", pairs, TOL[torch.float32])


def test_causal_race_block(dev, monkeypatch):
    cfg = {"emb_dim": 128, "n_heads": 2, "K": 2, "L": 5, "M": 1, "drop_rate": 0.0, "qkv_bias": False}
    import race_attention_amd.race as rr

    torch.manual_seed(12)
    blk = rr.RACEBlock(cfg)
    ref = copy.deepcopy(blk).double()
    g = torch.Generator().manual_seed(13)
    x = torch.randn(2, 64, 128, generator=g)
    gy = torch.randn(2, 64, 128, generator=g)
    xg = x.to(dev).requires_grad_(True)
    blk = blk.to(dev)
    blk(xg).backward(gy.to(dev))
    y = blk(xg.detach())
    monkeypatch.setattr(rr, "race_attention", _oracle_attention)
    xr = x.double().requires_grad_(True)
    yr = ref(xr)
    yr.backward(gy.double())
    pairs = [("y", y, yr), ("dx", xg.grad, xr.grad)]
    rp = dict(ref.named_parameters())
    pairs += [("d" + n, p.grad, rp[n].grad) for n, p in blk.named_parameters()]
    _check("race.RACEBlock", pairs, TOL[torch.float32])


def _ref_copy(model):
    return copy.deepcopy(model).double()


def test_vision_transformer_step(dev, monkeypatch):
    """vit.VisionTransformer (misc/vit.py:4918-4982) with RACE blocks, fp32 on
    the GPU, against its fp64 CPU copy whose attention core is the oracle:
    logits and every parameter gradient of a cross-entropy loss."""
    import race_attention_amd.vit as rv
    cfg = dict(img_size=12, patch_size=2, num_channels=1, embed_dim=128, num_heads=2, transformer_units=2,
               drop_rate=0.0, qkv_bias=False, K=2, L=5, M=1, num_classes=10)
    torch.manual_seed(21)
    m = rv.VisionTransformer(cfg)
    ref = _ref_copy(m)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(3, 1, 12, 12, generator=g)
    y = torch.randint(0, 10, (3,), generator=g)
    md = m.to(dev)
    out = md(x.to(dev))
    torch.nn.functional.cross_entropy(out, y.to(dev)).backward()
    torch.cuda.synchronize()
    monkeypatch.setattr(rv, "race_attention", _oracle_attention)
    out_r = ref(x.double())
    torch.nn.functional.cross_entropy(out_r, y).backward()
    monkeypatch.undo()
    rp = dict(ref.named_parameters())
    pairs = [("logits", out, out_r)] + [("d" + n, p.grad, rp[n].grad) for n, p in md.named_parameters()]
    _check("vit.VisionTransformer", pairs, TOL[torch.float32])


def test_lm_model_step(dev, monkeypatch):
    """lm.LMModel (misc/lm.py:37-74) with causal RACE blocks, fp32 on the
    GPU, against its fp64 CPU copy with the oracle attention core."""
    import race_attention_amd.lm as rl
    import race_attention_amd.race as rr
    cfg = dict(vocab_size=300, context_length=96, emb_dim=128, n_heads=2, n_layers=2, drop_rate=0.0, qkv_bias=False,
               K=2, L=4, M=2)
    torch.manual_seed(31)
    m = rl.LMModel(cfg)
    ref = _ref_copy(m)
    g = torch.Generator().manual_seed(32)
    ids = torch.randint(0, 300, (2, 96), generator=g)
    tgt = torch.randint(0, 300, (2, 96), generator=g)
    md = m.to(dev)
    out = md(ids.to(dev))
    torch.nn.functional.cross_entropy(out.flatten(0, 1), tgt.to(dev).flatten()).backward()
    torch.cuda.synchronize()
    monkeypatch.setattr(rr, "race_attention", _oracle_attention)
    out_r = ref(ids)
    torch.nn.functional.cross_entropy(out_r.flatten(0, 1), tgt.flatten()).backward()
    monkeypatch.undo()
    rp = dict(ref.named_parameters())
    pairs = [("logits", out, out_r)] + [("d" + n, p.grad, rp[n].grad) for n, p in md.named_parameters()]
    _check("lm.LMModel", pairs, TOL[torch.float32])


def test_device_temperature_bit_identical(dev):
    """A temperature passed as a device tensor (read in-kernel through
    inv_temp_ptr) gives the same bits as the same value passed as a float,
    forward and backward, including d(inv_temp)."""
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    q, k, v, do, planes = make_case(B=2, T=150, H=3, L=5, K=2, dtype=torch.bfloat16, unit=False, seed=41)
    qd, kd, vd, dod, pd = [x.to(dev) for x in (q, k, v, do, planes)]
    it_t = torch.tensor(0.8125, device=dev)
    for causal in (False, True):
        o1, s1 = race_fwd_raw(qd, kd, vd, pd, L=5, K=2, causal=causal, inv_temp=0.8125)
        o2, s2 = race_fwd_raw(qd, kd, vd, pd, L=5, K=2, causal=causal, inv_temp=it_t)
        g1 = race_bwd_raw(qd, kd, vd, pd, dod, s1, L=5, K=2, causal=causal, inv_temp=0.8125)
        g2 = race_bwd_raw(qd, kd, vd, pd, dod, s2, L=5, K=2, causal=causal, inv_temp=it_t)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
        for a, b in zip(g1, g2):
            assert torch.equal(a, b)


def test_learnable_temperature_no_host_sync(dev):
    """The non-causal module with its learnable temperature runs forward and
    backward without a device-to-host synchronisation (torch raises on one in
    sync-debug mode "error")."""
    from race_attention_amd.vit import RACEBlock
    torch.manual_seed(0)
    cfg = dict(embed_dim=128, drop_rate=0.0, num_heads=2, qkv_bias=False, L=5, K=2, M=1)
    blk = RACEBlock(cfg).to(dev)
    x = torch.randn(2, 77, 128, device=dev, requires_grad=True)
    blk(x).sum().backward()  # warm-up: first-call work outside the checked region
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        y = blk(x)
        y.sum().backward()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert torch.isfinite(blk.att.ace.logit_temp.grad).all()
