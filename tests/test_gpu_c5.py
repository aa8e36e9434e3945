"""Config C5: the GPT decoder of misc/lm.py:37-74 over the
causal RACE blocks of misc/race.py:144-206 -- 12 layers, d_model 768, 12 heads
(d=64), MLP 3072, vocab 50257, causal RACE with K=8 (256 buckets per table),
L=4, M=2 with the shared sketch of misc/race.py:33 (so the two estimators are
one computation), batch 8 x 8192 tokens, bf16 autocast, AdamW.

One full training step at that size:
  * the loss and every parameter's gradient are finite, and AdamW changes
    every parameter;
  * block 0's RACE core inside the step -- the bf16 Q, K, V it received
    (strided views of the projections, expanded over M), its output and the
    gradients that flowed through it -- against the fp64 oracle on two
    streams (batch row 0 / head 0 and batch row 7 / head 11), bf16 bar 2e-2.
"""
import math

import pytest
import torch

from helpers import TOL, relerr, to64

pytestmark = pytest.mark.gpu

B, T, H, D, L, K = 8, 8192, 12, 64, 4, 8
STREAMS = ((0, 0), (7, 11))  # (batch row, head)


def test_c5_gpt_training_step(dev, oracle, monkeypatch):
    from race_attention_amd import race as race_mod
    from race_attention_amd.lm import LMModel
    torch.manual_seed(0)
    cfg = dict(vocab_size=50257, context_length=T, emb_dim=768, n_heads=H, n_layers=12, drop_rate=0.1,
               qkv_bias=False, K=K, L=L, M=2)
    model = LMModel(cfg).to(dev)
    x = torch.randint(0, cfg["vocab_size"], (B, T), device=dev)
    y = torch.randint(0, cfg["vocab_size"], (B, T), device=dev)

    # record the first call of the attention core (block 0) inside the step
    rec = {}
    core = race_mod.race_attention

    def recording(q, k, v, planes, **kw):
        out = core(q, k, v, planes, **kw)
        if "out" not in rec:
            rec.update(q=q.detach().clone(), k=k.detach().clone(), v=v.detach().clone(),
                       planes=planes.detach().clone(), kw=dict(kw), out=out.detach().clone())
            for name, t in (("dq", q), ("dk", k), ("dv", v), ("gout", out)):
                t.register_hook(lambda g, name=name: rec.__setitem__(name, g.detach().clone()))
        return out

    monkeypatch.setattr(race_mod, "race_attention", recording)
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, weight_decay=0.1)
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    print(f"[C5 step] GPT 12 x (d=768, {H} heads, K={K} L={L} M=2 shared), vocab 50257, batch {B} x {T}, "
          "bf16 autocast", flush=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = model(x)
    loss = torch.nn.functional.cross_entropy(logits.flatten(0, 1).float(), y.flatten())
    del logits
    loss.backward()
    assert torch.isfinite(loss), float(loss)
    for n, p in model.named_parameters():
        assert p.grad is not None, n
        assert torch.isfinite(p.grad).all(), n
    opt.step()
    torch.cuda.synchronize()
    print(f"[C5 step] loss {float(loss):.4f}", flush=True)
    for n, p in model.named_parameters():
        assert not torch.equal(p.detach(), before[n]), f"{n} not updated"
    del before

    # block 0's core: shared sketch, so one estimator ([1, B, T, H, D] bf16 views)
    q = rec["q"]
    assert q.dtype == torch.bfloat16 and q.shape == (1, B, T, H, D), (q.dtype, q.shape)
    assert rec["kw"]["causal"] and abs(rec["kw"]["inv_temp"] - 1.0 / math.sqrt(D)) < 1e-12
    assert rec["planes"].shape == (L, K, D)
    sub = lambda z: torch.cat([z[:, b:b + 1, :, h:h + 1] for b, h in STREAMS], dim=1).contiguous()  # noqa: E731
    it = rec["kw"]["inv_temp"]
    pl = rec["planes"].double().cpu().numpy()[None]  # [1, L, K, D]: one shared sketch
    o_ref = oracle.race_forward(to64(sub(q)), to64(sub(rec["k"])), to64(sub(rec["v"])), pl, causal=True,
                                inv_temp=it)
    g_ref = oracle.race_backward(to64(sub(q)), to64(sub(rec["k"])), to64(sub(rec["v"])), to64(sub(rec["gout"])),
                                 pl, causal=True, inv_temp=it)
    errs = {"out": relerr(to64(sub(rec["out"])), o_ref)}
    errs.update({nm: relerr(to64(sub(rec[nm])), r) for nm, r in zip(("dq", "dk", "dv"), g_ref[:3])})
    print("[C5 step, block 0 core, 2 streams] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert max(errs.values()) <= TOL[torch.bfloat16]
