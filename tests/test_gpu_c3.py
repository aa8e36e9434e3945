"""Config C3: the ViT encoder of misc/vit.py:4918-4982
over the non-causal BatchedACE of misc/vit.py:918-979 -- 6 layers, d_model
384, 6 heads (d=64), MLP 1536, K=2, L=5, M=1, batch 64 x 785 tokens (784 patch
tokens + CLS; the last 32-token tile holds 17), bf16.

  * the operator at the C3 shape (B=64, H=6, T=785, bf16, non-causal, the
    initial temperature exp(0) = 1), every stream and d(inv_temp) against the
    fp64 oracle;
  * one full training step of the 6-layer model under bf16 autocast with
    AdamW: loss and every gradient finite, the RACE core of the first block
    checked inside the step (its recorded inputs, output and the gradients
    that flow through it against the oracle on a subset of streams), and the
    step changes every parameter that has a gradient.
"""
import pytest
import torch

from helpers import TOL, compare, make_case, relerr, run_gpu, run_oracle, to64

pytestmark = pytest.mark.gpu

B, T, H, D, L, K = 64, 785, 6, 64, 5, 2


def test_c3_operator(dev):
    q, k, v, do, planes = make_case(B=B, T=T, H=H, L=L, K=K, dtype=torch.bfloat16, unit=False, seed=33)
    print(f"[C3 operator] non-causal bf16 B={B} T={T} H={H} K={K} L={L}", flush=True)
    gpu = run_gpu(q, k, v, do, planes, L=L, K=K, causal=False, inv_temp=1.0, dev=dev)
    for x in gpu[:4]:
        assert torch.isfinite(x).all()
    ref = run_oracle(q, k, v, do, planes, causal=False, inv_temp=1.0)
    compare("C3 operator", gpu, ref, TOL[torch.bfloat16])


def test_c3_vit_training_step(dev, oracle):
    from race_attention_amd.vit import VisionTransformer
    torch.manual_seed(0)
    cfg = dict(img_size=28, patch_size=1, num_channels=1, embed_dim=384, num_heads=H, transformer_units=6,
               drop_rate=0.0, qkv_bias=False, K=K, L=L, M=1, num_classes=10)
    model = VisionTransformer(cfg).to(dev)
    x = torch.randn(B, 1, 28, 28, device=dev)
    y = torch.randint(0, 10, (B,), device=dev)
    ace = model.transformer_layers[0].att.ace
    rec = {}

    def fwd_hook(mod, inp, out):
        rec["in"] = [t.detach().clone() for t in inp]  # Khf, Vhf, Qhf
        rec["out"] = out.detach().clone()
        rec["inv_temp"] = float(1.0 / mod.scale())

    def bwd_hook(mod, gin, gout):
        rec["gin"] = [g.detach().clone() for g in gin]
        rec["gout"] = gout[0].detach().clone()

    h1 = ace.register_forward_hook(fwd_hook)
    h2 = ace.register_full_backward_hook(bwd_hook)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=0.1)
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    print(f"[C3 step] ViT 6 x (d=384, 6 heads, K={K} L={L}) batch {B} x {T} tokens, bf16 autocast", flush=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits = model(x)
    loss = torch.nn.functional.cross_entropy(logits.float(), y)
    loss.backward()
    h1.remove()
    h2.remove()
    assert torch.isfinite(loss), float(loss)
    for n, p in model.named_parameters():
        assert p.grad is not None, n
        assert torch.isfinite(p.grad).all(), n
    for blk in model.transformer_layers:
        assert blk.att.ace.logit_temp.grad.abs() > 0
        assert blk.att.q_proj.weight.grad.abs().sum() > 0
    opt.step()
    torch.cuda.synchronize()
    for n, p in model.named_parameters():
        assert not torch.equal(p.detach(), before[n]), f"{n} not updated"

    # the first block's RACE core inside the step: bf16 inputs as recorded
    kh, vh, qh = rec["in"]
    assert qh.dtype == torch.bfloat16 and qh.shape == (1, B, T, H, D)
    sub = lambda z: z[:, [0, 31, 63]].contiguous()  # noqa: E731
    ref = run_oracle(sub(qh), sub(kh), sub(vh), sub(rec["gout"]), ace.planes().detach().cpu(), causal=False,
                     inv_temp=rec["inv_temp"])
    dkh, dvh, dqh = rec["gin"]
    errs = {nm: relerr(to64(sub(a)), b) for nm, a, b in
            zip(("out", "dq", "dk", "dv"), (rec["out"], dqh, dkh, dvh), ref[:4])}
    print("[C3 step, block 0 core] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert max(errs.values()) <= TOL[torch.bfloat16]
