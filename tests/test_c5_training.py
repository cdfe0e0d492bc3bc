"""Config 5: training steps of a small MLA + MoE model with FP8 Linear and expert layers.

CPU: the harness model trains (losses finite and falling) and convert_to_fp8 picks the
layers the reference's rules pick (src/kernels.py:863-903).  GPU: 10 AdamW steps at the
config-5 sizes (batch 16 x seq 1024, seed 5) in FP8 mode and in the fp32 reference mode
from the same weights and batches; the loss must agree within 1e-2 relative at every step.
"""
import pytest
import torch

from tests.c5_model import C5Config, C5Model, loss_fn, to_fp8, train

TINY = dict(d_model=128, n_layers=1, vocab_size=256, hidden_dim=512, n_heads=2, d_ckv=64,
            d_cq=64, d_head=32, d_v=32, d_rope=16, n_routed=4, max_seq_len=64)


def test_c5_harness_trains_on_cpu():
    torch.manual_seed(0)
    model = C5Model(C5Config(**TINY))
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 256, (2, 33), generator=g)
    losses, mains, _ = train(model, [ids] * 4)
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < losses[0]
    # uniform-random tokens: the first main loss is near ln(vocab)
    assert abs(mains[0] - torch.log(torch.tensor(256.0)).item()) < 0.5


def test_c5_fp8_conversion_follows_reference_rules():
    from cinnamon_amd import kernels, layers

    torch.manual_seed(0)
    model = to_fp8(C5Model(C5Config(**TINY)))
    fp8 = {n: m for n, m in model.named_modules() if isinstance(m, kernels.FP8Linear)}
    # shared-expert SwiGLU and the MTP projection; attention, router, lm_head stay unquantized
    assert set(fp8) == {"layers.0.moe.shared_experts.0.w1", "layers.0.moe.shared_experts.0.w2",
                        "layers.0.moe.shared_experts.0.w3", "mtp.0.proj",
                        "mtp.0.block.moe.shared_experts.0.w1", "mtp.0.block.moe.shared_experts.0.w2",
                        "mtp.0.block.moe.shared_experts.0.w3"}
    assert fp8["layers.0.moe.shared_experts.0.w1"].round_scale
    assert not fp8["layers.0.moe.shared_experts.0.w3"].round_scale
    assert not fp8["mtp.0.proj"].round_scale
    experts = [m for m in model.modules() if isinstance(m, layers.GroupedExperts)]
    assert len(experts) == 2
    # same function as the unconverted model on the CPU (FP8Linear's CPU branch is F.linear)
    ids = torch.randint(0, 256, (2, 17), generator=torch.Generator().manual_seed(2))
    torch.manual_seed(0)
    ref = C5Model(C5Config(**TINY))
    with torch.no_grad():
        a, _ = loss_fn(ref, ids)
        b, _ = loss_fn(model, ids)
    assert torch.allclose(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
def test_c5_fp8_training_matches_reference(dev):
    c = C5Config()
    torch.manual_seed(5)
    base = C5Model(c)
    g = torch.Generator().manual_seed(5)
    batches = [torch.randint(0, c.vocab_size, (16, 1025), generator=g) for _ in range(10)]
    batches = [b.to(dev) for b in batches]
    print(f"\nC5: {sum(p.numel() for p in base.parameters()) / 1e6:.0f}M parameters, "
          f"batch 16 x 1024, 10 steps", flush=True)
    ref = base.to(dev)
    fp8 = to_fp8(ref)
    sync = torch.cuda.synchronize
    l8, m8, t8 = train(fp8, batches, sync)
    del fp8
    torch.cuda.empty_cache()
    lr, mr, tr = train(ref, batches, sync)
    tok = 16 * 1024
    print(f"C5 fp8 loss {['%.4f' % v for v in l8]}", flush=True)
    print(f"C5 ref loss {['%.4f' % v for v in lr]}", flush=True)
    print(f"C5 tokens/s (steps 2-10): fp8 {tok * 9 / sum(t8[1:]):.0f}, "
          f"fp32 reference {tok * 9 / sum(tr[1:]):.0f}", flush=True)
    for i, (a, b) in enumerate(zip(l8, lr)):
        assert abs(a - b) / b <= 1e-2, f"step {i}: fp8 loss {a} vs reference {b}"
    assert l8[-1] < l8[0]
