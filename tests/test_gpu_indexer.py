"""FP8 indexer scores (GPU) against the oracle's restatement of the reference's FP8 branch
of DSAIndexer.forward (src/attention.py:288-300).

The codes and scales come from the row-wise quantizer (bit-exact with the oracle, checked
in test_gpu_quant.py), so the scores differ from the oracle only in the code dot products.
Each product of two e4m3 codes is exact in fp32, and the oracle's fp32 einsum is within
1e-7 (normwise) of an exact fp64 evaluation on these inputs. The kernel sums the products
with v_mfma_f32_16x16x128_f8f6f4, whose product sums inside one instruction are not exact
fp32 sums: measured 1.3e-5 to 2.4e-5 of the largest score (normwise) and 1.1e-5 to
1.9e-5 (Frobenius) over these cases. Tolerance: max |error| <= 1e-4 * max |reference|
(normwise) and Frobenius relative error <= 5e-5, 20x tighter than the FP8 GEMM bar (2e-3
and 1e-3). The weights gradient (the
reference's autograd through the same branch) is held to the same bounds.
"""
import pytest
import torch

from cinnamon_amd import kernels
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def _inputs(B, L, S, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, H, d, generator=g).to(dtype)
    k = torch.randn(B, S, d, generator=g).to(dtype)
    w = torch.randn(B, L, H, generator=g) * H ** -0.5
    return q, k, w


def _check(got, want):
    got, want = got.detach(), want.detach()
    assert got.shape == want.shape and got.dtype == torch.float32
    normwise = float((got - want).abs().max() / want.abs().max())
    frob = orc.frob_rel(got, want)
    print(f"normwise {normwise:.3g} frobenius {frob:.3g}")
    assert normwise <= 1e-4 and frob <= 5e-5


@pytest.mark.parametrize("B,L,S,H,d,dtype", [
    (2, 1024, 1024, 4, 128, torch.bfloat16),   # the indexer with PoPE (d_rope 64 -> 128)
    (3, 512, 512, 4, 64, torch.bfloat16),      # RoPE, d_indexer_head 64
    (1, 77, 130, 3, 192, torch.float32),       # ragged tiles, two 1x128 tiles per row
    (2, 65, 63, 1, 32, torch.float16),
    (1, 200, 64, 8, 256, torch.bfloat16),
])
def test_scores_match_the_oracle(dev, B, L, S, H, d, dtype):
    q, k, w = _inputs(B, L, S, H, d, dtype, seed=B * 1000 + L + d)
    scale = d ** -0.5
    got = kernels.indexer_scores_fp8(q.to(dev), k.to(dev), w.to(dev), scale).cpu()
    _check(got, orc.indexer_scores_fp8_ref(q, k, w, scale))


@pytest.mark.parametrize("B,L,S,H,d,dtype", [
    (2, 1024, 1024, 4, 128, torch.bfloat16),   # the config-5 shape: two key ranges per token tile
    (2, 100, 300, 4, 128, torch.float16),
    (2, 70, 513, 3, 96, torch.float32),        # ragged token and key tiles, a partial 1x128 tile
    (1, 130, 700, 2, 256, torch.bfloat16),     # two 1x128 tiles per row
    (2, 65, 1030, 2, 160, torch.float32),      # three key ranges, the second tile 32 wide
    (1, 64, 5, 1, 32, torch.float16),          # S % 4 != 0: the scalar score stores
    (1, 33, 0, 2, 64, torch.bfloat16),         # no keys: only the codes are written
    # the 8-wave form (d <= 128, S > 512): a second half with 1 key, an empty second half in
    # the last 1024-key range, three ranges, one head
    (3, 100, 600, 4, 128, torch.bfloat16),
    (1, 200, 1500, 4, 64, torch.float16),
    (1, 77, 2049, 2, 32, torch.bfloat16),
    (2, 64, 1088, 1, 128, torch.float32),
])
def test_fused_q_quantization_equals_the_two_calls(dev, B, L, S, H, d, dtype):
    """cin_indexer_scores_fp8_q quantizes q inside the scoring kernel with the row-wise
    quantizer's arithmetic: its scores must equal, bit for bit, cin_indexer_quantize +
    cin_indexer_scores_fp8 on the same inputs, and the codes and first scales it writes
    (save_q) must equal cin_indexer_quantize's.  q carries NaN and +-inf elements: a 16-bit
    lane holding a NaN takes the maxnum path, an infinite amax the division path."""
    q, k, w = _inputs(B, L, S, H, d, dtype, seed=B * 7 + L + S + d)
    flat = q.view(-1)
    flat[::97] *= 50
    flat[5::1031] = float("nan")
    flat[7::2063] = float("inf")
    flat[9::4099] = -float("inf")
    q, k, w = q.to(dev), k.to(dev), w.to(dev)
    ops = torch.ops.cinnamon_amd
    q8, qs, k8, ks = ops.indexer_quantize(q, k)
    want = ops.indexer_scores_fp8(q8, qs, k8, ks, w, 0.125)
    k8b, ksb = ops.indexer_quantize_k(k, H)
    assert torch.equal(k8b.view(torch.uint8), k8.view(torch.uint8)) and torch.equal(ksb, ks)
    for save in (True, False):
        got, q8b, qsb = ops.indexer_scores_fp8_q(q, k8b, ksb, w, 0.125, save)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))  # NaN scores too
        if save:
            assert torch.equal(q8b.view(torch.uint8), q8.view(torch.uint8)) and torch.equal(qsb, qs)
        else:
            assert q8b.numel() == 0 and qsb.numel() == 0


@pytest.mark.parametrize("B,L,S,H,d", [(2, 1024, 1024, 4, 128), (1, 77, 2049, 2, 32), (2, 70, 600, 3, 96)])
def test_codes_entry_matches_the_oracle(dev, B, L, S, H, d):
    """cin_indexer_scores_fp8 on codes (the C entry for callers that quantize q themselves;
    8 waves per 1024 keys at these shapes) against the oracle, same bounds as above."""
    q, k, w = _inputs(B, L, S, H, d, torch.bfloat16, seed=B * 31 + L + S)
    ops = torch.ops.cinnamon_amd
    q8, qs, k8, ks = ops.indexer_quantize(q.to(dev), k.to(dev))
    got = ops.indexer_scores_fp8(q8, qs, k8, ks, w.to(dev), 0.125).cpu()
    _check(got, orc.indexer_scores_fp8_ref(q, k, w, 0.125))


def test_zero_rows_and_negative_weights(dev):
    q, k, w = _inputs(2, 100, 96, 4, 64, torch.bfloat16, seed=7)
    q[0, 3] = 0          # all heads of one query: zero row -> floor scale, zero scores
    k[1, 10:20] = 0      # zero keys
    w[:, :, 1] *= -1     # the reference's weights are a signed projection
    got = kernels.indexer_scores_fp8(q.to(dev), k.to(dev), w.to(dev), 0.125).cpu()
    want = orc.indexer_scores_fp8_ref(q, k, w, 0.125)
    _check(got, want)
    assert torch.equal(got[0, 3], torch.zeros(96)) and torch.equal(got[1, :, 10:20], torch.zeros(100, 10))


@pytest.mark.parametrize("B,L,S,H,d", [(2, 1024, 1024, 4, 128), (1, 77, 700, 3, 192), (2, 65, 63, 8, 64),
                                       (1, 130, 1100, 5, 256),
                                       # the 8-wave form: finished in place (S <= 1024), and
                                       # per-range sums with a one-key last range
                                       (2, 70, 600, 3, 96), (1, 77, 2049, 2, 32)])
def test_weights_gradient_matches_the_reference_autograd(dev, B, L, S, H, d):
    """The reference's autograd through its FP8 branch reaches `weights` only (the codes come
    from the quantizer); the oracle's restatement run under CPU autograd is the reference.
    Same tolerance as the scores: the logits inside the gradient come from the FP8 MFMA."""
    q, k, w = _inputs(B, L, S, H, d, torch.bfloat16, seed=B + L + S + d)
    g = torch.randn(B, L, S, generator=torch.Generator().manual_seed(5))
    scale = d ** -0.5
    qd = q.to(dev).requires_grad_(True)
    kd = k.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    kernels.indexer_scores_fp8(qd, kd, wd, scale).backward(g.to(dev))
    assert qd.grad is None and kd.grad is None
    wr = w.clone().requires_grad_(True)
    orc.indexer_scores_fp8_ref(q, k, wr, scale).backward(g)
    _check(wd.grad.cpu(), wr.grad)


def test_decode_shapes_bf16_weights_and_strided_inputs(dev):
    """One query token (decode), one key, 16 heads; bf16 weights (the gradient comes back
    in bf16); q and k as strided views of wider buffers."""
    g = torch.Generator().manual_seed(12)
    for B, L, S, H, d in [(3, 1, 1, 16, 64), (2, 1, 300, 16, 128), (1, 5, 1, 2, 32)]:
        qb = torch.randn(B, L, H, d + 32, generator=g).to(torch.bfloat16)
        kb = torch.randn(B, S, d + 64, generator=g).to(torch.bfloat16)
        q, k = qb[..., 16:16 + d], kb[..., 32:32 + d]
        w = (torch.randn(B, L, H, generator=g) * 0.3).to(torch.bfloat16)
        gs = torch.randn(B, L, S, generator=g)
        wd = w.to(dev).requires_grad_(True)
        got = kernels.indexer_scores_fp8(qb.to(dev)[..., 16:16 + d], kb.to(dev)[..., 32:32 + d], wd, d ** -0.5)
        got.backward(gs.to(dev))
        wr = w.float().requires_grad_(True)
        want = orc.indexer_scores_fp8_ref(q.contiguous(), k.contiguous(), wr, d ** -0.5)
        want.backward(gs)
        _check(got.cpu(), want)
        assert wd.grad.dtype == torch.bfloat16
        assert _close_bf16(wd.grad.cpu(), wr.grad)


def _close_bf16(got, want):
    """bf16 gradient: within one bf16 rounding of the fp32 reference gradient (plus the
    kernel's fp32 tolerance)."""
    return bool(((got.float() - want).abs() <= 2 ** -8 * want.abs() + 1e-4 * want.abs().max()).all())


def test_weights_gradient_is_deterministic(dev):
    q, k, w = _inputs(2, 300, 1500, 4, 128, torch.bfloat16, seed=9)
    g = torch.randn(2, 300, 1500, generator=torch.Generator().manual_seed(10)).to(dev)
    grads = []
    for _ in range(2):
        wd = w.to(dev).requires_grad_(True)
        kernels.indexer_scores_fp8(q.to(dev), k.to(dev), wd, 0.125).backward(g)
        grads.append(wd.grad)
    assert torch.equal(grads[0], grads[1])


@pytest.mark.parametrize("rows,d,dtype", [(300, 128, torch.bfloat16), (77, 192, torch.float32),
                                          (65, 96, torch.float16), (5, 256, torch.bfloat16),
                                          (6000, 128, torch.bfloat16), (6000, 192, torch.float32)])
@pytest.mark.parametrize("kdtype", [None, torch.float32])
def test_indexer_quantize_equals_the_rowwise_quantizer(dev, rows, d, dtype, kdtype):
    """Codes and first scales equal quantize_fp8_rowwise(block 128) and its [..., 0]: q and k
    of one dtype in the one-launch kernel (k 16 lanes per tile, q 8), of two dtypes in two
    launches (16 lanes per tile below 32768 tiles, 8 above)."""
    g = torch.Generator().manual_seed(rows + d)
    q = (torch.randn(2, rows, 3, d, generator=g) * 4).to(dtype).to(dev)
    k = (torch.randn(2, rows + 7, d, generator=g) * 4).to(kdtype or dtype).to(dev)
    q[0, 1] = 0  # zero rows take the floor scale
    q8, qs, k8, ks = torch.ops.cinnamon_amd.indexer_quantize(q, k)
    for x, c, sc in ((q, q8, qs), (k, k8, ks)):
        rq, rs = kernels.quantize_fp8_rowwise(x.reshape(-1, d), block_size=128)
        assert torch.equal(c.reshape(-1, d).view(torch.uint8), rq.view(torch.uint8))
        assert torch.equal(sc.reshape(-1), rs[:, 0])


def test_rejects_unsupported_head_dims(dev):
    q = torch.randn(1, 8, 2, 48, device=dev)
    k = torch.randn(1, 8, 48, device=dev)
    w = torch.randn(1, 8, 2, device=dev)
    with pytest.raises(AssertionError):
        kernels.indexer_scores_fp8(q, k, w, 0.1)
