"""Pins for the oracle's FP8 indexer scores (reference src/attention.py:288-300).

The restatement is checked against what the mathematics fixes, not against a retyping of
its own formula:
- lossless inputs: when every value is an e4m3 number and every 1x128 tile's amax is 448,
  the quantization is the identity (scale 1), so the FP8 scores must equal the reference's
  non-FP8 branch (:302-303, relu(einsum('bthd,bsd')) then einsum('bths,bth') with
  weights * softmax_scale), evaluated here in fp64 as a different formulation; with mixed
  signs over several heads this also fixes that the ReLU acts per head, before the head sum;
- the first-scale rule (:296-297): with d = 192 a row has two 1x128 tiles but only the
  first tile's scale multiplies the codes, so halving the second tile's amax doubles its
  codes' weight in the scores;
- the ReLU itself: scores(q, k) - scores(q, -k) is the weighted sum of the raw logits
  (relu(l) - relu(-l) = l), which a missing ReLU (2x) or an absolute value (0) would not give;
- positive homogeneity in q by powers of two (codes unchanged, scales doubled).
"""
import torch

from oracle import fp8_oracle as orc


def _e4m3_values(shape, g):
    """Random e4m3-representable values with both signs and exponents over a wide range."""
    x = torch.randn(shape, generator=g) * torch.exp2(torch.randint(-6, 4, shape, generator=g).float())
    return x.to(torch.float8_e4m3fn).float()


def _force_tile_amax(x, amax, d):
    """Set one element of every 1x128 tile of the last dim to +-amax (an e4m3 number)."""
    x = x.clone()
    for c in range(0, d, 128):
        x[..., c] = amax * torch.where(x[..., c] < 0, -1.0, 1.0)
        rest = x[..., c + 1:c + 128]
        rest.clamp_(-amax, amax)
    return x


def _textbook(q, k, weights, softmax_scale):
    """The reference's non-FP8 branch (src/attention.py:302-303) in fp64."""
    logits = torch.relu(torch.einsum("bthd,bsd->bths", q.double(), k.double()))
    return torch.einsum("bths,bth->bts", logits, weights.double() * softmax_scale)


def test_lossless_inputs_equal_the_unquantized_formula():
    g = torch.Generator().manual_seed(0)
    for B, L, S, H, d in [(2, 7, 9, 4, 64), (1, 5, 3, 2, 128), (2, 4, 6, 3, 32)]:
        q = _force_tile_amax(_e4m3_values((B, L, H, d), g), 448.0, d)
        k = _force_tile_amax(_e4m3_values((B, S, d), g), 448.0, d)
        w = torch.randn(B, L, H, generator=g)
        scale = d ** -0.5
        got = orc.indexer_scores_fp8_ref(q, k, w, scale).double()
        want = _textbook(q, k, w, scale)
        assert (got - want).abs().max() <= 1e-6 * want.abs().max(), (B, L, S, H, d)


def test_only_the_first_tile_scale_is_used():
    g = torch.Generator().manual_seed(1)
    B, L, S, H, d = 1, 6, 5, 2, 192
    q = _force_tile_amax(_e4m3_values((B, L, H, d), g), 448.0, d)
    q[..., 128:] = _force_tile_amax(_e4m3_values((B, L, H, 64), g).clamp(-224, 224), 224.0, 64)
    k = _force_tile_amax(_e4m3_values((B, S, d), g), 448.0, d)
    w = torch.rand(B, L, H, generator=g)
    # q's second tile has amax 224: its scale is 0.5 and its codes are 2x the values, but the
    # codes are multiplied by the first tile's scale (1.0)
    q_eff = q.clone()
    q_eff[..., 128:] *= 2
    got = orc.indexer_scores_fp8_ref(q, k, w, 0.125).double()
    want = _textbook(q_eff, k, w, 0.125)
    assert (got - want).abs().max() <= 1e-6 * want.abs().max()
    assert (got - _textbook(q, k, w, 0.125)).abs().max() > 1e-3 * want.abs().max()


def test_relu_is_applied_to_the_logits():
    g = torch.Generator().manual_seed(2)
    B, L, S, H, d = 2, 8, 8, 4, 64
    q = torch.randn(B, L, H, d, generator=g)
    k = torch.randn(B, S, d, generator=g)
    w = torch.randn(B, L, H, generator=g)
    diff = (orc.indexer_scores_fp8_ref(q, k, w, 0.1) - orc.indexer_scores_fp8_ref(q, -k, w, 0.1)).double()
    # quantization is sign-symmetric, so the codes of -k are minus the codes of k
    q8, qs = orc.quant_rowwise(q.reshape(-1, d), block_size=128)
    k8, ks = orc.quant_rowwise(k.reshape(-1, d), block_size=128)
    qd = q8.double().view(B, L, H, d) * qs.double().view(B, L, H)[..., None]
    kd = k8.double().view(B, S, d) * ks.double().view(B, S)[..., None]
    linear = torch.einsum("bthd,bsd,bth->bts", qd, kd, w.double() * 0.1)
    assert (diff - linear).abs().max() <= 1e-5 * linear.abs().max()


def test_power_of_two_homogeneity_in_q():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 5, 3, 128, generator=g)
    k = torch.randn(2, 6, 128, generator=g)
    w = torch.randn(2, 5, 3, generator=g)
    base = orc.indexer_scores_fp8_ref(q, k, w, 0.125)
    assert torch.equal(orc.indexer_scores_fp8_ref(q * 4, k, w, 0.125), base * 4)
