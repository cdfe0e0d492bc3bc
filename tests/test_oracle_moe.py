"""Pins of the oracle's MoE dispatch / combine restatement (reference src/layers.py:126-157).

The reference's own tests hold no MoE dispatch fixtures, so the restatement is pinned by:
- hand-computed known answers;
- an independent brute-force stable sort;
- an order-exact scalar loop for the combine;
- conservation identities (unit gates sum the expert rows; a 0/1 one-hot gate picks one
  row).
"""
import torch

from oracle import fp8_oracle as orc


def test_dispatch_known_answer():
    # expanded ids [2, 0, 0, 1, 2, 2]: id 0 at 1, 2; id 1 at 3; id 2 at 0, 4, 5
    top_idx = torch.tensor([[2, 0], [0, 1], [2, 2]])
    order, tok, counts, starts, ends = orc.moe_dispatch_ref(top_idx, 4)
    assert order.tolist() == [1, 2, 3, 0, 4, 5]
    assert tok.tolist() == [0, 1, 1, 0, 2, 2]
    assert counts.tolist() == [2, 1, 3, 0]
    assert starts.tolist() == [0, 2, 3, 6] and ends.tolist() == [2, 3, 6, 6]


def test_dispatch_is_the_stable_sort():
    g = torch.Generator().manual_seed(0)
    for T, k, E in [(1, 1, 1), (7, 3, 5), (300, 8, 32), (1000, 2, 17)]:
        top_idx = torch.randint(0, E, (T, k), generator=g)
        order, tok, counts, starts, ends = orc.moe_dispatch_ref(top_idx, E)
        ids = top_idx.reshape(-1).tolist()
        brute = sorted(range(T * k), key=lambda i: (ids[i], i))
        assert order.tolist() == brute
        assert tok.tolist() == [i // k for i in brute]
        for e in range(E):
            assert counts[e] == ids.count(e)
            assert all(ids[order[r]] == e for r in range(int(starts[e]), int(ends[e])))


def test_combine_known_answer_and_order():
    # 3 tokens, k = 2, ids [[1, 0], [0, 1], [1, 1]]; sorted rows carry their own values
    top_idx = torch.tensor([[1, 0], [0, 1], [1, 1]])
    scores = torch.tensor([[0.5, 0.25], [2.0, 1.0], [1.0, 3.0]])
    order, *_ = orc.moe_dispatch_ref(top_idx, 2)
    assert order.tolist() == [1, 2, 0, 3, 4, 5]
    y = torch.arange(6, dtype=torch.float32).unsqueeze(1) * torch.tensor([[1.0, 10.0]])
    out = orc.moe_combine_ref(y, scores, order, 3)
    # token 0: slot 1 (id 0) at row 0, slot 0 (id 1) at row 2 -> 0.25*y0 + 0.5*y2
    # token 1: slot 0 at row 1, slot 1 at row 3 -> 2*y1 + 1*y3
    # token 2: slots 0, 1 at rows 4, 5 -> 1*y4 + 3*y5
    want = torch.tensor([[0.25 * 0 + 0.5 * 2, 10 * (0.5 * 2)], [2 * 1 + 3, 10 * (2 * 1 + 3)],
                         [4 + 3 * 5, 10 * (4 + 3 * 5)]])
    assert torch.equal(out, want)


def test_combine_adds_in_sorted_position_order():
    g = torch.Generator().manual_seed(1)
    T, k, E, D = 200, 4, 9, 33
    top_idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    scores = torch.rand(T, k, generator=g).to(torch.bfloat16)
    y = torch.randn(T * k, D, generator=g)
    order, *_ = orc.moe_dispatch_ref(top_idx, E)
    out = orc.moe_combine_ref(y, scores, order, T)
    # scalar restatement: fp32 products, then fp32 adds in increasing sorted position
    pos = torch.empty(T * k, dtype=torch.long)
    pos[order] = torch.arange(T * k)
    want = torch.zeros(T, D)
    for t in range(T):
        terms = sorted((int(pos[t * k + j]), j) for j in range(k))
        for r, j in terms:
            want[t] = want[t] + y[r] * scores[t, j].float()
    assert torch.equal(out, want)


def test_combine_conservation():
    g = torch.Generator().manual_seed(2)
    T, k, E, D = 64, 3, 6, 8
    top_idx = torch.randint(0, E, (T, k), generator=g)
    y = torch.randn(T * k, D, generator=g, dtype=torch.float64)
    order, tok, *_ = orc.moe_dispatch_ref(top_idx, E)
    ones = torch.ones(T, k, dtype=torch.float64)
    out = orc.moe_combine_ref(y, ones, order, T)
    assert torch.allclose(out.sum(0), y.sum(0))
    # a one-hot gate on slot 0 returns the sorted row holding each token's slot 0
    onehot = torch.zeros(T, k, dtype=torch.float64)
    onehot[:, 0] = 1
    pos = torch.empty(T * k, dtype=torch.long)
    pos[order] = torch.arange(T * k)
    assert torch.equal(orc.moe_combine_ref(y, onehot, order, T), y[pos.view(T, k)[:, 0]])
