"""CPU pins of the MoE oracle (oracle/fp8_moe.py): the routed FP8 expert MLP
tracks an fp32 autograd of the same experts within the reference test's
bound (tests/test_fp8_mlp.py:57-109), an expert without tokens gets exactly
zero gradients, and planted mistakes fail the bound."""
import pytest
import torch

from oracle import fp8_mlp as O
from oracle import fp8_moe as M


def _case(seed=0, T=500, D=256, I=128, E=4, k=2):
    g = torch.Generator().manual_seed(seed)
    w_gu = torch.randn(E, 2 * I, D, generator=g) * 0.05
    w_d = torch.randn(E, D, I, generator=g) * 0.05
    x = torch.randn(T, D, generator=g).to(torch.bfloat16)
    # expert 2 gets no tokens; each token picks two distinct experts from {0, 1, 3}
    choices = torch.tensor([[0, 1], [1, 3], [0, 3]])
    selected = choices[torch.randint(0, 3, (T,), generator=g)]
    weights = torch.softmax(torch.randn(T, k, generator=g), -1).to(torch.bfloat16)
    probe = torch.randn(T, D, generator=g)
    return x, w_gu, w_d, selected, weights, probe


def oracle_step(x, w_gu, w_d, selected, weights, probe, scale, amax, planted=None):
    E, k = w_gu.shape[0], selected.shape[1]
    tok, inv, offsets, perm = M.route(selected, E)
    sw = weights.reshape(-1)[perm]
    rows, saved = M.moe_forward(x, w_gu, w_d, tok, offsets, scale, amax)
    if planted == "unweighted":
        sw = torch.ones_like(sw)
    y = M.combine_topk(rows, sw, inv, k)
    d_rows = M.combine_topk_backward(probe.to(torch.bfloat16), sw, tok)
    if planted == "rows_not_tokens":
        d_rows = probe.to(torch.bfloat16)[: d_rows.shape[0] // k].repeat(k, 1)
    (dx, dwgu, dwd), _ = M.moe_backward(d_rows, saved, scale, amax, inv, k)
    if planted == "swapped_experts":
        dwgu = dwgu.flip(0)
    return y, dx, dwgu, dwd


def _run(planted=None):
    x, w_gu, w_d, selected, weights, probe = _case()
    scale, amax = torch.ones(5), torch.zeros(5)
    oracle_step(x, w_gu, w_d, selected, weights, probe, scale, amax)
    assert bool((amax > 0).all()), amax
    O.update_scales(scale, amax)
    out = oracle_step(x, w_gu, w_d, selected, weights, probe, scale, amax, planted)
    ref = M.fp32_experts_reference(x, selected, weights, w_gu, w_d, probe)
    return out, ref


def test_moe_oracle_tracks_fp32_reference():
    out, ref = _run()
    for name, a, r in zip(("out", "dx", "dW_gate_up", "dW_down"), out, ref):
        assert torch.isfinite(a.float()).all(), name
        assert O.rel_l2(a.float(), r) < 0.12, name
    assert torch.equal(out[2][2], torch.zeros_like(out[2][2]))  # expert 2 has no tokens
    assert torch.equal(out[3][2], torch.zeros_like(out[3][2]))


@pytest.mark.parametrize("planted", ["unweighted", "rows_not_tokens", "swapped_experts"])
def test_moe_oracle_planted_mistakes_fail(planted):
    out, ref = _run(planted)
    assert max(O.rel_l2(a.float(), r) for a, r in zip(out, ref)) > 0.12


def test_route_matches_reference_bookkeeping():
    """token_index / inverse_permutation / offsets as train.py:2268-2290."""
    selected = torch.tensor([[2, 0], [1, 2], [0, 1]])
    tok, inv, offsets, perm = M.route(selected, 4)
    assert offsets.tolist() == [2, 4, 6, 6]
    assert tok.tolist() == [0, 2, 1, 2, 0, 1]
    # inverse_permutation[t*k + s] is the expert-order row of token t's slot s
    for t in range(3):
        for s in range(2):
            r = int(inv[t * 2 + s])
            assert int(tok[r]) == t
