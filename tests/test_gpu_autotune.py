"""GPU: the G2PTQ α autotune pattern (g2ptq_utils.py:1481-1577) — fasterquant re-run
for several α with the weights and Hessians restored in between — reuses one
factor per Hessian, gives bit-identical weights to a fresh instance per α, and
matches the oracle at every α (trust-region β, end-to-end parity protocol)."""
import pytest
import torch

from oracle import flows as oflows
from oracle import hessian as ohess
from tests._util import assert_beta_close, assert_flow_parity, gen

pytestmark = pytest.mark.gpu


def _setup(dev, seed=900):
    from g2ptq_amd import G2PTQ, WeightQuantizer, make_group_quantizers
    B, R, C, G, T, ch = 2, 64, 256, 2, 1024, 256
    g = gen(seed)
    W = (torch.randn(B, R, C, generator=g) * 0.02).bfloat16()
    X = (torch.randn(T, C, generator=g) * torch.exp(torch.randn(C, generator=g))).bfloat16()
    sal = torch.rand(T, G, generator=g)
    grad = torch.randn(B, R, C, generator=g) * 1e-3
    layers = []
    for b in range(B):
        lin = torch.nn.Linear(C, R, bias=False).to(torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(W[b])
        layers.append(lin.to(dev))
    sals = [[sal[i:i + ch].to(dev) for i in range(0, T, ch)] for _ in range(B)]
    gq = G2PTQ(layers, sals, [grad[b].to(dev) for b in range(B)], G)
    q = WeightQuantizer()
    q.configure(3, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, 128)
    st = ohess.g2ptq_state(B, G, C)
    for i in range(0, T, ch):
        xb = X[i:i + ch].reshape(1, ch, C)
        xd = xb.to(dev)
        for b in range(B):
            gq.add_batch(b, xd, None)
            ohess.g2ptq_add_batch(st, b, xb, sal[i:i + ch])
    gq._oracle = (st, grad)
    return gq, layers, W


def test_alpha_sweep_reuses_factor_and_matches_fresh(dev, monkeypatch):
    from g2ptq_amd import _core, make_group_quantizers
    calls = []
    real = _core.factor

    def counting(H, percdamp, *a, **k):
        calls.append(H.shape)
        return real(H, percdamp, *a, **k)

    monkeypatch.setattr(_core, "factor", counting)
    gq, layers, W0 = _setup(dev)
    saved_H = gq.H.cpu().clone()
    q0 = gq.quantizer[0]
    results = {}
    st, grad = gq._oracle
    for alpha in (0.05, 0.1, 0.2):
        gq.quantizer = make_group_quantizers(q0, 256, 128)
        gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, alpha=alpha, backend="hip",
                       export_compressed_tensors=True)
        torch.cuda.synchronize()
        results[alpha] = torch.stack([l.weight.detach().cpu().clone() for l in layers])
        ref = oflows.g2ptq_fasterquant(W0.float(), st["H"].clone(), grad, st["act_square"], 3,
                                       True, 2, groupsize=128, alpha=alpha)
        assert_beta_close(gq._beta.cpu(), ref["beta"], f"autotune alpha={alpha}")
        assert_flow_parity(f"autotune alpha={alpha}", layers, gq.quantizer, ref, W0.float(),
                           st["H"].reshape(-1, 256, 256), 3, 128, False)
        with torch.no_grad():
            for b, l in enumerate(layers):
                l.weight.copy_(W0[b].to(dev))
        gq.H.copy_(saved_H)
    assert len(calls) == 1, calls  # one factorization for the whole sweep
    # a fresh instance at α = 0.1 (no cache) gives the same bits
    calls.clear()
    fresh, flayers, _ = _setup(dev)
    fresh.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, alpha=0.1, backend="hip")
    torch.cuda.synchronize()
    assert len(calls) == 1
    got = torch.stack([l.weight.detach().cpu() for l in flayers])
    assert torch.equal(got, results[0.1])
    assert not torch.equal(results[0.05], results[0.2])  # α matters
    gq.free()
    assert gq._factor_cache is None
