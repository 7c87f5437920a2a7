"""Shared helpers for the parity tests (seeded CPU generators, comparisons)."""
import torch


def gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def ref_inputs(batch, columns, rows, maxq, asymmetric, seed):
    """The reference test's block generator (tests/test_triton_compensation.py:70-117),
    drawn from a CPU generator: per-element qparams, weights ±0.25 of a step away
    from rounding boundaries, upper-triangular hinv with diagonal in [0.75, 1.25]."""
    g = gen(seed)
    shape = (batch, columns, rows)
    minq = -(maxq + 1)
    scale = torch.rand(shape, generator=g).mul_(0.15).add_(0.05)
    if asymmetric:
        zero = torch.randint(minq, maxq + 1, shape, generator=g).float()
    else:
        zero = torch.zeros(shape)
    target = torch.randint(minq, maxq + 1, shape, generator=g).float()
    frac = torch.randint(0, 2, shape, generator=g).float().mul_(0.5).sub_(0.25)
    weight = (target - zero + frac) * scale
    hinv = torch.triu(torch.randn(batch, columns, columns, generator=g).mul_(0.002), diagonal=1)
    torch.diagonal(hinv, dim1=1, dim2=2).copy_(torch.rand(batch, columns, generator=g).mul_(0.5).add_(0.75))
    return weight.contiguous(), hinv.contiguous(), scale.contiguous(), zero.contiguous()


def g2_inputs(weight, scale, seed):
    """tests/test_triton_compensation.py:120-132."""
    g = gen(seed)
    z = torch.randn(weight.shape, generator=g).mul_(scale * 0.002)
    gh = torch.randn(weight.shape, generator=g).mul_(scale * 0.002)
    return z.contiguous(), gh.contiguous()


def gptaq_p(weight, seed):
    """tests/test_triton_compensation.py:135-143."""
    g = gen(seed)
    b, c, _ = weight.shape
    return torch.triu(torch.randn(b, c, c, generator=g).mul_(0.002), diagonal=1).contiguous()


def assert_bitexact(actual, expected, what=""):
    a = actual.detach().cpu()
    e = expected.detach().cpu()
    assert a.shape == e.shape, (what, a.shape, e.shape)
    same = (a == e) | (torch.isnan(a) & torch.isnan(e))
    if not bool(same.all()):
        idx = (~same).nonzero()[:5].tolist()
        raise AssertionError(f"{what}: {int((~same).sum())} mismatches, first at {idx}: "
                             f"{[float(a[tuple(i)]) for i in idx]} vs {[float(e[tuple(i)]) for i in idx]}")


def assert_close(actual, expected, rtol, atol, what=""):
    torch.testing.assert_close(actual.detach().cpu().float(), expected.detach().cpu().float(),
                               rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


class StoredQuantizer:
    """Fitted group parameters read back from a fixture (scale, zero, zraw)."""

    def __init__(self, scale, zero, zraw=None):
        self.scale, self.zero, self.zraw = scale, zero, zraw


from oracle.parity import check_flow as assert_flow_parity  # noqa: E402,F401


def assert_beta_close(beta, beta_ref, what):
    """G2PTQ's trust-region β per row within 1e-3 relative plus 2 ulps of 1:
    β = mean_j(1 − √(1 − x_j)) cancels in fp32 for small x_j (the reference
    evaluates it the same way), so each term has an absolute error floor."""
    err = (beta.double() - beta_ref.double()).abs()
    bound = 1e-3 * beta_ref.double().abs() + 2 * torch.finfo(torch.float32).eps
    worst = float((err / bound).max())
    print(f"{what}: beta max |diff| {float(err.max()):.3g}, {worst:.3g} of the bound", flush=True)
    assert worst <= 1.0, (what, worst)
