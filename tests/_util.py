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


def first_divergence_ties(codes_a, codes_b, x_over_s, tol=1e-4):
    """For each row whose codes differ, check the first differing element is a
    near-tie (|frac(x/s) - 0.5| < tol).  Returns (rows_diverged, non_tie_rows)."""
    a = codes_a.reshape(-1, codes_a.shape[-1]).cpu()
    b = codes_b.reshape(-1, codes_b.shape[-1]).cpu()
    r = x_over_s.reshape(-1, x_over_s.shape[-1]).cpu().double()
    diff = a != b
    rows = diff.any(1).nonzero().flatten().tolist()
    bad = []
    for row in rows:
        j = int(diff[row].nonzero()[0])
        f = float(r[row, j] - torch.floor(r[row, j]))
        if abs(f - 0.5) >= tol:
            bad.append((row, j, f))
    return rows, bad
