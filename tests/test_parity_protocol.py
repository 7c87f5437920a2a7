"""CPU: the end-to-end parity checker (oracle.parity) itself.

The checker must pass two runs whose Hessians differ at the level of fp32
summation order, and it must fail runs that differ by a real mistake (a wrong
damp, a dropped compensation term, a wrong zero-point rounding) or by a
perturbation larger than its tie window.
"""
import torch

from oracle import flows as oflows
from oracle import parity
from tests._util import gen


def _setup(seed, C=256, R=64, B=1, T=1024):
    g = gen(seed)
    sig = torch.exp(torch.randn(C, generator=g))
    X = (torch.randn(T, C, generator=g) * sig).bfloat16().double()
    H = ((2.0 / T) * X.T @ X).float().unsqueeze(0).repeat(B, 1, 1)
    W = (torch.randn(B, R, C, generator=g) * 0.02).bfloat16().float()
    return W, H


def _report(a, b, groupsize=128, static=False):
    B, R, C = a["Q"].shape
    N = B * R
    perm = a["perm"]
    ca = parity.loop_order(a["W_int"].reshape(N, C), perm)
    cb = parity.loop_order(b["W_int"].reshape(N, C), perm)
    sa, za, zraw = parity.element_params(a["quantizers"], N, C, groupsize, static, perm, "zraw")
    sb, zb = parity.element_params(b["quantizers"], N, C, groupsize, static, perm)
    return parity.stage_b(cb, ca, a["loop"]["X"].reshape(N, C), sb, sa, zb, za,
                          parity.loop_order(a["Q"].reshape(N, C), perm), zraw_ref=zraw)


def test_identical_runs_pass():
    W, H = _setup(1)
    a = oflows.gptq_fasterquant(W, H, 4, False, groupsize=128)
    b = oflows.gptq_fasterquant(W, H, 4, False, groupsize=128)
    rep = _report(a, b)
    assert rep["ok"] and rep["rows_diverged"] == 0
    parity.check_stage_b(rep)


def _perturbed_runs(rel, seeds):
    """Oracle flows on a Hessian and on the same Hessian times (1 + rel·N(0,1))."""
    out = []
    for seed in seeds:
        W, H = _setup(seed, C=512, R=256)
        Hp = H * (1 + rel * torch.randn(H.shape, generator=gen(100 + seed)))
        Hp = 0.5 * (Hp + Hp.transpose(-1, -2))
        for sym in (True, False):
            a = oflows.gptq_fasterquant(W, H, 4, sym, groupsize=128)
            b = oflows.gptq_fasterquant(W, Hp, 4, sym, groupsize=128)
            out.append(_report(a, b))
    return out


def test_rounding_level_perturbation_diverges_only_at_ties():
    """Hessian entries moved by 1e-5 relative (ten times what fp32 summation
    order does to a few thousand tokens) change codes only where the oracle's
    value was within 1e-4 of a rounding tie, and some rows do diverge."""
    reps = _perturbed_runs(1e-5, (2, 3))
    for rep in reps:
        assert rep["ok"], rep["reasons"]
    assert sum(r["rows_diverged"] for r in reps) >= 1


def test_large_perturbation_is_not_a_tie():
    """Hessian entries moved by 1e-4 relative move values by more than the tie
    window: the checker reports first divergences away from ties."""
    reps = _perturbed_runs(1e-4, (2, 3))
    assert any(not r["ok"] for r in reps)


def test_wrong_damp_fails():
    """A planted mistake: the other side damps with 0.02 instead of 0.01."""
    W, H = _setup(7)
    a = oflows.gptq_fasterquant(W, H, 4, True, groupsize=128)
    b = oflows.gptq_fasterquant(W, H, 4, True, groupsize=128, percdamp=0.02)
    rep = _report(a, b)
    assert not rep["ok"]
    assert any("not a rounding tie" in r for r in rep["reasons"])


def test_dropped_block_tail_fails():
    """A planted mistake: the other side skips the block-tail update of the
    first block (W[:, 128:] −= E·U[:128, 128:])."""
    W, H = _setup(8)
    a = oflows.gptq_fasterquant(W, H, 4, True, groupsize=128)
    Hd = H.clone()
    # a Hessian without coupling between the first block and the rest has a
    # factor whose off-diagonal block U[:128, 128:] is zero
    Hd[:, :128, 128:] = 0
    Hd[:, 128:, :128] = 0
    b = oflows.gptq_fasterquant(W, Hd, 4, True, groupsize=128)
    rep = _report(a, b)
    assert not rep["ok"]


def test_wrong_zero_point_rounding_fails():
    """A planted mistake: the other side's asymmetric zero points round half
    away from zero (x.5 → up) instead of half to even, and its scales are
    1e-2 off: both float checks and the zero-point check fire."""
    W, H = _setup(9)
    a = oflows.gptq_fasterquant(W, H, 4, False, groupsize=-1)
    b = oflows.gptq_fasterquant(W, H, 4, False, groupsize=-1)
    q = b["quantizers"][0]
    q.zero = torch.floor(q.zraw + 0.5).clamp(-8, 7)
    q.scale = q.scale * 1.01
    rep = _report(a, b, groupsize=-1)
    assert not rep["ok"]
    assert any("scale relative error" in r for r in rep["reasons"])


def test_unpack_codes_layout():
    """Field i of word w is column w·(32/bits) + i, offset by 2^(bits−1)."""
    for bits in (2, 3, 4, 8):
        pf = 32 // bits
        codes = torch.arange(2 * pf + 1) % (1 << bits) - (1 << (bits - 1))
        words = []
        for w0 in range(0, codes.numel(), pf):
            v = 0
            for i, c in enumerate(codes[w0:w0 + pf].tolist()):
                v |= (c + (1 << (bits - 1))) << (bits * i)
            words.append(v - (1 << 32) if v >= 1 << 31 else v)
        packed = torch.tensor([words], dtype=torch.int32)
        assert torch.equal(parity.unpack_codes(packed, bits, codes.numel())[0], codes)
