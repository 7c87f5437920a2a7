"""GPU: the fused weighted Gram (g2ptq_weighted_stage / _gram) against fp64 sums.

H[g] = beta·H[g] + alpha·Σ_t S[t,g]·s_scale·x_t·x_tᵀ (g2ptq_utils.py:182-201,
gptq_guided_utils.py:59-81), every group of a linear in one launch.  The cases
reach each launch shape of the kernel: one split per tile with beta applied in
the kernel's own epilogue (the grid of tiles × groups alone fills the GPU, or
too few tokens to split), a split chain cut in two and reduced with beta,
ragged feature counts (a partial 256-tile),
token counts that are not a multiple of the 64-token staging grid, a single
token, and the maximum of 64 groups.  The bar is the module's 2e-5 of
sqrt(H_ii·H_jj) in fp64 (the hi/lo split of x·s carries 16 significant bits),
and every group must be exactly symmetric.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _stage_and_gram(X, S, s_scale, alpha, beta, H0):
    from g2ptq_amd import _lib
    dev = X.device
    T, C = X.shape
    G = S.shape[1]
    st = _lib.stream_ptr()
    height = _lib.query_size_i64("g2ptq_hessian_stage_height", 2, 0, C, G)
    ldt = ((T + 63) // 64 * 64 + 2048 + 1024 + 7) // 8 * 8
    XT = torch.full((height, ldt), float("nan"), dtype=torch.bfloat16, device=dev)
    p = _lib.ptr
    _lib.call("g2ptq_weighted_stage", st, p(X), T, C, C, p(S), G, G, s_scale, p(XT), ldt, 0,
              None, 0.0, 1.0)
    ws = torch.empty(max(_lib.query_size("g2ptq_weighted_gram_workspace", T, C, G), 256),
                     dtype=torch.uint8, device=dev)
    H = H0.clone()
    _lib.call("g2ptq_weighted_gram", st, p(XT), ldt, T, C, G, alpha, beta, p(H), C, C * C, p(ws),
              ws.numel())
    torch.cuda.synchronize()
    return H


def _check(X, S, s_scale, alpha, beta, H0, H, what):
    T, C = X.shape
    G = S.shape[1]
    Xd = X.double()
    w = (S * s_scale).double()  # the staged weights are fp32(S·s_scale)
    worst = 0.0
    for g in range(G):
        ref = beta * H0[g].double() + alpha * ((Xd * w[:, g:g + 1]).T @ Xd)
        d = alpha * ((Xd * Xd) * w[:, g:g + 1]).sum(0) + abs(beta) * torch.diagonal(
            H0[g].double()).abs()
        scale = torch.sqrt(d[:, None] * d[None, :]).clamp_min(1e-30)
        worst = max(worst, ((H[g].double() - ref).abs() / scale).max().item())
        assert torch.equal(H[g], H[g].T), f"{what}: group {g} not symmetric"
    print(f"{what}: max |H − fp64| / sqrt(H_ii·H_jj) = {worst:.3g}", flush=True)
    assert worst <= 2e-5, (what, worst)


def _inputs(T, C, G, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    sig = torch.exp(torch.randn(C, device=dev, generator=g))
    X = (torch.randn(T, C, device=dev, generator=g) * sig).bfloat16()
    S = torch.rand(T, G, device=dev, generator=g) * 3 + 0.05
    return X, S


@pytest.mark.parametrize("T,C,G,beta", [
    (4096, 2600, 64, 0.5),   # 66 tiles × 64 groups fill the GPU: one split, beta in the epilogue
    (777, 1000, 3, 0.25),    # ragged C and T (too few tokens to split)
    (40000, 2600, 64, 0.5),  # one split would be a 40000-token chain: cut in two, reduced
    (1, 300, 2, 1.0),        # a single token
])
def test_weighted_gram_against_fp64(dev, T, C, G, beta):
    X, S = _inputs(T, C, G, 1000 + C + G, dev)
    H0 = torch.zeros(G, C, C, device=dev)
    if beta:
        Y = torch.randn(G, C, C, device=dev, generator=torch.Generator(device=dev).manual_seed(7))
        H0 = (Y + Y.transpose(1, 2)) / 2 + C * torch.eye(C, device=dev)
    s_scale, alpha = 1.0 / max(T, 1), 0.75
    H = _stage_and_gram(X, S, s_scale, alpha, beta, H0)
    _check(X, S, s_scale, alpha, beta, H0, H, f"T={T} C={C} G={G} beta={beta}")


def test_weighted_gram_groups_are_independent(dev):
    """Each group's Hessian depends only on its own weights: the G = 5 launch
    equals five G = 1 launches of the same tokens bit for bit (a tile's groups
    share panels and the XCD order, never accumulators)."""
    T, C, G = 2048, 700, 5
    X, S = _inputs(T, C, G, 31, dev)
    H0 = torch.zeros(G, C, C, device=dev)
    Hall = _stage_and_gram(X, S, 1.0 / T, 1.0, 0.0, H0)
    for g in range(G):
        Hg = _stage_and_gram(X, S[:, g:g + 1].contiguous(), 1.0 / T, 1.0, 0.0, H0[:1])
        # one group has fewer work items, so its split plan may differ: compare
        # against fp64 instead when it does
        from g2ptq_amd import _lib
        same_plan = (_lib.query_size("g2ptq_weighted_gram_workspace", T, C, 1) * G
                     == _lib.query_size("g2ptq_weighted_gram_workspace", T, C, G))
        if same_plan:
            assert torch.equal(Hg[0], Hall[g]), g
        else:
            _check(X, S[:, g:g + 1], 1.0 / T, 1.0, 0.0, H0[:1], Hg, f"group {g} alone")
