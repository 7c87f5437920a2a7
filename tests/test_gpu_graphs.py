"""GPU: ``graph=True`` (HIP-graph replay) gives, on every replay, exactly what the eager
path gives — replays run with other eager work and synchronisations in between
(the reference's graph path: gptq_utils/graph_utils.py:53-101)."""
import copy

import pytest
import torch

from tests._util import assert_bitexact, gen, ref_inputs

pytestmark = pytest.mark.gpu


def _quantizers(bits, sym, C, groupsize):
    from g2ptq_amd import WeightQuantizer, make_group_quantizers
    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=sym)
    return make_group_quantizers(q, C, groupsize)


def _factor(B, C, seed, dev):
    g = gen(seed)
    X = torch.randn(3 * C, C, generator=g) * torch.exp(0.5 * torch.randn(C, generator=g))
    H = (2 / X.shape[0]) * X.T @ X
    U = torch.linalg.cholesky(torch.linalg.inv(H.double() + 0.01 * H.diag().mean() *
                                               torch.eye(C, dtype=torch.float64)), upper=True)
    return U.float().expand(B, C, C).contiguous().to(dev)


def _run(cls, dev, W, U, extra, groupsize, static, graph):
    from g2ptq_amd import G2PTQ, GPTAQ, GPTQ
    B, R, C = W.shape
    r = object.__new__(cls)
    r.columns, r.num_layers, r.rows = C, B, R
    r.quantizer = _quantizers(4, True, C, groupsize)
    if static:
        for i, q in enumerate(r.quantizer):
            q.find_params(W[:, :, i * groupsize:(i + 1) * groupsize].reshape(B * R, -1))
    w = W.clone()
    if cls is GPTQ:
        out = r._run_compensation(w, U, 128, groupsize, static, None, backend="hip", graph=graph)
        return (*out, w)
    if cls is GPTAQ:
        out = r._run_compensation(w, U, extra["P"], 128, groupsize, static, None, backend="hip",
                                  graph=graph)
        return (*out, w)
    gh = extra["GH"].clone()
    out = r._run_compensation(w, U, extra["Z"], gh, 128, groupsize, static, None, backend="hip",
                              graph=graph)
    return (*out, w, gh)


@pytest.mark.parametrize("variant", ["GPTQ", "GPTAQ", "G2PTQ"])
@pytest.mark.parametrize("static", [False, True])
def test_compensation_graph_replays_match_eager(dev, variant, static):
    import g2ptq_amd
    from g2ptq_amd import _graphs
    cls = getattr(g2ptq_amd, variant)
    B, R, C, gs = 2, 64, 384, 128
    print(f"graph replay {variant} static={static}", flush=True)
    _graphs.clear()
    U = _factor(B, C, 31, dev)
    for rep in range(3):
        g = gen(900 + rep)
        W = (torch.randn(B, R, C, generator=g) * 0.02).to(dev)
        extra = {"P": (torch.triu(torch.randn(B, C, C, generator=g), 1) * 1e-3).to(dev),
                 "Z": (torch.randn(B, R, C, generator=g) * 1e-4).to(dev),
                 "GH": (torch.randn(B, R, C, generator=g) * 1e-4).to(dev)}
        eager = _run(cls, dev, W, U, extra, gs, static, graph=False)
        torch.cuda.synchronize()
        # unrelated eager work between the capture/replays
        junk = torch.randn(512, 512, device=dev) @ torch.randn(512, 512, device=dev)
        junk.sum().item()
        replay = _run(cls, dev, W, U, extra, gs, static, graph=True)
        torch.cuda.synchronize()
        for i, (a, e) in enumerate(zip(replay, eager)):
            assert_bitexact(a, e, f"{variant} replay {rep} output {i}")
    _graphs.clear()


def test_block_graph_replays_match_eager(dev):
    """The per-block ``_run_compensation_block(graph=True)`` path through ``run_graph``."""
    from g2ptq_amd import GPTQ, clear_graph_cache
    clear_graph_cache()
    B, R, bs = 2, 96, 128
    r = object.__new__(GPTQ)
    r.quantizer = _quantizers(4, False, bs, -1)
    for rep in range(3):
        w, h, s, z = ref_inputs(B, bs, R, 7, True, 1234 + rep)
        # reference block layout: weight (B, R, bs) → transposed inside
        Wb = w.transpose(1, 2).contiguous().to(dev)
        S = s.transpose(1, 2).contiguous().to(dev)
        Zp = z.transpose(1, 2).contiguous().to(dev)
        Hd = h.to(dev)
        e = r._run_compensation_block(Wb, Hd, S, Zp, "hip", False)
        torch.cuda.synchronize()
        torch.ones(1000, device=dev).cumsum(0).sum().item()
        g_ = r._run_compensation_block(Wb, Hd, S, Zp, "hip", True)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(g_, e)):
            assert_bitexact(a, b, f"block replay {rep} output {i}")
    clear_graph_cache()


@pytest.mark.parametrize("variant", ["G2PTQ", "GPTAQ"])
def test_block_graph_matches_eager_and_owns_outputs(dev, variant):
    """tests/test_triton_compensation.py:984-1040: the block operator replayed from
    a graph equals eager, and the outputs of one replay are not overwritten by
    the next (each call returns tensors it owns)."""
    import g2ptq_amd
    from g2ptq_amd import clear_graph_cache
    from tests._util import g2_inputs, gptaq_p
    clear_graph_cache()
    cls = getattr(g2ptq_amd, variant)
    B, bs, R, maxq = 2, 16, 193, 7
    r = object.__new__(cls)
    r.quantizer = _quantizers(4, False, bs, -1)
    retained = None
    for seed in (401, 402):
        w, h, s, z = ref_inputs(B, bs, R, maxq, True, seed)
        T = lambda t: t.transpose(1, 2).contiguous().to(dev)  # noqa: E731  (B, R, bs) layout
        if variant == "G2PTQ":
            zz, gh = g2_inputs(w, s, seed + 1000)
            args = (T(w), h.to(dev), T(s), T(z), T(zz), T(gh))
        else:
            args = (T(w), h.to(dev), gptaq_p(w, seed + 1000).to(dev), T(s), T(z))
        eager = r._run_compensation_block(*args, "hip", False)
        torch.cuda.synchronize()
        graph_out = r._run_compensation_block(*args, "hip", True)
        torch.cuda.synchronize()
        for i, (a, e) in enumerate(zip(graph_out, eager)):
            assert_bitexact(a, e, f"{variant} seed {seed} output {i}")
        if retained is not None:
            for i, (out, snap) in enumerate(zip(*retained)):
                assert_bitexact(out, snap, f"{variant} earlier output {i} was overwritten")
        retained = (graph_out, tuple(t.clone() for t in graph_out))
    clear_graph_cache()
