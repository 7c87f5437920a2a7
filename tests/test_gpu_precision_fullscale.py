"""GPU: the Hessian kinds whose staged operand is not bf16-exact, at the
benchmark configurations' calibration size, held to the end-to-end parity
protocol, and the tie window that protocol uses at this size measured
against fp64.

The weighted (G2PTQ) and GPTAQ Hessians stage x·s and X_fp − X as hi + lo
bf16 planes (16 significant bits; the reference keeps fp32's 24), so their
rounding differs from the reference's more than a plain Hessian's does.  Each
test accumulates the Hessians of 262,144 calibration tokens (32 batches of
8192, LogNormal channel scales) on the GPU, computes the same Hessians
exactly (fp64 on the GPU), and runs the oracle flow (oracle.flows) from the
exact Hessians on the CPU twice: in fp32 (the reference's arithmetic) and in
fp64.  The HIP flow from its own Hessians, and the HIP flow from the exact
ones (rounded to fp32), must both meet the bar of oracle.parity.check_flow
against the fp32 oracle: each row's first differing code at a rounding tie
of the exact run, such rows at most 0.01 % of the entries, scales and
dequantized weights within 1e-3 before them, reconstruction error within
0.5 %.  Over a 4096-column compensation any fp32 ordering moves x/s by a few
1e-4 at rare entries, so two fp32 computations can round a value that close
to a tie differently; which one strays is decided by the fp64 run.  A flow's
codes first differ from the fp64 run's only where the exact x/s lies within
that flow's own error of a tie, so the largest such tie distance measures how
far its x/s strays from exact arithmetic: the HIP flow's must be at most
twice the fp32 oracle's, and where the HIP and fp32 flows differ the exact
x/s must lie at most twice the oracle's own distance from a tie (at least
the protocol's 1e-4).

* config 3's G2PTQ at C = 4096 (one linear of 4 row groups × 256 rows, W3
  g128, α = 0.1, per-token saliencies);
* config 5's GPTAQ at C = 8192 (256 rows, W2 g64, α = 0.25, X_fp = X plus
  N(0, 0.05·σ_c)); config 5's own C = 28672 would take the CPU oracle minutes
  per run (its full width is checked on sampled rows in test_gpu_configs).
"""
import pytest
import torch

from oracle import flows as oflows
from oracle.parity import check_flow, element_params, exported_codes, loop_order, stage_b
from tests._util import gen

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

N_TOKENS, CHUNK = 262144, 8192


def _student_t3(shape, g):
    z = torch.randn(shape, generator=g)
    return z / torch.sqrt(torch.randn((3,) + tuple(shape), generator=g).pow(2).sum(0) / 3)


def _tokens(C, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    sig = torch.exp(torch.randn(C, device=dev, generator=g))
    X = torch.empty(N_TOKENS, C, device=dev, dtype=torch.bfloat16)
    for t0 in range(0, N_TOKENS, CHUNK):
        X[t0:t0 + CHUNK] = (torch.randn(CHUNK, C, device=dev, generator=g) * sig).bfloat16()
    return X, sig, g


def _linear(R, C, seed, dev):
    lin = torch.nn.Linear(C, R, bias=False, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(R, C, generator=gen(seed)).to(dev) * 0.02)
    return lin


# Ties are judged by the fp64 run.  A HIP code may differ from the fp32
# oracle's (first in its row) only where the exact x/s lies within
# NOISE_FACTOR × the fp32 oracle's own largest such distance of a tie (the
# oracle itself rounds away from exact that close to a tie), never less than
# the protocol's MIN_TIE; below FLOOR distances are single roundings.
NOISE_FACTOR, FLOOR, MIN_TIE = 2.0, 2e-5, 1e-4


def _first_divergence(a, b):
    """Per row, the first column where ``a`` and ``b`` differ (C if none)."""
    N, C = a.shape
    diff = a != b
    first = torch.full((N,), C, dtype=torch.int64)
    rows = diff.any(1)
    first[rows] = diff[rows].to(torch.int8).argmax(1)
    return first


def _exact_ties(label, codes, ref, ref64, gs):
    """The flow's first divergences from the fp32 oracle, each judged by the
    fp64 run: its x/s distance from a tie there.  Where the fp32 oracle's row
    already left the fp64 run's codes earlier, the fp64 value is of another
    history and the oracle's own x/s is used.  Returns the largest distance."""
    N, C = codes.shape
    perm = ref64["perm"]
    cr = loop_order(ref["W_int"].reshape(N, C), perm)
    c64 = loop_order(ref64["W_int"].reshape(N, C), perm)
    ch = loop_order(codes, perm)
    f_h = _first_divergence(ch, cr)
    f_64 = _first_divergence(cr, c64)
    s32, _ = element_params(ref["quantizers"], N, C, gs, False, perm)
    s64, _ = element_params(ref64["quantizers"], N, C, gs, False, perm)
    x32 = ref["loop"]["X"].reshape(N, C).double()
    x64 = ref64["loop"]["X"].reshape(N, C).double()
    worst, other = 0.0, 0
    for r in (f_h < C).nonzero().flatten().tolist():
        j = int(f_h[r])
        if int(f_64[r]) < j:
            t = float(x32[r, j] / s32[r, j].double())
            other += 1
        else:
            t = float(x64[r, j] / s64[r, j].double())
        worst = max(worst, abs(t - float(torch.floor(torch.tensor(t))) - 0.5))
    print(f"{label}: {int((f_h < C).sum())} rows first differ from the fp32 oracle, the exact "
          f"x/s at most {worst:.3g} from a tie there ({other} judged by the oracle's x/s)",
          flush=True)
    return worst


def _fp64_distance(label, codes, quantizers, ref64, gs):
    """How far a flow strays from exact arithmetic: its codes against the fp64
    oracle's, in loop order; at each row's first differing code, the fp64
    run's distance |frac(x/s) − ½| from a rounding tie.  Returns the report
    (``max_tie_distance``, ``rows_diverged``)."""
    N, C = codes.shape
    perm = ref64["perm"]
    s, z = element_params(quantizers, N, C, gs, False, perm)
    s64, z64 = element_params(ref64["quantizers"], N, C, gs, False, perm)
    rep = stage_b(loop_order(codes, perm), loop_order(ref64["W_int"].reshape(N, C), perm),
                  ref64["loop"]["X"].reshape(N, C), s, s64, z, z64,
                  loop_order(ref64["Q"].reshape(N, C), perm), tol=0.5)
    print(f"{label} vs fp64: {rep['rows_diverged']}/{rep['rows']} rows first differ, at most "
          f"{rep['max_tie_distance']:.3g} from a tie", flush=True)
    return rep


def _bar(label, layers, quantizers, layers2, quantizers2, ref, ref64, W0, H, bits, gs):
    """The flow from the staged Hessians and the flow from the exact ones.
    Each one's distance from the fp64 oracle may be at most NOISE_FACTOR × the
    fp32 oracle's; against the fp32 oracle, each first differing code must lie
    at a tie of the exact run, as close as the oracle's own divergences from
    exact (×NOISE_FACTOR); and the rest of the bar of check_flow (first
    divergences ≤ 0.01 % of entries, scales and dequantized weights within
    1e-3 before them, write-back, reconstruction error within 0.5 %)."""
    C = W0.shape[-1]
    d_ref = _fp64_distance(label + ", fp32 oracle", ref["W_int"].reshape(-1, C),
                           ref["quantizers"], ref64, gs)["max_tie_distance"]
    window = max(NOISE_FACTOR * max(d_ref, FLOOR), MIN_TIE)
    out = []
    for name, (lay, qz) in (("staged", (layers, quantizers)), ("exact", (layers2, quantizers2))):
        lab = f"{label}, HIP from {name} Hessians"
        codes = exported_codes(lay, bits, C)
        d = _fp64_distance(lab, codes, qz, ref64, gs)["max_tie_distance"]
        assert d <= NOISE_FACTOR * max(d_ref, FLOOR), (lab, d, d_ref)
        worst = _exact_ties(lab, codes, ref, ref64, gs)
        assert worst <= window, (lab, worst, window)
        out.append(check_flow(lab, lay, qz, ref, W0, H, bits, gs, False, tie_tol=1.0))
    return out


def test_g2ptq_weighted_hessians_at_config3_scale(dev):
    from g2ptq_amd import G2PTQ, WeightQuantizer, make_group_quantizers
    C, G, Rg, bits, gs, alpha = 4096, 4, 256, 3, 128, 0.1
    R = G * Rg
    print(f"G2PTQ full-scale precision: C={C} tokens={N_TOKENS} G={G} R={R}", flush=True)
    X, _, g = _tokens(C, 501, dev)
    sal = torch.exp(0.5 * torch.randn(N_TOKENS, 1, device=dev, generator=g)) * \
        torch.rand(N_TOKENS, G, device=dev, generator=g)
    lin = _linear(R, C, 502, dev)
    W0 = lin.weight.detach().float().cpu().unsqueeze(0)
    grads = 1e-3 * torch.randn(R, C, generator=gen(503)) * _student_t3((R, 1), gen(504)).abs()
    batches = range(0, N_TOKENS, CHUNK)
    gq = G2PTQ([lin], [[sal[i:i + CHUNK] for i in batches]], [grads.to(dev)], G)
    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, gs)
    for i in batches:
        gq.add_batch(0, X[i:i + CHUNK].unsqueeze(0), None)
    # exact: H_g = (1/N)·Σ_t s_tg·x_t·x_tᵀ (equal batches, g2ptq_utils.py:182-201),
    # act_square = (1/N)·Σ_t x_t²
    He = torch.zeros(G, C, C, device=dev, dtype=torch.float64)
    act = torch.zeros(C, device=dev, dtype=torch.float64)
    for i in batches:
        x = X[i:i + CHUNK].double()
        for grp in range(G):
            He[grp] += (x * sal[i:i + CHUNK, grp:grp + 1].double()).T @ x
        act += (x * x).sum(0)
    He64 = (He / N_TOKENS).cpu()
    He = He64.float()
    act = (act / N_TOKENS).float().cpu()
    Hd = gq.H[0].detach().cpu()
    rel = ((Hd - He).abs() / torch.sqrt(torch.diagonal(He, dim1=1, dim2=2).unsqueeze(2) *
                                        torch.diagonal(He, dim1=1, dim2=2).unsqueeze(1))).max()
    print(f"weighted Hessians: max |H − exact| / sqrt(H_ii·H_jj) = {rel.item():.3g}", flush=True)
    assert rel.item() <= 2e-5
    del X, sal
    # the same flow from the exact Hessians, on a copy of the layer
    lin2 = _linear(R, C, 502, dev)
    gq2 = G2PTQ([lin2], [[]], [grads.to(dev)], G)
    gq2.quantizer = make_group_quantizers(q, C, gs)
    gq2.H.copy_(He.to(dev).unsqueeze(0))
    for inst in (gq, gq2):
        inst.fasterquant(blocksize=128, percdamp=0.01, groupsize=gs, alpha=alpha, backend="hip",
                         export_compressed_tensors=True)
    torch.cuda.synchronize()
    ref = oflows.g2ptq_fasterquant(W0, He.unsqueeze(0).clone(), grads.unsqueeze(0),
                                   act.unsqueeze(0), bits, True, G, groupsize=gs, alpha=alpha)
    ref64 = oflows.g2ptq_fasterquant(W0, He64.unsqueeze(0).clone(), grads.unsqueeze(0),
                                     act.unsqueeze(0).double(), bits, True, G, groupsize=gs,
                                     alpha=alpha, dtype=torch.float64)
    _bar("G2PTQ C=4096, 262144 tokens", [lin], gq.quantizer, [lin2], gq2.quantizer, ref, ref64,
         W0, He, bits, gs)


def test_gptaq_cross_term_at_config5_scale(dev):
    from g2ptq_amd import GPTAQ, WeightQuantizer, make_group_quantizers
    C, R, bits, gs, alpha = 8192, 256, 2, 64, 0.25
    print(f"GPTAQ full-scale precision: C={C} tokens={N_TOKENS} R={R}", flush=True)
    X, sig, g = _tokens(C, 601, dev)
    lin = _linear(R, C, 602, dev)
    W0 = lin.weight.detach().float().cpu().unsqueeze(0)
    batches = range(0, N_TOKENS, CHUNK)
    gq = GPTAQ([lin])
    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, gs)
    He = torch.zeros(C, C, device=dev, dtype=torch.float64)
    De = torch.zeros(C, C, device=dev, dtype=torch.float64)
    for i in batches:
        x = X[i:i + CHUNK]
        xfp = (x.float() + 0.05 * sig * torch.randn(CHUNK, C, device=dev, generator=g)).bfloat16()
        gq.fp_inp[0].append(xfp)
        gq.add_batch(0, x.unsqueeze(0), None)
        xd = x.double()
        He += xd.T @ xd
        De += (xfp.double() - xd).T @ xd
    # one sequence per batch: H = (2/K)·Σ x·xᵀ, dXXT = (2/K)·Σ (x_fp − x)·xᵀ
    # over the K batches (gptaq_utils.py:130-148)
    K = len(batches)
    He64 = (He * (2.0 / K)).cpu()
    De64 = (De * (2.0 / K)).cpu()
    He, De = He64.float(), De64.float()
    Hd = gq.H[0].detach().cpu()
    Dd = gq.dXXT[0].detach().cpu()
    d = torch.diagonal(He)
    scale = torch.sqrt(d.unsqueeze(1) * d.unsqueeze(0))
    rh = ((Hd - He).abs() / scale).max().item()
    rd = ((Dd - De).abs() / scale).max().item()
    print(f"GPTAQ: max |H − exact| / sqrt(H_ii·H_jj) = {rh:.3g}, dXXT {rd:.3g}", flush=True)
    assert rh <= 2e-5 and rd <= 2e-5
    del X
    lin2 = _linear(R, C, 602, dev)
    gq2 = GPTAQ([lin2])
    gq2.quantizer = make_group_quantizers(q, C, gs)
    gq2.H.copy_(He.to(dev).unsqueeze(0))
    gq2.dXXT.copy_(De.to(dev).unsqueeze(0))
    for inst in (gq, gq2):
        inst.fasterquant(blocksize=128, percdamp=0.01, groupsize=gs, alpha=alpha, backend="hip",
                         export_compressed_tensors=True)
    torch.cuda.synchronize()
    ref = oflows.gptaq_fasterquant(W0, He.unsqueeze(0), De.unsqueeze(0), bits, True,
                                   groupsize=gs, alpha=alpha)
    ref64 = oflows.gptaq_fasterquant(W0, He64.unsqueeze(0), De64.unsqueeze(0), bits, True,
                                     groupsize=gs, alpha=alpha, dtype=torch.float64)
    _bar("GPTAQ C=8192, 262144 tokens", [lin], gq.quantizer, [lin2], gq2.quantizer, ref, ref64,
         W0, He.unsqueeze(0), bits, gs)


def test_g2ptq_more_than_16384_rows_in_one_loop(dev):
    """Config 3's G2PTQ W3 g128 (α = 0.1, 4 row groups) over two layers of
    8400 rows at C = 1024: 16800 rows in one compensation loop, where GPTQ and
    GPTAQ take a quad of lanes per row and G2PTQ keeps 16.  Judged like the
    cases above, against the fp32 and fp64 oracle flows from the same exact
    Hessians."""
    from g2ptq_amd import G2PTQ, WeightQuantizer, make_group_quantizers
    B, C, G, R, bits, gs, alpha = 2, 1024, 4, 8400, 3, 128, 0.1
    print(f"G2PTQ many rows: B={B} R={R} C={C} tokens={N_TOKENS} G={G}", flush=True)
    X, _, g = _tokens(C, 701, dev)
    sal = torch.exp(0.5 * torch.randn(N_TOKENS, 1, device=dev, generator=g)) * \
        torch.rand(N_TOKENS, G, device=dev, generator=g)
    lins = [_linear(R, C, 702 + b, dev) for b in range(B)]
    W0 = torch.stack([lin.weight.detach().float().cpu() for lin in lins])
    grads = 1e-3 * torch.randn(B, R, C, generator=gen(704)) * \
        _student_t3((B, R, 1), gen(705)).abs()
    batches = range(0, N_TOKENS, CHUNK)
    gq = G2PTQ(lins, [[sal[i:i + CHUNK] for i in batches] for _ in range(B)],
               [grads[b].to(dev) for b in range(B)], G)
    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, gs)
    for i in batches:
        xb = X[i:i + CHUNK].unsqueeze(0)
        for b in range(B):
            gq.add_batch(b, xb, None)
    # both layers read the same input: one exact set of weighted Hessians
    He = torch.zeros(G, C, C, device=dev, dtype=torch.float64)
    act = torch.zeros(C, device=dev, dtype=torch.float64)
    for i in batches:
        x = X[i:i + CHUNK].double()
        for grp in range(G):
            He[grp] += (x * sal[i:i + CHUNK, grp:grp + 1].double()).T @ x
        act += (x * x).sum(0)
    He64 = (He / N_TOKENS).cpu().unsqueeze(0).expand(B, G, C, C).contiguous()
    He = He64.float()
    act = (act / N_TOKENS).float().cpu().unsqueeze(0).expand(B, C).contiguous()
    del X, sal
    lins2 = [_linear(R, C, 702 + b, dev) for b in range(B)]
    gq2 = G2PTQ(lins2, [[] for _ in range(B)], [grads[b].to(dev) for b in range(B)], G)
    gq2.quantizer = make_group_quantizers(q, C, gs)
    gq2.H.copy_(He.to(dev))
    for inst in (gq, gq2):
        inst.fasterquant(blocksize=128, percdamp=0.01, groupsize=gs, alpha=alpha, backend="hip",
                         export_compressed_tensors=True)
    torch.cuda.synchronize()
    ref = oflows.g2ptq_fasterquant(W0, He.clone(), grads, act, bits, True, G, groupsize=gs,
                                   alpha=alpha)
    ref64 = oflows.g2ptq_fasterquant(W0, He64.clone(), grads, act.double(), bits, True, G,
                                     groupsize=gs, alpha=alpha, dtype=torch.float64)
    _bar("G2PTQ 2 x 8400 rows, C=1024", lins, gq.quantizer, lins2, gq2.quantizer, ref, ref64,
         W0, He.reshape(B * G, C, C), bits, gs)
