"""GPU parity of the complete per-layer flows against the CPU oracle."""
import copy

import pytest
import torch

from oracle import flows as oflows
from oracle import hessian as ohess
from oracle import original_loops as oloops
from oracle import quant as oquant
from tests._util import (assert_beta_close, assert_bitexact, assert_close, assert_flow_parity,
                         gen)

pytestmark = pytest.mark.gpu

FLOAT_RTOL = 2e-5
FLOAT_ATOL = 2e-5


def _prepare_loop_quantizers(weight, bits, symmetric, groupsize, static_groups):
    """tests/test_triton_compensation.py:377-407, for oracle and HIP quantizers."""
    from g2ptq_amd import WeightQuantizer
    batch, rows, columns = weight.shape
    otpl = oquant.WeightQuantizer().configure(bits, sym=symmetric)
    oorig = copy.deepcopy(otpl)
    oorig.find_params(weight.reshape(batch * rows, columns))
    ogroups = None
    if static_groups:
        ogroups = []
        for s in range(0, columns, groupsize):
            q = copy.deepcopy(oorig)
            q.find_params(weight[:, :, s:s + groupsize].reshape(batch * rows, -1))
            ogroups.append(q)
    # HIP quantizer list for the refactored loop
    dev = torch.device("cuda:0")
    htpl = WeightQuantizer()
    htpl.configure(bits, perchannel=True, sym=symmetric)
    wd = weight.to(dev)
    if static_groups:
        cur = []
        for s in range(0, columns, groupsize):
            q = copy.deepcopy(htpl)
            q.find_params(wd[:, :, s:s + groupsize].reshape(batch * rows, -1))
            cur.append(q)
    elif groupsize == -1:
        q = copy.deepcopy(htpl)
        q.find_params(wd.reshape(batch * rows, columns))
        cur = [q]
    else:
        cur = [copy.deepcopy(htpl) for _ in range((columns + groupsize - 1) // groupsize)]
    return oorig, ogroups, cur


# (name, groupsize, static_groups, actorder, (rows, columns, blocksize)).  The
# "fitted_in_sweep" cases have min/max groups that tile 32-column panels, which
# the sweep fits itself (the last block and its last group ragged in the first).
CONFIGS = (("ungrouped", -1, False, False, (37, 15, 5)),
           ("dynamic_groups", 4, False, False, (37, 15, 5)),
           ("static_groups_actorder", 4, True, True, (37, 15, 5)),
           ("dynamic_groups_fitted_in_sweep", 64, False, False, (37, 224, 128)),
           ("dynamic_groups32_fitted_in_sweep", 32, False, False, (21, 192, 64)))


@pytest.mark.parametrize("cfg", CONFIGS, ids=[c[0] for c in CONFIGS])
@pytest.mark.parametrize("symmetric", [True, False])
def test_compensation_matches_original_loops(dev, cfg, symmetric):
    """tests/test_triton_compensation.py:581-772 with the HIP loop in place of torch."""
    from g2ptq_amd import G2PTQ, GPTAQ, GPTQ, GPTQGuided
    name, groupsize, static_groups, actorder, (rows, columns, blocksize) = cfg
    batch, bits = 2, 4
    print(f"compensation case {name} sym={symmetric}", flush=True)
    g = gen(8000 + CONFIGS.index(cfg) * 100 + int(symmetric))
    original = torch.randn(batch, rows, columns, generator=g)
    perm = None
    weight = original.clone()
    if actorder:
        perm = torch.randperm(columns, generator=g)
        weight = weight[:, :, perm]
    hinv = torch.triu(torch.randn(batch, columns, columns, generator=g).mul_(0.002), diagonal=1)
    torch.diagonal(hinv, dim1=1, dim2=2).copy_(torch.rand(batch, columns, generator=g).mul_(0.5).add_(0.75))
    z = torch.randn(weight.shape, generator=g).mul_(0.002)
    ghinv = torch.randn(weight.shape, generator=g).mul_(0.002)
    p = torch.triu(torch.randn(batch, columns, columns, generator=g).mul_(0.002), diagonal=1)
    qperm = perm if static_groups and actorder else None

    def check(what, actual, expected):
        assert_bitexact(actual[1], expected[1], f"{what} codes")
        for i in (0, 2, 3) + ((4,) if len(expected) == 5 else ()):
            assert_close(actual[i], expected[i], FLOAT_RTOL, FLOAT_ATOL, f"{what}[{i}]")

    oorig, ogroups, _ = _prepare_loop_quantizers(original, bits, symmetric, groupsize, static_groups)
    exp = oloops.gptq_loop(weight.clone(), hinv.clone(), oorig, ogroups, blocksize, groupsize, qperm)
    for cls in (GPTQ, GPTQGuided):
        _, _, cur = _prepare_loop_quantizers(original, bits, symmetric, groupsize, static_groups)
        runner = object.__new__(cls)
        runner.columns, runner.num_layers, runner.rows, runner.quantizer = columns, batch, rows, cur
        w = weight.clone().to(dev)
        res = runner._run_compensation(w, hinv.clone().to(dev), blocksize, groupsize, static_groups,
                                       qperm, backend="hip", graph=False)
        torch.cuda.synchronize()
        check(cls.__name__, (*res, w), exp)

    oorig, ogroups, cur = _prepare_loop_quantizers(original, bits, symmetric, groupsize, static_groups)
    exp = oloops.g2ptq_loop(weight.clone(), hinv.clone(), z.clone(), ghinv.clone(), oorig, ogroups,
                            blocksize, groupsize, qperm)
    r = object.__new__(G2PTQ)
    r.columns, r.num_layers, r.rows, r.quantizer = columns, batch, rows, cur
    w, gh = weight.clone().to(dev), ghinv.clone().to(dev)
    res = r._run_compensation(w, hinv.clone().to(dev), z.clone().to(dev), gh, blocksize, groupsize,
                              static_groups, qperm, backend="hip", graph=False)
    torch.cuda.synchronize()
    check("G2PTQ", (*res, w, gh), exp)

    oorig, ogroups, cur = _prepare_loop_quantizers(original, bits, symmetric, groupsize, static_groups)
    exp = oloops.gptaq_loop(weight.clone(), hinv.clone(), p.clone(), oorig, ogroups, blocksize,
                            groupsize, qperm)
    r = object.__new__(GPTAQ)
    r.columns, r.num_layers, r.rows, r.quantizer = columns, batch, rows, cur
    w = weight.clone().to(dev)
    res = r._run_compensation(w, hinv.clone().to(dev), p.clone().to(dev), blocksize, groupsize,
                              static_groups, qperm, backend="hip", graph=False)
    torch.cuda.synchronize()
    check("GPTAQ", (*res, w), exp)


def _layer(rows, cols, seed, dtype=torch.bfloat16):
    lin = torch.nn.Linear(cols, rows, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(rows, cols, generator=gen(seed)) * 0.02)
    return lin.to(dtype)


def _acts(T, C, seed):
    g = gen(seed)
    sig = torch.exp(torch.randn(C, generator=g))
    return (torch.randn(T, C, generator=g) * sig).bfloat16()


def _student_t3(shape, g):
    z = torch.randn(shape, generator=g)
    return z / torch.sqrt(torch.randn((3,) + tuple(shape), generator=g).pow(2).sum(0) / 3)


def run_flow_from_x(dev, method, bits, sym, groupsize, actorder=False, B=2, R=256, C=1024,
                    T=4096, chunk=1024, G=4, alpha=None, seed=0, dead=None, drift=0.05):
    """One layer batch quantized from synthetic calibration data by the HIP
    classes and by the oracle on the same inputs (the data distributions of
    the benchmark configurations at reduced size): LogNormal channel scales,
    bf16 activations, bf16 weights ~N(0, 0.02); GPTAQ's X_fp = X plus
    N(0, drift·σ_c); G2PTQ's gradients 1e-3·N(0,1)·|t₃| per row and positive
    per-token saliencies.  ``dead`` input features never fire.
    Returns (layers, quantizers, oracle result, W0, H for the error, instance)."""
    from g2ptq_amd import G2PTQ, GPTAQ, GPTQ, GPTQGuided, WeightQuantizer, make_group_quantizers
    g = gen(seed)
    sig = torch.exp(torch.randn(C, generator=g))
    X = torch.randn(T, C, generator=g) * sig
    if dead is not None:
        X[:, dead] = 0
    X = X.bfloat16()
    Xfp = (X.float() + drift * sig * torch.randn(T, C, generator=g)).bfloat16()
    W = (torch.randn(B, R, C, generator=g) * 0.02).bfloat16()
    sal = torch.rand(T, G, generator=g) * torch.exp(0.5 * torch.randn(T, 1, generator=g))
    grads = 1e-3 * torch.randn(B, R, C, generator=g) * _student_t3((B, R, 1), g).abs()
    layers = []
    for b in range(B):
        lin = torch.nn.Linear(C, R, bias=False).to(torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(W[b])
        layers.append(lin.to(dev))
    W0 = W.float()
    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=sym)
    quantizers = make_group_quantizers(q, C, groupsize)
    static = bool(actorder)
    kw = dict(blocksize=128, percdamp=0.01, groupsize=groupsize, actorder=actorder,
              static_groups=static)
    batches = range(0, T, chunk)
    if method == "gptq":
        gq = GPTQ(layers)
        st = ohess.gptq_state(B, C)
    elif method == "gptaq":
        gq = GPTAQ(layers)
        st = ohess.gptaq_state(B, C)
        for b in range(B):
            gq.fp_inp[b] = [Xfp[i:i + chunk].to(dev) for i in batches]
    elif method == "g2ptq":
        gq = G2PTQ(layers, [[sal[i:i + chunk] for i in batches] for _ in range(B)],
                   [grads[b].to(dev) for b in range(B)], G)
        st = ohess.g2ptq_state(B, G, C)
    else:
        sal_g = sal.reshape(T // chunk, chunk, G)
        gq = GPTQGuided(layers, [sal_g for _ in range(B)], G)
        st = ohess.guided_state(B, G, C)
    gq.quantizer = quantizers
    for i in batches:
        xb = X[i:i + chunk].reshape(1, chunk, C)
        xd = xb.to(dev)
        for b in range(B):
            gq.add_batch(b, xd, None)
            if method == "gptq":
                ohess.gptq_add_batch(st, b, xb)
            elif method == "gptaq":
                ohess.gptaq_add_batch(st, b, xb, Xfp[i:i + chunk])
            elif method == "g2ptq":
                ohess.g2ptq_add_batch(st, b, xb, sal[i:i + chunk])
            else:
                ohess.guided_add_batch(st, b, xb, sal_g)
    H = st["H"].clone()
    if method == "gptq":
        gq.fasterquant(backend="hip", export_compressed_tensors=True, **kw)
        ref = oflows.gptq_fasterquant(W0, H, bits, sym, **kw)
        He = H
    elif method == "gptaq":
        gq.fasterquant(backend="hip", export_compressed_tensors=True, alpha=alpha, **kw)
        ref = oflows.gptaq_fasterquant(W0, H, st["dXXT"].clone(), bits, sym, alpha=alpha, **kw)
        He = H
    elif method == "g2ptq":
        gq.fasterquant(backend="hip", export_compressed_tensors=True, alpha=alpha, **kw)
        ref = oflows.g2ptq_fasterquant(W0, H.clone(), grads, st["act_square"], bits, sym, G,
                                       alpha=alpha, **kw)
        He = H.reshape(B * G, C, C)
    else:
        gq.fasterquant(backend="hip", export_compressed_tensors=True, **kw)
        ref = oflows.guided_fasterquant(W0, H.clone(), st["act_square"], bits, sym, G, **kw)
        He = H.reshape(B * G, C, C)
    torch.cuda.synchronize()
    return layers, quantizers, ref, W0, He, gq


# (name, method, bits, sym, groupsize, actorder, alpha): the settings of the
# benchmark configurations (1: GPTQ W4 asym g128; 2: W4 sym g128; 3: G2PTQ W3
# g128 α = 0.1 with 4 row groups; 5: GPTAQ W2 sym g64 α = 0.25, groups starting
# mid-block) and the remaining quantizer options.
FROM_X_CASES = (
    ("cfg1_gptq_w4_asym_g128", "gptq", 4, False, 128, False, None),
    ("cfg2_gptq_w4_sym_g128", "gptq", 4, True, 128, False, None),
    ("gptq_w3_sym_ungrouped", "gptq", 3, True, -1, False, None),
    ("gptq_w4_sym_g64_actorder_static", "gptq", 4, True, 64, True, None),
    ("cfg3_g2ptq_w3_g128_alpha0.1", "g2ptq", 3, True, 128, False, 0.1),
    ("cfg5_gptaq_w2_g64_alpha0.25", "gptaq", 2, True, 64, False, 0.25),
    ("gptaq_w4_asym_g128_actorder_static", "gptaq", 4, False, 128, True, 0.25),
    ("guided_w4_sym_g128", "guided", 4, True, 128, False, None),
    # act-order from calibration data: G2PTQ and GuidedQuant order columns by
    # act_square (g2ptq_utils.py:417-419), GPTQ/GPTAQ by the Hessian diagonal
    ("g2ptq_w3_sym_g128_actorder_static_alpha0.1", "g2ptq", 3, True, 128, True, 0.1),
    ("guided_w4_asym_g128_actorder_static", "guided", 4, False, 128, True, None),
)


@pytest.mark.parametrize("case", FROM_X_CASES, ids=[c[0] for c in FROM_X_CASES])
def test_flow_from_x_matches_oracle(dev, case):
    """Complete flows from calibration tokens (C = 1024, two layers of 256
    rows, 4096 tokens) against the oracle on the same inputs, held to the
    end-to-end parity protocol (oracle.parity): codes bit-exact except where a
    row's first differing code is at a rounding tie of the oracle's run (the
    Hessians and factors differ in fp32 summation order), such first
    divergences ≤ 0.01 % of entries, scales and dequantized weights within
    1e-3 before them, reconstruction error within 0.5 %."""
    name, method, bits, sym, gs, actorder, alpha = case
    print(f"flow from X: {name}", flush=True)
    layers, quantizers, ref, W0, H, gq = run_flow_from_x(
        dev, method, bits, sym, gs, actorder, alpha=alpha, seed=300 + FROM_X_CASES.index(case))
    assert_flow_parity(name, layers, quantizers, ref, W0, H, bits, gs, bool(actorder))
    if method == "g2ptq":
        assert_beta_close(gq._beta.cpu(), ref["beta"], name)


def test_flow_from_x_quad_lanes(dev):
    """Config 2's GPTQ W4 sym g128 with 2 × 8400 rows: more than 16384 rows
    take the sweep with a quad of lanes per row (the gate/up projections'
    28672 rows do).  Against the oracle under the parity protocol."""
    print("flow from X: gptq w4 sym g128, 2 x 8400 rows", flush=True)
    layers, quantizers, ref, W0, H, gq = run_flow_from_x(dev, "gptq", 4, True, 128, R=8400,
                                                         seed=395)
    assert_flow_parity("gptq quad lanes", layers, quantizers, ref, W0, H, 4, 128, False)


def test_g2ptq_dead_features_keep_gradients(dev):
    """g2ptq_utils.py:394-401: a dead input feature (zero Hessian diagonal)
    zeroes that weight column and sets H[d, d] = 1, but the gradients are
    cleared only together with an all-zero Hessian, so Grad's dead columns
    still enter every row's trust-region sums (c = Σ Grad⊙GA − GA²/diag A⁻¹)
    and thus β, Z and GH.  Flow against the oracle with α = 0.1."""
    dead = torch.tensor([3, 17, 100, 500, 1023])
    layers, quantizers, ref, W0, H, gq = run_flow_from_x(
        dev, "g2ptq", 3, True, 128, alpha=0.1, seed=390, dead=dead)
    Qd = torch.stack([l.weight.detach().float().cpu() for l in layers])
    assert torch.all(Qd[:, :, dead] == 0)
    assert_flow_parity("g2ptq dead features", layers, quantizers, ref, W0, H, 3, 128, False)
    assert_beta_close(gq._beta.cpu(), ref["beta"], "g2ptq dead features")


HCLIP_CASES = ("gptq_dynamic", "gptq_static_actorder", "gptaq_dynamic", "g2ptq_dynamic_actorder",
               "guided_static")


@pytest.mark.parametrize("case", HCLIP_CASES)
def test_fasterquant_hclip_matches_oracle(dev, case):
    """--w_clip --w_hclip: the clip search of every group fit (static fits on the
    unpermuted weights, dynamic fits inside the lazy-batch loop) weights its
    error with the undamped Hessian diagonal of the row's layer / saliency
    group, in the loop's column order (gptq_utils.py:248-270, 314-315 and the
    variants).  Both sides get the same Hessians; codes agree except where a
    near-tie of the clip search or a rounding tie cascades."""
    from g2ptq_amd import G2PTQ, GPTAQ, GPTQ, GPTQGuided, WeightQuantizer, make_group_quantizers
    print(f"hclip flow case {case}", flush=True)
    B, R, C, G, gs, bits = 2, 64, 128, 2, 32, 3
    actorder = case.endswith("actorder")
    static = "static" in case
    g = gen(4200 + HCLIP_CASES.index(case))
    layers = [_layer(R, C, 60 + b + 10 * HCLIP_CASES.index(case)).to(dev) for b in range(B)]
    W0 = torch.stack([l.weight.detach().float().cpu() for l in layers])
    sig = torch.exp(torch.randn(C, generator=g))

    def gram(groups):
        X = torch.randn(B, groups, 512, C, generator=g) * sig
        return (2 / 512) * X.transpose(-1, -2) @ X

    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=True, mse=True, hclip=True)
    quantizers = make_group_quantizers(q, C, gs)
    kw = dict(blocksize=128, percdamp=0.01, groupsize=gs, actorder=actorder,
              static_groups=static)
    if case.startswith("gptq"):
        H = gram(1)[:, 0]
        gq = GPTQ(layers)
        gq.quantizer = quantizers
        gq.H = H.to(dev)
        gq.fasterquant(backend="hip", **kw)
        ref = oflows.gptq_fasterquant(W0, H, bits, True, mse=True, hclip=True, **kw)
    elif case.startswith("gptaq"):
        H = gram(1)[:, 0]
        D = torch.randn(B, C, C, generator=g) * 0.01
        gq = GPTAQ(layers)
        gq.quantizer = quantizers
        gq.H = H.to(dev)
        gq.dXXT = D.to(dev)
        gq.fasterquant(backend="hip", **kw)
        ref = oflows.gptaq_fasterquant(W0, H, D, bits, True, mse=True, hclip=True, **kw)
    else:
        H = gram(G)
        act = torch.rand(B, C, generator=g)
        sal = [torch.ones(1, 1, G, device=dev) for _ in range(B)]
        if case.startswith("g2ptq"):
            grads = torch.randn(B, R, C, generator=g) * 1e-3
            gq = G2PTQ(layers, [[s] for s in sal], [grads[b].to(dev) for b in range(B)], G)
            gq.quantizer = quantizers
            gq.H = H.clone().to(dev)
            gq.act_square = act.to(dev)
            gq.fasterquant(backend="hip", alpha=0.0, **kw)
            ref = oflows.g2ptq_fasterquant(W0, H.clone(), grads, act, bits, True, G, alpha=0.0,
                                           mse=True, hclip=True, **kw)
        else:
            gq = GPTQGuided(layers, sal, G)
            gq.quantizer = quantizers
            gq.H = H.to(dev)
            gq.act_square = act.to(dev)
            gq.fasterquant(backend="hip", **kw)
            ref = oflows.guided_fasterquant(W0, H, act, bits, True, G, mse=True, hclip=True, **kw)
    torch.cuda.synchronize()
    Qd = torch.stack([l.weight.detach().float().cpu() for l in layers])
    Qr = ref["Q"].bfloat16().float()
    agree = (Qd == Qr).float().mean().item()
    assert agree >= 0.95, agree
    s_agree = torch.stack([(a.scale.cpu() == b.scale).float().mean()
                           for a, b in zip(quantizers, ref["quantizers"])]).mean().item()
    assert s_agree >= 0.95, s_agree
    Hr = H if H.dim() == 3 else H.sum(1)
    e_hip = oflows.reconstruction_error(W0, Qd, Hr)
    e_ref = oflows.reconstruction_error(W0, Qr, Hr)
    assert abs(e_hip - e_ref) <= 0.005 * e_ref, (e_hip, e_ref)


@pytest.mark.parametrize("sym", [True, False])
def test_gptq_without_calibration_is_rtn(dev, sym):
    """gptq_utils.py:275-277: an all-zero Hessian becomes the identity, the factor
    is diagonal, nothing propagates, and the weights equal round-to-nearest with
    the same groups (gptq_utils.py:598-680), code for code."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    B, R, C, gs = 2, 96, 384, 128
    layers = [_layer(R, C, 70 + b).to(dev) for b in range(B)]
    W0 = torch.stack([l.weight.detach().float().cpu() for l in layers])
    gq = GPTQ(layers)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=sym)
    gq.quantizer = make_group_quantizers(q, C, gs)
    gq.fasterquant(groupsize=gs, backend="hip")
    torch.cuda.synchronize()
    Qd = torch.stack([l.weight.detach().float().cpu() for l in layers])
    fq, _, _ = oflows.rtn(W0, 4, sym, gs)
    assert torch.equal(Qd, fq.bfloat16().float())


@pytest.mark.parametrize("method", ["gptq", "gptaq", "g2ptq", "guided"])
def test_offload_hessians_bit_identical(dev, method):
    """offload_hessians=True (gptq_utils.py:103-113, 507-509; the G2PTQ and
    GuidedQuant variants): the Hessians live in host memory, calibration runs
    inside the onload context (two windows, as a driver onloads per layer
    batch), and fasterquant onloads them again.  The weights and fitted
    group parameters equal a resident run's bit for bit (the resident run
    reads H where the offloaded one leaves its onload context, so both fold
    their staged tokens at the same points); outside an onload context the
    host Hessian is refused before any kernel runs."""
    from g2ptq_amd import G2PTQ, GPTAQ, GPTQ, GPTQGuided, WeightQuantizer, make_group_quantizers
    B, R, C, T, chunk, G, bits, gs = 2, 128, 512, 4096, 1024, 4, 4, 128
    print(f"offload_hessians: {method}", flush=True)
    g = gen(950)
    sig = torch.exp(torch.randn(C, generator=g))
    X = (torch.randn(T, C, generator=g) * sig).bfloat16().to(dev)
    Xfp = (X.float() + 0.05 * sig.to(dev) * torch.randn(T, C, generator=g).to(dev)).bfloat16()
    sal = (torch.rand(T, G, generator=g) + 0.1).to(dev)
    grads = [1e-3 * torch.randn(R, C, generator=g) for _ in range(B)]
    W = (torch.randn(B, R, C, generator=g) * 0.02).bfloat16()
    batches = list(range(0, T, chunk))

    def make(offload):
        layers = []
        for b in range(B):
            lin = torch.nn.Linear(C, R, bias=False).to(torch.bfloat16)
            with torch.no_grad():
                lin.weight.copy_(W[b])
            layers.append(lin.to(dev))
        if method == "gptq":
            gq = GPTQ(layers, offload_hessians=offload)
        elif method == "gptaq":
            gq = GPTAQ(layers, offload_hessians=offload)
            for b in range(B):
                gq.fp_inp[b] = [Xfp[i:i + chunk] for i in batches]
        elif method == "g2ptq":
            gq = G2PTQ(layers, [[sal[i:i + chunk] for i in batches] for _ in range(B)],
                       [gr.to(dev) for gr in grads], G, offload_hessians=offload)
        else:
            gq = GPTQGuided(layers, [sal.reshape(T // chunk, chunk, G) for _ in range(B)], G,
                            offload_hessians=offload)
        q = WeightQuantizer()
        q.configure(bits, perchannel=True, sym=True)
        gq.quantizer = make_group_quantizers(q, C, gs)
        return layers, gq

    def onload(gq):
        if method == "g2ptq":
            return gq._maybe_onload_hessian_grad()
        return gq._maybe_onload_hessian()

    kw = dict(blocksize=128, percdamp=0.01, groupsize=gs, backend="hip")
    if method in ("gptaq", "g2ptq"):
        kw["alpha"] = 0.25 if method == "gptaq" else 0.1
    out = []
    for offload in (False, True):
        layers, gq = make(offload)
        for window in (batches[:2], batches[2:]):
            with onload(gq):
                for i in window:
                    for b in range(B):
                        gq.add_batch(b, X[i:i + chunk].unsqueeze(0), None)
            if not offload:
                gq.H  # the offloaded run folds its staged tokens here (onload exit)
        if offload:
            assert gq.H.device.type == "cpu"
        gq.fasterquant(**kw)
        torch.cuda.synchronize()
        out.append((torch.stack([l.weight.detach().cpu() for l in layers]),
                    [(qz.scale.detach().cpu(), qz.zero.detach().cpu()) for qz in gq.quantizer]))
    (w_res, p_res), (w_off, p_off) = out
    assert torch.equal(w_res.view(torch.int16), w_off.view(torch.int16))
    for (s0, z0), (s1, z1) in zip(p_res, p_off):
        assert torch.equal(s0, s1) and torch.equal(z0, z1)
    # calibration outside the onload context: the staged tokens cannot be
    # folded into a host Hessian
    _, gq = make(True)
    gq.add_batch(0, X[:chunk].unsqueeze(0), None)
    with pytest.raises(RuntimeError, match="onload"):
        gq.H


def test_dead_columns_are_zeroed(dev):
    """gptq_utils.py:278-280: input features that never fire (zero Hessian
    diagonal) get H[d, d] = 1 and W[:, d] = 0, so their weights quantize to 0."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    B, R, C, T = 2, 128, 256, 2048
    layers = [_layer(R, C, 80 + b).to(dev) for b in range(B)]
    W0 = torch.stack([l.weight.detach().float().cpu() for l in layers])
    X = _acts(T, C, 81).float()
    dead = torch.tensor([3, 17, 100, 200, 255])
    X[:, dead] = 0
    X = X.bfloat16()
    gq = GPTQ(layers)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=False)
    gq.quantizer = make_group_quantizers(q, C, 128)
    st = ohess.gptq_state(B, C)
    xb = X.reshape(1, T, C)
    for b in range(B):
        gq.add_batch(b, xb.to(dev), None)
        ohess.gptq_add_batch(st, b, xb)
    gq.fasterquant(groupsize=128, backend="hip")
    torch.cuda.synchronize()
    Qd = torch.stack([l.weight.detach().float().cpu() for l in layers])
    assert torch.all(Qd[:, :, dead] == 0)
    ref = oflows.gptq_fasterquant(W0, st["H"].clone(), 4, False, groupsize=128)
    Qr = ref["Q"].bfloat16().float()
    assert torch.all(Qr[:, :, dead] == 0)
    assert (Qd == Qr).float().mean().item() >= 0.95


def test_nan_in_weights_raises(dev):
    """gptq_utils.py:346-350: a weight of +inf gives that row an infinite
    scale (inf > 0 passes the scale assertion), every code of the row is NaN,
    the write-back's NaN check fires and fasterquant raises the reference's
    ValueError("NaN in weights").  The oracle produces the same NaN row."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    R, C, T = 64, 256, 1024
    layers = [_layer(R, C, 91).to(dev)]
    with torch.no_grad():
        layers[0].weight[5, 17] = float("inf")
    W0 = layers[0].weight.detach().float().cpu().unsqueeze(0)
    X = _acts(T, C, 92)
    gq = GPTQ(layers)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, -1)
    st = ohess.gptq_state(1, C)
    gq.add_batch(0, X.reshape(1, T, C).to(dev), None)
    ohess.gptq_add_batch(st, 0, X.reshape(1, T, C))
    with pytest.raises(ValueError, match="NaN in weights"):
        gq.fasterquant(groupsize=-1, backend="hip")
    ref = oflows.gptq_fasterquant(W0, st["H"], 4, True, groupsize=-1)
    nan_rows = torch.isnan(ref["Q"][0]).any(1).nonzero().flatten().tolist()
    assert nan_rows == [5]


def test_nan_hessian_exhausts_the_damp_retry(dev):
    """gptq_utils.py:288-311: a factor with NaN fails at every damp, the damp
    climbs by 0.0015 past 1, and fasterquant raises the reference's ValueError."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    C = 64
    layers = [_layer(32, C, 90).to(dev)]
    gq = GPTQ(layers)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, -1)
    H = torch.eye(C).unsqueeze(0).clone()
    H[0, 5, 7] = H[0, 7, 5] = float("nan")
    gq.H = H.to(dev)
    with pytest.raises(ValueError, match="damp_percent"):
        gq.fasterquant(backend="hip")


@pytest.mark.parametrize("rows_q,rows_kv,C,mse", [(96, 32, 640, False), (96, 32, 640, True),
                                                   (4096, 1024, 1024, False)])
def test_shared_input_joint_fasterquant_matches_per_instance(dev, rows_q, rows_kv, C, mse):
    """SharedInputHessian.fasterquant (one compensation loop over q's and k/v's
    rows) gives every member the weights and group parameters of its own
    fasterquant, bit for bit."""
    from g2ptq_amd import GPTQ, SharedInputHessian, WeightQuantizer, make_group_quantizers
    print(f"joint fasterquant q={rows_q} kv={rows_kv} C={C} mse={mse}", flush=True)
    X = _acts(2048, C, 77)

    def setup():
        lq = _layer(rows_q, C, 1).to(dev)
        lk, lv = _layer(rows_kv, C, 2).to(dev), _layer(rows_kv, C, 3).to(dev)
        insts = [GPTQ([lq]), GPTQ([lk, lv])]
        for inst in insts:
            q = WeightQuantizer()
            q.configure(4, perchannel=True, sym=True, mse=mse)
            inst.quantizer = make_group_quantizers(q, C, 128)
        share = SharedInputHessian([(insts[0], 0), (insts[1], 0), (insts[1], 1)])
        for i in range(0, 2048, 512):
            share.add_batch(X[i:i + 512].reshape(1, 512, C).to(dev))
        share.finalize()
        return [lq, lk, lv], insts, share

    kw = dict(blocksize=128, percdamp=0.01, groupsize=128, actorder=False, static_groups=False,
              backend="hip")
    la, ia, _ = setup()
    for inst in ia:
        inst.fasterquant(**kw)
    lb, ib, share = setup()
    share.fasterquant(**kw)
    torch.cuda.synchronize()
    for x, y in zip(la, lb):
        assert torch.equal(x.weight, y.weight)
    for xa, xb in zip(ia, ib):
        for qa, qb in zip(xa.quantizer, xb.quantizer):
            assert torch.equal(qa.scale, qb.scale) and torch.equal(qa.zero, qb.zero)


def test_grouped_launch_factors_shared_slots_once(dev):
    """One launch of four linears in two shared-input pairs (an MoE chunk's
    gate/up): finalize maps slots 1 and 3 to 0 and 2, the batched factor
    factors two Hessians instead of four, and the written weights equal a run
    without the map bit for bit."""
    from g2ptq_amd import GPTQ, SharedInputHessian, WeightQuantizer, make_group_quantizers
    C, R = 256, 96
    g = gen(4711)
    w0 = [(torch.randn(R, C, generator=g) * 0.02).to(torch.bfloat16) for _ in range(4)]
    sig = torch.exp(torch.randn(C, generator=g))
    xs = [[(torch.randn(T, C, generator=g) * sig).to(torch.bfloat16).to(dev) for T in (300, 77, 512)]
          for _ in range(2)]

    def run(keep_map):
        layers = [torch.nn.Linear(C, R, bias=False, device=dev, dtype=torch.bfloat16)
                  for _ in range(4)]
        with torch.no_grad():
            for lin, w in zip(layers, w0):
                lin.weight.copy_(w.to(dev))
        gq = GPTQ(layers)
        q = WeightQuantizer()
        q.configure(4, perchannel=True, sym=True)
        gq.quantizer = make_group_quantizers(q, C, 128)
        shares = [SharedInputHessian([(gq, 0), (gq, 1)]), SharedInputHessian([(gq, 2), (gq, 3)])]
        for sh, batches in zip(shares, xs):
            for x in batches:
                sh.add_batch(x)
        for sh in shares:
            sh.finalize()
        assert gq._h_alias == {1: 0, 3: 2}
        if not keep_map:
            gq._h_alias = None
        gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip")
        torch.cuda.synchronize()
        return [lin.weight.detach().cpu().view(torch.int16) for lin in layers]

    with_map, without = run(True), run(False)
    for a, b in zip(with_map, without):
        assert torch.equal(a, b)
    assert not torch.equal(with_map[0], with_map[2])  # the two pairs differ
