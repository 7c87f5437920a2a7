"""GPU: the BASELINE configurations at their own shapes, against the oracle.

* Config 1 exactly as specified: one 4096×4096 **fp32** linear ~N(0, 0.02)
  with round(1 %·4096) = 41 input columns ×10, 262,144 calibration tokens
  (128 sequences × 2048, N(0,1)·LogNormal(0,1) channel scales, bf16), GPTQ
  W4 asym g128, damp 0.01, blocksize 128.  The oracle accumulates its own
  Hessian from the same tokens (gptq_utils.py:115-126, fp32 on the host) and
  runs the whole fasterquant flow (gptq_utils.py:234-353); the HIP flow is
  held to oracle.parity.check_flow at the 1e-4 tie window, and the fp32
  weight is written with no bf16 cast (gptq_utils.py:351-353).
* Config 5 at its full width (C = 28672, 8192 rows, GPTAQ W2 g64, α = 0.25,
  X_fp = X + N(0, 0.05·σ_c)), the stage-A protocol on sampled rows: rows are
  independent given U and P, so 64 rows of the HIP flow are compared with the
  oracle's compensation (gptaq_utils.py:193-261) run from the HIP's own U
  and P; and P (gptaq_utils.py:349-352) on sampled entries against fp64.
* Config 3's down_proj at its full width (C = 14336, 4096 rows in 4 row
  groups, G2PTQ W3 g128, α = 0.1, saliency-weighted Hessians, Student-t(3)
  gradient rows), sampled rows: β, Z and GH are row-local given U, so 16 rows
  of each group are checked against the oracle's trust region
  (g2ptq_utils.py:459-476) evaluated in fp64 on the HIP's U, and their codes
  against the oracle's compensation (g2ptq_utils.py:252-347) run from the
  HIP's own U, Z and GH (stage A).
* Config 4 at its own shapes: 32 experts' gate/up (768×2048) in one 64-slot
  launch whose Hessians come from SharedInputHessian slot copies, and 64
  experts' down_proj (2048×768: a 512-column super-block and a ragged one of
  256 columns), with routed 2-D inputs (top-8 Zipf(1.1) over 128 experts),
  each launch against the oracle flow under check_flow.
"""
import pytest
import torch

from oracle import compensate as ocomp
from oracle import flows as oflows
from oracle import hessian as ohess
from oracle import quant as oquant
from oracle.parity import check_flow, check_stage_b, element_params, stage_b, summary, \
    unpack_codes
from tests._util import gen

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

# β = mean_j(1 − √(1 − x_j)) in fp32 cancels for x_j ≪ 1: each term carries a
# few ulps of 1 whatever x_j's accuracy, so β is held to 1e-3 relative plus
# 2 ulps of 1.
BETA_FLOOR = 2 * torch.finfo(torch.float32).eps


def _tokens(n, C, g, dev, chunk=16384):
    sig = torch.exp(torch.randn(C, device=dev, generator=g))
    X = torch.empty(n, C, device=dev, dtype=torch.bfloat16)
    for t0 in range(0, n, chunk):
        t1 = min(n, t0 + chunk)
        X[t0:t1] = (torch.randn(t1 - t0, C, device=dev, generator=g) * sig).bfloat16()
    return X, sig


def test_config1_as_specified(dev):
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    R = C = 4096
    N, seq, batch = 262144, 2048, 8192
    print(f"config 1: fp32 {R}x{C}, 41 outlier columns x10, {N} tokens, GPTQ W4 asym g128",
          flush=True)
    g = torch.Generator(device=dev).manual_seed(42)
    X, _ = _tokens(N, C, g, dev)
    w = torch.randn(R, C, device=dev, generator=g) * 0.02
    cols = torch.randperm(C, device=dev, generator=g)[:round(0.01 * C)]
    assert cols.numel() == 41
    w[:, cols] *= 10
    lin = torch.nn.Linear(C, R, bias=False, device=dev, dtype=torch.float32)
    with torch.no_grad():
        lin.weight.copy_(w)
    W0 = lin.weight.detach().cpu().clone().unsqueeze(0)
    gq = GPTQ([lin])
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=False)
    gq.quantizer = make_group_quantizers(q, C, 128)
    st = ohess.gptq_state(1, C)
    for t0 in range(0, N, batch):
        xb = X[t0:t0 + batch].view(-1, seq, C)
        gq.add_batch(0, xb, None)
        ohess.gptq_add_batch(st, 0, xb.cpu())
    del X
    H = st["H"].clone()
    Hd = gq.H[0].detach().cpu()
    d = torch.diagonal(H[0]).double()
    hrel = ((Hd.double() - H[0].double()).abs() / torch.sqrt(d[:, None] * d[None, :])).max()
    print(f"Hessian: HIP vs the oracle's fp32 accumulation, max |ΔH| / sqrt(H_ii·H_jj) = "
          f"{hrel.item():.3g}", flush=True)
    assert hrel.item() <= 2e-5
    gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip",
                   export_compressed_tensors=True)
    torch.cuda.synchronize()
    assert lin.weight.dtype == torch.float32
    ref = oflows.gptq_fasterquant(W0, H, 4, False, groupsize=128)
    check_flow("config 1 (fp32 4096x4096, 262144 tokens)", [lin], gq.quantizer, ref, W0, H, 4,
               128, False)


def _p_fp64_rows(D, U, I, alpha, chunk=4096):
    """α·triu(D·Uᵀ, 1)[I, :] in fp64 (rows I of T = D·Uᵀ, entries k ≤ i zeroed),
    and the componentwise magnitude |D|·|U|ᵀ of the same rows."""
    C = U.shape[-1]
    Dr = D[I].double()
    T = torch.empty(I.numel(), C, dtype=torch.float64, device=U.device)
    Ta = torch.empty_like(T)
    for k0 in range(0, C, chunk):
        Uk = U[k0:k0 + chunk].double()
        T[:, k0:k0 + chunk] = Dr @ Uk.T
        Ta[:, k0:k0 + chunk] = Dr.abs() @ Uk.abs().T
    keep = torch.arange(C, device=U.device)[None, :] > I[:, None]
    return alpha * T * keep, alpha * Ta * keep


def test_config5_full_width_sampled_rows(dev):
    from g2ptq_amd import GPTAQ, WeightQuantizer, _core, _lib, make_group_quantizers
    R, C, N, tb, bits, gs, alpha = 8192, 28672, 65536, 4096, 2, 64, 0.25
    print(f"config 5: GPTAQ W{bits} g{gs}, {R}x{C}, {N} tokens, alpha {alpha}", flush=True)
    g = torch.Generator(device=dev).manual_seed(46)
    X, sig = _tokens(N, C, g, dev, chunk=8192)
    lin = torch.nn.Linear(C, R, bias=False, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(R, C, device=dev, generator=g) * 0.02)
    W0 = lin.weight.detach().float().clone().unsqueeze(0)
    gq = GPTAQ([lin])
    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, gs)
    for t0 in range(0, N, tb):
        x = X[t0:t0 + tb]
        xfp = (x.float() + 0.05 * sig * torch.randn(tb, C, device=dev, generator=g)).bfloat16()
        gq.fp_inp[0].append(xfp)
        gq.add_batch(0, x.unsqueeze(0), None)
    del X
    # the HIP's own U and P, as GPTAQ.fasterquant forms them (deterministic: the
    # flow below recomputes the same bits)
    H = gq.H.clone()
    Dx = gq.dXXT.clone()
    _core.prepare_hessian(H, W0.clone(), Dx=Dx)
    U, damps = _core.factor(H, 0.01)
    del H
    P = torch.empty_like(U)
    ws = torch.empty(C * C * 4 + 256, dtype=torch.uint8, device=dev)
    _lib.call("g2ptq_gptaq_p", _core.stream(), _lib.ptr(Dx), _lib.ptr(U), 1, C,
              _core.f32(alpha), _lib.ptr(P), _lib.ptr(ws), ws.numel())
    del ws
    torch.cuda.synchronize()
    # (1) P on 256 sampled entries against fp64, within 1e-5 of the
    # componentwise magnitude α·|triu(D·Uᵀ, 1)|·|U| (fp32-accurate products)
    gi = gen(47)
    I = torch.randint(0, C - 1, (64,), generator=gi).to(dev)
    J = torch.randint(0, C, (256,), generator=gi).to(dev)
    Ii = I.repeat_interleave(4)
    T64, Ta = _p_fp64_rows(Dx[0], U[0], I, alpha)
    del Dx
    UJ = U[0][:, J].double()
    rows = torch.arange(256, device=dev) // 4
    ref = (T64[rows] * UJ.T).sum(1)
    mag = (Ta[rows] * UJ.T.abs()).sum(1)
    got = P[0][Ii, J].double()
    perr = ((got - ref).abs() / mag.clamp_min(1e-30)).max().item()
    print(f"P: max |P − fp64| / (α·|T|·|U|) = {perr:.3g} over 256 entries "
          f"(max |P| {ref.abs().max().item():.3g})", flush=True)
    assert perr <= 1e-5
    del T64, Ta, UJ
    # (2) the full HIP flow, then 64 sampled rows through the oracle's
    # compensation with the HIP's U and P (stage A)
    gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=gs, alpha=alpha, backend="hip",
                   export_compressed_tensors=True)
    torch.cuda.synchronize()
    assert damps == [0.01]
    rs = torch.sort(torch.randperm(R, generator=gen(48))[:64]).values
    codes = unpack_codes(lin._export_qparams["weight_packed"], bits, C)[rs]
    S, Z = element_params(gq.quantizer, R, C, gs, False)
    Uc, Pc = U.cpu(), P.cpu()
    del U, P
    oq = oquant.make_group_quantizers(
        oquant.WeightQuantizer().configure(bits, perchannel=True, sym=True), C, gs)
    Wr = W0[:, rs.to(dev)].cpu().clone()
    rec = {}
    Qr, Ir, _ = ocomp.gptaq_compensation(Wr, Uc, Pc, oq, 128, gs, False, None, None, record=rec)
    so, zo = element_params(oq, 64, C, gs, False)
    rep = stage_b(codes, Ir.reshape(64, C), rec["X"].reshape(64, C), S[rs], so, Z[rs], zo,
                  Qr.reshape(64, C))
    print(f"config 5, 64 sampled rows, stage A: {summary(rep)}", flush=True)
    check_stage_b(rep)
    Qd = lin.weight.detach()[rs.to(dev)].float().cpu()
    qh = (S[rs] * (codes - Z[rs]).float()).bfloat16().float()
    assert torch.equal(Qd, qh)


def _g2ptq_hip_inputs(gq, q, G, gs, alpha):
    """U, the RTN estimate Q0, β, Z and GH of G2PTQ.fasterquant's trust-region
    step (g2ptq_utils.py:380-476), formed by the same library calls on copies
    of the layer's state (deterministic: the flow recomputes the same bits)."""
    from g2ptq_amd import _core, _lib, make_group_quantizers
    from g2ptq_amd.common_utils import fake_quantize_grouped
    W = gq.layers[0].weight.detach().float()
    R, C = W.shape
    Rg = R // G
    W_sub = W.view(G, Rg, C).clone()
    grads = gq.gradients.view(G, Rg, C).clone()
    H = gq.H.view(G, C, C).clone()
    _core.prepare_hessian(H, W_sub, Grad=grads)
    qs = make_group_quantizers(q, C, gs)
    for i, qq in enumerate(qs):
        qq.find_params(W_sub[:, :, i * gs:(i + 1) * gs].reshape(R, -1))
    Q0 = fake_quantize_grouped(qs, W_sub, gs).contiguous()
    U, damps = _core.factor(H, 0.01)
    del H
    beta = torch.empty(R, device=W.device)
    Z, GH = torch.empty_like(W_sub), torch.empty_like(W_sub)
    ws = torch.empty(_lib.query_size("g2ptq_trust_region_workspace", G, Rg, C),
                     dtype=torch.uint8, device=W.device)
    _lib.call("g2ptq_trust_region", _core.stream(), _lib.ptr(grads), _lib.ptr(U), _lib.ptr(Q0),
              _lib.ptr(W_sub), G, Rg, C, _core.f32(alpha), 1, _lib.ptr(beta), _lib.ptr(Z),
              _lib.ptr(GH), _lib.ptr(ws), ws.numel())
    torch.cuda.synchronize()
    return W_sub, grads, U, damps, Q0, beta.view(G, Rg), Z, GH


def test_config3_down_proj_full_width_sampled_rows(dev):
    from g2ptq_amd import G2PTQ, WeightQuantizer, make_group_quantizers
    R, C, G, N, tb, bits, gs, alpha = 4096, 14336, 4, 32768, 4096, 3, 128, 0.1
    Rg, per = R // G, 16
    print(f"config 3 down_proj: G2PTQ W{bits} g{gs}, {R}x{C} in {G} row groups, {N} tokens, "
          f"alpha {alpha}", flush=True)
    g = torch.Generator(device=dev).manual_seed(49)
    X, _ = _tokens(N, C, g, dev, chunk=8192)
    sal = torch.exp(0.5 * torch.randn(N, 1, device=dev, generator=g)) * \
        torch.rand(N, G, device=dev, generator=g)
    lin = torch.nn.Linear(C, R, bias=False, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(R, C, device=dev, generator=g) * 0.02)
    # per-output-channel gradients 1e-3·N(0,1) with Student-t(3) row scales
    chi = torch.randn(3, R, 1, device=dev, generator=g).pow(2).sum(0)
    tau = (torch.randn(R, 1, device=dev, generator=g) / torch.sqrt(chi / 3)).abs()
    grads = 1e-3 * torch.randn(R, C, device=dev, generator=g) * tau
    batches = range(0, N, tb)
    gq = G2PTQ([lin], [[sal[i:i + tb] for i in batches]], [grads], G)
    q = WeightQuantizer()
    q.configure(bits, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, gs)
    for i in batches:
        gq.add_batch(0, X[i:i + tb].unsqueeze(0), None)
    del X, sal
    W_sub, Gr, U, damps, Q0, beta, Z, GH = _g2ptq_hip_inputs(gq, q, G, gs, alpha)
    assert damps == [0.01] * G
    gi = gen(50)
    local = torch.stack([torch.sort(torch.randperm(Rg, generator=gi)[:per]).values
                         for _ in range(G)])                     # (G, per)
    rows = (local + Rg * torch.arange(G)[:, None]).flatten()     # rows of the layer
    li = local.to(dev)

    def pick(t):
        return torch.stack([t[k, li[k]] for k in range(G)])    # (G, per, C)

    Wr, Grr, Q0r, Zr, GHr = (pick(t) for t in (W_sub, Gr, Q0, Z, GH))
    br = torch.stack([beta[k, li[k]] for k in range(G)])
    del W_sub, Gr, Q0, Z, GH
    # (1) the trust region on the sampled rows against the oracle in fp64 on
    # the same U (β, Z and GH are row-local given U)
    ze, ge, be = 0.0, 0.0, 0.0
    for k in range(G):
        U64 = U[k].double()
        Ainv = (U64.T @ U64).cpu()
        b64, Z64, GH64 = oflows.g2ptq_trust_region(
            Grr[k:k + 1].double().cpu(), Ainv[None], U64.cpu()[None], Q0r[k:k + 1].double().cpu(),
            Wr[k:k + 1].double().cpu(), alpha, True)
        del Ainv, U64
        b = br[k].double().cpu()
        be = max(be, float(((b - b64[0]).abs() / (1e-3 * b64[0].abs() + BETA_FLOOR)).max()))
        for got, ref, acc in ((Zr[k], Z64[0], "z"), (GHr[k], GH64[0], "g")):
            # Z/β = Grad·Uᵀ and GH/β = Grad·A⁻¹, each row against its largest entry
            got = got.double().cpu() / b[:, None]
            ref = ref / b64[0][:, None]
            e = ((got - ref).abs().amax(-1) / ref.abs().amax(-1)).max().item()
            if acc == "z":
                ze = max(ze, e)
            else:
                ge = max(ge, e)
    print(f"trust region, {G}x{per} rows: beta range [{br.min():.4g}, {br.max():.4g}], "
          f"|β − fp64| / (1e-3·β + floor) ≤ {be:.3g}; Z/β rel to row max {ze:.3g}, GH/β {ge:.3g}",
          flush=True)
    assert float(br.min()) > 0
    assert be <= 1.0 and ze <= 1e-4 and ge <= 1e-4, (be, ze, ge)
    # (2) the full HIP flow, then the sampled rows through the oracle's
    # compensation with the HIP's U, Z and GH (stage A)
    gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=gs, alpha=alpha, backend="hip",
                   export_compressed_tensors=True)
    torch.cuda.synchronize()
    assert torch.equal(gq._beta, beta), "the flow's β differs from the same calls' β"
    codes = unpack_codes(lin._export_qparams["weight_packed"], bits, C)[rows]
    S, Zq = element_params(gq.quantizer, R, C, gs, False)
    Uc = U.cpu()
    del U
    oq = oquant.make_group_quantizers(
        oquant.WeightQuantizer().configure(bits, perchannel=True, sym=True), C, gs)
    rec = {}
    Qr, Ir, _ = ocomp.g2ptq_compensation(Wr.cpu(), Uc, Zr.cpu(), GHr.cpu().clone(), oq, 128, gs,
                                         False, None, None, record=rec)
    n = G * per
    so, zo = element_params(oq, n, C, gs, False)
    rep = stage_b(codes, Ir.reshape(n, C), rec["X"].reshape(n, C), S[rows], so, Zq[rows], zo,
                  Qr.reshape(n, C))
    print(f"config 3 down_proj, {n} sampled rows, stage A: {summary(rep)}", flush=True)
    check_stage_b(rep)
    Qd = lin.weight.detach()[rows.to(dev)].float().cpu()
    qh = (S[rows] * (codes - Zq[rows]).float()).bfloat16().float()
    assert torch.equal(Qd, qh)


def _routing(n, E, topk, g):
    """Gumbel-top-k over log p_e with p_e ∝ (e+1)^-1.1: each token's experts."""
    logp = -1.1 * torch.log(torch.arange(1, E + 1, dtype=torch.float32))
    u = torch.rand(n, E, generator=g).clamp_(1e-20, 1.0)
    return torch.topk(logp - torch.log(-torch.log(u)), topk, dim=1).indices


def test_config4_expert_shapes(dev):
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    from g2ptq_amd.shared import SharedInputHessian
    E, topk, hid, inter, n, tb = 128, 8, 2048, 768, 32768, 8192
    Egu, Ed = 32, 64
    print(f"config 4 shapes: {Egu} experts' gate/up {inter}x{hid} as 64 slots, {Ed} experts' "
          f"down {hid}x{inter}, {n} tokens top-{topk} of {E}", flush=True)
    g = gen(4045)
    sig_h = torch.exp(torch.randn(hid, generator=g))
    sig_i = torch.exp(torch.randn(inter, generator=g))

    def linear(R, C):
        lin = torch.nn.Linear(C, R, bias=False)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(R, C, generator=g) * 0.02)
        return lin.to(dev).to(torch.bfloat16)

    gu = [linear(inter, hid) for _ in range(2 * Egu)]     # e0.gate, e0.up, e1.gate, …
    dn = [linear(hid, inter) for _ in range(Ed)]
    W_gu = torch.stack([l.weight.detach().float().cpu() for l in gu])
    W_dn = torch.stack([l.weight.detach().float().cpu() for l in dn])
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    g_gu, g_dn = GPTQ(gu), GPTQ(dn)
    g_gu.quantizer = make_group_quantizers(q, hid, 128)
    g_dn.quantizer = make_group_quantizers(q, inter, 128)
    shares = [SharedInputHessian([(g_gu, 2 * e), (g_gu, 2 * e + 1)]) for e in range(Egu)]
    st_gu, st_dn = ohess.gptq_state(Egu, hid), ohess.gptq_state(Ed, inter)
    counts = torch.zeros(E, dtype=torch.int64)
    for t0 in range(0, n, tb):
        x = (torch.randn(tb, hid, generator=g) * sig_h).bfloat16()
        top = _routing(tb, E, topk, g)
        for e in range(Ed):
            sel = (top == e).any(1)
            k = int(sel.sum())
            counts[e] += k
            if k == 0:
                continue
            xg = x[sel]
            xd = (torch.randn(k, inter, generator=g) * sig_i).bfloat16()
            if e < Egu:
                shares[e].add_batch(xg.to(dev))
                ohess.gptq_add_batch(st_gu, e, xg)
            g_dn.add_batch(e, xd.to(dev), None)
            ohess.gptq_add_batch(st_dn, e, xd)
    print(f"routed tokens of the tested experts: {counts[:Ed].tolist()}", flush=True)
    assert counts[:Ed].min() > 0 and counts[0] > 8 * counts[Ed - 1]
    for sh in shares:
        sh.finalize()
    assert g_gu._h_alias == {2 * e + 1: 2 * e for e in range(Egu)}
    H_gu = st_gu["H"].repeat_interleave(2, dim=0)          # gate and up: one Hessian
    H_dn = st_dn["H"].clone()
    for inst in (g_gu, g_dn):
        inst.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip",
                         export_compressed_tensors=True)
    torch.cuda.synchronize()
    ref = oflows.gptq_fasterquant(W_gu, H_gu.clone(), 4, True, groupsize=128)
    check_flow("config 4 gate/up, 64 slots of 768x2048", gu, g_gu.quantizer, ref, W_gu, H_gu, 4,
               128, False)
    ref = oflows.gptq_fasterquant(W_dn, H_dn.clone(), 4, True, groupsize=128)
    check_flow("config 4 down, 64 experts of 2048x768", dn, g_dn.quantizer, ref, W_dn, H_dn, 4,
               128, False)
