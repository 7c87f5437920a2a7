"""GPU: size-independent properties at the benchmark configurations' full sizes.

The CPU oracle cannot run these sizes in a test, so each check is a property
exact arithmetic fixes, evaluated in fp64:

* config 2's down_proj (C = 14336, 262,144 calibration tokens): sampled
  Hessian entries equal (2/n)·Σ_t x_ti·x_tj (gptq_utils.py:115-126); and the
  compensation is self-consistent — with E = (W − Q)·U⁻¹ (the GPTQ identity
  W − Q = E·U, gptq_utils.py:28-51, 180-230), every pre-quantization value
  x_j = q_j + E_j·U_jj rounds to its code under its group's scale; and 64
  sampled rows match the oracle's compensation run from the HIP's own U
  (stage A: rows are independent given U);
* config 2's q/k/v input (C = 4096, 262,144 tokens): every Hessian entry
  against fp64 sums; this Gram splits K 15 ways (the count that fills the
  last wave of workgroups), so the tokens are zero-padded to a multiple of
  15·128;
* config 5's factor (C = 28672, GPTAQ's 70B down_proj width): A·UᵀU = I on
  sampled columns (A = H + 0.01·mean(diag H)·I, gptq_utils.py:291-302), with
  a residual no worse than the reference's own fp32 chain
  cholesky → cholesky_inverse → cholesky evaluated by torch on the same GPU.
"""
import pytest
import torch

from tests._util import gen

pytestmark = pytest.mark.gpu


def _acts(n, C, seed, dev, chunk=16384):
    """LogNormal-channel bf16 activations generated on the device (n × C)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    sig = torch.exp(torch.randn(C, device=dev, generator=g))
    x = torch.empty(n, C, device=dev, dtype=torch.bfloat16)
    for t0 in range(0, n, chunk):
        t1 = min(n, t0 + chunk)
        x[t0:t1] = (torch.randn(t1 - t0, C, device=dev, generator=g) * sig).bfloat16()
    return x


def _accumulate(inst, X, batch):
    """add_batch over (4, 2048)-token sequences like the reference scripts."""
    T, C = X.shape
    for t0 in range(0, T, batch):
        inst.add_batch(0, X[t0:t0 + batch].view(-1, 2048, C), None)


def test_down_proj_hessian_and_compensation_at_full_size(dev):
    from g2ptq_amd import GPTQ, WeightQuantizer, _core, make_group_quantizers
    R, C, N = 4096, 14336, 262144
    print(f"full-size down_proj: R={R} C={C} tokens={N}", flush=True)
    X = _acts(N, C, 71, dev)
    lin = torch.nn.Linear(C, R, bias=False, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(R, C, device=dev,
                                     generator=torch.Generator(device=dev).manual_seed(72)) * 0.02)
    W0 = lin.weight.detach().float().clone()
    gq = GPTQ([lin])
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, 128)
    _accumulate(gq, X, 8192)
    H = gq.H[0]
    # (1) sampled Hessian entries against fp64 sums over all tokens; n counts
    # the 128 sequences of 2048 tokens
    g = gen(73)
    I = torch.randint(0, C, (256,), generator=g).to(dev)
    J = torch.randint(0, C, (256,), generator=g).to(dev)
    I[:32] = J[:32]  # diagonal entries too
    cols = torch.unique(torch.cat([I, J]))
    pos = {int(c): k for k, c in enumerate(cols.tolist())}
    Xs = X[:, cols].double()
    G = Xs.T @ Xs * (2.0 / 128)
    ref = torch.stack([G[pos[int(i)], pos[int(j)]] for i, j in zip(I.tolist(), J.tolist())])
    got = H[I, J].double()
    d = torch.diagonal(H).double()
    scale = torch.sqrt(d[I] * d[J])
    err = ((got - ref).abs() / scale).max().item()
    print(f"Hessian: max |H_ij − fp64| / sqrt(H_ii·H_jj) = {err:.3g} over 256 entries", flush=True)
    assert err <= 2e-5, err
    del X, Xs
    # (2) the compensation: the factor it uses, then the run itself
    Hp = gq.H.clone()
    _core.prepare_hessian(Hp, W0.unsqueeze(0).clone())
    U, _ = _core.factor(Hp, 0.01)
    U = U[0]
    del Hp
    gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip",
                   export_compressed_tensors=True)
    torch.cuda.synchronize()
    from oracle.parity import element_params, unpack_codes
    codes = unpack_codes(lin._export_qparams["weight_packed"], 4, C).to(dev).double()
    S, Z = element_params(gq.quantizer, R, C, 128, False)
    S, Z = S.to(dev).double(), Z.to(dev).double()
    rows = torch.randint(0, R, (256,), generator=gen(74)).to(dev)
    Q = (S[rows] * (codes[rows] - Z[rows]))
    assert torch.equal(Q.float().bfloat16().float(), lin.weight[rows].float())
    D = W0[rows].double() - Q                        # = E·U
    E = torch.linalg.solve_triangular(U.double(), D, upper=True, left=False)
    x = Q + E * torch.diagonal(U).double()           # values when quantized
    t = x / S[rows] - (codes[rows] - Z[rows])        # offset from the chosen grid point
    inside = (codes[rows] > -8) & (codes[rows] < 7)  # not clamped at the grid's ends
    worst = t[inside].abs().max().item()
    over = (t[inside].abs() > 0.5).double().mean().item()
    print(f"compensation: max |x/s − (q − z)| = {worst:.6f} (0.5 at a rounding tie), "
          f"{100 * over:.4f} % of entries past 0.5", flush=True)
    assert worst <= 0.5 + 1e-3, worst
    assert over <= 1e-4, over
    # clamped codes lie beyond the grid on their side
    lo = codes[rows] == -8
    hi = codes[rows] == 7
    assert (t[lo] <= 0.5 + 1e-3).all() and (t[hi] >= -0.5 - 1e-3).all()
    # (3) stage A on 64 sampled rows: the oracle's compensation
    # (gptq_utils.py:165-232) from the HIP's own U, rows being independent
    # given U
    from oracle import compensate as ocomp
    from oracle import quant as oquant
    from oracle.parity import check_stage_b, stage_b, summary
    rs = torch.sort(torch.randperm(R, generator=gen(75))[:64]).values.to(dev)
    oq = oquant.make_group_quantizers(
        oquant.WeightQuantizer().configure(4, perchannel=True, sym=True), C, 128)
    rec = {}
    Qr, Ir, _ = ocomp.gptq_compensation(W0[rs].cpu().unsqueeze(0), U.cpu().unsqueeze(0), oq, 128,
                                        128, False, None, None, record=rec)
    so, zo = element_params(oq, 64, C, 128, False)
    rep = stage_b(codes[rs], Ir.reshape(64, C), rec["X"].reshape(64, C), S[rs], so, Z[rs], zo,
                  Qr.reshape(64, C))
    print(f"down_proj, 64 sampled rows, stage A: {summary(rep)}", flush=True)
    check_stage_b(rep)


def test_qkv_hessian_at_full_size(dev):
    from g2ptq_amd import GPTQ, _lib
    C, N = 4096, 262144
    tiles = (C // 256) * (C // 256 + 1) // 2
    splits = _lib.query_size("g2ptq_hessian_gram_workspace", N, C) // (tiles * 256 * 256 * 4)
    print(f"full-size q/k/v Hessian: C={C} tokens={N}, {splits} K splits", flush=True)
    assert splits == 15
    X = _acts(N, C, 81, dev)
    lin = torch.nn.Linear(C, 256, bias=False, device=dev, dtype=torch.bfloat16)
    gq = GPTQ([lin])
    _accumulate(gq, X, 8192)
    H = gq.H[0].double()
    Xd = X.double()
    del X
    ref = Xd.T @ Xd * (2.0 / 128)  # 128 sequences of 2048 tokens
    del Xd
    d = torch.diagonal(ref)
    err = ((H - ref).abs() / torch.sqrt(d.unsqueeze(1) * d.unsqueeze(0))).max().item()
    print(f"Hessian: max |H − fp64| / sqrt(H_ii·H_jj) = {err:.3g} over all entries", flush=True)
    assert err <= 2e-5, err


def test_cfg5_factor_at_full_width(dev):
    from g2ptq_amd import GPTQ, _core
    C, N = 28672, 65536
    print(f"full-width factor: C={C} tokens={N}", flush=True)
    lin = torch.nn.Linear(C, 64, bias=False, device=dev, dtype=torch.bfloat16)
    gq = GPTQ([lin])
    X = _acts(N, C, 81, dev, chunk=8192)
    _accumulate(gq, X, 4096)
    del X
    H = gq.H
    Hp = H.clone()
    _core.prepare_hessian(Hp, torch.zeros(1, 64, C, device=dev))
    U, damps = _core.factor(Hp, 0.01)
    U = U[0]
    assert damps == [0.01]
    A = Hp[0]
    damp = 0.01 * torch.diagonal(A).mean()
    A.diagonal().add_(damp)
    J = torch.randint(0, C, (64,), generator=gen(82)).to(dev)

    def residual(Uf):
        """‖A·(Uᵀ·U)·e_j − e_j‖ for the sampled columns, in fp64 by row blocks."""
        V = Uf[:, J].double()                          # U·e_j
        Wt = torch.zeros(C, J.numel(), dtype=torch.float64, device=dev)
        for r0 in range(0, C, 4096):
            Wt += Uf[r0:r0 + 4096].double().T @ V[r0:r0 + 4096]
        Rm = torch.zeros_like(Wt)
        for r0 in range(0, C, 4096):
            Rm[r0:r0 + 4096] = A[r0:r0 + 4096].double() @ Wt
        Rm[J, torch.arange(J.numel(), device=dev)] -= 1
        return Rm.norm(dim=0)

    ours = residual(U)
    # the reference's chain (gptq_utils.py:295-302) in torch fp32 on this GPU
    L = torch.linalg.cholesky(A)
    Ainv = torch.cholesky_inverse(L)
    del L
    Uref = torch.linalg.cholesky(Ainv, upper=True)
    del Ainv
    theirs = residual(Uref)
    gersh = A.abs().sum(1).max().item()
    cond_bound = gersh / damp.item()
    print(f"factor C={C}: residual max {ours.max().item():.3g} (reference chain "
          f"{theirs.max().item():.3g}), cond(A) ≤ {cond_bound:.3g}", flush=True)
    assert torch.isfinite(ours).all()
    assert ours.max().item() <= 2 * theirs.max().item() + 1e-6
    assert ours.max().item() <= 1e-7 * cond_bound
