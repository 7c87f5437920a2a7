"""GPU: G2PTQ's trust region (g2ptq_trust_region) against the oracle.

gptq_utils/g2ptq_utils.py:459-476.  The HIP entry forms Grad·A⁻¹ as
(Grad·Uᵀ)·U and diag(A⁻¹) as the column norms of U; the oracle follows the
reference (an explicit A⁻¹ from cholesky_inverse).  Both get the same U.
"""
import pytest
import torch

from oracle import factor as ofactor
from oracle import flows as oflows
from oracle import quant as oquant
from tests._util import gen

pytestmark = pytest.mark.gpu


def _hip_trust_region(grad, U, Q0, W0, alpha, enabled=True):
    from g2ptq_amd import _core, _lib
    dev = torch.device("cuda:0")
    BG, Rg, C = grad.shape
    g, u, q, w = (t.float().contiguous().to(dev) for t in (grad, U, Q0, W0))
    beta = torch.empty(BG * Rg, device=dev)
    Z = torch.empty(BG, Rg, C, device=dev)
    GH = torch.empty_like(Z)
    ws = torch.empty(_lib.query_size("g2ptq_trust_region_workspace", BG, Rg, C),
                     dtype=torch.uint8, device=dev)
    _lib.call("g2ptq_trust_region", _core.stream(), _lib.ptr(g), _lib.ptr(u), _lib.ptr(q),
              _lib.ptr(w), BG, Rg, C, _core.f32(alpha), int(enabled), _lib.ptr(beta), _lib.ptr(Z),
              _lib.ptr(GH), _lib.ptr(ws), ws.numel())
    torch.cuda.synchronize()
    return beta.view(BG, Rg).cpu(), Z.cpu(), GH.cpu()


def test_trust_region_hand_computed_case(dev):
    """The 1×2 case worked by hand (A = [[2, 1], [1, 2]], Grad = [1, 2],
    E0 = [1/2, −1/4]): β = 1 − (√(157/160) + √(139/160))/2 at α = 0.1 and
    (2 − √(5/8))/2 at α = 2, to fp32 accuracy."""
    import math
    Ainv = torch.tensor([[[2.0, -1.0], [-1.0, 2.0]]], dtype=torch.float64) / 3
    U = torch.linalg.cholesky(Ainv, upper=True)
    grad = torch.tensor([[[1.0, 2.0]]])
    W = torch.zeros(1, 1, 2)
    Q = torch.tensor([[[0.5, -0.25]]])
    for alpha, exp in ((0.1, 1 - (math.sqrt(157 / 160) + math.sqrt(139 / 160)) / 2),
                       (2.0, (2 - math.sqrt(5 / 8)) / 2)):
        beta, Z, GH = _hip_trust_region(grad, U, Q, W, alpha)
        assert abs(float(beta) - exp) <= 2e-6 * exp, (alpha, float(beta), exp)
        assert torch.allclose(GH[0, 0], torch.tensor([0.0, float(beta)]), atol=1e-6)


def _cfg3_inputs(C, Rg, G, seed, T=None, dead=None):
    """Config-3-style inputs: G row-group Hessians from LogNormal-scaled tokens
    with per-group saliency weights, W ~ N(0, 0.02), W3 sym g128 RTN estimate
    Q0 (groups fitted on W), gradients 1e-3·N(0,1)·|t₃| per row."""
    g = gen(seed)
    T = T or C
    sig = torch.exp(torch.randn(C, generator=g))
    X = (torch.randn(T, C, generator=g) * sig).bfloat16().float()
    if dead is not None:
        X[:, dead] = 0
    U, Ainv = [], []
    for _ in range(G):
        s = torch.rand(T, 1, generator=g) + 0.1
        H = (X * s).T @ X / T
        d = torch.diagonal(H)
        H[d == 0, d == 0] = 1
        u, _, a = ofactor.damp_chol_inv_upper(H, 0.01, want_inverse=True)
        U.append(u)
        Ainv.append(a)
    U, Ainv = torch.stack(U), torch.stack(Ainv)
    W = torch.randn(G, Rg, C, generator=g) * 0.02
    if dead is not None:
        W[:, :, dead] = 0
    qz = oquant.WeightQuantizer().configure(3, perchannel=True, sym=True)
    qs = oquant.make_group_quantizers(qz, C, 128)
    for i, q in enumerate(qs):
        q.find_params(W[:, :, i * 128:(i + 1) * 128].reshape(G * Rg, -1))
    Q0 = oquant.fake_quantize_grouped(qs, W, 128)
    z = torch.randn(G, Rg, C, generator=g)
    chi = torch.randn(3, G, Rg, 1, generator=g).pow(2).sum(0)
    tau = (torch.randn(G, Rg, 1, generator=g) / torch.sqrt(chi / 3)).abs()
    grad = 1e-3 * z * tau
    return grad, Ainv, U, Q0, W


# β = mean_j(1 − √(1 − x_j)) is evaluated in fp32 by the reference and here;
# for x_j ≪ 1 the subtraction cancels, and each term carries an absolute error
# of a few ulps of 1 whatever x_j's accuracy.  β is therefore held to 1e-3
# relative plus that floor, 2 ulps of 1 (2.4e-7).
BETA_FLOOR = 2 * torch.finfo(torch.float32).eps


def _beta_close(beta, beta_r, what):
    err = (beta - beta_r).abs()
    bound = 1e-3 * beta_r.abs() + BETA_FLOOR
    worst = float((err / bound).max())
    assert worst <= 1.0, (what, worst, float(err.max()))


@pytest.mark.parametrize("C,Rg", [(256, 64), (4096, 256)])
def test_trust_region_matches_oracle(dev, C, Rg):
    """Config 3 settings (G = 4, W3 g128, α = 0.1): β per row within 1e-3
    relative plus the fp32 cancellation floor; Z/β = Grad·Uᵀ and GH/β =
    Grad·A⁻¹ within 1e-3 of each row's largest entry.  An fp64 evaluation on
    the same U shows both sides' distance from exact arithmetic."""
    G, alpha = 4, 0.1
    print(f"trust region C={C} Rg={Rg}", flush=True)
    grad, Ainv, U, Q0, W = _cfg3_inputs(C, Rg, G, 500 + C)
    beta_r, Z_r, GH_r = oflows.g2ptq_trust_region(grad, Ainv, U, Q0, W, alpha, True)
    beta, Z, GH = _hip_trust_region(grad, U, Q0, W, alpha)
    U64 = U.double()
    beta_64, _, _ = oflows.g2ptq_trust_region(grad.double(), U64.transpose(1, 2) @ U64, U64,
                                              Q0.double(), W.double(), alpha, True)
    assert float(beta_r.min()) > 0
    e_h = float(((beta.double() - beta_64).abs() / beta_64).max())
    e_r = float(((beta_r.double() - beta_64).abs() / beta_64).max())
    br, b = beta_r.unsqueeze(2), beta.unsqueeze(2)
    zr = ((Z / b - Z_r / br).abs().amax(-1) / (Z_r / br).abs().amax(-1)).max().item()
    gr = ((GH / b - GH_r / br).abs().amax(-1) / (GH_r / br).abs().amax(-1)).max().item()
    print(f"C={C}: beta range [{beta_r.min():.4g}, {beta_r.max():.4g}]; max relative distance "
          f"from fp64: HIP {e_h:.3g}, oracle {e_r:.3g}; Grad·Uᵀ rel {zr:.3g}, "
          f"Grad·A⁻¹ rel {gr:.3g}", flush=True)
    _beta_close(beta, beta_r, f"beta C={C}")
    assert zr <= 1e-3, zr
    assert gr <= 1e-3, gr


def test_trust_region_dead_features(dev):
    """Dead features (zero Hessian diagonal set to 1, zero weight columns)
    keep their gradient columns (g2ptq_utils.py:394-401): they still count in
    every row's c sum, and β follows the oracle."""
    dead = torch.tensor([0, 5, 77, 255])
    grad, Ainv, U, Q0, W = _cfg3_inputs(256, 64, 4, 777, dead=dead)
    assert float(grad[:, :, dead].abs().min()) > 0
    beta_r, _, GH_r = oflows.g2ptq_trust_region(grad, Ainv, U, Q0, W, 0.1, True)
    beta, _, GH = _hip_trust_region(grad, U, Q0, W, 0.1)
    _beta_close(beta, beta_r, "beta with dead features")


def test_trust_region_disabled_is_zero(dev):
    grad, Ainv, U, Q0, W = _cfg3_inputs(256, 16, 2, 778)
    beta, Z, GH = _hip_trust_region(grad, U, Q0, W, 0.1, enabled=False)
    assert torch.all(beta == 0) and torch.all(Z == 0) and torch.all(GH == 0)
