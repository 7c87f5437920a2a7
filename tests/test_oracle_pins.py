"""Pins of the CPU oracle (no GPU): every oracle function is checked against
something other than its own formula — closed forms, known answers, fp64
brute force, invariants, and the reference test's independent pre-refactor
loops (restated in oracle.original_loops)."""
import copy
import math

import pytest
import torch

from oracle import compensate as ocomp
from oracle import factor as ofactor
from oracle import flows as oflows
from oracle import hessian as ohess
from oracle import original_loops as oloops
from oracle import pack as opack
from oracle import quant as oquant
from tests._util import g2_inputs, gen, gptaq_p, ref_inputs


# ---------------------------------------------------------------------------
# Quantizer (utils/quant_utils.py)
# ---------------------------------------------------------------------------

def test_quant_known_answer_asym_4bit():
    """b=4 asym over [-1.5, 2.25] (all values exact in fp32): s = 3.75/15 = 0.25,
    z = round(-8 + 1.5/0.25) = -2; codes clamp(round(x/s) + z, -8, 7)."""
    x = torch.tensor([[-1.5, 2.25, 0.625, 0.875, 0.1]])
    s, z = oquant.find_params(x, 4, sym=False)
    assert s.item() == 0.25 and z.item() == -2.0
    q, _, _ = oquant.asym_quant(x, s, z, 7)
    # 0.625/s = 2.5 → 2 (half-even); 0.875/s = 3.5 → 4; 0.1/s = 0.4 → 0
    assert q.tolist() == [[-8.0, 7.0, 0.0, 2.0, -2.0]]
    assert oquant.asym_dequant(q, s, z).tolist() == [[-1.5, 2.25, 0.5, 1.0, 0.0]]


def test_quant_known_answer_sym():
    """sym: s = max(|xmin|, xmax)/(bit_range/2); 4-bit bit_range/2 = 7.5."""
    x = torch.tensor([[-0.3, 0.75, 0.1]])
    s, z = oquant.find_params(x, 4, sym=True)
    assert s.item() == torch.tensor(0.75) / torch.tensor(7.5)
    assert z.item() == 0.0


def test_quant_half_to_even_ties():
    """torch.round is half-to-even: 2.5 → 2, -1.5 → -2, 0.5 → 0, 3.5 → 4."""
    s = torch.ones(1, 1)
    x = torch.tensor([[2.5, -1.5, 0.5, 3.5]])
    q, _, _ = oquant.asym_quant(x, s, torch.zeros(1, 1), 7)
    assert q.tolist() == [[2.0, -2.0, 0.0, 4.0]]


def test_quant_all_zero_group_scale_zero():
    s, _ = oquant.find_params(torch.zeros(2, 8), 4, sym=True)
    assert torch.all(s == 0)  # the reference asserts scale > 0 on this input


def test_quant_ranges_include_zero():
    x = torch.tensor([[0.5, 1.0], [-1.0, -0.25]])
    s, z = oquant.find_params(x, 4, sym=False)
    # xmin clamps to 0 on the positive row: s = 1/15, z = round(-8 - 0) = -8
    assert s[0, 0] == torch.tensor(1.0) / 15 and z[0, 0].item() == -8.0
    # xmax clamps to 0 on the negative row: z = clamp(round(-8 + 15)) = 7
    assert z[1, 0].item() == 7.0


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("sym", [True, False])
def test_quant_unified_asym_matches_fake_quantize(bits, sym):
    """tests/test_triton_compensation.py:537-579: the unified asym path with a
    zero-filled zero point equals WeightQuantizer.fake_quantize, bit for bit."""
    w = torch.randn(2, 37, 13, generator=gen(5000 + bits * 10 + int(sym)))
    q = oquant.WeightQuantizer().configure(bits, sym=sym)
    q.find_params(w.reshape(74, 13))
    fq, codes, _ = q.fake_quantize(w[:, :, 0].reshape(74, 1))
    c2, s2, z2 = oquant.asym_quant(w[:, :, 0], q.scale.reshape(2, 37), q.zero.reshape(2, 37), q.maxq)
    assert torch.equal(c2, codes.reshape(2, 37))
    assert torch.equal(oquant.asym_dequant(c2, s2, z2), fq.reshape(2, 37))


def test_quant_mse_never_worse_than_minmax():
    x = torch.randn(16, 64, generator=gen(1)) * 0.02
    for sym in (True, False):
        s0, z0 = oquant.find_params(x, 3, sym)
        s1, z1 = oquant.find_params(x, 3, sym, mse=True)

        def err(s, z):
            q = torch.clamp(torch.round(x / s) + z, -4, 3)
            return ((s * (q - z) - x).abs() ** 2.4).sum(-1)
        assert torch.all(err(s1, z1) <= err(s0, z0) + 1e-12)


def test_quant_hclip_uniform_weights():
    """hclip: a constant H_diag of 4 (an exact power-of-two scale of every error
    term) ranks candidates exactly like the unweighted squared error (norm 2),
    not like |err|^2.4; and the quantizer drops a constant H_diag altogether
    (quant_utils.py:395-397), giving the plain norm-2.4 search."""
    x = torch.randn(24, 64, generator=gen(11)) * 0.02
    for sym in (True, False):
        h4 = torch.full((1, 1, 64), 4.0)
        s_h, z_h = oquant.find_params(x, 3, sym, mse=True, H_diag=h4)
        s_2, z_2 = oquant.find_params(x, 3, sym, mse=True, norm=2.0)
        s_24, z_24 = oquant.find_params(x, 3, sym, mse=True)
        assert torch.equal(s_h, s_2) and torch.equal(z_h, z_2)
        assert not torch.equal(s_2, s_24)  # the data tells the two objectives apart
        q = oquant.WeightQuantizer().configure(3, sym=sym, mse=True, hclip=True)
        q.find_params(x, torch.full((2, 64), 0.3))
        assert torch.equal(q.scale, s_24) and torch.equal(q.zero, z_24)


def _brute_force_clip(xrow, w, bits, sym, grid=50, maxshrink=0.5, norm=None, scores=None):
    """First strict minimum over the clip grid of sum_c (fq_c - x_c)^2 * w_c
    (or, with ``norm``, of sum_c |fq_c - x_c|^norm), one row at a time with
    scalar fp32 arithmetic (independent of the oracle's tensor reshapes).
    ``scores`` (a list) receives every candidate's objective."""
    maxq = 2 ** (bits - 1) - 1
    minq = -(maxq + 1)
    f = lambda v: torch.tensor(v, dtype=torch.float32)
    xmin = min(f(xrow.min().item()), f(0.0))
    xmax = max(f(xrow.max().item()), f(0.0))
    best, choice = math.inf, None
    steps = int(maxshrink * grid)
    for i in range(steps):
        for j in range(steps):
            lo = (1 - i / grid) * xmin
            hi = (1 - j / grid) * xmax
            if sym:
                s = torch.maximum(lo.abs(), hi) / ((maxq - minq) / 2)
                z = f(0.0)
            else:
                s = (hi - lo) / (maxq - minq)
                z = torch.clamp(torch.round(minq - lo / s), minq, maxq)
            err = 0.0
            for c in range(xrow.numel()):
                if w is not None and w[c] == 0:
                    continue
                q = torch.clamp(torch.round(xrow[c] / s) + z, minq, maxq)
                d = (s * (q - z) - xrow[c]).double().item()
                err += abs(d) ** norm if norm is not None else d * d * float(w[c])
            if scores is not None:
                scores.append(err)
            if err < best:
                best, choice = err, (s.item(), torch.round(z).item())
    return choice


def test_quant_mse_norm_objective_brute_force():
    """The plain clip search (quant_utils.py:406-425, _quant_err :84-105)
    minimises sum_c |fq_c − x_c|^2.4.  Rows with one large entry gain from
    clipping, so the search moves off min/max; the oracle's choice must be
    the scalar brute force's first strict minimum wherever the runner-up is
    more than 1e-6 relative away (fp32 sums in another order cannot swap
    such candidates), and its objective the minimum everywhere."""
    g = gen(13)
    x = torch.randn(12, 16, generator=g) * 0.02
    x[torch.arange(12), torch.randint(0, 16, (12,), generator=g)] *= 6.0
    checked = moved = 0
    for sym in (True, False):
        s_o, z_o = oquant.find_params(x, 3, sym, mse=True)
        s_m, _ = oquant.find_params(x, 3, sym)
        for r in range(12):
            scores = []
            s_b, z_b = _brute_force_clip(x[r], None, 3, sym, norm=2.4, scores=scores)
            best = min(scores)
            second = min(v for v in scores if v > best) if any(v > best for v in scores) else best
            q = torch.clamp(torch.round(x[r] / s_o[r]) + z_o[r], -4, 3)
            e_o = float(((s_o[r] * (q - z_o[r]) - x[r]).double().abs() ** 2.4).sum())
            assert e_o <= best * (1 + 1e-6), (sym, r)
            if second > best * (1 + 1e-6):
                assert s_o[r].item() == s_b and z_o[r].item() == z_b, (sym, r)
                checked += 1
            moved += int(s_o[r].item() != s_m[r].item())
    assert checked >= 16 and moved >= 12, (checked, moved)


def test_quant_hclip_rows_use_their_block_and_group():
    """hclip weights: rows split into H_diag.shape[0] consecutive blocks, and with
    weight_groupsize each row's column group k uses H_diag[b, k*g:(k+1)*g].
    One-hot weights make every row's objective a single column's error, whose
    first strict minimum is found by brute force."""
    g = gen(12)
    x = torch.randn(6, 8, generator=g) * 0.05            # 2 blocks of 3 rows
    h = torch.zeros(2, 8)
    h[0, 1] = 1.0
    h[1, 6] = 2.0
    q = oquant.WeightQuantizer().configure(3, sym=False, mse=True, hclip=True)
    q.find_params(x, h)
    for r in range(6):
        s, z = _brute_force_clip(x[r], h[r // 3], 3, False)
        assert q.scale[r, 0].item() == s and q.zero[r, 0].item() == z, r
    # grouped: 2 groups of 4 columns per row, each with its own weight column
    h2 = torch.zeros(2, 8)
    h2[0, 2] = h2[0, 5] = 1.0
    h2[1, 0] = h2[1, 7] = 1.0
    q2 = oquant.WeightQuantizer().configure(4, sym=True, mse=True, hclip=True, weight_groupsize=4)
    q2.find_params(x, h2)
    for r in range(6):
        for k in range(2):
            s, z = _brute_force_clip(x[r, 4 * k:4 * k + 4], h2[r // 3, 4 * k:4 * k + 4], 4, True)
            assert q2.scale[r, k].item() == s and q2.zero[r, k].item() == z, (r, k)


# ---------------------------------------------------------------------------
# Hessians
# ---------------------------------------------------------------------------

def test_hessian_fp64_brute_force_and_streaming():
    """H = (2/n_seq)·Σ x xᵀ over all batches; streaming == one-shot; symmetric PSD."""
    g = gen(2)
    C = 24
    batches = [torch.randn(3, 16, C, generator=g) for _ in range(4)]
    st = ohess.gptq_state(1, C)
    for x in batches:
        ohess.gptq_add_batch(st, 0, x)
    X = torch.cat([b.reshape(-1, C) for b in batches]).double()
    n_seq = sum(b.shape[0] for b in batches)
    ref = (2.0 / n_seq) * X.T @ X
    assert torch.allclose(st["H"][0].double(), ref, rtol=1e-5, atol=1e-5)
    H = st["H"][0].double()
    assert torch.allclose(H, H.T, atol=1e-6)
    assert torch.linalg.eigvalsh(H).min() > -1e-6


def test_hessian_2d_input_counts_one_sample():
    """A 2-D (MoE) input counts as one sample (gptq_utils.py:116-118)."""
    st = ohess.gptq_state(1, 4)
    x = torch.randn(10, 4, generator=gen(3))
    ohess.gptq_add_batch(st, 0, x)
    assert st["nsamples"][0] == 1
    assert torch.allclose(st["H"][0], 2 * x.T @ x, rtol=1e-5)


def test_gptaq_cross_term_brute_force():
    g = gen(4)
    C = 12
    st = ohess.gptaq_state(1, C)
    xs, fs = [], []
    for _ in range(3):
        x = torch.randn(1, 20, C, generator=g)
        f = x.reshape(-1, C) + 0.1 * torch.randn(20, C, generator=g)
        ohess.gptaq_add_batch(st, 0, x, f)
        xs.append(x.reshape(-1, C))
        fs.append(f)
    X, F = torch.cat(xs).double(), torch.cat(fs).double()
    ref = (2.0 / 3) * (F - X).T @ X
    assert torch.allclose(st["dXXT"][0].double(), ref, rtol=1e-5, atol=1e-5)


def test_gptaq_cross_term_zero_when_fp_equals_input():
    st = ohess.gptaq_state(1, 8)
    x = torch.randn(1, 30, 8, generator=gen(5))
    ohess.gptaq_add_batch(st, 0, x, x.reshape(-1, 8).clone())
    assert torch.all(st["dXXT"] == 0)


def test_weighted_hessian_saliency_one_is_half_gptq_hessian():
    """With saliency ≡ 1 and K equal batches of n tokens (one sample each),
    H_g2ptq = XᵀX/(K·n) and H_gptq = 2·XᵀX/K, so H_gptq = 2n·H_g2ptq in every group."""
    g = gen(6)
    C, G = 16, 4
    a = ohess.g2ptq_state(1, G, C)
    b = ohess.gptq_state(1, C)
    for _ in range(3):
        x = torch.randn(32, C, generator=g)
        ohess.g2ptq_add_batch(a, 0, x, torch.ones(32, G))
        ohess.gptq_add_batch(b, 0, x.unsqueeze(0))
    for gi in range(G):
        assert torch.allclose(a["H"][0, gi] * 64, b["H"][0], rtol=1e-5, atol=1e-5)


def test_weighted_hessian_fp64_brute_force():
    g = gen(7)
    C, G = 10, 3
    st = ohess.g2ptq_state(1, G, C)
    xs, ss = [], []
    for _ in range(2):
        x = torch.randn(25, C, generator=g)
        s = torch.rand(25, G, generator=g)
        ohess.g2ptq_add_batch(st, 0, x, s)
        xs.append(x.double())
        ss.append(s.double())
    ref = sum(torch.einsum("t,ti,tj->ij", s[:, gi], x, x) / (25 * 2) for x, s in zip(xs, ss)
              for gi in [0])
    assert torch.allclose(st["H"][0, 0].double(), ref, rtol=1e-5, atol=1e-6)
    act = sum((x ** 2).sum(0) for x in xs) / 50
    assert torch.allclose(st["act_square"][0].double(), act, rtol=1e-5)


# ---------------------------------------------------------------------------
# Factor
# ---------------------------------------------------------------------------

def _spd(C, seed, scale_spread=1.0):
    g = gen(seed)
    X = torch.randn(4 * C, C, generator=g) * torch.exp(scale_spread * torch.randn(C, generator=g))
    return (2 / X.shape[0]) * X.T @ X


def test_factor_is_upper_inverse_cholesky():
    """UᵀU = (H + λI)⁻¹ and U upper with positive diagonal (the unique such factor)."""
    H = _spd(48, 8, 0.3)
    U, damp = ofactor.damp_chol_inv_upper(H, 0.01)
    assert damp == 0.01
    assert torch.all(torch.tril(U, -1) == 0) and torch.all(torch.diagonal(U) > 0)
    A = H.double() + 0.01 * torch.mean(torch.diag(H)).double() * torch.eye(48, dtype=torch.float64)
    assert torch.allclose(U.double().T @ U.double(), torch.linalg.inv(A), rtol=1e-3, atol=1e-5)
    Ut, _ = ofactor.exact_inv_upper(H, 0.01)
    assert ((U.double() - Ut).norm() / Ut.norm()).item() < 1e-4


def test_factor_reverse_cholesky_identity():
    """The identity the HIP factor relies on: chol(A⁻¹, upper) = J·chol(J·A·J)⁻¹·J."""
    A = _spd(40, 9).double() + 0.05 * torch.eye(40, dtype=torch.float64)
    J = torch.eye(40, dtype=torch.float64).flip(0)
    U1 = torch.linalg.cholesky(torch.linalg.inv(A), upper=True)
    U2 = J @ torch.linalg.inv(torch.linalg.cholesky(J @ A @ J)) @ J
    assert ((U1 - U2).norm() / U1.norm()).item() < 1e-7


def test_factor_damp_retry_then_error():
    """Indefinite H: damp grows by 0.0015 until PD; hopeless H raises ValueError."""
    H = _spd(32, 10)
    lam = torch.linalg.eigvalsh(H.double())[0].item()
    m = torch.mean(torch.diag(H.double())).item()
    m2 = (m - lam) / 1.0153
    H2 = (H.double() - (lam + 0.0153 * m2) * torch.eye(32, dtype=torch.float64)).float()
    _, d = ofactor.damp_chol_inv_upper(H2, 0.01)
    assert abs(d - 0.016) < 1e-9
    bad = -torch.eye(8)
    with pytest.raises(ValueError):
        ofactor.damp_chol_inv_upper(bad, 0.01)


def test_prepare_hessian_zero_and_dead():
    H = torch.zeros(2, 4, 4)
    H[1] = torch.diag(torch.tensor([1.0, 0.0, 2.0, 0.0]))
    W = torch.ones(2, 3, 4)
    ofactor.prepare_hessian(H, W)
    assert torch.equal(H[0], torch.eye(4))          # all-zero → identity (RTN)
    assert torch.equal(torch.diag(H[1]), torch.tensor([1.0, 1.0, 2.0, 1.0]))
    assert torch.all(W[0] == 1)
    assert torch.all(W[1][:, [1, 3]] == 0) and torch.all(W[1][:, [0, 2]] == 1)


# ---------------------------------------------------------------------------
# Compensation
# ---------------------------------------------------------------------------

def _quantizers(W, bits, sym, groupsize, static):
    B, R, C = W.shape
    qs = oquant.make_group_quantizers(oquant.WeightQuantizer().configure(bits, sym=sym), C, groupsize)
    if groupsize == -1:
        qs[0].find_params(W.reshape(B * R, C))
    elif static:
        for i, q in enumerate(qs):
            q.find_params(W.reshape(B * R, C)[:, i * groupsize:(i + 1) * groupsize])
    return qs


@pytest.mark.parametrize("groupsize", [-1, 8])
def test_gptq_identity_w_minus_q_equals_err_u(groupsize):
    """GPTQ: W − Q = E·U (exact arithmetic; fp64 here) for every block."""
    g = gen(11)
    B, R, C = 1, 6, 24
    W = torch.randn(B, R, C, generator=g, dtype=torch.float64)
    U = torch.triu(torch.randn(B, C, C, generator=g, dtype=torch.float64) * 0.05, 1)
    U += torch.diag_embed(1 + torch.rand(B, C, generator=g, dtype=torch.float64))
    # collect errors with an fp64 run of the block loop
    W0 = W.clone()
    qs = _quantizers(W.float(), 4, True, groupsize, False)
    for q in qs:
        q.scale = q.scale.double() if torch.is_tensor(q.scale) else q.scale
    Wd = W.clone()
    E = torch.zeros_like(W)
    Q = torch.zeros_like(W)
    bs = 8
    for i1 in range(0, C, bs):
        i2 = min(i1 + bs, C)
        W1 = Wd[:, :, i1:i2].clone()
        for j in range(i2 - i1):
            col = i1 + j
            gi = 0 if groupsize == -1 else col // groupsize
            if groupsize != -1 and col % groupsize == 0:
                s, z = oquant.find_params(Wd[0, :, col:col + groupsize].float(), 4, True)
                qs[gi].scale, qs[gi].zero = s.double(), z.double()
            s, z = qs[gi].scale.reshape(R).double(), qs[gi].zero.reshape(R).double()
            x = W1[0, :, j]
            qv = s * (torch.clamp(torch.round(x / s) + z, -8, 7) - z)
            e = (x - qv) / U[0, col, col]
            Q[0, :, col], E[0, :, col] = qv, e
            W1[0, :, j:] -= e[:, None] * U[0, col, i1 + j:i2][None, :]
        Wd[:, :, i2:] -= E[:, :, i1:i2] @ U[:, i1:i2, i2:]
    assert torch.allclose(W0 - Q, E @ U, atol=1e-10)


def test_gptq_diagonal_u_is_rtn():
    """U diagonal ⇒ no compensation ⇒ GPTQ == round-to-nearest, bit for bit."""
    g = gen(12)
    B, R, C = 2, 9, 20
    W = torch.randn(B, R, C, generator=g) * 0.1
    U = torch.diag_embed(1 + torch.rand(B, C, generator=g))
    qs = _quantizers(W, 4, False, -1, False)
    Q, codes, _ = ocomp.gptq_compensation(W.clone(), U, qs, 8)
    q = oquant.WeightQuantizer().configure(4, sym=False)
    q.find_params(W.reshape(B * R, C))
    fq, c2, _ = q.fake_quantize(W.reshape(B * R, C))
    assert torch.equal(Q.reshape(B * R, C), fq)
    assert torch.equal(codes.reshape(B * R, C), c2)


def test_gptq_blocksize_invariance():
    """With every group start on a block start, results do not depend on the block size."""
    g = gen(13)
    B, R, C = 1, 16, 32
    W = torch.randn(B, R, C, generator=g, dtype=torch.float64).float()
    H = _spd(C, 14).unsqueeze(0)
    U, _ = ofactor.damp_chol_inv_upper(H[0], 0.01)
    outs = []
    for bs in (4, 8, 16, 32):
        qs = _quantizers(W, 4, True, 8, True)
        outs.append(ocomp.gptq_compensation(W.clone(), U.unsqueeze(0), qs, bs, 8, True)[1])
    for o in outs[1:]:
        mismatch = (o != outs[0]).float().mean().item()
        assert mismatch <= 0.01  # only rounding-tie cascades may differ


def test_gptaq_with_zero_p_equals_gptq():
    g = gen(15)
    W = torch.randn(2, 11, 20, generator=g)
    H = torch.stack([_spd(20, 16), _spd(20, 17)])
    U = torch.stack([ofactor.damp_chol_inv_upper(h, 0.01)[0] for h in H])
    qa = _quantizers(W, 4, False, -1, False)
    qb = copy.deepcopy(qa)
    a = ocomp.gptq_compensation(W.clone(), U, qa, 8)
    b = ocomp.gptaq_compensation(W.clone(), U, torch.zeros_like(U), qb, 8)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_g2ptq_with_zero_gradient_terms_equals_gptq():
    g = gen(18)
    W = torch.randn(1, 12, 24, generator=g)
    U = ofactor.damp_chol_inv_upper(_spd(24, 19), 0.01)[0].unsqueeze(0)
    qa = _quantizers(W, 3, True, 8, True)
    qb = copy.deepcopy(qa)
    a = ocomp.gptq_compensation(W.clone(), U, qa, 8, 8, True)
    Z = torch.zeros_like(W)
    b = ocomp.g2ptq_compensation(W.clone(), U, Z, Z.clone(), qb, 8, 8, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_obs_brute_force_tiny_c():
    """Tiny C in fp64: GPTQ's lazy-batch loop equals the optimal-brain-surgeon
    sequence with explicit inverse downdates (the GPTQ paper's equivalence)."""
    g = gen(20)
    R, C = 5, 7
    W = torch.randn(R, C, generator=g, dtype=torch.float64)
    H = _spd(C, 21).double() + 0.1 * torch.eye(C, dtype=torch.float64)
    s = torch.full((R, 1), 0.3, dtype=torch.float64)

    def qf(x):
        return s[:, 0] * torch.clamp(torch.round(x / s[:, 0]), -8, 7)
    # OBS: quantize column j, update remaining with the current inverse, downdate the inverse
    Wo = W.clone()
    Hinv = torch.linalg.inv(H)
    Qo = torch.zeros_like(W)
    for j in range(C):
        q = qf(Wo[:, j])
        Qo[:, j] = q
        err = (Wo[:, j] - q) / Hinv[j, j]
        Wo[:, j:] -= err[:, None] * Hinv[j, j:][None, :]
        Hinv = Hinv - Hinv[:, j:j + 1] @ Hinv[j:j + 1, :] / Hinv[j, j]
    # GPTQ with U = chol(H⁻¹, upper)
    U = torch.linalg.cholesky(torch.linalg.inv(H), upper=True)
    Wg = W.clone()
    Qg = torch.zeros_like(W)
    for j in range(C):
        q = qf(Wg[:, j])
        Qg[:, j] = q
        e = (Wg[:, j] - q) / U[j, j]
        Wg[:, j:] -= e[:, None] * U[j, j:][None, :]
    assert torch.allclose(Qo, Qg, atol=1e-9)


@pytest.mark.parametrize("cfg", [("ungrouped", -1, False, False), ("dynamic", 4, False, False),
                                 ("static_actorder", 4, True, True)])
@pytest.mark.parametrize("sym", [True, False])
def test_refactored_loops_match_original_loops(cfg, sym):
    """tests/test_triton_compensation.py:581-772 on CPU: oracle.compensate (refactored
    torch backend) vs oracle.original_loops (pre-refactor loops)."""
    name, groupsize, static, actorder = cfg
    B, R, C, bs, bits = 2, 37, 15, 5, 4
    g = gen(8000 + len(name) * 100 + int(sym))
    original = torch.randn(B, R, C, generator=g)
    perm = None
    weight = original.clone()
    if actorder:
        perm = torch.randperm(C, generator=g)
        weight = weight[:, :, perm]
    hinv = torch.triu(torch.randn(B, C, C, generator=g).mul_(0.002), diagonal=1)
    torch.diagonal(hinv, dim1=1, dim2=2).copy_(torch.rand(B, C, generator=g).mul_(0.5).add_(0.75))
    z = torch.randn(weight.shape, generator=g).mul_(0.002)
    gh = torch.randn(weight.shape, generator=g).mul_(0.002)
    p = torch.triu(torch.randn(B, C, C, generator=g).mul_(0.002), diagonal=1)
    qperm = perm if static and actorder else None

    def prep():
        tpl = oquant.WeightQuantizer().configure(bits, sym=sym)
        orig = copy.deepcopy(tpl)
        orig.find_params(original.reshape(B * R, C))
        groups = None
        if static:
            groups = []
            for s in range(0, C, groupsize):
                q = copy.deepcopy(orig)
                q.find_params(original[:, :, s:s + groupsize].reshape(B * R, -1))
                groups.append(q)
            cur = copy.deepcopy(groups)
        elif groupsize == -1:
            cur = [copy.deepcopy(orig)]
        else:
            cur = [copy.deepcopy(tpl) for _ in range((C + groupsize - 1) // groupsize)]
        return orig, groups, cur

    def same(a, e):
        assert torch.equal(a[1], e[1])
        for i in (0, 2, 3) + ((4,) if len(e) == 5 else ()):
            torch.testing.assert_close(a[i], e[i], rtol=2e-5, atol=2e-5)

    o, gr, cur = prep()
    exp = oloops.gptq_loop(weight.clone(), hinv.clone(), o, gr, bs, groupsize, qperm)
    w = weight.clone()
    same((*ocomp.gptq_compensation(w, hinv.clone(), cur, bs, groupsize, static, qperm), w), exp)
    o, gr, cur = prep()
    exp = oloops.g2ptq_loop(weight.clone(), hinv.clone(), z.clone(), gh.clone(), o, gr, bs,
                            groupsize, qperm)
    w, ghc = weight.clone(), gh.clone()
    same((*ocomp.g2ptq_compensation(w, hinv.clone(), z.clone(), ghc, cur, bs, groupsize, static,
                                    qperm), w, ghc), exp)
    o, gr, cur = prep()
    exp = oloops.gptaq_loop(weight.clone(), hinv.clone(), p.clone(), o, gr, bs, groupsize, qperm)
    w = weight.clone()
    same((*ocomp.gptaq_compensation(w, hinv.clone(), p.clone(), cur, bs, groupsize, static, qperm),
          w), exp)


def test_gptaq_p_definition_brute_force():
    g = gen(22)
    D = torch.randn(1, 6, 6, generator=g, dtype=torch.float64)
    U = torch.triu(torch.rand(1, 6, 6, generator=g, dtype=torch.float64)) + torch.eye(6, dtype=torch.float64)
    P = ocomp.gptaq_P(D, U, 0.25)
    T = D[0] @ U[0].T
    ref = torch.zeros(6, 6, dtype=torch.float64)
    for i in range(6):
        for j in range(6):
            ref[i, j] = 0.25 * sum(T[i, k] * U[0, k, j] for k in range(i + 1, 6))
    assert torch.allclose(P[0], ref)


# ---------------------------------------------------------------------------
# G2PTQ trust region
# ---------------------------------------------------------------------------

def test_trust_region_beta_bounds_and_identities():
    g = gen(23)
    BG, Rg, C = 2, 8, 16
    H = torch.stack([_spd(C, 24), _spd(C, 25)])
    U, Ainv = [], []
    for h in H:
        u, _, a = ofactor.damp_chol_inv_upper(h, 0.01, want_inverse=True)
        U.append(u)
        Ainv.append(a)
    U, Ainv = torch.stack(U), torch.stack(Ainv)
    W = torch.randn(BG, Rg, C, generator=g) * 0.02
    Q = W + 0.001 * torch.randn(BG, Rg, C, generator=g)
    grad = 1e-3 * torch.randn(BG, Rg, C, generator=g)
    beta, Z, GH = oflows.g2ptq_trust_region(grad, Ainv, U, Q, W, 0.1, True)
    assert torch.all(beta >= 0) and torch.all(beta <= 1)
    # GHinv = Z·U = β·Grad·UᵀU = β·Grad·A⁻¹
    assert torch.allclose(GH, beta.unsqueeze(2) * torch.bmm(grad, Ainv), rtol=1e-3, atol=1e-9)
    b0, Z0, G0 = oflows.g2ptq_trust_region(grad, Ainv, U, Q, W, 0.0, False)
    assert torch.all(b0 == 0) and torch.all(Z0 == 0) and torch.all(G0 == 0)


def _tr_slip_drop_ga2(grad, Ainv, U, Q, W, alpha):
    """Planted mistake: c without its −GA²/diag(A⁻¹) term."""
    GA = torch.bmm(grad, Ainv)
    e = Q - W
    d = torch.diagonal(Ainv, dim1=1, dim2=2).unsqueeze(1)
    loss = ((e * GA + e ** 2 / 2) / d).abs()
    c = (grad * GA).sum(2, keepdim=True).expand_as(GA)
    c = c.clamp(min=2 * alpha * loss).clamp(min=torch.finfo(torch.float32).tiny)
    return (1 - torch.sqrt(torch.clamp(1 - 2 * alpha * loss / c, min=0.0))).mean(-1)


def _tr_slip_sign(grad, Ainv, U, Q, W, alpha):
    """Planted mistake: E0 = W − Q instead of Q − W."""
    return oflows.g2ptq_trust_region(grad, Ainv, U, W, Q, alpha, True)[0]


def _tr_slip_diag_u(grad, Ainv, U, Q, W, alpha):
    """Planted mistake: diag(U) used where diag(A⁻¹) belongs."""
    Ad = Ainv.clone()
    idx = torch.arange(Ainv.shape[-1])
    Ad[:, idx, idx] = torch.diagonal(U, dim1=1, dim2=2)
    GA = torch.bmm(grad, Ainv)
    e = Q - W
    d = torch.diagonal(Ad, dim1=1, dim2=2).unsqueeze(1)
    loss = ((e * GA + e ** 2 / 2) / d).abs()
    c = (grad * GA).sum(2, keepdim=True) - GA ** 2 / d
    c = c.clamp(min=2 * alpha * loss).clamp(min=torch.finfo(torch.float32).tiny)
    return (1 - torch.sqrt(torch.clamp(1 - 2 * alpha * loss / c, min=0.0))).mean(-1)


def _beta_true(grad, Ainv, U, Q, W, alpha):
    return oflows.g2ptq_trust_region(grad, Ainv, U, Q, W, alpha, True)[0]


def _hand_case():
    """One row, two columns, A = [[2, 1], [1, 2]]: A⁻¹ = [[2, −1], [−1, 2]]/3,
    Grad = [1, 2], E0 = Q0 − W0 = [1/2, −1/4]."""
    Ainv = torch.tensor([[[2.0, -1.0], [-1.0, 2.0]]], dtype=torch.float64) / 3
    U = torch.linalg.cholesky(Ainv, upper=True)
    grad = torch.tensor([[[1.0, 2.0]]], dtype=torch.float64)
    W = torch.tensor([[[0.0, 0.0]]], dtype=torch.float64)
    Q = torch.tensor([[[0.5, -0.25]]], dtype=torch.float64)
    return grad, Ainv, U, Q, W


def _hand_beta(alpha):
    """Worked by hand.  GA = Grad·A⁻¹ = [0, 1]; diag(A⁻¹) = [2/3, 2/3];
    loss = |(E0·GA + E0²/2)/diag| = [(1/8)·(3/2), |−1/4 + 1/32|·(3/2)]
         = [3/16, 21/64];
    c = Σ Grad⊙GA − GA²/diag = [2 − 0, 2 − 3/2] = [2, 1/2].
    α = 0.1: 2α·loss = [3/80, 21/320] < c, so 1 − 2α·loss/c = [157/160, 139/160]
    and β = 1 − (√(157/160) + √(139/160))/2.
    α = 2: 2α·loss = [3/4, 21/16]; the second exceeds c = 1/2, c is clamped up
    to it and its term is 1 − √0 = 1; the first is 1 − √(1 − 3/8):
    β = (1 + 1 − √(5/8))/2."""
    if alpha == 0.1:
        return 1 - (math.sqrt(157 / 160) + math.sqrt(139 / 160)) / 2
    if alpha == 2.0:
        return (2 - math.sqrt(5 / 8)) / 2
    raise ValueError(alpha)


def _diag_case(seed):
    """Diagonal Hessians, so A⁻¹ = diag(d): every term of the trust region
    reduces to scalars.  Rows mix clamped and unclamped columns."""
    g = gen(seed)
    BG, Rg, C = 2, 4, 6
    h = torch.rand(BG, C, generator=g, dtype=torch.float64) * 3 + 0.25
    H = torch.diag_embed(h)
    damp = 0.01 * h.mean(-1, keepdim=True)
    d = 1 / (h + damp)
    Ainv = torch.diag_embed(d)
    U = torch.diag_embed(torch.sqrt(d))
    grad = torch.randn(BG, Rg, C, generator=g, dtype=torch.float64)
    grad[:, :, 0] *= 6  # one dominant gradient column: c_0 is small, its clamp engages
    W = torch.randn(BG, Rg, C, generator=g, dtype=torch.float64)
    Q = W + 0.8 * torch.randn(BG, Rg, C, generator=g, dtype=torch.float64)
    return H, d, grad, Ainv, U, Q, W


def _diag_beta(d, grad, Q, W, alpha):
    """The diagonal closed form, entry by entry in Python floats:
    loss_j = |e_j·g_j + e_j²/(2·d_j)|, c_j = Σ_k g_k²·d_k − g_j²·d_j clamped to
    at least 2α·loss_j and the smallest normal float, β = mean_j(1 − √max(1 −
    2α·loss_j/c_j, 0)).  Also returns how many terms the clamp decided."""
    BG, Rg, C = grad.shape
    beta = torch.zeros(BG, Rg, dtype=torch.float64)
    clamped = 0
    tiny = torch.finfo(torch.float32).tiny
    for b in range(BG):
        for r in range(Rg):
            g = grad[b, r].tolist()
            e = (Q[b, r] - W[b, r]).tolist()
            dd = d[b].tolist()
            total = sum(gk * gk * dk for gk, dk in zip(g, dd))
            acc = 0.0
            for j in range(C):
                loss = abs(e[j] * g[j] + e[j] * e[j] / (2 * dd[j]))
                c = total - g[j] * g[j] * dd[j]
                if c < 2 * alpha * loss:
                    clamped += 1
                c = max(c, 2 * alpha * loss, tiny)
                acc += 1 - math.sqrt(max(1 - 2 * alpha * loss / c, 0.0))
            beta[b, r] = acc / C
    return beta, clamped


def test_trust_region_hand_computed_case():
    """g2ptq_utils.py:459-476 on a 1×2 case worked by hand (_hand_beta), at an
    α where no clamp engages and at one where a column's c is clamped."""
    grad, Ainv, U, Q, W = _hand_case()
    for alpha in (0.1, 2.0):
        beta, Z, GH = oflows.g2ptq_trust_region(grad, Ainv, U, Q, W, alpha, True)
        assert abs(float(beta) - _hand_beta(alpha)) < 1e-14
        # GH = β·Grad·A⁻¹ = β·[0, 1]; Z = β·Grad·Uᵀ
        assert torch.allclose(GH[0, 0], float(beta) * torch.tensor([0.0, 1.0], dtype=torch.float64),
                              atol=1e-15)
        assert torch.allclose(Z[0], float(beta) * grad[0] @ U[0].T, atol=1e-15)


def test_trust_region_diagonal_closed_form():
    """Diagonal Hessians, through the oracle's own factor: U = diag(√d) and
    A⁻¹ = diag(d) with d = 1/(h + 0.01·mean h), and β, Z = β·g·√d,
    GH = β·g·d equal the scalar closed form (_diag_beta), with the clamp
    deciding some terms and not others."""
    for seed in (31, 32):
        H, d, grad, Ainv, U, Q, W = _diag_case(seed)
        Uo, Ao = [], []
        for h in H.float():
            u, _, a = ofactor.damp_chol_inv_upper(h, 0.01, want_inverse=True)
            Uo.append(u)
            Ao.append(a)
        Uo, Ao = torch.stack(Uo).double(), torch.stack(Ao).double()
        assert torch.allclose(Uo, U, rtol=1e-6, atol=1e-7)
        assert torch.allclose(Ao, Ainv, rtol=1e-6, atol=1e-7)
        alpha = 0.5
        beta, Z, GH = oflows.g2ptq_trust_region(grad, Ainv, U, Q, W, alpha, True)
        ref, clamped = _diag_beta(d, grad, Q, W, alpha)
        assert 0 < clamped < grad.numel(), clamped
        assert torch.allclose(beta, ref, rtol=1e-12, atol=1e-14)
        b = ref.unsqueeze(2)
        assert torch.allclose(Z, b * grad * torch.sqrt(d).unsqueeze(1), rtol=1e-12, atol=1e-14)
        assert torch.allclose(GH, b * grad * d.unsqueeze(1), rtol=1e-12, atol=1e-14)


def test_trust_region_planted_mistakes_fail_the_pins():
    """Each plausible slip — dropping −GA²/diag(A⁻¹) from c, flipping the sign
    of E0, using diag(U) for diag(A⁻¹) — fails the hand-computed case or the
    diagonal closed form, while the oracle passes both."""
    grad, Ainv, U, Q, W = _hand_case()
    H, d, dgrad, dAinv, dU, dQ, dW = _diag_case(31)
    dref, _ = _diag_beta(d, dgrad, dQ, dW, 0.5)

    def fails(fn):
        hand = any(abs(float(fn(grad, Ainv, U, Q, W, a)) - _hand_beta(a)) > 1e-9
                   for a in (0.1, 2.0))
        diag = not torch.allclose(fn(dgrad, dAinv, dU, dQ, dW, 0.5), dref, rtol=1e-9, atol=1e-12)
        return hand or diag

    assert not fails(_beta_true)
    for slip in (_tr_slip_drop_ga2, _tr_slip_sign, _tr_slip_diag_u):
        assert fails(slip), slip.__doc__


# ---------------------------------------------------------------------------
# compressed-tensors packing (oracle/pack.py)
# ---------------------------------------------------------------------------

def _unpack_bits(packed, num_bits, cols):
    """Independent unpacker: bit by bit through Python integers."""
    pf = 32 // num_bits
    out = []
    for row in packed.tolist():
        vals = []
        for word in row:
            u = word & 0xFFFFFFFF
            for i in range(pf):
                field = 0
                for bit in range(num_bits):
                    field |= ((u >> (num_bits * i + bit)) & 1) << bit
                vals.append(field - (1 << (num_bits - 1)))
        out.append(vals[:cols])
    return torch.tensor(out, dtype=torch.int8)


def test_pack_known_answers():
    # 4 bits: codes -8..7 become fields 0..15 (uint4b8), first column lowest
    codes = torch.arange(-8, 8, dtype=torch.int8).reshape(1, 16)
    p = opack.pack_to_int32(codes, 4)
    assert p.dtype == torch.int32 and p.shape == (1, 2)
    assert p[0, 0].item() == 0x76543210
    assert p[0, 1].item() == 0xFEDCBA98 - (1 << 32)
    # 8 bits (uint8b128): [-128, -1, 0, 127] -> fields [0, 127, 128, 255]
    p8 = opack.pack_to_int32(torch.tensor([[-128, -1, 0, 127]], dtype=torch.int8), 8)
    assert p8[0, 0].item() == 0xFF807F00 - (1 << 32)
    # 2 bits: [-2, -1, 0, 1] -> fields [0, 1, 2, 3]; the 12 missing columns are zero fields
    p2 = opack.pack_to_int32(torch.tensor([[-2, -1, 0, 1]], dtype=torch.int8), 2)
    assert p2.shape == (1, 1) and p2[0, 0].item() == (0 | 1 << 2 | 2 << 4 | 3 << 6)
    with pytest.raises(ValueError):
        opack.pack_to_int32(codes.int(), 4)
    with pytest.raises(ValueError):
        opack.pack_to_int32(codes, 9)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 8])
def test_pack_round_trip_and_layout(bits):
    g = gen(600 + bits)
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    codes = torch.randint(lo, hi + 1, (5, 37), generator=g).to(torch.int8)
    p = opack.pack_to_int32(codes, bits)
    pf = 32 // bits
    assert p.shape == (5, -(-37 // pf))
    assert torch.equal(_unpack_bits(p, bits, 37), codes)
    # fields past the last column are zero (not offset codes)
    tail = 37 % pf
    if tail:
        used = bits * tail
        assert all((w & 0xFFFFFFFF) >> used == 0 for w in p[:, -1].tolist())


def test_compress_group_scales_and_assert():
    g = gen(610)
    rows, cols, gs = 6, 256, 128
    codes = torch.randint(-8, 8, (rows, cols), generator=g).float()
    gscale = torch.rand(rows, cols // gs, generator=g) + 0.5
    Scale = gscale.repeat_interleave(gs, dim=1)
    out = opack.compress((rows, cols), torch.bfloat16, Scale, codes, 4, gs)
    assert torch.equal(out["weight_scale"], gscale.to(torch.bfloat16))
    assert out["weight_shape"].tolist() == [rows, cols]
    assert torch.equal(_unpack_bits(out["weight_packed"], 4, cols), codes.to(torch.int8))
    Scale[2, 5] += 1.0
    with pytest.raises(AssertionError):
        opack.compress((rows, cols), torch.bfloat16, Scale, codes, 4, gs)


def test_stack_experts_index_map():
    """mixins.py:93-144: gate_up[e, r] is gate_e[r] for r < I and up_e[r − I] after;
    down[e] is down_e; scales likewise; the shape tensors are (E, 2I, H) and
    (E, H, I).  Checked element by element on distinct values."""
    E, I, H, W, G = 3, 4, 6, 2, 3
    val = iter(range(10 ** 6))

    def t(r, c, dtype=torch.int32):
        return torch.tensor([[next(val) for _ in range(c)] for _ in range(r)], dtype=dtype)
    gate = [{"weight_packed": t(I, W), "weight_scale": t(I, G, torch.float32),
             "weight_shape": torch.tensor((I, H))} for _ in range(E)]
    up = [{"weight_packed": t(I, W), "weight_scale": t(I, G, torch.float32),
           "weight_shape": torch.tensor((I, H))} for _ in range(E)]
    down = [{"weight_packed": t(H, 1), "weight_scale": t(H, 1, torch.float32),
             "weight_shape": torch.tensor((H, I))} for _ in range(E)]
    out = opack.stack_experts(gate, up, down, weight_packed=True)
    for e in range(E):
        for r in range(2 * I):
            src = gate[e] if r < I else up[e]
            for c in range(W):
                assert out["gate_up_proj_packed"][e, r, c] == src["weight_packed"][r % I, c]
            for c in range(G):
                assert out["gate_up_proj_scale"][e, r, c] == src["weight_scale"][r % I, c]
        for r in range(H):
            assert out["down_proj_packed"][e, r, 0] == down[e]["weight_packed"][r, 0]
            assert out["down_proj_scale"][e, r, 0] == down[e]["weight_scale"][r, 0]
    assert out["gate_up_proj_shape"].tolist() == [E, 2 * I, H]
    assert out["down_proj_shape"].tolist() == [E, H, I]
    wg = [{"weight": t(I, H, torch.float32)} for _ in range(E)]
    wu = [{"weight": t(I, H, torch.float32)} for _ in range(E)]
    wd = [{"weight": t(H, I, torch.float32)} for _ in range(E)]
    out = opack.stack_experts(wg, wu, wd)
    assert out["gate_up_proj"].shape == (E, 2 * I, H) and out["down_proj"].shape == (E, H, I)
    assert out["gate_up_proj"][1, I + 2, 3] == wu[1]["weight"][2, 3]
    assert out["down_proj"][2, 5, 1] == wd[2]["weight"][5, 1]


# ---------------------------------------------------------------------------
# Calibration statistics (gptq_utils/g2ptq_utils.py:586-766)
# ---------------------------------------------------------------------------

def test_calib_saliency_closed_forms():
    """Constant gradients give exact group means (c² with power-of-two sizes);
    random gradients match the fp64 mean of squares per group; groups are
    consecutive column ranges (a gradient nonzero in one range only lights
    only that group)."""
    from oracle import calib as ocalib
    g = torch.full((2, 3, 64), 0.5)
    s = ocalib.group_mean_square(g, 4)
    assert s.shape == (6, 4) and torch.all(s == 0.25)
    x = torch.randn(5, 96, generator=gen(21))
    s = ocalib.group_mean_square(x, 3)
    ref = (x.double() ** 2).view(5, 3, 32).mean(-1)
    assert torch.allclose(s.double(), ref, rtol=2e-6, atol=0)
    y = torch.zeros(4, 96)
    y[:, 40:50] = 1.0
    s = ocalib.group_mean_square(y, 3)
    assert s[:, 1].tolist() == [10 / 32] * 4 and torch.all(s[:, [0, 2]] == 0)


def test_calib_running_mean_closed_forms():
    """After K calls, cache = Σ_i grad_i / (n_i·K): the mean over batches of the
    per-token gradient (fp64 within fp32 rounding); identical batches leave
    grad/n; the first call is exactly grad·fp32(1/n)."""
    from oracle import calib as ocalib
    gg = gen(22)
    grads = [torch.randn(7, 9, generator=gg) for _ in range(5)]
    ns = [128, 64, 300, 1, 77]
    c = None
    for i, (gr, n) in enumerate(zip(grads, ns)):
        c = ocalib.running_mean(c, gr, n, i)
    ref = sum(gr.double() / n for gr, n in zip(grads, ns)) / len(grads)
    assert torch.allclose(c.double(), ref, rtol=1e-5, atol=1e-7)
    c = None
    for i in range(4):
        c = ocalib.running_mean(c, grads[0], 256, i)
    assert torch.allclose(c, grads[0] / 256, rtol=1e-6, atol=0)
    first = ocalib.running_mean(None, grads[1], 3, 0)
    assert torch.equal(first, grads[1] * torch.tensor(1.0, dtype=torch.float32).div(3.0))
