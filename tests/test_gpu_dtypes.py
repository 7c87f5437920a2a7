"""GPU: calibration activations in fp16 and fp32, which the reference accepts
like bf16 (``inp.float()``, gptq_utils/gptq_utils.py:125, gptaq_utils.py:
139-146, g2ptq_utils.py:193-201, gptq_guided_utils.py:59-81).

The HIP path stages such an activation as bf16 planes that sum to it exactly
(fp16: 2, fp32: 3) and runs every Gram product once per plane.  Each case
accumulates the Hessians from the same tokens as the oracle (fp32 on the
host), holds them to fp64 sums of the same tokens (1e-5 relative to
sqrt(H_ii·H_jj)), and holds the whole flow to oracle.parity.check_flow.
A calibration that changes dtype midway folds the staged tokens and goes
on, and the bf16 path of the any-dtype entry points equals the bf16 entry
points bit for bit.
"""
import pytest
import torch

from oracle import flows as oflows
from oracle import hessian as ohess
from oracle.parity import check_flow
from tests._util import gen

pytestmark = pytest.mark.gpu

B, R, C, T, CHUNK, G = 2, 128, 512, 4096, 1024, 4


def _inputs(seed, dtype):
    g = gen(seed)
    sig = torch.exp(torch.randn(C, generator=g))
    X = (torch.randn(T, C, generator=g) * sig).to(dtype)
    Xfp = (X.float() + 0.05 * sig * torch.randn(T, C, generator=g)).to(dtype)
    W = (torch.randn(B, R, C, generator=g) * 0.02).bfloat16()
    sal = torch.rand(T, G, generator=g) + 0.1
    grads = 1e-3 * torch.randn(B, R, C, generator=g)
    return X, Xfp, W, sal, grads


def _layers(W, dev):
    out = []
    for b in range(B):
        lin = torch.nn.Linear(C, R, bias=False).to(torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(W[b])
        out.append(lin.to(dev))
    return out


def _close_to_exact(label, Hd, He):
    d = torch.diagonal(He, dim1=-2, dim2=-1)
    scale = torch.sqrt(d.unsqueeze(-1) * d.unsqueeze(-2))
    err = ((Hd.double() - He).abs() / scale).max().item()
    print(f"{label}: max |H − fp64| / sqrt(H_ii·H_jj) = {err:.3g}", flush=True)
    assert err <= 1e-5, (label, err)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("method", ["gptq", "gptaq", "g2ptq", "guided"])
def test_non_bf16_activations_match_oracle(dev, method, dtype):
    from g2ptq_amd import G2PTQ, GPTAQ, GPTQ, GPTQGuided, WeightQuantizer, make_group_quantizers
    print(f"{method} with {dtype} activations", flush=True)
    X, Xfp, W, sal, grads = _inputs(900 + 7 * ["gptq", "gptaq", "g2ptq", "guided"].index(method),
                                    dtype)
    layers = _layers(W, dev)
    W0 = W.float()
    batches = list(range(0, T, CHUNK))
    if method == "gptq":
        gq, st = GPTQ(layers), ohess.gptq_state(B, C)
    elif method == "gptaq":
        gq, st = GPTAQ(layers), ohess.gptaq_state(B, C)
        for b in range(B):
            gq.fp_inp[b] = [Xfp[i:i + CHUNK].to(dev) for i in batches]
    elif method == "g2ptq":
        gq = G2PTQ(layers, [[sal[i:i + CHUNK] for i in batches] for _ in range(B)],
                   [grads[b].to(dev) for b in range(B)], G)
        st = ohess.g2ptq_state(B, G, C)
    else:
        sal_g = sal.reshape(T // CHUNK, CHUNK, G)
        gq, st = GPTQGuided(layers, [sal_g for _ in range(B)], G), ohess.guided_state(B, G, C)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, 128)
    for i in batches:
        xb = X[i:i + CHUNK].reshape(1, CHUNK, C)
        for b in range(B):
            gq.add_batch(b, xb.to(dev), None)
            if method == "gptq":
                ohess.gptq_add_batch(st, b, xb)
            elif method == "gptaq":
                ohess.gptaq_add_batch(st, b, xb, Xfp[i:i + CHUNK])
            elif method == "g2ptq":
                ohess.g2ptq_add_batch(st, b, xb, sal[i:i + CHUNK])
            else:
                ohess.guided_add_batch(st, b, xb, sal_g)
    # the same sums in fp64
    x = X.double()
    if method in ("gptq", "gptaq"):
        He = (2.0 / len(batches)) * x.T @ x           # one sequence per batch
        _close_to_exact(f"{method} {dtype} H", gq.H[0].cpu(), He)
        if method == "gptaq":
            De = (2.0 / len(batches)) * (Xfp.double() - x).T @ x
            d = torch.diagonal(He)
            err = ((gq.dXXT[0].cpu().double() - De).abs() / torch.sqrt(d[:, None] * d[None, :]))
            print(f"gptaq {dtype} dXXT: {err.max().item():.3g}", flush=True)
            assert err.max().item() <= 1e-5
    else:
        w = 1.0 / CHUNK / len(batches) if method == "g2ptq" else 1.0
        He = torch.stack([w * (x * sal[:, g:g + 1].double()).T @ x for g in range(G)])
        _close_to_exact(f"{method} {dtype} H", gq.H[0].cpu(), He)
        act = (x * x).sum(0) / (T if method == "g2ptq" else CHUNK)
        rel = ((gq.act_square[0].cpu().double() - act).abs() / act).max().item()
        print(f"{method} {dtype} act_square: {rel:.3g}", flush=True)
        assert rel <= 1e-5
    H = st["H"].clone()
    kw = dict(blocksize=128, percdamp=0.01, groupsize=128)
    if method == "gptq":
        gq.fasterquant(backend="hip", export_compressed_tensors=True, **kw)
        ref = oflows.gptq_fasterquant(W0, H, 4, True, **kw)
        He_b = H
    elif method == "gptaq":
        gq.fasterquant(backend="hip", export_compressed_tensors=True, alpha=0.25, **kw)
        ref = oflows.gptaq_fasterquant(W0, H, st["dXXT"].clone(), 4, True, alpha=0.25, **kw)
        He_b = H
    elif method == "g2ptq":
        gq.fasterquant(backend="hip", export_compressed_tensors=True, alpha=0.1, **kw)
        ref = oflows.g2ptq_fasterquant(W0, H.clone(), grads, st["act_square"], 4, True, G,
                                       alpha=0.1, **kw)
        He_b = H.reshape(B * G, C, C)
    else:
        gq.fasterquant(backend="hip", export_compressed_tensors=True, **kw)
        ref = oflows.guided_fasterquant(W0, H.clone(), st["act_square"], 4, True, G, **kw)
        He_b = H.reshape(B * G, C, C)
    torch.cuda.synchronize()
    check_flow(f"{method} {dtype}", layers, gq.quantizer, ref, W0, He_b, 4, 128, False)


def test_dtype_change_midway_folds_and_continues(dev):
    """Two bf16 batches, then fp16, then fp32: each change folds the staged
    tokens into H, and the result is the oracle's over the same sequence."""
    from g2ptq_amd import GPTQ
    g = gen(990)
    sig = torch.exp(torch.randn(C, generator=g))
    xs = [(torch.randn(CHUNK, C, generator=g) * sig).to(dt)
          for dt in (torch.bfloat16, torch.bfloat16, torch.float16, torch.float32)]
    lin = torch.nn.Linear(C, 16, bias=False, device=dev, dtype=torch.bfloat16)
    gq, st = GPTQ([lin]), ohess.gptq_state(1, C)
    for x in xs:
        gq.add_batch(0, x.unsqueeze(0).to(dev), None)
        ohess.gptq_add_batch(st, 0, x.unsqueeze(0))
    assert gq._stagers[0].dtype == 2
    Hd, Hr = gq.H[0].cpu().double(), st["H"][0].double()
    d = torch.diagonal(Hr)
    err = ((Hd - Hr).abs() / torch.sqrt(d[:, None] * d[None, :])).max().item()
    print(f"dtype change: max |H − oracle| / sqrt(H_ii·H_jj) = {err:.3g}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_any_dtype_entry_points_equal_bf16_ones(dev, kind):
    """g2ptq_hessian_stage_ex / _gram_ex with dtype 0 give the bf16 entry
    points' staged planes and outputs bit for bit (one C-ABI call each)."""
    from g2ptq_amd import _lib
    g = gen(980 + kind)
    Tk, Ck, Gk = 1536, 384, 3
    X = (torch.randn(Tk, Ck, generator=g) * 2).bfloat16().to(dev)
    F = (X.float() + 0.1 * torch.randn(Tk, Ck, generator=g).to(dev)).bfloat16()
    S = (torch.rand(Tk, Gk, generator=g) + 0.1).to(dev)
    st = _lib.stream_ptr()
    rows = _lib.query_size_i64("g2ptq_hessian_stage_rows", Ck)
    Gq = Gk if kind == 2 else 0
    planes = _lib.query_size_i64("g2ptq_hessian_stage_planes", kind, 0, Gq)
    assert planes == {0: 1, 1: 3, 2: 1}[kind]
    height = _lib.query_size_i64("g2ptq_hessian_stage_height", kind, 0, Ck, Gq)
    assert height == planes * rows + (2 * Gk if kind == 2 else 0)
    ldt = 8192
    outs = []
    for ex in (False, True):
        XT = torch.zeros(height, ldt, dtype=torch.bfloat16, device=dev)
        H = torch.full((max(Gq, 1), Ck, Ck), 0.5, device=dev)
        Dx = torch.full((Ck, Ck), 0.25, device=dev)
        act = torch.full((Ck,), 2.0, device=dev)
        p = _lib.ptr
        if ex:
            _lib.call("g2ptq_hessian_stage_ex", st, kind, 0, p(X), p(F), Tk, Ck, Ck, Ck, p(S), Gq,
                      Gk, 0.5, p(XT), ldt, 0, p(act), 0.25, 0.75)
            nb = _lib.query_size("g2ptq_hessian_gram_ex_workspace", kind, 0, Tk, Ck, Gq)
            ws = torch.empty(max(nb, 256), dtype=torch.uint8, device=dev)
            _lib.call("g2ptq_hessian_gram_ex", st, kind, 0, p(XT), ldt, Tk, Ck, Gq, 0.125, 0.5,
                      p(H), Ck, Ck * Ck, p(Dx), Ck, p(ws), ws.numel())
        else:
            if kind == 0:
                _lib.call("g2ptq_hessian_stage", st, p(X), Tk, Ck, Ck, p(XT), ldt, 0)
                name = "g2ptq_hessian_gram_workspace"
            elif kind == 1:
                _lib.call("g2ptq_gptaq_stage", st, p(X), p(F), Tk, Ck, Ck, Ck, p(XT), ldt, 0)
                name = "g2ptq_gptaq_gram_workspace"
            else:
                _lib.call("g2ptq_weighted_stage", st, p(X), Tk, Ck, Ck, p(S), Gk, Gk, 0.5, p(XT),
                          ldt, 0, p(act), 0.25, 0.75)
                name = "g2ptq_weighted_gram_workspace"
            qargs = (Tk, Ck, Gk) if kind == 2 else (Tk, Ck)
            ws = torch.empty(max(_lib.query_size(name, *qargs), 256), dtype=torch.uint8,
                             device=dev)
            if kind == 0:
                _lib.call("g2ptq_hessian_gram", st, p(XT), ldt, Tk, Ck, 0.125, 0.5, p(H), Ck,
                          p(ws), ws.numel())
            elif kind == 1:
                _lib.call("g2ptq_gptaq_gram", st, p(XT), ldt, Tk, Ck, 0.125, 0.5, p(H), p(Dx), Ck,
                          p(ws), ws.numel())
            else:
                _lib.call("g2ptq_weighted_gram", st, p(XT), ldt, Tk, Ck, Gk, 0.125, 0.5, p(H), Ck,
                          Ck * Ck, p(ws), ws.numel())
        torch.cuda.synchronize()
        outs.append([t.cpu() for t in (XT, H, Dx, act)])
    for a, b, what in zip(outs[0], outs[1], ("staged planes", "H", "Dx", "act")):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)), what
