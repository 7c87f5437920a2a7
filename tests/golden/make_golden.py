"""Writes the golden fixtures of this directory from seeded inputs and the CPU oracle.

    python -m tests.golden.make_golden        (from the repository root)

The reference stores no golden vectors: its tests generate inputs on the fly
(tests/test_triton_compensation.py:70-143, 410-469) and compare backends on
the same box.  These fixtures freeze (a) the reference test's small
loop-comparison cases (B=2, R=37, C=15, bs=5 as at :582-583) with the expected
outputs of its pre-refactor loops, and (b) complete per-layer flows at C=256
(g128) for every quantizer class, so the HIP path is checked against stored
data and the oracle is checked against its own earlier outputs.

Only numbers are stored (``numpy.savez_compressed``; read with
``allow_pickle=False``).  bf16 tensors are stored as their int16 bit patterns.
"""
import copy
import os

import numpy as np
import torch

from oracle import flows as oflows
from oracle import hessian as ohess
from oracle import original_loops as oloops
from oracle import quant as oquant

HERE = os.path.dirname(os.path.abspath(__file__))
LOOPS_FILE = os.path.join(HERE, "loops_b2_r37_c15.npz")
FLOWS_FILE = os.path.join(HERE, "flows_c256_g128.npz")

LOOP_CONFIGS = (("ungrouped", -1, False, False), ("dynamic_groups", 4, False, False),
                ("static_groups_actorder", 4, True, True))
LOOP_SHAPE = dict(batch=2, rows=37, columns=15, blocksize=5, bits=4)

FLOW = dict(B=2, R=32, C=256, T=512, chunk=256, groupsize=128)


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def loop_inputs(ci, symmetric):
    """Inputs of the loop-comparison case ``ci`` (tests/test_triton_compensation.py:581-610)."""
    name, groupsize, static_groups, actorder = LOOP_CONFIGS[ci]
    b, r, c = LOOP_SHAPE["batch"], LOOP_SHAPE["rows"], LOOP_SHAPE["columns"]
    g = _gen(8000 + ci * 100 + int(symmetric))
    original = torch.randn(b, r, c, generator=g)
    perm = torch.randperm(c, generator=g) if actorder else torch.arange(c)
    weight = original[:, :, perm].clone() if actorder else original.clone()
    hinv = torch.triu(torch.randn(b, c, c, generator=g).mul_(0.002), diagonal=1)
    torch.diagonal(hinv, dim1=1, dim2=2).copy_(torch.rand(b, c, generator=g).mul_(0.5).add_(0.75))
    z = torch.randn(weight.shape, generator=g).mul_(0.002)
    ghinv = torch.randn(weight.shape, generator=g).mul_(0.002)
    p = torch.triu(torch.randn(b, c, c, generator=g).mul_(0.002), diagonal=1)
    return dict(original=original, perm=perm, weight=weight, hinv=hinv, z=z, ghinv=ghinv, p=p)


def _loop_quantizers(original, bits, symmetric, groupsize, static_groups):
    b, r, c = original.shape
    tpl = oquant.WeightQuantizer().configure(bits, sym=symmetric)
    orig = copy.deepcopy(tpl)
    orig.find_params(original.reshape(b * r, c))
    groups = None
    if static_groups:
        groups = []
        for s in range(0, c, groupsize):
            q = copy.deepcopy(orig)
            q.find_params(original[:, :, s:s + groupsize].reshape(b * r, -1))
            groups.append(q)
    return orig, groups


def make_loops():
    out = {}
    bs, bits = LOOP_SHAPE["blocksize"], LOOP_SHAPE["bits"]
    for ci, (name, groupsize, static_groups, actorder) in enumerate(LOOP_CONFIGS):
        for symmetric in (True, False):
            key = f"{name}_{'sym' if symmetric else 'asym'}"
            d = loop_inputs(ci, symmetric)
            for k in ("weight", "hinv", "z", "ghinv", "p"):
                out[f"{key}/in_{k}"] = d[k].numpy()
            out[f"{key}/in_original"] = d["original"].numpy()
            out[f"{key}/in_perm"] = d["perm"].numpy().astype(np.int64)
            qperm = d["perm"] if static_groups and actorder else None
            runs = {
                "gptq": lambda o, g_: oloops.gptq_loop(d["weight"].clone(), d["hinv"].clone(), o, g_,
                                                       bs, groupsize, qperm),
                "g2ptq": lambda o, g_: oloops.g2ptq_loop(d["weight"].clone(), d["hinv"].clone(),
                                                         d["z"].clone(), d["ghinv"].clone(), o, g_,
                                                         bs, groupsize, qperm),
                "gptaq": lambda o, g_: oloops.gptaq_loop(d["weight"].clone(), d["hinv"].clone(),
                                                         d["p"].clone(), o, g_, bs, groupsize,
                                                         qperm),
            }
            for variant, fn in runs.items():
                o, g_ = _loop_quantizers(d["original"], bits, symmetric, groupsize, static_groups)
                res = fn(o, g_)
                names = ("q", "codes", "scale", "weight") + (("ghinv",) if len(res) == 5 else ())
                for n, t in zip(names, res):
                    arr = t.numpy()
                    out[f"{key}/{variant}_{n}"] = arr.astype(np.int8) if n == "codes" else arr
    np.savez_compressed(LOOPS_FILE, **out)
    return out


def student_t3(shape, g):
    """Student-t samples with ν = 3 from the seeded generator: N(0,1)/sqrt(χ²₃/3),
    χ²₃ a sum of three squared normals."""
    z = torch.randn(shape, generator=g)
    chi2 = torch.randn((3,) + tuple(shape), generator=g).pow(2).sum(0)
    return z / torch.sqrt(chi2 / 3)


def flow_inputs():
    """Seeded inputs of the C=256 flow fixtures: LogNormal channel scales, bf16
    activations, bf16 weights ~N(0, 0.02), a perturbed full-precision input
    stream (GPTAQ), per-token saliencies and heavy-tailed row gradients (G2PTQ)."""
    B, R, C, T = FLOW["B"], FLOW["R"], FLOW["C"], FLOW["T"]
    g = _gen(4242)
    sigma = torch.exp(torch.randn(C, generator=g))
    X = (torch.randn(T, C, generator=g) * sigma).bfloat16()
    Xfp = (X.float() + 0.05 * sigma * torch.randn(T, C, generator=g)).bfloat16()
    W = (torch.randn(B, R, C, generator=g) * 0.02).bfloat16()
    G = 2
    sal = torch.rand(T, G, generator=g) * torch.exp(0.5 * torch.randn(T, 1, generator=g))
    tau = student_t3((B, R, 1), g).abs()
    grad = 1e-3 * torch.randn(B, R, C, generator=g) * tau
    return dict(X=X, Xfp=Xfp, W=W, sal=sal, grad=grad, G=G)


def flow_hessians(d):
    """Oracle Hessians accumulated chunk by chunk exactly as the classes see them."""
    B, C, T, ch, G = FLOW["B"], FLOW["C"], FLOW["T"], FLOW["chunk"], d["G"]
    st = ohess.gptq_state(B, C)
    sa = ohess.gptaq_state(B, C)
    s2 = ohess.g2ptq_state(B, G, C)
    sg = ohess.guided_state(B, G, C)
    sal_g = d["sal"].reshape(T // ch, ch, G)
    for i in range(0, T, ch):
        xb = d["X"][i:i + ch].reshape(1, ch, C)
        for b in range(B):
            ohess.gptq_add_batch(st, b, xb)
            ohess.gptaq_add_batch(sa, b, xb, d["Xfp"][i:i + ch])
            ohess.g2ptq_add_batch(s2, b, xb, d["sal"][i:i + ch])
            ohess.guided_add_batch(sg, b, xb, sal_g)
    return st, sa, s2, sg


def make_flows():
    d = flow_inputs()
    st, sa, s2, sg = flow_hessians(d)
    W0 = d["W"].float()
    gs = FLOW["groupsize"]
    out = {"in_X": d["X"].view(torch.int16).numpy(), "in_Xfp": d["Xfp"].view(torch.int16).numpy(),
           "in_W": d["W"].view(torch.int16).numpy(), "in_sal": d["sal"].numpy(),
           "in_grad": d["grad"].numpy()}
    res = {
        "gptq_asym": oflows.gptq_fasterquant(W0, st["H"], 4, False, groupsize=gs),
        "gptq_sym_actorder": oflows.gptq_fasterquant(W0, st["H"], 4, True, groupsize=gs,
                                                     actorder=True, static_groups=True),
        "gptaq_sym": oflows.gptaq_fasterquant(W0, sa["H"], sa["dXXT"], 4, True, groupsize=gs),
        "g2ptq_w3": oflows.g2ptq_fasterquant(W0, s2["H"].clone(), d["grad"], s2["act_square"], 3,
                                             True, d["G"], groupsize=gs, alpha=0.1),
        "guided_sym": oflows.guided_fasterquant(W0, sg["H"], sg["act_square"], 4, True, d["G"],
                                                groupsize=gs),
    }
    hs = {"gptq": st["H"], "gptaq": sa["H"], "gptaq_dXXT": sa["dXXT"], "g2ptq": s2["H"],
          "guided": sg["H"]}
    for k, H in hs.items():
        out[f"H_{k}_diag"] = torch.diagonal(H, dim1=-2, dim2=-1).numpy()
        out[f"H_{k}_rowsum"] = H.sum(-1).numpy()
    for k, r in res.items():
        out[f"{k}/codes"] = r["W_int"].numpy().astype(np.int8)
        out[f"{k}/q"] = r["Q"].numpy()
        if "beta" in r:
            out[f"{k}/beta"] = r["beta"].numpy()
        # what the end-to-end parity protocol (oracle.parity) needs: the values
        # at quantization time in loop order, the loop order, the fitted groups
        out[f"{k}/x"] = r["loop"]["X"].numpy()
        perm = r["perm"]
        out[f"{k}/perm"] = (perm if perm is not None else torch.arange(W0.shape[2])).numpy()
        qs = r["quantizers"]
        out[f"{k}/qscale"] = torch.stack([q.scale.reshape(-1) for q in qs]).numpy()
        out[f"{k}/qzero"] = torch.stack([q.zero.reshape(-1) for q in qs]).numpy()
        if qs[0].zraw is not None:
            out[f"{k}/qzraw"] = torch.stack([q.zraw.reshape(-1) for q in qs]).numpy()
    np.savez_compressed(FLOWS_FILE, **out)
    return out


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


if __name__ == "__main__":
    torch.set_num_threads(1)
    a = make_loops()
    b = make_flows()
    for p in (LOOPS_FILE, FLOWS_FILE):
        print(p, os.path.getsize(p), "bytes")
