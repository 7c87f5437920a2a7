"""Oracle: streaming Hessian accumulation (test infrastructure only).

torch-CPU fp32 restatements of the reference ``add_batch`` methods.  State is
passed explicitly (a small dict) instead of living on a class.
"""
import math

import torch


def gptq_state(num_layers, columns):
    return {"H": torch.zeros(num_layers, columns, columns), "nsamples": [0] * num_layers}


def gptq_add_batch(state, idx, inp):
    """gptq_utils/gptq_utils.py:115-126."""
    H = state["H"]
    if len(inp.shape) == 2:
        inp = inp.unsqueeze(0)
    tmp = inp.shape[0]
    if len(inp.shape) == 3:
        inp = inp.reshape((-1, inp.shape[-1]))
    inp = inp.t()
    n = state["nsamples"][idx]
    H[idx] *= n / (n + tmp)
    n += tmp
    state["nsamples"][idx] = n
    inp = math.sqrt(2 / n) * inp.float()
    H[idx] += inp.matmul(inp.t())


def gptaq_state(num_layers, columns):
    st = gptq_state(num_layers, columns)
    st["dXXT"] = torch.zeros(num_layers, columns, columns)
    return st


def gptaq_add_batch(state, idx, inp, fp_inp):
    """gptq_utils/gptaq_utils.py:130-148 (``fp_inp`` is the FIFO head)."""
    H, D = state["H"], state["dXXT"]
    fp = fp_inp.to(inp).t()
    if fp.dim() == 3:                          # (bsz, T, C).t() is not defined; flatten first
        raise ValueError("pass 2-D fp_inp")
    if len(inp.shape) == 2:
        inp = inp.unsqueeze(0)
    tmp = inp.shape[0]
    if len(inp.shape) == 3:
        inp = inp.reshape((-1, inp.shape[-1]))
    inp = inp.t()
    n = state["nsamples"][idx]
    H[idx] *= n / (n + tmp)
    D[idx] *= n / (n + tmp)
    n += tmp
    state["nsamples"][idx] = n
    inp = math.sqrt(2 / n) * inp.float()
    H[idx] += inp.matmul(inp.t())
    dX = fp.float() * math.sqrt(2 / n) - inp
    D[idx] += dX.matmul(inp.t())


def g2ptq_state(num_layers, num_groups, columns):
    return {
        "H": torch.zeros(num_layers, num_groups, columns, columns),
        "act_square": torch.zeros(num_layers, columns),
        "index": [0] * num_layers,
        "total_tokens": [0] * num_layers,
    }


def g2ptq_add_batch(state, idx, inp, sal):
    """gptq_utils/g2ptq_utils.py:182-201 (``sal`` is the per-batch (T, G) saliency)."""
    H, act = state["H"], state["act_square"]
    if inp.dim() == 3:
        inp = inp.reshape(-1, inp.shape[-1])
    inp = inp.float()
    n_tokens = inp.shape[0]
    sal = sal.float()
    k = state["index"][idx]
    H[idx] *= k / (k + 1)
    k += 1
    state["index"][idx] = k
    tt = state["total_tokens"][idx]
    act[idx] *= tt / (tt + n_tokens)
    tt += n_tokens
    state["total_tokens"][idx] = tt
    sal_weighted = torch.einsum("nj,ng->njg", inp, sal)
    block = torch.einsum("ni,njg->gij", inp, sal_weighted)
    H[idx].add_(block, alpha=1 / (n_tokens * k))
    act[idx].add_((inp ** 2).sum(0), alpha=1 / tt)


def guided_state(num_layers, num_groups, columns):
    return {
        "H": torch.zeros(num_layers, num_groups, columns, columns),
        "act_square": torch.zeros(num_layers, columns),
        "index": [0] * num_layers,
    }


def guided_add_batch(state, idx, inp, saliencies):
    """gptq_utils/gptq_guided_utils.py:59-81 (``saliencies`` is (N, seq, G))."""
    H, act = state["H"], state["act_square"]
    if inp.dim() == 2:
        inp = inp.unsqueeze(0)
    bsz = inp.shape[0]
    k = state["index"][idx]
    sal = saliencies[k:k + bsz]
    state["index"][idx] = k + bsz
    inp = inp.reshape(-1, inp.shape[-1])
    sal = sal.reshape(-1, sal.shape[-1])
    inp = inp.float()
    sal = sal.float()
    n_tokens = inp.shape[0]
    sal_weighted = torch.einsum("nj,ng->njg", inp, sal)
    block = torch.einsum("ni,njg->gij", inp, sal_weighted)
    H[idx].add_(block)
    act[idx].add_((inp ** 2).sum(0), alpha=1 / n_tokens)
