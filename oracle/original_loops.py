"""Oracle #2: the reference test's "pre-refactor" full loops (test infrastructure only).

Restates tests/test_triton_compensation.py:176-374 of the reference.  These
loops use a different formulation from the refactored ``_run_compensation``
(whole-row ``bmm`` updates including the current column, ``fake_quantize`` on
the quantizer instead of the unified asym primitive), so agreement between the
two oracles pins the block/loop restatement in ``compensate``.
"""
import torch


def _select(quantizer, groups, weight, i1, i, groupsize, perm, batch, rows):
    if groupsize != -1:
        if groups is None:
            if (i1 + i) % groupsize == 0:
                quantizer.find_params(weight[:, :, i1 + i:i1 + i + groupsize].reshape(batch * rows, -1))
        else:
            index = i1 + i
            if perm is not None:
                index = int(perm[index])
            quantizer = groups[index // groupsize]
    return quantizer


def gptq_loop(weight, hinv, quantizer, groups, blocksize, groupsize, perm):
    """tests/test_triton_compensation.py:176-232."""
    batch, rows, columns = weight.shape
    scale = torch.zeros_like(weight)
    int_weight = torch.zeros_like(weight)
    qweight = torch.zeros_like(weight)
    for i1 in range(0, columns, blocksize):
        i2 = min(i1 + blocksize, columns)
        w1 = weight[:, :, i1:i2].clone()
        q1, n1, s1, e1 = (torch.zeros_like(w1) for _ in range(4))
        h1 = hinv[:, i1:i2, i1:i2]
        for i in range(i2 - i1):
            w = w1[:, :, i]
            d = h1[:, i, i]
            quantizer = _select(quantizer, groups, weight, i1, i, groupsize, perm, batch, rows)
            q, qi, qs = quantizer.fake_quantize(w.view(batch * rows, 1))
            q = q.view(batch, rows)
            q1[:, :, i] = q
            n1[:, :, i] = qi.view(batch, rows)
            s1[:, :, i] = qs.view(batch, rows)
            err = (w - q) / d.unsqueeze(1)
            w1[:, :, i:] -= torch.bmm(err.unsqueeze(2), h1[:, i, i:].unsqueeze(1))
            e1[:, :, i] = err
        qweight[:, :, i1:i2] = q1
        int_weight[:, :, i1:i2] = n1
        scale[:, :, i1:i2] = s1
        weight[:, :, i2:] -= torch.bmm(e1, hinv[:, i1:i2, i2:])
    return qweight, int_weight, scale, weight


def g2ptq_loop(weight, hinv, z, ghinv, quantizer, groups, blocksize, groupsize, perm):
    """tests/test_triton_compensation.py:235-310.  The tail after the last block
    is skipped, as the production loop does (gptq_utils/g2ptq_utils.py:324-325):
    it updates no column, and with a ragged last block the distance vector
    (blocksize entries) would not match the block's width."""
    batch, rows, columns = weight.shape
    scale = torch.zeros_like(weight)
    int_weight = torch.zeros_like(weight)
    qweight = torch.zeros_like(weight)
    distance = torch.arange(blocksize - 1, -1, -1).to(ghinv)
    for i1 in range(0, columns, blocksize):
        i2 = min(i1 + blocksize, columns)
        w1 = weight[:, :, i1:i2].clone()
        q1, n1, s1, e1 = (torch.zeros_like(w1) for _ in range(4))
        h1 = hinv[:, i1:i2, i1:i2]
        g1 = ghinv[:, :, i1:i2].clone()
        zz = z[:, :, i1:i2]
        for i in range(i2 - i1):
            w = w1[:, :, i]
            d = h1[:, i, i]
            quantizer = _select(quantizer, groups, weight, i1, i, groupsize, perm, batch, rows)
            q, qi, qs = quantizer.fake_quantize(w.view(batch * rows, 1))
            q = q.view(batch, rows)
            q1[:, :, i] = q
            n1[:, :, i] = qi.view(batch, rows)
            s1[:, :, i] = qs.view(batch, rows)
            err = (w - q - g1[:, :, i]) / d.unsqueeze(1)
            w1[:, :, i:] -= torch.bmm(err.unsqueeze(2), h1[:, i, i:].unsqueeze(1)) + g1[:, :, i:]
            e1[:, :, i] = err
            g1[:, :, i:] -= torch.bmm(zz[:, :, i].unsqueeze(2), h1[:, i, i:].unsqueeze(1))
        qweight[:, :, i1:i2] = q1
        int_weight[:, :, i1:i2] = n1
        scale[:, :, i1:i2] = s1
        if i2 == columns:
            continue
        upd = blocksize * ghinv[:, :, i2:] - torch.bmm(zz * distance.reshape(1, 1, -1),
                                                        hinv[:, i1:i2, i2:])
        weight[:, :, i2:] -= torch.bmm(e1, hinv[:, i1:i2, i2:]) + upd
        ghinv[:, :, i2:] -= torch.bmm(z[:, :, i1:i2], hinv[:, i1:i2, i2:])
    return qweight, int_weight, scale, weight, ghinv


def gptaq_loop(weight, hinv, p, quantizer, groups, blocksize, groupsize, perm):
    """tests/test_triton_compensation.py:313-374."""
    batch, rows, columns = weight.shape
    scale = torch.zeros_like(weight)
    int_weight = torch.zeros_like(weight)
    qweight = torch.zeros_like(weight)
    for i1 in range(0, columns, blocksize):
        i2 = min(i1 + blocksize, columns)
        w1 = weight[:, :, i1:i2].clone()
        q1, n1, s1, e1 = (torch.zeros_like(w1) for _ in range(4))
        h1 = hinv[:, i1:i2, i1:i2]
        p1 = p[:, i1:i2, i1:i2]
        for i in range(i2 - i1):
            w = w1[:, :, i]
            d = h1[:, i, i]
            quantizer = _select(quantizer, groups, weight, i1, i, groupsize, perm, batch, rows)
            q, qi, qs = quantizer.fake_quantize(w.view(batch * rows, 1))
            q = q.view(batch, rows)
            q1[:, :, i] = q
            n1[:, :, i] = qi.view(batch, rows)
            s1[:, :, i] = qs.view(batch, rows)
            err = (w - q) / d.unsqueeze(1)
            w1[:, :, i:] -= (torch.bmm(err.unsqueeze(2), h1[:, i, i:].unsqueeze(1))
                             - torch.bmm(w.unsqueeze(2), p1[:, i, i:].unsqueeze(1)))
            e1[:, :, i] = err
        qweight[:, :, i1:i2] = q1
        int_weight[:, :, i1:i2] = n1
        scale[:, :, i1:i2] = s1
        weight[:, :, i2:] -= torch.bmm(e1, hinv[:, i1:i2, i2:]) - torch.bmm(w1, p[:, i1:i2, i2:])
    return qweight, int_weight, scale, weight
