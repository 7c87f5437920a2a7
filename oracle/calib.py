"""Oracle: calibration statistics (test infrastructure only).

Restates the per-batch reductions of ``SaliencyCache.grad_hook`` and
``GradientCache.cache_gradient`` (gptq_utils/g2ptq_utils.py:604-618,
704-714) in torch-CPU fp32, with the fp32 arithmetic torch performs for
these expressions on the GPU: a mean is the sum times fp32(1/count), and a
division by a Python number is a multiplication by its fp32 reciprocal.

Parity: pinned by closed forms (constant gradients give exact means;
the running mean after K batches equals the fp64 mean of grad_i / n_i) in
tests/test_oracle_pins.py.
"""
import numpy as np
import torch


def group_mean_square(grad, num_groups):
    """g2ptq_utils.py:609-616: (n_tokens, G) mean of grad² over channel groups."""
    grad = grad.reshape(-1, grad.shape[-1])
    n_tokens, hidden = grad.shape
    group_size = hidden // num_groups
    sq = grad.float().pow(2).view(n_tokens, num_groups, group_size)
    return sq.sum(dim=-1) * torch.tensor(1.0 / group_size, dtype=torch.float32)


def running_mean(cache, grad, n_tokens, index):
    """g2ptq_utils.py:706-713 for call number ``index`` (0-based); ``cache`` is
    None on the first call (the reference's int 0)."""
    keep = torch.tensor(np.float32(index / (index + 1)))
    inv = torch.tensor(np.float32(1.0) / np.float32(n_tokens * (index + 1)))
    d = grad.float() * inv
    if cache is None:
        return 0.0 + d
    return cache * keep + d
