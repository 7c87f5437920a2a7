"""Token staging for the GPTQ Hessian (one Gram launch per flush, not per batch).

``GPTQ.add_batch`` (gptq_utils/gptq_utils.py:115-126) updates
``H ← H·n/(n+t) + (2/(n+t))·XᵀX`` once per calibration batch.  After any
number of batches since the state (H₀, n₀) this is, exactly in real
arithmetic, ``H = (n₀/n)·H₀ + (2/n)·Σ XᵀX``: every batch carries the same
final weight 2/n.  The stager therefore only transposes each batch into a
feature-major bf16 buffer and runs the Gram product over everything staged
when the buffer fills or when ``H`` is read, which amortises the Gram
kernel's per-launch work (reading β·H, writing both triangles) over many
batches and gives the kernel long K runs.

The buffer grows ×4 at flush points (it is empty then, so nothing is copied),
up to ``budget_bytes`` (default 8 GiB, env ``G2PTQ_STAGE_BYTES``): MI355X's
288 GB of HBM holds a whole decoder block's calibration set staged.
"""
import os

import torch

from . import _lib

DEFAULT_BUDGET = int(os.environ.get("G2PTQ_STAGE_BYTES", str(8 << 30)))

# Optional launch timing: when a list, every Gram launch appends
# (start event, end event, 2·K·C² flops), events recorded on the launch stream.
TIMING = None
_GRAM_PAD = 2048      # the Gram call may zero-pad K up to a multiple of this
_FIRST_TOKENS = 65536


def _ceil(x, m):
    return (x + m - 1) // m * m


class GramStager:
    def __init__(self, columns, device, budget_bytes=None):
        self.C = columns
        self.device = device
        self.rows = _lib.query_size_i64("g2ptq_hessian_stage_rows", columns)
        budget = DEFAULT_BUDGET if budget_bytes is None else budget_bytes
        self.max_tokens = max(_GRAM_PAD * 2, budget // (self.rows * 2) // _GRAM_PAD * _GRAM_PAD)
        self.buf = None
        self.cap = 0        # token columns of buf
        self.k = 0          # staged token columns (multiples of 64)

    def fits(self, T):
        return self.buf is not None and self.k + _ceil(T, 64) + _GRAM_PAD <= self.cap

    def can_stage(self, T):
        """Whether a batch of T tokens can ever be staged (else update directly)."""
        return _ceil(T, 64) + _GRAM_PAD <= self.max_tokens

    def reserve(self, T):
        """With the buffer empty (just flushed because T more tokens did not fit,
        or never allocated): allocate the first buffer, or one 4× larger, up to
        the budget."""
        assert self.k == 0
        need = _ceil(T, 64) + _GRAM_PAD
        cap = max(_FIRST_TOKENS, need) if self.buf is None else max(need, self.cap * 4)
        cap = _ceil(max(need, min(cap, self.max_tokens)), _GRAM_PAD)
        if self.buf is not None and cap <= self.cap:
            return
        self.buf = None
        self.buf = torch.empty(self.rows, cap, dtype=torch.bfloat16, device=self.device)
        self.cap = cap

    def stage(self, X):
        T, C = X.shape
        _lib.call("g2ptq_hessian_stage", _lib.stream_ptr(), _lib.ptr(X), T, C, C,
                  _lib.ptr(self.buf), self.cap, self.k)
        self.k += _ceil(T, 64)

    def flush(self, H, alpha, beta):
        """H = beta·H + alpha·Σ staged XᵀX; empties the buffer."""
        if self.k == 0:
            return
        if not H.is_cuda:
            raise RuntimeError("staged Hessian tokens need the Hessian on the GPU: call "
                               "add_batch inside _maybe_onload_hessian()")
        nbytes = _lib.query_size("g2ptq_hessian_gram_workspace", self.k, self.C)
        ws = _lib.workspace(nbytes, self.buf.device)
        if TIMING is not None:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
        _lib.call("g2ptq_hessian_gram", _lib.stream_ptr(), _lib.ptr(self.buf), self.cap, self.k,
                  self.C, float(alpha), float(beta), _lib.ptr(H), self.C, _lib.ptr(ws), ws.numel())
        if TIMING is not None:
            e1.record()
            TIMING.append((e0, e1, 2.0 * self.k * self.C * self.C, self.k, self.C))
        self.k = 0

    def release(self):
        self.buf = None
        self.cap = 0
        self.k = 0
