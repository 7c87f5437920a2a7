"""Token staging for the Hessians (one Gram launch per flush, not per batch).

``GPTQ.add_batch`` (gptq_utils/gptq_utils.py:115-126) updates
``H ← H·n/(n+t) + (2/(n+t))·XᵀX`` once per calibration batch.  After any
number of batches since the state (H₀, n₀) this is, exactly in real
arithmetic, ``H = (n₀/n)·H₀ + (2/n)·Σ XᵀX``: every batch carries the same
final weight 2/n.  The same holds for GPTAQ's cross term
(gptaq_utils.py:130-148), for GPTQGuided's plain sums
(gptq_guided_utils.py:59-81) and, once each batch's 1/T_b is folded into its
staged tokens, for G2PTQ's per-batch means (g2ptq_utils.py:182-201).  The
stager therefore only transposes each batch into feature-major bf16 planes
and runs the Gram products over everything staged when the buffer fills or
when the Hessian is read, which amortises the Gram kernel's per-launch work
(reading β·H, writing both triangles) over many batches and gives the kernel
long K runs.

Planes per kind: 0 (GPTQ) Xᵀ; 1 (GPTAQ) Xᵀ and the bf16 hi/lo parts of
(X_fp − X)ᵀ; 2 (weighted, G groups) Xᵀ and G fp32 rows of per-token weights
s[t,g]·(1/T_b), from which the Gram kernel forms x·s itself.  Activations
that are not bf16 take P bf16 planes for Xᵀ that sum to it exactly (fp16: 2,
fp32: 3; the reference's ``inp.float()``, gptq_utils.py:125), and the
weighted kind then stages the hi/lo parts of (x·s[t,g])ᵀ as planes: every
Gram product runs once per plane of its column operand (four, resp. nine
times the bf16 Gram work for GPTQ).  The library gives each layout's height
(``g2ptq_hessian_stage_height``).

The first buffer holds 32 batches of the first batch's size (at least 65536
tokens): a calibration run is typically 32 or more batches, so its whole set
is usually one flush.  Later buffers grow ×4 at flush points (the buffer is
empty then, so nothing is copied), all up to ``budget_bytes`` (default a
quarter of the device's memory, at most 64 GiB; env ``G2PTQ_STAGE_BYTES``):
MI355X's 288 GB of HBM holds a whole decoder block's calibration set staged.
A read of the Hessian (the calibration is complete, or the caller looks at
it) flushes and frees the buffer; a later ``add_batch`` allocates a new one.

The buffer's row pitch is a multiple of 2048 tokens plus 1024 (an odd
multiple of 2 KiB): power-of-two-like pitches alias the rows of a Gram panel
onto few memory channels (measured on MI355X, C = 14336, K = 204800: a
528384-byte pitch, 512 KiB + 4 KiB, made the Gram 20 % slower than 518 to
560 KiB pitches).

Linears that read the same input (q/k/v, gate/up) get views of the same
tensor from their forward hooks (``inp[0].data``), so a driver that keeps one
Hessian per linear (gptq_utils.py:497-505) stages the same tokens once per
linear.  Each staged GPTQ batch records where its tokens came from (address,
count, row stride).  When a stager's first flush computes the Gram of a
sequence of batches that other live stagers have staged from the same
addresses, in the same order, the result and the staged tokens are kept for
them; each of their flushes compares its staged tokens with the kept ones on
the device (``g2ptq_staged_equal``) and copies the kept Gram only when they
are bit-identical, else runs its own.  The Gram is deterministic, so every
Hessian holds exactly the values it would have computed itself.
"""
import itertools
import os
import weakref

import torch

from . import _lib

# Staging budget in bytes per stager; None: a quarter of the device's memory,
# at most 64 GiB.
DEFAULT_BUDGET = (int(os.environ["G2PTQ_STAGE_BYTES"]) if os.environ.get("G2PTQ_STAGE_BYTES")
                  else None)
_MAX_BUDGET = 64 << 30
_FIRST_BATCHES = 32   # batches of the first batch's size that the first buffer holds
_PITCH_SKEW = 1024    # tokens added to every buffer's pitch (see above)
_FREE_MARGIN = 4 << 30  # device memory a new buffer leaves free

# Optional launch timing: when a list, every Gram flush appends
# (start event, end event, algorithmic flops, K, C), events recorded on the
# launch stream.
TIMING = None
_GRAM_PAD = 2048      # the Gram call may zero-pad K up to a multiple of this
_FIRST_TOKENS = 65536

KIND_GPTQ, KIND_GPTAQ, KIND_WEIGHTED = 0, 1, 2
_GRAM_WS = {KIND_GPTQ: "g2ptq_hessian_gram_workspace",
            KIND_GPTAQ: "g2ptq_gptaq_gram_workspace",
            KIND_WEIGHTED: "g2ptq_weighted_gram_workspace"}
# activation dtype codes of the any-dtype entry points, and the bf16 planes
# each stages for Xᵀ
DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2
_X_PLANES = {DTYPE_BF16: 1, DTYPE_F16: 2, DTYPE_F32: 3}


def _ceil(x, m):
    return (x + m - 1) // m * m


_QUERY_BYTES = 1 << 30  # buffers from this size on are checked against free memory
_MEMORY = {}


def _device_memory(device):
    """Total memory of a device (cached: the property query is a device call)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _MEMORY:
        _MEMORY[idx] = torch.cuda.get_device_properties(idx).total_memory
    return _MEMORY[idx]


def batch_source(X):
    """Where a (T, C) token matrix comes from: (address, T, row stride)."""
    return (X.data_ptr(), X.shape[0], X.stride(0))


# Gram results kept for stagers that staged from the same sources: key →
# (H, the staged buffer, its pitch, the waiting stagers, a serial number
# unique to the result).  Stagers by the first source they staged since their
# last flush, to find those that may share a flush.
_SHARED = {}
_BY_FIRST = {}
_SERIALS = itertools.count(1)


def _share_key(st, alpha):
    return (st.device, st.C, st.k, float(alpha), tuple(st.ids))


def _drop_waiter(st):
    """``st`` will not read the results kept for it (released, or flushed
    another way); results nobody waits for any more are freed."""
    for key in [k for k, v in _SHARED.items() if st in v[3] or not v[3]]:
        ws = _SHARED[key][3]
        ws.discard(st)
        if not ws:
            del _SHARED[key]


class GramStager:
    def __init__(self, columns, device, kind=KIND_GPTQ, groups=0, budget_bytes=None,
                 dtype=DTYPE_BF16):
        self.C = columns
        self.device = device
        self.kind = kind
        self.G = groups
        self.dtype = dtype
        # rows of staged bf16 per token column
        self.height = _lib.query_size_i64("g2ptq_hessian_stage_height", kind, dtype, columns,
                                          groups if kind == KIND_WEIGHTED else 0)
        budget = budget_bytes if budget_bytes is not None else DEFAULT_BUDGET
        if budget is None:
            budget = min(_MAX_BUDGET, _device_memory(torch.device(device)) // 4)
        per_token = self.height * 2
        self.max_tokens = max(_GRAM_PAD * 2, budget // per_token // _GRAM_PAD * _GRAM_PAD)
        self.buf = None
        self.cap = 0        # token columns of buf
        self.k = 0          # staged token columns (multiples of 64)
        # batch_source of each batch staged since the last flush; None once a
        # batch without one was staged
        self.ids = []
        self._first = None

    def fits(self, T):
        return self.buf is not None and self.k + _ceil(T, 64) + _GRAM_PAD <= self.cap

    def can_stage(self, T):
        """Whether a batch of T tokens can ever be staged (else update directly)."""
        return _ceil(T, 64) + _GRAM_PAD <= self.max_tokens

    def reserve(self, T):
        """With the buffer empty (just flushed because T more tokens did not fit,
        or never allocated): allocate the first buffer (room for 32 batches of T
        tokens, at least 65536), or one 4× larger, up to the budget."""
        assert self.k == 0
        need = _ceil(T, 64) + _GRAM_PAD
        if self.buf is None:
            cap = max(_FIRST_TOKENS, need, _FIRST_BATCHES * _ceil(T, 64) + _GRAM_PAD)
        else:
            cap = max(need, self.cap * 4)
        cap = _ceil(max(need, min(cap, self.max_tokens)), _GRAM_PAD) + _PITCH_SKEW
        if self.buf is not None and cap <= self.cap:
            return
        self.buf = None
        # Stay within what the device has free (other stagers of the same layer
        # group, the caller's tensors): shrink a large buffer rather than fail.
        # Buffers under _QUERY_BYTES skip the query (a device call per buffer:
        # the many small per-expert stagers of an MoE block would pay it often).
        per_token = self.height * 2
        if cap * per_token >= _QUERY_BYTES:
            free, _ = torch.cuda.mem_get_info(self.device)
            cached = (torch.cuda.memory_reserved(self.device)
                      - torch.cuda.memory_allocated(self.device))
            avail = free + cached - _FREE_MARGIN
            if cap * per_token > avail:
                cap = _ceil(max(need, avail // per_token - _PITCH_SKEW - _GRAM_PAD),
                            _GRAM_PAD) + _PITCH_SKEW
        self.buf = torch.empty(self.height, cap, dtype=torch.bfloat16, device=self.device)
        self.cap = cap

    def stage(self, X, Xfp=None, S=None, s_scale=1.0, act=None, act_alpha=0.0, act_beta=1.0,
              share=False):
        """Append one (T, C) bf16 batch: X_fp for GPTAQ; the (T, G) fp32
        saliencies, their scale and the act-square update for the weighted kind.
        ``share``: record the batch's source (a GPTQ batch whose Gram may be
        shared with other stagers of the same tokens)."""
        T, C = X.shape
        if self.ids is not None:
            if not share:
                self.ids = None
            else:
                src = batch_source(X)
                if not self.ids:
                    _BY_FIRST.setdefault(src, weakref.WeakSet()).add(self)
                    self._first = src
                self.ids.append(src)
        st, xt = _lib.stream_ptr(), _lib.ptr(self.buf)
        if self.dtype != DTYPE_BF16:
            _lib.call("g2ptq_hessian_stage_ex", st, self.kind, self.dtype, _lib.ptr(X),
                      _lib.ptr(Xfp), T, C, C, C, _lib.ptr(S), self.G,
                      S.stride(0) if S is not None else 0, float(s_scale), xt, self.cap, self.k,
                      _lib.ptr(act), float(act_alpha), float(act_beta))
        elif self.kind == KIND_GPTQ:
            fast = _lib.fastcall()
            if fast is None:
                _lib.call("g2ptq_hessian_stage", st, _lib.ptr(X), T, C, C, xt, self.cap, self.k)
            else:
                status = fast.hessian_stage(st, X.data_ptr(), T, C, C, xt, self.cap, self.k)
                if status:
                    _lib.raise_status("g2ptq_hessian_stage", status)
        elif self.kind == KIND_GPTAQ:
            _lib.call("g2ptq_gptaq_stage", st, _lib.ptr(X), _lib.ptr(Xfp), T, C, C, C, xt,
                      self.cap, self.k)
        else:
            _lib.call("g2ptq_weighted_stage", st, _lib.ptr(X), T, C, C, _lib.ptr(S), self.G,
                      S.stride(0), float(s_scale), xt, self.cap, self.k, _lib.ptr(act),
                      float(act_alpha), float(act_beta))
        self.k += _ceil(T, 64)

    def flush(self, H, alpha, beta, Dx=None):
        """H = beta·H + alpha·(Gram of the staged tokens) (and Dx for GPTAQ;
        H is (G, C, C) for the weighted kind); empties the buffer.  Returns the
        serial number of a Gram result shared with other stagers (kept for
        them, or copied from one), else None."""
        if self.k == 0:
            return None
        if not H.is_cuda or (Dx is not None and not Dx.is_cuda):
            raise RuntimeError("staged Hessian tokens need the Hessian on the GPU: call "
                               "add_batch inside the onload context of the Hessian")
        # A first flush (beta = 0: H = alpha·Gram) of GPTQ batches staged from
        # the sources whose Gram another stager computed with the same alpha
        # copies it, once the device has found the staged tokens identical.
        key = None
        if (self.kind == KIND_GPTQ and self.dtype == DTYPE_BF16 and self.ids and beta == 0.0
                and Dx is None):
            key = _share_key(self, alpha)
            kept = _SHARED.get(key)
            if kept is not None and self in kept[3]:
                Hk, buf, cap, _, serial = kept
                equal = torch.ones(1, dtype=torch.int32, device=H.device)
                _lib.call("g2ptq_staged_equal", _lib.stream_ptr(), _lib.ptr(self.buf), self.cap,
                          _lib.ptr(buf), cap, self.height, self.k, _lib.ptr(equal))
                if equal.item():
                    H.copy_(Hk)
                    self._flushed()
                    return serial
        if self.dtype != DTYPE_BF16:
            nbytes = _lib.query_size("g2ptq_hessian_gram_ex_workspace", self.kind, self.dtype,
                                     self.k, self.C, self.G)
        elif self.kind == KIND_WEIGHTED:
            nbytes = _lib.query_size(_GRAM_WS[self.kind], self.k, self.C, self.G)
        else:
            nbytes = _lib.query_size(_GRAM_WS[self.kind], self.k, self.C)
        ws = _lib.workspace(nbytes, self.buf.device)
        if TIMING is not None:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
        st, xt, C = _lib.stream_ptr(), _lib.ptr(self.buf), self.C
        if self.dtype != DTYPE_BF16:
            _lib.call("g2ptq_hessian_gram_ex", st, self.kind, self.dtype, xt, self.cap, self.k, C,
                      self.G, float(alpha), float(beta), _lib.ptr(H), C, C * C, _lib.ptr(Dx), C,
                      _lib.ptr(ws), ws.numel())
            flops = 2.0 * self.k * C * C * {KIND_GPTQ: 1, KIND_GPTAQ: 2,
                                            KIND_WEIGHTED: self.G}[self.kind]
        elif self.kind == KIND_GPTQ:
            _lib.call("g2ptq_hessian_gram", st, xt, self.cap, self.k, C, float(alpha),
                      float(beta), _lib.ptr(H), C, _lib.ptr(ws), ws.numel())
            flops = 2.0 * self.k * C * C
        elif self.kind == KIND_GPTAQ:
            _lib.call("g2ptq_gptaq_gram", st, xt, self.cap, self.k, C, float(alpha), float(beta),
                      _lib.ptr(H), _lib.ptr(Dx), C, _lib.ptr(ws), ws.numel())
            flops = 4.0 * self.k * C * C
        else:
            _lib.call("g2ptq_weighted_gram", st, xt, self.cap, self.k, C, self.G, float(alpha),
                      float(beta), _lib.ptr(H), C, C * C, _lib.ptr(ws), ws.numel())
            flops = 2.0 * self.G * self.k * C * C
        if TIMING is not None:
            e1.record()
            TIMING.append((e0, e1, flops, self.k, C))
        if key is not None:
            # the live stagers holding the same staged sequence, each not yet flushed
            waiting = [st for st in list(_BY_FIRST.get(self.ids[0], ()))
                       if st is not self and st.k > 0 and st.kind == KIND_GPTQ and
                       st.dtype == self.dtype and st.ids == self.ids and
                       _share_key(st, alpha) == key]
            serial = None
            if waiting:
                serial = next(_SERIALS)
                _SHARED[key] = (H.clone(), self.buf, self.cap, weakref.WeakSet(waiting), serial)
            self._flushed()
            return serial
        self._flushed()
        return None

    def _flushed(self):
        """The buffer is empty: a new token sequence starts."""
        _drop_waiter(self)
        if self._first is not None:
            ws = _BY_FIRST.get(self._first)
            if ws is not None:
                ws.discard(self)
                if not ws:
                    del _BY_FIRST[self._first]
            self._first = None
        if len(_BY_FIRST) > 4096:  # stagers collected while holding tokens
            for t in [t for t, ws in _BY_FIRST.items() if not ws]:
                del _BY_FIRST[t]
        self.ids = []
        self.k = 0

    def release(self):
        self.buf = None
        self.cap = 0
        self._flushed()


def stager_for(owner, idx, device, kind, groups, dtype):
    """Layer ``idx``'s stager for batches of activation ``dtype``.  A stager
    holding tokens of another dtype is folded into the Hessian first and
    replaced (the running averages hold across any flush point)."""
    st = owner._stagers[idx]
    if st is not None and st.dtype != dtype:
        owner._flush_staged(idx)
        st.release()
        st = None
    if st is None:
        st = owner._stagers[idx] = GramStager(owner.columns, device, kind, groups, dtype=dtype)
    return st


def single_batch_stager(columns, device, kind, groups, dtype, T):
    """A stager holding exactly one batch of T tokens: the path of a batch
    larger than the staging budget for activations without a one-shot
    update entry point (fp16, fp32)."""
    st = GramStager(columns, device, kind, groups, dtype=dtype)
    st.max_tokens = _ceil(_ceil(T, 64) + _GRAM_PAD, _GRAM_PAD)
    st.reserve(T)
    return st


def lazy_counter(name):
    """A per-layer int64 device counter (``nsamples``, ``index``, ``total_tokens``)
    whose ``add_batch`` increments (``bump``) collect on the host and reach the
    tensor in one in-place add when it is read: a device op per call would
    cost more host time than the rest of ``add_batch``.  Readers get the
    stored tensor itself, so in-place updates by callers behave as on the
    reference's attribute."""
    private, pend = "_" + name, "_" + name + "_pending"

    def get(self):
        t = getattr(self, private, None)
        p = getattr(self, pend, None)
        if t is not None and p and any(p):
            t += torch.tensor(p, dtype=t.dtype).to(t.device)
            setattr(self, pend, [0] * len(p))
        return t

    def set(self, value):
        setattr(self, private, value)
        setattr(self, pend, [0] * (len(value) if value is not None else 0))

    return property(get, set)


def bump(owner, name, idx, amount):
    """``owner.<name>[idx] += amount`` for a ``lazy_counter`` attribute."""
    getattr(owner, "_" + name + "_pending")[idx] += amount


def staged_attr(name):
    """A Hessian attribute whose reads first fold every staged token into it
    (the owner's ``_flush_staged``) and free the staging buffers, and whose
    deletion (``= None``) folds them in and then drops the buffers."""
    private = "_" + name

    def get(self):
        self._flush_staged()
        for st in getattr(self, "_stagers", None) or ():
            if st is not None and st.buf is not None:
                st.release()
        return getattr(self, private, None)

    def set(self, value):
        if value is None and getattr(self, private, None) is not None:
            self._flush_staged()
        elif (value is not None and getattr(self, private, None) is not None
              and not self.__dict__.get("_same_values")):
            # a replaced Hessian is no longer the one a shared-input group's
            # cached factor (or its slot copies) came from
            self.__dict__.pop("_shared_factor", None)
            self.__dict__.pop("_h_alias", None)
            self.__dict__.pop("_gram_src", None)
        setattr(self, private, value)
        if value is None:
            for st in getattr(self, "_stagers", None) or ():
                if st is not None:
                    st.release()

    return property(get, set)
