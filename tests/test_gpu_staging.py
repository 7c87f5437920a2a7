"""GPU: GPTQ.add_batch's staged Hessian (tokens transposed into a staging buffer,
one Gram launch per flush) equals the reference's per-batch running average
(gptq_utils/gptq_utils.py:115-126) at every point where H is read."""
import pytest
import torch

from oracle import hessian as ohess
from tests._util import gen

pytestmark = pytest.mark.gpu


def _layers(B, R, C, dev):
    return [torch.nn.Linear(C, R, bias=False).to(device=dev, dtype=torch.bfloat16) for _ in range(B)]


def _close(Hd, Hr, what):
    Hd = Hd.detach().cpu()
    scale = Hr.abs().max().item()
    err = (Hd - Hr).abs().max().item()
    assert err <= 2e-6 * scale * 8, f"{what}: max err {err} (scale {scale})"
    assert torch.equal(Hd, Hd.T), f"{what}: not symmetric"


def test_staged_hessian_across_flushes_growth_and_reads(dev, monkeypatch):
    from g2ptq_amd import GPTQ, _lib, _stage
    C, B = 640, 2
    rows = _lib.query_size_i64("g2ptq_hessian_stage_rows", C)
    # a budget of 8192 staged tokens: the first buffer holds 8192 columns, so the
    # batches below overflow it (flush), and the 9000-token batch bypasses staging
    monkeypatch.setattr(_stage, "DEFAULT_BUDGET", rows * 2 * 8192)
    gq = GPTQ(_layers(B, 64, C, dev))
    st = ohess.gptq_state(B, C)
    g = gen(77)
    sig = torch.exp(torch.randn(C, generator=g))
    shapes = [(2, 1000), (1, 2048), (3, 300), (1, 2500), (1, 9000), (4, 512), (1, 64), (1, 1)]
    for step, (bsz, T) in enumerate(shapes):
        x = (torch.randn(bsz, T, C, generator=g) * sig).bfloat16()
        for b in range(B):
            xin = x if b == 0 else x[:, : max(1, T // 2)].contiguous()
            gq.add_batch(b, xin.to(dev), None)
            ohess.gptq_add_batch(st, b, xin)
        if step == 3:  # read H mid-way: flushes, and accumulation continues after
            torch.cuda.synchronize()
            for b in range(B):
                _close(gq.H[b], st["H"][b], f"mid-way layer {b}")
    torch.cuda.synchronize()
    for b in range(B):
        _close(gq.H[b], st["H"][b], f"final layer {b}")
    assert gq.nsamples.tolist() == st["nsamples"]
    # 2-D input counts as one sample (gptq_utils.py:116-118)
    x2 = torch.randn(100, C, generator=g).bfloat16()
    gq.add_batch(0, x2.to(dev), None)
    ohess.gptq_add_batch(st, 0, x2)
    _close(gq.H[0], st["H"][0], "2-D batch")


def test_staged_hessian_feeds_fasterquant_and_free(dev):
    """fasterquant consumes the staged tokens (H read) and free() drops the buffers."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    from oracle import flows as oflows
    C, R = 256, 96
    layers = _layers(1, R, C, dev)
    with torch.no_grad():
        layers[0].weight.copy_((torch.randn(R, C, generator=gen(5)) * 0.02).bfloat16())
    W0 = layers[0].weight.detach().float().cpu().unsqueeze(0)
    gq = GPTQ(layers)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, 128)
    st = ohess.gptq_state(1, C)
    g = gen(6)
    for _ in range(5):
        x = torch.randn(1, 700, C, generator=g).bfloat16()
        gq.add_batch(0, x.to(dev), None)
        ohess.gptq_add_batch(st, 0, x)
    gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip")
    torch.cuda.synchronize()
    assert gq.H is None and all(s is None or s.buf is None for s in gq._stagers)
    Qd = layers[0].weight.detach().float().cpu().unsqueeze(0)
    ref = oflows.gptq_fasterquant(W0, st["H"], 4, True, groupsize=128)
    e_hip = oflows.reconstruction_error(W0, Qd, st["H"])
    e_ref = oflows.reconstruction_error(W0, ref["Q"].bfloat16().float(), st["H"])
    assert abs(e_hip - e_ref) <= 0.005 * e_ref
    gq.free()


def _small_budget(monkeypatch, C, kind, G=0, tokens=8192):
    """A staging budget of ``tokens`` token columns of the kind's layout."""
    from g2ptq_amd import _lib, _stage
    height = _lib.query_size_i64("g2ptq_hessian_stage_height", kind, 0, C, G)
    monkeypatch.setattr(_stage, "DEFAULT_BUDGET", height * 2 * tokens)


# (bsz, T) batches: overflow the 8192-token staging buffer (flush), grow it, and
# one batch (9000 tokens) larger than the budget takes the direct update.
_SHAPES = [(2, 700), (1, 2048), (3, 300), (1, 2500), (1, 9000), (4, 512), (1, 64), (1, 1)]


def test_staged_gptaq_across_flushes_growth_and_reads(dev, monkeypatch):
    """GPTAQ.add_batch staged (Xᵀ and the hi/lo planes of (X_fp − X)ᵀ) equals the
    reference's per-batch update of H and dXXT (gptaq_utils.py:130-148)."""
    from g2ptq_amd import GPTAQ
    C, B = 640, 2
    _small_budget(monkeypatch, C, 1, tokens=4096)
    gq = GPTAQ(_layers(B, 64, C, dev))
    st = ohess.gptaq_state(B, C)
    g = gen(78)
    sig = torch.exp(torch.randn(C, generator=g))
    for step, (bsz, T) in enumerate(_SHAPES):
        x = (torch.randn(bsz, T, C, generator=g) * sig).bfloat16()
        xf = (x.float() + 0.05 * sig * torch.randn(bsz, T, C, generator=g)).bfloat16()
        for b in range(B):
            gq.fp_inp[b].append(xf.reshape(-1, C).to(dev))
            gq.add_batch(b, x.to(dev), None)
            ohess.gptaq_add_batch(st, b, x, xf.reshape(-1, C))
        if step == 3:
            torch.cuda.synchronize()
            for b in range(B):
                _close(gq.H[b], st["H"][b], f"mid-way H {b}")
    torch.cuda.synchronize()
    for b in range(B):
        _close(gq.H[b], st["H"][b], f"final H {b}")
        D, Dr = gq.dXXT[b].cpu(), st["dXXT"][b]
        assert (D - Dr).abs().max() <= 5e-5 * Dr.abs().max(), f"dXXT {b}"
    assert gq.nsamples.tolist() == st["nsamples"]


def _weighted_close(Hd, Hr, what):
    Hd = Hd.detach().cpu()
    for gi in range(Hd.shape[0]):
        assert torch.equal(Hd[gi], Hd[gi].T), f"{what}: group {gi} not symmetric"
    err = (Hd - Hr).abs().max().item()
    assert err <= 1e-5 * Hr.abs().max().item(), f"{what}: max err {err}"


def test_staged_g2ptq_across_flushes_growth_and_reads(dev, monkeypatch):
    """G2PTQ.add_batch staged (per-batch 1/T_b folded into the staged token
    weights) equals the reference's running per-batch mean
    (g2ptq_utils.py:182-201)."""
    from g2ptq_amd import G2PTQ
    C, B, G = 384, 2, 4
    _small_budget(monkeypatch, C, 2, G, tokens=4096)
    g = gen(79)
    shapes = [(1, 700), (1, 2048), (1, 300), (1, 2500), (1, 5000), (1, 512), (1, 64), (1, 1)]
    xs = [(torch.randn(T, C, generator=g) * 2).bfloat16() for _, T in shapes]
    sals = [torch.rand(T, G, generator=g) * 3 for _, T in shapes]
    gq = G2PTQ(_layers(B, 64, C, dev), [[s.to(dev) for s in sals] for _ in range(B)],
               [None] * B, G)
    st = ohess.g2ptq_state(B, G, C)
    for step, (x, s) in enumerate(zip(xs, sals)):
        for b in range(B):
            gq.add_batch(b, x.to(dev), None)
            ohess.g2ptq_add_batch(st, b, x, s)
        if step == 3:
            torch.cuda.synchronize()
            for b in range(B):
                _weighted_close(gq.H[b], st["H"][b], f"mid-way layer {b}")
    torch.cuda.synchronize()
    for b in range(B):
        _weighted_close(gq.H[b], st["H"][b], f"final layer {b}")
        act = gq.act_square[b].cpu()
        assert (act - st["act_square"][b]).abs().max() <= 1e-5 * st["act_square"][b].abs().max()
    assert gq.index.tolist() == st["index"]
    assert gq.total_tokens.tolist() == st["total_tokens"]


def test_staged_guided_across_flushes(dev, monkeypatch):
    """GPTQGuided.add_batch staged equals the reference's plain sums
    (gptq_guided_utils.py:59-81)."""
    from g2ptq_amd import GPTQGuided
    C, G, seq = 320, 2, 600
    _small_budget(monkeypatch, C, 2, G, tokens=4096)
    g = gen(80)
    N = 12
    x = torch.randn(N, seq, C, generator=g).bfloat16()
    sal = torch.rand(N, seq, G, generator=g)
    gq = GPTQGuided(_layers(1, 32, C, dev), [sal], G)
    st = ohess.guided_state(1, G, C)
    for bsz in (1, 3, 2, 5, 1):
        k = st["index"][0]
        gq.add_batch(0, x[k:k + bsz].to(dev), None)
        ohess.guided_add_batch(st, 0, x[k:k + bsz], sal)
    torch.cuda.synchronize()
    _weighted_close(gq.H[0], st["H"][0], "guided")
    act = gq.act_square[0].cpu()
    assert (act - st["act_square"][0]).abs().max() <= 1e-5 * st["act_square"][0].abs().max()


def test_staging_buffer_shrinks_to_free_memory(dev, monkeypatch):
    """With little device memory free, the first buffer is cut to what fits
    (at least one batch), and the Hessian still equals the oracle's."""
    import torch as _t
    from g2ptq_amd import GPTQ, _lib, _stage
    C = 384
    rows = _lib.query_size_i64("g2ptq_hessian_stage_rows", C)
    real = _t.cuda.mem_get_info

    def tight(device=None):
        free, total = real(device)
        # room for about 12000 tokens beyond the margin, whatever torch has cached
        cached = _t.cuda.memory_reserved(device) - _t.cuda.memory_allocated(device)
        return _stage._FREE_MARGIN + rows * 2 * 12000 - cached, total

    monkeypatch.setattr(_t.cuda, "mem_get_info", tight)
    # buffers this small skip the free-memory query unless the threshold is lowered
    monkeypatch.setattr(_stage, "_QUERY_BYTES", 0)
    gq = GPTQ(_layers(1, 64, C, dev))
    st = ohess.gptq_state(1, C)
    g = gen(81)
    for _ in range(6):
        x = torch.randn(1, 3000, C, generator=g).bfloat16()
        gq.add_batch(0, x.to(dev), None)
        ohess.gptq_add_batch(st, 0, x)
    cap = gq._stagers[0].cap
    assert 3000 <= cap < 32 * 3000, cap
    torch.cuda.synchronize()
    _close(gq.H[0], st["H"][0], "shrunk staging")


def _shared_insts(dev, C, B):
    from g2ptq_amd import GPTQ
    return GPTQ(_layers(1, 64, C, dev)), GPTQ(_layers(B, 64, C, dev))


def test_linears_fed_the_same_tensors_share_their_gram(dev):
    """The reference's driver keeps one Hessian per linear (gptq_utils.py:497-505):
    q and the k/v pair receive views of the same input tensors from their hooks
    (``inp[0].data``).  Their first flushes run one Gram and copy it to the
    others after the device compare of the staged tokens, bit for bit what each
    computes on its own (a control fed clones of the same tensors, which stages
    and multiplies by itself), and nothing is kept once every slot has read it."""
    from g2ptq_amd import GPTQ, _stage
    C = 768
    g = gen(4101)
    xs = [(torch.randn(2, 512, C, generator=g) * 2).bfloat16().to(dev) for _ in range(4)]
    q, kv = _shared_insts(dev, C, 2)
    ctl = GPTQ(_layers(1, 64, C, dev))
    for x in xs:
        q.add_batch(0, x.data, None)
        kv.add_batch(0, x.data, None)
        kv.add_batch(1, x.data, None)
        ctl.add_batch(0, x.clone(), None)
    old, _stage.TIMING = _stage.TIMING, []
    try:
        Hq, Hkv, Hc = q.H.clone(), kv.H.clone(), ctl.H.clone()
        grams = len(_stage.TIMING)
    finally:
        _stage.TIMING = old
    torch.cuda.synchronize()
    assert grams == 2, grams  # q's (kept for the k/v slots) and the control's
    assert torch.equal(Hq[0], Hc[0])
    assert torch.equal(Hkv[0], Hc[0]) and torch.equal(Hkv[1], Hc[0])
    assert not _stage._SHARED
    # the result matches the reference's running average
    st = ohess.gptq_state(1, C)
    for x in xs:
        ohess.gptq_add_batch(st, 0, x.cpu())
    _close(Hc[0], st["H"][0], "shared Gram")


def test_changed_or_different_batches_do_not_share(dev):
    """A tensor changed in place after one linear staged it (same address, other
    tokens: the device compare refuses the copy), a batch only one linear saw,
    and a second flush (beta ≠ 0) each make the Hessians compute their own
    Gram; a result kept for a linear that then flushes differently is freed."""
    from g2ptq_amd import GPTQ, _stage
    C = 512
    g = gen(4102)
    x1 = torch.randn(1, 1024, C, generator=g).bfloat16().to(dev)
    x2 = torch.randn(1, 1024, C, generator=g).bfloat16().to(dev)
    # changed in place between the two linears' hooks
    a, b = _shared_insts(dev, C, 1)
    a.add_batch(0, x1, None)
    x1.mul_(2)
    b.add_batch(0, x1, None)
    old, _stage.TIMING = _stage.TIMING, []
    try:
        Ha, Hb = a.H.clone(), b.H.clone()
        grams = len(_stage.TIMING)
    finally:
        _stage.TIMING = old
    torch.cuda.synchronize()
    assert grams == 2 and not _stage._SHARED
    assert torch.equal(Hb[0], 4 * Ha[0])  # bf16 doubling and the Gram's sums are exact
    # an extra batch on one linear: another sequence, nothing shared or kept
    a, b = _shared_insts(dev, C, 1)
    for inst in (a, b):
        inst.add_batch(0, x2, None)
    b.add_batch(0, x1, None)
    old, _stage.TIMING = _stage.TIMING, []
    try:
        a.H, b.H  # noqa: B018 (reads flush)
        grams = len(_stage.TIMING)
    finally:
        _stage.TIMING = old
    assert grams == 2 and not _stage._SHARED
    # same batches, but the second linear's own Hessian had an earlier flush
    # (its next flush has beta ≠ 0): it computes its own Gram, and the result
    # kept for it is freed when it does
    a, b = _shared_insts(dev, C, 1)
    b.add_batch(0, x1, None)
    b.H  # noqa: B018
    for inst in (a, b):
        inst.add_batch(0, x2, None)
    Ha, Hb = a.H.clone(), b.H.clone()
    torch.cuda.synchronize()
    assert not _stage._SHARED
    ctl = GPTQ(_layers(1, 64, C, dev))
    ctl.add_batch(0, x1.clone(), None)
    ctl.H  # noqa: B018 (the same two flushes as the second linear's)
    ctl.add_batch(0, x2.clone(), None)
    assert torch.equal(Hb[0], ctl.H[0])
    c2 = GPTQ(_layers(1, 64, C, dev))
    c2.add_batch(0, x2.clone(), None)
    assert torch.equal(Ha[0], c2.H[0])


def test_slots_holding_one_shared_gram_factor_once(dev):
    """A two-slot instance (gate/up) whose slots staged the same hook inputs: the
    second slot copies the first's Gram, the instance records the slots as
    copies, and its batched factor factors one of them; the quantized weights
    equal those of an instance fed clones (two Grams, two factors) bit for bit."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers, _stage
    C, R = 512, 96
    g = gen(4103)
    xs = [(torch.randn(2, 256, C, generator=g) * torch.exp(torch.randn(C, generator=g)))
          .bfloat16().to(dev) for _ in range(3)]
    w = [(torch.randn(R, C, generator=g) * 0.02).bfloat16() for _ in range(2)]

    def inst(clone):
        lins = _layers(2, R, C, dev)
        for lin, wi in zip(lins, w):
            with torch.no_grad():
                lin.weight.copy_(wi.to(dev))
        gq = GPTQ(lins)
        q = WeightQuantizer()
        q.configure(4, perchannel=True, sym=True)
        gq.quantizer = make_group_quantizers(q, C, 128)
        # the control's clones all stay alive: no two at one address
        inputs = [[x.clone() if clone else x.data for _ in range(2)] for x in xs]
        for xb in inputs:
            for b in range(2):
                gq.add_batch(b, xb[b], None)
        return gq, lins

    a, la = inst(False)
    c, lc = inst(True)
    Ha, Hc = a.H.clone(), c.H.clone()
    assert a.__dict__.get("_h_alias") == {1: 0}
    assert "_h_alias" not in c.__dict__
    assert torch.equal(Ha, Hc) and not _stage._SHARED
    for gq in (a, c):
        gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip")
    torch.cuda.synchronize()
    for x, y in zip(la, lc):
        assert torch.equal(x.weight, y.weight)


def test_instances_holding_one_shared_gram_factor_once(dev, monkeypatch):
    """q and the k/v pair hold copies of one Gram result: q's fasterquant factors
    it, the k/v instance reuses that factor (one factor launch for both), and
    the quantized weights equal those of instances fed separate clones."""
    from g2ptq_amd import GPTQ, WeightQuantizer, _lib, make_group_quantizers
    C, R = 512, 80
    g = gen(4104)
    xs = [(torch.randn(2, 256, C, generator=g) * torch.exp(torch.randn(C, generator=g)))
          .bfloat16().to(dev) for _ in range(3)]
    w = [(torch.randn(R, C, generator=g) * 0.02).bfloat16() for _ in range(3)]

    def make(ws):
        lins = _layers(len(ws), R, C, dev)
        for lin, wi in zip(lins, ws):
            with torch.no_grad():
                lin.weight.copy_(wi.to(dev))
        gq = GPTQ(lins)
        q = WeightQuantizer()
        q.configure(4, perchannel=True, sym=True)
        gq.quantizer = make_group_quantizers(q, C, 128)
        return gq, lins

    (q, lq), (kv, lkv) = make(w[:1]), make(w[1:])
    (qc, lqc), (kvc, lkvc) = make(w[:1]), make(w[1:])
    clones = [[x.clone() for _ in range(3)] for x in xs]  # all alive: distinct addresses
    for x, cl in zip(xs, clones):
        q.add_batch(0, x.data, None)
        kv.add_batch(0, x.data, None)
        kv.add_batch(1, x.data, None)
        qc.add_batch(0, cl[0], None)
        kvc.add_batch(0, cl[1], None)
        kvc.add_batch(1, cl[2], None)
    calls = []
    real = _lib.call

    def counting(name, *args):
        if name == "g2ptq_inv_chol_upper":
            calls.append(name)
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", counting)
    for gq in (q, kv):
        gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip")
    shared_factors = len(calls)
    for gq in (qc, kvc):
        gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip")
    torch.cuda.synchronize()
    assert shared_factors == 1 and len(calls) == 3, calls
    for x, y in zip(lq + lkv, lqc + lkvc):
        assert torch.equal(x.weight, y.weight)
