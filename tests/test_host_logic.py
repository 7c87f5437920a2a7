"""CPU: host-side logic of the drop-in classes (no kernels run)."""
import pytest
import torch

from g2ptq_amd import (SharedInputHessian, build_chunk_specs, make_group_quantizers,
                       merge_group_quantizers, validate_tensors)
from g2ptq_amd import _core
from g2ptq_amd.quant_utils import WeightQuantizer


def _linear(r, c):
    return torch.nn.Linear(c, r, bias=False)


def test_build_chunk_specs_groups_by_shape_and_chunks():
    """gptq_utils/common_utils.py:60-85: same-shaped modules batched, ``layer_bsz`` per chunk,
    first-seen order kept."""
    subset = {"q": _linear(64, 32), "k": _linear(16, 32), "v": _linear(16, 32),
              "o": _linear(64, 32), "gate": _linear(128, 32), "up": _linear(128, 32)}
    specs = build_chunk_specs(subset, layer_bsz=2)
    assert [s.chunk_names for s in specs] == [("q", "o"), ("k", "v"), ("gate", "up")]
    assert [(s.rows, s.columns) for s in specs] == [(64, 32), (16, 32), (128, 32)]
    specs = build_chunk_specs(subset, layer_bsz=1)
    assert len(specs) == 6 and all(s.num_layers == 1 for s in specs)


def test_build_chunk_specs_group_key():
    subset = {"a.q": _linear(8, 8), "a.o": _linear(8, 8), "b.q": _linear(8, 8)}
    specs = build_chunk_specs(subset, layer_bsz=4, group_key_fn=lambda n: n.split(".")[1])
    assert sorted(s.chunk_names for s in specs) == [("a.o",), ("a.q", "b.q")]


def test_make_and_merge_group_quantizers():
    """gptq_utils/common_utils.py:13-30: per-group copies; merging slices rows start:end
    and concatenates the groups' (rows, 1) parameters column-wise."""
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    qs = make_group_quantizers(q, 300, 128)
    assert len(qs) == 3 and qs[0] is not qs[1]
    assert len(make_group_quantizers(q, 300, -1)) == 1
    for g, qq in enumerate(qs):
        qq.scale = torch.arange(6, dtype=torch.float32).reshape(6, 1) + 10 * g
        qq.zero = torch.zeros(6, 1)
        qq._ready = True
    m = merge_group_quantizers(qs, 2, 4, 128)
    assert m.scale.shape == (2, 3)
    assert m.scale.tolist() == [[2, 12, 22], [3, 13, 23]]
    assert m.weight_groupsize == 128 and m.ready()


def test_validate_tensors_messages():
    """gptq_utils/graph_utils.py:12-20 — CPU tensors are rejected with RuntimeError."""
    with pytest.raises(RuntimeError, match="requires every tensor to be on CUDA"):
        validate_tensors("x", torch.zeros(2))


def test_backends_other_than_hip_are_rejected():
    with pytest.raises(NotImplementedError):
        _core.check_backend("triton")
    with pytest.raises(NotImplementedError):
        _core.check_backend("torch")
    _core.check_backend("hip")


def test_f32_rounding():
    assert _core.f32(0.1) == float(torch.tensor(0.1, dtype=torch.float32))
    n = 7
    assert _core.f32(n / (n + 3)) == float(torch.tensor(n / (n + 3), dtype=torch.float32))


def test_shared_input_hessian_membership():
    class Fake:
        def __init__(self, n):
            self.num_layers = n
            self.H = torch.zeros(n, 2, 2)
            self._n = [0] * n
            self.nsamples = torch.zeros(n, dtype=torch.long)
            self.calls = []

        def add_batch(self, idx, inp, out):
            self.calls.append(idx)
            self.H[idx] += 1
            self._n[idx] += 1
            self.nsamples[idx] += 1

    a, b = Fake(1), Fake(2)
    sh = SharedInputHessian([(a, 0), (b, 0), (b, 1)])
    sh.add_batch(None)
    sh.add_batch(None)
    sh.finalize()
    assert a.calls == [0, 0] and b.calls == []          # accumulated once, on the owner
    assert torch.equal(b.H[0], a.H[0]) and torch.equal(b.H[1], a.H[0])
    assert b._n == [2, 2] and b.nsamples.tolist() == [2, 2]
    assert a._shared_factor is sh and b._shared_factor is sh
    c = Fake(2)
    sh2 = SharedInputHessian([(c, 0)])
    sh2.finalize()
    assert not hasattr(c, "_shared_factor")             # not every slot is a member


def test_shared_input_factor_cache_invalidation():
    """A re-finalized group forgets the factors of its earlier calibration, and
    a member whose Hessian is replaced stops using the group's cached factor."""
    from g2ptq_amd import GPTQ
    a = GPTQ([torch.nn.Linear(8, 4, bias=False)])
    b = GPTQ([torch.nn.Linear(8, 4, bias=False)])
    sh = SharedInputHessian([(a, 0), (b, 0)])
    sh.store_factor((0.01, False), torch.eye(8), 0.01)
    sh.finalize()
    assert sh.cached_factor((0.01, False)) is None
    assert a._shared_factor is sh and b._shared_factor is sh
    a.H = torch.ones(1, 8, 8)
    assert not hasattr(a, "_shared_factor") and b._shared_factor is sh


def test_shared_input_refuses_non_plain_hessians():
    """GPTAQ, G2PTQ and GuidedQuant Hessians depend on more than the shared
    input: such members are refused."""
    from g2ptq_amd import GPTAQ, GPTQ
    lin = torch.nn.Linear(8, 4, bias=False)
    with pytest.raises(ValueError, match="GPTAQ"):
        SharedInputHessian([(GPTQ([lin]), 0), (GPTAQ([lin]), 0)])


def test_shared_input_slot_copies_map():
    """finalize maps an instance's later member slots to its first one (the
    batched factor factors that one only); the map goes away when the
    instance's Hessian is replaced, and each share adds its own slots."""
    from g2ptq_amd import GPTQ
    g = GPTQ([torch.nn.Linear(8, 4, bias=False) for _ in range(4)])
    SharedInputHessian([(g, 0), (g, 1)]).finalize()
    SharedInputHessian([(g, 2), (g, 3)]).finalize()
    assert g._h_alias == {1: 0, 3: 2}
    assert not hasattr(g, "_shared_factor")  # two shares: no single cached factor
    g.H = torch.ones(4, 8, 8)
    assert "_h_alias" not in g.__dict__


def test_shared_input_slot_map_rebuilt_after_recalibration():
    """add_batch on a two-slot member drops its slot map, and the next
    finalize builds it again (re-calibration of an MoE-chunk-like instance)."""
    from g2ptq_amd import GPTQ
    g = GPTQ([torch.nn.Linear(8, 4, bias=False) for _ in range(2)])
    sh = SharedInputHessian([(g, 0), (g, 1)])
    sh.finalize()
    assert g._h_alias == {1: 0}
    # the map is dropped before the input is checked (a CPU tensor is refused)
    with pytest.raises(RuntimeError, match="GPU"):
        g.add_batch(0, torch.zeros(1, 3, 8, dtype=torch.bfloat16), None)
    assert "_h_alias" not in g.__dict__
    sh.finalize()
    assert g._h_alias == {1: 0}


def test_onload_keeps_shared_factor_and_slot_map():
    """Moving an offloaded Hessian onto the device and back is the same
    Hessian: the group's cached factor and the slot map survive the swap,
    while a genuinely new Hessian still drops them."""
    from g2ptq_amd import GPTQ, _core
    g = GPTQ([torch.nn.Linear(8, 4, bias=False) for _ in range(2)], offload_hessians=True)
    sh = SharedInputHessian([(g, 0), (g, 1)])
    sh.finalize()
    with _core.onload_attrs(g, ("H",), enabled=True, device="cpu"):
        assert g._shared_factor is sh and g._h_alias == {1: 0}
    assert g._shared_factor is sh and g._h_alias == {1: 0}
    g.H = torch.ones(2, 8, 8)
    assert "_shared_factor" not in g.__dict__ and "_h_alias" not in g.__dict__


def test_factor_alias_map_is_checked(monkeypatch):
    """_core.factor factors the unaliased slots once, as one batch, and hands
    each aliased slot its source's U and damp."""
    from g2ptq_amd import _core
    seen = []

    def fake(H, percdamp, shared=None, key=None, alias=None):
        if alias:
            return real(H, percdamp, shared, key, alias)
        seen.append(H[:, 0, 0].tolist())
        return H * 2, [percdamp + i for i in range(H.shape[0])]

    real = _core.factor
    monkeypatch.setattr(_core, "factor", fake)
    H = torch.arange(4.0).view(4, 1, 1).expand(4, 2, 2).contiguous()
    H[1] = H[0]
    H[3] = H[2]
    U, d = real(H, 0.5, alias={1: 0, 3: 2})
    assert seen == [[0.0, 2.0]]
    assert torch.equal(U, H * 2) and d == [0.5, 0.5, 1.5, 1.5]


def test_weight_quantizer_deepcopy_is_independent():
    """make_group_quantizers deep-copies one quantizer per group: the copies are
    independent modules with the same configuration and buffers."""
    import copy
    from g2ptq_amd import WeightQuantizer, make_group_quantizers
    q = WeightQuantizer()
    q.configure(3, perchannel=True, sym=False, mse=True, grid=25)
    q.scale = torch.full((4, 1), 0.5)
    q.zero = torch.full((4, 1), -2.0)
    c = copy.deepcopy(q)
    assert type(c) is WeightQuantizer
    assert (c.bits, c.sym, c.mse, c.grid, c.maxq, c.minq) == (3, False, True, 25, 3, -4)
    assert torch.equal(c.scale, q.scale) and torch.equal(c.zero, q.zero)
    c.scale.mul_(2)
    c.bits = 4
    assert q.scale[0, 0] == 0.5 and q.bits == 3
    assert list(dict(c.named_buffers())) == ["scale", "zero"]
    assert set(c.state_dict()) == {"scale", "zero"}
    qs = make_group_quantizers(q, 300, 128)
    assert len(qs) == 3 and len({id(x.scale) for x in qs}) == 3


def _fp_cache_model():
    torch.manual_seed(0)
    return torch.nn.ModuleDict({"q": _linear(8, 16), "k": _linear(4, 16), "v": _linear(4, 16),
                                "o": _linear(16, 8)})


@pytest.mark.parametrize("offload", [False, True])
def test_fp_inputs_cache_shared_groups(offload):
    """gptaq_utils.py:442-555: each name's FIFO receives its input per batch (2-D
    view); offloaded, shared-input members point at the one host slice their
    first member copied, consecutive batches fill consecutive rows."""
    from g2ptq_amd.calib_utils import FPInputsCache
    m = _fp_cache_model()
    full = dict(m.items())
    cache = FPInputsCache([["q", "k", "v"], ["o"]], full, nsamples=4, seqlen=5,
                          dtype=torch.float32, offload_inps=offload,
                          shared_input_groups=[("q", "k", "v"), ("o",), ("not_here",)])
    cache.add_hook(full)
    xs = [torch.randn(1, 5, 16) for _ in range(3)]
    for x in xs:
        for n in ("q", "k", "v"):
            full[n](x)
        full["o"](torch.randn(1, 5, 8))
    cache.clear_hook()
    for n in ("q", "k", "v"):
        assert len(cache.fp_cache[n]) == 3
        for got, x in zip(cache.fp_cache[n], xs):
            assert torch.equal(got, x.reshape(5, 16))
    if offload:
        assert set(cache.slabs) == {"q", "o"}
        assert cache.slabs["q"].members == ("q", "k", "v")
        assert cache.slabs["q"].filled == 15 and cache.slabs["o"].filled == 15
        assert cache.fp_cache["k"][1].data_ptr() == cache.fp_cache["q"][1].data_ptr()
        assert torch.equal(cache.slabs["q"].buffer[5:10], xs[1].reshape(5, 16))
        # a member receiving another tensor than its group-mate is a spec error
        cache.add_hook(full)
        full["q"](xs[0])
        with pytest.raises(AssertionError, match="received a different tensor"):
            full["k"](torch.randn(1, 5, 16))
        cache.clear_hook()
    cache.clear_cache()
    assert cache.fp_cache == {} and cache.slabs == {}


def test_fp_inputs_cache_members_firing_out_of_order():
    """A member's k-th batch is its group's k-th batch whatever order the
    members fire in: q twice, then k twice, then v, all see the right rows."""
    from g2ptq_amd.calib_utils import FPInputsCache
    m = _fp_cache_model()
    full = dict(m.items())
    cache = FPInputsCache([["q", "k", "v"]], full, nsamples=2, seqlen=5, dtype=torch.float32,
                          offload_inps=True, shared_input_groups=[("q", "k", "v")])
    cache.add_hook(full)
    xs = [torch.randn(1, 5, 16) for _ in range(2)]
    for n in ("q", "k"):
        for x in xs:
            full[n](x)
    full["v"](xs[0])
    cache.clear_hook()
    assert cache.slabs["q"].filled == 10
    for n, k in (("q", 2), ("k", 2), ("v", 1)):
        assert len(cache.fp_cache[n]) == k
        for got, x in zip(cache.fp_cache[n], xs):
            assert torch.equal(got, x.reshape(5, 16))
        assert cache.fp_cache[n][0].data_ptr() == cache.slabs["q"].buffer.data_ptr()


def test_fp_inputs_cache_overflow():
    from g2ptq_amd.calib_utils import FPInputsCache
    m = _fp_cache_model()
    full = dict(m.items())
    cache = FPInputsCache([["o"]], full, nsamples=1, seqlen=4, dtype=torch.float32,
                          offload_inps=True, shared_input_groups=[("o",)])
    cache.add_hook(full)
    with pytest.raises(AssertionError, match="overflowed"):
        full["o"](torch.randn(1, 5, 8))


def test_lazy_counter_folds_host_increments_on_read():
    """nsamples / index: add_batch increments collect on the host and reach the
    stored tensor in one in-place add when it is read; callers get that tensor
    itself (in-place updates stick), and assignment resets the pending counts."""
    from g2ptq_amd._stage import bump, lazy_counter

    class Owner:
        nsamples = lazy_counter("nsamples")

    o = Owner()
    o.nsamples = torch.zeros(3, dtype=torch.long)
    bump(o, "nsamples", 1, 5)
    bump(o, "nsamples", 1, 2)
    bump(o, "nsamples", 0, 1)
    t = o.nsamples
    assert t.tolist() == [1, 7, 0]
    t[2] += 4
    assert o.nsamples is t and o.nsamples.tolist() == [1, 7, 4]
    bump(o, "nsamples", 2, 1)
    o.nsamples = torch.ones(3, dtype=torch.long)
    assert o.nsamples.tolist() == [1, 1, 1]
    o.nsamples = None
    assert o.nsamples is None


def test_guided_gptq_reuses_gptq_compensation():
    """tests/test_triton_compensation.py:908-916."""
    from g2ptq_amd import GPTQ, GPTQGuided
    assert GPTQGuided._run_compensation_block is GPTQ._run_compensation_block
    assert GPTQGuided._run_compensation is GPTQ._run_compensation



def test_batch_source_of_hook_views():
    """The source a staged GPTQ batch records: a hook's ``inp[0].data`` view of
    the same input gives the same source, other storage or another token count
    another (a shared Gram is still taken only after the device has compared
    the staged tokens)."""
    from g2ptq_amd._stage import batch_source
    x = torch.randn(8, 16)
    assert batch_source(x.data) == batch_source(x) == batch_source(x.view(8, 16))
    assert batch_source(x.clone()) != batch_source(x)
    assert batch_source(x[:4]) != batch_source(x)


def test_gram_factor_cache_keeps_two_results():
    """The factor cache of shared Gram results: keyed by the result's serial
    number and the factor options, the two most recently used kept."""
    from g2ptq_amd.gptq_utils import _GramFactors
    _GramFactors._cache.clear()
    a, b, c = _GramFactors(1), _GramFactors(2), _GramFactors(3)
    a.store_factor((0.01, False), "Ua", 0.01)
    b.store_factor((0.01, False), "Ub", 0.01)
    assert a.cached_factor((0.01, False)) == ("Ua", 0.01)  # a is now the most recent
    assert a.cached_factor((0.01, True)) is None           # other options: not cached
    c.store_factor((0.01, False), "Uc", 0.01)              # evicts b
    assert b.cached_factor((0.01, False)) is None
    assert a.cached_factor((0.01, False)) == ("Ua", 0.01)
    assert c.cached_factor((0.01, False)) == ("Uc", 0.01)
    _GramFactors._cache.clear()
