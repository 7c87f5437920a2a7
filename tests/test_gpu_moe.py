"""GPU: MoE expert stacking of the checkpoint (utils/models/mixins.py:93-144)
through ``g2ptq_concat``, bit-exact against the CPU oracle."""
import pytest
import torch
from torch import nn

from oracle import pack as opack
from tests._util import gen

pytestmark = pytest.mark.gpu


class _Expert(nn.Module):
    def __init__(self, hidden, inter):
        super().__init__()
        self.gate_proj = nn.Linear(hidden, inter, bias=False)
        self.up_proj = nn.Linear(hidden, inter, bias=False)
        self.down_proj = nn.Linear(inter, hidden, bias=False)


class _Experts(nn.ModuleList):
    def __init__(self, n, hidden, inter):
        super().__init__([_Expert(hidden, inter) for _ in range(n)])
        self.num_experts = n


def _experts(dev, E, hidden, inter, seed):
    torch.manual_seed(seed)
    return _Experts(E, hidden, inter).to(device=dev, dtype=torch.bfloat16)


def _export_rtn(experts, bits, gs):
    """RTN + compressed-tensors export of every expert linear (gptq_utils.py:598-680)."""
    from g2ptq_amd import WeightQuantizer
    from g2ptq_amd.compressed_tensors_utils import compress, register_qparam_buffers
    for ex in experts:
        for lin in (ex.gate_proj, ex.up_proj, ex.down_proj):
            W = lin.weight.data.float()
            q = WeightQuantizer()
            q.configure(bits, perchannel=True, sym=True, weight_groupsize=gs)
            q.find_params(W)
            fq, codes, scale = q.fake_quantize(W)
            Scale = scale.unsqueeze(-1).expand(-1, -1, gs).reshape(W.shape)
            compress(lin, Scale, codes, bits, gs)
            register_qparam_buffers([lin])
            lin.weight.data.copy_(fq.to(lin.weight.dtype))


def _snapshot(experts, names):
    return [[{n: getattr(getattr(ex, p), n).detach().cpu() for n in names}
             for ex in experts] for p in ("gate_proj", "up_proj", "down_proj")]


@pytest.mark.parametrize("E,hidden,inter,bits", [(8, 256, 96, 4), (5, 128, 40, 8)])
def test_stack_experts_packed_matches_oracle(dev, E, hidden, inter, bits):
    from g2ptq_amd.moe_utils import stack_experts
    experts = _experts(dev, E, hidden, inter, 5 + E)
    _export_rtn(experts, bits, 32 if inter % 32 == 0 else 8)
    g, u, d = _snapshot(experts, ("weight_packed", "weight_scale", "weight_shape"))
    ref = opack.stack_experts(g, u, d, weight_packed=True)
    stack_experts(experts, weight_packed=True)
    torch.cuda.synchronize()
    for k, v in ref.items():
        got = getattr(experts, k)
        assert got.dtype == v.dtype and tuple(got.shape) == tuple(v.shape), k
        assert torch.equal(got.detach().cpu(), v), k
    assert len(experts._modules) == 0
    assert not experts.gate_up_proj_packed.requires_grad
    with pytest.raises(NotImplementedError):
        experts(torch.zeros(1, hidden), None, None)


def test_stack_experts_weights_matches_oracle(dev):
    from g2ptq_amd.moe_utils import stack_experts
    E, hidden, inter = 16, 192, 64
    experts = _experts(dev, E, hidden, inter, 3)
    g, u, d = _snapshot(experts, ("weight",))
    ref = opack.stack_experts(g, u, d)
    stack_experts(experts)
    torch.cuda.synchronize()
    for k, v in ref.items():
        assert torch.equal(getattr(experts, k).detach().cpu(), v), k


def test_stack_cat_ragged_and_unaligned(dev):
    """Blocks of odd byte sizes at odd offsets take the byte path; row counts per
    group may differ between members but must sum equally (torch.stack rule)."""
    from g2ptq_amd.moe_utils import stack_cat
    gg = gen(6)
    a = [torch.randint(0, 255, (r, 3), generator=gg, dtype=torch.uint8) for r in (5, 2, 7, 1, 6)]
    groups = [(a[0], a[1]), (a[2],), (a[3], a[4])]
    out = stack_cat([tuple(t.to(dev) for t in grp) for grp in groups])
    ref = torch.stack([torch.cat(grp, 0) for grp in groups], 0)
    assert torch.equal(out.cpu(), ref)
    big = [torch.randn(3000, 17, generator=gg) for _ in range(3)]   # 204000 B, 16-aligned
    out = stack_cat([(t.to(dev),) for t in big])
    assert torch.equal(out.cpu(), torch.stack(big, 0))
    with pytest.raises(RuntimeError, match="equal size"):
        stack_cat([(a[0].to(dev),), (a[1].to(dev),)])
    with pytest.raises(RuntimeError):
        stack_cat([(a[0].to(dev), big[0].to(dev))])


def test_grouped_experts_with_routed_inputs_match_oracle(dev):
    """Config 4's structure at reduced size: 64 same-shape expert linears
    quantized as ONE layer batch (common_utils.py:60-85), each with its own
    routed 2-D calibration inputs (one sample per call, gptq_utils.py:115-126):
    Zipf-uneven token counts, experts called with empty batches (a sample with
    no tokens), one expert never called (no calibration: RTN).  GPTQ W4 sym
    g128 against the oracle under the end-to-end parity protocol."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    from oracle import flows as oflows
    from oracle import hessian as ohess
    from tests._util import assert_flow_parity
    E, R, C, batches, tb = 64, 64, 256, 8, 1024
    g = gen(640)
    sig = torch.exp(torch.randn(C, generator=g))
    p = torch.arange(1, E + 1, dtype=torch.float64) ** -1.1
    p[E - 1] = 0.0                                      # never routed, never called
    p[E - 2] = 0.0                                      # called with empty batches only
    lins = []
    for e in range(E):
        lin = nn.Linear(C, R, bias=False)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(R, C, generator=g) * 0.02)
        lins.append(lin.to(dev).to(torch.bfloat16))
    W0 = torch.stack([l.weight.detach().float().cpu() for l in lins])
    gq = GPTQ(lins)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, 128)
    st = ohess.gptq_state(E, C)
    counts = torch.zeros(E, dtype=torch.int64)
    empties = 0
    for _ in range(batches):
        x = (torch.randn(tb, C, generator=g) * sig).bfloat16()
        top = torch.multinomial(p.expand(tb, E), 2, replacement=False, generator=g)
        for e in range(E - 1):
            xe = x[(top == e).any(1)]
            if xe.shape[0] == 0 and e != E - 2 and e % 3:
                continue                                # most idle experts are not called
            empties += xe.shape[0] == 0
            counts[e] += xe.shape[0]
            gq.add_batch(e, xe.to(dev), None)
            ohess.gptq_add_batch(st, e, xe)
    assert empties > 0 and counts[E - 2] == 0 and counts[:8].min() > counts[32:E - 2].max()
    print(f"routed tokens per expert: {counts.tolist()}", flush=True)
    assert torch.equal(gq.nsamples.cpu(), torch.tensor(st["nsamples"]))
    H = st["H"].clone()
    gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip",
                   export_compressed_tensors=True)
    torch.cuda.synchronize()
    ref = oflows.gptq_fasterquant(W0, H, 4, True, groupsize=128)
    He = H.clone()
    idle = torch.tensor([bool((h == 0).all()) for h in He])
    He[idle] = torch.eye(C)                             # the Hessian RTN minimizes
    assert idle[E - 1] and idle[E - 2]
    assert_flow_parity("64 routed experts", lins, gq.quantizer, ref, W0, He, 4, 128, False)
