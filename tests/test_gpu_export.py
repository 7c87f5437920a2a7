"""GPU: compressed-tensors export (utils/compressed_tensors_utils.py:22-53) through
g2ptq_pack_quantized, against the pinned oracle (oracle/pack.py)."""
import pytest
import torch

from oracle import pack as opack
from tests._util import gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits,rows,cols", [(4, 33, 4096), (4, 7, 100), (8, 5, 67), (3, 9, 130),
                                            (2, 4, 64)])
def test_pack_to_int32_matches_oracle(dev, bits, rows, cols):
    from g2ptq_amd.compressed_tensors_utils import pack_to_int32
    g = gen(700 + bits + cols)
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    codes = torch.randint(lo, hi + 1, (rows, cols), generator=g).to(torch.int8)
    got = pack_to_int32(codes.to(dev), bits)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), opack.pack_to_int32(codes, bits))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_compress_matches_oracle(dev, dtype):
    from g2ptq_amd.compressed_tensors_utils import compress, register_qparam_buffers
    g = gen(720)
    rows, cols, gs = 96, 512, 128
    layer = torch.nn.Linear(cols, rows, bias=False).to(device=dev, dtype=dtype)
    codes = torch.randint(-8, 8, (rows, cols), generator=g).float()
    Scale = (torch.rand(rows, cols // gs, generator=g) * 0.01 + 1e-3).repeat_interleave(gs, 1)
    compress(layer, Scale.to(dev), codes.to(dev), 4, gs)
    torch.cuda.synchronize()
    ref = opack.compress((rows, cols), dtype, Scale, codes, 4, gs)
    got = layer._export_qparams
    assert torch.equal(got["weight_packed"].cpu(), ref["weight_packed"])
    assert got["weight_scale"].dtype == dtype
    assert torch.equal(got["weight_scale"].cpu(), ref["weight_scale"])
    assert got["weight_shape"].tolist() == [rows, cols]
    register_qparam_buffers([layer])
    assert not hasattr(layer, "_export_qparams")
    assert {n for n, _ in layer.named_buffers()} == {"weight_packed", "weight_scale", "weight_shape"}
    bad = Scale.clone()
    bad[3, 200] *= 2
    with pytest.raises(AssertionError):
        compress(layer, bad.to(dev), codes.to(dev), 4, gs)


def _dequant_from_export(q, gs):
    """Unpack weight_packed (4-bit) and scale by weight_scale."""
    p = q["weight_packed"].cpu().to(torch.int64) & 0xFFFFFFFF
    rows, words = p.shape
    fields = torch.stack([(p >> (4 * i)) & 0xF for i in range(8)], dim=-1).reshape(rows, words * 8)
    codes = (fields - 8).float()
    scale = q["weight_scale"].cpu().float().repeat_interleave(gs, 1)
    return codes, codes * scale


@pytest.mark.parametrize("variant", ["gptq", "gptaq"])
def test_fasterquant_export_is_consistent(dev, variant):
    """fasterquant(export_compressed_tensors=True): the exported codes and group
    scales reproduce the written weights (sym W4 g128)."""
    from g2ptq_amd import GPTAQ, GPTQ, WeightQuantizer, make_group_quantizers
    C, R, gs = 256, 64, 128
    g = gen(730)
    layers = [torch.nn.Linear(C, R, bias=False).to(device=dev, dtype=torch.bfloat16) for _ in range(2)]
    with torch.no_grad():
        for l in layers:
            l.weight.copy_((torch.randn(R, C, generator=g) * 0.02).bfloat16())
    gq = GPTQ(layers) if variant == "gptq" else GPTAQ(layers)
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True)
    gq.quantizer = make_group_quantizers(q, C, gs)
    for _ in range(3):
        x = torch.randn(1, 512, C, generator=g).bfloat16().to(dev)
        for b in range(2):
            if variant == "gptaq":
                gq.fp_inp[b].append((x.float() + 0.01).bfloat16().reshape(-1, C))
            gq.add_batch(b, x, None)
    gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=gs, export_compressed_tensors=True,
                   backend="hip")
    for l in layers:
        codes, deq = _dequant_from_export(l._export_qparams, gs)
        assert codes.min() >= -8 and codes.max() <= 7
        w = l.weight.detach().float().cpu()
        # weight = bf16(scale·code); export = bf16(scale)·code: equal to bf16 rounding
        assert torch.allclose(deq, w, rtol=2 ** -7, atol=0)


def test_rtn_export(dev):
    """The RTN path (gptq_utils.py:598-680): grouped find_params + fake_quantize,
    then compress with the per-group scales expanded to columns."""
    from g2ptq_amd import WeightQuantizer
    from g2ptq_amd.compressed_tensors_utils import compress
    C, R, gs = 512, 48, 128
    g = gen(740)
    layer = torch.nn.Linear(C, R, bias=False).to(device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        layer.weight.copy_((torch.randn(R, C, generator=g) * 0.02).bfloat16())
    q = WeightQuantizer()
    q.configure(4, perchannel=True, sym=True, weight_groupsize=gs)
    W = layer.weight.data.float()
    q.find_params(W)
    qw, codes, scale = q.fake_quantize(W)
    Scale = scale.unsqueeze(-1).expand(-1, -1, gs).reshape(R, C)
    compress(layer, Scale, codes, q.bits, gs)
    torch.cuda.synchronize()
    ref = opack.compress((R, C), torch.bfloat16, Scale.cpu(), codes.cpu(), 4, gs)
    assert torch.equal(layer._export_qparams["weight_packed"].cpu(), ref["weight_packed"])
    assert torch.equal(layer._export_qparams["weight_scale"].cpu(), ref["weight_scale"])
