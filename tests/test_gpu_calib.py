"""GPU: calibration statistics (gptq_utils/g2ptq_utils.py:586-766) — the HIP
reductions against the CPU oracle and against the reference's own torch
expressions evaluated on the GPU."""
import numpy as np
import pytest
import torch
from torch import nn

from oracle import calib as ocalib
from tests._util import gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,G,dtype", [((2, 96, 512), 4, torch.bfloat16),
                                           ((300, 768), 8, torch.float32),
                                           ((1, 5, 4096), 4, torch.float16)])
def test_group_mean_square_matches_oracle(dev, shape, G, dtype):
    from g2ptq_amd.calib_utils import group_mean_square
    x = (torch.randn(*shape, generator=gen(31)) * 1e-3).to(dtype)
    got = group_mean_square(x.to(dev), G).cpu()
    ref = ocalib.group_mean_square(x, G)
    assert got.shape == ref.shape
    assert torch.allclose(got, ref, rtol=3e-6, atol=0)
    # the reference's expression on the GPU (summation order differs only)
    xd = x.to(dev).reshape(-1, shape[-1])
    t = xd.float().pow(2).view(xd.shape[0], G, -1).mean(dim=-1).cpu()
    assert torch.allclose(got, t, rtol=3e-6, atol=0)


def test_group_mean_square_rejects_ragged_groups(dev):
    from g2ptq_amd.calib_utils import group_mean_square
    with pytest.raises(RuntimeError):
        group_mean_square(torch.zeros(4, 10, device=dev), 3)


def test_running_mean_is_the_reference_expression(dev):
    """cache·(k/(k+1)) + grad.float()/(n·(k+1)) over five batches: bit-exact against
    torch evaluating the reference's expression on the GPU, and the oracle."""
    from g2ptq_amd.calib_utils import running_mean_update
    gg = gen(32)
    grads = [(torch.randn(96, 130, generator=gg) * 1e-2).bfloat16() for _ in range(5)]
    ns = [8192, 4096, 777, 1, 12000]
    c_hip, c_t, c_o = None, 0, None
    for i, (gr, n) in enumerate(zip(grads, ns)):
        gd = gr.to(dev)
        c_hip = running_mean_update(c_hip, gd, n, i)
        c_t = c_t * (i / (i + 1))                      # g2ptq_utils.py:709-712
        c_t = c_t + gd.float() / (n * (i + 1))
        c_o = ocalib.running_mean(c_o, gr, n, i)
        torch.cuda.synchronize()
        assert torch.equal(c_hip.cpu(), c_t.cpu()), i
        assert torch.equal(c_hip.cpu(), c_o), i


def _block(dev, hidden=256, inter=384):
    torch.manual_seed(7)
    m = nn.ModuleDict({"up": nn.Linear(hidden, inter, bias=False),
                       "down": nn.Linear(inter, hidden, bias=False)}).to(dev)
    return m


def _run(m, x):
    return m["down"](torch.relu(m["up"](x)))


def test_saliency_and_gradient_caches_end_to_end(dev):
    """The caches hooked into a two-linear block over three batches and two loss
    types, then summarized with loss weights: equal to the reference's
    expressions on the same autograd gradients."""
    from g2ptq_amd.calib_utils import GradientCache, SaliencyCache
    m = _block(dev)
    full = {"up": m["up"], "down": m["down"]}
    names, G = ["up", "down"], 4
    sal, grd = SaliencyCache(names, G), GradientCache(names, G)
    sal.set_forward_hook(full)
    grd.set_forward_hook(full)
    gg = gen(33)
    xs = [torch.randn(2, 64, 256, generator=gg).to(dev) for _ in range(3)]
    ref_sal = {n: {"block": [], "kl": []} for n in names}
    ref_grad = {n: {} for n in names}
    ref_idx = {n: {} for n in names}
    for x in xs:
        for loss_type in ("block", "kl"):
            out = _run(m, x)
            loss = out.pow(2).mean() if loss_type == "block" else out.abs().mean()
            outs = [sal.outs[n] for n in names]
            gouts = torch.autograd.grad(loss, outs, retain_graph=True)
            wgrads = torch.autograd.grad(loss, [full[n].weight for n in names], retain_graph=True)
            for n, go, gw in zip(names, gouts, wgrads):
                g2 = go.reshape(-1, go.shape[-1])
                ref_sal[n][loss_type].append(
                    g2.float().pow(2).view(g2.shape[0], G, -1).mean(dim=-1))
                k = ref_idx[n].get(loss_type, 0)
                c = ref_grad[n].get(loss_type, 0) * (k / (k + 1))
                ref_grad[n][loss_type] = c + gw.float() / (x.numel() // x.shape[-1] * (k + 1))
                ref_idx[n][loss_type] = k + 1
            sal.backward(loss, loss_type=loss_type, retain_graph=True)
            with grd.set_backward_hook(full, loss_type=loss_type):
                loss.backward()
            m.zero_grad(set_to_none=True)
    weights = {"block": 1.0, "kl": 0.5, "absent": 3.0}
    sal.summarize_saliency(weights)
    grd.summarize_gradients(weights)
    torch.cuda.synchronize()
    for n in names:
        exp = [1.0 * a + 0.5 * b for a, b in zip(ref_sal[n]["block"], ref_sal[n]["kl"])]
        assert len(sal.saliency_cache[n]) == 3
        for got, e in zip(sal.saliency_cache[n], exp):
            assert torch.allclose(got, e, rtol=3e-6, atol=1e-30)
        e = 1.0 * ref_grad[n]["block"] + 0.5 * ref_grad[n]["kl"]
        assert torch.equal(grd.gradients_cache[n], e), n
    sal.clear_hook()
    grd.clear_hook()
    sal.clear_cache()
    grd.clear_cache()
    assert sal.saliency_cache["up"] == {} and grd.gradients_cache["down"] == {}


def test_fp_inputs_cache_offload_from_gpu(dev):
    """gptaq_utils.py:442-555 with device activations: offloaded batches go to
    page-locked host slabs through a copy stream and are complete once the hooks
    are cleared; shared-input members get the same host rows; GPTAQ consumes
    the FIFO exactly as it would the device tensors.  Each source tensor is
    dropped right after its forward and its memory refilled at once: the
    copy stream keeps the freed block reserved until the copy has read it."""
    from g2ptq_amd import GPTAQ
    from g2ptq_amd.calib_utils import FPInputsCache
    torch.manual_seed(11)
    full = {n: nn.Linear(256, 64, bias=False).to(dev).to(torch.bfloat16) for n in ("q", "k")}
    cache = FPInputsCache([["q", "k"]], full, nsamples=3, seqlen=128, dtype=torch.bfloat16,
                          offload_inps=True, shared_input_groups=[("q", "k")])
    cache.add_hook(full)
    refill = []
    for _ in range(3):
        x = torch.randn(1, 128, 256, device=dev).bfloat16()
        for n in ("q", "k"):
            full[n](x)
        del x  # the block returns to the allocator while its copy may be in flight
        refill.append(torch.zeros(1, 128, 256, device=dev, dtype=torch.bfloat16))
    cache.clear_hook()
    for n in ("q", "k"):
        assert len(cache.fp_cache[n]) == 3
        assert not cache.fp_cache[n][0].is_cuda and cache.fp_cache[n][0].is_pinned()
    assert cache.fp_cache["k"][2].data_ptr() == cache.fp_cache["q"][2].data_ptr()
    torch.manual_seed(11)
    ref = [torch.randn(1, 128, 256, device=dev).bfloat16() for _ in range(3)]
    for got, x in zip(cache.fp_cache["q"], ref):
        assert torch.equal(got, x.reshape(128, 256).cpu())
    # the FIFO feeds GPTAQ.add_batch like device tensors would
    a, b = GPTAQ([full["q"]]), GPTAQ([full["q"]])
    a.fp_inp[0] = list(cache.fp_cache["q"])
    b.fp_inp[0] = [x.reshape(128, 256) for x in ref]
    for x in ref:
        a.add_batch(0, x, None)
        b.add_batch(0, x, None)
    assert torch.equal(a.dXXT, b.dXXT) and torch.equal(a.H, b.H)
    cache.clear_cache()
