"""GPU: g2ptq_compensate_noalloc (the scratch-array variant of g2ptq_compensate)
against g2ptq_compensate on the same inputs, through the C ABI.

The two run the same kernels in the same order (the existing entry point is
given a workspace that selects the same super-block width, or a one-buffer
workspace beyond the scratch's super-block range), so every output is
compared bit for bit.  Two calls in a row, the second on a smaller input,
show that the shared scratch array carries nothing from one call to the next.
"""
import math

import pytest
import torch

from tests._util import assert_bitexact, gen

pytestmark = pytest.mark.gpu

BS = 128
SCRATCH = 32 << 20


def _inputs(B, R, C, seed):
    g = gen(seed)
    W = torch.randn(B, R, C, generator=g) * 0.02
    U = torch.triu(torch.randn(B, C, C, generator=g) * 0.002, diagonal=1)
    torch.diagonal(U, dim1=1, dim2=2).copy_(torch.rand(B, C, generator=g) * 0.5 + 0.75)
    P = torch.triu(torch.randn(B, C, C, generator=g) * 0.002, diagonal=1)
    Z = torch.randn(B, R, C, generator=g) * 1e-4
    GH = torch.randn(B, R, C, generator=g) * 1e-4
    return W, U, P, Z, GH


def _run(entry, variant, inputs, bits, sym, groupsize, ws_bytes=None):
    from g2ptq_amd import _core, _lib
    dev = torch.device("cuda:0")
    W, U, P, Z, GH = (t.to(dev).contiguous() for t in inputs)
    B, R, C = W.shape
    ngroups = 1 if groupsize == -1 else math.ceil(C / groupsize)
    stab = torch.zeros(ngroups, B * R, device=dev)
    ztab = torch.zeros(ngroups, B * R, device=dev)
    if groupsize == -1:  # one static group: parameters come in filled
        stab.fill_(0.01)
    Q, Wint, Scale = torch.empty_like(W), torch.empty_like(W), torch.empty_like(W)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    p = _lib.ptr
    args = [_core.stream(), variant, B, R, C, BS, p(W), p(U), p(P) if variant == 1 else None,
            p(Z) if variant == 2 else None, p(GH) if variant == 2 else None, bits, int(sym),
            groupsize, 0, 0, 2.4, 0.5, None, 0, None, p(stab), p(ztab), p(Q), p(Wint), p(Scale),
            p(flags)]
    if entry == "g2ptq_compensate":
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        args += [p(ws), ws.numel()]
    _lib.call(entry, *args)
    torch.cuda.synchronize()
    out = {"W": W, "Q": Q, "Wint": Wint, "Scale": Scale, "stab": stab, "ztab": ztab,
           "flags": flags}
    if variant == 2:
        out["GH"] = GH
    return {k: v.cpu() for k, v in out.items()}


def _al256(n):
    return (n + 255) // 256 * 256


# (variant, bits, sym, groupsize, first call (B, R, C), second call (B, R, C))
CASES = (
    (0, 4, True, 128, (2, 512, 1024), (1, 256, 512)),
    (0, 4, False, 64, (2, 384, 896), (1, 96, 320)),
    (1, 2, True, 64, (1, 512, 768), (1, 128, 256)),
    (2, 3, True, 128, (2, 256, 640), (1, 64, 384)),
    (0, 4, True, -1, (1, 300, 512), (1, 37, 200)),
)


@pytest.mark.parametrize("case", CASES, ids=[f"v{c[0]}_w{c[1]}_g{c[3]}" for c in CASES])
def test_noalloc_matches_compensate_twice(dev, case):
    variant, bits, sym, gs, first, second = case
    for i, (B, R, C) in enumerate((first, second)):
        print(f"noalloc case v{variant} w{bits} g{gs} call {i} B={B} R={R} C={C}", flush=True)
        inputs = _inputs(B, R, C, 900 + 10 * i + variant)
        # the super-block width the scratch allows, one buffer (no side-stream
        # lookahead); G2PTQ also holds one block's near-tail operand
        sb, extra = 512, (_al256(B * R * BS * 4) if variant == 2 else 0)
        if _al256(B * R * sb * 4) + extra > SCRATCH:
            sb, extra = BS, 0
        ref = _run("g2ptq_compensate", variant, inputs, bits, sym, gs,
                   ws_bytes=_al256(B * R * sb * 4) + extra)
        got = _run("g2ptq_compensate_noalloc", variant, inputs, bits, sym, gs)
        for k in ref:
            assert_bitexact(got[k], ref[k], f"call {i} {k}")


def test_noalloc_beyond_the_super_block_range(dev):
    """B·R above 16384 rows: the scratch holds one 128-column block's errors
    only, and the result equals g2ptq_compensate's with a one-block
    workspace; then a small call again."""
    for i, (B, R, C) in enumerate(((1, 20000, 640), (1, 512, 256))):
        print(f"noalloc large case call {i} B={B} R={R} C={C}", flush=True)
        inputs = _inputs(B, R, C, 950 + i)
        width = min(512, math.ceil(C / BS) * BS)  # the loop's super-block width
        sb = width if B * R * width * 4 <= SCRATCH else BS
        ref = _run("g2ptq_compensate", 0, inputs, 4, True, 128, ws_bytes=_al256(B * R * sb * 4))
        got = _run("g2ptq_compensate_noalloc", 0, inputs, 4, True, 128)
        for k in ref:
            assert_bitexact(got[k], ref[k], f"call {i} {k}")


def test_noalloc_rejects_sizes_beyond_the_scratch(dev):
    from g2ptq_amd import _core, _lib
    fake = _lib.ptr(torch.empty(1, device="cuda:0"))
    with pytest.raises(ValueError, match="exceeds the 33554432-byte scratch"):
        _lib.call("g2ptq_compensate_noalloc", _core.stream(), 0, 1, 65537, 256, 128, fake, fake,
                  None, None, None, 4, 1, 128, 0, 0, 2.4, 0.5, None, 0, None, fake, fake, fake,
                  None, None, fake)
