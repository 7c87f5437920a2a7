"""CPU: the oracle against the committed golden fixtures (tests/golden/)."""
import copy

import numpy as np
import pytest
import torch

from oracle import compensate as ocomp
from oracle import flows as oflows
from oracle import original_loops as oloops
from oracle import quant as oquant
from tests.golden import make_golden as mg


@pytest.fixture(scope="module")
def loops():
    return mg.load(mg.LOOPS_FILE)


@pytest.fixture(scope="module")
def flows():
    return mg.load(mg.FLOWS_FILE)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def _current_quantizers(original, bits, sym, groupsize, static):
    b, r, c = original.shape
    tpl = oquant.WeightQuantizer().configure(bits, sym=sym)
    if static:
        cur = []
        for s in range(0, c, groupsize):
            q = copy.deepcopy(tpl)
            q.find_params(original[:, :, s:s + groupsize].reshape(b * r, -1))
            cur.append(q)
        return cur
    if groupsize == -1:
        q = copy.deepcopy(tpl)
        q.find_params(original.reshape(b * r, c))
        return [q]
    return [copy.deepcopy(tpl) for _ in range((c + groupsize - 1) // groupsize)]


@pytest.mark.parametrize("ci", range(len(mg.LOOP_CONFIGS)))
@pytest.mark.parametrize("sym", [True, False])
def test_fixture_inputs_reproduce(loops, ci, sym):
    """The seeded generator still produces the stored inputs (guards the GPU tests,
    which regenerate nothing and read the stored arrays)."""
    key = f"{mg.LOOP_CONFIGS[ci][0]}_{'sym' if sym else 'asym'}"
    d = mg.loop_inputs(ci, sym)
    for k in ("weight", "hinv", "z", "ghinv", "p", "original"):
        assert torch.equal(d[k], _t(loops[f"{key}/in_{k}"])), k


@pytest.mark.parametrize("ci", range(len(mg.LOOP_CONFIGS)))
@pytest.mark.parametrize("sym", [True, False])
def test_refactored_oracle_matches_golden_loops(loops, ci, sym):
    """oracle.compensate (the reference's refactored torch path) reproduces the stored
    outputs of the pre-refactor loops: codes exactly, floats within 2e-5."""
    name, groupsize, static, actorder = mg.LOOP_CONFIGS[ci]
    key = f"{name}_{'sym' if sym else 'asym'}"
    bs, bits = mg.LOOP_SHAPE["blocksize"], mg.LOOP_SHAPE["bits"]
    f = {k: _t(loops[f"{key}/in_{k}"]) for k in ("weight", "hinv", "z", "ghinv", "p", "original",
                                                  "perm")}
    qperm = f["perm"] if static and actorder else None

    def check(variant, got):
        assert torch.equal(got[1], _t(loops[f"{key}/{variant}_codes"]).float()), variant
        for i, n in [(0, "q"), (2, "scale"), (3, "weight"), (4, "ghinv")]:
            if i < len(got):
                torch.testing.assert_close(got[i], _t(loops[f"{key}/{variant}_{n}"]),
                                           rtol=2e-5, atol=2e-5)

    w = f["weight"].clone()
    cur = _current_quantizers(f["original"], bits, sym, groupsize, static)
    check("gptq", (*ocomp.gptq_compensation(w, f["hinv"], cur, bs, groupsize, static, qperm), w))
    w, gh = f["weight"].clone(), f["ghinv"].clone()
    cur = _current_quantizers(f["original"], bits, sym, groupsize, static)
    check("g2ptq", (*ocomp.g2ptq_compensation(w, f["hinv"], f["z"], gh, cur, bs, groupsize, static,
                                              qperm), w, gh))
    w = f["weight"].clone()
    cur = _current_quantizers(f["original"], bits, sym, groupsize, static)
    check("gptaq", (*ocomp.gptaq_compensation(w, f["hinv"], f["p"], cur, bs, groupsize, static,
                                              qperm), w))


def test_original_loops_are_deterministic_against_golden(loops):
    """One stored case recomputed with the original loops: bit-identical."""
    name, groupsize, static, actorder = mg.LOOP_CONFIGS[1]
    key = f"{name}_sym"
    f = {k: _t(loops[f"{key}/in_{k}"]) for k in ("weight", "hinv", "original")}
    o = oquant.WeightQuantizer().configure(4, sym=True)
    o.find_params(f["original"].reshape(-1, f["original"].shape[-1]))
    res = oloops.gptq_loop(f["weight"].clone(), f["hinv"], o, None, 5, groupsize, None)
    assert torch.equal(res[1], _t(loops[f"{key}/gptq_codes"]).float())
    assert torch.equal(res[0], _t(loops[f"{key}/gptq_q"]))


def test_flow_hessians_match_golden(flows):
    d = mg.flow_inputs()
    assert np.array_equal(d["X"].view(torch.int16).numpy(), flows["in_X"])
    assert np.array_equal(d["W"].view(torch.int16).numpy(), flows["in_W"])
    st, sa, s2, sg = mg.flow_hessians(d)
    for k, H in {"gptq": st["H"], "gptaq": sa["H"], "gptaq_dXXT": sa["dXXT"], "g2ptq": s2["H"],
                 "guided": sg["H"]}.items():
        torch.testing.assert_close(torch.diagonal(H, dim1=-2, dim2=-1), _t(flows[f"H_{k}_diag"]),
                                   rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(H.sum(-1), _t(flows[f"H_{k}_rowsum"]), rtol=1e-4, atol=1e-4)


def test_flow_gptq_matches_golden(flows):
    """End-to-end oracle GPTQ flow from the stored X and W reproduces the stored codes."""
    d = mg.flow_inputs()
    st, _, _, _ = mg.flow_hessians(d)
    r = oflows.gptq_fasterquant(d["W"].float(), st["H"], 4, False, groupsize=128)
    codes = _t(flows["gptq_asym/codes"]).float()
    assert (r["W_int"] == codes).float().mean().item() >= 0.999
    e1 = oflows.reconstruction_error(d["W"].float(), r["Q"], st["H"])
    e2 = oflows.reconstruction_error(d["W"].float(), _t(flows["gptq_asym/q"]), st["H"])
    assert abs(e1 - e2) <= 1e-4 * e2


def test_flow_fixture_inputs_reproduce(flows):
    """The seeded flow generator (every draw from one CPU generator) still
    produces the stored flow inputs."""
    d = mg.flow_inputs()
    for k in ("X", "Xfp", "W"):
        assert torch.equal(d[k].view(torch.int16), _t(flows[f"in_{k}"])), k
    for k in ("sal", "grad"):
        assert torch.equal(d[k], _t(flows[f"in_{k}"])), k
