#!/usr/bin/env python3
"""Benchmark: one Llama-3-8B-shaped decoder block quantized per step (MI355X).

Workload: q/o 4096×4096, k/v 1024×4096, gate/up
14336×4096, down 4096×14336, random-init weights ~N(0, 0.02) in bf16;
calibration activations 128 × 2048 = 262,144 tokens per input, N(0,1) times a
per-channel LogNormal(0,1) scale, bf16, generated on the GPU and resident in
HBM before timing.  GPTQ W4 (symmetric, the reference default) g128,
blocksize 128, damp 0.01, act-order off.  Linears are grouped as the
reference driver does (true-sequential groups, same-shape layer batching):
{q}, {k, v}, {o}, {gate, up}, {down}; linears fed by the same input share
one Hessian.

A step = Hessian accumulation over all 262,144 tokens (add_batch per
calibration batch of 4 × 2048 tokens, like the reference scripts' --bsz 4)
+ fasterquant (damp, inverse-Cholesky factor, lazy-batch compensation,
write-back) for every group.

Prints one JSON line (rank 0).  ``--gpus N`` with N > 1 exits: this build
runs on one GPU.
"""
import argparse
import contextlib
import gc
import json
import os
import platform
import sys
import time

import torch

METRIC = "sec per 8B-shaped decoder block quantized (W4 g128) + Hessian TFLOP/s"
LINEARS = {
    "q_proj": (4096, 4096, "qkv"), "k_proj": (1024, 4096, "qkv"), "v_proj": (1024, 4096, "qkv"),
    "o_proj": (4096, 4096, "o"), "gate_proj": (14336, 4096, "mlp"), "up_proj": (14336, 4096, "mlp"),
    "down_proj": (4096, 14336, "down"),
}
SEQUENTIAL = [["q_proj", "k_proj", "v_proj"], ["o_proj"], ["gate_proj", "up_proj"], ["down_proj"]]
INPUT_DIM = {"qkv": 4096, "o": 4096, "mlp": 4096, "down": 14336}
N_TOKENS = 128 * 2048
SEQ = 2048
BSZ = 4
BITS, GROUPSIZE, SYM = 4, 128, True
PEAK_BF16 = 2.5e15
SEED = 42 + 1  # reference seed + config index


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-kernel-rates", action="store_true",
                   help="skip the standalone factor / sweep / tail-product timings")
    p.add_argument("--no-unchanged-driver", action="store_true",
                   help="skip the block timed the way the reference driver runs it "
                        "(per-linear Hessians, per-instance fasterquant)")
    p.add_argument("--no-g2ptq", action="store_true",
                   help="skip the config-3 G2PTQ block reported beside the benchmark line")
    p.add_argument("--no-config1", action="store_true",
                   help="skip config 1 (one fp32 linear) reported beside the benchmark line")
    p.add_argument("--tokens", type=int, default=N_TOKENS)
    p.add_argument("--calibrate-copy", action="store_true",
                   help="run one 1 GiB device copy first (the known-size reference kernel "
                        "for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling)")
    p.add_argument("--workload", default="cfg2", choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5"],
                   help="BASELINE.json config (cfg2 is the benchmark line; the others "
                        "report per-stage times of the parity configs)")
    return p.parse_args()


# ---------------------------------------------------------------------------
# The other BASELINE.json configs, reported per stage (not the benchmark line).
# ---------------------------------------------------------------------------

def _lognormal_channels(C, g, dev):
    return torch.exp(torch.randn(C, device=dev, generator=g))


def _tokens(n, C, sig, g, dev, chunk=16384):
    x = torch.empty(n, C, device=dev, dtype=torch.bfloat16)
    for t0 in range(0, n, chunk):
        t1 = min(n, t0 + chunk)
        x[t0:t1] = (torch.randn(t1 - t0, C, device=dev, generator=g) * sig).bfloat16()
    return x


def _linear(R, C, dtype, g, dev, outlier_cols=0):
    lin = torch.nn.Linear(C, R, bias=False, device=dev, dtype=dtype)
    w = torch.randn(R, C, device=dev, generator=g) * 0.02
    if outlier_cols:
        cols = torch.randperm(C, device=dev, generator=g)[:outlier_cols]
        w[:, cols] *= 10
    with torch.no_grad():
        lin.weight.copy_(w.to(dtype))
    return lin


def cfg1_inputs(dev):
    """configs[0]'s inputs: 262144 tokens × 4096 (LogNormal channels, bf16) and one
    4096×4096 fp32 linear ~N(0, 0.02) with round(1 %·4096) input columns ×10."""
    g = torch.Generator(device=dev).manual_seed(42)
    C, R, n = 4096, 4096, N_TOKENS
    X = _tokens(n, C, _lognormal_channels(C, g, dev), g, dev)
    lin = _linear(R, C, torch.float32, g, dev, outlier_cols=round(0.01 * C))
    return X, lin


def workload_cfg1(dev, steps, warmup):
    """one 4096×4096 fp32 linear (1 % of input columns ×10), GPTQ W4
    asym g128, 262144 tokens in batches of 8192."""
    from g2ptq_amd import GPTQ, WeightQuantizer, make_group_quantizers
    C, n = 4096, N_TOKENS
    X, lin = cfg1_inputs(dev)
    w0 = lin.weight.detach().clone()

    def step(ev):
        lin.weight.data.copy_(w0)
        gq = GPTQ([lin])
        q = WeightQuantizer()
        q.configure(4, perchannel=True, sym=False)
        gq.quantizer = make_group_quantizers(q, C, 128)
        e = ev()
        e[0].record()
        for t0 in range(0, n, 8192):
            gq.add_batch(0, X[t0:t0 + 8192].view(-1, SEQ, C), None)
        gq.H  # fold the staged tokens
        e[1].record()
        e[2].record()
        gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip")
        e[3].record()
        return e, 2.0 * n * C * C
    return step, "llama-free single linear 4096x4096 fp32, GPTQ W4 asym g128, 1% outlier columns"


def workload_cfg3(dev, steps, warmup):
    """the 8B-shaped block with G2PTQ W3 g128, 4 row groups, α = 0.1,
    gradients 1e-3·N(0,1)·|StudentT(3)| per row, saliencies σ_t²·χ²_{R/G}/(R/G)
    with σ_t ~ LogNormal(0, 0.5).  Saliency-weighted Hessians are per linear."""
    from g2ptq_amd import G2PTQ, WeightQuantizer, make_group_quantizers
    g = torch.Generator(device=dev).manual_seed(42 + 2)
    G, n, tb = 4, N_TOKENS, BSZ * SEQ
    acts = {k: _tokens(n, C, _lognormal_channels(C, g, dev), g, dev) for k, C in INPUT_DIM.items()}
    lins = {name: _linear(R, C, torch.bfloat16, g, dev) for name, (R, C, _) in LINEARS.items()}
    w0 = {k: v.weight.detach().clone() for k, v in lins.items()}
    grads, sals = {}, {}
    # the Student-t and χ² draws use the device's default generator: seed it
    torch.cuda.manual_seed(42 + 2)
    t_dist = torch.distributions.StudentT(torch.tensor(3.0, device=dev))
    for name, (R, C, key) in LINEARS.items():
        tau = t_dist.sample((R,)).abs()
        grads[name] = torch.randn(R, C, device=dev, generator=g) * 1e-3 * tau[:, None]
        chi = torch.distributions.Chi2(torch.tensor(float(R // G), device=dev))
        sal = []
        for _ in range(0, n, tb):
            sig = torch.exp(0.5 * torch.randn(tb, 1, device=dev, generator=g))
            sal.append((sig ** 2 * chi.sample((tb, G)) / (R // G)).float())
        sals[name] = sal
    flops = 0.0
    for name, (R, C, key) in LINEARS.items():
        flops += G * 2.0 * n * C * C

    def step(ev):
        for k, v in lins.items():
            v.weight.data.copy_(w0[k])
        e = ev()
        e[0].record()
        insts = []
        for names in SEQUENTIAL:
            # same-shape linears of a group are layer-batched (k/v, gate/up)
            by_shape = {}
            for nm in names:
                by_shape.setdefault(tuple(lins[nm].weight.shape), []).append(nm)
            for shape, nms in by_shape.items():
                gq = G2PTQ([lins[nm] for nm in nms], [list(sals[nm]) for nm in nms],
                           [grads[nm] for nm in nms], G)
                q = WeightQuantizer()
                q.configure(3, perchannel=True, sym=True)
                gq.quantizer = make_group_quantizers(q, shape[1], 128)
                X = acts[LINEARS[nms[0]][2]]
                for t0 in range(0, n, tb):
                    for b in range(len(nms)):
                        gq.add_batch(b, X[t0:t0 + tb], None)
                gq.H
                insts.append(gq)
        e[1].record()
        e[2].record()
        for gq in insts:
            gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, alpha=0.1,
                           enable_gradient_update=True, backend="hip")
            gq.free()
        e[3].record()
        return e, flops
    return step, "llama3-8b-block G2PTQ W3 sym g128, 4 row groups, alpha 0.1, 262144 tokens"


def workload_cfg5(dev, steps, warmup):
    """Llama-3-70B down_proj 8192×28672 bf16, GPTAQ W2 sym g64,
    α = 0.25, X_fp = X + N(0, 0.05·σ_c), 262144 tokens in batches of 8192."""
    from g2ptq_amd import GPTAQ, WeightQuantizer, make_group_quantizers
    g = torch.Generator(device=dev).manual_seed(42 + 4)
    C, R, n, tb = 28672, 8192, N_TOKENS, 8192
    sig = _lognormal_channels(C, g, dev)
    X = _tokens(n, C, sig, g, dev)
    Xfp = torch.empty_like(X)
    for t0 in range(0, n, 8192):
        Xfp[t0:t0 + 8192] = (X[t0:t0 + 8192].float() + 0.05 * sig *
                             torch.randn(8192, C, device=dev, generator=g)).bfloat16()
    lin = _linear(R, C, torch.bfloat16, g, dev)
    w0 = lin.weight.detach().clone()

    def step(ev):
        lin.weight.data.copy_(w0)
        gq = GPTAQ([lin])
        q = WeightQuantizer()
        q.configure(2, perchannel=True, sym=True)
        gq.quantizer = make_group_quantizers(q, C, 64)
        e = ev()
        e[0].record()
        for t0 in range(0, n, tb):
            gq.fp_inp[0].append(Xfp[t0:t0 + tb])
            gq.add_batch(0, X[t0:t0 + tb].view(-1, 4096, C), None)
        gq.H
        e[1].record()
        e[2].record()
        gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=64, alpha=0.25, backend="hip")
        e[3].record()
        gq.free()
        return e, 4.0 * n * C * C
    return step, "llama3-70b down_proj 8192x28672, GPTAQ W2 sym g64, alpha 0.25, 262144 tokens"


def workload_cfg4(dev, steps, warmup):
    """Qwen3-MoE-style block, hidden 2048, 128 experts (gate/up
    768×2048, down 2048×768), top-8 routing of 262144 tokens with Zipf(1.1)
    expert popularity (Gumbel-top-8 on log p_e, p_e ∝ (e+1)^-1.1), GPTQ W4 sym
    g128.  Each calibration batch (8192 tokens) delivers every expert its
    routed tokens as a 2-D input (one sample, as the reference's MoE hooks);
    an expert's gate and up share one Hessian; the 384 linears are
    layer-batched 64 per launch by shape."""
    from g2ptq_amd import GPTQ, WeightQuantizer, build_chunk_specs, make_group_quantizers
    from g2ptq_amd.shared import SharedInputHessian
    g = torch.Generator(device=dev).manual_seed(42 + 3)
    E, topk, H, I, n, tb = 128, 8, 2048, 768, N_TOKENS, BSZ * SEQ
    X = _tokens(n, H, _lognormal_channels(H, g, dev), g, dev)
    sig_i = _lognormal_channels(I, g, dev)
    logp = -1.1 * torch.log(torch.arange(1, E + 1, device=dev, dtype=torch.float32))
    logp = logp - torch.logsumexp(logp, 0)
    routed = []  # per batch: per expert (gate/up input, down input)
    counts = torch.zeros(E, dtype=torch.int64, device=dev)
    for t0 in range(0, n, tb):
        u = torch.rand(tb, E, device=dev, generator=g).clamp_(1e-20, 1.0)
        top = torch.topk(logp - torch.log(-torch.log(u)), topk, dim=1).indices
        order = torch.argsort(top.reshape(-1), stable=True)
        tok = torch.div(order, topk, rounding_mode="floor")
        per = torch.bincount(top.reshape(-1), minlength=E)
        counts += per
        splits = per.tolist()
        xs = X[t0:t0 + tb][tok].split(splits)
        batch = []
        for e in range(E):
            xi = (torch.randn(splits[e], I, device=dev, generator=g) * sig_i).bfloat16()
            batch.append((xs[e], xi))
        routed.append(batch)
    names = [f"e{e}.{k}" for e in range(E) for k in ("gate", "up", "down")]
    shapes = {"gate": (I, H), "up": (I, H), "down": (H, I)}
    lins = {nm: _linear(*shapes[nm.split(".")[1]], torch.bfloat16, g, dev) for nm in names}
    w0 = {k: v.weight.detach().clone() for k, v in lins.items()}
    flops = float((counts * (2 * H * H + 2 * I * I)).sum().item())
    stats = {"min_tokens": int(counts.min()), "max_tokens": int(counts.max())}

    def step(ev):
        for k, v in lins.items():
            v.weight.data.copy_(w0[k])
        e_ = ev()
        e_[0].record()
        specs = build_chunk_specs(lins, 64)
        slot, insts = {}, []
        for spec in specs:
            gq = GPTQ([lins[nm] for nm in spec.chunk_names])
            q = WeightQuantizer()
            q.configure(4, perchannel=True, sym=True)
            gq.quantizer = make_group_quantizers(q, spec.columns, 128)
            insts.append(gq)
            for i, nm in enumerate(spec.chunk_names):
                slot[nm] = (gq, i)
        shares = [SharedInputHessian([slot[f"e{e}.gate"], slot[f"e{e}.up"]]) for e in range(E)]
        for batch in routed:
            for e in range(E):
                xg, xd = batch[e]
                if xg.shape[0]:
                    shares[e].add_batch(xg)
                    gq, i = slot[f"e{e}.down"]
                    gq.add_batch(i, xd, None)
        for sh in shares:
            sh.finalize()
        for gq in insts:
            gq.H
        e_[1].record()
        e_[2].record()
        for gq in insts:
            gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=128, backend="hip")
            gq.free()
        e_[3].record()
        return e_, flops
    return step, (f"qwen3-moe-style block, 128 experts (768x2048 gate/up, 2048x768 down), top-8 "
                  f"Zipf(1.1) routing of 262144 tokens (per-expert tokens {stats['min_tokens']}.."
                  f"{stats['max_tokens']}), GPTQ W4 sym g128, 64 linears per launch")


@contextlib.contextmanager
def quiet_collector():
    """The timed steps with the interpreter's long-lived objects (torch's and
    this process's set-up) moved out of the garbage collector's generations:
    a full collection otherwise re-traverses all of them (about 60 ms on this
    image) and, when it falls while the GPU waits for the host, stalls the
    step (config 1 measured 6 ms per Hessian stage, 70 ms in the step with
    the collection).  Objects the steps create are still collected; no work
    of the path is skipped."""
    gc.collect()
    gc.freeze()
    try:
        yield
    finally:
        gc.unfreeze()


def run_other(args, dev):
    make = {"cfg1": workload_cfg1, "cfg3": workload_cfg3, "cfg4": workload_cfg4,
            "cfg5": workload_cfg5}[args.workload]
    step, desc = make(dev, args.steps, args.warmup)
    torch.cuda.synchronize()

    def ev():
        return [torch.cuda.Event(enable_timing=True) for _ in range(4)]

    for _ in range(args.warmup):
        step(ev)
    torch.cuda.synchronize()
    with quiet_collector():
        t0 = time.perf_counter()
        recs = [step(ev) for _ in range(args.steps)]
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
    h = sum(e[0].elapsed_time(e[1]) for e, _ in recs) / len(recs)
    qz = sum(e[2].elapsed_time(e[3]) for e, _ in recs) / len(recs)
    flops = recs[0][1]
    print(json.dumps({"workload": args.workload, "config": desc, "sec_per_step": round(wall, 4),
                      "stages_ms": {"hessian": round(h, 2), "factor_and_compensation": round(qz, 2)},
                      "hessian_tflops": round(flops / (h / 1e3) / 1e12, 1),
                      "hessian_flop_convention": "2*N*C^2 per Hessian product (GEMM convention)",
                      "steps": args.steps, "warmup": args.warmup}), flush=True)


def make_inputs(dev, n_tokens):
    g = torch.Generator(device=dev).manual_seed(SEED)
    acts = {}
    for key, C in INPUT_DIM.items():
        sig = torch.exp(torch.randn(C, device=dev, generator=g))
        x = torch.empty(n_tokens, C, device=dev, dtype=torch.bfloat16)
        for t0 in range(0, n_tokens, 16384):
            t1 = min(n_tokens, t0 + 16384)
            x[t0:t1] = (torch.randn(t1 - t0, C, device=dev, generator=g) * sig).bfloat16()
        acts[key] = x
    layers, w0 = {}, {}
    for name, (R, C, _) in LINEARS.items():
        lin = torch.nn.Linear(C, R, bias=False, device=dev, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_((torch.randn(R, C, device=dev, generator=g) * 0.02).bfloat16())
        layers[name] = lin
        w0[name] = lin.weight.detach().clone()
    return acts, layers, w0


def hessian_flops(n_tokens):
    """Unique Hessian work: one 2·N·C² Gram per distinct input."""
    return sum(2.0 * n_tokens * C * C for C in INPUT_DIM.values())


def run_step(acts, layers, w0, n_tokens, ev):
    from g2ptq_amd import GPTQ, WeightQuantizer, build_chunk_specs, make_group_quantizers
    from g2ptq_amd.shared import SharedInputHessian
    for name, lin in layers.items():
        lin.weight.data.copy_(w0[name])
    stream = torch.cuda.current_stream()
    hess_ms = 0.0
    quant_ms = 0.0
    for names in SEQUENTIAL:
        subset = {n: layers[n] for n in names}
        specs = build_chunk_specs(subset, 64)
        insts = []
        for spec in specs:
            gq = GPTQ([subset[n] for n in spec.chunk_names])
            q = WeightQuantizer()
            q.configure(BITS, perchannel=True, sym=SYM)
            gq.quantizer = make_group_quantizers(q, spec.columns, GROUPSIZE)
            insts.append((gq, spec))
        share = SharedInputHessian([(gq, i) for gq, spec in insts for i in range(spec.num_layers)])
        X = acts[LINEARS[names[0]][2]]
        C = X.shape[1]
        e0, e1 = ev()
        e0.record(stream)
        step_tok = BSZ * SEQ
        for t0 in range(0, n_tokens, step_tok):
            share.add_batch(X[t0:t0 + step_tok].view(-1, SEQ, C))
        share.finalize()  # reads H: runs the Gram over the staged tokens
        e1.record(stream)
        e2, e3 = ev()
        e2.record(stream)
        # every instance's fasterquant; instances that share the input (q and
        # k/v) run as one compensation loop over all their rows
        share.fasterquant(blocksize=128, percdamp=0.01, groupsize=GROUPSIZE, actorder=False,
                          static_groups=False, backend="hip")
        e3.record(stream)
        torch.cuda.synchronize()
        hess_ms += e0.elapsed_time(e1)
        quant_ms += e2.elapsed_time(e3)
    return hess_ms, quant_ms


def run_step_unchanged(acts, layers, w0, n_tokens, ev):
    """The same block the way the reference's gptq_fwrd driver (gptq_utils.py:478-563)
    runs it with only the backend switched: per true-sequential stage, one
    instance per same-shape chunk (build_chunk_specs), each linear's forward hook
    feeding its own Hessian (7 Hessians, no shared-input de-duplication), then
    each instance's own fasterquant."""
    from g2ptq_amd import GPTQ, WeightQuantizer, build_chunk_specs, make_group_quantizers
    for name, lin in layers.items():
        lin.weight.data.copy_(w0[name])
    stream = torch.cuda.current_stream()
    hess_ms = quant_ms = 0.0
    for names in SEQUENTIAL:
        subset = {n: layers[n] for n in names}
        insts = []
        for spec in build_chunk_specs(subset, 64):
            gq = GPTQ([subset[n] for n in spec.chunk_names])
            q = WeightQuantizer()
            q.configure(BITS, perchannel=True, sym=SYM)
            gq.quantizer = make_group_quantizers(q, spec.columns, GROUPSIZE)
            insts.append(gq)
        X = acts[LINEARS[names[0]][2]]
        C = X.shape[1]
        e0, e1 = ev()
        e0.record(stream)
        step_tok = BSZ * SEQ
        for t0 in range(0, n_tokens, step_tok):
            xb = X[t0:t0 + step_tok].view(-1, SEQ, C)
            for gq in insts:
                for i in range(gq.num_layers):
                    gq.add_batch(i, xb.data, None)  # each hook passes inp[0].data
        for gq in insts:
            gq.H  # the calibration pass ends: fold the staged tokens
        e1.record(stream)
        e2, e3 = ev()
        e2.record(stream)
        for gq in insts:
            gq.fasterquant(blocksize=128, percdamp=0.01, groupsize=GROUPSIZE, actorder=False,
                           static_groups=False, backend="hip")
            gq.free()
        e3.record(stream)
        torch.cuda.synchronize()
        hess_ms += e0.elapsed_time(e1)
        quant_ms += e2.elapsed_time(e3)
    return hess_ms, quant_ms


def unchanged_driver(acts, layers, w0, n_tokens, steps=3, warmup=1):
    """Seconds per block through run_step_unchanged (mean of ``steps``)."""
    def ev():
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    for _ in range(warmup):
        run_step_unchanged(acts, layers, w0, n_tokens, ev)
    torch.cuda.synchronize()
    hs, qs = [], []
    with quiet_collector():
        t0 = time.perf_counter()
        for _ in range(steps):
            h, q = run_step_unchanged(acts, layers, w0, n_tokens, ev)
            hs.append(h)
            qs.append(q)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / steps
    flops = sum(2.0 * n_tokens * C * C for _, C, _ in LINEARS.values())
    h = sum(hs) / steps
    return {"sec_per_block": round(wall, 4), "steps": steps, "warmup": warmup,
            "stages_ms": {"hessian": round(h, 2), "factor_and_compensation": round(sum(qs) / steps, 2)},
            "hessian_tflops_per_linear": round(flops / (h / 1e3) / 1e12, 1),
            "note": "reference driver layout with only the backend switched: 7 per-linear "
                    "Hessians fed inp[0].data views, one instance per same-shape chunk, "
                    "per-instance fasterquant (linears staged from the same inputs share "
                    "Gram results after a device compare of their staged tokens)"}


def _cpu_threads():
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    cores = len(os.sched_getaffinity(0))
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(cores)
    return cores


def _timed_cpu(fn):
    t = time.perf_counter()
    out = fn()
    return out, time.perf_counter() - t


def cpu_baseline(acts, w0, dev):
    """The oracle (torch-CPU restatement of the reference arithmetic) on the
    benchmark's own inputs, copied to the host, for one block as the reference
    computes it (7 per-linear Hessians, factors and compensations):
    Hessians on token slices scaled by N (the cost is ∝ N); every linear's
    damp + Cholesky chain in full, on the step's Hessians (computed on the GPU
    over all tokens and copied over); every weight row of every linear's
    compensation in full."""
    from g2ptq_amd import GPTQ
    from oracle import compensate as ocomp
    from oracle import factor as ofactor
    from oracle import hessian as ohess
    from oracle import quant as oquant
    cores = _cpu_threads()
    parts = {}
    for key, slice_tok in (("qkv", 8192), ("down", 2048)):
        x = acts[key][:slice_tok].cpu().unsqueeze(0)
        C = x.shape[-1]
        count = sum(1 for _, c, _ in LINEARS.values() if c == C)
        st = ohess.gptq_state(1, C)
        _, dt = _timed_cpu(lambda: ohess.gptq_add_batch(st, 0, x))
        parts[f"hessian_C{C}_x{count}"] = dt * (N_TOKENS / slice_tok) * count
    # the step's four distinct Hessians, from the GPU
    Hs = {}
    for key, X in acts.items():
        C = X.shape[1]
        gq = GPTQ([torch.nn.Linear(C, 1, bias=False, device=dev, dtype=torch.bfloat16)])
        for t0 in range(0, N_TOKENS, BSZ * SEQ):
            gq.add_batch(0, X[t0:t0 + BSZ * SEQ].view(-1, SEQ, C), None)
        Hs[key] = gq.H[0].cpu()
        gq.free()
    Us = {}
    for name, (R, C, key) in LINEARS.items():
        H = Hs[key].clone()
        W = w0[name].float().cpu().unsqueeze(0)
        (U, _), dt = _timed_cpu(lambda: ofactor.damp_chol_inv_upper(H, 0.01))
        parts[f"factor_{name}"] = dt
        qs = [oquant.WeightQuantizer().configure(BITS, sym=SYM) for _ in range(C // GROUPSIZE)]
        _, dt = _timed_cpu(lambda: ocomp.gptq_compensation(W, U.unsqueeze(0), qs, 128, GROUPSIZE,
                                                           False, None))
        parts[f"compensation_{name}"] = dt
        del U, W
    total = sum(parts.values())
    del Hs
    return {"value": total, "unit": "s", "cores": cores, "kind": "port", "cpu": _cpu_model(),
            "sample": ("oracle (torch-CPU, reference op order) on this run's own inputs: the 7 "
                       "per-linear Hessians on 8192 (C=4096) / 2048 (C=14336) token slices "
                       "scaled by N; every linear's damp+cholesky+cholesky_inverse+cholesky and "
                       "its whole compensation (every weight row) in full, on the step's "
                       "Hessians"),
            "parts_s": {k: round(v, 3) for k, v in parts.items()},
            "config1": cpu_baseline_config1(dev)}


def cpu_baseline_config1(dev):
    """configs[0] (the reference's CPU-runnable case) on the oracle, in full, on the
    benchmark's config-1 inputs copied to the host: the Hessian over all 262144
    tokens, damp + Cholesky chain, compensation of all 4096 rows."""
    from oracle import compensate as ocomp
    from oracle import factor as ofactor
    from oracle import hessian as ohess
    from oracle import quant as oquant
    X, lin = cfg1_inputs(dev)
    Xh = X.cpu()
    W = lin.weight.detach().cpu().unsqueeze(0)
    del X, lin
    torch.cuda.empty_cache()
    cores = _cpu_threads()
    C = W.shape[-1]
    st = ohess.gptq_state(1, C)
    parts = {}
    t = time.perf_counter()
    for t0 in range(0, N_TOKENS, BSZ * SEQ):
        ohess.gptq_add_batch(st, 0, Xh[t0:t0 + BSZ * SEQ].view(-1, SEQ, C))
    parts["hessian"] = time.perf_counter() - t
    del Xh
    H = st["H"]

    def quantize():
        ofactor.prepare_hessian(H, W)
        U, _ = ofactor.damp_chol_inv_upper(H[0], 0.01)
        qs = [oquant.WeightQuantizer().configure(4, sym=False) for _ in range(C // 128)]
        ocomp.gptq_compensation(W, U.unsqueeze(0), qs, 128, 128, False, None)

    _, parts["factor_and_compensation"] = _timed_cpu(quantize)
    return {"value": round(sum(parts.values()), 2), "unit": "s per layer", "cores": cores,
            "kind": "port", "sample": "the whole of configs[0], nothing scaled",
            "parts_s": {k: round(v, 2) for k, v in parts.items()}}


def config1_gpu(dev, steps=3, warmup=1):
    """configs[0] on the HIP path: seconds per layer (workload_cfg1, mean of ``steps``)."""
    step, desc = workload_cfg1(dev, steps, warmup)

    def ev():
        return [torch.cuda.Event(enable_timing=True) for _ in range(4)]

    for _ in range(warmup):
        step(ev)
    torch.cuda.synchronize()
    with quiet_collector():
        t0 = time.perf_counter()
        for _ in range(steps):
            step(ev)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / steps
    return {"workload": desc, "sec_per_layer": round(wall, 4), "steps": steps, "warmup": warmup}


def kernel_rates(dev, acts, reps=10):
    """Standalone launches of the path's other kernels at the step's shapes,
    timed with HIP events on the launching stream (mean of ``reps``): the
    factor (2·C³/3 algorithmic flop), the compensation sweep of one 128-column
    block (20 bytes per weight: W read; Q, codes, scales and errors written),
    and the compensation's trailing tail product (2·R·N·K flop)."""
    from g2ptq_amd import GPTQ, _core, _lib
    stream = torch.cuda.current_stream()
    out = {}

    def timed(fn):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    for key, C in (("qkv", 4096), ("down", 14336)):
        lin = torch.nn.Linear(C, 64, bias=False, device=dev, dtype=torch.bfloat16)
        gq = GPTQ([lin])
        for t0 in range(0, 65536, 8192):
            gq.add_batch(0, acts[key][t0:t0 + 8192].view(-1, SEQ, C), None)
        H = gq.H.clone()
        _core.prepare_hessian(H, torch.zeros(1, 64, C, device=dev))
        U = torch.empty_like(H)
        info = torch.zeros(1, dtype=torch.int32, device=dev)
        ws = _lib.workspace(_lib.query_size("g2ptq_factor_workspace", 1, C), dev)
        ms = timed(lambda: _lib.call("g2ptq_inv_chol_upper", _core.stream(), _lib.ptr(H), 1, C,
                                     0.01, None, _lib.ptr(U), _lib.ptr(info), _lib.ptr(ws),
                                     ws.numel()))
        out[f"factor_C{C}"] = {"ms": round(ms, 3),
                               "tflops": round(2 * C ** 3 / 3 / (ms / 1e3) / 1e12, 1)}
        R = 4096
        W = torch.randn(1, R, C, device=dev) * 0.02
        # one 128-column block in the reference's transposed block layout
        wt = W[:, :, :128].transpose(1, 2).contiguous()
        hinv = U[:, :128, :128].contiguous()
        sc = torch.full_like(wt, 0.01)
        zr = torch.zeros_like(wt)
        it, et = torch.empty_like(wt), torch.empty_like(wt)
        w_keep = wt.clone()

        def sweep():
            wt.copy_(w_keep)
            _lib.call("g2ptq_block_sweep", _core.stream(), 0, 1, 128, R, 7, _lib.ptr(wt),
                      _lib.ptr(hinv), None, _lib.ptr(sc), _lib.ptr(zr), None, None, None,
                      _lib.ptr(it), _lib.ptr(et), None)
        copy_ms = timed(lambda: wt.copy_(w_keep))
        ms = timed(sweep) - copy_ms
        nbytes = R * 128 * 20
        out[f"sweep_R{R}_C{C}"] = {"us_per_block": round(ms * 1e3, 1),
                                   "GBps": round(nbytes / (ms / 1e3) / 1e9, 1),
                                   "frac_hbm": round(nbytes / (ms / 1e3) / 8e12, 4)}
        K, N = 512, C - 512
        E = torch.randn(1, R, K, device=dev) * 1e-3
        Wt = torch.randn(1, R, C, device=dev)
        ms = timed(lambda: _lib.call(
            "g2ptq_gemm_f32", _core.stream(), R, N, K, 1, _lib.ptr(E), K, R * K,
            _lib.ptr(U[0, :K, K:]), C, C * C, 0, _lib.ptr(Wt[0, :, K:]), C, R * C,
            _lib.ptr(Wt[0, :, K:]), C, R * C, -1.0, 1.0))
        out[f"tail_gemm_R{R}_N{N}_K{K}"] = {"ms": round(ms, 3),
                                            "tflops": round(2 * R * N * K / (ms / 1e3) / 1e12, 1)}
        del gq, H, U, W, Wt
    torch.cuda.empty_cache()
    return out


def g2ptq_block(dev, steps=2, warmup=1):
    """Config 3 (the north-star workload with G2PTQ compensation) in the default
    run: seconds per block and per stage over ``steps`` timed steps."""
    step, desc = workload_cfg3(dev, steps, warmup)

    def ev():
        return [torch.cuda.Event(enable_timing=True) for _ in range(4)]

    for _ in range(warmup):
        step(ev)
    torch.cuda.synchronize()
    with quiet_collector():
        t0 = time.perf_counter()
        recs = [step(ev) for _ in range(steps)]
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / steps
    h = sum(e[0].elapsed_time(e[1]) for e, _ in recs) / steps
    qz = sum(e[2].elapsed_time(e[3]) for e, _ in recs) / steps
    return {"workload": desc, "sec_per_block": round(wall, 4), "steps": steps, "warmup": warmup,
            "stages_ms": {"hessian": round(h, 2), "factor_and_compensation": round(qz, 2)},
            "hessian_tflops": round(recs[0][1] / (h / 1e3) / 1e12, 1),
            "hessian_flop_convention": "2*N*C^2 per (linear, row group) weighted Hessian"}


def traffic_per_launch():
    """HBM bytes per Gram launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by its reading for a plain copy of
    known size), or None when no such summary is present."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "gram256_config2_pmc_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return json.loads(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the quantization path on one GPU; --gpus must be 1",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    from g2ptq_amd import _lib
    _lib.load()
    if args.workload != "cfg2":
        run_other(args, dev)
        return
    acts, layers, w0 = make_inputs(dev, args.tokens)
    torch.cuda.synchronize()
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # reads 1 GiB, writes 1 GiB
        torch.cuda.synchronize()
        del src, dst

    def ev():
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    from g2ptq_amd import _stage
    for _ in range(args.warmup):
        run_step(acts, layers, w0, args.tokens, ev)
    torch.cuda.synchronize()
    hess, quant = [], []
    _stage.TIMING = []  # HIP events around every Gram launch of the timed steps
    with quiet_collector():
        t0 = time.perf_counter()
        for _ in range(args.steps):
            h, q = run_step(acts, layers, w0, args.tokens, ev)
            hess.append(h)
            quant.append(q)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
    grams, _stage.TIMING = _stage.TIMING, None
    hflops = hessian_flops(args.tokens)
    h_avg = sum(hess) / len(hess) / 1e3
    stage_rate = hflops / h_avg
    g_ms = [e0.elapsed_time(e1) for e0, e1, _, _, _ in grams]
    g_flops = sum(f for _, _, f, _, _ in grams)
    achieved = g_flops / (sum(g_ms) / 1e3)
    shapes = {}
    for (_, _, f, k, c), ms in zip(grams, g_ms):
        d = shapes.setdefault(f"C{c}_K{k}", [0, 0.0])
        d[0] += 1
        d[1] += ms
    out = {
        "metric": METRIC,
        "value": round(wall, 4),
        "unit": "s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16/fp32",
        "data": "synthetic (seeded GPU RNG, random-init weights, resident in HBM)",
        "config": {"workload": "llama3-8b-block GPTQ W4 sym g128, 262144 tokens, bs128, "
                               "groups {q},{k,v},{o},{gate,up},{down}",
                   "tokens": args.tokens, "calib_batch_tokens": BSZ * SEQ},
        "hessian_tflops": round(stage_rate / 1e12, 1),
        "stages_ms": {"hessian": round(h_avg * 1e3, 2),
                      "factor_and_compensation": round(sum(quant) / len(quant), 2)},
        "roofline": {"bound": "mfma",
                     "kernel": "gram256_kernel via g2ptq_hessian_gram (bf16 MFMA Gram of the "
                               "staged tokens; one launch per flush)",
                     "achieved": round(achieved / 1e12, 2), "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16, 4),
                     "traffic": traffic_per_launch(),
                     "work_per_launch": "2*K*C^2 flop (K staged tokens, C features)",
                     "launches_per_step": len(grams) // max(1, args.steps),
                     "avg_launch_ms": round(sum(g_ms) / max(1, len(g_ms)), 4),
                     "launches": {k: {"n": v[0] // max(1, args.steps),
                                      "avg_ms": round(v[1] / v[0], 4)}
                                  for k, v in sorted(shapes.items())}},
        "cpu_baseline": None,
    }
    if not args.no_kernel_rates:
        out["kernels"] = kernel_rates(dev, acts)
    if not args.no_unchanged_driver:
        out["unchanged_driver"] = unchanged_driver(acts, layers, w0, args.tokens)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(acts, w0, dev)
    if not args.no_g2ptq:
        del acts, layers, w0
        torch.cuda.empty_cache()
        out["g2ptq_block"] = g2ptq_block(dev)
    if not args.no_config1:
        out["config1"] = config1_gpu(dev)
    if out["cpu_baseline"] and "config1" in out:
        out["config1"]["cpu_over_gpu"] = round(
            out["cpu_baseline"]["config1"]["value"] / out["config1"]["sec_per_layer"], 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
