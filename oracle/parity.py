"""Oracle: the end-to-end parity protocol (test infrastructure only).

The checker that ``tests/`` and ``__graft_entry__.smoke()`` apply to a complete
``fasterquant`` flow from calibration data, against the oracle flow of
``oracle.flows`` on the same inputs:

* integer codes bit-exact, except where a row's **first** differing code sits
  at a rounding tie: the oracle's value was within ``tol`` of k + 1/2 steps
  (``|frac(x/s) − 1/2| < tol``), or the group's zero point was within ``tol``
  of a rounding tie before its ``round`` (asymmetric min/max fits).  Two fp32
  computations that differ only in summation order can round such a value
  either way; everything after it in the row then legitimately differs (the
  quantization error is fed forward), so only first divergences are counted;
* first divergences at most ``max_first`` of all entries (1e-4 = 0.01 %);
* scales within ``rtol`` relative, zero points equal, and dequantized weights
  within ``rtol`` relative, on every entry of a row before its first
  divergence (the protocol of the reference's own backend test,
  tests/test_triton_compensation.py:46-47 and :90-104, applied from X);
* the layer reconstruction error tr(ΔW·H·ΔWᵀ) (= ‖WX − QX‖²·2/n) within
  ``recon_rtol`` of the oracle's.

Everything works in the compensation loop's column order: with act-order the
loop quantizes column ``perm[i]`` at step i, and a tie cascades in that order.
"""
import torch


def unpack_codes(packed, bits, cols):
    """compressed-tensors ``pack_to_int32`` words (rows, words) → int64 codes
    (rows, cols): field i of a word is column ``w·(32/bits) + i``, offset by
    2^(bits−1)."""
    pf = 32 // bits
    w = packed.detach().cpu().to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(pf, dtype=torch.int64) * bits
    f = (w.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)
    return f.reshape(w.shape[0], -1)[:, :cols] - (1 << (bits - 1))


def element_params(quantizers, rows, cols, groupsize, static_groups, perm=None, attr=None):
    """Per-entry (scale, zero[, attr]) of fitted group quantizers, (rows, cols)
    in loop column order.  Column i of the loop uses group i // g (dynamic
    groups), group perm[i] // g (static groups), or the one quantizer."""
    def get(q, name):
        v = getattr(q, name)
        return None if v is None else v.detach().reshape(rows, -1)[:, :1].cpu().float()

    if groupsize == -1:
        idx = [0] * cols
    elif static_groups and perm is not None:
        idx = [int(p) // groupsize for p in perm.tolist()]
    else:
        idx = [i // groupsize for i in range(cols)]
    out = []
    for name in ("scale", "zero") + ((attr,) if attr else ()):
        per = [get(q, name) for q in quantizers]
        if any(p is None for p in per):
            out.append(None)
            continue
        out.append(torch.cat([per[k] for k in idx], dim=1))
    return out


def stage_b(codes_hip, codes_ref, x_ref, scale_hip, scale_ref, zero_hip, zero_ref, q_ref,
            zraw_ref=None, tol=1e-4, rtol=1e-3):
    """Compare two flows' outputs, all (rows, cols) in loop column order.

    Returns a report dict; ``report["ok"]`` is False when a first divergence
    is not at a tie or a float bound fails (the reasons are listed)."""
    ch = codes_hip.reshape(-1, codes_hip.shape[-1]).cpu().double()
    cr = codes_ref.reshape(-1, codes_ref.shape[-1]).cpu().double()
    n, c = cr.shape
    x = x_ref.reshape(n, c).cpu().double()
    sh, sr = scale_hip.reshape(n, c).cpu().double(), scale_ref.reshape(n, c).cpu().double()
    zh, zr = zero_hip.reshape(n, c).cpu().double(), zero_ref.reshape(n, c).cpu().double()
    qr = q_ref.reshape(n, c).cpu().double()
    diff = ch != cr
    first = torch.full((n,), c, dtype=torch.int64)
    rows = diff.any(1)
    first[rows] = diff[rows].to(torch.int8).argmax(1)
    reasons = []
    ties = {"rounding": 0, "zero_point": 0}
    dist = []
    for r in rows.nonzero().flatten().tolist():
        j = int(first[r])
        t = float(x[r, j] / sr[r, j])
        dist.append(abs(t - float(torch.floor(torch.tensor(t))) - 0.5))
        if dist[-1] < tol:
            ties["rounding"] += 1
            continue
        if zraw_ref is not None and zh[r, j] != zr[r, j]:
            zt = float(zraw_ref.reshape(n, c)[r, j])
            if abs(zt - float(torch.floor(torch.tensor(zt))) - 0.5) < tol:
                ties["zero_point"] += 1
                continue
        reasons.append(f"row {r} first differs at loop column {j}: code {ch[r, j]:.0f} vs "
                       f"{cr[r, j]:.0f}, x/s = {t:.6f} is not a rounding tie")
    before = torch.arange(c).unsqueeze(0) < first.unsqueeze(1)
    s_rel = ((sh - sr).abs() / sr.abs().clamp_min(1e-30))[before]
    s_err = float(s_rel.max()) if s_rel.numel() else 0.0
    z_bad = int((zh != zr)[before].sum())
    qh = sh * (ch - zh)
    q_rel = ((qh - qr).abs() / qr.abs().clamp_min(1e-30))[before & (qr != 0)]
    q_err = float(q_rel.max()) if q_rel.numel() else 0.0
    q_zero_bad = int(((qh != 0) & (qr == 0))[before].sum())
    n_first = int(rows.sum())
    first_frac = n_first / (n * c)
    if s_err > rtol:
        reasons.append(f"scale relative error {s_err:.3g} > {rtol} before the first divergence")
    if z_bad:
        reasons.append(f"{z_bad} zero points differ before the first divergence")
    if q_err > rtol or q_zero_bad:
        reasons.append(f"dequantized relative error {q_err:.3g} (bound {rtol}), "
                       f"{q_zero_bad} nonzero where the oracle has 0")
    return {
        "ok": not reasons, "reasons": reasons, "entries": n * c, "rows": n,
        "rows_diverged": n_first, "first_divergence_frac": first_frac,
        "mismatch_frac": float(diff.double().mean()), "ties": ties,
        "scale_rel_err": s_err, "dequant_rel_err": q_err,
        "max_tie_distance": max(dist) if dist else 0.0,
    }


def check_stage_b(report, max_first=1e-4):
    """Raise AssertionError unless the report meets the bar (first divergences
    at ties only, at most ``max_first`` of all entries, floats in bound)."""
    reasons = list(report["reasons"])
    if report["first_divergence_frac"] > max_first:
        reasons.append(f"first divergences {report['first_divergence_frac']:.3g} of entries "
                       f"> {max_first}")
    if reasons:
        raise AssertionError("; ".join(reasons[:8]) + f" (report: {summary(report)})")


def summary(report):
    return (f"{report['rows_diverged']}/{report['rows']} rows diverge "
            f"(first divergences {100 * report['first_divergence_frac']:.4f} % of "
            f"{report['entries']} entries; ties {report['ties']}), "
            f"farthest from a tie {report.get('max_tie_distance', 0.0):.2g}, "
            f"{100 * report['mismatch_frac']:.3f} % codes differ in all, "
            f"scale err {report['scale_rel_err']:.2g}, dequant err {report['dequant_rel_err']:.2g}")


def loop_order(t, perm):
    """(…, C) in column order → loop order (``t[..., perm]``)."""
    return t if perm is None else t[..., perm]


def exported_codes(layers, bits, cols):
    """Integer codes of a flow run with ``export_compressed_tensors=True``:
    the layers' packed words unpacked, stacked (B·R, C) in column order."""
    return torch.cat([unpack_codes(l._export_qparams["weight_packed"], bits, cols)
                      for l in layers])


def check_flow(label, layers, quantizers, ref, W0, H, bits, groupsize, static_groups,
               max_first=1e-4, recon_rtol=0.005, check=True, tie_tol=1e-4):
    """The whole bar for a ``fasterquant`` run with
    ``export_compressed_tensors=True`` on ``layers`` (fitted ``quantizers``)
    against an oracle flow ``ref`` on the same inputs: the stage-B report,
    the written weights equal to the exported codes dequantized with the fitted
    fp32 scales and cast to the weight dtype, and the reconstruction error
    tr(ΔW·H·ΔWᵀ) within ``recon_rtol``.  ``H`` is (B, C, C), or (B·G, C, C)
    with one Hessian per row group.  Returns the report."""
    B = len(layers)
    R, C = layers[0].weight.shape
    N = B * R
    dtype = layers[0].weight.dtype
    perm = ref["perm"]
    ch = loop_order(exported_codes(layers, bits, C), perm)
    cr = loop_order(ref["W_int"].reshape(N, C), perm)
    x = ref["loop"]["X"].reshape(N, C)
    sh, zh = element_params(quantizers, N, C, groupsize, static_groups, perm)
    sr, zr, zraw = element_params(ref["quantizers"], N, C, groupsize, static_groups, perm,
                                  attr="zraw")
    qr = loop_order(ref["Q"].reshape(N, C), perm)
    rep = stage_b(ch, cr, x, sh, sr, zh, zr, qr, zraw_ref=zraw, tol=tie_tol)
    inv = None if perm is None else torch.argsort(perm)
    qh = loop_order(sh * (ch - zh).float(), inv).reshape(B, R, C)
    Qd = torch.stack([l.weight.detach().float().cpu() for l in layers])
    wb = int((Qd != qh.to(dtype).float()).sum())
    nb = H.shape[0]
    Qr = ref["Q"].reshape(B, R, C).to(dtype).float()
    e_hip = reconstruction_error(W0.reshape(nb, -1, C), Qd.reshape(nb, -1, C), H)
    e_ref = reconstruction_error(W0.reshape(nb, -1, C), Qr.reshape(nb, -1, C), H)
    rep["recon_hip"], rep["recon_ref"], rep["writeback_mismatch"] = e_hip, e_ref, wb
    print(f"{label}: {summary(rep)}; recon {e_hip:.6g} vs {e_ref:.6g} "
          f"({100 * (e_hip / e_ref - 1):+.3f} %)", flush=True)
    if check:
        if wb:
            raise AssertionError(f"{label}: {wb} written weights differ from the exported codes")
        if not abs(e_hip - e_ref) <= recon_rtol * e_ref:
            raise AssertionError(f"{label}: reconstruction error {e_hip} vs oracle {e_ref}")
        check_stage_b(rep, max_first)
    return rep


def reconstruction_error(W, Q, H):
    """‖WX − QX‖²·2/n = tr(ΔW·H·ΔWᵀ) summed over layers, H = (2/n)·XᵀX (fp64)."""
    d = W.double() - Q.double()
    return torch.einsum("brc,bcd,brd->", d, H.double(), d).item()
