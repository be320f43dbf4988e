"""Parity harness: run the HIP sampler through its C ABI and compare with the oracle.

The comparison bar (per sampled row, every row checked):
  * greedy rows: ids bit-exact, no exemption;
  * the top-k threshold (scaled logit of the k-th largest) bit-exact;
  * the kept-token count equal to the oracle's, or, on a row whose top-p prefix
    sum comes within 1e-6 of top_p, to the count of one of the row's admissible
    cuts (``OracleResult.alt_kept``); that alternative then fixes the rest:
  * the token id among that alternative's allowed ids: its own pick, plus, where
    the uniform lies within 1e-6 of one of its cumulative-mass boundaries, the
    kept tokens whose float64 CDF interval lies within 1e-6 of the uniform;
  * final probabilities within 1e-5 relative (plus a 1e-12 absolute floor) of
    that alternative's, every token of every sampled row.
When neither the kept count nor the probabilities are known (an ids-only
call), the id must be among the union of the alternatives' allowed ids.
"""
from __future__ import annotations

import numpy as np
import torch

from conftest import pkg

W = pkg("workloads")
L = pkg("_lib")
S = pkg("sampler")
C = pkg("config")

# kernel modes under test: path name -> (workspace, mode).  "shipped" is what
# Sampler.sample launches: AUTO mode, the cached workspace and the row-kind hint
# of the call's parameters.  "topk" is per-row mode declared to hold only small-k
# rows: every call takes the kernel that requests each row at entry, and rows of
# other kinds (greedy, top-k off, penalties below 1) its fallback to the general
# per-row code (the hint never changes a result).  "split" is segmented mode declared
# to hold only small-k rows: calls of up to 64 rows take the split-row kernel (each row
# over several workgroups, merged by the last to arrive), and rows of other kinds its
# fallback to the general per-row code.
PATHS = {"segmented": ("auto", L.NS_MODE_SEGMENTED), "per-row": (None, L.NS_MODE_PER_ROW),
         "shipped": ("auto", L.NS_MODE_AUTO), "topk": (None, L.NS_MODE_PER_ROW),
         "split": ("auto", L.NS_MODE_SEGMENTED)}


def path_kinds(path):
    """The row_kinds argument run_gpu takes for the named path."""
    return "hint" if path == "shipped" else (L.NS_KIND_SMALL_K if path in ("topk", "split") else 0)

PROB_RTOL = 1e-5
PROB_ATOL = 1e-12


def params_of(w):
    return [C.SamplingParams(temperature=float(w.temperature[i]), top_k=int(w.top_k[i]), top_p=float(w.top_p[i]),
                             repetition_penalty=float(w.repetition_penalty[i])) for i in range(w.batch)]


def run_path(w, device, path, **kw):
    """run_gpu with the workspace, mode and row-kind hint of the named PATHS entry."""
    ws, mode = PATHS[path]
    return run_gpu(w, device, workspace=ws, mode=mode, row_kinds=path_kinds(path), **kw)


def run_gpu(w, device, logits=None, want_probs=True, uniforms=None, workspace="auto", mode=None, row_kinds=0,
            penalty_rounding="division"):
    """One ns_sample call over workload ``w``; returns ids, probs (CPU) and info words.

    ``mode``: NS_MODE_SEGMENTED (greedy and small-k rows split over several
    workgroups, the per-row kernel for the rest), NS_MODE_PER_ROW (one workgroup
    per row), or NS_MODE_AUTO (the default: chosen from the batch size).
    ``row_kinds``: the NS_KIND_* hint, or "hint" for the one PackedRows derives
    from the parameters (as Sampler.sample passes it).  ``penalty_rounding``:
    "division" or "reciprocal" (the oracle's option of the same name).
    """
    packed = S.PackedRows(params_of(w), w.histories, w.vocab, penalty_rounding=penalty_rounding)
    if isinstance(row_kinds, str):
        row_kinds = packed.row_kinds
    d = packed.to_device(device)
    if logits is None:
        logits = w.device_logits(device)
    B, V = w.batch, w.vocab
    u = torch.from_numpy(np.asarray(w.uniforms if uniforms is None else uniforms, dtype=np.float32)).to(device)
    sidx = torch.from_numpy(w.sample_indices).to(device) if w.sample_indices is not None else None
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    probs = torch.zeros((B, V), dtype=torch.float32, device=device) if want_probs else None
    info = torch.zeros((B, L.NS_INFO_WORDS), dtype=torch.int32, device=device)
    L.sample_raw(logits, d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"], u, out,
                 sample_idx=sidx, hist_offsets=d["hist_offsets"], hist_ids=d["hist_ids"],
                 max_hist=packed.max_hist, out_probs=probs, out_info=info, workspace=workspace,
                 mode=L.NS_MODE_AUTO if mode is None else mode, row_kinds=int(row_kinds),
                 penalty_rounding=packed.penalty_rounding, rep_penalty_recip=d["rep_penalty_recip"])
    torch.cuda.synchronize()
    return {"ids": out.cpu().numpy(), "probs": None if probs is None else probs.cpu(),
            "info": info.cpu().numpy()}


def f32_bits(x) -> int:
    return int(np.asarray(x, dtype=np.float32).view(np.int32))


def gpu_kept(g, i):
    """The kept-token count of GPU row ``i``: its diagnostics word, else its nonzero probabilities."""
    if g.get("info") is not None:
        return int(g["info"][i][1])
    if g.get("probs") is not None:
        return int((g["probs"][i] > 0).sum())
    return None


def compare(g, r, check_probs: bool = True, max_report: int = 8):
    """Return (failures, stats) comparing GPU output ``g`` with OracleResult ``r``."""
    B = len(r.ids)
    fails = []
    stats = {"rows": B, "exempt": 0, "draw_boundary": 0, "topp_boundary": 0, "zone_rows": 0, "alt_cut_rows": 0,
             "greedy": int(r.greedy.sum()), "id_equal": 0, "max_allowed": 0, "max_prob_rel": 0.0}
    for i in range(B):
        gi, ri = int(g["ids"][i]), int(r.ids[i])
        info = g["info"][i] if g.get("info") is not None else None
        where = f"path {info[0]}, flags {info[5]}" if info is not None else "sampler"
        greedy = bool(r.greedy[i])
        if gi == ri:
            stats["id_equal"] += 1
        if greedy:
            if gi != ri:
                fails.append(f"row {i}: greedy id {gi} != oracle {ri} ({where})")
            continue
        stats["draw_boundary"] += int(bool(r.draw_boundary[i]))
        stats["topp_boundary"] += int(bool(r.topp_boundary[i]))
        stats["zone_rows"] += int(len(r.alt_kept[i]) > 1)
        po, allowed = r.probs[i], r.allowed_ids[i]
        kept = None if r.nan_row[i] else gpu_kept(g, i)
        if kept is not None:
            alt = r.alternative(i, kept)
            if alt is None:
                fails.append(f"row {i}: kept {kept} not among the admissible counts {r.alt_kept[i].tolist()} "
                             f"({where})")
                po = None
            else:
                po, allowed = alt
                stats["alt_cut_rows"] += int(kept != int(r.n_kept[i]))
        stats["max_allowed"] = max(stats["max_allowed"], len(allowed))
        stats["exempt"] += int(len(allowed) > 1)
        if gi not in allowed:
            fails.append(f"row {i}: id {gi} not among the allowed ids {allowed[:8].tolist()} (oracle {ri}, {where})")
        if info is not None and not r.nan_row[i]:
            if not np.isnan(r.topk_thr[i]) and int(info[2]) != f32_bits(r.topk_thr[i]):
                g_thr = np.int32(info[2]).view(np.float32)
                fails.append(f"row {i}: top-k threshold {g_thr!r} != oracle {r.topk_thr[i]!r} (path {info[0]})")
        if check_probs and g.get("probs") is not None and po is not None:
            pg = g["probs"][i].double()
            po = po.double()
            diff = (pg - po).abs()
            tol = PROB_RTOL * torch.maximum(pg.abs(), po.abs()) + PROB_ATOL
            bad = diff > tol
            rel = (diff / torch.clamp(po.abs(), min=1e-30))[po > 1e-9]
            if rel.numel():
                stats["max_prob_rel"] = max(stats["max_prob_rel"], float(rel.max()))
            if bool(bad.any()):
                j = int(torch.nonzero(bad)[0, 0])
                fails.append(f"row {i}: prob[{j}] {float(pg[j])!r} vs oracle {float(po[j])!r} "
                             f"({int(bad.sum())} tokens off, {where})")
    if len(fails) > max_report:
        fails = fails[:max_report] + [f"... {len(fails) - max_report} more"]
    return fails, stats
