"""The HIP sampler against the committed golden fixtures (GPU).

Tiny hand-built rows (ties, special values, penalties < 1 and > 1, temperature
and top-p edge cases; full inputs in tests/golden/tiny_cases.json) and the
c0-c4 workloads and a mixed bf16 decode batch (regenerated from their seeds,
confirmed by digest), in every launch set: greedy ids exact, top-k thresholds
bit-exact, the kept count one of the row's admissible top-p cuts (the oracle's
own unless its prefix sum comes within 1e-6 of top_p), the token id among that
cut's allowed ids (its pick alone unless the uniform lies within 1e-6 of one of
its cumulative-mass boundaries), and for the tiny rows the final probabilities
of that cut within 1e-5 relative.
"""
import numpy as np
import pytest
import torch

import golden_data as G
from parity import L, PATHS, run_gpu, run_path

pytestmark = pytest.mark.gpu

CONFIGS = G.configs()
TINY = G.tiny()
PROB_RTOL = 1e-5


def _check_rows(name, g, expected, probs=None):
    """The comparison of tests/parity.py against fixture records instead of an oracle run."""
    fails = []
    for i, e in enumerate(expected):
        info = g["info"][i]
        gid = int(g["ids"][i])
        if e["greedy"]:
            if gid != e["id"]:
                fails.append(f"{name} row {i}: greedy id {gid} != {e['id']} (path {info[0]})")
            continue
        allowed, j = e["allowed"], None
        if not e["nan_row"]:
            if e["thr_bits"] is not None and int(np.uint32(info[2])) != e["thr_bits"]:
                fails.append(f"{name} row {i}: threshold bits {int(np.uint32(info[2])):#x} != {e['thr_bits']:#x}")
            if int(info[1]) not in e["alt_kept"]:
                fails.append(f"{name} row {i}: kept {int(info[1])} not among {e['alt_kept']}")
            else:
                j = e["alt_kept"].index(int(info[1]))
                allowed = e["alt_allowed"][j]
        if gid not in allowed:
            fails.append(f"{name} row {i}: id {gid} not among the allowed ids {allowed[:8]} (oracle {e['id']}, "
                         f"path {info[0]})")
        if probs is not None and (j is not None or e["nan_row"]):
            bits = e["alt_probs_bits"][j if j is not None else 0]
            po = torch.from_numpy(np.asarray(bits, dtype=np.uint32).view(np.float32).copy()).double()
            pg = probs[i].double()
            diff = (pg - po).abs()
            tol = PROB_RTOL * torch.maximum(pg.abs(), po.abs()) + 1e-12
            bad = (diff > tol).nonzero().flatten()
            if bad.numel() > 0:
                k = int(bad[0])
                fails.append(f"{name} row {i}: prob[{k}] {float(pg[k])!r} vs {float(po[k])!r} ({bad.numel()} off)")
    return fails


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("case", TINY, ids=[c["name"] for c in TINY])
def test_tiny_cases(case, path, device):
    w = G.tiny_workload(case)
    print(f"[golden] tiny {case['name']} V={w.vocab} rows={w.batch} path={path}", flush=True)
    g = run_path(w, device, path)
    fails = _check_rows(case["name"], g, case["expected"], probs=g["probs"])
    assert not fails, "\n".join(fails[:12])


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_config_fixture(name, path, device):
    rec = CONFIGS[name]
    w = G.config_workload(rec)
    assert w.digest() == rec["digest"], f"{name}: workload regenerated differently on this machine"
    print(f"[golden] {name} B={w.batch} V={w.vocab} dtype={w.dtype} path={path}", flush=True)
    g = run_path(w, device, path, want_probs=False)
    fails = _check_rows(name, g, rec["rows"])
    assert not fails, "\n".join(fails[:12])


def test_shared_workspace_across_shapes(device):
    """One cached workspace serves segmented calls of changing batch size, vocabulary and
    dtype in a row: the arrival counters persist between calls at fixed positions, so a
    change of shape never leaves a row unfinalised or finalised early."""
    ws, mode = PATHS["segmented"]
    tiny = {c["name"]: c for c in TINY}
    seq = [("tiny", "special"), ("cfg", "c4"), ("tiny", "coarse"), ("cfg", "c0"), ("cfg", "c2"), ("tiny", "ties"),
           ("cfg", "c1"), ("cfg", "c4")]
    for kind, name in seq:
        if kind == "tiny":
            w, expected = G.tiny_workload(tiny[name]), tiny[name]["expected"]
        else:
            rec = CONFIGS[name]
            w, expected = G.config_workload(rec), rec["rows"]
        print(f"[golden] shared workspace: {w.name} B={w.batch} V={w.vocab} {w.dtype}", flush=True)
        g = run_gpu(w, device, want_probs=False, workspace=ws, mode=mode)
        fails = _check_rows(w.name, g, expected)
        assert not fails, "\n".join(fails[:12])
