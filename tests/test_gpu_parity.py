"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle.

Seeded inputs, oracle on the same inputs; the comparison bar is described in
tests/parity.py (every row checked: ids among the oracle's allowed ids, which
is the oracle's pick itself on every row without a boundary within 1e-6 of
its uniform).  Full-size configurations run at their real shapes, in three
launch sets: segmented, per-row, and the one Sampler.sample ships (AUTO mode
with the row-kind hint).  The oracle finishes each in a few seconds.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import PATHS, compare, params_of, run_path

W = pkg("workloads")
S = pkg("sampler")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu

L = pkg("_lib")

_ORACLE = {}


def _oracle(w, rounding="division"):
    key = (w.name, w.batch, rounding)
    if key not in _ORACLE:
        _ORACLE[key] = O.sample_workload(w, penalty_rounding=rounding)
    return _ORACLE[key]


def _check(w, device, path="segmented", rounding="division", **kw):
    print(f"[parity] {w.name} B={w.batch} V={w.vocab} dtype={w.dtype} path={path} penalty={rounding}", flush=True)
    g = run_path(w, device, path, penalty_rounding=rounding, **kw)
    r = _oracle(w, rounding)
    fails, stats = compare(g, r)
    stats["paths"] = {int(c): int((g["info"][:, 0] == c).sum()) for c in np.unique(g["info"][:, 0])}
    print(f"[parity] {w.name} {path}: {stats}", flush=True)
    assert not fails, "\n".join(fails)
    return g, r, stats


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("cfg", [0, 2])
def test_config_topk_rows(device, cfg, path):
    g, r, stats = _check(W.make_workload(cfg), device, path)
    if cfg == 2 or path in ("segmented", "shipped", "split"):
        assert stats["paths"].get(6, 0) == len(r.ids)   # every row finalised inside one wave


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("cfg", [1, 4])
def test_config_mixed_rows(device, cfg, path):
    g, r, _ = _check(W.make_workload(cfg), device, path)
    # greedy rows report no flags: these workloads hold no invalid history id or row
    assert not g["info"][r.greedy, 5].any(), g["info"][r.greedy, 5]


@pytest.mark.parametrize("path", list(PATHS))
def test_config_long_nucleus(device, path):
    """c3 at its full 128 rows x 256000 tokens (top-p 0.99 over heavy-tailed logits)."""
    _check(W.make_workload(3), device, path)


@pytest.mark.parametrize("path", list(PATHS))
def test_mixed_bf16_decode_batch(device, path):
    """bf16 rows at a decode batch of 256 with mixed parameters: in the shipped launch
    set the wide rows (top-k off or k > 64) go to wide_stats_kernel and the rest to
    the one-workgroup-per-row kernel."""
    _check(W.make_mixed_decode(256), device, path)


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("cfg", [0, 1, 2, 4, "mixed"])
def test_penalty_reciprocal_rounding(device, cfg, path):
    """NS_PENALTY_RECIPROCAL: the penalty's positive branch as torch computes it on a GPU, the
    reference's default device (x * fl32(1 / p)), against the oracle in the same mode."""
    w = W.make_mixed_decode(256) if cfg == "mixed" else W.make_workload(cfg)
    _check(w, device, path, rounding="reciprocal")


@pytest.mark.parametrize("path", list(PATHS))
def test_run_twice_identical(device, path):
    w = W.make_workload(1, batch=16)
    a = run_path(w, device, path)
    b = run_path(w, device, path)
    assert np.array_equal(a["ids"], b["ids"])
    assert torch.equal(a["probs"], b["probs"])
    assert np.array_equal(a["info"], b["info"])


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4])
def test_sampler_surface(device, cfg):
    """Sampler.sample() itself, called as the engine would (positional params and
    histories, sample_indices for the flat c4 layout, the workload's uniforms),
    against the oracle: ids and the returned probabilities."""
    w = W.make_workload(cfg)
    print(f"[parity] Sampler.sample {w.name} B={w.batch} V={w.vocab} dtype={w.dtype}", flush=True)
    logits = w.device_logits(device)
    hist = [h.tolist() for h in w.histories]
    sidx = torch.from_numpy(w.sample_indices).to(device) if w.sample_indices is not None else None
    u = torch.from_numpy(w.uniforms).to(device)
    sampler = S.Sampler(device)
    ids, probs = sampler.sample(logits, params_of(w), hist, sample_indices=sidx, uniforms=u, return_probs=True)
    ids_only = sampler.sample(logits, params_of(w), hist, sample_indices=sidx, uniforms=u)
    torch.cuda.synchronize()
    assert ids.dtype == torch.int64 and ids.device == logits.device and tuple(ids.shape) == (w.batch,)
    g = {"ids": ids.cpu().numpy(), "probs": probs.cpu(), "info": None}
    r = _oracle(w)
    fails, stats = compare(g, r)
    print(f"[parity] Sampler.sample {w.name}: {stats}", flush=True)
    assert not fails, "\n".join(fails)
    # the call without debug probabilities launches the same kernels minus the probability writes
    assert np.array_equal(ids_only.cpu().numpy(), g["ids"])
