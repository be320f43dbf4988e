"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle.

Seeded inputs, oracle on the same inputs; the comparison bar is described in
tests/parity.py.  Full-size configurations run at their real shapes; the
oracle finishes each in a few seconds.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import compare, run_gpu

W = pkg("workloads")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu


def _check(w, device, **kw):
    print(f"[parity] {w.name} B={w.batch} V={w.vocab} dtype={w.dtype}", flush=True)
    g = run_gpu(w, device, **kw)
    r = O.sample_workload(w)
    fails, stats = compare(g, r)
    print(f"[parity] {w.name}: {stats}", flush=True)
    assert not fails, "\n".join(fails)
    return g, r, stats


@pytest.mark.parametrize("cfg", [0, 2])
def test_config_topk_rows(device, cfg):
    _check(W.make_workload(cfg), device)


@pytest.mark.parametrize("cfg", [1, 4])
def test_config_mixed_rows(device, cfg):
    _check(W.make_workload(cfg), device)


def test_config_long_nucleus(device):
    _check(W.make_workload(3, batch=32), device)


def test_run_twice_identical(device):
    w = W.make_workload(1, batch=16)
    a = run_gpu(w, device)
    b = run_gpu(w, device)
    assert np.array_equal(a["ids"], b["ids"])
    assert torch.equal(a["probs"], b["probs"])
    assert np.array_equal(a["info"], b["info"])
