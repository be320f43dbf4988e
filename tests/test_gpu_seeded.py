"""GPU: seeded requests (SamplingParams.seed) draw reproducible uniforms.

ns_seeded_uniforms against the numpy restatement of Philox4x32-10 (oracle/philox.py, pinned
by the published known-answer vectors and rocRAND in tests/test_philox.py), bit for bit;
Sampler.sample with seeds: the same ids on every call, ids among the oracle's allowed ids
for the uniforms the seeds and history lengths give, and a fresh uniform once a decode
step has appended a token to a device-resident history.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import params_of

W = pkg("workloads")
L = pkg("_lib")
S = pkg("sampler")
O = pytest.importorskip("oracle.sampler_oracle")
from oracle import philox as P  # noqa: E402

pytestmark = pytest.mark.gpu


def test_kernel_matches_restatement(device):
    rng = np.random.default_rng(31)
    n = 1000
    seeds = [int(x) for x in rng.integers(0, 2 ** 63, size=n)]
    seeds[:4] = [0, -1, 2 ** 64 - 1, -(2 ** 40)]
    steps = [int(x) for x in rng.integers(0, 2 ** 40, size=n)]
    steps[:3] = [0, 1, 2 ** 33 + 7]
    rows = rng.permutation(n + 5)[:n].tolist()
    out = torch.full((n + 5,), -1.0, dtype=torch.float32, device=device)
    L.seeded_uniforms(seeds, steps, rows, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = P.seeded_uniform(seeds, steps)
    assert np.array_equal(got[rows].view(np.uint32), want.view(np.uint32))
    untouched = sorted(set(range(n + 5)) - set(rows))
    assert (got[untouched] == -1.0).all()


def _seeded_params(w, seeds):
    ps = params_of(w)
    for p, s in zip(ps, seeds):
        p.seed = s
    return ps


@pytest.mark.parametrize("cfg", [0, 1])
def test_seeded_sampling_is_reproducible_and_matches_oracle(device, cfg):
    w = W.make_workload(cfg, batch=16 if cfg == 1 else None)
    B = w.batch
    seeds = [1000 + 7 * i for i in range(B)]
    hist = [h.tolist() for h in w.histories]
    sampler = S.Sampler(device)
    logits = w.device_logits(device)
    a = sampler.sample(logits, _seeded_params(w, seeds), hist).cpu().numpy()
    b = sampler.sample(logits, _seeded_params(w, seeds), hist).cpu().numpy()
    assert np.array_equal(a, b)
    u = P.seeded_uniform(seeds, [len(h) for h in hist])
    r = O.sample(w.rows, w.temperature, w.top_k, w.top_p, w.repetition_penalty, w.histories, u)
    for i in range(B):
        assert a[i] in r.allowed_ids[i], (i, int(a[i]), int(r.ids[i]))


def test_seeded_rows_beside_unseeded_rows(device):
    """Half the rows seeded: those repeat across calls whatever the device RNG draws for the rest."""
    w = W.make_workload(0)
    B = w.batch
    seeds = [None if i % 2 else 77 + i for i in range(B)]
    hist = [h.tolist() for h in w.histories]
    sampler = S.Sampler(device)
    logits = w.device_logits(device)
    a = sampler.sample(logits, _seeded_params(w, seeds), hist).cpu().numpy()
    torch.rand(1000, device=device)   # move the global generator
    b = sampler.sample(logits, _seeded_params(w, seeds), hist).cpu().numpy()
    seeded = [i for i in range(B) if seeds[i] is not None]
    assert np.array_equal(a[seeded], b[seeded])
    u = P.seeded_uniform([seeds[i] for i in seeded], [len(hist[i]) for i in seeded])
    r = O.sample(w.rows[seeded], w.temperature[seeded], w.top_k[seeded], w.top_p[seeded],
                 w.repetition_penalty[seeded], [w.histories[i] for i in seeded], u)
    for j, i in enumerate(seeded):
        assert a[i] in r.allowed_ids[j]


def test_device_histories_advance_the_counter(device):
    """With device-resident histories the counter is the slot length: each decode step appends
    a token, so the next step's uniform is Philox at length + 1 (checked through the oracle)."""
    w = W.make_workload(0)
    B = w.batch
    seeds = [5 + i for i in range(B)]
    sampler = S.Sampler(device)
    dh = S.DeviceHistories(device, B, capacity=256)
    hist = [h.tolist() for h in w.histories]
    for i, h in enumerate(hist):
        dh.open(i, h)
    logits = w.device_logits(device)
    for step in range(3):
        ids = sampler.sample(logits, _seeded_params(w, seeds), None, device_histories=dh,
                             history_requests=list(range(B))).cpu().numpy()
        u = P.seeded_uniform(seeds, [len(h) for h in hist])
        r = O.sample(w.rows, w.temperature, w.top_k, w.top_p, w.repetition_penalty,
                     [np.asarray(h, dtype=np.int32) for h in hist], u)
        for i in range(B):
            assert ids[i] in r.allowed_ids[i], (step, i, int(ids[i]), int(r.ids[i]))
            hist[i].append(int(ids[i]))
