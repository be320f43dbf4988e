"""GPU: the engine's sampling contract over many steps (integration tier).

A small restatement of the scheduler's batching drives ``Sampler.sample`` the way
the engine loop does (nanoserve/engine/engine.py:230-254):

* continuous batching as scheduler.py:100-150 and :152-246 build it: at most 64
  running requests, decodes take one token each, prefilling requests take
  chunks of at most 512 prompt tokens under a budget of 2048 tokens per step
  (config.py:49-53), waiting requests are admitted while the budget lasts; and
  the same at the size of the chunked-prefill benchmark batch (256 decoding
  requests and prefill chunks under a 4096-token budget, about 270 sampled rows
  of a 4096-row flat tensor per step);
* one flat (tokens, V) float32 logits tensor per step and ``sample_indices`` =
  ``query_start_loc[i] + q_len_i - 1`` for every sequence whose chunk completes
  its prompt or that is decoding (scheduler.py:240-246), handed over as the
  scheduler's host list, so the gather is fused into the kernel;
* per-request ``SamplingParams`` mixed as in the batch-64 workload, histories
  on the device (``DeviceHistories``: the prompt copied when the request is
  admitted, each sampled id appended by the kernel that draws it), and the ids
  read through ``async_ids`` handles (engine.py:250's ``.tolist()``);
* ``update_with_sampled`` (scheduler.py:264-312): every batched request advances
  by its q_len, sampling requests append their id, and stop on an EOS id, a stop
  id or max_tokens; finished requests free their history slot and new ones take
  it.

Every step is checked against the oracle on the step's sampled logits rows with
the histories rebuilt on the host as prompt + output (engine.py:242-246): ids,
probabilities and kept counts, to tests/parity.py's bar.  The same steps are
run a second time through the reference's own call shape (the history lists
passed every step, synchronous ids) and must give the same id stream.
"""
from __future__ import annotations

from collections import deque

import numpy as np
import pytest
import torch

from conftest import pkg
from parity import compare

S = pkg("sampler")
C = pkg("config")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu

V = 128256
MAX_MODEL_LEN = 8192
EOS_IDS = {128001, 128009}   # Llama-3 end-of-text / end-of-turn
# the reference's scheduler limits (config.py:49-53), and a larger batch shaped like the
# chunked-prefill benchmark batch: 256 requests decoding from the first step, prefill chunks
# of waiting requests filling a 4096-token budget
CONFIGS = {
    "reference": dict(max_num_seqs=64, budget=2048, chunk=512, n_requests=96, prompt_max=1500, decoding=0,
                      steps=8),
    "chunked-prefill-batch": dict(max_num_seqs=320, budget=4096, chunk=512, n_requests=420, prompt_max=4096,
                                  decoding=256, steps=5),
}


class Req:
    def __init__(self, rid, prompt, params):
        self.rid = rid
        self.prompt = prompt
        self.params = params
        self.output: list = []
        self.computed = 0
        self.finished = False

    @property
    def prompt_done(self):
        return self.computed >= len(self.prompt)


def make_requests(seed, n, prompt_max):
    rng = np.random.default_rng(seed)
    reqs = []
    for i in range(n):
        L = int(rng.integers(1, prompt_max))
        prompt = rng.zipf(1.1, size=L)
        prompt = ((prompt - 1) % V).astype(np.int64).tolist()
        sp = C.SamplingParams(max_tokens=int(rng.integers(2, 9)),
                              temperature=float(rng.choice([0.0, 0.7, 1.0, 1.3])),
                              top_k=int(rng.choice([-1, 1, 20, 50, 1000])),
                              top_p=float(rng.choice([1.0, 0.95, 0.5])),
                              repetition_penalty=float(rng.choice([1.0, 1.2])),
                              stop_token_ids=[int(v) for v in rng.integers(0, V, size=2)])
        reqs.append(Req(f"req-{i}", prompt, sp))
    return reqs


def schedule(running, waiting, on_admit, cfg):
    """scheduler.py:100-150 and :152-246: the step's batch and its sample indices."""
    budget = max(cfg["budget"] - sum(1 for r in running if r.prompt_done), 0)
    chunk = {}
    for r in running:
        if not r.prompt_done:
            c = min(len(r.prompt) - r.computed, cfg["chunk"], budget)
            if c > 0:
                chunk[r.rid] = c
                budget -= c
    while waiting and len(running) < cfg["max_num_seqs"] and budget > 0:
        r = waiting.popleft()
        c = min(len(r.prompt), cfg["chunk"], budget)
        running.append(r)
        on_admit(r)
        chunk[r.rid] = c
        budget -= c
    batch, qlens, sample_indices, sampling = [], [], [], []
    start = 0
    for r in running:
        if r.prompt_done:
            q, samples = 1, True
        else:
            q = chunk.get(r.rid, 0)
            if q <= 0:
                continue
            samples = r.computed + q >= len(r.prompt)
        batch.append(r)
        qlens.append(q)
        if samples:
            sample_indices.append(start + q - 1)
            sampling.append(r)
        start += q
    return batch, qlens, sample_indices, sampling, start


def update_with_sampled(batch, qlens, sampling, ids, running):
    """scheduler.py:264-312: advance, append, stop conditions."""
    for r, q in zip(batch, qlens):
        r.computed += q
    finished = []
    for r, tok in zip(sampling, ids):
        r.output.append(int(tok))
        if not r.params.ignore_eos and tok in EOS_IDS:
            r.finished = True
        elif tok in r.params.stop_token_ids:
            r.finished = True
        elif len(r.output) >= r.params.max_tokens:
            r.finished = True
        elif len(r.prompt) + len(r.output) >= MAX_MODEL_LEN:
            r.finished = True
        if r.finished:
            finished.append(r)
    for r in finished:
        running.remove(r)
    return finished


def run_engine(device, cfg, fast: bool, check: bool):
    """cfg["steps"] engine steps; returns the id stream.  fast: device histories, async ids and
    the host sample-index list; otherwise the reference's call shape."""
    reqs = make_requests(4242, cfg["n_requests"], cfg["prompt_max"])
    sampler = S.Sampler(device)
    dh = S.DeviceHistories(device, cfg["max_num_seqs"], capacity=MAX_MODEL_LEN) if fast else None
    on_admit = (lambda r: dh.open(r.rid, r.prompt)) if fast else (lambda r: None)
    # requests already decoding: prompt computed and a first token sampled
    running = reqs[:cfg["decoding"]]
    for i, r in enumerate(running):
        r.computed = len(r.prompt)
        r.output = [(7919 * i) % V]
        if fast:
            dh.open(r.rid, r.prompt + r.output)
    waiting = deque(reqs[cfg["decoding"]:])
    gen = torch.Generator(device=device)
    gen.manual_seed(99)
    rng = np.random.default_rng(5)
    stream, sampled_steps, finished_total = [], 0, 0
    for step in range(cfg["steps"]):
        batch, qlens, sidx, sampling, ntok = schedule(running, waiting, on_admit, cfg)
        logits = torch.randn((ntok, V), generator=gen, device=device, dtype=torch.float32).mul_(2.5)
        ids = []
        if sidx:
            params = [r.params for r in sampling]
            u = torch.from_numpy(rng.random(len(sidx), dtype=np.float32)).to(device)
            hist = [r.prompt + r.output for r in sampling]      # engine.py:242-246
            print(f"[engine] step {step} fast={fast}: {len(batch)} seqs, {ntok} tokens, {len(sidx)} sampled, "
                  f"{sum(1 for r in sampling if len(r.output) == 0)} first tokens", flush=True)
            if fast:
                handle, probs = sampler.sample(logits, params, None, sample_indices=sidx, uniforms=u,
                                               device_histories=dh, history_requests=[r.rid for r in sampling],
                                               async_ids=True, return_probs=check)
                ids = handle.tolist()
            else:
                out = sampler.sample(logits, params, hist, sample_indices=torch.tensor(sidx, device=device),
                                     uniforms=u, return_probs=check)
                out, probs = out if check else (out, None)
                ids = out.tolist()
            if check:
                rows = logits[torch.tensor(sidx, device=device)].cpu().numpy()
                r = O.sample(rows, [p.temperature for p in params], [p.top_k for p in params],
                             [p.top_p for p in params], [p.repetition_penalty for p in params],
                             [np.asarray(h, dtype=np.int64) for h in hist], u.cpu().numpy())
                fails, stats = compare({"ids": np.asarray(ids), "probs": probs.cpu(), "info": None}, r)
                print(f"[engine] step {step}: {stats}", flush=True)
                assert not fails, f"step {step}:\n" + "\n".join(fails)
            sampled_steps += 1
        del logits
        stream.append(ids)
        finished = update_with_sampled(batch, qlens, sampling, ids, running)
        finished_total += len(finished)
        if fast:
            for r in finished:
                dh.close(r.rid)
            for r in running:     # the device lists are prompt + output, as the host rebuilds them
                assert dh.length(r.rid) == len(r.prompt) + len(r.output), r.rid
    if fast:
        torch.cuda.synchronize()
        assert int(dh.state.overflow.item()) == 0
    return stream, sampled_steps, finished_total


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_engine_loop_device_histories_async_ids(device, name):
    cfg = CONFIGS[name]
    fast, steps_fast, fin = run_engine(device, cfg, fast=True, check=True)
    assert steps_fast >= 4 and fin > 0
    slow, _, _ = run_engine(device, cfg, fast=False, check=False)
    assert fast == slow
