"""GPU: histories longer than 8192 ids (the reference's max_model_len, config.py:52) against
the oracle.

Every kernel streams a row's history ids into its LDS bitmap in batches, so the history
length is bounded only by NS_MAX_HISTORY (2^20 ids).  The general per-row code also keeps
the row's distinct history ids with their penalized values; up to 8192 of them fit in LDS,
more go to the row's region of the workspace (ns_sample_workspace_bytes with max_hist).
Shapes: 16384 ids per row (about 15,000 distinct over 128256 tokens, so the workspace
region is used), 40000 ids, and a history three times longer than a 20000-token vocabulary
(every token at least once, most many times), fp32 and bf16, with penalties above and
below 1 and 1 itself, greedy, small-k, large-k and top-k-off rows; in every launch set
(segmented, per-row with a workspace, shipped, the top-k kernel, the split-row kernel) and
from both history sources (CSR arrays and device-resident request slots).  Same bar as
tests/parity.py.  A call with such histories and no workspace is refused.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import compare, params_of

W = pkg("workloads")
L = pkg("_lib")
S = pkg("sampler")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu

# launch sets: (mode, row_kinds); every one with the cached workspace
SETS = {"segmented": (L.NS_MODE_SEGMENTED, 0), "per-row": (L.NS_MODE_PER_ROW, 0),
        "shipped": (L.NS_MODE_AUTO, "hint"), "topk": (L.NS_MODE_PER_ROW, L.NS_KIND_SMALL_K),
        "split": (L.NS_MODE_SEGMENTED, L.NS_KIND_SMALL_K)}

_ORACLE = {}


def long_workload(name, B, V, H, seed, bf16=False, small_k_only=False):
    rng = np.random.default_rng(seed)
    raw = (rng.standard_normal((B, V), dtype=np.float32) * 2.5).astype(np.float32)
    bits = W.f32_to_bf16_bits(raw) if bf16 else None
    vals = W.bf16_bits_to_f32(bits) if bf16 else raw
    t = np.array([0.0, 0.8, 1.0, 1.3, 0.6, 1.1])[np.arange(B) % 6]
    if small_k_only:
        t = np.where(t == 0.0, 0.9, t)
        k = np.array([50, 1, 64, 20])[np.arange(B) % 4]
    else:
        k = np.array([50, 0, 1000, 1, 64, 0])[np.arange(B) % 6]
    p = np.array([0.9, 0.95, 1.0, 0.6])[np.arange(B) % 4]
    pen = np.array([1.1, 0.7, 1.5, 1.0, 2.0])[np.arange(B) % 5]
    if small_k_only:
        pen = np.maximum(pen, 1.1)
    hists = [rng.integers(0, V, size=H, dtype=np.int64).astype(np.int32) for _ in range(B)]
    return W.Workload(name=name, vocab=V, rows=vals, bf16_bits=bits, temperature=t, top_k=k.astype(np.int64),
                      top_p=p, repetition_penalty=pen, histories=hists, uniforms=rng.random(B, dtype=np.float32),
                      n_rows_total=B)


def run(w, device, mode, row_kinds, source):
    B, V = w.batch, w.vocab
    H = max(len(h) for h in w.histories)
    extra = {}
    if source == "slots":
        dh = S.DeviceHistories(device, B + 1, capacity=H)
        for r in range(B):
            dh.open(r, w.histories[r])
        packed = S.PackedRows(params_of(w), None, V, slots=dh.slots(list(range(B))), slot_max_hist=H)
        extra["hist_state"] = dh.state
    else:
        packed = S.PackedRows(params_of(w), w.histories, V)
    assert packed.max_hist == H > L.NS_LDS_HISTORY
    if isinstance(row_kinds, str):
        row_kinds = packed.row_kinds
    d = packed.to_device(device)
    if source == "slots":
        extra["hist_slot"] = d["hist_slot"]
    else:
        extra["hist_offsets"], extra["hist_ids"] = d["hist_offsets"], d["hist_ids"]
    u = torch.from_numpy(np.asarray(w.uniforms, dtype=np.float32)).to(device)
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    probs = torch.zeros((B, V), dtype=torch.float32, device=device)
    info = torch.zeros((B, L.NS_INFO_WORDS), dtype=torch.int32, device=device)
    L.sample_raw(w.device_logits(device), d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"], u, out,
                 max_hist=packed.max_hist, out_probs=probs, out_info=info, workspace="auto", mode=mode,
                 row_kinds=int(row_kinds), **extra)
    torch.cuda.synchronize()
    return {"ids": out.cpu().numpy(), "probs": probs.cpu(), "info": info.cpu().numpy()}


def check(w, device, name):
    if w.name not in _ORACLE:
        _ORACLE[w.name] = O.sample_workload(w)
    r = _ORACLE[w.name]
    mode, kinds = SETS[name]
    for source in ("csr", "slots"):
        print(f"[long-hist] {w.name} B={w.batch} V={w.vocab} H={len(w.histories[0])} {name} {source}", flush=True)
        g = run(w, device, mode, kinds, source)
        fails, stats = compare(g, r)
        stats["paths"] = {int(c): int((g["info"][:, 0] == c).sum()) for c in np.unique(g["info"][:, 0])}
        print(f"[long-hist] {w.name} {name} {source}: {stats}", flush=True)
        assert not fails, "\n".join(fails)
        assert not (g["info"][:, 0] == 9).any(), "a row was reported as an error"
        assert not g["info"][r.greedy, 5].any(), g["info"][r.greedy, 5]


WORKLOADS = {
    "h16384-f32": lambda: long_workload("long-h16384-f32", 6, 128256, 16384, seed=1601),
    "h16384-bf16": lambda: long_workload("long-h16384-bf16", 6, 128256, 16384, seed=1602, bf16=True),
    "h40000-f32": lambda: long_workload("long-h40000-f32", 5, 128256, 40000, seed=1603),
    "h60000-v20000": lambda: long_workload("long-h60000-v20000", 6, 20000, 60000, seed=1604),
    "h16384-smallk": lambda: long_workload("long-h16384-smallk", 4, 128256, 16384, seed=1605, small_k_only=True),
}


@pytest.mark.parametrize("name", list(SETS))
@pytest.mark.parametrize("wl", list(WORKLOADS))
def test_long_histories(device, wl, name):
    check(WORKLOADS[wl](), device, name)


def test_long_history_needs_a_workspace(device):
    w = long_workload("long-nows", 2, 4096, 9000, seed=1606)
    packed = S.PackedRows(params_of(w), w.histories, w.vocab)
    d = packed.to_device(device)
    out = torch.zeros(2, dtype=torch.int64, device=device)
    with pytest.raises(L.SamplerLibraryError, match="needs a workspace"):
        L.sample_raw(w.device_logits(device), d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"],
                     torch.zeros(2, dtype=torch.float32, device=device), out, hist_offsets=d["hist_offsets"],
                     hist_ids=d["hist_ids"], max_hist=packed.max_hist, workspace=None, mode=L.NS_MODE_PER_ROW)
