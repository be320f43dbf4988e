"""GPU: device-resident histories (ns_hist_state_bytes / ns_hist_assign /
ns_hist_append, the ``DeviceHistories`` class).

Holding the same ids as the CSR histories, they must give bit-identical ids,
diagnostics and probabilities in every launch set (every kernel reads a row's
history through the same start/length pair).  Over a multi-step decode loop,
appending each sampled token on the device must track the host-side lists the
reference's engine rebuilds every step (engine.py:242-246,
scheduler.py:281-284), and every step's ids must meet the oracle run on that
step's logits, host histories and uniforms.  The append fused into the sampling
kernels (hist_append) must leave the same lists, ids, diagnostics and
probabilities as the call without it followed by ns_hist_append, in every
launch set, over two steps (the second reads the appended ids).
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import PATHS, compare, params_of, path_kinds, run_path

O = pytest.importorskip("oracle.sampler_oracle")

W = pkg("workloads")
L = pkg("_lib")
S = pkg("sampler")

pytestmark = pytest.mark.gpu


def open_all(w, device, extra_slots=3):
    dh = S.DeviceHistories(device, w.batch + extra_slots, capacity=L.NS_LDS_HISTORY)
    for r in range(w.batch):
        dh.open(r, w.histories[r])
    return dh


def run_slots(w, device, dh, workspace, mode, row_kinds=0, append=False, overflow=None):
    """run_gpu's call with the histories read from ``dh`` (request r on row r); with
    ``append`` the kernels also append each row's id to its slot."""
    slots = dh.slots(list(range(w.batch)))
    max_hist = int(max(dh.length(r) for r in range(w.batch)))
    packed = S.PackedRows(params_of(w), None, w.vocab, slots=slots, slot_max_hist=max_hist)
    if isinstance(row_kinds, str):
        row_kinds = packed.row_kinds
    d = packed.to_device(device)
    logits = w.device_logits(device)
    B, V = w.batch, w.vocab
    u = torch.from_numpy(np.asarray(w.uniforms, dtype=np.float32)).to(device)
    sidx = torch.from_numpy(w.sample_indices).to(device) if w.sample_indices is not None else None
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    probs = torch.zeros((B, V), dtype=torch.float32, device=device)
    info = torch.zeros((B, L.NS_INFO_WORDS), dtype=torch.int32, device=device)
    L.sample_raw(logits, d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"], u, out,
                 sample_idx=sidx, max_hist=packed.max_hist, out_probs=probs, out_info=info, workspace=workspace,
                 mode=mode, row_kinds=int(row_kinds), hist_state=dh.state, hist_slot=d["hist_slot"],
                 hist_append=append, hist_overflow=overflow)
    torch.cuda.synchronize()
    if append:
        dh._appended(slots)
    return {"ids": out.cpu().numpy(), "probs": probs.cpu(), "info": info.cpu().numpy()}


def read_state(dh, request_ids):
    """The id lists the device holds for these requests."""
    words = dh.state.buffer.view(torch.int32).cpu().numpy()
    lens = words[:dh.state.n_slots]
    base = (dh.state.n_slots * 4 + 255) // 256 * 64
    out = []
    for r in request_ids:
        s = dh.slots([r])[0]
        out.append(words[base + s * dh.state.capacity: base + s * dh.state.capacity + lens[s]].tolist())
    return out


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("cfg", [1, 2, 4])
def test_device_histories_match_csr(device, cfg, path):
    w = W.make_workload(cfg, batch=64 if cfg == 2 else None)
    print(f"[history] config {cfg} B={w.batch} path={path}", flush=True)
    ws, mode = PATHS[path]
    ref = run_path(w, device, path)
    dh = open_all(w, device)
    got = run_slots(w, device, dh, ws, mode, row_kinds=path_kinds(path))
    assert np.array_equal(got["ids"], ref["ids"])
    bad = np.nonzero((got["info"] != ref["info"]).any(axis=1))[0]
    assert bad.size == 0, [(int(i), ref["info"][i].tolist(), got["info"][i].tolist()) for i in bad[:4]]
    assert torch.equal(got["probs"], ref["probs"])


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_fused_append_matches_separate_append(device, cfg, path):
    w = W.make_workload(cfg, batch=64 if cfg == 2 else (48 if cfg == 3 else None))
    ws, mode = PATHS[path]
    sep, fused = open_all(w, device), open_all(w, device)
    reqs = list(range(w.batch))
    over = torch.zeros(1, dtype=torch.int32, device=device)
    for step in range(2):
        print(f"[history] fused append: config {cfg} B={w.batch} path={path} step {step}", flush=True)
        a = run_slots(w, device, sep, ws, mode, row_kinds=path_kinds(path))
        slots = torch.from_numpy(sep.slots(reqs)).to(device)
        sep.state.append(slots, torch.from_numpy(a["ids"]).to(device))
        sep._appended(sep.slots(reqs))
        b = run_slots(w, device, fused, ws, mode, row_kinds=path_kinds(path), append=True, overflow=over)
        assert np.array_equal(a["ids"], b["ids"]), f"step {step}: rows {np.nonzero(a['ids'] != b['ids'])[0][:8]}"
        bad = np.nonzero((a["info"] != b["info"]).any(axis=1))[0]
        assert bad.size == 0, [(int(i), a["info"][i].tolist(), b["info"][i].tolist()) for i in bad[:4]]
        assert torch.equal(a["probs"], b["probs"])
        torch.cuda.synchronize()
        assert read_state(fused, reqs) == read_state(sep, reqs)
        assert all(fused.length(r) == len(h) for r, h in zip(reqs, read_state(fused, reqs)))
    assert int(over.item()) == 0 and int(sep.state.overflow.item()) == 0


def test_fused_append_counts_full_slots(device):
    """A full slot keeps its ids and is counted; rows without a slot append nothing."""
    w = W.make_workload(1)
    B = w.batch
    cap = max(len(h) for h in w.histories)
    dh = S.DeviceHistories(device, B + 1, capacity=cap)
    for r in range(B):
        dh.open(r, w.histories[r] if r % 3 == 0 else w.histories[r][:cap - 20])
    full = [r for r in range(B) if dh.length(r) == cap]
    assert full and len(full) < B
    before = read_state(dh, list(range(B)))
    slots = dh.slots(list(range(B))).copy()
    slots[1] = -1
    if 1 in full:
        full.remove(1)
    packed = S.PackedRows(params_of(w), None, w.vocab, slots=slots, slot_max_hist=cap)
    d = packed.to_device(device)
    u = torch.from_numpy(np.asarray(w.uniforms, dtype=np.float32)).to(device)
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    over = torch.zeros(1, dtype=torch.int32, device=device)
    L.sample_raw(w.device_logits(device), d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"], u, out,
                 max_hist=cap, hist_state=dh.state, hist_slot=d["hist_slot"], hist_append=True, hist_overflow=over,
                 row_kinds=packed.row_kinds)
    torch.cuda.synchronize()
    ids = out.cpu().numpy()
    after = read_state(dh, list(range(B)))
    assert int(over.item()) == len(full)
    for r in range(B):
        want = before[r] if (r == 1 or r in full) else before[r] + [int(ids[r])]
        assert after[r] == want, r


def test_decode_loop_appends_on_device(device):
    """Four decode steps of the mixed batch: at every step the ids meet the oracle run on
    the step's logits with the host lists, the device-history call returns the same ids,
    and the device lists equal the host lists afterwards."""
    w = W.make_workload(1)
    B = w.batch
    params = params_of(w)
    base = w.device_logits(device)
    sampler = S.Sampler(device)
    host = [list(map(int, h)) for h in w.histories]
    dh = S.DeviceHistories(device, B + 5, capacity=1024)
    order = list(range(B))[::-1]                     # slots taken in a different order than rows
    for r in order:
        dh.open(r, host[r])
    rng = np.random.default_rng(77)
    for step in range(4):
        print(f"[history] decode step {step}", flush=True)
        logits = torch.roll(base, shifts=977 * (step + 1), dims=1).contiguous()
        u = torch.from_numpy(rng.random(B, dtype=np.float32)).to(device)
        ids_host = sampler.sample(logits, params, host, uniforms=u)
        ids_dev = sampler.sample(logits, params, None, uniforms=u, device_histories=dh,
                                 history_requests=list(range(B)))
        a, b = ids_host.cpu().numpy(), ids_dev.cpu().numpy()
        assert np.array_equal(a, b), f"step {step}: rows {np.nonzero(a != b)[0][:8]}"
        r = O.sample(logits.cpu().numpy(), w.temperature, w.top_k, w.top_p, w.repetition_penalty,
                     [np.asarray(h, dtype=np.int32) for h in host], u.cpu().numpy())
        fails, stats = compare({"ids": a, "probs": None, "info": None}, r)
        print(f"[history] step {step}: {stats}", flush=True)
        assert not fails, f"step {step}:\n" + "\n".join(fails)
        for r in range(B):
            host[r].append(int(a[r]))
    torch.cuda.synchronize()
    assert read_state(dh, list(range(B))) == host
    assert all(dh.length(r) == len(host[r]) for r in range(B))
    assert int(dh.state.overflow.item()) == 0
    # a freed slot is reused with the new request's prompt only
    dh.close(3)
    dh.open("new", [5, 6, 7])
    torch.cuda.synchronize()
    assert read_state(dh, ["new"]) == [[5, 6, 7]]


def test_full_slot_is_refused(device):
    dh = S.DeviceHistories(device, 2, capacity=4)
    dh.open("a", [1, 2, 3])
    slots = torch.tensor([dh.slots(["a"])[0]], dtype=torch.int32, device=device)
    dh.state.append(slots, torch.tensor([9], dtype=torch.int64, device=device))
    dh.state.append(slots, torch.tensor([8], dtype=torch.int64, device=device))   # full: not appended
    torch.cuda.synchronize()
    assert int(dh.state.overflow.item()) == 1
    words = dh.state.buffer.view(torch.int32).cpu().numpy()
    s = int(slots[0])
    assert words[s] == 4
    assert words[64 + s * 4: 64 + s * 4 + 4].tolist() == [1, 2, 3, 9]


def test_async_ids_match_and_overlap(device):
    """async_ids: the same ids as the synchronous call, readable later, several in flight."""
    w = W.make_workload(2, batch=64)
    params = params_of(w)
    sampler = S.Sampler(device)
    hist = [list(map(int, h)) for h in w.histories]
    u = torch.from_numpy(np.asarray(w.uniforms, dtype=np.float32)).to(device)
    base = w.device_logits(device)
    sync_ids, handles = [], []
    for step in range(6):
        logits = torch.roll(base, shifts=131 * step, dims=1).contiguous()
        sync_ids.append(sampler.sample(logits, params, hist, uniforms=u).cpu().tolist())
        handles.append(sampler.sample(logits, params, hist, uniforms=u, async_ids=True))
    for step, h in enumerate(handles):
        assert isinstance(h, S.SampledIds) and len(h) == w.batch
        assert h.tolist() == sync_ids[step]
        assert h.ready()
        assert h.tensor.cpu().tolist() == sync_ids[step]


def test_out_of_range_sample_index_is_refused_and_lengths_stay(device):
    """A sample index outside the logits is refused before any launch (the reference's
    index_select at engine.py:234 raises there), from a host list and from a device tensor with
    device histories, so the host lengths never count an append the kernel skipped."""
    w = W.make_workload(1, batch=8)
    params = params_of(w)
    sampler = S.Sampler(device)
    dh = S.DeviceHistories(device, 8, capacity=1024)
    for r in range(8):
        dh.open(r, list(map(int, w.histories[r])))
    before = [dh.length(r) for r in range(8)]
    logits = w.device_logits(device)
    u = torch.from_numpy(np.asarray(w.uniforms, dtype=np.float32)).to(device)
    bad = list(range(8))
    bad[5] = 8
    for sidx in (bad, torch.tensor(bad, device=device), [-1] + list(range(1, 8))):
        with pytest.raises(IndexError):
            sampler.sample(logits, params, None, sample_indices=sidx, uniforms=u, device_histories=dh,
                           history_requests=list(range(8)))
    assert [dh.length(r) for r in range(8)] == before
    torch.cuda.synchronize()
    assert read_state(dh, list(range(8))) == [list(map(int, h)) for h in w.histories]
    # a valid call afterwards appends once per row
    ids = sampler.sample(logits, params, None, sample_indices=list(range(8)), uniforms=u, device_histories=dh,
                         history_requests=list(range(8)))
    assert [dh.length(r) for r in range(8)] == [b + 1 for b in before]
    assert read_state(dh, list(range(8))) == [list(map(int, h)) + [int(i)] for h, i in zip(w.histories,
                                                                                          ids.tolist())]


def test_readback_ring_reuses_its_buffers(device):
    """async_ids through the ring: more handles in flight than the ring's depth, read late and
    out of order, all equal the synchronous ids; the ring holds depth buffers, no more."""
    w = W.make_workload(2, batch=32)
    params = params_of(w)
    sampler = S.Sampler(device)
    hist = [list(map(int, h)) for h in w.histories]
    base = w.device_logits(device)
    u = torch.from_numpy(np.asarray(w.uniforms, dtype=np.float32)).to(device)
    handles, want = [], []
    for step in range(11):
        logits = torch.roll(base, shifts=313 * step, dims=1).contiguous()
        want.append(sampler.sample(logits, params, hist, uniforms=u).tolist())
        handles.append(sampler.sample(logits, params, hist, uniforms=u, async_ids=True))
    ring = sampler._ring
    assert len(ring._slots) == ring.depth
    for step in [10, 3, 0, 7, 9, 1, 2, 4, 5, 6, 8]:
        assert handles[step].tolist() == want[step], step
        assert handles[step].ready()
