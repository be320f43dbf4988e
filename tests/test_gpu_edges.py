"""GPU: boundary shapes against the oracle -- the largest vocabulary and history the
ABI accepts, a one-token vocabulary, a bf16 vocabulary that is not a multiple of the
16-byte chunk read through a padded row stride, and an empty batch.  Same bar as
tests/parity.py (every id among the oracle's allowed ids, thresholds bit-exact,
probabilities within 1e-5 relative), in the segmented, per-row and shipped launch sets.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import PATHS, compare, path_kinds, run_gpu, run_path

W = pkg("workloads")
L = pkg("_lib")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu


def workload(name, B, V, seed, hist_len, bf16=False, scale=3.0):
    rng = np.random.default_rng(seed)
    raw = (rng.standard_normal((B, V), dtype=np.float32) * scale).astype(np.float32)
    bits = W.f32_to_bf16_bits(raw) if bf16 else None
    rows = W.bf16_bits_to_f32(bits) if bf16 else raw
    t = rng.choice(np.array([0.0, 0.7, 1.0, 1.3]), size=B)
    k = rng.choice(np.array([0, 1, 50, 1000]), size=B).astype(np.int64)
    p = rng.choice(np.array([1.0, 0.95, 0.5]), size=B)
    pen = rng.choice(np.array([1.0, 0.8, 1.3]), size=B)
    hist = [rng.integers(0, V, size=min(hist_len, 10 ** 9), dtype=np.int64).astype(np.int32) for _ in range(B)]
    u = rng.random(B, dtype=np.float32)
    return W.Workload(name=name, vocab=V, rows=rows, bf16_bits=bits, temperature=t, top_k=k, top_p=p,
                      repetition_penalty=pen, histories=hist, uniforms=u, n_rows_total=B)


def check(w, device, path, logits=None):
    print(f"[edges] {w.name} B={w.batch} V={w.vocab} path={path}", flush=True)
    g = run_path(w, device, path, logits=logits)
    r = O.sample_workload(w)
    fails, stats = compare(g, r)
    print(f"[edges] {w.name}: {stats}", flush=True)
    assert not fails, "\n".join(fails)
    return g


@pytest.mark.parametrize("path", list(PATHS))
def test_largest_vocab_and_history(device, path):
    """V = NS_MAX_VOCAB (fp32) with NS_LDS_HISTORY ids per row (duplicates included)."""
    w = workload("max-vocab-history", 6, L.NS_MAX_VOCAB, seed=91, hist_len=L.NS_LDS_HISTORY)
    check(w, device, path)


@pytest.mark.parametrize("path", list(PATHS))
def test_one_token_vocab(device, path):
    w = workload("one-token", 5, 1, seed=92, hist_len=3)
    g = check(w, device, path)
    assert (g["ids"] == 0).all()


@pytest.mark.parametrize("path", list(PATHS))
def test_bf16_ragged_vocab_padded_stride(device, path):
    """V = 50257 bf16 (not a multiple of 8): the rows are read through a padded stride of
    50264 elements, and the last partial chunk of each row comes from the tail path."""
    V, stride = 50257, 50264
    w = workload("bf16-ragged", 12, V, seed=93, hist_len=300, bf16=True)
    padded = torch.full((w.batch, stride), float("nan"), dtype=torch.bfloat16, device=device)
    src = torch.from_numpy(w.bf16_bits.view(np.int16)).view(torch.bfloat16).to(device)
    padded[:, :V] = src
    check(w, device, path, logits=padded[:, :V])


def test_empty_batch(device):
    """n_sample = 0: nothing is launched or written."""
    logits = torch.randn((4, 64), device=device)
    z32 = torch.zeros(0, dtype=torch.float32, device=device)
    out = torch.full((1,), -7, dtype=torch.int64, device=device)
    L.sample_raw(logits, z32, torch.zeros(0, dtype=torch.int32, device=device), z32, z32, z32, out[:0],
                 sample_idx=torch.zeros(0, dtype=torch.int64, device=device))
    torch.cuda.synchronize()
    assert int(out[0]) == -7


@pytest.mark.parametrize("path", list(PATHS))
def test_invalid_rows_and_history_ids_are_reported(device, path):
    """A sample index outside the logits tensor gives id -1 with PATH_ERROR and FLAG_BAD_ROW
    (no read out of bounds); history ids outside [0, V) are ignored and flagged
    (FLAG_BAD_HIST_ID), and the row samples as the oracle does without them."""
    V, N = 1000, 6
    rng = np.random.default_rng(95)
    flat = (rng.standard_normal((N, V), dtype=np.float32) * 3.0).astype(np.float32)
    sidx = np.array([0, -1, 5, 6, 2], dtype=np.int64)
    B = len(sidx)
    hists = [[1, 2], [3], [-5, 10, V + 3, 20], [4], []]
    offs = np.zeros(B + 1, dtype=np.int32)
    offs[1:] = np.cumsum([len(h) for h in hists])
    ids = np.array([i for h in hists for i in h], dtype=np.int32)
    t = torch.full((B,), 1.0, device=device)
    k = torch.full((B,), 50, dtype=torch.int32, device=device)
    p = torch.full((B,), 0.9, device=device)
    pen = torch.full((B,), 1.2, device=device)
    u_np = rng.random(B, dtype=np.float32)
    u = torch.from_numpy(u_np).to(device)
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    info = torch.zeros((B, L.NS_INFO_WORDS), dtype=torch.int32, device=device)
    ws, mode = PATHS[path]
    kinds = L.row_kinds(np.ones(B), np.full(B, 50), V) if path == "shipped" else path_kinds(path)
    print(f"[edges] invalid rows path={path}", flush=True)
    L.sample_raw(torch.from_numpy(flat).to(device), t, k, p, pen, u, out,
                 sample_idx=torch.from_numpy(sidx).to(device),
                 hist_offsets=torch.from_numpy(offs).to(device), hist_ids=torch.from_numpy(ids).to(device),
                 max_hist=4, out_info=info, workspace=ws, mode=mode, row_kinds=kinds)
    torch.cuda.synchronize()
    g, inf = out.cpu().numpy(), info.cpu().numpy()
    for r in (1, 3):
        assert g[r] == -1 and inf[r][0] == 9 and (inf[r][5] & 4), (r, g[r], inf[r].tolist())
    assert inf[2][5] & 1, inf[2].tolist()
    good = [0, 2, 4]
    clean = [[1, 2], [10, 20], []]
    r = O.sample(flat[sidx[good]], np.ones(3), np.full(3, 50), np.full(3, 0.9), np.full(3, 1.2),
                 [np.asarray(h, dtype=np.int32) for h in clean], u_np[good])
    for j, row in enumerate(good):
        assert g[row] in r.allowed_ids[j], (row, g[row], r.ids[j], r.allowed_ids[j].tolist())


@pytest.mark.parametrize("path", list(PATHS))
def test_misaligned_vocab_with_invalid_sample_indices(device, path):
    """An fp32 vocab of 50257 (rows not 16-byte aligned: the binding copies the sampled
    rows into padded ones) with sample indices outside the logits tensor: the copy
    gathers clamped indices, the bad rows still come back as id -1 with FLAG_BAD_ROW,
    and the valid rows match the oracle."""
    V, N = 50257, 6
    rng = np.random.default_rng(96)
    flat = (rng.standard_normal((N, V), dtype=np.float32) * 3.0).astype(np.float32)
    sidx = np.array([0, -1, 5, N, 2, -(2 ** 40)], dtype=np.int64)
    B = len(sidx)
    t_np, k_np = np.array([1.0, 1.0, 0.0, 0.8, 1.3, 1.0]), np.array([50, 50, 0, 0, 20, 1000])
    t = torch.from_numpy(t_np.astype(np.float32)).to(device)
    k = torch.from_numpy(k_np.astype(np.int32)).to(device)
    p = torch.full((B,), 0.9, device=device)
    pen = torch.full((B,), 1.0, device=device)
    u_np = rng.random(B, dtype=np.float32)
    u = torch.from_numpy(u_np).to(device)
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    info = torch.zeros((B, L.NS_INFO_WORDS), dtype=torch.int32, device=device)
    ws, mode = PATHS[path]
    kinds = L.row_kinds(t_np, k_np, V) if path == "shipped" else path_kinds(path)
    logits = torch.from_numpy(flat).to(device)
    assert (logits.stride(0) * 4) % 16 != 0
    print(f"[edges] misaligned vocab with invalid sample indices path={path}", flush=True)
    L.sample_raw(logits, t, k, p, pen, u, out, sample_idx=torch.from_numpy(sidx).to(device), out_info=info,
                 workspace=ws, mode=mode, row_kinds=kinds)
    torch.cuda.synchronize()
    g, inf = out.cpu().numpy(), info.cpu().numpy()
    for r in (1, 3, 5):
        assert g[r] == -1 and inf[r][0] == 9 and (inf[r][5] & 4), (r, g[r], inf[r].tolist())
    good = [0, 2, 4]
    r = O.sample(flat[sidx[good]], t_np[good], k_np[good], np.full(3, 0.9), np.ones(3), [[], [], []], u_np[good])
    for j, row in enumerate(good):
        assert g[row] in r.allowed_ids[j], (row, g[row], r.ids[j], r.allowed_ids[j].tolist())


@pytest.mark.parametrize("rounding", ["division", "reciprocal"])
@pytest.mark.parametrize("path", ["shipped", "segmented"])
def test_wide_rows_small_kept_set(device, path, rounding):
    """Wide fp32 rows (top-k 200 to 2000, with and without top-p) whose kept set is small
    next to the 16,384-token segment the uniform falls in: the draw lists only the tokens
    whose raw logit can reach the kept set's smallest value (its preimage under the
    temperature, lowered by a few units in the last place).  Temperatures from 1e-3 to 40;
    penalties 1, 1.2 and 0.8 (below 1 no raw bound holds and every token is walked), with
    each row's 40 largest logits in its history so that penalized tokens sit at the bound;
    uniforms spread over [0, 1)."""
    B, V = 24, 128256
    rng = np.random.default_rng(97)
    rows = (rng.standard_normal((B, V), dtype=np.float32) * 2.5).astype(np.float32)
    t = np.array([1e-3, 0.5, 1.0, 1.3, 40.0, 0.7])[np.arange(B) % 6]
    k = np.array([200, 1000, 2000])[np.arange(B) % 3].astype(np.int64)
    p = np.array([1.0, 0.9, 1.0, 0.9])[np.arange(B) % 4]
    pen = np.array([1.0, 1.2, 0.8, 1.2, 1.2])[np.arange(B) % 5]
    hist = [np.concatenate([np.argsort(-rows[i])[:40], rng.integers(0, V, size=60)]).astype(np.int32)
            for i in range(B)]
    u = ((np.arange(B) + 0.5) / B).astype(np.float32)
    w = W.Workload(name="wide-small-kept", vocab=V, rows=rows, bf16_bits=None, temperature=t, top_k=k, top_p=p,
                   repetition_penalty=pen, histories=hist, uniforms=u, n_rows_total=B)
    print(f"[edges] {w.name} B={B} V={V} path={path} rounding={rounding}", flush=True)
    g = run_path(w, device, path, penalty_rounding=rounding)
    r = O.sample_workload(w, penalty_rounding=rounding)
    fails, stats = compare(g, r)
    print(f"[edges] {w.name}: {stats}", flush=True)
    assert not fails, "\n".join(fails)
    # the rows at temperature 0.5 and above are planned and drawn by the wide path (info word 0
    # holds the path code, 7); at 1e-3 the k-th largest lies beyond the histograms' 32 units and
    # the general per-row code takes the row
    planned = t >= 0.5
    assert (g["info"][planned, 0] == 7).all(), g["info"][:, 0]
