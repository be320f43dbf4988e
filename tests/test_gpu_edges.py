"""GPU: boundary shapes against the oracle -- the largest vocabulary and history the
ABI accepts, a one-token vocabulary, a bf16 vocabulary that is not a multiple of the
16-byte chunk read through a padded row stride, and an empty batch.  Same bar as
tests/parity.py (ids bit-exact outside exempt rows, thresholds bit-exact, probabilities
within 1e-5 relative), in both kernel modes.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import PATHS, compare, run_gpu

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
    ws, mode = PATHS[path]
    g = run_gpu(w, device, logits=logits, workspace=ws, mode=mode)
    r = O.sample_workload(w)
    fails, stats = compare(g, r)
    print(f"[edges] {w.name}: {stats}", flush=True)
    assert not fails, "\n".join(fails)
    return g


@pytest.mark.parametrize("path", list(PATHS))
def test_largest_vocab_and_history(device, path):
    """V = NS_MAX_VOCAB (fp32) with NS_MAX_HISTORY ids per row (duplicates included)."""
    w = workload("max-vocab-history", 6, L.NS_MAX_VOCAB, seed=91, hist_len=L.NS_MAX_HISTORY)
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
