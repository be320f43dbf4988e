"""GPU: small batches of top-k rows against the oracle, in three launch sets: the
split-row kernel (each row spread over several workgroups and merged by the last to
arrive), the one-workgroup-per-row top-k kernel (rows of up to 512 KiB, streamed in one
or two phases; the first phase's chunks that reach the bound are read again), and what
AUTO ships for such calls.  Shapes and values that exercise both: geometries from one
row to 64 rows, fp32 and bf16, slices of unequal length with the partial chunk in the last,
history ids on slice boundaries, ties of equal values spread over slices, a slice
whose values the penalty pushes under its own bound (it then bounds again from its
penalized values), NaN and +inf in single slices, rows of -inf, sample indices, and
calls in a row sharing the workspace's arrival counters.  Same bar as tests/parity.py.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from parity import compare, run_path

W = pkg("workloads")
L = pkg("_lib")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu


def topk_workload(name, B, V, seed, bf16=False, hist_len=64, scale=3.0, k_choices=(1, 8, 50, 64),
                  pen_choices=(1.0, 1.1, 1.5), rows=None, hists=None):
    rng = np.random.default_rng(seed)
    raw = rows if rows is not None else (rng.standard_normal((B, V), dtype=np.float32) * scale).astype(np.float32)
    bits = W.f32_to_bf16_bits(raw) if bf16 else None
    vals = W.bf16_bits_to_f32(bits) if bf16 else raw
    t = rng.choice(np.array([0.6, 1.0, 1.4]), size=B)
    k = rng.choice(np.array(k_choices), size=B).astype(np.int64)
    k = np.minimum(k, V - 1)
    p = rng.choice(np.array([1.0, 0.95, 0.6]), size=B)
    pen = rng.choice(np.array(pen_choices), size=B)
    if hists is None:
        hists = [rng.integers(0, V, size=hist_len, dtype=np.int64).astype(np.int32) for _ in range(B)]
    u = rng.random(B, dtype=np.float32)
    return W.Workload(name=name, vocab=V, rows=vals, bf16_bits=bits, temperature=t, top_k=k, top_p=p,
                      repetition_penalty=pen, histories=hists, uniforms=u, n_rows_total=B)


PATHS3 = ["split", "topk", "shipped"]


def check(w, device, path="split", logits=None, expect_wave_set=True):
    print(f"[split] {w.name} B={w.batch} V={w.vocab} dtype={w.dtype} path={path}", flush=True)
    g = run_path(w, device, path, logits=logits)
    r = O.sample_workload(w)
    fails, stats = compare(g, r)
    paths = {int(c): int((g["info"][:, 0] == c).sum()) for c in np.unique(g["info"][:, 0])}
    print(f"[split] {w.name}: {stats} paths={paths}", flush=True)
    assert not fails, "\n".join(fails)
    if expect_wave_set:
        assert paths.get(6, 0) == w.batch, paths   # merged and drawn on the split path
    return g


GEOMETRIES = [
    # (B, V, bf16): one row over the most slices; the B=8 fp32 decode batch; slice lengths that are
    # not a multiple of the workgroup's chunk row, with and without a partial chunk; bf16 rows
    # with a tail; 33 and 64 rows (fewer, longer slices); the largest vocabulary
    # (one-workgroup kernel: one phase up to 65536 fp32 / 131072 bf16 tokens, two up to twice
    # that, a second phase of only the partial chunk at V = 65537 fp32; longer rows go to the
    # general per-row code on that path)
    (1, 128256, False), (2, 128256, True), (8, 128256, False), (5, 131084, False), (3, 16387, False),
    (7, 50257, True), (16, 32771, True), (33, 128256, True), (64, 128256, False), (4, 262144, False),
    (2, 262144, True), (3, 131072, False), (6, 65537, False), (1, 65536, False),
]


def phases(V, bf16):
    """Streaming phases of 16384 chunks the one-workgroup top-k kernel takes for a row."""
    nch = -(-V // (8 if bf16 else 4))
    return -(-nch // 16384)


@pytest.mark.parametrize("path", PATHS3)
@pytest.mark.parametrize("B,V,bf16", GEOMETRIES)
def test_geometries(device, B, V, bf16, path):
    w = topk_workload(f"split-geom-{B}x{V}{'-bf16' if bf16 else ''}", B, V, seed=700 + B + V % 97, bf16=bf16,
                      hist_len=300)
    check(w, device, path, expect_wave_set=not (path == "topk" and phases(V, bf16) > 2))


@pytest.mark.parametrize("path", PATHS3)
def test_history_on_slice_boundaries(device, path):
    """History ids at the first and last token of every slice (and duplicates of them) with
    the largest values of the row placed there: each slice's bitmap covers its own range.
    Slice s of S holds chunks [s * nch / S, (s + 1) * nch / S); the edges of every S the
    host can pick for this shape are marked."""
    B, V = 4, 128256
    rng = np.random.default_rng(711)
    rows = (rng.standard_normal((B, V), dtype=np.float32) * 2.0).astype(np.float32)
    nch = V // 4
    edges = []
    for S in range(2, 17):
        for s in range(S):
            a, b = s * nch // S * 4, (s + 1) * nch // S * 4
            edges += [a, b - 1]
    edges = np.unique(np.array(edges, dtype=np.int64))
    rows[:, edges] = 9.0 + rng.random((B, edges.size), dtype=np.float32)
    hists = [np.concatenate([edges, edges[:10]]).astype(np.int32) for _ in range(B)]
    w = topk_workload("split-boundaries", B, V, seed=712, rows=rows, hists=hists, pen_choices=(1.3, 2.0))
    check(w, device, path)


@pytest.mark.parametrize("path", PATHS3)
def test_ties_across_slices(device, path):
    """Values on a coarse grid: the k-th largest value is shared by many tokens spread over
    every slice; the kept set is all of them (sampler.py:56-58).  Rows whose ties outgrow
    a slice's list go to the general code, with the same results."""
    B, V = 6, 128256
    rng = np.random.default_rng(713)
    rows = np.round(rng.standard_normal((B, V), dtype=np.float32) * 2.0).astype(np.float32)
    w = topk_workload("split-ties", B, V, seed=714, rows=rows, pen_choices=(1.0,))
    check(w, device, path, expect_wave_set=False)


@pytest.mark.parametrize("path", PATHS3)
def test_penalty_under_the_slice_bound(device, path):
    """Slice 0 holds 60 tokens of value 10, one in each of 60 of its 8-lane groups (token 32 g),
    whose history penalty (x3) leaves them at 3.33, under the slice's first bound (10): its
    first list is empty, and it bounds again from the maxima of its penalized values and
    hands the 60 over.  The one-workgroup kernel meets the same list short of k over the
    whole row and bounds again the same way (its first phase read again).  Row 0: 100 tokens of 50 elsewhere hold the row's top-k.  Row 1:
    nothing above 10 elsewhere, and the penalized tokens are among the row's top-k.  Tokens
    [0, 16384) are -inf otherwise, so slice 0 is the same at 1, 2 or 4 chunks per thread."""
    B, V = 2, 128256
    rng = np.random.default_rng(715)
    rows = (rng.standard_normal((B, V), dtype=np.float32)).astype(np.float32)
    rows[:, :16384] = -np.inf
    hot = 32 * rng.choice(128, size=60, replace=False)
    rows[:, hot] = 10.0
    far = 20000 + rng.choice(100000, size=100, replace=False)
    rows[0, far] = 50.0
    hists = [hot.astype(np.int32), hot.astype(np.int32)]
    w = topk_workload("split-penalty-bound", B, V, seed=716, rows=rows, hists=hists, k_choices=(50,),
                      pen_choices=(3.0,))
    check(w, device, path)


@pytest.mark.parametrize("path", PATHS3)
def test_special_values_in_one_slice(device, path):
    """NaN in one slice (row 0), +inf in one slice (row 1), both in different slices (row 2),
    a row of -inf (row 3), a row with a single finite token (row 4): the NaN guard's uniform
    row (sampler.py:77-80) or the general code, as the oracle."""
    B, V = 5, 128256
    rng = np.random.default_rng(717)
    rows = (rng.standard_normal((B, V), dtype=np.float32) * 3.0).astype(np.float32)
    rows[0, 70000] = np.nan
    rows[1, 5] = np.inf
    rows[2, 100] = np.inf
    rows[2, 120000] = np.nan
    rows[3, :] = -np.inf
    rows[4, :] = -np.inf
    rows[4, 99999] = 1.5
    w = topk_workload("split-special", B, V, seed=718, rows=rows, k_choices=(20,))
    check(w, device, path, expect_wave_set=False)


@pytest.mark.parametrize("path", PATHS3)
def test_sample_indices(device, path):
    """Sampled rows picked from a larger flat tensor (the chunked-prefill layout)."""
    w = W.make_workload(4)
    keep = [i for i in range(w.batch) if 1 <= w.top_k[i] <= 64 and w.temperature[i] > 0][:40]
    sub = W.Workload(name="split-sidx", vocab=w.vocab, rows=w.rows[keep], bf16_bits=None,
                     temperature=w.temperature[keep], top_k=w.top_k[keep], top_p=w.top_p[keep],
                     repetition_penalty=np.maximum(w.repetition_penalty[keep], 1.0),
                     histories=[w.histories[i] for i in keep], uniforms=w.uniforms[keep],
                     n_rows_total=w.n_rows_total, sample_indices=w.sample_indices[keep],
                     filler_seed=w.filler_seed)
    check(sub, device, path)


@pytest.mark.parametrize("path", PATHS3)
def test_consecutive_calls_share_counters(device, path):
    """Calls of different shapes back to back on one workspace: each leaves the arrival
    counters at zero for the next."""
    a = topk_workload("split-a", 8, 128256, seed=719)
    b = topk_workload("split-b", 3, 50257, seed=720, bf16=True)
    for w in (a, b, a, b):
        check(w, device, path)


@pytest.mark.parametrize("bf16,V", [(False, 128256), (True, 128256), (False, 50000)])
def test_topk_kernel_temperature_range(device, bf16, V):
    """The top-k kernel's bound maps the k-th largest group maximum through the temperature
    (the smallest raw value whose quotient reaches the bound's): searched by the whole wave
    when the window of keys fits it (temperatures up to about 11.75), by the serial search
    otherwise.  Temperatures from 1e-3 to 1e4, k from 1 to 64, with penalties, in one phase
    (bf16 and fp32 V=50000) and two (fp32 V=128256, whose first phase's kept 16-bit maxima
    are compared with the bound as keys)."""
    B = 14
    w = topk_workload(f"topk-temps-{'bf16' if bf16 else 'f32'}-{V}", B, V, seed=311 + V, bf16=bf16, hist_len=200,
                      k_choices=(1, 7, 50, 64), pen_choices=(1.0, 1.1, 1.5))
    w.temperature[:] = np.array([1e-3, 0.05, 0.3, 0.8, 1.0, 1.7, 3.3, 8.0, 11.5, 12.5, 40.0, 333.0, 1e4, 0.8])[:B]
    check(w, device, "topk")
    check(w, device, "shipped")
