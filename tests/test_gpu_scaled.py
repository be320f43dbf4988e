"""GPU: the penalized, temperature-scaled logits bit for bit (sampler.py:31-38 then :41-51).

``ns_debug_scaled`` writes every logit of every sampled row through one of the three
routines the sampling kernels use for it: the streaming / top-k / split-row / segment
kernels' (correctly rounded multiply-and-correct division, NS_DEBUG_STREAM), the wide
path's (the same per chunk, IEEE division for a chunk with an operand out of range,
NS_DEBUG_WIDE) and the general per-row code's (IEEE division for the penalty,
NS_DEBUG_GENERAL).  Per-row and segmented mode differ only in which of these kernels
run, so each routine is compared with the oracle's float32 tensor expression (the
tensor ``OracleResult.scaled`` holds), every element, in both history sources (CSR
histories, and device-resident request slots), under both penalty roundings (the
division torch computes on the CPU, and the reciprocal multiply it computes on a GPU,
NS_PENALTY_RECIPROCAL).  The bar: equal float32 bits; a NaN
matches a NaN (torch and the GPU may carry different NaN payloads, which no later step
reads).  Workloads: the batch-8 fp32 decode batch, the mixed decode batch, the
batch-256 bf16 decode batch with 2048-id histories, the chunked-prefill batch (sample
indices, histories up to 4096 ids), every tiny golden case, and rows of random float32
bit patterns (subnormals, zeros, huge values, infinities, NaN) under extreme
temperatures and penalties, which drive every division onto its out-of-range branch.
"""
import numpy as np
import pytest
import torch

import golden_data as G
from conftest import pkg
from parity import params_of

W = pkg("workloads")
L = pkg("_lib")
S = pkg("sampler")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu

FORMULAS = {"stream": L.NS_DEBUG_STREAM, "wide": L.NS_DEBUG_WIDE, "general": L.NS_DEBUG_GENERAL}
SOURCES = ("csr", "slots")


def oracle_scaled(w, rounding="division"):
    """The oracle's scaled logits of workload ``w`` (the computation OracleResult.scaled holds)."""
    rows = torch.as_tensor(np.asarray(w.rows, dtype=np.float32))
    return O.penalized_scaled(rows, w.temperature, w.repetition_penalty, w.histories, rounding)[1]


def debug_scaled(w, device, formula, source, logits, rounding="division"):
    """One ns_debug_scaled call over ``w``; the (B, V) float32 bits on the host."""
    B, V = w.batch, w.vocab
    if source == "slots":
        dh = S.DeviceHistories(device, B + 2, capacity=max(16, max(len(h) for h in w.histories)))
        for r in range(B):
            dh.open(r, w.histories[r])
        packed = S.PackedRows(params_of(w), None, V, slots=dh.slots(list(range(B))),
                              slot_max_hist=max(len(h) for h in w.histories), penalty_rounding=rounding)
        extra = {"hist_state": dh.state}
    else:
        packed = S.PackedRows(params_of(w), w.histories, V, penalty_rounding=rounding)
        extra = {}
    d = packed.to_device(device)
    if source == "slots":
        extra["hist_slot"] = d["hist_slot"]
    else:
        extra["hist_offsets"], extra["hist_ids"] = d["hist_offsets"], d["hist_ids"]
    u = torch.zeros(B, dtype=torch.float32, device=device)
    ids = torch.zeros(B, dtype=torch.int64, device=device)
    sidx = torch.from_numpy(w.sample_indices).to(device) if w.sample_indices is not None else None
    out = torch.full((B, V), float("nan"), dtype=torch.float32, device=device)
    L.sample_raw(logits, d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"], u, ids, sample_idx=sidx,
                 max_hist=packed.max_hist, workspace=None, debug_scaled=(formula, out),
                 penalty_rounding=packed.penalty_rounding, rep_penalty_recip=d["rep_penalty_recip"], **extra)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32)


def compare_bits(name, got, want):
    want = np.ascontiguousarray(want.numpy(), dtype=np.float32).view(np.uint32)
    assert got.shape == want.shape
    gf, wf = got.view(np.float32), want.view(np.float32)
    both_nan = np.isnan(gf) & np.isnan(wf)
    bad = (got != want) & ~both_nan
    if bad.any():
        r, c = np.argwhere(bad)[0]
        pytest.fail(f"{name}: {int(bad.sum())} of {bad.size} logits differ; first row {r} token {c}: "
                    f"{gf[r, c]!r} ({got[r, c]:#010x}) vs oracle {wf[r, c]!r} ({want[r, c]:#010x})")


def check_workload(w, device, rounding="division"):
    want = oracle_scaled(w, rounding)
    logits = w.device_logits(device)
    for source in SOURCES:
        for fname, formula in FORMULAS.items():
            print(f"[scaled] {w.name} B={w.batch} V={w.vocab} dtype={w.dtype} {fname} {source} {rounding}", flush=True)
            compare_bits(f"{w.name} {fname} {source} {rounding}",
                         debug_scaled(w, device, formula, source, logits, rounding), want)


@pytest.mark.parametrize("rounding", ["division", "reciprocal"])
@pytest.mark.parametrize("cfg", [0, 1, 2, 4])
def test_configs(device, cfg, rounding):
    check_workload(W.make_workload(cfg), device, rounding)


@pytest.mark.parametrize("rounding", ["division", "reciprocal"])
@pytest.mark.parametrize("case", G.tiny(), ids=[c["name"] for c in G.tiny()])
def test_tiny_cases(device, case, rounding):
    check_workload(G.tiny_workload(case), device, rounding)


def random_bits_workload(name, B, V, seed, bf16):
    """Rows of uniformly random float32 (or bf16) bit patterns, temperatures from the
    clamp (1e-9 -> 1e-6) to 1e30, penalties from 1e-3 to 1e30 on histories covering
    about half the row with repeats."""
    rng = np.random.default_rng(seed)
    if bf16:
        bits = rng.integers(0, 1 << 16, size=(B, V), dtype=np.uint32).astype(np.uint16)
        rows = W.bf16_bits_to_f32(bits)
    else:
        bits = None
        rows = rng.integers(0, 1 << 32, size=(B, V), dtype=np.uint64).astype(np.uint32).view(np.float32)
    temps = np.array([0.0, 1e-9, 3e-6, 0.3, 1.0, 2.7, 1e20, 1e30])
    pens = np.array([1.0, 1.1, 0.5, 3.0, 1e-3, 7.0e5, 1e30, 1.3])
    t = temps[np.arange(B) % temps.size]
    pen = pens[(np.arange(B) // temps.size + np.arange(B)) % pens.size]
    hists = [rng.integers(0, V, size=V // 2, dtype=np.int64).astype(np.int32) for _ in range(B)]
    return W.Workload(name=name, vocab=V, rows=np.ascontiguousarray(rows), bf16_bits=bits, temperature=t,
                      top_k=np.full(B, 50, dtype=np.int64), top_p=np.full(B, 0.9), repetition_penalty=pen,
                      histories=hists, uniforms=rng.random(B, dtype=np.float32), n_rows_total=B)


@pytest.mark.parametrize("rounding", ["division", "reciprocal"])
@pytest.mark.parametrize("bf16", [False, True])
def test_random_bit_patterns(device, bf16, rounding):
    check_workload(random_bits_workload(f"scaled-bits{'-bf16' if bf16 else ''}", 24, 8195, 901 + int(bf16), bf16),
                   device, rounding)


def test_invalid_rows_written_as_nan(device):
    """A sample index outside the logits gives its row as NaN; the other rows are unaffected."""
    w = W.make_workload(0)
    B, V = w.batch, w.vocab
    packed = S.PackedRows(params_of(w), w.histories, V)
    d = packed.to_device(device)
    logits = w.device_logits(device)
    sidx = torch.arange(B, dtype=torch.int64, device=device)
    sidx[3] = B + 5
    out = torch.zeros((B, V), dtype=torch.float32, device=device)
    L.sample_raw(logits, d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"],
                 torch.zeros(B, dtype=torch.float32, device=device), torch.zeros(B, dtype=torch.int64, device=device),
                 sample_idx=sidx, hist_offsets=d["hist_offsets"], hist_ids=d["hist_ids"], max_hist=packed.max_hist,
                 workspace=None, debug_scaled=(L.NS_DEBUG_STREAM, out))
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.isnan(got[3]).all()
    keep = [i for i in range(B) if i != 3]
    want = oracle_scaled(w)[keep]
    compare_bits("valid rows", got[keep].numpy().view(np.uint32), want)
