"""GPU: the lm_head GEMM (ns_lm_head_bf16) against a plain PyTorch fp32 reference.

logits = bf16_rne(hidden[rows] @ weight.T) with fp32 accumulation.  The bar, per
element: |ours - ref| <= 2^-8 |ref| (half a bf16 ulp of rounding) + 2^-14 S, where
ref is the fp32 product and S = |hidden| @ |weight|.T bounds the fp32 summation-order
error (the kernel's k order differs from torch's).  A wrong row, column or k mapping
is off by O(S) and fails.  Almost every element must also equal the bf16 rounding of
the reference exactly.
"""
import numpy as np
import pytest
import torch

from conftest import pkg

L = pkg("_lib")

pytestmark = pytest.mark.gpu


def make(device, n_hidden, vocab, k, seed, scale=1.0):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    hidden = torch.randn((n_hidden, k), generator=g, device=device).to(torch.bfloat16)
    weight = (torch.randn((vocab, k), generator=g, device=device) * (scale / k ** 0.5)).to(torch.bfloat16)
    return hidden, weight


def check(ours, hidden, weight, rows=None):
    h = hidden.float() if rows is None else hidden.float().index_select(0, rows)
    wt = weight.float().t().contiguous()
    ref = torch.mm(h, wt)
    s = torch.mm(h.abs(), wt.abs())
    diff = (ours.float() - ref).abs()
    tol = ref.abs() * 2.0 ** -8 + s * 2.0 ** -14
    bad = diff > tol
    assert not bool(bad.any()), (f"{int(bad.sum())} of {bad.numel()} off; first at "
                                 f"{tuple(torch.nonzero(bad)[0].tolist())}: {float(ours.float()[bad][0])!r} vs "
                                 f"{float(ref[bad][0])!r}")
    exact = float((ours == ref.to(torch.bfloat16)).float().mean())
    print(f"[lm_head] exact bf16 match fraction {exact:.6f}", flush=True)
    assert exact > 0.99


@pytest.mark.parametrize("m,vocab,k", [(256, 128256, 2048), (7, 1000, 128), (300, 129, 64), (64, 4096, 4096),
                                       (1, 257, 192)])
def test_lm_head_matches_fp32(device, m, vocab, k):
    print(f"[lm_head] m={m} V={vocab} k={k}", flush=True)
    hidden, weight = make(device, m, vocab, k, seed=m + vocab + k, scale=3.0)
    ours = L.lm_head_bf16(hidden, weight)
    torch.cuda.synchronize()
    assert ours.shape == (m, vocab) and ours.dtype == torch.bfloat16
    check(ours, hidden, weight)


@pytest.mark.parametrize("m,vocab,k", [(256, 128256, 2048), (64, 128256, 2048), (1, 128256, 2048), (77, 1000, 192),
                                       (300, 300, 64)])
def test_packed_weight_gives_the_same_logits(device, m, vocab, k):
    """The packed layout changes only where the weight is read from: bit-identical logits."""
    print(f"[lm_head] packed m={m} V={vocab} k={k}", flush=True)
    hidden, weight = make(device, m, vocab, k, seed=7 + m, scale=3.0)
    pw = L.PackedLmHead(weight)
    plain = L.lm_head_bf16(hidden, weight)
    packed = L.lm_head_bf16(hidden, pw)
    torch.cuda.synchronize()
    assert torch.equal(plain.view(torch.int16), packed.view(torch.int16))
    if m == 256:
        check(packed, hidden, weight)


def test_lm_head_gathers_rows_and_strides(device):
    """Sample positions gathered in the kernel (engine.py:233-234), a padded hidden row
    stride and a logits buffer wider than the vocab."""
    hidden_full, weight = make(device, 500, 3000, 256, seed=11)
    hidden = torch.zeros((500, 320), dtype=torch.bfloat16, device=device)[:, :256]
    hidden.copy_(hidden_full)
    rows = torch.from_numpy(np.sort(np.random.default_rng(3).choice(500, 77, replace=False))).to(device)
    out_full = torch.full((77, 3100), 7.0, dtype=torch.bfloat16, device=device)
    out = out_full[:, :3000]
    L.lm_head_bf16(hidden, weight, rows=rows, out=out)
    torch.cuda.synchronize()
    check(out, hidden_full, weight, rows=rows)
    assert bool((out_full[:, 3000:] == 7.0).all())   # nothing written past n


def test_gather_index_out_of_range_gives_nan_row(device):
    """A gathered index outside the hidden tensor reads nothing out of bounds: its logits
    row is NaN (the sampler then reports a NaN row) and the other rows are unaffected."""
    hidden, weight = make(device, 40, 700, 128, seed=21)
    rows = torch.tensor([3, -1, 39, 40, 1 << 40, 7], dtype=torch.int64, device=device)
    for w in (weight, L.PackedLmHead(weight)):
        out = L.lm_head_bf16(hidden, w, rows=rows).float()
        torch.cuda.synchronize()
        bad = torch.tensor([False, True, False, True, True, False], device=device)
        assert bool(torch.isnan(out[bad]).all())
        good = rows[~bad]
        check(out[~bad].to(torch.bfloat16), hidden, weight, rows=good)


def test_lm_head_special_values(device):
    """Inf and NaN inputs propagate as in IEEE arithmetic; large values round to inf."""
    hidden, weight = make(device, 4, 256, 64, seed=5)
    hidden[1, 3] = float("inf")
    hidden[2, 0] = float("nan")
    ours = L.lm_head_bf16(hidden, weight).float()
    torch.cuda.synchronize()
    ref = torch.mm(hidden.float(), weight.float().t().contiguous())
    assert torch.equal(torch.isnan(ours), torch.isnan(ref))
    assert torch.equal(torch.isinf(ours), torch.isinf(ref))
    fin = torch.isfinite(ref)
    assert bool(((ours[fin] - ref[fin]).abs() <= ref[fin].abs() * 2.0 ** -8 + 1e-3).all())


@pytest.mark.parametrize("m", [100, 260])
def test_packed_large_batch_gathers_rows_and_flags_bad_indices(device, m):
    """Packed batches beyond 64 rows (the column-owner kernel, one and two workgroup rows):
    gathered rows, a padded hidden stride, invalid indices as NaN rows, a logits buffer wider
    than the vocab; the same bits as the weight as stored."""
    hidden_full, weight = make(device, 700, 1300, 192, seed=31 + m, scale=3.0)
    hidden = torch.zeros((700, 200), dtype=torch.bfloat16, device=device)[:, :192]
    hidden.copy_(hidden_full)
    g = np.random.default_rng(m)
    rows_np = g.integers(0, 700, size=m).astype(np.int64)
    bad_pos = g.choice(m, 5, replace=False)
    rows_np[bad_pos] = np.array([-1, 700, 701, -5, 1 << 40], dtype=np.int64)
    rows = torch.from_numpy(rows_np).to(device)
    pw = L.PackedLmHead(weight)
    out_full = torch.full((m, 1400), 7.0, dtype=torch.bfloat16, device=device)
    out = out_full[:, :1300]
    L.lm_head_bf16(hidden, pw, rows=rows, out=out)
    plain = L.lm_head_bf16(hidden, weight, rows=rows)
    torch.cuda.synchronize()
    assert bool((out_full[:, 1300:] == 7.0).all())   # nothing written past n
    bad = torch.zeros(m, dtype=torch.bool, device=device)
    bad[torch.from_numpy(bad_pos).to(device)] = True
    assert bool(torch.isnan(out.float()[bad]).all())
    good = ~bad
    check(out[good], hidden_full, weight, rows=rows[good])
    assert torch.equal(out[good].contiguous().view(torch.int16), plain[good].contiguous().view(torch.int16))
