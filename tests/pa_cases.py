"""Seeded inputs for the paged-attention tests: paged KV caches with shuffled physical blocks,
block tables, and the batch layout the reference's engine builds (query_start_loc, query_lens)."""
from __future__ import annotations

import math

import numpy as np
import torch

DECODE_LLAMA32_3B = dict(hq=24, hkv=8, d=128, block_size=16)


def make_case(seed, seq_lens, query_lens, hq=24, hkv=8, d=128, block_size=16, dtype=torch.bfloat16,
              spare_blocks=5, spare_cols=2, qkv_view=False):
    """CPU tensors of a paged-attention call; values exactly representable in ``dtype``."""
    rng = np.random.default_rng(seed)
    seq_lens = [int(x) for x in seq_lens]
    query_lens = [int(x) for x in query_lens]
    num_seqs = len(seq_lens)
    per_seq = [math.ceil(x / block_size) for x in seq_lens]
    cols = max(per_seq + [1]) + spare_cols
    num_blocks = sum(per_seq) + spare_blocks
    perm = rng.permutation(num_blocks)
    bt = np.zeros((num_seqs, cols), dtype=np.int32)
    at = 0
    for s, n in enumerate(per_seq):
        bt[s, :n] = perm[at:at + n]
        at += n
    total_q = sum(query_lens)
    qsl = np.zeros(num_seqs + 1, dtype=np.int32)
    qsl[1:] = np.cumsum(query_lens)
    k = torch.from_numpy(rng.standard_normal((num_blocks, block_size, hkv, d), dtype=np.float32)).to(dtype)
    v = torch.from_numpy(rng.standard_normal((num_blocks, block_size, hkv, d), dtype=np.float32)).to(dtype)
    if qkv_view:
        # the layout the reference's Attention.forward hands over: a view into the fused QKV output
        qkv = torch.from_numpy(rng.standard_normal((total_q, (hq + 2 * hkv) * d), dtype=np.float32)).to(dtype)
        q = qkv[:, :hq * d].view(total_q, hq, d)
    else:
        q = torch.from_numpy(rng.standard_normal((total_q, hq, d), dtype=np.float32)).to(dtype)
    return dict(query=q, k_cache=k, v_cache=v, block_tables=torch.from_numpy(bt),
                seq_lens=torch.tensor(seq_lens, dtype=torch.int32), query_start_loc=torch.from_numpy(qsl),
                query_lens=torch.tensor(query_lens, dtype=torch.int32), scale=1.0 / math.sqrt(d),
                block_size=block_size)


def oracle_args(case):
    """The case as float64/int numpy arrays for the oracle."""
    out = {}
    for key, val in case.items():
        out[key] = val.double().numpy() if isinstance(val, torch.Tensor) and val.is_floating_point() else (
            val.numpy() if isinstance(val, torch.Tensor) else val)
    return out


def to_device(case, device):
    out = {}
    for key, val in case.items():
        if isinstance(val, torch.Tensor):
            if key == "query" and not val.is_contiguous():
                # keep the strided view: move its base and re-take the view on the device
                base = val._base if val._base is not None else val
                dev_base = base.to(device)
                out[key] = dev_base.as_strided(val.shape, val.stride(), val.storage_offset())
            else:
                out[key] = val.to(device)
        else:
            out[key] = val
    return out


# output tolerance per dtype: the kernels compute in float32 and round the output once
TOL = {torch.float32: (1e-5, 1e-4), torch.float16: (1e-4, 2.0 ** -9), torch.bfloat16: (1e-4, 2.0 ** -7)}


# unit roundoff of the kernels' arithmetic per input type: float32 throughout for float32 inputs;
# for 16-bit inputs the weights enter the MFMA value product as a high and a low 16-bit part
# (16 significant bits at least)
UNIT = {torch.float32: 2.0 ** -24, torch.float16: 2.0 ** -16, torch.bfloat16: 2.0 ** -16}
OUT_BITS = {torch.float32: None, torch.float16: 11, torch.bfloat16: 8}
# Arithmetic bound: |out - oracle| <= half an output ulp + K * UNIT * cond, cond = S * dev + Vabs
# per element (the oracle's condition term).  Worst ratios over the GPU suite
# (|err| - half ulp) / (UNIT * cond): float32 2.4, float16 0.0017, bfloat16 0.026; K sits a few
# times above each.
ARITH_K = {torch.float32: 8.0, torch.float16: 0.25, torch.bfloat16: 0.25}


def half_ulp(x, dtype):
    """Half a unit in the last place of |x| in the output type (0 for float32 outputs)."""
    bits = OUT_BITS[dtype]
    if bits is None:
        return np.zeros_like(x)
    _, e = np.frexp(np.abs(x))
    h = np.ldexp(1.0, e - 1 - bits)
    if dtype == torch.float16:
        h = np.maximum(h, 2.0 ** -25)   # subnormal spacing
    return h


def arithmetic_ratio(out, ref, cond, dtype):
    """max over elements of (|err| - half an output ulp) / (u * cond): the error in units of the
    arithmetic's rounding scaled by the element's condition term."""
    got = out.double().cpu().numpy()
    err = np.abs(got - ref) - half_ulp(np.maximum(np.abs(ref), np.abs(got)), dtype)
    return float((err / (UNIT[dtype] * np.maximum(cond, 1e-30))).max())


def assert_close_to_oracle(out, ref, dtype):
    """``ref``: the oracle's output, or (output, condition terms) for the arithmetic bound."""
    if isinstance(ref, tuple):
        ref, cond = ref
        got = out.double().cpu().numpy()
        err = np.abs(got - ref)
        bound = half_ulp(np.maximum(np.abs(ref), np.abs(got)), dtype) + ARITH_K[dtype] * UNIT[dtype] * cond
        ratio = arithmetic_ratio(out, ref, cond, dtype)
        print(f"paged attention: arithmetic error ratio {ratio:.3g} (bound {ARITH_K[dtype]})", flush=True)
        bad = err > bound
        assert not bad.any(), (
            f"{int(bad.sum())} of {bad.size} outputs outside half an ulp + {ARITH_K[dtype]} * u * cond; worst ratio "
            f"{ratio:.3g} at {np.unravel_index(int(np.argmax(err - bound)), err.shape)}")
        return
    atol, rtol = TOL[dtype]
    got = out.double().cpu().numpy()
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    assert not bad.any(), (
        f"{int(bad.sum())} of {bad.size} outputs outside atol {atol} + rtol {rtol}; worst |err| "
        f"{float(err.max()):.3g} at {np.unravel_index(int(np.argmax(err - bound)), err.shape)}")
