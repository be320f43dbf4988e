"""CPU oracle: a restatement of NanoServe's paged attention.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and ``__graft_entry__.smoke()`` as the checker of
the HIP paged-attention kernel, never by the product.

Follows the reference's two backends, which compute the same function:
  * nanoserve/kernels/paged_attention_triton.py:19-106 -- per query token and query head, KV head
    ``h // num_kv_groups`` (:41), keys at positions ``t < seq_len`` and ``t <= kv_pos`` (:64-66),
    softmax of ``scale * q.k`` over them (:77-85), weighted sum of values (:96), zero output when
    no key is visible (:103-104);
  * the launcher's index set-up (:109-131): query tokens of sequence s are consecutive, ``kv_pos``
    of the i-th one is ``seq_len - q_len + i``;
  * nanoserve/kernels/paged_attention_torch.py:17-28 (block-table gather: position t in block
    ``block_table[t // block_size]``, slot ``t % block_size``) and :68-98 (the same mask stated as
    causal / decode / chunked-prefill cases).
Arithmetic in float64 on the inputs' values (the kernels compute in float32; the tests' tolerance
covers the difference and the output rounding).

Pinned by tests/test_paged_attention_oracle.py against: torch's scaled_dot_product_attention on
the CPU (the reference's own SDPA path, restated per sequence with its three mask cases), constant
keys (softmax uniform: output = mean of the visible values), a single visible key (output = that
value), and an explicit dense-cache brute force with the block indirection removed.
"""
from __future__ import annotations

import numpy as np


def query_places(seq_lens, query_start_loc, query_lens):
    """(sequence, kv_len) of every query token (paged_attention_triton.py:109-131, :64-66)."""
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    ql = np.asarray(query_lens, dtype=np.int64)
    out = []
    for s in range(len(seq_lens)):
        for i in range(int(ql[s])):
            kv_pos = int(seq_lens[s] - ql[s] + i)
            kv_len = max(0, min(kv_pos + 1, int(seq_lens[s])))
            out.append((s, kv_len, int(qsl[s]) + i))
    return out


def paged_attention(query, k_cache, v_cache, block_tables, seq_lens, query_start_loc, query_lens,
                    scale: float, block_size: int, terms: bool = False):
    """float64 (total_q, Hq, D) attention output (paged_attention_triton.py:19-106).

    ``terms``: also return, per output element, the condition term ``S * dev + Vabs`` that scales a
    float computation's rounding error: S = max over visible keys of ``scale * sum_i |q_i k_i|``
    (a dot product's error is at most proportional to it, and it moves the output by the softmax
    weights times ``v - o``), dev = ``sum_t w_t |v_t - o|``, Vabs = ``sum_t w_t |v_t|`` (the
    weighted sum's own error bound, w the normalised weights)."""
    q = np.asarray(query, dtype=np.float64)
    kc = np.asarray(k_cache, dtype=np.float64)
    vc = np.asarray(v_cache, dtype=np.float64)
    bt = np.asarray(block_tables, dtype=np.int64)
    total_q, hq, d = q.shape
    hkv = kc.shape[2]
    groups = hq // hkv
    out = np.zeros((total_q, hq, d), dtype=np.float64)
    cond = np.zeros((total_q, hq, d), dtype=np.float64) if terms else None
    for s, kv_len, row in query_places(seq_lens, query_start_loc, query_lens):
        if kv_len == 0:
            continue
        t = np.arange(kv_len)
        blk = bt[s, t // block_size]
        slot = t % block_size
        k = kc[blk, slot]  # (kv_len, Hkv, D)
        v = vc[blk, slot]
        for h in range(hq):
            kvh = h // groups
            sc = (k[:, kvh, :] @ q[row, h]) * scale
            w = np.exp(sc - sc.max())
            out[row, h] = (w @ v[:, kvh, :]) / w.sum()
            if terms:
                wn = w / w.sum()
                vv = v[:, kvh, :]
                smax = float((np.abs(k[:, kvh, :]) @ np.abs(q[row, h])).max()) * abs(scale)
                cond[row, h] = smax * (wn @ np.abs(vv - out[row, h])) + wn @ np.abs(vv)
    return (out, cond) if terms else out
