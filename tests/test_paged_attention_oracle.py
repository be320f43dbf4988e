"""Pins of the paged-attention oracle (CPU): each check reaches the reference's function by a route
that does not reuse the oracle's code, chosen so that a dropped mask term, a wrong GQA head index,
a transposed block/slot or a missing scale fails at least one of them."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from pa_cases import make_case, oracle_args
from oracle import paged_attention_oracle as PA


def sdpa_reference(case):
    """The reference's SDPA backend restated (paged_attention_torch.py:31-100): per sequence, gather
    its KV through the block table, repeat KV heads for GQA, and use SDPA's causal / decode /
    explicit-mask cases; float32 on the CPU."""
    q = case["query"].float()
    k_cache = case["k_cache"].float()
    v_cache = case["v_cache"].float()
    bs = case["block_size"]
    out = torch.zeros_like(q)
    groups = q.shape[1] // k_cache.shape[2]
    qsl = case["query_start_loc"].tolist()
    for s, (kv_len, q_len) in enumerate(zip(case["seq_lens"].tolist(), case["query_lens"].tolist())):
        if q_len == 0:
            continue
        nblk = (kv_len + bs - 1) // bs
        blocks = case["block_tables"][s, :nblk].long()
        k = k_cache.index_select(0, blocks).reshape(-1, k_cache.shape[2], k_cache.shape[3])[:kv_len]
        v = v_cache.index_select(0, blocks).reshape(-1, v_cache.shape[2], v_cache.shape[3])[:kv_len]
        k = k.repeat_interleave(groups, dim=1)
        v = v.repeat_interleave(groups, dim=1)
        qt = q[qsl[s]:qsl[s + 1]].transpose(0, 1).unsqueeze(0)
        kt = k.transpose(0, 1).unsqueeze(0)
        vt = v.transpose(0, 1).unsqueeze(0)
        if q_len == kv_len:
            a = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=case["scale"])
        elif q_len == 1:
            a = F.scaled_dot_product_attention(qt, kt, vt, scale=case["scale"])
        else:
            mask = torch.arange(kv_len).unsqueeze(0) <= (torch.arange(q_len) + kv_len - q_len).unsqueeze(1)
            a = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask[None, None], scale=case["scale"])
        out[qsl[s]:qsl[s + 1]] = a.squeeze(0).transpose(0, 1)
    return out.double().numpy()


@pytest.mark.parametrize("hq,hkv,d", [(24, 8, 128), (8, 8, 64), (32, 4, 64)])
def test_oracle_matches_sdpa_backend(hq, hkv, d):
    # decode rows, a full prefill (causal), a chunked prefill (explicit mask), an empty sequence
    case = make_case(1, [1, 17, 40, 33, 5], [1, 1, 40, 12, 0], hq=hq, hkv=hkv, d=d, block_size=16,
                     dtype=torch.float32)
    ref = PA.paged_attention(**oracle_args(case))
    np.testing.assert_allclose(ref, sdpa_reference(case), rtol=2e-5, atol=2e-6)


def test_oracle_constant_keys_average_visible_values():
    # equal keys: every visible position has the same score, so the output is the plain mean of
    # the visible values -- of positions 0..kv_pos only (causal), of the query's KV head only
    case = make_case(2, [20, 7], [4, 7], hq=4, hkv=2, d=64, block_size=4, dtype=torch.float32)
    case["k_cache"][:] = 0.25
    a = oracle_args(case)
    ref = PA.paged_attention(**a)
    bt, vc = a["block_tables"], a["v_cache"]
    for s, kv_len, row in PA.query_places(a["seq_lens"], a["query_start_loc"], a["query_lens"]):
        t = np.arange(kv_len)
        vals = vc[bt[s, t // 4], t % 4]  # (kv_len, Hkv, D)
        for h in range(4):
            np.testing.assert_allclose(ref[row, h], vals[:, h // 2, :].mean(axis=0), rtol=1e-12, atol=1e-12)


def test_oracle_single_visible_key_returns_its_value_and_scale_matters():
    # the first query of a full prefill sees only position 0: output = v at position 0 whatever the scores
    case = make_case(3, [9], [9], hq=2, hkv=1, d=64, block_size=4, dtype=torch.float32)
    a = oracle_args(case)
    ref = PA.paged_attention(**a)
    v0 = a["v_cache"][a["block_tables"][0, 0], 0, 0]
    np.testing.assert_allclose(ref[0, 0], v0, rtol=0, atol=0)
    np.testing.assert_allclose(ref[0, 1], v0, rtol=0, atol=0)
    # a different scale changes every output that sees more than one key
    b = dict(a, scale=a["scale"] * 2)
    assert not np.allclose(PA.paged_attention(**b)[1:], ref[1:])


def test_oracle_block_indirection_matches_dense_brute_force():
    # remove the paging: lay every sequence's KV out densely in position order and attend by brute force
    case = make_case(4, [33, 18], [2, 18], hq=6, hkv=3, d=64, block_size=8, dtype=torch.float32)
    a = oracle_args(case)
    ref = PA.paged_attention(**a)
    for s, kv_len, row in PA.query_places(a["seq_lens"], a["query_start_loc"], a["query_lens"]):
        dense_k = np.stack([a["k_cache"][a["block_tables"][s, t // 8], t % 8] for t in range(kv_len)])
        dense_v = np.stack([a["v_cache"][a["block_tables"][s, t // 8], t % 8] for t in range(kv_len)])
        for h in range(6):
            sc = np.array([math.fsum(a["query"][row, h] * dense_k[t, h // 2]) for t in range(kv_len)]) * a["scale"]
            p = np.exp(sc - sc.max())
            p /= p.sum()
            np.testing.assert_allclose(ref[row, h], p @ dense_v[:, h // 2], rtol=1e-10, atol=1e-12)


def test_query_places_match_the_reference_launcher():
    # repeat_interleave of the sequence ids and kv_pos = seq_len - q_len + i (triton.py:109-131)
    places = PA.query_places([5, 3, 9], [0, 2, 2, 6], [2, 0, 4])
    assert [(s, kv, r) for s, kv, r in places] == [(0, 4, 0), (0, 5, 1), (2, 6, 2), (2, 7, 3), (2, 8, 4), (2, 9, 5)]


def test_oracle_condition_terms_closed_forms():
    # the condition term the GPU tolerance scales with: a single visible key gives dev = 0 and
    # cond = |v|; constant keys and constant values give dev = 0, cond = |v|; and the terms leave
    # the output unchanged
    case = make_case(5, [9, 6], [9, 1], hq=2, hkv=1, d=64, block_size=4, dtype=torch.float32)
    a = oracle_args(case)
    out, cond = PA.paged_attention(**a, terms=True)
    np.testing.assert_array_equal(out, PA.paged_attention(**a))
    v0 = a["v_cache"][a["block_tables"][0, 0], 0, 0]
    np.testing.assert_allclose(cond[0, 0], np.abs(v0), rtol=1e-15, atol=0)
    case["k_cache"][:] = 0.5
    case["v_cache"][:] = -1.5
    a = oracle_args(case)
    out, cond = PA.paged_attention(**a, terms=True)
    np.testing.assert_allclose(out, -1.5, rtol=1e-15)
    np.testing.assert_allclose(cond, 1.5, rtol=1e-15)
    # two keys, hand-computed: q = e0, k0 = 2 e0, k1 = -e0 (scale 1), v0 = 1, v1 = 3 in dim 0
    q = np.zeros((1, 1, 4)); q[0, 0, 0] = 1.0
    kc = np.zeros((1, 2, 1, 4)); kc[0, 0, 0, 0] = 2.0; kc[0, 1, 0, 0] = -1.0
    vc = np.zeros((1, 2, 1, 4)); vc[0, 0, 0, 0] = 1.0; vc[0, 1, 0, 0] = 3.0
    out, cond = PA.paged_attention(q, kc, vc, np.zeros((1, 1), np.int64), [2], [0, 1], [1], 1.0, 2, terms=True)
    w0, w1 = math.exp(2) / (math.exp(2) + math.exp(-1)), math.exp(-1) / (math.exp(2) + math.exp(-1))
    o = w0 * 1 + w1 * 3
    np.testing.assert_allclose(out[0, 0, 0], o, rtol=1e-14)
    np.testing.assert_allclose(cond[0, 0, 0], 2.0 * (w0 * abs(1 - o) + w1 * abs(3 - o)) + w0 * 1 + w1 * 3,
                               rtol=1e-14)
