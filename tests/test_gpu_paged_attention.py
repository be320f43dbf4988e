"""GPU parity of the HIP paged-attention kernels (through the C-ABI) against the CPU oracle
(float64 restatement of nanoserve/kernels/paged_attention_triton.py:19-131). Tolerance per output
element: half an ulp of the output type (none for float32) + K * u * cond, cond = S * dev + Vabs the
oracle's condition term (the largest |q|.|k| score scale times the weighted spread of the values,
plus the weighted |v|), u = 2^-24 for float32 and 2^-16 for the 16-bit types, K = 8 resp. 0.25
(tests/pa_cases.py)."""
import numpy as np
import pytest
import torch

from conftest import pkg
from pa_cases import assert_close_to_oracle, make_case, oracle_args, to_device
from oracle import paged_attention_oracle as PA

pytestmark = pytest.mark.gpu
A = pkg("paged_attention")


def run(case, device, **kw):
    c = to_device(case, device)
    print(f"paged attention: q {tuple(case['query'].shape)} {case['query'].dtype} seqs {case['seq_lens'].tolist()} "
          f"q_lens {case['query_lens'].tolist()}", flush=True)
    out = A.paged_attention_hip(c["query"], c["k_cache"], c["v_cache"], c["block_tables"], c["seq_lens"],
                                c["query_start_loc"], c["query_lens"], c["scale"], c["block_size"], **kw)
    torch.cuda.synchronize()
    return out


def check(case, device, **kw):
    out = run(case, device, **kw)
    ref = PA.paged_attention(**oracle_args(case), terms=True)
    assert_close_to_oracle(out, ref, case["query"].dtype)
    return out


def test_decode_llama32_3b_split_partitions(device):
    # 8 decode rows, lengths around block edges and long enough to be split and merged
    case = make_case(10, [1, 15, 16, 17, 100, 513, 1500, 4000], [1] * 8)
    check(case, device)


def test_decode_batch_64_ctx_2048(device):
    # the benchmark's shape: 64 decode rows of 2048 positions, Llama-3.2-3B heads, bf16
    case = make_case(11, [2048] * 64, [1] * 64, spare_blocks=0, spare_cols=0)
    check(case, device)


def test_chunked_prefill_mix(device):
    # full prefill (causal), decode, chunked prefill, an empty sequence, a short full prefill
    case = make_case(12, [37, 64, 300, 20, 9], [37, 1, 45, 0, 9])
    check(case, device)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (16, 8, 64), (32, 8, 128), (32, 4, 64), (24, 8, 64), (64, 8, 128)])
def test_head_layouts_and_dtypes(device, dtype, hq, hkv, d):
    case = make_case(13 + hq + d, [70, 1, 260, 33], [1, 1, 30, 33], hq=hq, hkv=hkv, d=d, block_size=16,
                     dtype=dtype)
    check(case, device)


@pytest.mark.parametrize("block_size", [1, 7, 8, 12, 32])
def test_block_sizes(device, block_size):
    case = make_case(20 + block_size, [45, 130, 7], [1, 3, 7], block_size=block_size)
    check(case, device)


def test_strided_query_view_of_fused_qkv(device):
    # query as the view into the fused QKV output that Attention.forward passes
    case = make_case(30, [50, 200], [50, 1], qkv_view=True)
    assert not case["query"].is_contiguous()
    check(case, device)


def test_zero_visible_keys_gives_zeros(device):
    # a sequence of length 0 holding one query token (malformed batch): the reference's l == 0 guard
    case = make_case(31, [0, 20], [1, 1])
    out = check(case, device)
    assert torch.count_nonzero(out[0].float()).item() == 0


def test_long_rows_through_merge_and_repeat_bit_exact(device):
    case = make_case(32, [8192, 3], [1, 1], hq=32, hkv=8, d=128)
    a = check(case, device)
    b = run(case, device)
    assert torch.equal(a, b)


def test_status_flags_bad_block_and_short_max_seq_len(device):
    case = make_case(33, [40, 40], [1, 1])
    nb = case["k_cache"].shape[0]
    bad = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    bad["block_tables"][0, 1] = nb + 7  # out of the cache: the kernel skips those keys and flags it
    status = torch.zeros(1, dtype=torch.int32, device=device)
    out = run(bad, device, status=status)
    assert status.item() & A.STATUS_BAD_BLOCK
    ref, cond = PA.paged_attention(**oracle_args(case), terms=True)
    # the other sequence is untouched by the bad entry
    assert_close_to_oracle(out[1:], (ref[1:], cond[1:]), case["query"].dtype)
    status.zero_()
    run(case, device, status=status)
    assert status.item() == 0
    # a max_seq_len below a sequence's length: flagged when the grid cannot cover that sequence
    # (400 positions need 7 partitions of 64, the grid sized for 16 positions holds one)
    long_case = make_case(36, [400, 40], [1, 1])
    run(long_case, device, status=status, max_seq_len=16)
    assert status.item() & A.STATUS_SEQ_TOO_LONG


def test_empty_batch_and_argument_errors(device):
    case = make_case(34, [5], [0])
    out = run(case, device)
    assert out.shape[0] == 0
    c = to_device(make_case(35, [5], [1]), device)
    with pytest.raises(A.PagedAttentionError, match="block_size"):
        A.paged_attention_hip(c["query"], c["k_cache"], c["v_cache"], c["block_tables"], c["seq_lens"],
                              c["query_start_loc"], c["query_lens"], c["scale"], 8)


def test_split_rows_leave_the_counters_at_zero(device):
    # split rows are merged by their last partition's workgroup through arrival counters; each call
    # must leave them at zero, so repeated calls of different shapes on one counters buffer (and a
    # reused workspace holding an earlier call's partials) stay exact
    counters = torch.zeros(4096, dtype=torch.int32, device=device)
    ws = torch.full((32 << 20,), 0x7F, dtype=torch.uint8, device=device)  # largest need: 15.9 MB
    for seed, lens in ((37, [3000, 700, 5000]), (38, [64] * 70 + [9000]), (39, [2500] * 3)):
        case = make_case(seed, lens, [1] * len(lens))
        q = case["query"]
        assert A.workspace_bytes(q.shape[0], q.shape[1], case["k_cache"].shape[2], q.shape[2], max(lens)) > 0
        ref = PA.paged_attention(**oracle_args(case), terms=True)
        outs = []
        for _ in range(2):
            out = run(case, device, workspace=ws, counters=counters)
            assert_close_to_oracle(out, ref, q.dtype)
            outs.append(out)
        assert torch.equal(outs[0], outs[1])
        assert torch.count_nonzero(counters).item() == 0


def test_more_partitions_than_the_lds_weight_table(device):
    # one KV head and one long row: 1094 partitions of 64 positions, more than the merging
    # workgroup's LDS weight table (1024 entries) holds, so the one-pass rescaled merge runs
    case = make_case(40, [70000], [1], hq=8, hkv=1, d=128)
    assert A.workspace_bytes(1, 8, 1, 128, 70000) == 1 * 8 * 1094 * (128 + 2) * 4
    check(case, device)


def test_side_stream_and_output_stride(device):
    """A call on a side stream (its temporaries and counters made on that stream) equals the
    call on the current stream bit for bit; an output whose head_dim stride is not 1 is refused
    (the kernel writes out[token, head, d] with a unit stride along d)."""
    case = make_case(21, [1500, 7, 300], [1, 1, 20])
    want = run(case, device)
    side = torch.cuda.Stream(device=device)
    c = to_device(case, device)
    torch.cuda.synchronize()
    got = A.paged_attention_hip(c["query"], c["k_cache"], c["v_cache"], c["block_tables"], c["seq_lens"],
                                c["query_start_loc"], c["query_lens"], c["scale"], c["block_size"], stream=side)
    side.synchronize()
    assert torch.equal(got, want)
    raw = A.paged_attention_hip(c["query"], c["k_cache"], c["v_cache"], c["block_tables"], c["seq_lens"],
                                c["query_start_loc"], c["query_lens"], c["scale"], c["block_size"],
                                stream=side.cuda_stream)
    side.synchronize()
    assert torch.equal(raw, want)
    # a raw handle of 0 is the null stream, torch's default stream: the call is ordered after the
    # default stream's unsynchronized work (the caches written just before it)
    torch.cuda.synchronize()
    with torch.cuda.stream(torch.cuda.default_stream(device)):
        kc, vc = c["k_cache"].clone(), c["v_cache"].clone()
        null = A.paged_attention_hip(c["query"], kc, vc, c["block_tables"], c["seq_lens"], c["query_start_loc"],
                                     c["query_lens"], c["scale"], c["block_size"], stream=0)
    torch.cuda.default_stream(device).synchronize()
    assert torch.equal(null, want)
    q = c["query"]
    bad = torch.empty((q.shape[0], q.shape[1], q.shape[2] * 2), dtype=q.dtype, device=device)[:, :, ::2]
    with pytest.raises(A.PagedAttentionError, match="unit head_dim stride"):
        A.paged_attention_hip(q, c["k_cache"], c["v_cache"], c["block_tables"], c["seq_lens"],
                              c["query_start_loc"], c["query_lens"], c["scale"], c["block_size"], out=bad)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,d", [(24, 8, 128), (32, 8, 128), (8, 8, 64), (16, 8, 64), (64, 8, 128)])
def test_prefill_tiles_head_layouts(device, dtype, hq, hkv, d):
    # sequences of several query tokens go by MFMA query tile (128 // G tokens each): a chunk in the
    # middle of a long sequence, a full prefill, chunks shorter than a tile, and decode rows beside them
    case = make_case(50 + hq + d, [700, 300, 190, 1, 90, 45], [200, 300, 3, 1, 17, 1], hq=hq, hkv=hkv, d=d,
                     dtype=dtype)
    check(case, device)


def test_prefill_chunk_512_over_4096_positions(device):
    # the reference's chunked_prefill_size (config.py:53): a 512-token chunk at the end of a 4096-position
    # sequence, split over KV partitions merged by the last to arrive, and a second chunk of another sequence
    case = make_case(60, [4096, 1500], [512, 512])
    check(case, device)


@pytest.mark.parametrize("block_size", [1, 7, 16, 32])
def test_prefill_tiles_block_sizes(device, block_size):
    case = make_case(70 + block_size, [130, 77], [64, 77], block_size=block_size)
    check(case, device)


def test_prefill_tiles_repeat_bit_exact_and_strided_query(device):
    case = make_case(80, [900, 64], [300, 64], qkv_view=True)
    a = check(case, device)
    b = run(case, device)
    assert torch.equal(a, b)


def test_prefill_bad_tile_is_flagged(device):
    # a tile reaching past its sequence's query tokens is refused by the kernel (status bit), nothing
    # out of bounds is touched, and the other tiles and tokens are exact
    import ctypes

    case = make_case(90, [100, 40], [40, 1])
    c = to_device(case, device)
    q = c["query"]
    out = torch.full_like(q, 7.0)
    tiles = torch.tensor([[0, 0, 21], [0, 21, 19], [0, 30, 21]], dtype=torch.int32, device=device)
    tokens = torch.tensor([40], dtype=torch.int32, device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    lib = A.load()
    bt = c["block_tables"]
    a = A.NsPagedAttnArgs(
        q.data_ptr(), c["k_cache"].data_ptr(), c["v_cache"].data_ptr(), out.data_ptr(), bt.data_ptr(),
        c["seq_lens"].data_ptr(), c["query_start_loc"].data_ptr(), c["query_lens"].data_ptr(), status.data_ptr(),
        None, 0, None, q.stride(0), q.stride(1), c["k_cache"].stride(0), c["k_cache"].stride(1),
        c["k_cache"].stride(2), c["v_cache"].stride(0), c["v_cache"].stride(1), c["v_cache"].stride(2),
        out.stride(0), out.stride(1), bt.stride(0), q.shape[0], 2, 24, 8, 128, 16, c["k_cache"].shape[0], bt.shape[1],
        100, A.NS_PA_DTYPE_BF16, c["scale"])
    a.decode_tokens, a.n_decode_tokens = tokens.data_ptr(), 1
    a.prefill_tiles, a.n_prefill_tiles = tiles.data_ptr(), 3
    nb, nc = ctypes.c_uint64(0), ctypes.c_uint64(0)
    assert lib.ns_paged_attention_call_workspace(ctypes.byref(a), ctypes.byref(nb), ctypes.byref(nc)) == 0
    ws = torch.empty(max(int(nb.value), 1), dtype=torch.uint8, device=device)
    cnt = torch.zeros(max(int(nc.value), 1), dtype=torch.int32, device=device)
    a.workspace, a.workspace_bytes, a.counters = ws.data_ptr(), int(nb.value), cnt.data_ptr()
    assert lib.ns_paged_attention(ctypes.byref(a), None) == 0
    torch.cuda.synchronize()
    assert status.item() & A.STATUS_BAD_TILE
    ref = PA.paged_attention(**oracle_args(case), terms=True)
    assert_close_to_oracle(out, ref, q.dtype)   # the two valid tiles cover tokens 0..39, the list token 40
    assert torch.count_nonzero(cnt).item() == 0


def test_plan_reused_across_layers_and_refused_for_another_layout(device):
    # one host plan per step serves every layer's call (two caches here): same outputs as the
    # calls that plan for themselves, and a plan of another layout is refused
    case = make_case(95, [1200, 333, 64, 9], [400, 333, 1, 1])
    other = make_case(96, [1200, 333, 64, 9], [400, 333, 1, 1])
    c, o = to_device(case, device), to_device(other, device)
    plan = A.PagedAttentionPlan(c["seq_lens"], c["query_start_loc"], c["query_lens"], 24, 8, device)
    assert plan.tiles is not None and plan.tokens[1] == 2
    outs = []
    for x in (c, o):
        args = (x["query"], x["k_cache"], x["v_cache"], x["block_tables"], x["seq_lens"], x["query_start_loc"],
                x["query_lens"], x["scale"], x["block_size"])
        with_plan = A.paged_attention_hip(*args, plan=plan)
        without = A.paged_attention_hip(*args)
        torch.cuda.synchronize()
        assert torch.equal(with_plan, without)
        outs.append(with_plan)
    for case_, out in zip((case, other), outs):
        assert_close_to_oracle(out, PA.paged_attention(**oracle_args(case_), terms=True), torch.bfloat16)
    bad = A.PagedAttentionPlan(c["seq_lens"], c["query_start_loc"], c["query_lens"], 32, 8, device)
    with pytest.raises(A.PagedAttentionError, match="another batch layout"):
        A.paged_attention_hip(c["query"], c["k_cache"], c["v_cache"], c["block_tables"], c["seq_lens"],
                              c["query_start_loc"], c["query_lens"], c["scale"], c["block_size"], plan=bad)


@pytest.mark.parametrize("d", [128, 64])
def test_prefill_tile_merged_from_many_partitions(device, d):
    # one tile over 9000 positions splits into more partitions than the merge's LDS weight table
    # holds (the one-pass rescaled merge) and a 4000-position tile into fewer (the table)
    case = make_case(97 + d, [9000, 4000], [20, 30], d=d)
    check(case, device)
