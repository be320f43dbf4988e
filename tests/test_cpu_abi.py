"""CPU-only checks of the boundary: the C-ABI library loads, exports every symbol
declared in include/ns_sampling.h, reports its ABI version and validates
arguments without touching a GPU; the host packing mirrors the reference."""
import ctypes
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

from conftest import ROOT, pkg

L = pkg("_lib")
S = pkg("sampler")
C = pkg("config")

HEADER = os.path.join(ROOT, "include", "ns_sampling.h")


def header_functions():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(ns_\w+)\s*\(", txt, flags=re.M)))


def test_header_declares_the_binding_exports():
    assert header_functions() == sorted(L.EXPORTS)


def test_library_exports_every_header_symbol():
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(L.LIB_PATH)
    for name in header_functions():
        assert hasattr(lib, name), name
    assert L.load().ns_abi_version() == L.ABI_VERSION


def test_struct_layout_matches_header():
    # ns_sample_args field order/types must match the C declaration
    txt = open(HEADER).read()
    body = txt[txt.index("typedef struct ns_sample_args"):txt.index("} ns_sample_args;")]
    names = re.findall(r"^\s*[\w\s\*]+?\b(\w+);", body, flags=re.M)
    assert names == [f[0] for f in L.NsSampleArgs._fields_]
    # every field's offset and the size, as the C compiler lays the header's struct out
    src = "#include <stdio.h>\n#include <stddef.h>\n#include \"ns_sampling.h\"\nint main(void) {\n"
    src += '  printf("%zu\\n", sizeof(ns_sample_args));\n'
    for n in names:
        src += f'  printf("%zu\\n", offsetof(ns_sample_args, {n}));\n'
    src += "  return 0;\n}\n"
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        with open(c, "w") as f:
            f.write(src)
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", "-I", os.path.dirname(HEADER), "-I",
                        os.path.join(rocm, "include"), c, "-o", exe], check=True)
        got = [int(v) for v in subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()]
    assert got[0] == ctypes.sizeof(L.NsSampleArgs)
    assert got[1:] == [getattr(L.NsSampleArgs, n).offset for n in names]


def test_lds_bytes_and_argument_errors():
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("library not built")
    assert L.lds_bytes(128256, 2048) <= 160 * 1024
    assert L.lds_bytes(262144, 8192) <= 160 * 1024
    with pytest.raises(L.SamplerLibraryError, match="vocab"):
        L.lds_bytes(0, 0)
    with pytest.raises(L.SamplerLibraryError, match="max_hist"):
        L.lds_bytes(1000, L.NS_MAX_HISTORY + 1)
    # histories past NS_LDS_HISTORY take no more LDS; their distinct ids (and the tail) go to
    # a workspace region of min(max_hist, vocab) + 8 entries of 8 bytes per row
    assert L.lds_bytes(128256, L.NS_MAX_HISTORY) == L.lds_bytes(128256, L.NS_LDS_HISTORY)
    for dt in (L.NS_DTYPE_F32, L.NS_DTYPE_BF16):
        base = L.workspace_bytes(256, 128256, dt)
        assert L.workspace_bytes(256, 128256, dt, L.NS_LDS_HISTORY) == base
        assert L.workspace_bytes(256, 128256, dt, 16384) == base + 256 * (16384 + 8) * 8
        assert L.workspace_bytes(3, 1000, dt, L.NS_MAX_HISTORY) == L.workspace_bytes(3, 1000, dt) + 24320   # align256(3 * 1008 * 8)
    with pytest.raises(L.SamplerLibraryError, match="max_hist"):
        L.workspace_bytes(8, 1000, L.NS_DTYPE_F32, L.NS_MAX_HISTORY + 1)
    lib = L.load()
    a = L.NsSampleArgs()
    a.n_sample = 1
    assert lib.ns_sample(ctypes.byref(a), None) == 1
    assert "NULL" in L.last_error()
    a.n_sample = 0
    assert lib.ns_sample(ctypes.byref(a), None) == 0


def test_history_state_layout_and_argument_errors():
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("library not built")
    # int32 lengths padded to 256 bytes, then n_slots * capacity int32 ids
    assert L.hist_state_bytes(3, 100) == 256 + 3 * 100 * 4
    assert L.hist_state_bytes(64, 8192) == 256 + 64 * 8192 * 4
    assert L.hist_state_bytes(4, 16384) == 256 + 4 * 16384 * 4
    with pytest.raises(L.SamplerLibraryError, match="hist_capacity"):
        L.hist_state_bytes(4, L.NS_MAX_HISTORY + 1)
    with pytest.raises(L.SamplerLibraryError, match="2\\^31"):
        L.hist_state_bytes(4096, L.NS_MAX_HISTORY)
    with pytest.raises(L.SamplerLibraryError, match="hist_n_slots"):
        L.hist_state_bytes(0, 10)
    lib = L.load()
    assert lib.ns_hist_assign(None, 4, 10, 0, None, 0, None) == 1 and "state" in L.last_error()
    assert lib.ns_hist_assign(256, 4, 10, 4, None, 0, None) == 1 and "slot" in L.last_error()
    assert lib.ns_hist_assign(256, 4, 10, 0, None, 11, None) == 1 and "capacity" in L.last_error()
    assert lib.ns_hist_append(256, 4, 10, None, None, 2, None, None) == 1 and "NULL" in L.last_error()
    assert lib.ns_hist_append(256, 4, 10, None, None, 0, None, None) == 0
    # the device histories exclude the CSR ones; a slot table is required (checked before any launch)
    a = L.NsSampleArgs()
    a.n_sample, a.dtype, a.vocab, a.row_stride, a.n_rows_total = 1, L.NS_DTYPE_F32, 64, 64, 1
    a.logits = a.temperature = a.top_k = a.top_p = a.rep_penalty = a.uniforms = a.out_ids = 256
    a.hist_state, a.hist_n_slots, a.hist_capacity = 256, 4, 16
    a.hist_offsets, a.hist_ids = 512, 768
    assert lib.ns_sample(ctypes.byref(a), None) == 1 and "excludes" in L.last_error()
    a.hist_offsets = a.hist_ids = None
    assert lib.ns_sample(ctypes.byref(a), None) == 1 and "hist_slot" in L.last_error()
    # appending the sampled ids in the kernels needs the device-resident histories
    a.hist_state, a.hist_n_slots, a.hist_capacity, a.hist_append = None, 0, 0, 1
    assert lib.ns_sample(ctypes.byref(a), None) == 1 and "hist_append needs hist_state" in L.last_error()


def test_packing_with_history_slots():
    P = C.SamplingParams
    params = [P(repetition_penalty=1.2), P(), P(temperature=0.0)]
    pk = S.PackedRows(params, None, vocab=10, slots=np.array([2, -1, 0]), slot_max_hist=7)
    assert pk.hist_offsets is None and pk.hist_ids is None and pk.max_hist == 7
    d = pk.to_device("cpu")
    assert d["hist_slot"].tolist() == [2, -1, 0] and d["hist_offsets"] is None and d["hist_ids"] is None
    assert d["top_k"].tolist() == [-1, -1, -1]


def test_packing_follows_reference_rules():
    P = C.SamplingParams
    params = [P(temperature=0.0), P(temperature=1e-9), P(temperature=-2.0), P(temperature=0.7, top_k=2**40),
              P(top_k=-5, top_p=0.95, repetition_penalty=1.2), P(repetition_penalty=1.0)]
    hist = [[1, 2], [3], [], [4, 4, 4], [9, 0, 9], [7]]
    pk = S.PackedRows(params, hist, vocab=10)
    # sampler.py:42: t' = max(t, 1e-6) if t > 0 else 1.0; greedy encoded as 0
    assert pk.temperature.tolist() == [0.0, np.float32(1e-6), 1.0, np.float32(0.7), 1.0, 1.0]
    assert pk.top_k.tolist() == [-1, -1, -1, 2**31 - 1, -1, -1]
    # only penalised rows carry their history (sampler.py:33)
    assert pk.hist_offsets.tolist() == [0, 0, 0, 0, 0, 3, 3]
    assert pk.hist_ids.tolist() == [9, 0, 9]
    assert pk.max_hist == 3
    with pytest.raises(IndexError):
        S.PackedRows([P(repetition_penalty=1.1)], [[10]], vocab=10)


def test_sampling_params_match_reference_defaults():
    p = C.SamplingParams()
    assert (p.max_tokens, p.temperature, p.top_p, p.top_k, p.repetition_penalty, p.ignore_eos, p.seed) == \
        (128, 1.0, 1.0, -1, 1.0, False, None)
    assert p.stop_token_ids == [] and p.stop == []


def test_aligned_rows_pads_misaligned_vocab():
    import torch
    L = pkg("_lib")
    x = torch.arange(3 * 17, dtype=torch.float32).reshape(3, 17)
    y, idx = L.aligned_rows(x, None)
    assert y.shape == (3, 17) and y.stride(0) == 20 and idx is None
    assert torch.equal(y, x)
    sel = torch.tensor([2, 0], dtype=torch.int64)
    y2, idx2 = L.aligned_rows(x, sel)
    assert idx2.tolist() == [0, 1] and torch.equal(y2, x[[2, 0]]) and (y2.stride(0) * 4) % 16 == 0
    # indices outside the tensor: the gather reads clamped rows and the kernel index marks them -1
    bad = torch.tensor([1, -1, 3, 2, -(2 ** 40)], dtype=torch.int64)
    y3, idx3 = L.aligned_rows(x, bad)
    assert idx3.tolist() == [0, -1, -1, 3, -1]
    assert torch.equal(y3[0], x[1]) and torch.equal(y3[3], x[2])
    b = torch.zeros(4, 24, dtype=torch.bfloat16)            # 48-byte rows: already aligned
    yb, ib = L.aligned_rows(b, sel)
    assert yb.data_ptr() == b.data_ptr() and ib is sel
    b9 = torch.ones(2, 9, dtype=torch.bfloat16)             # 18-byte rows: padded to 16 elements
    yb9, _ = L.aligned_rows(b9, None)
    assert yb9.stride(0) == 16 and torch.equal(yb9, b9)


def test_lm_head_argument_errors():
    """ns_lm_head_bf16 rejects bad shapes, strides and alignment before any launch; an empty
    product is a no-op."""
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("library not built")
    lib = L.load()
    f = lib.ns_lm_head_bf16
    h, w, o = 4096, 8192, 12288    # 16-byte aligned stand-in addresses (never dereferenced)
    assert f(None, 64, 4, None, w, 64, o, 64, 1, 1, 64, None) == 1 and "NULL" in L.last_error()
    assert f(h, 128, 4, None, w, 128, o, 64, 1, 1, 100, None) == 1 and "multiple of 64" in L.last_error()
    assert f(h, 60, 4, None, w, 128, o, 64, 1, 1, 64, None) == 1 and "ld_hidden" in L.last_error()
    assert f(h, 64, 4, None, w, 64, o, 4, 1, 8, 64, None) == 1 and "ld_logits" in L.last_error()
    assert f(h + 8, 64, 4, None, w, 64, o, 64, 1, 1, 64, None) == 2 and "aligned" in L.last_error()   # NS_ERR_ALIGN
    assert f(h, 64, 4, None, w, 64, o, 64, -1, 1, 64, None) == 1
    assert f(h, 64, 4, None, w, 1 << 24, o, 64, 1, 1, 64, None) == 1 and "ld_weight" in L.last_error()
    assert f(h, 64, 4, None, w, 64, o, 64, 0, 5, 64, None) == 0      # nothing to compute
    assert f(h, 64, 4, None, w, 64, o, 64, 3, 0, 64, None) == 0
    nb = ctypes.c_uint64(0)
    assert lib.ns_lm_head_packed_bytes(128256, 2048, ctypes.byref(nb)) == 0
    assert nb.value == 501 * 32 * 256 * 64 * 2          # 256-row blocks x 64-wide stages x 32 KB
    assert lib.ns_lm_head_packed_bytes(257, 64, ctypes.byref(nb)) == 0 and nb.value == 2 * 32768
    assert lib.ns_lm_head_packed_bytes(10, 100, ctypes.byref(nb)) == 1
    assert lib.ns_lm_head_pack_bf16(None, 64, 10, 64, h, None) == 1 and "NULL" in L.last_error()
    assert lib.ns_lm_head_bf16_packed(h, 64, 4, None, w, 32768, o, 64, 1, 1, 65, None) == 1
    # a buffer packed for another shape is refused before any launch
    assert lib.ns_lm_head_bf16_packed(h, 64, 4, None, w, 32768, o, 300, 1, 300, 64, None) == 1
    assert "packed_bytes" in L.last_error()
    assert f(h, 64, 0, None, w, 64, o, 64, 1, 1, 64, None) == 1 and "n_hidden" in L.last_error()
    assert f(h, 64, 2, None, w, 64, o, 64, 3, 1, 64, None) == 1 and "n_hidden" in L.last_error()
