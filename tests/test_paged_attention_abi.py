"""CPU checks of the paged-attention boundary: the library loads, exports what
include/ns_paged_attention.h declares, its argument struct matches the header, and it refuses
invalid arguments before touching a GPU."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from conftest import ROOT, pkg

PA = pkg("paged_attention")
HEADER = os.path.join(ROOT, "include", "ns_paged_attention.h")


def header_functions():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(ns_\w+)\s*\(", txt, flags=re.M)))


def built():
    if not os.path.exists(PA.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")


def test_header_declares_the_binding_exports():
    assert header_functions() == sorted(PA.EXPORTS)


def test_library_exports_every_header_symbol():
    built()
    lib = ctypes.CDLL(PA.LIB_PATH)
    for name in header_functions():
        assert hasattr(lib, name), name
    assert PA.load().ns_pa_abi_version() == PA.ABI_VERSION


def test_struct_layout_matches_header():
    txt = open(HEADER).read()
    body = txt[txt.index("typedef struct ns_paged_attn_args"):txt.index("} ns_paged_attn_args;")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)   # comments may hold semicolons
    names = []
    for decl in re.findall(r"^\s*([^/{}]+?);", body, flags=re.M):
        names += [n.strip().lstrip("*") for n in re.sub(r"^.*?\b(\w+)\s*(,|$)", r"\1\2", decl, count=1).split(",")]
    assert names == [f[0] for f in PA.NsPagedAttnArgs._fields_]
    # every field's offset and the size, as the C compiler lays the header's struct out
    src = "#include <stdio.h>\n#include <stddef.h>\n#include \"ns_paged_attention.h\"\nint main(void) {\n"
    src += '  printf("%zu\\n", sizeof(ns_paged_attn_args));\n'
    for n in names:
        src += f'  printf("%zu\\n", offsetof(ns_paged_attn_args, {n}));\n'
    src += "  return 0;\n}\n"
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        with open(c, "w") as f:
            f.write(src)
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", "-I", os.path.dirname(HEADER), "-I",
                        os.path.join(rocm, "include"), c, "-o", exe], check=True)
        got = [int(v) for v in subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()]
    assert got[0] == ctypes.sizeof(PA.NsPagedAttnArgs)
    assert got[1:] == [getattr(PA.NsPagedAttnArgs, n).offset for n in names]


def test_plan_tiles_covers_every_token_once():
    """The host plan of a chunked-prefill batch: sequences with several query tokens cut into tiles
    of TILE_COLUMNS // G consecutive tokens of one sequence, every other token listed once, for any G;
    TILE_COLUMNS is the header's NS_PA_TILE_COLUMNS."""
    import numpy as np

    with open(os.path.join(ROOT, "include", "ns_paged_attention.h")) as fh:
        assert int(re.search(r"#define NS_PA_TILE_COLUMNS (\d+)", fh.read()).group(1)) == PA.TILE_COLUMNS

    rng = np.random.default_rng(3)
    for hq, hkv in ((24, 8), (32, 8), (8, 8), (16, 8), (64, 8)):
        qlens = np.concatenate([rng.integers(0, 3, 40), rng.integers(2, 700, 12), [0, 1, 64, 65]])
        rng.shuffle(qlens)
        qsl = np.zeros(qlens.size + 1, dtype=np.int64)
        qsl[1:] = np.cumsum(qlens)
        seq_lens = qlens + rng.integers(0, 3000, qlens.size)
        tiles, tokens = PA.plan_tiles(seq_lens, qsl, qlens, hq, hkv)
        bq = PA.TILE_COLUMNS // (hq // hkv)
        owner = np.full(int(qsl[-1]), -1)
        for s, t0, n in tiles.tolist():
            assert 1 <= n <= bq and qlens[s] >= PA.PREFILL_MIN_QUERY
            assert qsl[s] <= t0 and t0 + n <= qsl[s + 1]
            assert (owner[t0:t0 + n] == -1).all()
            owner[t0:t0 + n] = 1
        for t in tokens.tolist():
            s = int(np.searchsorted(qsl, t, side="right") - 1)
            assert qlens[s] < PA.PREFILL_MIN_QUERY and owner[t] == -1
            owner[t] = 0
        assert (owner >= 0).all()


def test_workspace_sizes():
    built()
    # a grid already wide enough (256 queries x 8 KV heads at one 1024-position partition): no workspace
    assert PA.workspace_bytes(256, 24, 8, 128, 1024) == 0
    # 64 decode rows of 512 positions: 512 workgroups, so split into two 256-position partitions
    # (partials: head_dim + 2 floats per query token, query head and partition)
    assert PA.workspace_bytes(64, 24, 8, 128, 512) == 64 * 24 * 2 * (128 + 2) * 4
    # a single long decode row is split into 64-position partitions: (D + 2) floats per partition and head
    assert PA.workspace_bytes(1, 24, 8, 128, 8192) == 1 * 24 * (8192 // 64) * (128 + 2) * 4
    with pytest.raises(PA.PagedAttentionError, match="multiple"):
        PA.workspace_bytes(1, 24, 7, 128, 16)
    with pytest.raises(PA.PagedAttentionError, match="head_dim"):
        PA.workspace_bytes(1, 24, 8, 96, 16)
    with pytest.raises(PA.PagedAttentionError, match="1, 2, 3, 4 or 8"):
        PA.workspace_bytes(1, 40, 8, 128, 16)


def test_argument_errors_without_a_gpu():
    built()
    lib = PA.load()
    a = PA.NsPagedAttnArgs()
    a.total_q, a.num_seqs, a.num_heads_q, a.num_kv_heads, a.head_dim = 1, 1, 24, 8, 128
    a.block_size, a.num_blocks, a.max_seq_len, a.dtype = 16, 4, 16, PA.NS_PA_DTYPE_BF16
    assert lib.ns_paged_attention(ctypes.byref(a), None) != 0
    assert b"NULL" in lib.ns_pa_last_error()
    a.dtype = 7
    assert lib.ns_paged_attention(ctypes.byref(a), None) != 0
    assert b"dtype" in lib.ns_pa_last_error()
    a.dtype, a.block_size = PA.NS_PA_DTYPE_BF16, 0
    assert lib.ns_paged_attention(ctypes.byref(a), None) != 0
    assert b"block_size" in lib.ns_pa_last_error()
    # an empty batch is a no-op
    a.total_q = 0
    assert lib.ns_paged_attention(ctypes.byref(a), None) == 0
