"""GPU: ns_sample_noalloc, the entry point that allocates nothing (its workspace is the
library's fixed device array), against ns_sample with a caller workspace.

Two calls in a row through the C ABI -- the chunked-prefill batch (320 of 4096 rows, mixed
parameters: the largest workspace of the benchmark shapes) and then the smaller 8-row
batch -- each compared with ns_sample on the same inputs: ids, probabilities and
diagnostics bit for bit (the same kernels run on the same data).  A call whose workspace
exceeds the array is refused with a clear error and launches nothing.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import pkg
from parity import params_of

W = pkg("workloads")
L = pkg("_lib")
S = pkg("sampler")

pytestmark = pytest.mark.gpu


def _args(w, device, mode, keep):
    """ns_sample_args over workload w (tensors kept alive in `keep`); no workspace."""
    packed = S.PackedRows(params_of(w), w.histories, w.vocab)
    d = packed.to_device(device)
    logits = w.device_logits(device)
    B, V = w.batch, w.vocab
    u = torch.from_numpy(np.asarray(w.uniforms, dtype=np.float32)).to(device)
    sidx = torch.from_numpy(w.sample_indices).to(device) if w.sample_indices is not None else None
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    probs = torch.zeros((B, V), dtype=torch.float32, device=device)
    info = torch.zeros((B, L.NS_INFO_WORDS), dtype=torch.int32, device=device)
    keep += [packed, d, logits, u, sidx, out, probs, info]
    a = L.NsSampleArgs()
    a.logits = logits.data_ptr()
    a.dtype = L.NS_DTYPE_BF16 if logits.dtype == torch.bfloat16 else L.NS_DTYPE_F32
    a.n_sample = B
    a.n_rows_total = int(logits.shape[0])
    a.vocab = V
    a.row_stride = int(logits.stride(0))
    a.sample_idx = 0 if sidx is None else sidx.data_ptr()
    a.temperature = d["temperature"].data_ptr()
    a.top_k = d["top_k"].data_ptr()
    a.top_p = d["top_p"].data_ptr()
    a.rep_penalty = d["rep_penalty"].data_ptr()
    a.hist_offsets = 0 if d["hist_offsets"] is None else d["hist_offsets"].data_ptr()
    a.hist_ids = 0 if d["hist_ids"] is None else d["hist_ids"].data_ptr()
    a.max_hist = packed.max_hist
    a.uniforms = u.data_ptr()
    a.out_ids = out.data_ptr()
    a.out_probs = probs.data_ptr()
    a.out_info = info.data_ptr()
    a.mode = mode
    a.row_kinds = packed.row_kinds if mode == L.NS_MODE_AUTO else 0
    return a, out, probs, info


def _run(w, device, mode, noalloc):
    lib = L.load()
    keep = []
    a, out, probs, info = _args(w, device, mode, keep)
    stream = ctypes.c_void_p(int(torch.cuda.current_stream(device).cuda_stream))
    if noalloc:
        rc = lib.ns_sample_noalloc(ctypes.byref(a), stream)
    else:
        ws = L.workspace_for(device, w.batch, w.vocab, a.dtype)
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()
        rc = lib.ns_sample(ctypes.byref(a), stream)
    assert rc == 0, L.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy(), probs.cpu(), info.cpu().numpy()


@pytest.mark.parametrize("mode", [L.NS_MODE_SEGMENTED, L.NS_MODE_AUTO], ids=["segmented", "auto"])
def test_noalloc_matches_workspace_call(device, mode):
    for cfg in (4, 0):   # the larger workspace first, then a smaller input on the same scratch
        w = W.make_workload(cfg)
        need = L.workspace_bytes(w.batch, w.vocab, L.NS_DTYPE_F32)
        assert need <= L.NS_NOALLOC_SCRATCH_BYTES
        print(f"[noalloc] {w.name} B={w.batch} mode={mode} workspace {need} bytes", flush=True)
        ids_a, probs_a, info_a = _run(w, device, mode, noalloc=False)
        ids_b, probs_b, info_b = _run(w, device, mode, noalloc=True)
        assert np.array_equal(ids_a, ids_b), np.nonzero(ids_a != ids_b)[0][:8]
        assert torch.equal(probs_a, probs_b)
        assert np.array_equal(info_a, info_b)


def test_noalloc_refuses_oversize_workspace(device):
    """1024 bf16 rows need more workspace than the scratch: refused, nothing written."""
    B, V = 1024, 128256
    assert L.workspace_bytes(B, V, L.NS_DTYPE_BF16) > L.NS_NOALLOC_SCRATCH_BYTES
    lib = L.load()
    logits = torch.zeros((B, V), dtype=torch.bfloat16, device=device)
    z = torch.ones(B, dtype=torch.float32, device=device)
    k = torch.full((B,), 50, dtype=torch.int32, device=device)
    u = torch.full((B,), 0.5, dtype=torch.float32, device=device)
    out = torch.full((B,), -7, dtype=torch.int64, device=device)
    a = L.NsSampleArgs()
    a.logits = logits.data_ptr(); a.dtype = L.NS_DTYPE_BF16; a.n_sample = B; a.n_rows_total = B
    a.vocab = V; a.row_stride = V; a.temperature = z.data_ptr(); a.top_k = k.data_ptr(); a.top_p = z.data_ptr()
    a.rep_penalty = z.data_ptr(); a.uniforms = u.data_ptr(); a.out_ids = out.data_ptr()
    a.mode = L.NS_MODE_SEGMENTED
    rc = lib.ns_sample_noalloc(ctypes.byref(a), ctypes.c_void_p(int(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    assert rc == 1 and "scratch" in L.last_error()
    assert int(out[0]) == -7
    # a caller workspace is refused too
    a.workspace = logits.data_ptr()
    a.workspace_bytes = 256
    a.n_sample = 8
    rc = lib.ns_sample_noalloc(ctypes.byref(a), ctypes.c_void_p(int(torch.cuda.current_stream().cuda_stream)))
    assert rc == 1 and "workspace must be NULL" in L.last_error()
