"""GPU: the logits producer's bf16 output handed to the sampler directly.

The reference's engine upcasts the lm_head output before sampling
(engine.py:235-236: ``compute_logits(...).float()``, then sampler.py:28).  The
kernels read bf16 rows and widen each value exactly, so sampling the GEMM's
bf16 output must match the oracle run on its float32 upcast (the reference's
input), and must give the same ids as the kernels run on that upcast.
"""
import dataclasses

import numpy as np
import pytest
import torch

from conftest import pkg
from parity import PATHS, compare, run_path

W = pkg("workloads")
L = pkg("_lib")
O = pytest.importorskip("oracle.sampler_oracle")

pytestmark = pytest.mark.gpu


def lm_head_workload(w, device, hidden_size=512, seed=0, producer="library"):
    """Workload ``w`` with its logits replaced by a random-init lm_head GEMM's bf16 output:
    hidden (B, H) times an (H, V) weight through the library GEMM, or ``producer="native"``:
    ns_lm_head_bf16 with the same weight in the (V, H) lm_head layout."""
    g = torch.Generator(device=device)
    g.manual_seed(1234 + seed)
    hidden = torch.randn((w.batch, hidden_size), generator=g, device=device).to(torch.bfloat16)
    weight = (torch.randn((hidden_size, w.vocab), generator=g, device=device) * (3.0 / hidden_size ** 0.5)
              ).to(torch.bfloat16)
    if producer == "native":
        logits = L.lm_head_bf16(hidden, weight.t().contiguous())
    else:
        logits = torch.mm(hidden, weight)
    assert logits.dtype == torch.bfloat16 and logits.is_contiguous()
    bits = logits.view(torch.int16).cpu().numpy().view(np.uint16)
    rows = W.bf16_bits_to_f32(bits)
    return dataclasses.replace(w, name=f"{w.name}+lm_head", rows=rows, bf16_bits=bits), logits


@pytest.mark.parametrize("producer", ["library", "native"])
@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("cfg", [1, 2])
def test_bf16_gemm_output_matches_the_upcast(device, cfg, path, producer):
    base = W.make_workload(cfg, batch=64 if cfg == 2 else None)
    w, logits = lm_head_workload(base, device, seed=cfg, producer=producer)
    print(f"[producer] {w.name} B={w.batch} V={w.vocab} path={path} producer={producer}", flush=True)
    g_bf = run_path(w, device, path, logits=logits)
    g_f32 = run_path(w, device, path, logits=logits.float())
    r = O.sample_workload(w)
    for name, g in (("bf16", g_bf), ("f32", g_f32)):
        fails, stats = compare(g, r)
        print(f"[producer] {name}: {stats}", flush=True)
        assert not fails, f"{name} input:\n" + "\n".join(fails)
    keep = ~np.asarray(r.exempt, dtype=bool) | np.asarray(r.greedy, dtype=bool)
    assert np.array_equal(g_bf["ids"][keep], g_f32["ids"][keep])
