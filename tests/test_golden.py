"""The oracle against the committed golden fixtures (CPU).

Checks that every workload regenerates bit-identically (SHA-256 of logits,
parameters, histories and uniforms) and that the oracle still produces the
fixture's token ids, allowed ids, top-k thresholds, kept counts, admissible
top-p cuts and exemption flags, and for the tiny hand-built rows the exact final
probabilities of every admissible cut.
"""
import os
import sys

import numpy as np
import pytest

import golden_data as G
from oracle import sampler_oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
from make_golden import alt_probs_bits as G_alt_probs  # noqa: E402
from make_golden import row_records as G_rows  # noqa: E402

CONFIGS = G.configs()
TINY = G.tiny()


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_config_fixture(name):
    rec = CONFIGS[name]
    w = G.config_workload(rec)
    assert w.digest() == rec["digest"], f"{name}: workload generation changed"
    r = O.sample_workload(w)
    got = G_rows(r)
    for i, (g, e) in enumerate(zip(got, rec["rows"])):
        assert g == e, f"{name} row {i}: {g} != fixture {e}"


@pytest.mark.parametrize("case", TINY, ids=[c["name"] for c in TINY])
def test_tiny_fixture(case):
    w = G.tiny_workload(case)
    r = O.sample(w.rows, w.temperature, w.top_k, w.top_p, w.repetition_penalty, w.histories, w.uniforms)
    for i, e in enumerate(case["expected"]):
        assert int(r.ids[i]) == e["id"], f"{case['name']} row {i}"
        assert r.probs[i].numpy().view(np.uint32).tolist() == e["probs_bits"], f"{case['name']} row {i} probs"
        assert G_alt_probs(r, i) == e["alt_probs_bits"], f"{case['name']} row {i} alternative probs"
    got = G_rows(r)
    for i, e in enumerate(case["expected"]):
        e = {k: v for k, v in e.items() if k not in ("probs_bits", "alt_probs_bits")}
        assert got[i] == e, f"{case['name']} row {i}: {got[i]} != fixture {e}"
