"""Loading of the golden fixtures in tests/golden/ (written by tests/golden/make_golden.py)."""
from __future__ import annotations

import importlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
W = importlib.import_module("nanoserve---custom-llm-inference-engine_amd.workloads")
GOLDEN = os.path.join(HERE, "golden")


def configs() -> dict:
    with open(os.path.join(GOLDEN, "configs.json")) as f:
        return json.load(f)


def tiny() -> list:
    with open(os.path.join(GOLDEN, "tiny_cases.json")) as f:
        return json.load(f)


def bits_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


def tiny_workload(case) -> "W.Workload":
    """A float32 workload holding one group of tiny rows."""
    rows = np.stack([bits_f32(r) for r in case["rows_bits"]])
    B = rows.shape[0]
    return W.Workload(name=f"tiny-{case['name']}", vocab=int(case["vocab"]), rows=rows, bf16_bits=None,
                      temperature=np.asarray(case["temperature"], dtype=np.float64),
                      top_k=np.asarray(case["top_k"], dtype=np.int64),
                      top_p=np.asarray(case["top_p"], dtype=np.float64),
                      repetition_penalty=np.asarray(case["repetition_penalty"], dtype=np.float64),
                      histories=[np.asarray(h, dtype=np.int32) for h in case["histories"]],
                      uniforms=np.asarray(case["uniforms"], dtype=np.float32), n_rows_total=B)


def config_workload(rec) -> "W.Workload":
    if rec["cfg"] == "mixed":
        return W.make_mixed_decode(int(rec["batch_arg"]))
    return W.make_workload(int(rec["cfg"]), batch=rec["batch_arg"])
