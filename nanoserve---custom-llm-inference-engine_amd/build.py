"""Build the gfx950 sampler library in-tree: csrc/*.hip -> libns_sampling.so.

    python build.py            # from the package directory, or
    python -c "import build; build.build()"

hipcc flags: gfx950 only, -O3, no fast-math, no FMA contraction (the sampler's
float arithmetic must round exactly as the reference's separate torch ops),
packed-fp32 instruction selection disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "ns_sample.hip")
OUT = os.path.join(HERE, "libns_sampling.so")
# paged attention (its own ABI, include/ns_paged_attention.h)
PA_SRC = os.path.join(HERE, "csrc", "ns_paged_attention.hip")
PA_OUT = os.path.join(HERE, "libns_paged_attention.so")
# the benchmark's bandwidth reference (not part of the sampler's ABI)
PROBE_SRC = os.path.join(HERE, "csrc", "ns_probe.hip")
PROBE_OUT = os.path.join(HERE, "libns_probe.so")
# the sampler with the top-k kernel's phase stamps (bench.py --phase-stamps; never loaded by
# the package)
STAMPS_OUT = os.path.join(HERE, "libns_sampling_stamps.so")
ARCH = os.environ.get("NS_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _command(src: str, out: str, defines=()) -> list:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        # every atomic on a uniform address is aggregated in the source already (one lane per
        # wave); the compiler's own aggregation only wraps those single-lane atomics in
        # another exec-mask count (measured: the wide path 5-7% faster without it)
        "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
        "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
        *[f"-D{d}" for d in defines], src, "-o", out + ".tmp",
    ]


def build(verbose: bool = False) -> str:
    """Compile every library, the four hipcc processes side by side."""
    jobs = [(SRC, OUT, ()), (PA_SRC, PA_OUT, ()), (PROBE_SRC, PROBE_OUT, ()),
            (SRC, STAMPS_OUT, ("NS_PHASE_STAMPS",))]
    procs = []
    for src, out, defines in jobs:
        cmd = _command(src, out, defines)
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((out, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for out, proc in procs:
        log, _ = proc.communicate()
        if proc.returncode != 0:
            sys.stderr.write(log)
            failed.append(os.path.basename(out))
        else:
            os.replace(out + ".tmp", out)
    if failed:
        raise RuntimeError(f"hipcc failed for {', '.join(failed)}")
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
