"""MI355X-native token sampler for NanoServe.

A drop-in for ``nanoserve.scheduler.sampler.Sampler`` (sampler.py:17-89): the
``Sampler`` class keeps the reference's constructor and ``sample()`` surface and
runs the whole sampling step in hand-written gfx950 HIP kernels reached through
the C ABI declared in ``include/ns_sampling.h``.

The directory name is not a Python identifier; import it with
``importlib.import_module("nanoserve---custom-llm-inference-engine_amd")`` (the
repository root on ``sys.path``).
"""
from .config import SamplingParams
from .sampler import DeviceHistories, PackedRows, ReadbackRing, SampledIds, Sampler, effective_temperature

__all__ = ["Sampler", "SamplingParams", "PackedRows", "DeviceHistories", "SampledIds", "ReadbackRing",
           "effective_temperature"]
