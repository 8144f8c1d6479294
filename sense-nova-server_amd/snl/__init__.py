"""MI355X-native MTP speculative decode step (Python side of the C ABI in include/snl.h).

`Engine` mirrors the reference's Engine API (src/engine.rs) over libsnl.so; `generate` runs the
greedy MTP loop of src/worker.rs:123-255 inside the library, and `Worker` adds the worker's
prefix cache (src/worker.rs:115-174).  Nothing here computes on the CPU:
every call goes to the HIP library, and loading fails loudly when it is missing.
"""
from .config import ModelConfig, SnlConfig, nine_b_config, tiny_config  # noqa: F401
from .engine import Engine, Rng, Sampler, Sampling, SnlError, Worker, lib, kernels  # noqa: F401
