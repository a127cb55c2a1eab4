"""teamredbench_amd -- MI355X-native stream and GEMM backends for TeamRedBench.

The hot path (``backend: native`` of the ``hbm`` and ``mfu`` benchmarks) runs
hand-written gfx950 HIP kernels from ``libmi355bench.so`` through a C ABI
(include/mi355bench.h) bound with ctypes; PyTorch-ROCm only allocates device
buffers and provides the stream. The surrounding registry / suite / record /
metric API keeps the reference's names and semantics
(src/teamredbench/registry.py, runner.py, benchmarks/base.py).
"""

__all__ = ["__version__"]

__version__ = "0.1.0"
