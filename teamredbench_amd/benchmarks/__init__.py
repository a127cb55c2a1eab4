"""Built-in benchmark plugins: ``hbm`` (stream) and ``mfu`` (GEMM)."""
