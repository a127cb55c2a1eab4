"""Launch the stream kernels a fixed number of times for counter collection.

Run under ``rocprofv3 --pmc FETCH_SIZE`` (and, in a second pass,
``--pmc WRITE_SIZE``): every launch is one dispatch whose DRAM traffic the
counters report. The copy launches move a known number of bytes (read n*4,
write n*4), which calibrates the counters; the triad launches are the
workload being measured (read 2*n*4, write n*4).

Two one-direction references for comparing the memory's behaviour by
traffic mix (read latency, requests in flight, write-credit stalls) under
the same counters: ``read`` (torch.sum over b: n*4 bytes read, nothing
written but the sum) and ``write`` (torch's fill_ of a: n*4 bytes written).
They are PyTorch's kernels, not this library's.

    python -m teamredbench_amd.profiling.stream_probe [--elements N] [--launches K]
                                                      [--ops copy,triad,read,write]
                                                      [--configs THREADSxUNROLLxBLOCKS_PER_CU,...]

``--configs`` launches the triad once more per listed launch shape (threads per
block, 16-byte chunks per trip, blocks per CU; set through mb_set_tuning) after
the ops above, for comparing the memory's behaviour as the requests in flight
grow.
"""
from __future__ import annotations

import argparse
import json
import sys


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--elements", type=int, default=1 << 28)
    parser.add_argument("--launches", type=int, default=5)
    parser.add_argument("--ops", default="copy,triad", help="comma-separated subset of copy,triad,read,write")
    parser.add_argument("--configs", default="", help="triad launch shapes THREADSxUNROLLxBLOCKS_PER_CU, comma-separated")
    args = parser.parse_args(argv)
    ops = [o for o in args.ops.split(",") if o]
    if not ops or any(o not in ("copy", "triad", "read", "write") for o in ops):
        parser.error("--ops takes copy, triad, read and/or write")

    import torch

    from teamredbench_amd.native import capi

    torch.cuda.set_device(0)
    lib = capi.load_library()
    n = args.elements
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    b = torch.empty(n, device="cuda").uniform_(-1.0, 1.0, generator=gen)
    c = torch.empty(n, device="cuda").uniform_(-1.0, 1.0, generator=gen)
    a = torch.empty_like(b)
    stream = torch.cuda.current_stream().cuda_stream
    launched = {}
    for name, op in (("copy", capi.OP_COPY), ("triad", capi.OP_TRIAD)):
        if name not in ops:
            continue
        for _ in range(args.launches):
            lib.stream(op, capi.DT_FLOAT32, a.data_ptr(), b.data_ptr(), c.data_ptr(), n, 3.0, 0, stream)
        torch.cuda.synchronize()
        launched[name] = {
            "launches": args.launches,
            "algorithmic_read_bytes": (1 if name == "copy" else 2) * 4 * n,
            "algorithmic_write_bytes": 4 * n,
            "kernel": lib.stream_info(op, capi.DT_FLOAT32, n),
        }
    if "read" in ops:
        for _ in range(args.launches):
            torch.sum(b)
        torch.cuda.synchronize()
        launched["read"] = {"launches": args.launches, "algorithmic_read_bytes": 4 * n, "kernel": "torch.sum"}
    if "write" in ops:
        for _ in range(args.launches):
            a.fill_(0.5)
        torch.cuda.synchronize()
        launched["write"] = {"launches": args.launches, "algorithmic_write_bytes": 4 * n, "kernel": "torch fill_"}
    for shape in filter(None, args.configs.split(",")):
        threads, unroll, bpc = (int(x) for x in shape.split("x"))
        with lib.tuned(stream_threads=threads, stream_unroll=unroll):
            for _ in range(args.launches):
                lib.stream(capi.OP_TRIAD, capi.DT_FLOAT32, a.data_ptr(), b.data_ptr(), c.data_ptr(), n, 3.0, bpc, stream)
            torch.cuda.synchronize()
            launched[f"triad {shape}"] = {"launches": args.launches,
                                          "kernel": lib.stream_info(capi.OP_TRIAD, capi.DT_FLOAT32, n, bpc)}
    print(json.dumps({"elements": n, "cases": launched}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
