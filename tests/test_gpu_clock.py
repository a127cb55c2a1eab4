"""Clock stamps (mb_clock_stamp) on the GPU (-m gpu): two stamps around a region of work give every XCD's
mean shader clock over it, within the part's clock range."""
from __future__ import annotations

import pytest
import torch

from teamredbench_amd.native import capi
from teamredbench_amd.profiling.clock import ClockWindow

pytestmark = pytest.mark.gpu


def test_clock_window_over_a_triad_loop(lib):
    n = 1 << 26
    b = torch.rand(n, device="cuda")
    c = torch.rand(n, device="cuda")
    a = torch.empty_like(b)
    stream = torch.cuda.current_stream().cuda_stream
    window = ClockWindow(torch, lib, stream)
    print("[clock] stamps around 40 triad launches over 2^26 fp32 elements", flush=True)
    window.start()
    for _ in range(40):
        lib.stream(capi.OP_TRIAD, capi.DT_FLOAT32, a.data_ptr(), b.data_ptr(), c.data_ptr(), n, 3.0, 0, stream)
    window.stop()
    torch.cuda.synchronize()
    summary = window.summary()
    print(f"[clock] {summary}", flush=True)
    assert summary["available"], summary
    props = torch.cuda.get_device_properties(0)
    xcds = {str(x) for x in range(8)} if props.multi_processor_count == 256 else None
    if xcds is not None:
        assert set(summary["gfxclk_mhz_per_xcd"]) == xcds
    assert all(100.0 <= v <= 2600.0 for v in summary["gfxclk_mhz_per_xcd"].values()), summary
    assert summary["window_s"] > 0


def test_clock_stamp_rejects_a_null_buffer(lib):
    with pytest.raises(capi.NativeLibraryError) as err:
        lib.clock_stamp(0, None)
    assert err.value.status == capi.MB_ERR_INVALID_ARG
