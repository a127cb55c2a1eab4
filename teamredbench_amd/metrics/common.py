"""Built-in metrics over a record's raw counters.

Formulas and names are the reference's (src/teamredbench/metrics/common.py:14-84):
  latency_us           = elapsed_s * 1e6
  hbm_bandwidth_gbps   = moved_bytes / elapsed_s / 1e9
  hbm_efficiency_pct   = hbm_bandwidth_gbps / peak_bandwidth_gbps * 100
  achieved_tops        = achieved_ops / elapsed_s / 1e12
  mfu_pct              = achieved_tops / peak_tops * 100
  payload/bus/link     = collective metrics, kept so suites naming them resolve
Every metric returns None when an input it needs is missing or zero.
"""
from __future__ import annotations

from typing import Any

from teamredbench_amd.registry import register_metric


def _num(raw: dict[str, Any], key: str) -> float | None:
    value = raw.get(key)
    return None if value is None else float(value)


def _per_second(amount: float | None, elapsed: float | None, unit: float) -> float | None:
    """amount / elapsed / unit -- the same operation order as the reference."""
    if amount is None or elapsed is None or elapsed == 0:
        return None
    return amount / elapsed / unit


def _percent(current: float | None, peak: float | None) -> float | None:
    if current is None or peak is None or peak == 0:
        return None
    return current / peak * 100.0


@register_metric("latency_us", "Average iteration latency in microseconds.")
def latency_us(raw: dict[str, Any]) -> float | None:
    elapsed = _num(raw, "elapsed_s")
    return None if elapsed is None else elapsed * 1e6


@register_metric("hbm_bandwidth_gbps", "Device memory bandwidth derived from moved bytes.")
def hbm_bandwidth_gbps(raw: dict[str, Any]) -> float | None:
    return _per_second(_num(raw, "moved_bytes"), _num(raw, "elapsed_s"), 1e9)


@register_metric("hbm_efficiency_pct", "HBM bandwidth as a percentage of configured peak.")
def hbm_efficiency_pct(raw: dict[str, Any]) -> float | None:
    return _percent(hbm_bandwidth_gbps(raw), _num(raw, "peak_bandwidth_gbps"))


@register_metric("payload_bandwidth_gbps", "Collective payload bandwidth in GB/s.")
def payload_bandwidth_gbps(raw: dict[str, Any]) -> float | None:
    return _per_second(_num(raw, "payload_bytes"), _num(raw, "elapsed_s"), 1e9)


@register_metric("bus_bandwidth_gbps", "Collective link bandwidth in GB/s after bus factor.")
def bus_bandwidth_gbps(raw: dict[str, Any]) -> float | None:
    payload = payload_bandwidth_gbps(raw)
    factor = _num(raw, "bus_factor")
    return None if payload is None or factor is None else payload * factor


@register_metric("link_efficiency_pct", "Collective bandwidth as a percentage of configured peak link bandwidth.")
def link_efficiency_pct(raw: dict[str, Any]) -> float | None:
    return _percent(bus_bandwidth_gbps(raw), _num(raw, "peak_link_bandwidth_gbps"))


@register_metric("achieved_tops", "Achieved throughput in tera-ops per second.")
def achieved_tops(raw: dict[str, Any]) -> float | None:
    return _per_second(_num(raw, "achieved_ops"), _num(raw, "elapsed_s"), 1e12)


@register_metric("mfu_pct", "Measured throughput as a percentage of configured peak.")
def mfu_pct(raw: dict[str, Any]) -> float | None:
    return _percent(achieved_tops(raw), _num(raw, "peak_tops"))


@register_metric("gemm_bandwidth_gbps", "Effective GEMM HBM bandwidth: (MK+KN)*in_bytes + MN*out_bytes per call.")
def gemm_bandwidth_gbps(raw: dict[str, Any]) -> float | None:
    return _per_second(_num(raw, "gemm_bytes"), _num(raw, "elapsed_s"), 1e9)
