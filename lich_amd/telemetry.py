"""GPU telemetry and a thermal guard for sustained runs on AMD GPUs.

The reference samples ``nvidia-smi`` (``src/ipc_tilelang/thermal.py:61-84``) and
pauses the training loop while the GPU is too hot or thermally throttled
(``ThermalGuard``, ``thermal.py:87-166``).  Here the sample comes from
``amd-smi metric -g <i> -t -p -c -u --json`` (ROCm's system-management CLI):
junction (hotspot) and memory temperature, socket power, the current GFX clock
of every XCD, the memory clock, GFX / memory-controller activity and the
throttle status.  Sampling is rate-limited off the hot path (one cached sample
per ``telemetry_interval_s``), the guard never changes any device setting, and
a missing or failing ``amd-smi`` yields an all-``None`` sample, which never
pauses.
"""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import time
from dataclasses import dataclass
from typing import Any

AMD_SMI_ARGS = ("metric", "-t", "-p", "-c", "-u", "--json")


@dataclass(frozen=True)
class Telemetry:
    temperature_c: float | None       # junction (hotspot) temperature
    power_w: float | None             # socket power
    clock_gfx_mhz: float | None       # mean current GFX clock over the XCDs
    clock_mem_mhz: float | None
    util_gpu_pct: float | None        # GFX activity
    util_mem_pct: float | None        # memory-controller activity
    throttle_status: str | None = None
    clock_gfx_max_mhz: float | None = None
    temperature_mem_c: float | None = None

    @property
    def clock_sm_mhz(self) -> float | None:
        """The reference's field name for the shader clock."""
        return self.clock_gfx_mhz

    def _status(self) -> str:
        s = (self.throttle_status or "").upper()
        return "" if s in ("", "N/A", "NONE", "UNTHROTTLED", "0") else s

    @property
    def thermal_throttle(self) -> bool:
        return "THERM" in self._status() or "TEMP" in self._status()

    @property
    def power_limited(self) -> bool:
        s = self._status()
        return "POWER" in s or "PPT" in s

    @property
    def hardware_slowdown(self) -> bool:
        s = self._status()
        return "PROCHOT" in s or "HW" in s or "VR" in s


def _value(node: Any) -> float | None:
    """``{"value": v, "unit": u}`` or a bare number -> float; "N/A" -> None."""
    if isinstance(node, dict):
        node = node.get("value")
    if node is None or isinstance(node, bool):
        return None
    try:
        return float(node)
    except (TypeError, ValueError):
        return None


def parse_amd_smi_metric(payload: Any, index: int = 0) -> Telemetry:
    """Telemetry from the JSON of ``amd-smi metric ... --json`` (a dict for
    one GPU, a list of them, or ``{"gpu_data": [...]}``)."""
    if isinstance(payload, dict) and "gpu_data" in payload:
        payload = payload["gpu_data"]
    if isinstance(payload, list):
        match = [g for g in payload if isinstance(g, dict) and g.get("gpu") == index]
        payload = match[0] if match else (payload[0] if payload else {})
    if not isinstance(payload, dict):
        return Telemetry(None, None, None, None, None, None)
    temp = payload.get("temperature") or {}
    power = payload.get("power") or {}
    clock = payload.get("clock") or {}
    usage = payload.get("usage") or {}
    gfx = [_value((v or {}).get("clk")) for k, v in clock.items() if k.startswith("gfx_") and isinstance(v, dict)]
    gfx = [g for g in gfx if g is not None]
    gfx_max = [_value((v or {}).get("max_clk")) for k, v in clock.items() if k.startswith("gfx_") and isinstance(v, dict)]
    gfx_max = [g for g in gfx_max if g is not None]
    mem = clock.get("mem_0") if isinstance(clock.get("mem_0"), dict) else {}
    hot = _value(temp.get("hotspot"))
    if hot is None:
        hot = _value(temp.get("edge"))
    status = power.get("throttle_status")
    return Telemetry(
        temperature_c=hot,
        power_w=_value(power.get("socket_power")),
        clock_gfx_mhz=(sum(gfx) / len(gfx)) if gfx else None,
        clock_mem_mhz=_value(mem.get("clk")),
        util_gpu_pct=_value(usage.get("gfx_activity")),
        util_mem_pct=_value(usage.get("umc_activity")),
        throttle_status=None if status is None else str(status),
        clock_gfx_max_mhz=max(gfx_max) if gfx_max else None,
        temperature_mem_c=_value(temp.get("mem")),
    )


def read_telemetry(index: int = 0, *, timeout_s: float = 10.0) -> Telemetry:
    exe = shutil.which("amd-smi") or ("/opt/rocm/bin/amd-smi" if os.path.exists("/opt/rocm/bin/amd-smi") else None)
    empty = Telemetry(None, None, None, None, None, None)
    if not exe:
        return empty
    try:
        p = subprocess.run([exe, AMD_SMI_ARGS[0], "-g", str(int(index)), *AMD_SMI_ARGS[1:]],
                           capture_output=True, text=True, check=False, timeout=timeout_s)
    except (OSError, subprocess.TimeoutExpired):
        return empty
    if p.returncode != 0 or not p.stdout.strip():
        return empty
    try:
        return parse_amd_smi_metric(json.loads(p.stdout), index)
    except ValueError:
        return empty


class ThermalGuard:
    """Workload-side thermal governor (reference ``ThermalGuard``): call
    ``wait_until_safe()`` between batches; it returns at once unless the
    junction temperature is above ``max_temp_c`` or a thermal throttle is
    reported, and then polls every ``poll_s`` until the temperature is back
    under ``resume_temp_c`` (hysteresis).  ``reader`` replaces the amd-smi
    query (tests, other telemetry sources)."""

    def __init__(self, *, max_temp_c: float = 95.0, resume_temp_c: float | None = None, poll_s: float = 0.5,
                 telemetry_interval_s: float = 1.0, device_index: int = 0, reader=None):
        self.max_temp_c = float(max_temp_c)
        self.resume_temp_c = float(resume_temp_c if resume_temp_c is not None else max_temp_c - 4.0)
        self.poll_s = float(poll_s)
        self.telemetry_interval_s = float(telemetry_interval_s)
        self.device_index = int(device_index)
        self._reader = reader or (lambda: read_telemetry(self.device_index))
        self._last_query_monotonic = -float("inf")
        self._cached: Telemetry | None = None
        self.pauses = 0

    def sample(self, *, force: bool = False) -> Telemetry:
        now = time.monotonic()
        if not force and self._cached is not None and now - self._last_query_monotonic < self.telemetry_interval_s:
            return self._cached
        self._cached = self._reader()
        self._last_query_monotonic = now
        return self._cached

    def _hot(self, t: Telemetry, limit: float) -> bool:
        return t.temperature_c is not None and t.temperature_c > limit

    def wait_until_safe(self, *, verbose: bool = False, max_wait_s: float | None = None) -> Telemetry:
        last = self.sample()
        if not self._hot(last, self.max_temp_c) and not last.thermal_throttle:
            return last
        self.pauses += 1
        start = time.monotonic()
        while self._hot(last, self.resume_temp_c) or last.thermal_throttle:
            if verbose:
                reasons = []
                if self._hot(last, self.resume_temp_c):
                    reasons.append(f"{last.temperature_c:.1f}C > resume {self.resume_temp_c:.1f}C")
                if last.thermal_throttle:
                    reasons.append(f"thermal throttle ({last.throttle_status})")
                print("[thermal-guard] pausing: " + "; ".join(reasons), flush=True)
            if max_wait_s is not None and time.monotonic() - start >= max_wait_s:
                break
            time.sleep(self.poll_s)
            last = self.sample(force=True)
        return last

    def check(self, *, force: bool = False) -> Telemetry:
        return self.sample(force=force)

    def assert_no_thermal_throttle(self) -> Telemetry:
        t = self.sample(force=True)
        if t.thermal_throttle:
            raise RuntimeError(f"GPU thermal throttle is active: status={t.throttle_status}, "
                               f"temperature={t.temperature_c}")
        return t

    @staticmethod
    def format_status(t: Telemetry) -> str:
        temp = "n/a" if t.temperature_c is None else f"{t.temperature_c:.1f}C"
        power = "n/a" if t.power_w is None else f"{t.power_w:.1f}W"
        gfx = "n/a" if t.clock_gfx_mhz is None else f"{t.clock_gfx_mhz:.0f}MHz"
        status = "n/a" if t.throttle_status is None else t.throttle_status
        flags = [name for name, on in (("power-cap", t.power_limited), ("thermal-throttle", t.thermal_throttle),
                                       ("hw-slowdown", t.hardware_slowdown)) if on]
        suffix = " [" + ",".join(flags) + "]" if flags else ""
        return f"temp={temp} power={power} gfx={gfx} throttle={status}{suffix}"
