"""Per-operation profiling of the Context mirror, as Kidi's KIDI_PROFILE_OPS (src/kidi/ops/context.cpp:117-133,
:406-438, :450-455, :502-515).

KIDI_PROFILE_OPS=host times each call on the host; =sync also synchronizes the stream after every call and times
the wait. KIDI_PROFILE_OPS_SKIP=n leaves the first n requests (phases "encoder" / "gemma4_request") unprofiled.
Calls aggregate under the reference's key "phase=...|op=...|shapes=[..];[..]|attrs=..,"; the report lines are the
reference's ("kidi_op|device=...|mode=...|<key>|calls=..|prepare_ns=..|dispatch_ns=..|run_ns=..|wait_ns=..|
allocations=..|allocated_bytes=..|output_bytes=..") with one field more, device_ns: the GPU time between two HIP
events recorded on the stream around the call's kernels. Context.synchronize adds "kidi_op_sync|device=..|phase=..|
calls=..|wait_ns=..".
"""

from __future__ import annotations

import os
import sys
import time
from contextlib import contextmanager

import torch


def profile_key(phase: str, op: str, shapes, attrs) -> str:
    """The reference's aggregation key (context.cpp:421-429): every extent and attribute followed by a comma."""
    s = "".join(f"[{''.join(f'{int(d)},' for d in shape)}]" if i == 0 else f";[{''.join(f'{int(d)},' for d in shape)}]"
                for i, shape in enumerate(shapes))
    return f"phase={phase}|op={op}|shapes={s}|attrs={''.join(f'{int(a)},' for a in attrs)}"


class Profiler:
    FIELDS = ("calls", "prepare_ns", "dispatch_ns", "run_ns", "wait_ns", "allocations", "allocated_bytes", "output_bytes")

    def __init__(self, device, env=None):
        env = os.environ if env is None else env
        mode = env.get("KIDI_PROFILE_OPS", "")
        self.device = device
        self.requested = mode in ("host", "sync")
        self.sync = mode == "sync"
        self.skip = int(env.get("KIDI_PROFILE_OPS_SKIP", "0") or 0)
        self.active = self.requested and not self.skip
        self.requests = 0
        self.phase = "unspecified"
        self.profiles: dict[str, dict] = {}
        self.synchronization: dict[str, list] = {}
        self.prepare_ns = 0  # time spent preparing operators (weight packing), charged to the call that did it
        self._reported = False

    def profile_phase(self, phase: str) -> None:
        """Context::profile_phase (context.cpp:511-515)."""
        if not self.requested:
            return
        if phase in ("encoder", "gemma4_request"):
            self.requests += 1
            self.active = self.requests > self.skip
        self.phase = phase

    @contextmanager
    def call(self, op: str, shapes, attrs):
        """Time one operation; the body sets out["output"] to the result (for output_bytes and allocations)."""
        out = {}
        if not self.active:
            yield out
            return
        entered = time.perf_counter_ns()
        prep_before = self.prepare_ns
        ev0 = ev1 = None
        if self.device.type == "cuda":
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
        started = time.perf_counter_ns()
        yield out
        run_ns = time.perf_counter_ns() - started
        if ev1 is not None:
            ev1.record()
        wait_ns = 0
        if self.sync and self.device.type == "cuda":
            t = time.perf_counter_ns()
            torch.cuda.synchronize(self.device)
            wait_ns = time.perf_counter_ns() - t
        prepare = self.prepare_ns - prep_before
        p = self.profiles.setdefault(profile_key(self.phase, op, shapes, attrs),
                                     dict.fromkeys(self.FIELDS, 0) | {"device_ns": 0, "_events": []})
        p["calls"] += 1
        p["prepare_ns"] += prepare
        p["dispatch_ns"] += max(0, started - entered)
        p["run_ns"] += max(0, run_ns - prepare)
        p["wait_ns"] += wait_ns
        y = out.get("output")
        if isinstance(y, torch.Tensor):  # every call allocates its output
            p["allocations"] += 1
            p["allocated_bytes"] += y.numel() * y.element_size()
            p["output_bytes"] += y.numel() * y.element_size()
        if ev0 is not None:
            p["_events"].append((ev0, ev1))
            if len(p["_events"]) > 4096:
                self._fold(p)

    @staticmethod
    def _fold(p):
        for e0, e1 in p["_events"]:
            e1.synchronize()
            p["device_ns"] += int(e0.elapsed_time(e1) * 1e6)
        p["_events"].clear()

    def synchronize(self) -> None:
        """Context::synchronize (context.cpp:502-509)."""
        if not self.active:
            if self.device.type == "cuda":
                torch.cuda.synchronize(self.device)
            return
        t = time.perf_counter_ns()
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        c = self.synchronization.setdefault(self.phase, [0, 0])
        c[0] += 1
        c[1] += time.perf_counter_ns() - t

    def report(self) -> list[str]:
        """The report lines (context.cpp:119-129), with device_ns appended to each kidi_op line."""
        mode = "sync" if self.sync else "host"
        lines = []
        for key in sorted(self.profiles):
            p = self.profiles[key]
            self._fold(p)
            fields = "|".join(f"{f}={p[f]}" for f in self.FIELDS)
            lines.append(f"kidi_op|device={self.device}|mode={mode}|{key}|{fields}|device_ns={p['device_ns']}")
        for label in sorted(self.synchronization):
            calls, wait = self.synchronization[label]
            lines.append(f"kidi_op_sync|device={self.device}|phase={label}|calls={calls}|wait_ns={wait}")
        return lines

    def close(self, stream=None) -> None:
        """Print the report once (the reference prints it when the context is destroyed)."""
        if self._reported or not (self.profiles or self.synchronization):
            return
        self._reported = True
        out = stream or sys.stderr
        for line in self.report():
            print(line, file=out)
