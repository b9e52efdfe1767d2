"""Scheduler-side epoch counters for benchmark runs.

Mirrors src/vllm_ascend_resident_epoch/benchmark_metrics.py:11-190: enabled
by VLLM_ASCEND_RESIDENT_EPOCH_BENCHMARK_METRICS_PATH (an absolute path under
/dev/shm); every schedule and result is appended to an event journal
(``<stem>.events.jsonl``) as it happens, and the aggregated record is
written at exit.  ``replay_event_journal`` rebuilds the record from the
journal when the process ended without running its exit hooks.
"""
from __future__ import annotations

import atexit
import json
import os
from collections import Counter
from pathlib import Path
from typing import Any

METRICS_ENV = "VLLM_ASCEND_RESIDENT_EPOCH_BENCHMARK_METRICS_PATH"
_RESULT_SUMS = ("feed_calls", "fetch_calls", "wall_us", "native_cpu_us", "socket_send_calls", "socket_receive_calls")


def _validated_metrics_path(raw: str) -> Path:
    path = Path(raw)
    if not path.is_absolute():
        raise ValueError(f"{METRICS_ENV} must be an absolute path")
    resolved = path.resolve(strict=False)
    shm = Path("/dev/shm").resolve(strict=False)
    if resolved == shm or shm not in resolved.parents:
        raise ValueError(f"{METRICS_ENV} must be under /dev/shm")
    return resolved


class ResidentEpochBenchmarkMetrics:
    def __init__(self, path: Path | None = None) -> None:
        self.path = path
        self.counters: Counter[str] = Counter()
        self.rejections: Counter[str] = Counter()
        self.epoch_steps: Counter[int] = Counter()
        self._journal = None
        if path is not None:
            journal = path.with_name(f"{path.stem}.events.jsonl")
            self._journal = os.open(journal, os.O_WRONLY | os.O_CREAT | os.O_APPEND, 0o600)

    @classmethod
    def from_env(cls) -> "ResidentEpochBenchmarkMetrics":
        raw = os.getenv(METRICS_ENV)
        metrics = cls(_validated_metrics_path(raw) if raw else None)
        if metrics.path is not None:
            atexit.register(metrics.flush)
        return metrics

    @property
    def enabled(self) -> bool:
        return self.path is not None

    def _event(self, event: dict[str, Any]) -> None:
        if self._journal is not None:
            os.write(self._journal, (json.dumps(event, sort_keys=True) + "\n").encode())

    # -- counting (shared with the journal replay) ------------------------------
    def _count_schedule(self, device: bool, request_count: int = 0, max_steps: int = 0, rejection: str | None = None):
        self.counters["schedule_calls"] += 1
        if device:
            self.counters["device_plan_calls"] += 1
            self.counters["device_planned_requests"] += request_count
            self.counters["device_planned_model_calls"] += max_steps
            self.epoch_steps[max_steps] += 1
        else:
            self.counters["host_schedule_calls"] += 1
            self.rejections[rejection or "unspecified"] += 1

    def _count_device_result(self, event: dict[str, Any]) -> None:
        self.counters["device_epochs"] += 1
        self.counters["device_model_calls"] += int(event["model_calls"])
        self.counters["device_request_tokens"] += sum(int(v) for v in event["computed_steps"].values())
        for name in _RESULT_SUMS:
            self.counters["native_wall_us" if name == "wall_us" else name] += int(event[name])
        if event.get("kv_imported"):
            self.counters["kv_imports"] += 1

    # -- recording -------------------------------------------------------------
    def record_schedule(self, plan: Any | None, rejection: str | None) -> None:
        if not self.enabled:
            return
        if plan is None:
            self._count_schedule(False, rejection=rejection)
            self._event({"kind": "schedule", "device": False, "rejection": rejection})
        else:
            n, k = len(plan.requests), int(plan.max_steps)
            self._count_schedule(True, n, k)
            self._event({"kind": "schedule", "device": True, "request_count": n, "max_steps": k})

    def record_result(self, result: Any) -> None:
        if not self.enabled:
            return
        if result.route != "device":
            self.counters["non_device_results"] += 1
            self._event({"kind": "result", "route": result.route})
            return
        event = {
            "kind": "result",
            "route": "device",
            "model_calls": int(result.model_calls),
            "computed_steps": {str(k): int(v) for k, v in result.computed_steps.items()},
            "kv_imported": bool(result.kv_imported),
            **{name: int(getattr(result, name)) for name in _RESULT_SUMS},
        }
        self._count_device_result(event)
        self._event(event)

    def as_record(self) -> dict[str, Any]:
        return {
            "schema_version": 1,
            "kind": "resident epoch benchmark counters",
            "counters": dict(sorted(self.counters.items())),
            "epoch_steps": {str(k): v for k, v in sorted(self.epoch_steps.items())},
            "rejections": dict(sorted(self.rejections.items())),
        }

    def flush(self) -> None:
        if not self.enabled:
            return
        self.path.parent.mkdir(parents=True, exist_ok=True)
        staging = self.path.with_name(f".{self.path.name}.{os.getpid()}.tmp")
        staging.write_text(json.dumps(self.as_record(), indent=2, sort_keys=True) + "\n", encoding="utf-8")
        os.replace(staging, self.path)
        if self._journal is not None:
            os.close(self._journal)
            self._journal = None


def replay_event_journal(path: Path) -> dict[str, Any]:
    """The aggregated record rebuilt from an event journal."""
    metrics = ResidentEpochBenchmarkMetrics()
    with Path(path).open(encoding="utf-8") as stream:
        for line in stream:
            event = json.loads(line)
            if event.get("kind") == "schedule":
                if event.get("device"):
                    metrics._count_schedule(True, int(event["request_count"]), int(event["max_steps"]))
                else:
                    metrics._count_schedule(False, rejection=event.get("rejection"))
            elif event.get("kind") == "result":
                if event.get("route") != "device":
                    metrics.counters["non_device_results"] += 1
                else:
                    metrics._count_device_result(event)
    return metrics.as_record()
