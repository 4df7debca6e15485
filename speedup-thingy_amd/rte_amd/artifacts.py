"""Run manifests and metric files in the reference's on-disk format (rte/artifacts.py:1-120,
rte/reporting.py:10-42): manifest.json holds the config (and its hash), git state, hardware and
the kernel backend status that benchmarks/speed_audit.py:49-53 checks before a speed proof;
metrics.jsonl holds one JSON object per logged step (tensors reduced to their mean)."""

from __future__ import annotations

import dataclasses
import hashlib
import json
import platform
import subprocess
import sys
from pathlib import Path
from typing import Any

import torch

from rte_amd.kernels import optimized


def json_default(value: Any) -> Any:
    """JSON encoding of values the metrics hold: scalar tensors as floats, other tensors as lists,
    dataclasses as dicts, anything else as its string."""
    if isinstance(value, torch.Tensor):
        return float(value.detach().float().cpu()) if value.numel() == 1 else value.detach().cpu().tolist()
    if dataclasses.is_dataclass(value):
        return dataclasses.asdict(value)
    return str(value)


def config_hash(config) -> str:
    blob = json.dumps(dataclasses.asdict(config), sort_keys=True, default=json_default)
    return hashlib.sha256(blob.encode("utf-8")).hexdigest()


def git_info(cwd: str | Path = ".") -> dict[str, Any]:
    def run(args):
        try:
            return subprocess.check_output(args, cwd=cwd, text=True, stderr=subprocess.DEVNULL).strip()
        except Exception:
            return None

    dirty = run(["git", "status", "--short"])
    return {"commit": run(["git", "rev-parse", "HEAD"]), "dirty": bool(dirty),
            "dirty_files": dirty.splitlines() if dirty else []}


def hardware_info() -> dict[str, Any]:
    """The reference's keys (cuda_device is the ROCm device's name under ROCm torch) plus the gfx
    architecture of device 0."""
    dev_ok = torch.cuda.is_available()
    mps = bool(hasattr(torch.backends, "mps") and torch.backends.mps.is_available())
    info = {"platform": platform.platform(), "python": sys.version, "torch": torch.__version__,
            "device": "cuda" if dev_ok else ("mps" if mps else "cpu"),
            "cuda_device": torch.cuda.get_device_name(0) if dev_ok else None, "mps_available": mps,
            "hip": torch.version.hip}
    if dev_ok:
        info["gcn_arch"] = getattr(torch.cuda.get_device_properties(0), "gcnArchName", None)
    return info


def build_manifest(config, *, command: list[str] | None = None, extra: dict[str, Any] | None = None) -> dict[str, Any]:
    manifest = {"config_hash": config_hash(config), "config": dataclasses.asdict(config), "git": git_info(Path.cwd()),
                "hardware": hardware_info(), "backend": optimized.backend_status(), "command": command or sys.argv}
    if extra:
        manifest.update(extra)
    return manifest


def write_json(path: str | Path, payload: dict[str, Any]) -> None:
    p = Path(path)
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_text(json.dumps(payload, indent=2, sort_keys=True, default=json_default) + "\n")


def read_jsonl(path: str | Path) -> list[dict[str, Any]]:
    p = Path(path)
    if not p.exists() or p.stat().st_size == 0:
        return []
    return [json.loads(line) for line in p.read_text().splitlines() if line.strip()]


def summarize_metrics(path: str | Path) -> dict[str, Any]:
    """First / last step, the last row and the mean of every numeric key of a metrics.jsonl (or
    the one in a run directory), with the run's manifest when present (rte/artifacts.py:95-120)."""
    run = Path(path)
    mpath = run if run.is_file() else run / "metrics.jsonl"
    rows = read_jsonl(mpath)
    if not rows:
        raise ValueError(f"no metrics found in {mpath}")
    keys = {k for row in rows for k, v in row.items() if isinstance(v, (int, float))}
    means = {}
    for key in sorted(keys):
        vals = [float(row[key]) for row in rows if isinstance(row.get(key), (int, float))]
        if vals:
            means[f"mean_{key}"] = sum(vals) / len(vals)
    out = {"metrics_path": str(mpath), "rows": len(rows), "first_step": rows[0].get("step"),
           "last_step": rows[-1].get("step"), "last": rows[-1], "means": means}
    man = mpath.parent / "manifest.json"
    if man.exists():
        out["manifest"] = json.loads(man.read_text())
    return out


class JsonlLogger:
    """Appends one sorted-key JSON object per row; tensors become the float of their mean
    (rte/reporting.py:10-29).  Device tensors of one row are copied to the host together."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self.path.parent.mkdir(parents=True, exist_ok=True)
        self.file = self.path.open("a")
        self.rows_written = 0

    def write(self, row: dict[str, Any]) -> None:
        tens = {k: v for k, v in row.items() if isinstance(v, torch.Tensor)}
        host = optimized.k_metrics_reduce(tens) if tens else {}
        clean = {k: (host[k] if k in host else v) for k, v in row.items()}
        self.file.write(json.dumps(clean, sort_keys=True, default=json_default) + "\n")
        self.file.flush()
        self.rows_written += 1

    def close(self) -> None:
        self.file.close()


def summarize_time_to_target(rows: list[dict[str, Any]], target_loss: float) -> dict[str, Any]:
    """First logged time at which val_loss reached the target (rte/reporting.py:32-42)."""
    reached = [row for row in rows if row.get("val_loss", float("inf")) <= target_loss]
    if not reached:
        return {"target_loss": target_loss, "reached": False, "time_to_target_loss": None}
    first = min(reached, key=lambda r: r.get("elapsed_train_time", float("inf")))
    return {"target_loss": target_loss, "reached": True, "time_to_target_loss": first.get("elapsed_train_time"),
            "step": first.get("step")}


def speed_proof_allowed(manifest_or_status: dict[str, Any]) -> bool:
    """The check of benchmarks/speed_audit.py:49-53: a speed proof is refused when the backend
    uses the reference fallback (accepts a manifest or a backend_status dict)."""
    status = manifest_or_status.get("backend", manifest_or_status)
    return not bool(status.get("uses_reference_fallback", True))
