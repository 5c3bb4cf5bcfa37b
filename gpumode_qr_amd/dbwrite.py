"""Run records in the reference's results-DB form: one JSON file per run.

What is kept alike is the schema its readers depend on (reference
src/qrbench/dbwrite.py:61-93, AGENTS.md): the file name
``<UTC yyyymmddThhmmssZ>_<impl>.json`` and the top-level keys, in the order of
``RECORD_KEYS``, with ``extra`` present only when given. How each provenance
field is obtained is this module's own:

* ``git_commit``: ``QR_SOURCE_REVISION`` if set (a copy of the tree without
  its ``.git``, as on a remote GPU host, can be told its revision), else
  ``git rev-parse HEAD`` with ``-dirty`` appended when tracked files differ
  from it (``git status --porcelain --untracked-files=no``), else "unknown";
* ``rocm_version``: the HIP version torch was built against;
* ``gpu_name``: device 0 as torch names it ("cpu" without a GPU).
"""

from __future__ import annotations

import json
import os
import subprocess
from datetime import datetime, timezone
from pathlib import Path

import torch

RECORD_KEYS = ("impl", "git_commit", "date", "rocm_version", "docker_image", "torch_version",
               "gpu_name", "hip_visible_devices", "benchmark_results", "extra")


def _git(repo_dir: str, *args: str) -> str | None:
    try:
        done = subprocess.run(["git", "-C", repo_dir, *args], capture_output=True, text=True,
                              timeout=30)
    except (OSError, subprocess.TimeoutExpired):
        return None
    return done.stdout.strip() if done.returncode == 0 else None


def source_revision(repo_dir: str) -> str:
    given = os.environ.get("QR_SOURCE_REVISION")
    if given:
        return given
    head = _git(repo_dir, "rev-parse", "HEAD")
    if not head:
        return "unknown"
    changes = _git(repo_dir, "status", "--porcelain", "--untracked-files=no")
    return head + ("-dirty" if changes else "")


def provenance(repo_dir: str, docker_image: str | None = None) -> dict:
    """The record's provenance fields, in schema order."""
    has_gpu = torch.cuda.is_available()
    return {
        "git_commit": source_revision(repo_dir),
        "date": datetime.now(timezone.utc).isoformat(),
        "rocm_version": getattr(torch.version, "hip", None) or "unknown",
        "docker_image": docker_image or os.environ.get("DOCKER_IMAGE") or "unknown",
        "torch_version": torch.__version__,
        "gpu_name": torch.cuda.get_device_name(0) if has_gpu else "cpu",
        "hip_visible_devices": os.environ.get("HIP_VISIBLE_DEVICES", ""),
    }


def write_record(db_dir: str | Path, impl: str, provenance_fields: dict,
                 benchmark_results: list[dict], extra: dict | None = None) -> Path:
    """Write one record and return its path."""
    fields = {"impl": impl, **provenance_fields, "benchmark_results": benchmark_results}
    if extra:
        fields["extra"] = extra
    record = {k: fields[k] for k in RECORD_KEYS if k in fields}
    missing = [k for k in RECORD_KEYS[:-1] if k not in record]
    if missing:
        raise KeyError(f"record lacks {missing}")
    out = Path(db_dir)
    out.mkdir(parents=True, exist_ok=True)
    stamp = datetime.now(timezone.utc).strftime("%Y%m%dT%H%M%SZ")
    path = out / f"{stamp}_{impl}.json"
    path.write_text(json.dumps(record, indent=2) + "\n")
    return path
