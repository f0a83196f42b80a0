"""Shared helpers of the test suite."""

import hashlib
import importlib
from pathlib import Path

import numpy as np

PACKAGE = "low-latency-distributed-llm-serving-infrastructure-custom-k8s-control-plane_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"


def pkg(sub: str = ""):
    """Import the package (its directory name is not a Python identifier)."""
    return importlib.import_module(PACKAGE + ("." + sub if sub else ""))


def sha256(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def load_golden(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf16_close(got, ref, rel: float = 2e-2):
    """bf16 tolerance: max|g-r| / max|r| <= rel and |g-r| <= rel*|r| + rel*rms(r)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    scale = np.max(np.abs(ref)) if ref.size else 0.0
    rms = np.sqrt(np.mean(ref * ref)) if ref.size else 0.0
    worst = float(err.max() / scale) if ref.size and scale > 0 else 0.0
    elementwise = bool(np.all(err <= rel * np.abs(ref) + rel * rms)) if ref.size else True
    return worst <= rel and elementwise, worst
