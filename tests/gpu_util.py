"""Shared helpers for the GPU parity tests."""
import numpy as np
import torch


def rel_l2(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / den) if den > 0 else float(np.linalg.norm(got))


def to_np(t):
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
