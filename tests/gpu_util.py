"""Helpers for the GPU parity tests: host<->device moves of raw bf16 / E4M3
bits and a loud progress line before each GPU step."""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

DEV = "cuda:0"
NTHREADS = max(1, min(16, os.cpu_count() or 1))


def step(msg: str) -> None:
    print(f"[gpu-step] {msg}", flush=True)
    sys.stdout.flush()


def bf16_dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(DEV)


def u8_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(DEV)


def f32_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def int_dev(v: int) -> torch.Tensor:
    return torch.tensor([v], dtype=torch.int32, device=DEV)


def bf16_host(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def sync() -> None:
    torch.cuda.synchronize()


def i32_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)
