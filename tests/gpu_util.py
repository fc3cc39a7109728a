"""Helpers shared by the GPU parity tests."""
import sys

import torch


def device():
    assert torch.cuda.is_available(), "GPU test run without a HIP device"
    return torch.device("cuda:0")


def announce(msg):
    """Name the case before a GPU step (flushed, so it survives a crash)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()
