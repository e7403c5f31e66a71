"""Helpers for the GPU parity tests: numpy <-> device buffers via torch."""
import numpy as np
import torch

from taraference_amd import capi


# Every device buffer made here stays referenced until the test ends
# (conftest clears KEEP after a device synchronize): a temporary whose
# address was handed to an asynchronous launch must not be recycled by the
# caching allocator before the kernel has run.
KEEP: list = []


def dev(a: np.ndarray) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    KEEP.append(t)
    return t


def empty(n, dtype=torch.float32) -> torch.Tensor:
    t = torch.empty(n, dtype=dtype, device="cuda")
    KEEP.append(t)
    return t


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


P = capi.ptr


def S():
    return capi.stream_ptr()


def call(name, *args):
    print(f"[gpu] {name}", flush=True)
    capi.call(name, *args)
