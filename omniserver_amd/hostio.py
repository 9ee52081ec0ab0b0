"""Host -> device transfers that do not stall the host.

A pageable host tensor copied to the GPU makes the host wait for the copy, and the copy
waits for the work already queued on the stream: inside a forward that drains the whole
queue, after which the GPU idles while the host enqueues the next launches.  ``to_device``
stages a small host array in pinned memory and copies it with ``non_blocking=True`` on the
current stream (torch's caching host allocator keeps a pinned block until the copies that
read it have run, so the staging tensor may be dropped at once).  For a CPU device it is a
plain tensor.
"""

from __future__ import annotations

import torch


def to_device(values, dtype: torch.dtype, device) -> torch.Tensor:
    """values (a list / nested list, or a CPU tensor) as a dtype tensor on device."""
    device = torch.device(device)
    if isinstance(values, torch.Tensor):
        host = values.to(dtype=dtype)
        if device.type != "cuda":
            return host.to(device)
        return host.contiguous().pin_memory().to(device, non_blocking=True)
    if device.type != "cuda":
        return torch.tensor(values, dtype=dtype, device=device)
    return torch.tensor(values, dtype=dtype, pin_memory=True).to(device, non_blocking=True)
