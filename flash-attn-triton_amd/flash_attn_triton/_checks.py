"""Argument checks on device tensors, fetched with one host synchronization.

The reference validates cache lengths, page tables and cu_seqlens with a
chain of ``torch.any(...)`` / ``.item()`` calls, each of which waits for the
stream to drain (flash_attn_interface.py:433-470, :583-627).  ``Deferred``
queues those checks as device flags and reads them all with one
device-to-host copy.  Exceptions keep the reference's order: a check that
fails on the host first raises the first failing device check queued before
it, exactly as the reference's sequential checks would have.
"""
from __future__ import annotations

from typing import List, Tuple

import torch


class Deferred:
    def __init__(self) -> None:
        self._flags: List[Tuple[torch.Tensor, BaseException]] = []
        self._values: List[torch.Tensor] = []

    def check(self, bad: torch.Tensor, exc: BaseException) -> None:
        """Queue ``raise exc`` if the device boolean ``bad`` is true."""
        self._flags.append((bad.reshape(()), exc))

    def value(self, t: torch.Tensor) -> int:
        """Queue a device scalar to fetch; returns its index in ``flush()``'s result."""
        self._values.append(t.reshape(()))
        return len(self._values) - 1

    def fail(self, exc: BaseException) -> None:
        """A host-side check failed: device checks queued earlier win."""
        self.flush()
        raise exc

    def flush(self) -> list:
        """Raise the first failing queued check; return the queued values."""
        flags, values = self._flags, self._values
        self._flags, self._values = [], []
        if not flags and not values:
            return []
        dev = (flags[0][0] if flags else values[0]).device
        host = torch.stack([t.to(device=dev, dtype=torch.int64) for t, _ in flags] +
                           [v.to(device=dev, dtype=torch.int64) for v in values]).tolist()
        for (_, exc), bad in zip(flags, host):
            if bad:
                raise exc
        return host[len(flags):]
