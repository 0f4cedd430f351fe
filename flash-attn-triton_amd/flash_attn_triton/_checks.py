"""Argument checks on device tensors, fetched with one host synchronization.

The reference validates cache lengths, page tables and cu_seqlens with a
chain of ``torch.any(...)`` / ``.item()`` calls, each of which waits for the
stream to drain (flash_attn_interface.py:433-470, :583-627).  ``Deferred``
queues those checks as device scalars and reads them all with one
device-to-host copy.  Range checks cost one ``aminmax`` launch each, and the
queued scalars are packed by reinterpreting them as 32-bit words (no
conversion launches).  A call whose launch is safe on unchecked arguments
(``side=True``, the decode path) queues range checks only; they reduce in one
native launch (``fa_check_ranges``) that writes min and max straight into
pinned host memory, on a second stream.  Exceptions keep the reference's
order: a check that fails on the host first raises the first failing device
check queued before it, exactly as the reference's sequential checks would
have.
"""
from __future__ import annotations

import struct
from typing import List, Optional

import torch

from . import _native

_WORDS = {torch.int32: 1, torch.float32: 1, torch.int64: 2, torch.float64: 2}


def _decode(words: List[int], dtype: torch.dtype):
    if dtype == torch.int32:
        return words[0]
    if dtype == torch.int64:
        return (words[1] << 32) | (words[0] & 0xFFFFFFFF)
    raw = struct.pack("<" + "i" * len(words), *words)
    return struct.unpack("<f" if dtype == torch.float32 else "<d", raw)[0]


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> "torch.cuda.Stream":
    """A second stream per device (default priority) for argument checks."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get(key)
    if st is None:
        st = torch.cuda.Stream(device=key)
        _SIDE_STREAMS[key] = st
    return st


class Deferred:
    def __init__(self, side: bool = False) -> None:
        # (kind, exception or None, lo, hi, device scalars); kind "flag": one
        # boolean, raise if true; "range": (min, max), raise if outside
        # [lo, hi]; "value": one scalar to return.
        #
        # side=True: range checks only, reduced at flush time by one
        # fa_check_ranges launch on a second stream that first waits for the
        # current one, so a launch passed to flush() starts on the current
        # stream without queueing behind them.
        self._items: list = []
        self._minmax: dict = {}   # id(tensor) -> (tensor, min, max): one aminmax per tensor
        self._side = side

    def check(self, bad: torch.Tensor, exc: BaseException) -> None:
        """Queue ``raise exc`` if the device boolean ``bad`` is true."""
        if self._side:
            raise RuntimeError("Deferred(side=True) queues range checks only")
        self._items.append(("flag", exc, None, None, [bad.reshape(())]))

    def check_range(self, t: torch.Tensor, lo: Optional[int], hi: Optional[int],
                    exc: BaseException, plus: Optional[torch.Tensor] = None) -> None:
        """Queue ``raise exc`` unless every element of the integer tensor ``t``
        (plus ``plus`` elementwise, when given) lies in ``[lo, hi]``
        (``None``: unbounded on that side)."""
        if t.numel() == 0:
            return
        if self._side:
            a = t.reshape(-1)
            if a.dtype not in (torch.int32, torch.int64):
                a = a.long()
            b = None if plus is None else plus.reshape(-1)
            if b is not None and b.dtype not in (torch.int32, torch.int64):
                b = b.long()
            self._items.append(("range", exc, lo, hi, [a.contiguous(),
                                                       None if b is None else b.contiguous()]))
            return
        if plus is not None:
            t = t.long() + plus
        hit = self._minmax.get(id(t))
        if hit is None or hit[0] is not t:
            hit = (t, *torch.aminmax(t))
            self._minmax[id(t)] = hit
        self._items.append(("range", exc, lo, hi, [hit[1], hit[2]]))

    def value(self, t: torch.Tensor) -> int:
        """Queue a device scalar to fetch; returns its index in ``flush()``'s result."""
        if self._side:
            raise RuntimeError("Deferred(side=True) queues range checks only")
        self._items.append(("value", None, None, None, [t.reshape(())]))
        return sum(1 for it in self._items if it[0] == "value") - 1

    def fail(self, exc: BaseException) -> None:
        """A host-side check failed: device checks queued earlier win."""
        self.flush()
        raise exc

    def flush(self, launch=None) -> list:
        """Raise the first failing queued check; return the queued values.

        With ``launch`` (a callable that enqueues kernels on the current
        stream), the queued scalars are copied to pinned host memory first,
        ``launch()`` runs, and only then does the host wait, for the copy
        alone: the launched work runs while the host reads the checks, and
        a failing check still raises before this call returns.  With
        ``side=True`` the range checks reduce in one launch on a second
        stream, so the launch does not queue behind them.  Only kernels that
        stay inside their buffers whatever the checked arrays hold may be
        launched this way."""
        items, self._items = self._items, []
        self._minmax = {}
        if not items:
            if launch is not None:
                launch()
            return []
        if self._side:
            return self._flush_side(items, launch)
        scalars, dtypes = [], []
        for it in items:
            for s in it[4]:
                s = s.reshape(1)
                if s.dtype not in _WORDS:
                    s = s.to(torch.int32 if s.dtype == torch.bool else torch.int64)
                scalars.append(s.view(torch.int32))
                dtypes.append(s.dtype)
        packed = torch.cat(scalars) if len(scalars) > 1 else scalars[0]
        if launch is None:
            words = packed.tolist()
        else:
            host = torch.empty(packed.shape, dtype=packed.dtype, pin_memory=True)
            host.copy_(packed, non_blocking=True)
            done = torch.cuda.Event()
            done.record()
            launch()
            done.synchronize()
            words = host.tolist()
        host, pos = [], 0
        for dt in dtypes:
            n = _WORDS[dt]
            host.append(_decode(words[pos:pos + n], dt))
            pos += n
        values, k = [], 0
        for kind, exc, lo, hi, ts in items:
            got = host[k:k + len(ts)]
            k += len(ts)
            if kind == "flag" and got[0]:
                raise exc
            if kind == "range" and ((lo is not None and got[0] < lo) or
                                    (hi is not None and got[1] > hi)):
                raise exc
            if kind == "value":
                values.append(got[0])
        return values

    @staticmethod
    def _flush_side(items: list, launch) -> list:
        """Side-stream flush: every item is a range check [array, addend]."""
        device = items[0][4][0].device
        side = _side_stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        arrays = [(ts[0], ts[1]) for _, _, _, _, ts in items]
        host = torch.empty(2 * len(arrays), dtype=torch.int64, pin_memory=True)
        step = _native.MAX_RANGE_CHECKS
        with torch.cuda.stream(side):
            for i in range(0, len(arrays), step):
                chunk = arrays[i:i + step]
                _native.check_ranges(chunk, host[2 * i:2 * (i + len(chunk))])
            done = torch.cuda.Event()
            done.record()
        if launch is not None:
            launch()
        # `arrays` holds every checked tensor until the side stream has read
        # it: none of them returns to the caching allocator (whose next user
        # could overwrite it on the current stream) before this wait.
        done.synchronize()
        got = host.tolist()
        del arrays
        for i, (_, exc, lo, hi, _) in enumerate(items):
            if (lo is not None and got[2 * i] < lo) or (hi is not None and got[2 * i + 1] > hi):
                raise exc
        return []
