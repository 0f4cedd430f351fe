"""Argument checks on device tensors, fetched with one host synchronization.

The reference validates cache lengths, page tables and cu_seqlens with a
chain of ``torch.any(...)`` / ``.item()`` calls, each of which waits for the
stream to drain (flash_attn_interface.py:433-470, :583-627).  ``Deferred``
queues those checks and reads them all with one synchronization.  Range
checks on device tensors (an array, an array plus an elementwise addend, or
the differences of adjacent elements) reduce in one native launch per eight
arrays (``fa_check_ranges``), which writes min and max straight into pinned
host memory; other device scalars (flags, values) are packed by
reinterpreting them as 32-bit words and copied with one device-to-host copy.
A call whose launch is safe on unchecked arguments (``side=True``, the decode
path) queues range checks only; they reduce on a second stream, so the launch
does not queue behind them.  Exceptions keep the reference's order: a check
that fails on the host first raises the first failing device check queued
before it, exactly as the reference's sequential checks would have.
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


def _as_int(t: torch.Tensor) -> torch.Tensor:
    t = t.reshape(-1)
    if t.dtype not in (torch.int32, torch.int64):
        t = t.long()
    return t.contiguous()


def _host_minmax(a: torch.Tensor, b: Optional[torch.Tensor], diff: bool):
    """min and max of a (+ b) or of a's adjacent differences, on the host
    (for tensors that are not on a GPU)."""
    x = a.long()
    if diff:
        x = x[1:] - x[:-1]
    elif b is not None:
        x = x + b.long()
    return int(x.min()), int(x.max())


class Deferred:
    def __init__(self, side: bool = False) -> None:
        # (kind, exception or None, lo, hi, payload), in queue order:
        #   "range":  payload (a, b, diff); raise exc unless the min and max of
        #             a (+ b), or of a's adjacent differences, lie in [lo, hi]
        #   "minmax": payload as "range"; (min, max) is returned as a value
        #   "flag":   payload [bad]; raise exc if the device boolean is true
        #   "value":  payload [t]; the device scalar is returned as a value
        #
        # side=True: range checks only, reduced at flush time on a second
        # stream that first waits for the current one, so a launch passed to
        # flush() starts on the current stream without queueing behind them.
        self._items: list = []
        self._nvalues = 0
        self._side = side

    def check(self, bad: torch.Tensor, exc: BaseException) -> None:
        """Queue ``raise exc`` if the device boolean ``bad`` is true."""
        if self._side:
            raise RuntimeError("Deferred(side=True) queues range checks only")
        self._items.append(("flag", exc, None, None, [bad.reshape(())]))

    def check_range(self, t: torch.Tensor, lo: Optional[int], hi: Optional[int],
                    exc: BaseException, plus: Optional[torch.Tensor] = None,
                    diff: bool = False) -> None:
        """Queue ``raise exc`` unless every element of the integer tensor ``t``
        (plus ``plus`` elementwise, when given; or every difference of
        adjacent elements, with ``diff``) lies in ``[lo, hi]`` (``None``:
        unbounded on that side)."""
        if t.numel() - (1 if diff else 0) <= 0:
            return
        self._items.append(("range", exc, lo, hi,
                            (_as_int(t), None if plus is None else _as_int(plus), diff)))

    def value_range(self, t: torch.Tensor, diff: bool = False) -> int:
        """Queue the (min, max) of an integer tensor as one value; returns its
        index in ``flush()``'s result."""
        if self._side:
            raise RuntimeError("Deferred(side=True) queues range checks only")
        self._items.append(("minmax", None, None, None, (_as_int(t), None, diff)))
        self._nvalues += 1
        return self._nvalues - 1

    def value(self, t: torch.Tensor) -> int:
        """Queue a device scalar to fetch; returns its index in ``flush()``'s result."""
        if self._side:
            raise RuntimeError("Deferred(side=True) queues range checks only")
        self._items.append(("value", None, None, None, [t.reshape(())]))
        self._nvalues += 1
        return self._nvalues - 1

    def fail(self, exc: BaseException) -> None:
        """A host-side check failed: device checks queued earlier win."""
        self.flush()
        raise exc

    def flush(self, launch=None) -> list:
        """Raise the first failing queued check; return the queued values.

        With ``launch`` (a callable that enqueues kernels on the current
        stream), the checks' results go to pinned host memory first,
        ``launch()`` runs, and only then does the host wait, for the checks
        alone: the launched work runs while the host reads them, and a
        failing check still raises before this call returns.  With
        ``side=True`` the range checks reduce on a second stream, so the
        launch does not queue behind them.  Only kernels that stay inside
        their buffers whatever the checked arrays hold may be launched this
        way."""
        items, self._items = self._items, []
        self._nvalues = 0
        if not items:
            if launch is not None:
                launch()
            return []
        # Range reductions: one fa_check_ranges launch per eight device
        # arrays, results in pinned host memory; host tensors on the host.
        ranged = [i for i, it in enumerate(items) if it[0] in ("range", "minmax")]
        on_dev = [i for i in ranged if items[i][4][0].is_cuda]
        results = {i: _host_minmax(*items[i][4]) for i in ranged if not items[i][4][0].is_cuda}
        done = None
        host_rng = None
        if on_dev:
            device = items[on_dev[0]][4][0].device
            stream = torch.cuda.current_stream(device)
            if self._side:
                side = _side_stream(device)
                side.wait_stream(stream)
                stream = side
            host_rng = torch.empty(2 * len(on_dev), dtype=torch.int64, pin_memory=True)
            step = _native.MAX_RANGE_CHECKS
            with torch.cuda.stream(stream):
                for s0 in range(0, len(on_dev), step):
                    chunk = on_dev[s0:s0 + step]
                    _native.check_ranges([items[i][4][:2] for i in chunk],
                                         host_rng[2 * s0:2 * (s0 + len(chunk))],
                                         diff=[items[i][4][2] for i in chunk])
                done = torch.cuda.Event()
                done.record()
        # Flags and values: packed into 32-bit words, one copy.
        scal = [i for i, it in enumerate(items) if it[0] in ("flag", "value")]
        words, dtypes, host_sc = [], [], None
        if scal:
            scalars = []
            for i in scal:
                s = items[i][4][0].reshape(1)
                if s.dtype not in _WORDS:
                    s = s.to(torch.int32 if s.dtype == torch.bool else torch.int64)
                scalars.append(s.view(torch.int32))
                dtypes.append(s.dtype)
            packed = torch.cat(scalars) if len(scalars) > 1 else scalars[0]
            if packed.is_cuda:
                host_sc = torch.empty(packed.shape, dtype=packed.dtype, pin_memory=True)
                host_sc.copy_(packed, non_blocking=True)
                done = torch.cuda.Event()   # same stream as the range launches
                done.record()
            else:
                words = packed.tolist()
        if launch is not None:
            launch()
        if done is not None:
            # Every tensor checked on the device is referenced by `items` until
            # this wait: none returns to the caching allocator (whose next user
            # could overwrite it on the current stream) while a check reads it.
            done.synchronize()
        if host_rng is not None:
            got = host_rng.tolist()
            for k, i in enumerate(on_dev):
                results[i] = (got[2 * k], got[2 * k + 1])
        if host_sc is not None:
            words = host_sc.tolist()
        scalars_dec, pos = [], 0
        for dt in dtypes:
            n = _WORDS[dt]
            scalars_dec.append(_decode(words[pos:pos + n], dt))
            pos += n
        values, k = [], 0
        for i, (kind, exc, lo, hi, _) in enumerate(items):
            if kind == "range":
                mn, mx = results[i]
                if (lo is not None and mn < lo) or (hi is not None and mx > hi):
                    raise exc
            elif kind == "minmax":
                values.append(results[i])
            else:
                got = scalars_dec[k]
                k += 1
                if kind == "flag" and got:
                    raise exc
                if kind == "value":
                    values.append(got)
        return values
