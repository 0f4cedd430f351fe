"""Host logic of the deferred argument checks (flash_attn_triton/_checks.py):
range checks, flags and fetched values of several dtypes, in queue order,
read with one device-to-host copy.  Runs on CPU tensors."""
import pytest
import torch

from flash_attn_triton._checks import Deferred


def test_values_of_every_dtype_round_trip():
    chk = Deferred()
    i32 = chk.value(torch.tensor(-7, dtype=torch.int32))
    i64 = chk.value(torch.tensor(-(1 << 40) - 3, dtype=torch.int64))
    f32 = chk.value(torch.tensor(1.5, dtype=torch.float32))
    b = chk.value(torch.tensor(True))
    f64 = chk.value(torch.tensor(-2.25, dtype=torch.float64))
    u8 = chk.value(torch.tensor(200, dtype=torch.uint8))
    got = chk.flush()
    assert (got[i32], got[i64], got[f32], got[b], got[f64], got[u8]) == (
        -7, -(1 << 40) - 3, 1.5, 1, -2.25, 200)


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_range_checks(dtype):
    t = torch.tensor([3, 0, 9], dtype=dtype)
    chk = Deferred()
    chk.check_range(t, 0, 9, ValueError("a"))
    chk.check_range(t, None, None, ValueError("b"))
    chk.check_range(t[:0], 5, 1, ValueError("empty tensors pass"))
    assert chk.flush() == []
    for lo, hi in ((1, None), (None, 8)):
        chk.check_range(t, lo, hi, ValueError("out of range"))
        with pytest.raises(ValueError, match="out of range"):
            chk.flush()


def test_first_failing_check_in_queue_order_wins():
    chk = Deferred()
    chk.check(torch.tensor(False), ValueError("flag ok"))
    chk.check_range(torch.tensor([5]), 0, 4, KeyError("range first"))
    chk.check(torch.tensor(True), IndexError("flag second"))
    with pytest.raises(KeyError):
        chk.flush()
    # A host-side failure raises queued device failures first.
    chk.check(torch.tensor(True), IndexError("device"))
    with pytest.raises(IndexError):
        chk.fail(RuntimeError("host"))
    chk.check(torch.tensor(False), IndexError("device"))
    with pytest.raises(RuntimeError):
        chk.fail(RuntimeError("host"))


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_adjacent_difference_ranges_and_value_ranges(dtype):
    # cu_seqlens-style monotonicity: the differences of adjacent elements.
    cu = torch.tensor([0, 3, 3, 10], dtype=dtype)
    chk = Deferred()
    chk.check_range(cu, 0, 7, ValueError("lengths"), diff=True)
    chk.check_range(cu[:1], 0, 0, ValueError("start"), diff=True)   # no difference: skipped
    i = chk.value_range(cu, diff=True)
    j = chk.value_range(torch.tensor([5, -2, 9], dtype=dtype))
    assert chk.flush() == [(0, 7), (-2, 9)]
    chk.check_range(torch.tensor([0, 4, 2], dtype=dtype), 0, None, ValueError("order"), diff=True)
    with pytest.raises(ValueError, match="order"):
        chk.flush()
    # An addend: lengths + left pads against a capacity.
    chk.check_range(torch.tensor([4, 1], dtype=dtype), None, 5, ValueError("fit"),
                    plus=torch.tensor([1, 5], dtype=torch.int64))
    with pytest.raises(ValueError, match="fit"):
        chk.flush()
    assert (i, j) == (0, 1)
