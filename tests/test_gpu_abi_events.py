"""Timing events armed with dscq_time_next_kernel belong to the next call only.

A call that returns without launching -- an argument error, or a shape with
nothing to do -- must leave no events armed, or a later unrelated launch would
stamp them and the caller would read a wrong interval.
"""
import time

import pytest
import torch

from dscquant_amd import _lib, w4a4

pytestmark = pytest.mark.gpu


def _stamped_events():
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()  # torch creates the HIP events on their first record
    stop.record()
    torch.cuda.synchronize()
    return start, stop


def _assert_not_restamped(start, fail_call, x):
    L = _lib.lib()
    L.dscq_time_next_kernel(start.cuda_event, None)
    fail_call(L)
    time.sleep(0.02)
    mid = torch.cuda.Event(enable_timing=True)
    mid.record()
    w4a4.quantize(x, 1.0, True, 128)  # a good call: it must not stamp `start`
    torch.cuda.synchronize()
    # start still holds its first record, ~20 ms before mid; a re-stamp by the
    # good call would put it after mid.
    assert start.elapsed_time(mid) > 10.0


def test_argument_error_disarms(gpu):
    x = torch.randn(64, 256, device=gpu).half()
    start, _ = _stamped_events()
    print("case: bad dtype", flush=True)

    def bad(L):
        rc = L.dscq_quantize(x.data_ptr(), 7, 64, 256, 1.0, 1, 128, 16, 16, 16, None, None)
        assert rc != 0 and "FP16" in L.dscq_last_error().decode()
    _assert_not_restamped(start, bad, x)


def test_empty_call_disarms(gpu):
    x = torch.randn(64, 256, device=gpu).half()
    start, _ = _stamped_events()
    print("case: pack_int4 of an empty matrix", flush=True)

    def empty(L):
        assert L.dscq_pack_int4(None, 0, 16, None, None) == 0
    _assert_not_restamped(start, empty, x)
