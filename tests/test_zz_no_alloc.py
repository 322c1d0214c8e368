"""GPU: bfly_argmax_rows_noalloc (static device workspace, no allocation) against
bfly_argmax_rows (caller workspace), through the C ABI, on consecutive calls of
shrinking size; and its refusal of row counts beyond its static workspace."""
from __future__ import annotations

import ctypes as C

import pytest
import torch

from butterfly_amd import _native

pytestmark = pytest.mark.gpu


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _with_workspace(x):
    rows, n = x.shape
    ws = torch.empty(rows * 3072 + 8, dtype=torch.uint8, device=x.device)
    out = torch.full((rows,), -7, dtype=torch.int64, device=x.device)
    rc = _native.lib().bfly_argmax_rows(x.data_ptr(), rows, n, x.stride(0), x.stride(1), ws.data_ptr(), ws.numel(),
                                        out.data_ptr(), _stream())
    assert rc == 0, _native.lib().bfly_last_error()
    return out


def _noalloc(x):
    rows, n = x.shape
    out = torch.full((rows,), -7, dtype=torch.int64, device=x.device)
    rc = _native.lib().bfly_argmax_rows_noalloc(x.data_ptr(), rows, n, x.stride(0), x.stride(1), out.data_ptr(),
                                                _stream())
    assert rc == 0, _native.lib().bfly_last_error()
    return out


def test_noalloc_argmax_equals_workspace_argmax_on_consecutive_calls():
    g = torch.Generator(device="cuda").manual_seed(17)
    # first call: the full static workspace (64 rows, 256 workgroups per row) with large values
    big = (torch.randn(64, 151936, generator=g, device="cuda") * 50 + 100).bfloat16()
    big[3, 77] = float("nan")                      # NaN wins, as in torch.argmax
    a1, b1 = _noalloc(big), _with_workspace(big)
    torch.cuda.synchronize()
    assert torch.equal(a1, b1) and int(a1[3]) == 77
    # second call, smaller and with small values: stale candidates of the first call would win
    small = torch.randn(5, 7000, generator=g, device="cuda").bfloat16()
    small[2, :] = 0.25                              # ties: the lowest index
    a2, b2 = _noalloc(small), _with_workspace(small)
    torch.cuda.synchronize()
    assert torch.equal(a2, b2) and int(a2[2]) == 0
    assert torch.equal(a2.cpu(), small.float().cpu().argmax(-1))
    # a strided view (columns of a [n, rows] tensor)
    t = torch.randn(9000, 7, generator=g, device="cuda").bfloat16()
    a3, b3 = _noalloc(t.t()), _with_workspace(t.t())
    torch.cuda.synchronize()
    assert torch.equal(a3, b3) and torch.equal(a3.cpu(), t.t().float().cpu().argmax(-1))


def test_noalloc_argmax_refuses_rows_beyond_its_workspace():
    x = torch.zeros(65, 16, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(65, dtype=torch.int64, device="cuda")
    rc = _native.lib().bfly_argmax_rows_noalloc(x.data_ptr(), 65, 16, 16, 1, out.data_ptr(), _stream())
    assert rc == _native.ERR_INVALID and b"64" in _native.lib().bfly_last_error()
