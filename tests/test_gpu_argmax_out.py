"""GPU: ``argmax_rows_noalloc(x, out=...)`` writes the picks into the caller's tensor (the greedy
graph step passes its token buffer) and refuses an output of the wrong shape, dtype or layout."""
from __future__ import annotations

import pytest
import torch

from butterfly_amd.decoder import argmax_rows_noalloc

pytestmark = pytest.mark.gpu


def test_argmax_noalloc_writes_into_out():
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(3, 151936, generator=g, device="cuda").bfloat16()
    tok = torch.full((3, 1), -1, dtype=torch.long, device="cuda")
    got = argmax_rows_noalloc(x, out=tok)
    torch.cuda.synchronize()
    assert got.data_ptr() == tok.data_ptr()
    assert torch.equal(tok.view(-1).cpu(), x.float().cpu().argmax(-1))


@pytest.mark.parametrize("bad", ["shape", "dtype", "layout"])
def test_argmax_noalloc_rejects_a_bad_out(bad):
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda")
    out = {"shape": torch.empty(4, dtype=torch.long, device="cuda"),
           "dtype": torch.empty(4, 1, dtype=torch.int32, device="cuda"),
           "layout": torch.empty(1, 8, dtype=torch.long, device="cuda")[:, ::2].t()}[bad]
    with pytest.raises(ValueError):
        argmax_rows_noalloc(x, out=out)
