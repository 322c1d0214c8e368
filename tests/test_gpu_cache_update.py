"""GPU: the one-launch cache update (bfly_cache_update) equals bfly_cache_append followed by
bfly_cache_compress bit for bit: ring rows, pool rows, and the rows neither call touches.

The separate calls are themselves checked against the oracle cache in test_gpu_cache.py
(compressed_cache.py:104-149); here the cases are chosen so that due blocks take tokens
from the old tail, from the appended chunk and from both, with and without a ring wrap.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from butterfly_amd import _native
from butterfly_amd.attention import _dtype_code

pytestmark = pytest.mark.gpu


def _rand(seed, shape, dtype):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dtype).cuda()


def _two_calls(kn, vn, rk, rv, pk, pv, ring, offset, first_pos, n_blocks, bs, first_slot):
    b, h, step, d = kn.shape
    st = torch.cuda.current_stream().cuda_stream
    _native.call("bfly_cache_append", kn.data_ptr(), vn.data_ptr(), _dtype_code(kn), b, h, step, d, rk.data_ptr(),
                 rv.data_ptr(), ring, offset, st)
    _native.call("bfly_cache_compress", rk.data_ptr(), rv.data_ptr(), _dtype_code(kn), b, h, d, ring, first_pos,
                 n_blocks, bs, pk.data_ptr(), pv.data_ptr(), pk.shape[2], first_slot, st)


def _one_call(kn, vn, rk, rv, pk, pv, ring, offset, first_pos, n_blocks, bs, first_slot):
    b, h, step, d = kn.shape
    _native.call("bfly_cache_update", kn.data_ptr(), vn.data_ptr(), _dtype_code(kn), b, h, step, d, rk.data_ptr(),
                 rv.data_ptr(), ring, offset, first_pos, n_blocks, bs, pk.data_ptr(), pv.data_ptr(), pk.shape[2],
                 first_slot, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 64), (torch.bfloat16, 128), (torch.bfloat16, 256),
                                     (torch.float32, 64), (torch.float32, 128)])
@pytest.mark.parametrize("ring,offset,step,first_pos,n_blocks,bs", [
    (1088, 640, 384, 512, 3, 128),     # blocks 512..896: old tail then the chunk (the cfg4 pattern)
    (1088, 1000, 384, 896, 3, 128),    # ring wrap inside a due block and inside the chunk
    (200, 130, 50, 64, 1, 64),         # one block wholly from the old tail
    (200, 130, 50, 128, 0, 64),        # append only
    (96, 48, 48, 64, 1, 32),           # block wholly from the chunk
    (300, 0, 256, 0, 2, 100),          # first chunk, block size not a power of two
])
def test_update_equals_append_then_compress(dtype, d, ring, offset, step, first_pos, n_blocks, bs):
    b, h, pool = 2, 3, 12
    kn, vn = _rand(1, (b, h, step, d), dtype), _rand(2, (b, h, step, d), dtype)
    rk0, rv0 = _rand(3, (b, h, ring, d), dtype), _rand(4, (b, h, ring, d), dtype)
    pk0, pv0 = _rand(5, (b, h, pool, d), dtype), _rand(6, (b, h, pool, d), dtype)
    first_slot = 4
    want = [x.clone() for x in (rk0, rv0, pk0, pv0)]
    got = [x.clone() for x in (rk0, rv0, pk0, pv0)]
    _two_calls(kn, vn, *want, ring, offset, first_pos, n_blocks, bs, first_slot)
    _one_call(kn, vn, *got, ring, offset, first_pos, n_blocks, bs, first_slot)
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        assert torch.equal(g, w)


def test_update_rejects_blocks_outside_the_tail():
    kn = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device="cuda")
    rk = torch.zeros(1, 1, 32, 64, dtype=torch.bfloat16, device="cuda")
    pk = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):   # block [0, 16) precedes the tail [16, 48) after the append
        _one_call(kn, kn, rk, rk.clone(), pk, pk.clone(), 32, 40, 0, 1, 16, 0)
    with pytest.raises(ValueError):   # block [40, 56) ends past the appended chunk
        _one_call(kn, kn, rk, rk.clone(), pk, pk.clone(), 32, 40, 40, 1, 16, 0)
    with pytest.raises(ValueError):   # pool overflow
        _one_call(kn, kn, rk, rk.clone(), pk, pk.clone(), 32, 40, 32, 1, 16, 4)
