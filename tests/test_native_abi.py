"""The C-ABI library loads and exports every entry point declared in include/*.h.

Runs without a GPU: only host-side functions (stage metadata, partner bits,
error reporting) are called; device entry points are checked for presence and
argument validation only.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from butterfly_amd import _native
from oracle import topology as tp

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(bfly_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_entry_points():
    names = _declared_symbols()
    assert {"bfly_prefill", "bfly_attend_cache", "bfly_block_mean", "bfly_block_neighbors"} <= names


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in sorted(_declared_symbols()):
        assert hasattr(lib, name), name
    assert set(_native.SIGNATURES) == _declared_symbols()
    assert lib.bfly_abi_version() == 2


@pytest.mark.parametrize("rule", list(tp.RULES))
def test_host_stage_meta_matches_oracle(rule):
    lib = _native.lib()
    s, c, w = C.c_int32(), C.c_int32(), C.c_int32()
    for n in [1, 2, 3, 7, 32, 33, 512, 1024, 1025, 2048, 100003]:
        for layer in [0, 1, 4, 9, 13, 40]:
            assert lib.bfly_stage_meta(n, layer, _native.RULES[rule], C.byref(s), C.byref(c), C.byref(w)) == 0
            assert (s.value, c.value) == tp.stage_meta(n, layer, rule)
            assert w.value == tp.width(n)
            bits = (C.c_int32 * 3)()
            assert lib.bfly_partner_bits(s.value, c.value, w.value, 3, _native.RULES[rule], bits) == 0
            assert list(bits) == tp.partner_bits(s.value, c.value, w.value, 3, rule)


def test_errors_are_reported():
    lib = _native.lib()
    s = C.c_int32()
    rc = lib.bfly_stage_meta(8, 0, 99, C.byref(s), C.byref(s), C.byref(s))
    assert rc == _native.ERR_INVALID
    assert b"partner rule" in lib.bfly_last_error()
    with pytest.raises(ValueError):
        _native.check(rc, "bfly_stage_meta")
    # device entry points validate arguments before touching the GPU
    rc = lib.bfly_prefill(None, None, None, None, None, 1, 1, 8, 2, 64, 128, None, 1, 4, 128, 64, 1.0, None, None)
    assert rc == _native.ERR_INVALID
    rc = lib.bfly_block_neighbors(16, 0, 3, 1, 1, 1, None, 2, None, None)
    assert rc == _native.ERR_INVALID and b"kcap" in lib.bfly_last_error()


@pytest.mark.parametrize("args,msg", [
    ((256, 1024, 256, 8, 2048, 48, 512, None), b"group"),             # group not a multiple of 32
    ((256, 1024, 256, 8, 8256, 64, 512, None), b"8192"),              # in_features above the limit
    ((256, 1024, 256, 8, 2000, 64, 512, None), b"multiple of group"),
    ((264, 1024, 256, 8, 2048, 64, 512, None), b"16-byte"),           # x not 16-byte aligned
    ((256, 1024, 258, 8, 2048, 64, 512, None), b"scale_bias"),
    ((256, 1024, 256, 0, 2048, 64, 512, None), b"out_features"),
])
def test_q4_gemv_validates_before_launch(args, msg):
    """Fake, never dereferenced addresses: every case fails its checks before a launch."""
    lib = _native.lib()
    assert lib.bfly_q4_gemv(*args) == _native.ERR_INVALID
    assert msg in lib.bfly_last_error()
    x, w, sb, n, k, g, out, st = args
    assert lib.bfly_q4_gemv_silu(x, w, sb, n, k, g, n, out, st) == _native.ERR_INVALID
    if n > 0:   # up rows overlapping the gate rows
        assert lib.bfly_q4_gemv_silu(256, 1024, 256, 8, 2048, 64, 4, 512, None) == _native.ERR_INVALID
        assert b"up_row_offset" in lib.bfly_last_error()


@pytest.mark.parametrize("rule", list(tp.RULES))
def test_topology_init_matches_oracle(rule):
    lib = _native.lib()
    for n in [1, 2, 33, 512, 1025, 2048]:
        for layer in [0, 3, 11, 29]:
            t = _native.Topology()
            assert lib.bfly_topology_init(n, layer, _native.RULES[rule], 1, 1, 2, C.byref(t)) == 0
            s, count = tp.stage_meta(n, layer, rule)
            assert (t.stage_idx, t.stage_count, t.width) == (s, count, tp.width(n))
            assert list(t.partner_bits[:2]) == tp.partner_bits(s, count, tp.width(n), 2, rule)
            assert (t.rule, t.local_window_blocks, t.sink_count, t.partner_count) == (_native.RULES[rule], 1, 1, 2)
    t = _native.Topology()
    assert lib.bfly_topology_init(8, 0, 3, 1, 1, 17, C.byref(t)) == _native.ERR_INVALID


def test_decode_state_words_match_the_host_layout():
    from butterfly_amd.compressed_cache import _DEV_SLOT, _dev_copies

    lib = _native.lib()
    # up to 16 sequences: 64 copies each (the fused output projection's attending workgroups)
    assert lib.bfly_decode_state_words(1, 1) == 8 + (64 + 8) * _DEV_SLOT
    assert lib.bfly_decode_state_words(4, 4) == 8 + (16 * 64 + 8) * _DEV_SLOT
    assert lib.bfly_decode_state_words(17, 1) == 8 + (17 + 8) * _DEV_SLOT    # one copy per sequence beyond
    assert lib.bfly_decode_state_words(32, 2) == 8 + 72 * _DEV_SLOT
    assert lib.bfly_decode_state_words(0, 2) == 0
    for n in (1, 4, 16, 17, 64):
        assert lib.bfly_decode_state_words(n, 1) == 8 + (n * _dev_copies(n) + 8) * _DEV_SLOT


def test_decode_step_qk_norm_validates_before_launch():
    """Fake, never dereferenced addresses: missing norm weights, a misaligned table and a
    head_dim other than 128 are refused before any launch."""
    lib = _native.lib()
    base = (256, _native.DTYPE_BF16, 1, 8, 2, 128, 512, 768, 1024, 1280, 256, 1536, 1792, 16, 2048, 0, 3, 1, 1, 1,
            128, 64, 64, 0.088)
    tail = (64, 1e-6, 0x3000, None)                    # rope_rows, eps, out, stream
    assert lib.bfly_decode_step_qk_norm(*base, None, 0x2100, 0x2200, 0x2300, *tail) == _native.ERR_INVALID
    assert lib.bfly_decode_step_qk_norm(*base, 0x2000, 0x2100, 0x2208, 0x2300, *tail) == _native.ERR_INVALID
    assert b"16-byte" in lib.bfly_last_error()
    d64 = base[:5] + (64,) + base[6:]
    assert lib.bfly_decode_step_qk_norm(*d64, 0x2000, 0x2100, 0x2200, 0x2300, *tail) == _native.ERR_INVALID
    assert b"head_dim 128" in lib.bfly_last_error()


def test_decode_step_qk_norm_oproj_validates_before_launch():
    """Fake, never dereferenced addresses: shapes other than 16 query heads over 4 kv heads of
    128, batches past 16 sequences, bad o_group / o_out_features and missing or misaligned
    projection buffers are refused before any launch."""
    lib = _native.lib()

    def call(b=1, hq=16, hkv=4, d=128, o_packed=0x4000, o_sb=0x5000, n_out=2048, group=64, parts=0x6000):
        head = (256, _native.DTYPE_BF16, b, hq, hkv, d, 512, 768, 1024, 1280, 256, 1536, 1792, 16, 2048, 0, 3, 1,
                1, 1, 128, 64, 64, 0.088, 0x2000, 0x2100, 0x2200, 0x2300, 64, 1e-6)
        return lib.bfly_decode_step_qk_norm_oproj(*head, o_packed, o_sb, n_out, group, parts, 0x3000, None)

    for kw, msg in [(dict(hq=8, hkv=2), b"16 query heads"), (dict(d=64), b"16 query heads"),
                    (dict(b=5), b"<= 16"), (dict(group=48), b"power of two"), (dict(group=16), b"power of two"),
                    (dict(n_out=2000), b"multiple of 32"), (dict(n_out=64 * 65), b"multiple of 32"),
                    (dict(parts=None), b"null"), (dict(o_packed=0x4008), b"16-byte"), (dict(o_sb=0x5002), b"16-byte")]:
        assert call(**kw) == _native.ERR_INVALID, kw
        assert msg in lib.bfly_last_error(), (kw, lib.bfly_last_error())


def test_add_rms_norm_q4_gemv_silu_parts_validates_before_launch():
    """Four 16-byte aligned partial rows, else refused before a launch (fake addresses)."""
    lib = _native.lib()
    tail = (512, 768, 1e-6, 1024, 1280, 1536, 8, 2048, 64, 8, 2048, None)
    assert lib.bfly_add_rms_norm_q4_gemv_silu_parts(0x1000, 3, *tail) == _native.ERR_INVALID
    assert b"four partial rows" in lib.bfly_last_error()
    assert lib.bfly_add_rms_norm_q4_gemv_silu_parts(0x1008, 4, *tail) == _native.ERR_INVALID
    assert b"16-byte" in lib.bfly_last_error()
    bad_in = tail[:7] + (3072,) + tail[8:]
    assert lib.bfly_add_rms_norm_q4_gemv_silu_parts(0x1000, 4, *bad_in) == _native.ERR_INVALID


def test_greedy_entry_points_validate_before_launch():
    """Workspace size and alignment, and the advance's shapes, are checked before a launch
    (fake addresses)."""
    lib = _native.lib()
    need = lib.bfly_q4_argmax_workspace_bytes(151936, 2048)
    # an int64 count and 1024 candidate keys, one per workgroup, whatever the grid (the lm_head's: 950)
    assert need == 16 + 8 * 1024 and lib.bfly_q4_argmax_workspace_bytes(0, 2048) == 0
    head = (256, 512, 768, 1e-6, 1024, 1280, 1536, 151936, 2048, 64, 2048)
    assert lib.bfly_add_rms_norm_q4_gemv_argmax(*head, 0x8000, need - 1, None) == _native.ERR_INVALID
    assert b"workspace" in lib.bfly_last_error()
    assert lib.bfly_add_rms_norm_q4_gemv_argmax(*head, 0x8008, need, None) == _native.ERR_INVALID
    adv = lib.bfly_greedy_advance
    assert adv(0x1000, need, 0x2000, 100, 2044, 0x3000, 0x4000, 0x5000, 8, 0x6000, None) == \
        _native.ERR_INVALID                                      # hidden not a multiple of 8
    assert adv(0x1000, need, 0x2008, 100, 2048, 0x3000, 0x4000, 0x5000, 8, 0x6000, None) == \
        _native.ERR_INVALID                                      # embed misaligned
    assert adv(None, need, 0x2000, 100, 2048, 0x3000, 0x4000, 0x5000, 8, 0x6000, None) == _native.ERR_INVALID
    assert adv(0x1000, need - 8, 0x2000, 100, 2048, 0x3000, 0x4000, 0x5000, 8, 0x6000, None) == \
        _native.ERR_INVALID                                      # a workspace short of the 1024 slots
    assert b"workspace_bytes" in lib.bfly_last_error()


def test_decode_step_checks_the_cache_window_before_launch():
    """The cache's own window must be positive, below 2^20, and fit the ring with a block."""
    lib = _native.lib()
    head = (256, _native.DTYPE_BF16, 1, 8, 2, 128, 512, 768, 1024, 1280, 256, 1536, 1792, 16, 2048, 0, 3, 1, 1, 1,
            128, 64)
    for cw in (0, 200, 1 << 20):                      # 200 + 128 rows do not fit a ring of 256
        assert lib.bfly_decode_step(*head, cw, 0.088, 0x3000, None) == _native.ERR_INVALID
        assert b"cache_window" in lib.bfly_last_error()


def test_noalloc_argmax_refuses_before_any_device_call():
    """Row counts beyond the static workspace and bad shapes fail before any HIP call (fake addresses)."""
    lib = _native.lib()
    assert lib.bfly_argmax_rows_noalloc(0x1000, 65, 16, 16, 1, 0x2000, None) == _native.ERR_INVALID
    assert b"64" in lib.bfly_last_error()
    assert lib.bfly_argmax_rows_noalloc(0x1000, 0, 16, 16, 1, 0x2000, None) == _native.ERR_INVALID
    assert lib.bfly_argmax_rows_noalloc(None, 2, 16, 16, 1, 0x2000, None) == _native.ERR_INVALID


@pytest.mark.parametrize("args,msg", [
    ((256, 512, 768, 1e-6, 1024, 1280, 1536, 8, 8192, 64, 2048, None), b"2048, 4096 or 6144"),
    ((256, 512, 768, 1e-6, 1024, 1280, 1536, 8, 3072, 64, 2048, None), b"2048, 4096 or 6144"),
    ((256, 520, 768, 1e-6, 1024, 1280, 1536, 8, 2048, 64, 2048, None), b"16-byte"),   # residual misaligned
    ((256, 512, 768, 1e-6, None, 1280, 1536, 8, 2048, 64, 2048, None), b"both"),      # residual without h_out
    ((256, 512, None, 1e-6, 1024, 1280, 1536, 8, 2048, 64, 2048, None), b"norm weight"),
])
def test_add_rms_norm_q4_gemv_validates_before_launch(args, msg):
    """Fake, never dereferenced addresses: every case fails its checks before a launch."""
    lib = _native.lib()
    assert lib.bfly_add_rms_norm_q4_gemv(*args) == _native.ERR_INVALID
    assert msg in lib.bfly_last_error()
    *head, out, st = args
    assert lib.bfly_add_rms_norm_q4_gemv_silu(*head, head[7], out, st) == _native.ERR_INVALID
    assert msg in lib.bfly_last_error()
