"""CPU tests of the C ABI: the library loads, exports every symbol that
include/goinfer_paged.h declares, and the host allocator (the C++ form of
pkg/engine/paged_kv.go:49-148) behaves like the reference's, checked against
the reference's own test and the oracle's restatement.  No kernel runs."""
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "goinfer_paged.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_binding_knows(gi):
    assert declared_functions() == sorted(gi.EXPORTS)


def test_library_exports_every_declared_symbol(gi):
    lib = gi.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_nm_exports(gi):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", gi.LIB_PATH], stdout=subprocess.PIPE,
                         text=True, check=True).stdout
    syms = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [n for n in declared_functions() if n not in syms]
    assert not missing


def test_reference_paged_kv_test(gi):
    # pkg/engine/paged_kv_test.go:7-40, through the C ABI
    mgr = gi.PagedKVManager(4, 64, 10, 16)
    seq1 = mgr.AllocateSequence()
    assert seq1 == 1
    for _ in range(35):
        b, s = mgr.AppendToken(seq1)
        assert b >= 0 and 0 <= s < 16
    t = mgr.Tables[seq1]
    assert len(t.BlockIDs) == 3 and t.NumTokens == 35
    mgr.FreeSequence(seq1)
    assert len(mgr.FreeBlocks) == 10


def test_allocator_matches_oracle_restatement(gi, oracle):
    # Random interleaving of allocate / append / free against the Python
    # restatement of paged_kv.go; every returned pair and the free list must
    # agree.
    rng = np.random.default_rng(17)
    a = gi.PagedKVManager(2, 64, 40, 8)
    b = oracle.PagedKVManager(2, 64, 40, 8)
    live = []
    for step in range(3000):
        r = rng.random()
        if r < 0.05 or not live:
            sa, sb = a.AllocateSequence(), b.AllocateSequence()
            assert sa == sb
            live.append(sa)
        elif r < 0.1:
            sid = live.pop(int(rng.integers(len(live))))
            a.FreeSequence(sid)
            b.FreeSequence(sid)
        else:
            sid = live[int(rng.integers(len(live)))]
            try:
                want = b.AppendToken(sid)
            except oracle.OutOfPages:
                with pytest.raises(gi.GIError) as ei:
                    a.AppendToken(sid)
                assert ei.value.code == -4
                continue
            assert a.AppendToken(sid) == want
        if step % 97 == 0:
            assert a.FreeBlocks == b.FreeBlocks
    for sid in live:
        assert a.Tables[sid].BlockIDs == b.Tables[sid]["BlockIDs"]


def test_allocator_errors_and_bulk_append(gi):
    mgr = gi.PagedKVManager(1, 32, 4, 16)
    with pytest.raises(gi.GIError) as ei:
        mgr.AppendToken(7)                       # paged_kv.go:111-114
    assert ei.value.code == -6 and "not found" in str(ei.value)
    s = mgr.AllocateSequence()
    ids, slots = mgr.AppendTokens(s, 64)
    assert list(ids) == [3] * 16 + [2] * 16 + [1] * 16 + [0] * 16
    assert list(slots) == list(range(16)) * 4
    with pytest.raises(gi.GIError) as ei:
        mgr.AppendToken(s)                       # paged_kv.go:118-120
    assert ei.value.code == -4 and "out of paged KV memory" in str(ei.value)
    mgr.FreeSequence(12345)                      # unknown ids are ignored
    mgr.FreeSequence(s)
    assert mgr.FreeBlocks == [3, 2, 1, 0]
    # defaults of NewPagedKVManager (paged_kv.go:63-68)
    d = gi.PagedKVManager(1, 32, 0, 0)
    s = d.AllocateSequence()
    assert d.AppendToken(s) == (255, 0)


def test_set_free_list_shuffled_pool(gi):
    mgr = gi.PagedKVManager(1, 32, 8, 4)
    mgr.SetFreeList([5, 1, 7, 0, 2, 6, 3, 4])
    s = mgr.AllocateSequence()
    ids, _ = mgr.AppendTokens(s, 9)
    assert list(ids) == [4] * 4 + [3] * 4 + [6]
    with pytest.raises(gi.GIError):
        mgr.SetFreeList([4, 0])                 # 4 is held by the sequence
    with pytest.raises(gi.GIError):
        mgr.SetFreeList([0, 0])                 # repeated


def test_no_device_paths_fail_cleanly(gi):
    import ctypes
    lib = gi.lib()
    if lib.gi_device_count() > 0:
        pytest.skip("a device is visible")
    h = ctypes.c_void_p()
    rc = lib.gi_paged_create(2, 4, 64, 16, 8, 0, ctypes.byref(h))
    assert rc == -1 and not h.value
    buf = ctypes.create_string_buffer(64)
    assert lib.gi_device_name(buf, 64) == -1
    # shape errors are reported before any device work
    assert lib.gi_paged_create(2, 4, 60, 16, 8, 0, ctypes.byref(h)) == -3
    assert lib.gi_paged_create(2, 4, 64, 16, 8, 2, ctypes.byref(h)) in (-1, -3)
    assert lib.gi_paged_create(2, 4, 48, 16, 8, 2, ctypes.byref(h)) == -3   # q8_0: hd % 32
    assert lib.gi_paged_decode_attention(None, 0, 1, 8, None, None, None, 1, None, 1,
                                         ctypes.c_float(1.0)) == -3


def test_attn_scale_matches_reference_bits(gi):
    assert np.float32(gi.attn_scale(64)).view(np.uint32) == 0x3E000000
    assert np.float32(gi.attn_scale(128)).view(np.uint32) == 0x3DB504F3


def test_wrapper_shape_checks_refuse_before_the_kernels(gi):
    """A q/out, k/v or block-table size that does not match batch, heads and
    kv_dim would send the kernels past the ends of the buffers: the wrappers
    refuse it (GI_ERR_BAD_ARG) before any call reaches the library."""
    import torch
    p = object.__new__(gi.PagedKVCache)
    p._h = None
    p.num_layers, p.num_kv_heads, p.head_dim, p.page_tokens = 1, 8, 128, 16
    p.num_pages, p.kv_type, p.kv_dim = 4, gi.KV_F16, 1024

    def i32(*s):
        return torch.zeros(s, dtype=torch.int32)

    def f32(*s):
        return torch.zeros(s, dtype=torch.float32)

    cases = [
        lambda: p.Write(0, i32(3), i32(2), f32(3, 1024), f32(3, 1024)),
        lambda: p.Write(0, i32(3), i32(3), f32(2, 1024), f32(3, 1024)),
        lambda: p.WriteAtLen(0, i32(2, 4), i32(3), f32(3, 1024), f32(3, 1024)),
        lambda: p.WriteAtLen(0, i32(3, 4), i32(3), f32(3, 1000), f32(3, 1024)),
        lambda: p.Get(0, i32(2), 33),
        lambda: p.AttentionGQA(f32(2, 4096), f32(2, 4096), 0, i32(3, 4), i32(2), 32, 0.1),
        lambda: p.AttentionGQA(f32(2, 4096), f32(2, 4000), 0, i32(2, 4), i32(2), 32, 0.1),
        lambda: p.AttentionGQA(f32(2, 4096), f32(2, 4096), 0, i32(8), i32(2), 32, 0.1),
        lambda: p.DecodeStep(f32(2, 4096), f32(2, 4096), f32(2, 1000), f32(2, 1024), 0, i32(2, 4),
                             i32(2), 32, 0.1),
        lambda: p.RoPEDecodeStep(f32(2, 4096), f32(2, 4096), f32(2, 1024), f32(1, 1024), 0, i32(2, 4),
                                 i32(2), 32, 0.1),
        lambda: p.RoPEWrite(0, i32(2), i32(2), i32(2), f32(2, 4000), f32(2, 1024), f32(2, 1024)),
        lambda: p.RoPEWriteAtLen(0, i32(2, 4), i32(2), f32(2, 4096), f32(2, 1024), f32(3, 1024)),
        lambda: p.AttentionGQABatch(f32(2, 5, 4096), f32(2, 4, 4096), 0, i32(2, 4), i32(2), 32, 0.1, 5),
    ]
    for i, c in enumerate(cases):
        with pytest.raises(gi.GIError) as e:
            c()
        assert e.value.code == -3, i
        msg = str(e.value)
        assert "must be [" in msg or "must hold" in msg or "maps fewer" in msg, (i, msg)
