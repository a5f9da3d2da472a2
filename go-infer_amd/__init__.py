"""go-infer_amd: MI355X paged KV-cache path for go-infer.

Host-side mirror of the reference's interface for this path, over the C ABI
in include/goinfer_paged.h (libgoinfer_paged.so, hand-written HIP for gfx950):

  PagedKVManager  pkg/engine/paged_kv.go:49-148 (block allocator, C++ on the
                  host: NewPagedKVManager / AllocateSequence / AppendToken /
                  FreeSequence, Tables, FreeBlocks)
  PagedKVCache    the device page pool; Write / Get restate KVCache.Write /
                  Get (pkg/engine/kvcache.go:146-214) on pages, AttentionGQA /
                  AttentionGQABatch restate the decode and chunked-prefill
                  attention of pkg/engine/forward.go:242-267 / 547-577 (the
                  seams metal.AttentionGQA / AttentionGQABatch,
                  pkg/metal/metal_darwin.go:711-727, 963-981).

Errors are raised as GIError carrying the library's negative code, where the
Go code returns an error value.  Device buffers are torch tensors on the
pool's device; nothing here falls back to the CPU: if the library is not
built, loading it raises.
"""
import ctypes
import os

__all__ = ["lib", "GIError", "PagedKVManager", "PagedKVCache", "PrefixCache", "BatchDecoder", "Weights",
           "AttentionPlan",
           "GGML_F32", "GGML_F16", "GGML_Q4_0", "GGML_Q8_0", "KV_F32", "KV_F16",
           "KV_Q8_0", "KV_Q4_0", "EXPORTS", "LIB_PATH", "attn_scale"]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgoinfer_paged.so")

KV_F32, KV_F16, KV_Q8_0, KV_Q4_0 = 0, 1, 2, 3
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8    # pkg/gguf/types.go:25-31
GI_OK = 0
ERR_NAMES = {-1: "GI_ERR_NO_DEVICE", -2: "GI_ERR_OOM", -3: "GI_ERR_BAD_ARG",
             -4: "GI_ERR_POOL_EXHAUSTED", -5: "GI_ERR_HIP", -6: "GI_ERR_UNKNOWN_SEQ",
             -7: "GI_ERR_BAD_PAGE", -8: "GI_ERR_SHARED_PAGE"}

_c_int, _c_i64, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)
_intp = ctypes.POINTER(ctypes.c_int)



class AttentionPlan(ctypes.Structure):
    """gi_attention_plan: the launch plan gi_paged_attention_plan reports."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "decode_kernel", "decode_fallback", "decode_splits", "decode_split_tokens", "decode_waves",
        "decode_step_fused", "prefill_kernel", "prefill_fallback")]


# Every symbol include/goinfer_paged.h declares, with its ctypes signature.
EXPORTS = {
    "gi_last_error": (ctypes.c_char_p, []),
    "gi_device_count": (_c_int, []),
    "gi_device_name": (_c_int, [ctypes.c_char_p, _c_int]),
    "gi_kvmgr_create": (_c_int, [_c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_vp)]),
    "gi_kvmgr_destroy": (None, [_vp]),
    "gi_kvmgr_allocate_sequence": (_c_int, [_vp, _intp]),
    "gi_kvmgr_append_token": (_c_int, [_vp, _c_int, _i32p, _i32p]),
    "gi_kvmgr_append_tokens": (_c_int, [_vp, _c_int, _c_int, _i32p, _i32p, _intp]),
    "gi_kvmgr_free_sequence": (_c_int, [_vp, _c_int]),
    "gi_kvmgr_block_table": (_c_int, [_vp, _c_int, _i32p, _c_int, _intp, _intp]),
    "gi_kvmgr_free_list": (_c_int, [_vp, _i32p, _c_int, _intp]),
    "gi_kvmgr_set_free_list": (_c_int, [_vp, _i32p, _c_int]),
    "gi_kvmgr_fork_sequence": (_c_int, [_vp, _c_int, _c_int, _intp]),
    "gi_kvmgr_append_token_cow": (_c_int, [_vp, _c_int, _i32p, _i32p, _i32p]),
    "gi_kvmgr_append_tokens_cow": (_c_int, [_vp, _c_int, _c_int, _i32p, _i32p, _i32p, _i32p, _intp]),
    "gi_kvmgr_block_refs": (_c_int, [_vp, ctypes.c_int32, _intp]),
    "gi_kvmgr_block_size": (_c_int, [_vp]),
    "gi_kvmgr_append_batch": (_c_int, [_vp, _c_int, _intp, _i32p, _i32p, _i32p]),
    "gi_weights_upload": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, ctypes.POINTER(_vp)]),
    "gi_weights_destroy": (None, [_vp]),
    "gi_matmul_batch": (_c_int, [_vp, _c_int, _vp, _vp]),
    "gi_batch_create": (_c_int, [_vp, _vp, _c_int, _c_int, ctypes.POINTER(_vp)]),
    "gi_batch_destroy": (None, [_vp]),
    "gi_batch_add": (_c_int, [_vp, _c_int, _intp]),
    "gi_batch_remove": (_c_int, [_vp, _c_int]),
    "gi_batch_step": (_c_int, [_vp, _intp]),
    "gi_batch_rows": (_c_int, [_vp, _i32p, _i32p, _c_int, _intp]),
    "gi_batch_row_table": (_c_int, [_vp, _c_int, _i32p, _c_int, _intp]),
    "gi_batch_device_tables": (_c_int, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _intp]),
    "gi_batch_decode_layer": (_c_int, [_vp, _c_int, _c_int, _vp, _vp, _vp, _vp, ctypes.c_float,
                                       _c_int]),
    "gi_prefix_create": (_c_int, [_vp, _c_int, ctypes.POINTER(_vp)]),
    "gi_prefix_destroy": (None, [_vp]),
    "gi_prefix_store": (_c_int, [_vp, _i32p, _c_int, _c_int]),
    "gi_prefix_find_longest": (_c_int, [_vp, _i32p, _c_int, _intp, _intp]),
    "gi_prefix_size": (_c_int, [_vp, _intp]),
    "gi_paged_copy_pages": (_c_int, [_vp, _c_int, _vp, _vp]),
    "gi_paged_create": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_i64, _c_int,
                                 ctypes.POINTER(_vp)]),
    "gi_paged_destroy": (None, [_vp]),
    "gi_paged_page_bytes": (_c_int, [_vp, ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64)]),
    "gi_paged_set_stream": (_c_int, [_vp, _vp]),
    "gi_paged_stream": (_vp, [_vp]),
    "gi_synchronize": (_c_int, [_vp]),
    "gi_dev_alloc": (_c_int, [_vp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "gi_dev_free": (_c_int, [_vp, _vp]),
    "gi_memcpy_h2d": (_c_int, [_vp, _vp, _vp, ctypes.c_size_t]),
    "gi_memcpy_d2h": (_c_int, [_vp, _vp, _vp, ctypes.c_size_t]),
    "gi_paged_append": (_c_int, [_vp, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "gi_paged_append_at_len": (_c_int, [_vp, _c_int, _c_int, _vp, _c_int, _vp, _vp, _vp]),
    "gi_paged_gather": (_c_int, [_vp, _c_int, _vp, _c_int, _vp, _vp, _c_int]),
    "gi_paged_decode_attention": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int,
                                           _vp, _c_int, ctypes.c_float]),
    "gi_paged_decode_attention_noalloc": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp,
                                                   _c_int, _vp, _c_int, ctypes.c_float]),
    "gi_paged_decode_step": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp,
                                      _c_int, _vp, _c_int, ctypes.c_float]),
    "gi_paged_prefill_attention": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp,
                                            _c_int, _vp, ctypes.c_float]),
    "gi_paged_set_rope": (_c_int, [_vp, ctypes.c_float, _c_int, _c_int]),
    "gi_paged_rope_append": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _vp]),
    "gi_paged_rope_append_at_len": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp, _vp,
                                             _vp, _vp, _vp]),
    "gi_paged_rope_decode_step": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp,
                                           _c_int, _vp, _c_int, ctypes.c_float]),
    "gi_paged_decode_kernel": (_c_int, [_vp, _c_int]),
    "gi_paged_attention_plan": (_c_int, [_vp, _c_int, _c_int, _c_int, ctypes.POINTER(AttentionPlan)]),
    "gi_paged_set_decode_kernel": (_c_int, [_vp, _c_int]),
}

_lib = None


def lib():
    """Loads libgoinfer_paged.so (built by go-infer_amd/build.py).  Raises if
    it is missing: there is no other implementation to fall back to."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libgoinfer_paged.so is not built: run python go-infer_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class GIError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("%s (%d): %s" % (ERR_NAMES.get(code, "GI_ERR"), code, msg))
        self.code = code


def _check(rc):
    if rc != GI_OK:
        msg = lib().gi_last_error()
        raise GIError(rc, msg.decode() if msg else "")
    return rc


def attn_scale(head_dim):
    """float32(1 / math_sqrt(head_dim)) (pkg/engine/forward.go:33, 771-780):
    ten Newton steps from x/2 in float64, then rounded to float32."""
    import numpy as np
    x = float(head_dim)
    if x <= 0:
        return np.float32(0.0)
    z = x / 2
    for _ in range(10):
        z = (z + x / z) / 2
    return np.float32(1.0 / z)


class _Table:
    """BlockTable (paged_kv.go:41-46) snapshot."""

    def __init__(self, seq_id, ids, num_tokens, block_size):
        self.SequenceID, self.BlockIDs, self.NumTokens, self.BlockSize = (
            seq_id, ids, num_tokens, block_size)


class PagedKVManager:
    """NewPagedKVManager(numLayers, kvDim, totalBlocks, blockSize)
    (paged_kv.go:62-87), backed by the C++ allocator in the library."""

    def __init__(self, num_layers, kv_dim, total_blocks, block_size):
        h = _vp()
        _check(lib().gi_kvmgr_create(num_layers, kv_dim, total_blocks, block_size,
                                     ctypes.byref(h)))
        self._h = h
        self.NumLayers, self.KVDim = num_layers, kv_dim
        self.BlockSize = block_size if block_size > 0 else 16
        self.TotalBlocks = total_blocks if total_blocks > 0 else 256

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.gi_kvmgr_destroy(h)
            self._h = None

    def AllocateSequence(self):
        sid = _c_int()
        _check(lib().gi_kvmgr_allocate_sequence(self._h, ctypes.byref(sid)))
        return sid.value

    def AppendToken(self, seq_id):
        """Returns (blockID, slotOffset); raises GIError with
        GI_ERR_UNKNOWN_SEQ / GI_ERR_POOL_EXHAUSTED (paged_kv.go:111-120)."""
        b, s = ctypes.c_int32(), ctypes.c_int32()
        _check(lib().gi_kvmgr_append_token(self._h, seq_id, ctypes.byref(b), ctypes.byref(s)))
        return b.value, s.value

    def AppendTokens(self, seq_id, n):
        """n AppendToken calls; returns (block_ids, slots) int32 arrays."""
        import numpy as np
        ids = np.zeros(max(n, 1), np.int32)
        slots = np.zeros(max(n, 1), np.int32)
        done = _c_int()
        _check(lib().gi_kvmgr_append_tokens(self._h, seq_id, n, ids.ctypes.data_as(_i32p),
                                            slots.ctypes.data_as(_i32p), ctypes.byref(done)))
        return ids[:n], slots[:n]

    def FreeSequence(self, seq_id):
        _check(lib().gi_kvmgr_free_sequence(self._h, seq_id))

    def BlockTable(self, seq_id):
        import numpy as np
        nb, nt = _c_int(), _c_int()
        _check(lib().gi_kvmgr_block_table(self._h, seq_id, None, 0, ctypes.byref(nb),
                                          ctypes.byref(nt)))
        ids = np.zeros(max(nb.value, 1), np.int32)
        _check(lib().gi_kvmgr_block_table(self._h, seq_id, ids.ctypes.data_as(_i32p), ids.size,
                                          ctypes.byref(nb), ctypes.byref(nt)))
        return _Table(seq_id, [int(x) for x in ids[:nb.value]], nt.value, self.BlockSize)

    @property
    def Tables(self):
        """Lookup by sequence id: mgr.Tables[seq].BlockIDs / .NumTokens."""
        mgr = self

        class _View:
            def __getitem__(self, sid):
                return mgr.BlockTable(sid)

            def __contains__(self, sid):
                try:
                    mgr.BlockTable(sid)
                    return True
                except GIError:
                    return False
        return _View()

    @property
    def FreeBlocks(self):
        import numpy as np
        n = _c_int()
        _check(lib().gi_kvmgr_free_list(self._h, None, 0, ctypes.byref(n)))
        ids = np.zeros(max(n.value, 1), np.int32)
        _check(lib().gi_kvmgr_free_list(self._h, ids.ctypes.data_as(_i32p), ids.size,
                                        ctypes.byref(n)))
        return [int(x) for x in ids[:n.value]]

    def SetFreeList(self, ids):
        import numpy as np
        a = np.ascontiguousarray(ids, np.int32)
        _check(lib().gi_kvmgr_set_free_list(self._h, a.ctypes.data_as(_i32p), a.size))

    # -- copy-on-write prefix sharing (replaces KVCache.ForkAt deep copies) --
    def ForkSequence(self, src_seq, n_tokens):
        """ForkAt(n_tokens) (kvcache.go:225-284) over shared pages: a new
        sequence holding src_seq's first n_tokens tokens."""
        sid = _c_int()
        _check(lib().gi_kvmgr_fork_sequence(self._h, src_seq, n_tokens, ctypes.byref(sid)))
        return sid.value

    def AppendTokenCOW(self, seq_id):
        """AppendToken with copy-on-write: (blockID, slot, copy_from), where
        copy_from is -1 or the shared block to copy into blockID first."""
        b, s, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        _check(lib().gi_kvmgr_append_token_cow(self._h, seq_id, ctypes.byref(b), ctypes.byref(s),
                                               ctypes.byref(c)))
        return b.value, s.value, c.value

    def AppendTokensCOW(self, seq_id, n):
        """n tokens: (block_ids, slots, (copy_src, copy_dst)), the copy pair
        (-1, -1) when no shared block was touched."""
        import numpy as np
        ids = np.zeros(max(n, 1), np.int32)
        slots = np.zeros(max(n, 1), np.int32)
        cs, cd = ctypes.c_int32(), ctypes.c_int32()
        done = _c_int()
        _check(lib().gi_kvmgr_append_tokens_cow(self._h, seq_id, n, ids.ctypes.data_as(_i32p),
                                                slots.ctypes.data_as(_i32p), ctypes.byref(cs),
                                                ctypes.byref(cd), ctypes.byref(done)))
        return ids[:n], slots[:n], (cs.value, cd.value)

    def BlockRefs(self, block_id):
        r = _c_int()
        _check(lib().gi_kvmgr_block_refs(self._h, block_id, ctypes.byref(r)))
        return r.value

    def AppendBatch(self, seq_ids):
        """One copy-on-write AppendToken per sequence, all or nothing:
        (block_ids, slots, copy_src) int32 arrays, copy_src -1 where no
        shared block was copied."""
        import numpy as np
        ids = np.ascontiguousarray(seq_ids, np.int32)
        n = ids.size
        b = np.zeros(max(n, 1), np.int32)
        sl = np.zeros(max(n, 1), np.int32)
        cf = np.zeros(max(n, 1), np.int32)
        _check(lib().gi_kvmgr_append_batch(self._h, n, ids.ctypes.data_as(_intp),
                                           b.ctypes.data_as(_i32p), sl.ctypes.data_as(_i32p),
                                           cf.ctypes.data_as(_i32p)))
        return b[:n], sl[:n], cf[:n]


class PrefixCache:
    """NewPrefixCache(maxSize) (prefix_cache.go:20-28) over a PagedKVManager:
    entries share pages with the sequences they were stored from, and a hit
    returns a new sequence forked from the entry instead of a deep copy."""

    def __init__(self, mgr, max_size):
        h = _vp()
        _check(lib().gi_prefix_create(mgr._h, max_size, ctypes.byref(h)))
        self._h, self._mgr = h, mgr

    def close(self):
        # The entries hold pages of the manager; if the garbage collector
        # finalised the manager first (objects in one reference cycle are
        # finalised in no set order), those pages went with it and the
        # cache's own destroy, which releases them through the manager, is
        # skipped.
        if self._h and _lib is not None and getattr(self._mgr, "_h", None):
            _lib.gi_prefix_destroy(self._h)
        self._h = None

    def __del__(self):
        if getattr(self, "_h", None):
            self.close()

    def Store(self, tokens, seq_id):
        """Store(tokens, kv) (prefix_cache.go:97-119); kv is the sequence."""
        import numpy as np
        a = np.ascontiguousarray(tokens, np.int32)
        _check(lib().gi_prefix_store(self._h, a.ctypes.data_as(_i32p), a.size, seq_id))

    def FindLongestPrefix(self, tokens):
        """(matched length, new sequence id) or (0, None)
        (prefix_cache.go:76-95)."""
        import numpy as np
        a = np.ascontiguousarray(tokens, np.int32)
        m, sid = _c_int(), _c_int()
        _check(lib().gi_prefix_find_longest(self._h, a.ctypes.data_as(_i32p), a.size,
                                            ctypes.byref(m), ctypes.byref(sid)))
        return (m.value, sid.value) if m.value else (0, None)

    def __len__(self):
        n = _c_int()
        _check(lib().gi_prefix_size(self._h, ctypes.byref(n)))
        return n.value


def _ptr(t, dtype=None, what="tensor"):
    """Device pointer of a contiguous torch tensor (None -> NULL)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise GIError(-3, "%s must be a device tensor" % what)
    if not t.is_contiguous():
        raise GIError(-3, "%s must be contiguous" % what)
    if dtype is not None and t.dtype != dtype:
        raise GIError(-3, "%s must be %s, got %s" % (what, dtype, t.dtype))
    return _vp(t.data_ptr())


def _run(call):
    """Makes a (C function name, arguments) call and raises on failure."""
    name, args = call
    _check(getattr(lib(), name)(*args))


def _need(ok, msg):
    """Shape check of a wrapper: a mismatch would send the kernels past the
    ends of the buffers, so it is refused here as GI_ERR_BAD_ARG."""
    if not ok:
        raise GIError(-3, msg)


def _numel(t):
    return 0 if t is None else int(t.numel())


def _tables(block_tables, batch, what="block_tables"):
    """max_blocks of a [batch, max_blocks] table (0 for an empty batch)."""
    if batch == 0:
        return 0
    _need(block_tables is not None and block_tables.dim() == 2 and int(block_tables.shape[0]) == batch,
          "%s must be [batch=%d, max_blocks]" % (what, batch))
    return int(block_tables.shape[1])


class PagedKVCache:
    """Device page pool for num_layers layers (one page id covers every
    layer, like KVBlock in paged_kv.go:13-38).  kv_type: KV_F32, KV_F16,
    KV_Q8_0 or KV_Q4_0."""

    def __init__(self, num_layers, num_kv_heads, head_dim, page_tokens, num_pages,
                 kv_type=KV_F32, stream=None):
        """stream: a torch.cuda.Stream (default: torch's current stream), so
        the pool's kernels are ordered with the torch work that produces and
        consumes its device buffers."""
        import torch
        h = _vp()
        _check(lib().gi_paged_create(num_layers, num_kv_heads, head_dim, page_tokens, num_pages,
                                     kv_type, ctypes.byref(h)))
        self._h = h
        if stream is None:
            stream = torch.cuda.current_stream()
        self.set_stream(stream.cuda_stream)
        self.num_layers, self.num_kv_heads, self.head_dim = num_layers, num_kv_heads, head_dim
        self.page_tokens, self.num_pages, self.kv_type = page_tokens, num_pages, kv_type
        self.kv_dim = num_kv_heads * head_dim

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.gi_paged_destroy(self._h)
        self._h = None

    def __del__(self):
        self.close()

    @property
    def handle(self):
        return self._h

    def bytes_per_vec(self):
        """Stored bytes of one token vector (kvcache.go:92-105: q8_0 is
        ((kvDim+31)/32)*34, q4_0 ((kvDim+31)/32)*18)."""
        if self.kv_type == KV_F32:
            return 4 * self.kv_dim
        if self.kv_type == KV_F16:
            return 2 * self.kv_dim
        if self.kv_type == KV_Q4_0:
            return (self.kv_dim + 31) // 32 * 18
        return (self.kv_dim + 31) // 32 * 34

    def page_bytes(self):
        pb, tot = _c_i64(), _c_i64()
        _check(lib().gi_paged_page_bytes(self._h, ctypes.byref(pb), ctypes.byref(tot)))
        return pb.value, tot.value

    def set_stream(self, stream_handle):
        """Raw hipStream_t value (0 = HIP's default stream)."""
        _check(lib().gi_paged_set_stream(self._h, _vp(stream_handle) if stream_handle else None))

    def stream(self):
        return lib().gi_paged_stream(self._h)

    def synchronize(self):
        _check(lib().gi_synchronize(self._h))

    def decode_kernel(self, num_heads):
        """0: vector-ALU kernel, 1: matrix-core kernel."""
        return lib().gi_paged_decode_kernel(self._h, num_heads)

    def attention_plan(self, batch, num_heads, max_seq_len=0):
        """gi_paged_attention_plan as a dict: kernel family, split plan,
        waves per workgroup and whether the decode step's token store is
        fused, for this pool and shape (nothing is launched)."""
        p = AttentionPlan()
        _check(lib().gi_paged_attention_plan(self._h, int(batch), int(num_heads), int(max_seq_len),
                                             ctypes.byref(p)))
        return {n: getattr(p, n) for n, _ in AttentionPlan._fields_}

    def decode_step_fuses(self, batch, num_heads, max_seq_len=0):
        """Whether gi_paged_decode_step stores the token inside the decode
        launch for this shape (else in an append launch before it)."""
        return self.attention_plan(batch, num_heads, max_seq_len)["decode_step_fused"] == 1

    def set_decode_kernel(self, kind):
        """-1 automatic, 0 vector ALU, 1 matrix core where supported."""
        _check(lib().gi_paged_set_decode_kernel(self._h, kind))

    # -- KVCache.Write / Get on pages ------------------------------------
    def Write(self, layer, block_ids, slots, k, v):
        """Stores token vectors k, v [n, kv_dim] float32 at (block_ids[i],
        slots[i]) of one layer (KVCache.Write, kvcache.go:146-180)."""
        import torch
        n = int(block_ids.numel())
        _need(_numel(slots) == n, "Write: slots must hold %d entries" % n)
        _need(_numel(k) == n * self.kv_dim and _numel(v) == n * self.kv_dim,
              "Write: k and v must be [%d, %d]" % (n, self.kv_dim))
        _check(lib().gi_paged_append(self._h, layer, n, _ptr(block_ids, torch.int32, "block_ids"),
                                     _ptr(slots, torch.int32, "slots"),
                                     _ptr(k, torch.float32, "k"), _ptr(v, torch.float32, "v")))

    def WriteAtLen(self, layer, block_tables, seq_lens, k, v):
        _run(self._write_at_len(layer, block_tables, seq_lens, k, v))

    def _write_at_len(self, layer, block_tables, seq_lens, k, v):
        import torch
        batch = int(seq_lens.numel())
        mb = _tables(block_tables, batch)
        _need(_numel(k) == batch * self.kv_dim and _numel(v) == batch * self.kv_dim,
              "WriteAtLen: k and v must be [%d, %d]" % (batch, self.kv_dim))
        return ("gi_paged_append_at_len",
                (self._h, layer, batch, _ptr(block_tables, torch.int32, "block_tables"),
                 mb, _ptr(seq_lens, torch.int32, "seq_lens"),
                 _ptr(k, torch.float32, "k"), _ptr(v, torch.float32, "v")))

    def Get(self, layer, block_table, n_tok, widen=False):
        """Contiguous K, V of tokens [0, n_tok) (KVCache.Get/ForkAt layout).
        widen=False: stored bytes as uint8 [n_tok, bytes_per_vec];
        widen=True: float32 [n_tok, kv_dim]."""
        import torch
        dev = block_table.device
        _need(n_tok >= 0 and _numel(block_table) * self.page_tokens >= n_tok,
              "Get: block_table maps fewer than %d tokens" % n_tok)
        if widen:
            ko = torch.empty((n_tok, self.kv_dim), dtype=torch.float32, device=dev)
        else:
            ko = torch.empty((n_tok, self.bytes_per_vec()), dtype=torch.uint8, device=dev)
        vo = torch.empty_like(ko)
        _check(lib().gi_paged_gather(self._h, layer, _ptr(block_table, torch.int32, "block_table"),
                                     n_tok, _ptr(ko), _ptr(vo), 1 if widen else 0))
        return ko, vo

    def CopyPages(self, src_ids, dst_ids):
        """Page dst_ids[i] <- page src_ids[i] in every layer (device int32
        tensors): the copy a copy-on-write append asks for."""
        import torch
        n = int(src_ids.numel())
        if int(dst_ids.numel()) != n:
            raise GIError(-3, "CopyPages: src_ids and dst_ids differ in length")
        _check(lib().gi_paged_copy_pages(self._h, n, _ptr(src_ids, torch.int32, "src_ids"),
                                         _ptr(dst_ids, torch.int32, "dst_ids")))

    # -- attention -------------------------------------------------------
    def AttentionGQA(self, out, q, layer, block_tables, seq_lens, num_heads, attn_scale,
                     max_seq_len=None):
        """Decode attention of forward.go:242-267 for a batch; q/out
        [batch, num_heads*head_dim] float32."""
        _run(self._attention_gqa(out, q, layer, block_tables, seq_lens, num_heads, attn_scale,
                                 max_seq_len))

    def _attention_gqa(self, out, q, layer, block_tables, seq_lens, num_heads, attn_scale,
                       max_seq_len=None):
        import torch
        batch = int(seq_lens.numel())
        mb = _tables(block_tables, batch)
        qn = batch * num_heads * self.head_dim
        _need(_numel(q) == qn and _numel(out) == qn,
              "AttentionGQA: q and out must be [%d, %d]" % (batch, num_heads * self.head_dim))
        if max_seq_len is None:
            max_seq_len = 0   # the kernels read the lengths on the device
        return ("gi_paged_decode_attention",
                (self._h, layer, batch, num_heads, _ptr(q, torch.float32, "q"),
                 _ptr(out, torch.float32, "out"), _ptr(block_tables, torch.int32, "block_tables"),
                 mb, _ptr(seq_lens, torch.int32, "seq_lens"),
                 int(max_seq_len), float(attn_scale)))

    def AttentionGQANoAlloc(self, out, q, layer, block_tables, seq_lens, num_heads, attn_scale,
                            max_seq_len=None):
        """AttentionGQA through the entry point that allocates nothing (its
        split partials in the library's fixed per-device scratch)."""
        import torch
        batch = int(seq_lens.numel())
        mb = _tables(block_tables, batch)
        qn = batch * num_heads * self.head_dim
        _need(_numel(q) == qn and _numel(out) == qn,
              "AttentionGQANoAlloc: q and out must be [%d, %d]" % (batch, num_heads * self.head_dim))
        _check(lib().gi_paged_decode_attention_noalloc(
            self._h, layer, batch, num_heads, _ptr(q, torch.float32, "q"),
            _ptr(out, torch.float32, "out"), _ptr(block_tables, torch.int32, "block_tables"),
            mb, _ptr(seq_lens, torch.int32, "seq_lens"), int(max_seq_len or 0), float(attn_scale)))

    def DecodeStep(self, out, q, k, v, layer, block_tables, seq_lens, num_heads, attn_scale,
                   max_seq_len=None):
        """Append the new token at position seq_lens[b]-1, then decode
        attention over seq_lens[b] tokens (forward.go:236-267)."""
        _run(self._decode_step(out, q, k, v, layer, block_tables, seq_lens, num_heads, attn_scale,
                               max_seq_len))

    def _decode_step(self, out, q, k, v, layer, block_tables, seq_lens, num_heads, attn_scale,
                     max_seq_len=None):
        import torch
        batch = int(seq_lens.numel())
        mb = _tables(block_tables, batch)
        qn = batch * num_heads * self.head_dim
        _need(_numel(q) == qn and _numel(out) == qn,
              "DecodeStep: q and out must be [%d, %d]" % (batch, num_heads * self.head_dim))
        _need(_numel(k) == batch * self.kv_dim and _numel(v) == batch * self.kv_dim,
              "DecodeStep: k and v must be [%d, %d]" % (batch, self.kv_dim))
        if max_seq_len is None:
            max_seq_len = 0
        return ("gi_paged_decode_step",
                (self._h, layer, batch, num_heads, _ptr(q, torch.float32, "q"),
                 _ptr(k, torch.float32, "k"), _ptr(v, torch.float32, "v"),
                 _ptr(out, torch.float32, "out"), _ptr(block_tables, torch.int32, "block_tables"),
                 mb, _ptr(seq_lens, torch.int32, "seq_lens"),
                 int(max_seq_len), float(attn_scale)))

    # -- RoPE fused with the append (forward.go:228-240, 527-545) ------------
    def SetRoPE(self, theta, rope_dim=0, max_positions=8192):
        """Table of ApplyRoPE's (cos, sin) (pkg/math/kernels.go:22-35) for
        positions [0, max_positions); rope_dim 0 means head_dim."""
        _check(lib().gi_paged_set_rope(self._h, float(theta), int(rope_dim), int(max_positions)))

    def RoPEWrite(self, layer, positions, block_ids, slots, q, k, v, q_out=None):
        """ApplyRoPE on q [n, num_heads*head_dim] (into q_out, default in
        place) and k [n, kv_dim] at positions[i], then Write of k, v."""
        import torch
        n = int(block_ids.numel())
        num_heads = 0
        if q is not None:
            num_heads = int(q.shape[-1]) // self.head_dim
            if q_out is None:
                q_out = q
            _need(_numel(q) == n * num_heads * self.head_dim and _numel(q_out) == _numel(q),
                  "RoPEWrite: q and q_out must be [%d, num_heads * %d]" % (n, self.head_dim))
        _need(_numel(slots) == n and _numel(positions) == n, "RoPEWrite: positions and slots "
              "must hold %d entries" % n)
        _need(_numel(k) == n * self.kv_dim and _numel(v) == n * self.kv_dim,
              "RoPEWrite: k and v must be [%d, %d]" % (n, self.kv_dim))
        _check(lib().gi_paged_rope_append(
            self._h, layer, n, num_heads, _ptr(positions, torch.int32, "positions"),
            _ptr(block_ids, torch.int32, "block_ids"), _ptr(slots, torch.int32, "slots"),
            _ptr(q, torch.float32, "q"), _ptr(q_out, torch.float32, "q_out"),
            _ptr(k, torch.float32, "k"), _ptr(v, torch.float32, "v")))

    def RoPEWriteAtLen(self, layer, block_tables, seq_lens, q, k, v, q_out=None):
        """Decode form: token b at position seq_lens[b]-1 of sequence b."""
        _run(self._rope_write_at_len(layer, block_tables, seq_lens, q, k, v, q_out))

    def _rope_write_at_len(self, layer, block_tables, seq_lens, q, k, v, q_out=None):
        import torch
        batch = int(seq_lens.numel())
        mb = _tables(block_tables, batch)
        num_heads = 0
        if q is not None:
            num_heads = int(q.shape[-1]) // self.head_dim
            if q_out is None:
                q_out = q
            _need(_numel(q) == batch * num_heads * self.head_dim and _numel(q_out) == _numel(q),
                  "RoPEWriteAtLen: q and q_out must be [%d, num_heads * %d]" % (batch, self.head_dim))
        _need(_numel(k) == batch * self.kv_dim and _numel(v) == batch * self.kv_dim,
              "RoPEWriteAtLen: k and v must be [%d, %d]" % (batch, self.kv_dim))
        return ("gi_paged_rope_append_at_len",
                (self._h, layer, batch, num_heads, _ptr(block_tables, torch.int32, "block_tables"),
                 mb, _ptr(seq_lens, torch.int32, "seq_lens"),
                 _ptr(q, torch.float32, "q"), _ptr(q_out, torch.float32, "q_out"),
                 _ptr(k, torch.float32, "k"), _ptr(v, torch.float32, "v")))

    def RoPEDecodeStep(self, out, q, k, v, layer, block_tables, seq_lens, num_heads, attn_scale,
                       max_seq_len=None):
        """forward.go:228-267 for a batch: q (rotated in place) and k turned
        at position seq_lens[b]-1, k/v appended, then decode attention."""
        _run(self._rope_decode_step(out, q, k, v, layer, block_tables, seq_lens, num_heads,
                                    attn_scale, max_seq_len))

    def _rope_decode_step(self, out, q, k, v, layer, block_tables, seq_lens, num_heads, attn_scale,
                          max_seq_len=None):
        import torch
        batch = int(seq_lens.numel())
        mb = _tables(block_tables, batch)
        qn = batch * num_heads * self.head_dim
        _need(_numel(q) == qn and _numel(out) == qn,
              "RoPEDecodeStep: q and out must be [%d, %d]" % (batch, num_heads * self.head_dim))
        _need(_numel(k) == batch * self.kv_dim and _numel(v) == batch * self.kv_dim,
              "RoPEDecodeStep: k and v must be [%d, %d]" % (batch, self.kv_dim))
        if max_seq_len is None:
            max_seq_len = 0
        return ("gi_paged_rope_decode_step",
                (self._h, layer, batch, num_heads, _ptr(q, torch.float32, "q"),
                 _ptr(k, torch.float32, "k"), _ptr(v, torch.float32, "v"),
                 _ptr(out, torch.float32, "out"), _ptr(block_tables, torch.int32, "block_tables"),
                 mb, _ptr(seq_lens, torch.int32, "seq_lens"),
                 int(max_seq_len), float(attn_scale)))

    # -- prepared calls ------------------------------------------------------
    _PREPARABLE = {"WriteAtLen": "_write_at_len", "AttentionGQA": "_attention_gqa",
                   "DecodeStep": "_decode_step", "RoPEWriteAtLen": "_rope_write_at_len",
                   "RoPEDecodeStep": "_rope_decode_step"}

    def Prepare(self, method, *args, **kw):
        """One of WriteAtLen / AttentionGQA / DecodeStep / RoPEWriteAtLen /
        RoPEDecodeStep with its arguments checked and converted once: returns
        a function of no arguments that makes the same C call, as a compiled
        host repeats a call whose buffers it keeps (each call costs the C
        ABI's own host time, not the wrapper's checks).  The tensors must
        stay alive, in place and unchanged in shape while it is used."""
        if method not in self._PREPARABLE:
            raise GIError(-3, "Prepare: %s is not one of %s" % (method, sorted(self._PREPARABLE)))
        name, cargs = getattr(self, self._PREPARABLE[method])(*args, **kw)
        fn = getattr(lib(), name)
        conv = tuple(a if isinstance(a, c) else c(a) for c, a in zip(fn.argtypes, cargs))

        def call():
            rc = fn(*conv)
            if rc != GI_OK:
                _check(rc)
        return call

    def AttentionGQABatch(self, out, q, layer, block_tables, start_pos, num_heads, attn_scale,
                          chunk_len):
        """Chunked-prefill causal attention of forward.go:547-577; q/out
        [batch, chunk_len, num_heads*head_dim] float32."""
        import torch
        batch = int(start_pos.numel())
        mb = _tables(block_tables, batch)
        qn = batch * chunk_len * num_heads * self.head_dim
        _need(_numel(q) == qn and _numel(out) == qn,
              "AttentionGQABatch: q and out must be [%d, %d, %d]"
              % (batch, chunk_len, num_heads * self.head_dim))
        _check(lib().gi_paged_prefill_attention(
            self._h, layer, batch, chunk_len, num_heads, _ptr(q, torch.float32, "q"),
            _ptr(out, torch.float32, "out"), _ptr(block_tables, torch.int32, "block_tables"),
            mb, _ptr(start_pos, torch.int32, "start_pos"),
            float(attn_scale)))


class BatchDecoder:
    """Continuous-batching decode driver (gi_batch_*): a dense running set of
    sequences over a PagedKVManager and (optionally) a PagedKVCache, with
    device-resident block tables updated in place each step.  Replaces the
    reference's one-sequence-at-a-time decode under Engine.mu
    (pkg/engine/engine.go:417)."""

    def __init__(self, mgr, pool, max_batch, max_blocks):
        h = _vp()
        _check(lib().gi_batch_create(mgr._h, pool.handle if pool is not None else None, max_batch,
                                     max_blocks, ctypes.byref(h)))
        self._h, self._mgr, self._pool = h, mgr, pool
        self.max_batch, self.max_blocks = max_batch, max_blocks

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.gi_batch_destroy(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def Add(self, seq_id):
        r = _c_int()
        _check(lib().gi_batch_add(self._h, seq_id, ctypes.byref(r)))
        return r.value

    def Remove(self, seq_id):
        _check(lib().gi_batch_remove(self._h, seq_id))

    def Step(self):
        n = _c_int()
        _check(lib().gi_batch_step(self._h, ctypes.byref(n)))
        return n.value

    def Rows(self):
        """(sequence ids, lengths) by row."""
        import numpy as np
        n = _c_int()
        ids = np.zeros(self.max_batch, np.int32)
        lens = np.zeros(self.max_batch, np.int32)
        _check(lib().gi_batch_rows(self._h, ids.ctypes.data_as(_i32p), lens.ctypes.data_as(_i32p),
                                   self.max_batch, ctypes.byref(n)))
        return ids[:n.value].copy(), lens[:n.value].copy()

    def RowTable(self, row):
        import numpy as np
        n = _c_int()
        ids = np.zeros(self.max_blocks, np.int32)
        _check(lib().gi_batch_row_table(self._h, row, ids.ctypes.data_as(_i32p), self.max_blocks,
                                        ctypes.byref(n)))
        return ids[:n.value].copy()

    def DeviceTables(self):
        """Raw device pointers (block tables, lengths) and max_blocks."""
        t, l, mb = _vp(), _vp(), _c_int()
        _check(lib().gi_batch_device_tables(self._h, ctypes.byref(t), ctypes.byref(l),
                                            ctypes.byref(mb)))
        return t.value, l.value, mb.value

    def DecodeLayer(self, layer, num_heads, q, k, v, out, attn_scale, rope=False):
        import torch
        _check(lib().gi_batch_decode_layer(
            self._h, layer, num_heads, _ptr(q, torch.float32, "q"), _ptr(k, torch.float32, "k"),
            _ptr(v, torch.float32, "v"), _ptr(out, torch.float32, "out"), float(attn_scale),
            1 if rope else 0))


class Weights:
    """A weight matrix [rows][cols] uploaded from its GGUF bytes (numpy uint8
    or float32 array on the host) for gi_matmul_batch on the pool's device:
    MatMul / MatMulBatch of pkg/engine/weights.go:237-350."""

    def __init__(self, pool, ggml_type, rows, cols, raw):
        import numpy as np
        buf = np.ascontiguousarray(raw)
        h = _vp()
        _check(lib().gi_weights_upload(pool.handle, ggml_type, rows, cols, _vp(buf.ctypes.data),
                                       ctypes.byref(h)))
        self._h, self._pool = h, pool
        self.ggml_type, self.rows, self.cols = ggml_type, rows, cols

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.gi_weights_destroy(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def MatMulBatch(self, y, x):
        """y [batch, rows] = x [batch, cols] W^T (device float32 tensors)."""
        import torch
        batch = int(x.shape[0]) if x.dim() > 1 else 1
        _check(lib().gi_matmul_batch(self._h, batch, _ptr(x, torch.float32, "x"),
                                     _ptr(y, torch.float32, "y")))
