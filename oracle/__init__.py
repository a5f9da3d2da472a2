"""The oracle: a CPU restatement of go-infer's paged-KV / attention path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this package, and only as the checker
(or, for the baseline, as the CPU path being timed).  The product library
(go-infer_amd) never imports or links it.

Contents
  * ctypes wrappers over oracle/cpu_ref.c (the float/byte arithmetic, with
    the Go functions each one restates cited in that file);
  * PagedKVManager: restatement of pkg/engine/paged_kv.go:49-148;
  * a counter-based seeded generator (SplitMix64 -> Box-Muller) used for
    every synthetic input, so any sub-range of a tensor can be regenerated.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libcpuref.so")
_lib = None

KV_F32, KV_F16, KV_Q8_0, KV_Q4_0 = 0, 1, 2, 3

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64
_int = ctypes.c_int


def lib():
    """Load oracle/libcpuref.so, building it with gcc first if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            from . import build as _b
            _b.build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "ref_fp16_to_fp32": (ctypes.c_float, [ctypes.c_uint16]),
            "ref_fp32_to_fp16": (ctypes.c_uint16, [ctypes.c_float]),
            "ref_fp32_to_fp16_array": (None, [_f32p, _u16p, _i64]),
            "ref_fp16_to_fp32_array": (None, [_u16p, _f32p, _i64]),
            "ref_quantize_q8_0": (None, [_f32p, _i64, _u8p]),
            "ref_dequantize_q8_0": (None, [_u8p, _i64, _f32p]),
            "ref_quantize_q4_0": (None, [_f32p, _i64, _u8p]),
            "ref_dequantize_q4_0": (None, [_u8p, _i64, _f32p]),
            "ref_dot_vec_f32": (ctypes.c_float, [_f32p, _f32p, _int]),
            "ref_softmax": (None, [_f32p, _int]),
            "ref_math_sqrt": (ctypes.c_double, [ctypes.c_double]),
            "ref_attn_scale": (ctypes.c_float, [_int]),
            "ref_attention_decode": (None, [_f32p, _f32p, _f32p, _f32p, _int, _int, _int, _int,
                                            ctypes.c_float, _f32p]),
            "ref_attention_prefill": (None, [_f32p, _f32p, _f32p, _f32p, _int, _int, _int, _int,
                                             _int, _int, ctypes.c_float, _f32p]),
            "ref_attention_decode_mt": (_int, [_f32p, _f32p, _f32p, _f32p, _int, _int, _int, _int,
                                               ctypes.c_float, _int]),
            "ref_attention_prefill_mt": (_int, [_f32p, _f32p, _f32p, _f32p, _int, _int, _int, _int,
                                                _int, _int, ctypes.c_float, _int]),
            "ref_decode_batch_mt": (_int, [_int, _f32p, _u8p, _u8p, _i64p, _i32p, _int, _f32p,
                                           _int, _int, _int, ctypes.c_float, _f32p, _f32p, _int]),
            "ref_bytes_per_vec": (_i64, [_int, _int]),
            "ref_kv_write": (None, [_int, _int, _int, _u8p, _u8p, _int, _f32p, _f32p]),
            "ref_kv_widen": (None, [_int, _int, _u8p, _i64, _f32p]),
            "ref_paged_store": (None, [_int, _int, _int, _int, _u8p, _u8p, _int, _int, _i32p,
                                       _i32p, _f32p, _f32p]),
            "ref_paged_gather": (None, [_int, _int, _int, _int, _u8p, _u8p, _int, _i32p, _int,
                                        _u8p, _u8p]),
            "ref_decode_batch": (None, [_int, _f32p, _u8p, _u8p, _i64p, _i32p, _int, _f32p, _int,
                                        _int, _int, ctypes.c_float, _f32p, _f32p, _f32p]),
            "ref_apply_rope": (None, [_f32p, _int, _int, ctypes.c_float]),
            "ref_rope_heads": (None, [_f32p, _int, _int, _int, _int, ctypes.c_float]),
            "ref_rope_table": (None, [ctypes.c_float, _int, _int, _int, _f32p]),
            "ref_dot_vec_f16": (ctypes.c_float, [_f32p, _u16p, _int]),
            "ref_dot_vec_q8_0": (ctypes.c_float, [_f32p, _u8p, _int]),
            "ref_dot_vec_q4_0": (ctypes.c_float, [_f32p, _u8p, _int]),
            "ref_weight_row_bytes": (_i64, [_int, _int]),
            "ref_matmul": (None, [_int, _int, _int, _int, _u8p, _f32p, _f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- element conversions (pkg/quant/fp16.go) ------------------------------

def fp32_to_fp16(x):
    """FP32ToFP16 (fp16.go:38-69), truncating; returns uint16 bit patterns."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().ref_fp32_to_fp16_array(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def fp16_to_fp32(h):
    """FP16ToFP32 (fp16.go:8-35) of uint16 bit patterns."""
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ref_fp16_to_fp32_array(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


# ---- Q8_0 (pkg/quant/quant.go) ---------------------------------------------

def quantize_q8_0(x):
    """QuantizeQ8_0 (quant.go:407-456) of a 1-D float32 vector -> bytes."""
    x = _c(x, np.float32).ravel()
    out = np.empty(((x.size + 31) // 32) * 34, np.uint8)
    lib().ref_quantize_q8_0(_p(x, _f32p), x.size, _p(out, _u8p))
    return out


def dequantize_q8_0(data, n):
    """DequantizeQ8_0 (quant.go:196-213) -> float32[n]."""
    data = _c(data, np.uint8)
    out = np.zeros(n, np.float32)
    lib().ref_dequantize_q8_0(_p(data, _u8p), n, _p(out, _f32p))
    return out


def quantize_q4_0(x):
    """QuantizeQ4_0 (quant.go:458-521) of a 1-D float32 vector -> bytes."""
    x = _c(x, np.float32).ravel()
    out = np.empty(((x.size + 31) // 32) * 18, np.uint8)
    lib().ref_quantize_q4_0(_p(x, _f32p), x.size, _p(out, _u8p))
    return out


def dequantize_q4_0(data, n):
    """DequantizeQ4_0 (quant.go:96-116) -> float32[n]."""
    data = _c(data, np.uint8)
    out = np.zeros(n, np.float32)
    lib().ref_dequantize_q4_0(_p(data, _u8p), n, _p(out, _f32p))
    return out


def dot_vec_f32(x, w):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    return np.float32(lib().ref_dot_vec_f32(_p(x, _f32p), _p(w, _f32p), x.size))


def softmax(x):
    x = _c(x, np.float32).copy()
    lib().ref_softmax(_p(x, _f32p), x.size)
    return x


def math_sqrt(x):
    return lib().ref_math_sqrt(float(x))


def attn_scale(head_dim):
    return np.float32(lib().ref_attn_scale(int(head_dim)))


# ---- rotary position embedding (pkg/math/kernels.go:22-35) -----------------

def apply_rope(vec, pos, head_dim, theta):
    """ApplyRoPE(vec, pos, headDim, theta) on a copy of one float32 vector."""
    x = _c(vec, np.float32).copy()
    lib().ref_apply_rope(_p(x, _f32p), int(pos), int(head_dim), float(theta))
    return x


def rope_heads(x, positions, n_heads, head_dim, rope_dim, theta):
    """RoPE of token vectors x [n, n_heads*head_dim] at positions[n], every
    head turned as Forward does (forward.go:228-234; rope_dim < head_dim as in
    forward.go:945-977).  Returns a new array."""
    x = _c(x, np.float32).copy()
    n = x.shape[0]
    for i in range(n):
        lib().ref_rope_heads(_p(x[i], _f32p), n_heads, head_dim, rope_dim, int(positions[i]),
                             float(theta))
    return x


def rope_table(theta, rope_dim, pos0, n_pos):
    """float32 [n_pos, rope_dim/2, 2] (cos, sin) pairs ApplyRoPE uses."""
    out = np.empty((n_pos, rope_dim // 2, 2), np.float32)
    lib().ref_rope_table(float(theta), rope_dim, pos0, n_pos, _p(out, _f32p))
    return out


# ---- weight matrices (pkg/math/gemv.go, pkg/quant/quant.go DotVec*) --------

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8     # pkg/gguf/types.go:25-31


def weight_row_bytes(ggml_type, cols):
    return int(lib().ref_weight_row_bytes(ggml_type, cols))


def quantize_weights(ggml_type, wf):
    """GGUF bytes of a float32 matrix [rows, cols] stored as ggml_type (F32
    bits, FP32ToFP16 halves, or QuantizeQ8_0 / QuantizeQ4_0 blocks per row)."""
    wf = _c(wf, np.float32)
    rows, cols = wf.shape
    if ggml_type == GGML_F32:
        return wf.view(np.uint8).reshape(rows, -1).copy()
    if ggml_type == GGML_F16:
        return fp32_to_fp16(wf).view(np.uint8).reshape(rows, -1)
    q = quantize_q8_0 if ggml_type == GGML_Q8_0 else quantize_q4_0
    return q(wf).reshape(rows, -1)


def matmul(ggml_type, w_raw, x, rows, cols):
    """MatMul of gemv.go for every row of x [batch, cols] -> y [batch, rows]."""
    w_raw = _c(w_raw, np.uint8)
    x = _c(x, np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), np.float32)
    lib().ref_matmul(ggml_type, x.shape[0], rows, cols, _p(w_raw, _u8p), _p(x, _f32p), _p(y, _f32p))
    return y


def dot_vec_q4_0(x, blocks):
    x = _c(x, np.float32)
    blocks = _c(blocks, np.uint8)
    return np.float32(lib().ref_dot_vec_q4_0(_p(x, _f32p), _p(blocks, _u8p), x.size))


# ---- KVCache semantics ------------------------------------------------------

def bytes_per_vec(kv_type, kv_dim):
    return int(lib().ref_bytes_per_vec(kv_type, kv_dim))


def store_vectors(kv_type, x):
    """Stored-format bytes of token vectors x[n, kv_dim] as KVCache.Write
    stores them (kvcache.go:146-180): f32 bits, truncated halves, or Q8_0
    blocks of the whole kvDim vector.  Returns uint8[n, bytes_per_vec]."""
    x = _c(x, np.float32)
    n, kv_dim = x.shape
    bpv = bytes_per_vec(kv_type, kv_dim)
    if kv_type == KV_F32:
        return x.view(np.uint8).reshape(n, bpv).copy()
    if kv_type == KV_F16:
        return fp32_to_fp16(x).view(np.uint8).reshape(n, bpv)
    if kv_dim % 32 == 0:
        # quantised blocks never straddle token vectors: one call over all rows
        q = quantize_q4_0 if kv_type == KV_Q4_0 else quantize_q8_0
        return q(x).reshape(n, bpv)
    out = np.zeros((n, bpv), np.uint8)
    dummy = np.zeros((1, bpv), np.uint8)
    for i in range(n):
        row = out[i:i + 1]
        lib().ref_kv_write(kv_type, kv_dim, 1, _p(row, _u8p), _p(dummy, _u8p), 0,
                           _p(x[i], _f32p), _p(x[i], _f32p))
    return out


def widen(kv_type, kv_dim, stored):
    """float32 values the attention loop reads from stored token vectors
    (KVCache.Get, kvcache.go:183-214; FP16ToFP32 / DequantizeQ8_0)."""
    stored = _c(stored, np.uint8)
    n = stored.shape[0]
    out = np.empty((n, kv_dim), np.float32)
    lib().ref_kv_widen(kv_type, kv_dim, _p(stored, _u8p), n, _p(out, _f32p))
    return out


# ---- attention (pkg/engine/forward.go) --------------------------------------

def host_threads():
    """Host threads for the multi-threaded oracle: the CPUs this process may
    run on, at most 16 (the host share of one GPU on the MI355X boxes)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def attention_decode(q, kc, vc, H, KVH, hd, L, scale, threads=1):
    """Decode GQA attention of forward.go:242-267 over float32 caches kc/vc
    [>=L, KVH*hd]; q [H*hd] -> out [H*hd].  threads > 1 splits the q-heads
    over host threads; the result is bit-identical."""
    q = _c(q, np.float32)
    kc = _c(kc, np.float32)
    vc = _c(vc, np.float32)
    out = np.empty(H * hd, np.float32)
    if threads > 1:
        rc = lib().ref_attention_decode_mt(_p(q, _f32p), _p(kc, _f32p), _p(vc, _f32p),
                                           _p(out, _f32p), H, KVH, hd, L, float(scale), threads)
        if rc != 0:
            raise MemoryError("ref_attention_decode_mt failed")
        return out
    scores = np.empty(max(L, 1), np.float32)
    lib().ref_attention_decode(_p(q, _f32p), _p(kc, _f32p), _p(vc, _f32p), _p(out, _f32p),
                               H, KVH, hd, L, float(scale), _p(scores, _f32p))
    return out


def attention_prefill(q, kc, vc, H, KVH, hd, start_pos, chunk, max_seq, scale, threads=1):
    """Chunked-prefill causal attention of forward.go:547-577; q [chunk, H*hd].
    threads > 1 splits the (query, q-head) rows over host threads; the result
    is bit-identical."""
    q = _c(q, np.float32)
    kc = _c(kc, np.float32)
    vc = _c(vc, np.float32)
    out = np.empty((chunk, H * hd), np.float32)
    if threads > 1:
        rc = lib().ref_attention_prefill_mt(_p(q, _f32p), _p(kc, _f32p), _p(vc, _f32p),
                                            _p(out, _f32p), H, KVH, hd, start_pos, chunk, max_seq,
                                            float(scale), threads)
        if rc != 0:
            raise MemoryError("ref_attention_prefill_mt failed")
        return out
    scores = np.empty(max(min(start_pos + chunk, max_seq), 1), np.float32)
    lib().ref_attention_prefill(_p(q, _f32p), _p(kc, _f32p), _p(vc, _f32p), _p(out, _f32p),
                                H, KVH, hd, start_pos, chunk, max_seq, float(scale),
                                _p(scores, _f32p))
    return out


def decode_batch(kv_type, q, kcat, vcat, tok_off, seq_lens, H, KVH, hd, scale, threads=1):
    """Decode attention for a batch from stored-format caches (CPU baseline).
    threads > 1 widens each sequence and splits its q-heads over host
    threads; the result is bit-identical.  Returns out, or (out, threads
    that ran) when threads > 1."""
    q = _c(q, np.float32)
    kcat = _c(kcat, np.uint8)
    vcat = _c(vcat, np.uint8)
    tok_off = _c(tok_off, np.int64)
    seq_lens = _c(seq_lens, np.int32)
    batch = seq_lens.size
    out = np.empty((batch, H * hd), np.float32)
    Lmax = max(int(seq_lens.max()) if batch else 1, 1)
    wk = np.empty(Lmax * KVH * hd, np.float32)
    wv = np.empty(Lmax * KVH * hd, np.float32)
    if threads > 1:
        ran = lib().ref_decode_batch_mt(kv_type, _p(q, _f32p), _p(kcat, _u8p), _p(vcat, _u8p),
                                        _p(tok_off, _i64p), _p(seq_lens, _i32p), batch,
                                        _p(out, _f32p), H, KVH, hd, float(scale), _p(wk, _f32p),
                                        _p(wv, _f32p), threads)
        if ran < 1:
            raise MemoryError("ref_decode_batch_mt failed")
        return out, ran
    sc = np.empty(Lmax, np.float32)
    lib().ref_decode_batch(kv_type, _p(q, _f32p), _p(kcat, _u8p), _p(vcat, _u8p),
                           _p(tok_off, _i64p), _p(seq_lens, _i32p), batch, _p(out, _f32p),
                           H, KVH, hd, float(scale), _p(wk, _f32p), _p(wv, _f32p), _p(sc, _f32p))
    return out


# ---- paged pool in the reference layout (paged_kv.go:13-46) ---------------

class RefPagedPool:
    """KVBlock pool: [block][layer][token_in_block][bytes_per_vec] for K and V
    (paged_kv.go:13-38 keeps Key[layer][token_idx*kvDim] per block)."""

    def __init__(self, kv_type, num_layers, kv_dim, num_blocks, block_size):
        self.kv_type, self.num_layers, self.kv_dim = kv_type, num_layers, kv_dim
        self.num_blocks, self.block_size = num_blocks, block_size
        self.bpv = bytes_per_vec(kv_type, kv_dim)
        self.k = np.zeros(num_blocks * num_layers * block_size * self.bpv, np.uint8)
        self.v = np.zeros_like(self.k)

    def store(self, layer, block_ids, slots, k, v):
        block_ids = _c(block_ids, np.int32)
        slots = _c(slots, np.int32)
        k = _c(k, np.float32)
        v = _c(v, np.float32)
        lib().ref_paged_store(self.kv_type, self.num_layers, self.block_size, self.kv_dim,
                              _p(self.k, _u8p), _p(self.v, _u8p), layer, block_ids.size,
                              _p(block_ids, _i32p), _p(slots, _i32p), _p(k, _f32p), _p(v, _f32p))

    def gather(self, layer, block_table, n_tok):
        block_table = _c(block_table, np.int32)
        ko = np.zeros((n_tok, self.bpv), np.uint8)
        vo = np.zeros((n_tok, self.bpv), np.uint8)
        lib().ref_paged_gather(self.kv_type, self.num_layers, self.block_size, self.kv_dim,
                               _p(self.k, _u8p), _p(self.v, _u8p), layer, _p(block_table, _i32p),
                               n_tok, _p(ko, _u8p), _p(vo, _u8p))
        return ko, vo


class OutOfPages(Exception):
    pass


class UnknownSequence(Exception):
    pass


class PagedKVManager:
    """Restatement of pkg/engine/paged_kv.go:49-148 (host-side allocator).

    FreeBlocks starts as [0..N) (paged_kv.go:70-74) and is used as a stack:
    AppendToken pops from the tail (122-123), FreeSequence pushes a table's
    ids back in table order (144-146).  Sequence ids start at 1 (85)."""

    def __init__(self, num_layers, kv_dim, total_blocks, block_size):
        if block_size <= 0:
            block_size = 16
        if total_blocks <= 0:
            total_blocks = 256
        self.NumLayers, self.KVDim = num_layers, kv_dim
        self.BlockSize, self.TotalBlocks = block_size, total_blocks
        self.FreeBlocks = list(range(total_blocks))
        self.Tables = {}
        self._next = 1

    def AllocateSequence(self):
        sid = self._next
        self._next += 1
        self.Tables[sid] = {"BlockIDs": [], "NumTokens": 0}
        return sid

    def AppendToken(self, sid):
        t = self.Tables.get(sid)
        if t is None:
            raise UnknownSequence("sequence %d not found" % sid)
        needed = t["NumTokens"] // self.BlockSize + 1
        if len(t["BlockIDs"]) < needed:
            if not self.FreeBlocks:
                raise OutOfPages("out of paged KV memory (no free blocks available)")
            t["BlockIDs"].append(self.FreeBlocks.pop())
        slot = t["NumTokens"] % self.BlockSize
        t["NumTokens"] += 1
        return t["BlockIDs"][-1], slot

    def FreeSequence(self, sid):
        t = self.Tables.pop(sid, None)
        if t is not None:
            self.FreeBlocks.extend(t["BlockIDs"])


class RefKVCache:
    """KVCache of pkg/engine/kvcache.go restated over stored bytes: per layer
    a contiguous [MaxSeq][bytes_per_vec] K and V (f32, FP32ToFP16 halves or
    34-byte q8_0 blocks, the formats of Write, kvcache.go:146-180).  ForkAt
    (225-284) is a deep copy of slots [0, maxSlot), the rest zero.  Used as
    the model that paged prefix sharing must reproduce."""

    def __init__(self, kv_type, num_layers, kv_dim, max_seq):
        self.kv_type, self.num_layers, self.kv_dim, self.max_seq = kv_type, num_layers, kv_dim, max_seq
        self.bpv = bytes_per_vec(kv_type, kv_dim)
        self.K = np.zeros((num_layers, max_seq, self.bpv), np.uint8)
        self.V = np.zeros_like(self.K)
        self.CurPos = 0

    def Write(self, layer, slot, k, v):
        if 0 <= layer < self.num_layers and 0 <= slot < self.max_seq:   # kvcache.go:147-149
            self.K[layer, slot] = store_vectors(self.kv_type, np.reshape(k, (1, -1)))[0]
            self.V[layer, slot] = store_vectors(self.kv_type, np.reshape(v, (1, -1)))[0]

    def ForkAt(self, max_slot):
        c = RefKVCache(self.kv_type, self.num_layers, self.kv_dim, self.max_seq)
        c.CurPos = self.CurPos
        n = min(max(max_slot, 0), self.max_seq)                          # kvcache.go:241-246
        c.K[:, :n] = self.K[:, :n]
        c.V[:, :n] = self.V[:, :n]
        return c

    def Clone(self):
        return self.ForkAt(self.max_seq)                                 # kvcache.go:217-222


class RefPrefixCache:
    """PrefixCache of pkg/engine/prefix_cache.go:7-150: entries keyed by the
    whole token list; FindLongestPrefix tries l = len-1 .. 1 (85-93); Store
    ignores lists shorter than 4 (99-101) and, when full, drops one entry
    first (106-112: whichever Go's randomised map iteration yields; here the
    oldest, the choice the paged cache makes)."""

    def __init__(self, max_size):
        self.max_size = max_size if max_size > 0 else 32
        self.entries = {}

    def FindLongestPrefix(self, tokens):
        for l in range(len(tokens) - 1, 0, -1):
            e = self.entries.get(tuple(tokens[:l]))
            if e is not None:
                return l, e
        return 0, None

    def Store(self, tokens, kv):
        if len(tokens) < 4:
            return
        if len(self.entries) >= self.max_size:
            del self.entries[next(iter(self.entries))]
        key = tuple(tokens)
        self.entries.pop(key, None)
        self.entries[key] = kv


# ---- seeded synthetic inputs ------------------------------------------------

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z):
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(seed, idx):
    """SplitMix64 output number idx (0-based) of the stream seeded with seed."""
    with np.errstate(over="ignore"):
        return _mix(np.uint64(seed) + (np.asarray(idx, np.uint64) + np.uint64(1)) * _GOLDEN)


def normal(seed, shape, offset=0):
    """float32 N(0,1) samples: element i uses SplitMix64 outputs 2(offset+i)
    and 2(offset+i)+1 as uniforms for one Box-Muller cosine branch, so any
    sub-range of a tensor can be regenerated on its own."""
    n = int(np.prod(shape)) if len(shape) else 1
    i = np.arange(n, dtype=np.uint64) + np.uint64(offset)
    a = splitmix64(seed, np.uint64(2) * i)
    b = splitmix64(seed, np.uint64(2) * i + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (b >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return z.astype(np.float32).reshape(shape)


def normal_with_outliers(seed, shape, frac=0.01, sigma=8.0, offset=0):
    """N(0,1) with a Bernoulli(frac) mask replaced by +-sigma (random sign)."""
    x = normal(seed, shape, offset)
    n = x.size
    i = np.arange(n, dtype=np.uint64) + np.uint64(offset)
    h = splitmix64(np.uint64(seed) ^ np.uint64(0x5DEECE66D), i)
    u = (h >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    sign = np.where((h & np.uint64(1)) == 1, 1.0, -1.0).astype(np.float32)
    flat = x.reshape(-1)
    m = u < frac
    flat[m] = sign[m] * np.float32(sigma)
    return x
