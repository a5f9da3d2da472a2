//go:build linux && cgo && rocm

// HIP paged KV cache for the engine: the device page pool, the KV store and
// the paged attention of pkg/engine/forward.go, bound through cgo to
// libgoinfer_paged.so (C ABI in include/goinfer_paged.h).  It sits beside the
// Metal seams (pkg/metal/metal_darwin.go:601-999) and binds the library the way
// c_bridge_cgo.go binds inference_core.h.  Builds without HIP use
// paged_hip_nohip.go, as c_bridge_nocgo.go and metal_fallback.go do.
//
// Beside the pool (HIPPagedKV) it binds the host-side allocator with
// copy-on-write prefix sharing (HIPKVManager, HIPPrefixCache), the
// continuous-batching decode driver (HIPBatchDecoder) and the O-projection
// after attention (HIPWeights).
//
// Host slices are staged into device buffers the pool owns; C never keeps a
// Go pointer after a call returns.
package engine

/*
#cgo CFLAGS: -I${SRCDIR}/../../third_party/goinfer_paged/include
#cgo LDFLAGS: -L${SRCDIR}/../../third_party/goinfer_paged/lib -lgoinfer_paged -Wl,-rpath,${SRCDIR}/../../third_party/goinfer_paged/lib
#include <stdlib.h>
#include "goinfer_paged.h"
*/
import "C"

import (
	"fmt"
	"runtime"
	"sync"
	"unsafe"
)

// KVTypeF16 stores K/V as fp16 halves truncated by quant.FP32ToFP16
// (pkg/quant/fp16.go:38-69); the reference's own types are kvcache.go:11-15.
const KVTypeF16 KVCacheType = "f16"

// HIPAvailable reports whether a HIP device is present (model_has_metal's
// role, inference_core.c:113-117).
func HIPAvailable() bool {
	return C.gi_device_count() > 0
}

// HIPDeviceName names the current HIP device (model_device_name,
// inference_core.c:119-122).
func HIPDeviceName() string {
	var buf [256]C.char
	if C.gi_device_name(&buf[0], C.int(len(buf))) != C.GI_OK {
		return ""
	}
	return C.GoString(&buf[0])
}

// cCall makes one C call and, when it fails, reads gi_last_error on the same
// OS thread: the library keeps the message per thread, and a goroutine could
// otherwise move to another thread between the call and the read.
func cCall(what string, f func() C.int) error {
	runtime.LockOSThread()
	defer runtime.UnlockOSThread()
	rc := f()
	if rc == C.GI_OK {
		return nil
	}
	return fmt.Errorf("%s failed: %d (%s)", what, int(rc), C.GoString(C.gi_last_error()))
}

func i32p(p unsafe.Pointer) *C.int32_t { return (*C.int32_t)(p) }

// HIPPagedKV is a device page pool: one page id covers every layer, like
// KVBlock (paged_kv.go:13-38). Block ids come from the Go PagedKVManager
// (paged_kv.go:49-148) or from HIPKVManager. Calls are serialised by mu, as
// CModelContext does (c_bridge_cgo.go:19-22).
type HIPPagedKV struct {
	mu       sync.Mutex
	h        *C.gi_paged
	Layers   int
	KVHeads  int
	HeadDim  int
	PageSize int
	stage    map[string]unsafe.Pointer // device staging buffers by role
	stageCap map[string]int
}

func kvTypeCode(t KVCacheType) (C.int, error) {
	switch t {
	case KVTypeF32:
		return C.GI_KV_F32, nil
	case KVTypeF16:
		return C.GI_KV_F16, nil
	case KVTypeQ8_0:
		return C.GI_KV_Q8_0, nil
	case KVTypeQ4_0:
		return C.GI_KV_Q4_0, nil
	}
	return 0, fmt.Errorf("kv type %q has no device layout", t)
}

// NewHIPPagedKV allocates totalBlocks pages of blockSize tokens for every
// layer (NewQuantizedKVCache, kvcache.go:82-117, as one device pool).
func NewHIPPagedKV(numLayers, numKVHeads, headDim, blockSize, totalBlocks int, t KVCacheType) (*HIPPagedKV, error) {
	code, err := kvTypeCode(t)
	if err != nil {
		return nil, err
	}
	var h *C.gi_paged
	if err := cCall("gi_paged_create", func() C.int {
		return C.gi_paged_create(C.int(numLayers), C.int(numKVHeads), C.int(headDim), C.int(blockSize),
			C.int64_t(totalBlocks), code, &h)
	}); err != nil {
		return nil, err
	}
	return &HIPPagedKV{h: h, Layers: numLayers, KVHeads: numKVHeads, HeadDim: headDim,
		PageSize: blockSize, stage: map[string]unsafe.Pointer{}, stageCap: map[string]int{}}, nil
}

// buf returns a device buffer of at least n bytes for role, holding the
// contents of src when src is non-nil.  The caller holds p.mu.
func (p *HIPPagedKV) buf(role string, n int, src unsafe.Pointer) (unsafe.Pointer, error) {
	if p.stageCap[role] < n {
		if old := p.stage[role]; old != nil {
			C.gi_dev_free(p.h, old)
			delete(p.stage, role)
			p.stageCap[role] = 0
		}
		var d unsafe.Pointer
		if err := cCall("gi_dev_alloc", func() C.int { return C.gi_dev_alloc(p.h, C.size_t(n), &d) }); err != nil {
			return nil, err
		}
		p.stage[role], p.stageCap[role] = d, n
	}
	d := p.stage[role]
	if src != nil && n > 0 {
		if err := cCall("gi_memcpy_h2d", func() C.int { return C.gi_memcpy_h2d(p.h, d, src, C.size_t(n)) }); err != nil {
			return nil, err
		}
	}
	return d, nil
}

// floats stages a float32 slice (nil contents: an output buffer).
func (p *HIPPagedKV) floats(role string, x []float32, upload bool) (unsafe.Pointer, error) {
	var src unsafe.Pointer
	if upload {
		src = unsafe.Pointer(&x[0])
	}
	return p.buf(role, 4*len(x), src)
}

// sync waits for the pool's stream and reports bad ids the kernels met.
func (p *HIPPagedKV) sync() error {
	return cCall("gi_synchronize", func() C.int { return C.gi_synchronize(p.h) })
}

// download copies n float32 from a device buffer into x.
func (p *HIPPagedKV) download(x []float32, d unsafe.Pointer) error {
	return cCall("gi_memcpy_d2h", func() C.int {
		return C.gi_memcpy_d2h(p.h, unsafe.Pointer(&x[0]), d, C.size_t(4*len(x)))
	})
}

// Write stores token vectors at (blockIDs[i], slots[i]) of one layer, the
// pairs PagedKVManager.AppendToken returned (KVCache.Write semantics,
// kvcache.go:146-180; metal.KVWrite, metal_darwin.go:601-614).
func (p *HIPPagedKV) Write(layer int, blockIDs, slots []int32, k, v []float32) error {
	p.mu.Lock()
	defer p.mu.Unlock()
	n := len(blockIDs)
	kvDim := p.KVHeads * p.HeadDim
	if len(slots) != n || len(k) != n*kvDim || len(v) != n*kvDim {
		return fmt.Errorf("Write: %d ids, %d slots, %d k and %d v values for kvDim %d",
			n, len(slots), len(k), len(v), kvDim)
	}
	if n == 0 {
		return nil
	}
	ids, err := p.buf("ids", 4*n, unsafe.Pointer(&blockIDs[0]))
	if err != nil {
		return err
	}
	sl, err := p.buf("slots", 4*n, unsafe.Pointer(&slots[0]))
	if err != nil {
		return err
	}
	dk, err := p.floats("k", k, true)
	if err != nil {
		return err
	}
	dv, err := p.floats("v", v, true)
	if err != nil {
		return err
	}
	if err := cCall("gi_paged_append", func() C.int {
		return C.gi_paged_append(p.h, C.int(layer), C.int(n), i32p(ids), i32p(sl), (*C.float)(dk), (*C.float)(dv))
	}); err != nil {
		return err
	}
	return p.sync()
}

// Get gathers tokens [0, n) of one layer of one sequence as float32
// [n][kvDim] K and V (KVCache.Get / ForkAt, kvcache.go:183-284: stored
// values widened by FP16ToFP32 or DequantizeQ8_0 / Q4_0).
func (p *HIPPagedKV) Get(layer int, table []int32, n int) ([]float32, []float32, error) {
	p.mu.Lock()
	defer p.mu.Unlock()
	kvDim := p.KVHeads * p.HeadDim
	if n <= 0 {
		return nil, nil, nil
	}
	if len(table)*p.PageSize < n {
		return nil, nil, fmt.Errorf("Get: %d pages hold fewer than %d tokens", len(table), n)
	}
	dt, err := p.buf("table", 4*len(table), unsafe.Pointer(&table[0]))
	if err != nil {
		return nil, nil, err
	}
	k := make([]float32, n*kvDim)
	v := make([]float32, n*kvDim)
	dk, err := p.floats("gk", k, false)
	if err != nil {
		return nil, nil, err
	}
	dv, err := p.floats("gv", v, false)
	if err != nil {
		return nil, nil, err
	}
	if err := cCall("gi_paged_gather", func() C.int {
		return C.gi_paged_gather(p.h, C.int(layer), i32p(dt), C.int(n), dk, dv, 1)
	}); err != nil {
		return nil, nil, err
	}
	if err := p.sync(); err != nil {
		return nil, nil, err
	}
	if err := p.download(k, dk); err != nil {
		return nil, nil, err
	}
	if err := p.download(v, dv); err != nil {
		return nil, nil, err
	}
	return k, v, nil
}

// decodeArgs stages a decode batch: q (and k, v for a step), the output
// buffer, the block tables and the lengths.
type decodeArgs struct {
	q, k, v, out, tables, lens unsafe.Pointer
	maxBlocks                  int
}

func (p *HIPPagedKV) stageDecode(what string, out, q, k, v []float32, tables [][]int32, seqLens []int32,
	numHeads int, withKV bool) (*decodeArgs, error) {
	batch := len(seqLens)
	rowLen := numHeads * p.HeadDim
	kvDim := p.KVHeads * p.HeadDim
	if len(tables) != batch || len(q) != batch*rowLen || len(out) != batch*rowLen {
		return nil, fmt.Errorf("%s: %d tables, %d q and %d out values for batch %d x %d",
			what, len(tables), len(q), len(out), batch, rowLen)
	}
	if withKV && (len(k) != batch*kvDim || len(v) != batch*kvDim) {
		return nil, fmt.Errorf("%s: %d k and %d v values for batch %d x %d", what, len(k), len(v), batch, kvDim)
	}
	flat, maxBlocks, err := flatTables(tables, seqLens, p.PageSize)
	if err != nil {
		return nil, err
	}
	a := &decodeArgs{maxBlocks: maxBlocks}
	if a.q, err = p.floats("q", q, true); err != nil {
		return nil, err
	}
	if withKV {
		if a.k, err = p.floats("k", k, true); err != nil {
			return nil, err
		}
		if a.v, err = p.floats("v", v, true); err != nil {
			return nil, err
		}
	}
	if a.out, err = p.floats("out", out, false); err != nil {
		return nil, err
	}
	if a.tables, err = p.buf("tables", 4*len(flat), unsafe.Pointer(&flat[0])); err != nil {
		return nil, err
	}
	if a.lens, err = p.buf("lens", 4*batch, unsafe.Pointer(&seqLens[0])); err != nil {
		return nil, err
	}
	return a, nil
}

// AttentionGQA runs decode attention of one layer for a batch, reading K/V
// from pages (forward.go:242-267; metal.AttentionGQA, metal_darwin.go:711-727):
// out, q are [batch][numHeads*headDim], sequence b attends its first
// seqLens[b] tokens.
func (p *HIPPagedKV) AttentionGQA(out, q []float32, layer int, tables [][]int32, seqLens []int32,
	numHeads int, attnScale float32) error {
	p.mu.Lock()
	defer p.mu.Unlock()
	batch := len(seqLens)
	if batch == 0 {
		return nil
	}
	a, err := p.stageDecode("AttentionGQA", out, q, nil, nil, tables, seqLens, numHeads, false)
	if err != nil {
		return err
	}
	// the kernels read the lengths on the device; max_seq_len is not needed
	if err := cCall("gi_paged_decode_attention", func() C.int {
		return C.gi_paged_decode_attention(p.h, C.int(layer), C.int(batch), C.int(numHeads), (*C.float)(a.q),
			(*C.float)(a.out), i32p(a.tables), C.int(a.maxBlocks), i32p(a.lens), 0, C.float(attnScale))
	}); err != nil {
		return err
	}
	if err := p.sync(); err != nil {
		return err
	}
	return p.download(out, a.out)
}

// DecodeStep is one decode step of one layer (forward.go:236-267): the new
// token's k, v ([batch][kvDim]) are stored at position seqLens[b]-1 of
// sequence b, then decode attention runs over seqLens[b] tokens.  Where the
// grid fills the device once (small batches) the token store happens inside
// the attention launch (AttentionPlan().DecodeStepFused).
func (p *HIPPagedKV) DecodeStep(out, q, k, v []float32, layer int, tables [][]int32, seqLens []int32,
	numHeads int, attnScale float32) error {
	p.mu.Lock()
	defer p.mu.Unlock()
	batch := len(seqLens)
	if batch == 0 {
		return nil
	}
	a, err := p.stageDecode("DecodeStep", out, q, k, v, tables, seqLens, numHeads, true)
	if err != nil {
		return err
	}
	if err := cCall("gi_paged_decode_step", func() C.int {
		return C.gi_paged_decode_step(p.h, C.int(layer), C.int(batch), C.int(numHeads), (*C.float)(a.q),
			(*C.float)(a.k), (*C.float)(a.v), (*C.float)(a.out), i32p(a.tables), C.int(a.maxBlocks),
			i32p(a.lens), 0, C.float(attnScale))
	}); err != nil {
		return err
	}
	if err := p.sync(); err != nil {
		return err
	}
	return p.download(out, a.out)
}

// SetRoPE builds the (cos, sin) table of ApplyRoPE (pkg/math/kernels.go:22-35)
// for positions [0, maxPositions); ropeDim 0 means headDim.
func (p *HIPPagedKV) SetRoPE(theta float32, ropeDim, maxPositions int) error {
	p.mu.Lock()
	defer p.mu.Unlock()
	return cCall("gi_paged_set_rope", func() C.int {
		return C.gi_paged_set_rope(p.h, C.float(theta), C.int(ropeDim), C.int(maxPositions))
	})
}

// RoPEDecodeStep is forward.go:228-267 for a batch: q and k turned by
// ApplyRoPE at position seqLens[b]-1 (q in place, as Forward turns a.Q), k and
// v stored, then decode attention.  Needs SetRoPE.
func (p *HIPPagedKV) RoPEDecodeStep(out, q, k, v []float32, layer int, tables [][]int32, seqLens []int32,
	numHeads int, attnScale float32) error {
	p.mu.Lock()
	defer p.mu.Unlock()
	batch := len(seqLens)
	if batch == 0 {
		return nil
	}
	a, err := p.stageDecode("RoPEDecodeStep", out, q, k, v, tables, seqLens, numHeads, true)
	if err != nil {
		return err
	}
	if err := cCall("gi_paged_rope_decode_step", func() C.int {
		return C.gi_paged_rope_decode_step(p.h, C.int(layer), C.int(batch), C.int(numHeads), (*C.float)(a.q),
			(*C.float)(a.k), (*C.float)(a.v), (*C.float)(a.out), i32p(a.tables), C.int(a.maxBlocks),
			i32p(a.lens), 0, C.float(attnScale))
	}); err != nil {
		return err
	}
	if err := p.sync(); err != nil {
		return err
	}
	if err := p.download(q, a.q); err != nil {
		return err
	}
	return p.download(out, a.out)
}

// AttentionGQABatch runs chunked-prefill causal attention of one layer
// (forward.go:547-577; metal.AttentionGQABatch, metal_darwin.go:963-981): the
// chunk's K/V are already written; query i of sequence b attends tokens
// [0, startPos[b]+i+1). out, q are [batch][chunkLen][numHeads*headDim].
func (p *HIPPagedKV) AttentionGQABatch(out, q []float32, layer int, tables [][]int32, startPos []int32,
	numHeads, chunkLen int, attnScale float32) error {
	p.mu.Lock()
	defer p.mu.Unlock()
	batch := len(startPos)
	if batch == 0 || chunkLen == 0 {
		return nil
	}
	n := batch * chunkLen * numHeads * p.HeadDim
	if len(tables) != batch || len(q) != n || len(out) != n {
		return fmt.Errorf("AttentionGQABatch: %d tables, %d q and %d out values for %d rows",
			len(tables), len(q), len(out), n)
	}
	need := make([]int32, batch)
	for b, s := range startPos {
		need[b] = s + int32(chunkLen)
	}
	flat, maxBlocks, err := flatTables(tables, need, p.PageSize)
	if err != nil {
		return err
	}
	dq, err := p.floats("q", q, true)
	if err != nil {
		return err
	}
	dout, err := p.floats("out", out, false)
	if err != nil {
		return err
	}
	dbt, err := p.buf("tables", 4*len(flat), unsafe.Pointer(&flat[0]))
	if err != nil {
		return err
	}
	dsp, err := p.buf("start", 4*batch, unsafe.Pointer(&startPos[0]))
	if err != nil {
		return err
	}
	if err := cCall("gi_paged_prefill_attention", func() C.int {
		return C.gi_paged_prefill_attention(p.h, C.int(layer), C.int(batch), C.int(chunkLen), C.int(numHeads),
			(*C.float)(dq), (*C.float)(dout), i32p(dbt), C.int(maxBlocks), i32p(dsp), C.float(attnScale))
	}); err != nil {
		return err
	}
	if err := p.sync(); err != nil {
		return err
	}
	return p.download(out, dout)
}

// AttentionPlan is gi_attention_plan: how the pool's attention calls would
// run for a shape, worked out without launching anything.
type AttentionPlan struct {
	DecodeKernel      int  // 0 vector ALU, 1 matrix core
	DecodeFallback    bool // matrix core selected but not supported for this shape
	DecodeSplits      int  // split-K ranges per (sequence, kv head)
	DecodeSplitTokens int
	DecodeWaves       int  // waves per matrix-core workgroup
	DecodeStepFused   bool // DecodeStep stores the token inside the attention launch
	PrefillKernel     int
	PrefillFallback   bool
}

// AttentionPlan reports the launch plan for batch sequences of up to
// maxSeqLen tokens with numHeads query heads.
func (p *HIPPagedKV) AttentionPlan(batch, numHeads, maxSeqLen int) (AttentionPlan, error) {
	p.mu.Lock()
	defer p.mu.Unlock()
	var pl C.gi_attention_plan
	if err := cCall("gi_paged_attention_plan", func() C.int {
		return C.gi_paged_attention_plan(p.h, C.int(batch), C.int(numHeads), C.int(maxSeqLen), &pl)
	}); err != nil {
		return AttentionPlan{}, err
	}
	return AttentionPlan{
		DecodeKernel: int(pl.decode_kernel), DecodeFallback: pl.decode_fallback != 0,
		DecodeSplits: int(pl.decode_splits), DecodeSplitTokens: int(pl.decode_split_tokens),
		DecodeWaves: int(pl.decode_waves), DecodeStepFused: pl.decode_step_fused != 0,
		PrefillKernel: int(pl.prefill_kernel), PrefillFallback: pl.prefill_fallback != 0,
	}, nil
}

// CopyPages copies whole pages in every layer, dst[i] <- src[i]: the copy a
// copy-on-write append of a forked sequence asks for (Clone / ForkAt,
// kvcache.go:217-284, without the deep copy).
func (p *HIPPagedKV) CopyPages(src, dst []int32) error {
	p.mu.Lock()
	defer p.mu.Unlock()
	if len(src) != len(dst) {
		return fmt.Errorf("CopyPages: %d sources, %d destinations", len(src), len(dst))
	}
	if len(src) == 0 {
		return nil
	}
	ds, err := p.buf("copy_src", 4*len(src), unsafe.Pointer(&src[0]))
	if err != nil {
		return err
	}
	dd, err := p.buf("copy_dst", 4*len(dst), unsafe.Pointer(&dst[0]))
	if err != nil {
		return err
	}
	if err := cCall("gi_paged_copy_pages", func() C.int {
		return C.gi_paged_copy_pages(p.h, C.int(len(src)), i32p(ds), i32p(dd))
	}); err != nil {
		return err
	}
	return p.sync()
}

// Close frees the device pool and its staging buffers (free_model,
// inference_core.c:124-130).
func (p *HIPPagedKV) Close() {
	if p == nil || p.h == nil {
		return
	}
	p.mu.Lock()
	defer p.mu.Unlock()
	for _, d := range p.stage {
		C.gi_dev_free(p.h, d)
	}
	C.gi_paged_destroy(p.h)
	p.h = nil
}

// ---- the allocator with copy-on-write prefix sharing -------------------

// HIPKVManager is PagedKVManager (paged_kv.go:49-148) with a reference count
// per block, so that forks share their prefix's pages instead of the deep
// copies of Clone / ForkAt (kvcache.go:217-284, per consensus sample at
// engine.go:749).  It runs on the host; the library serialises its calls.
type HIPKVManager struct {
	m *C.gi_kvmgr
}

// NewHIPKVManager is NewPagedKVManager (paged_kv.go:62-87).
func NewHIPKVManager(numLayers, kvDim, totalBlocks, blockSize int) (*HIPKVManager, error) {
	var m *C.gi_kvmgr
	if err := cCall("gi_kvmgr_create", func() C.int {
		return C.gi_kvmgr_create(C.int(numLayers), C.int(kvDim), C.int(totalBlocks), C.int(blockSize), &m)
	}); err != nil {
		return nil, err
	}
	return &HIPKVManager{m: m}, nil
}

// AllocateSequence is paged_kv.go:90-104 (ids count up from 1).
func (m *HIPKVManager) AllocateSequence() (int, error) {
	var id C.int
	err := cCall("gi_kvmgr_allocate_sequence", func() C.int { return C.gi_kvmgr_allocate_sequence(m.m, &id) })
	return int(id), err
}

// AppendToken is paged_kv.go:107-132 with copy-on-write: copyFrom is -1, or
// the shared block whose pages the caller copies into blockID (CopyPages)
// before it writes the token.
func (m *HIPKVManager) AppendToken(seqID int) (blockID, slot, copyFrom int32, err error) {
	var b, s, c C.int32_t
	err = cCall("gi_kvmgr_append_token_cow", func() C.int {
		return C.gi_kvmgr_append_token_cow(m.m, C.int(seqID), &b, &s, &c)
	})
	return int32(b), int32(s), int32(c), err
}

// AppendBatch reserves one token for each of the distinct seqIDs, all or
// nothing (the decode step of a running batch): blockIDs[i] / slots[i] as
// AppendToken gives them, copySrc[i] -1 or the shared block to copy first.
func (m *HIPKVManager) AppendBatch(seqIDs []int) (blockIDs, slots, copySrc []int32, err error) {
	n := len(seqIDs)
	if n == 0 {
		return nil, nil, nil, nil
	}
	ids := make([]C.int, n)
	for i, s := range seqIDs {
		ids[i] = C.int(s)
	}
	blockIDs, slots, copySrc = make([]int32, n), make([]int32, n), make([]int32, n)
	err = cCall("gi_kvmgr_append_batch", func() C.int {
		return C.gi_kvmgr_append_batch(m.m, C.int(n), &ids[0], i32p(unsafe.Pointer(&blockIDs[0])),
			i32p(unsafe.Pointer(&slots[0])), i32p(unsafe.Pointer(&copySrc[0])))
	})
	return blockIDs, slots, copySrc, err
}

// ForkSequence is ForkAt(nTokens) (kvcache.go:225-284) on shared pages: a new
// sequence whose first nTokens tokens are src's.
func (m *HIPKVManager) ForkSequence(src, nTokens int) (int, error) {
	var id C.int
	err := cCall("gi_kvmgr_fork_sequence", func() C.int {
		return C.gi_kvmgr_fork_sequence(m.m, C.int(src), C.int(nTokens), &id)
	})
	return int(id), err
}

// FreeSequence is paged_kv.go:135-148: a block returns to the free list when
// its last reference goes.
func (m *HIPKVManager) FreeSequence(seqID int) error {
	return cCall("gi_kvmgr_free_sequence", func() C.int { return C.gi_kvmgr_free_sequence(m.m, C.int(seqID)) })
}

// BlockTable returns a sequence's block ids and token count (BlockTable,
// paged_kv.go:41-46).
func (m *HIPKVManager) BlockTable(seqID int) ([]int32, int, error) {
	var nb, nt C.int
	if err := cCall("gi_kvmgr_block_table", func() C.int {
		return C.gi_kvmgr_block_table(m.m, C.int(seqID), nil, 0, &nb, &nt)
	}); err != nil {
		return nil, 0, err
	}
	ids := make([]int32, int(nb)+1)
	if err := cCall("gi_kvmgr_block_table", func() C.int {
		return C.gi_kvmgr_block_table(m.m, C.int(seqID), i32p(unsafe.Pointer(&ids[0])), C.int(len(ids)), &nb, &nt)
	}); err != nil {
		return nil, 0, err
	}
	return ids[:int(nb)], int(nt), nil
}

// BlockRefs is the number of references held on a block (0 when free).
func (m *HIPKVManager) BlockRefs(blockID int32) (int, error) {
	var r C.int
	err := cCall("gi_kvmgr_block_refs", func() C.int { return C.gi_kvmgr_block_refs(m.m, C.int32_t(blockID), &r) })
	return int(r), err
}

// Close frees the manager.
func (m *HIPKVManager) Close() {
	if m == nil || m.m == nil {
		return
	}
	C.gi_kvmgr_destroy(m.m)
	m.m = nil
}

// HIPPrefixCache is PrefixCache (prefix_cache.go:7-150) over shared pages:
// an entry holds a sequence forked from the stored one, and a hit forks it
// again, where the reference deep-copies whole caches (cloneKVCachePrefix,
// prefix_cache.go:122-150).
type HIPPrefixCache struct {
	c *C.gi_prefix
}

// NewHIPPrefixCache makes a cache of up to maxSize entries (<= 0: 32).
func NewHIPPrefixCache(m *HIPKVManager, maxSize int) (*HIPPrefixCache, error) {
	var c *C.gi_prefix
	if err := cCall("gi_prefix_create", func() C.int { return C.gi_prefix_create(m.m, C.int(maxSize), &c) }); err != nil {
		return nil, err
	}
	return &HIPPrefixCache{c: c}, nil
}

// Store is prefix_cache.go:97-119: keeps tokens of seqID under the key tokens.
func (c *HIPPrefixCache) Store(tokens []int32, seqID int) error {
	if len(tokens) == 0 {
		return nil
	}
	return cCall("gi_prefix_store", func() C.int {
		return C.gi_prefix_store(c.c, i32p(unsafe.Pointer(&tokens[0])), C.int(len(tokens)), C.int(seqID))
	})
}

// FindLongestPrefix is prefix_cache.go:76-95: the longest stored prefix of
// tokens, and a new sequence forked from it (0, 0 when there is none).
func (c *HIPPrefixCache) FindLongestPrefix(tokens []int32) (matched, newSeq int, err error) {
	if len(tokens) == 0 {
		return 0, 0, nil
	}
	var l, s C.int
	err = cCall("gi_prefix_find_longest", func() C.int {
		return C.gi_prefix_find_longest(c.c, i32p(unsafe.Pointer(&tokens[0])), C.int(len(tokens)), &l, &s)
	})
	return int(l), int(s), err
}

// Size is the number of entries.
func (c *HIPPrefixCache) Size() (int, error) {
	var n C.int
	err := cCall("gi_prefix_size", func() C.int { return C.gi_prefix_size(c.c, &n) })
	return int(n), err
}

// Close releases the entries' pages and the cache.
func (c *HIPPrefixCache) Close() {
	if c == nil || c.c == nil {
		return
	}
	C.gi_prefix_destroy(c.c)
	c.c = nil
}

// ---- the continuous-batching decode driver ------------------------------

// HIPBatchDecoder steps a running set of sequences together, where the
// reference decodes one sequence at a time under Engine.mu (engine.go:417):
// Step reserves a token for every running sequence and updates the
// device-resident block tables in place, DecodeLayer runs RoPE + append +
// paged attention of one layer (forward.go:228-267) for all of them.
type HIPBatchDecoder struct {
	b *C.gi_batch
	p *HIPPagedKV
}

// NewHIPBatchDecoder drives up to maxBatch sequences of up to maxBlocks
// blocks over the manager m and the pool p.
func NewHIPBatchDecoder(m *HIPKVManager, p *HIPPagedKV, maxBatch, maxBlocks int) (*HIPBatchDecoder, error) {
	var b *C.gi_batch
	if err := cCall("gi_batch_create", func() C.int {
		return C.gi_batch_create(m.m, p.h, C.int(maxBatch), C.int(maxBlocks), &b)
	}); err != nil {
		return nil, err
	}
	return &HIPBatchDecoder{b: b, p: p}, nil
}

// Add appends an allocated sequence (its tokens already in the pool) as the
// last row.
func (d *HIPBatchDecoder) Add(seqID int) (int, error) {
	var row C.int
	err := cCall("gi_batch_add", func() C.int { return C.gi_batch_add(d.b, C.int(seqID), &row) })
	return int(row), err
}

// Remove takes a running sequence out (the last row moves into its place);
// freeing it stays the caller's.
func (d *HIPBatchDecoder) Remove(seqID int) error {
	return cCall("gi_batch_remove", func() C.int { return C.gi_batch_remove(d.b, C.int(seqID)) })
}

// Step reserves one token for every running sequence (all or nothing) and
// returns the running count.
func (d *HIPBatchDecoder) Step() (int, error) {
	var n C.int
	err := cCall("gi_batch_step", func() C.int { return C.gi_batch_step(d.b, &n) })
	return int(n), err
}

// Rows returns the running sequence ids and lengths by row.
func (d *HIPBatchDecoder) Rows() ([]int32, []int32, error) {
	var n C.int
	if err := cCall("gi_batch_rows", func() C.int { return C.gi_batch_rows(d.b, nil, nil, 0, &n) }); err != nil {
		return nil, nil, err
	}
	ids, lens := make([]int32, int(n)+1), make([]int32, int(n)+1)
	if err := cCall("gi_batch_rows", func() C.int {
		return C.gi_batch_rows(d.b, i32p(unsafe.Pointer(&ids[0])), i32p(unsafe.Pointer(&lens[0])), C.int(len(ids)), &n)
	}); err != nil {
		return nil, nil, err
	}
	return ids[:int(n)], lens[:int(n)], nil
}

// DecodeLayer runs one layer of the step for every running row: q
// [rows][numHeads*headDim] (turned in place when rope, which needs SetRoPE),
// k, v [rows][kvDim], out [rows][numHeads*headDim].
func (d *HIPBatchDecoder) DecodeLayer(layer, numHeads int, q, k, v, out []float32, attnScale float32, rope bool) error {
	p := d.p
	p.mu.Lock()
	defer p.mu.Unlock()
	kvDim := p.KVHeads * p.HeadDim
	rows := len(q) / (numHeads * p.HeadDim)
	if rows == 0 {
		return nil
	}
	if len(q) != rows*numHeads*p.HeadDim || len(out) != len(q) || len(k) != rows*kvDim || len(v) != rows*kvDim {
		return fmt.Errorf("DecodeLayer: %d q, %d out, %d k and %d v values", len(q), len(out), len(k), len(v))
	}
	dq, err := p.floats("q", q, true)
	if err != nil {
		return err
	}
	dk, err := p.floats("k", k, true)
	if err != nil {
		return err
	}
	dv, err := p.floats("v", v, true)
	if err != nil {
		return err
	}
	dout, err := p.floats("out", out, false)
	if err != nil {
		return err
	}
	r := C.int(0)
	if rope {
		r = 1
	}
	if err := cCall("gi_batch_decode_layer", func() C.int {
		return C.gi_batch_decode_layer(d.b, C.int(layer), C.int(numHeads), (*C.float)(dq), (*C.float)(dk),
			(*C.float)(dv), (*C.float)(dout), C.float(attnScale), r)
	}); err != nil {
		return err
	}
	if err := p.sync(); err != nil {
		return err
	}
	if rope {
		if err := p.download(q, dq); err != nil {
			return err
		}
	}
	return p.download(out, dout)
}

// Close frees the driver (not the manager or the pool).
func (d *HIPBatchDecoder) Close() {
	if d == nil || d.b == nil {
		return
	}
	C.gi_batch_destroy(d.b)
	d.b = nil
}

// ---- the O-projection after attention -----------------------------------

// HIPWeights is one weight matrix on the pool's device, uploaded once from
// its GGUF bytes (the layout weights.go:237-350 loads), for MatMulBatch.
type HIPWeights struct {
	w          *C.gi_weights
	p          *HIPPagedKV
	Rows, Cols int
}

// UploadWeights uploads a [rows][cols] matrix given as GGUF bytes of type
// ggmlType (F32, F16, Q4_0 or Q8_0; pkg/gguf/types.go:25-31).
func (p *HIPPagedKV) UploadWeights(ggmlType, rows, cols int, raw []byte) (*HIPWeights, error) {
	if len(raw) == 0 {
		return nil, fmt.Errorf("UploadWeights: no bytes")
	}
	p.mu.Lock()
	defer p.mu.Unlock()
	var w *C.gi_weights
	if err := cCall("gi_weights_upload", func() C.int {
		return C.gi_weights_upload(p.h, C.int(ggmlType), C.int(rows), C.int(cols), unsafe.Pointer(&raw[0]), &w)
	}); err != nil {
		return nil, err
	}
	return &HIPWeights{w: w, p: p, Rows: rows, Cols: cols}, nil
}

// MatMulBatch is out[b][r] = sum_c W[r][c] x[b][c] for b < batch
// (metal.MatMulBatch, metal_darwin.go:849-880; MatMul, forward.go:270).
func (w *HIPWeights) MatMulBatch(out, x []float32, batch int) error {
	p := w.p
	p.mu.Lock()
	defer p.mu.Unlock()
	if batch == 0 {
		return nil
	}
	if len(x) != batch*w.Cols || len(out) != batch*w.Rows {
		return fmt.Errorf("MatMulBatch: %d x and %d out values for batch %d of %d x %d",
			len(x), len(out), batch, w.Rows, w.Cols)
	}
	dx, err := p.floats("mm_x", x, true)
	if err != nil {
		return err
	}
	dy, err := p.floats("mm_y", out, false)
	if err != nil {
		return err
	}
	if err := cCall("gi_matmul_batch", func() C.int {
		return C.gi_matmul_batch(w.w, C.int(batch), (*C.float)(dx), (*C.float)(dy))
	}); err != nil {
		return err
	}
	if err := p.sync(); err != nil {
		return err
	}
	return p.download(out, dy)
}

// Close frees the device copy of the weights.
func (w *HIPWeights) Close() {
	if w == nil || w.w == nil {
		return
	}
	C.gi_weights_destroy(w.w)
	w.w = nil
}
