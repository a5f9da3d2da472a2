//go:build linux && cgo && rocm

// HIP paged KV cache for the engine: the device page pool, the KV store and
// the paged attention of pkg/engine/forward.go, bound through cgo to
// libgoinfer_paged.so (C ABI in include/goinfer_paged.h).  It sits beside the
// Metal seams (pkg/metal/metal_darwin.go:601-999) and binds the library the way
// c_bridge_cgo.go binds inference_core.h.  Builds without HIP use
// paged_hip_nohip.go, as c_bridge_nocgo.go and metal_fallback.go do.
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

// HIPPagedKV is a device page pool: one page id covers every layer, like
// KVBlock (paged_kv.go:13-38). Block ids come from the Go PagedKVManager
// (paged_kv.go:49-148). Calls are serialised by mu, as CModelContext does
// (c_bridge_cgo.go:19-22).
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

func giErr(rc C.int, what string) error {
	if rc == C.GI_OK {
		return nil
	}
	return fmt.Errorf("%s failed: %d (%s)", what, int(rc), C.GoString(C.gi_last_error()))
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
	rc := C.gi_paged_create(C.int(numLayers), C.int(numKVHeads), C.int(headDim), C.int(blockSize),
		C.int64_t(totalBlocks), code, &h)
	if err := giErr(rc, "gi_paged_create"); err != nil {
		return nil, err
	}
	return &HIPPagedKV{h: h, Layers: numLayers, KVHeads: numKVHeads, HeadDim: headDim,
		PageSize: blockSize, stage: map[string]unsafe.Pointer{}, stageCap: map[string]int{}}, nil
}

// buf returns a device buffer of at least n bytes for role, holding the
// contents of src when src is non-nil.
func (p *HIPPagedKV) buf(role string, n int, src unsafe.Pointer) (unsafe.Pointer, error) {
	if p.stageCap[role] < n {
		if old := p.stage[role]; old != nil {
			C.gi_dev_free(p.h, old)
			delete(p.stage, role)
			p.stageCap[role] = 0
		}
		var d unsafe.Pointer
		if err := giErr(C.gi_dev_alloc(p.h, C.size_t(n), &d), "gi_dev_alloc"); err != nil {
			return nil, err
		}
		p.stage[role], p.stageCap[role] = d, n
	}
	d := p.stage[role]
	if src != nil && n > 0 {
		if err := giErr(C.gi_memcpy_h2d(p.h, d, src, C.size_t(n)), "gi_memcpy_h2d"); err != nil {
			return nil, err
		}
	}
	return d, nil
}

// flatTables lays out per-sequence block tables as [len(tables)][maxBlocks].
func flatTables(tables [][]int32) ([]int32, int) {
	maxBlocks := 1
	for _, t := range tables {
		if len(t) > maxBlocks {
			maxBlocks = len(t)
		}
	}
	flat := make([]int32, len(tables)*maxBlocks)
	for i, t := range tables {
		copy(flat[i*maxBlocks:], t)
	}
	return flat, maxBlocks
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
	dk, err := p.buf("k", 4*len(k), unsafe.Pointer(&k[0]))
	if err != nil {
		return err
	}
	dv, err := p.buf("v", 4*len(v), unsafe.Pointer(&v[0]))
	if err != nil {
		return err
	}
	rc := C.gi_paged_append(p.h, C.int(layer), C.int(n), (*C.int32_t)(ids), (*C.int32_t)(sl),
		(*C.float)(dk), (*C.float)(dv))
	if err := giErr(rc, "gi_paged_append"); err != nil {
		return err
	}
	return giErr(C.gi_synchronize(p.h), "gi_synchronize")
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
	dk, err := p.buf("gk", 4*n*kvDim, nil)
	if err != nil {
		return nil, nil, err
	}
	dv, err := p.buf("gv", 4*n*kvDim, nil)
	if err != nil {
		return nil, nil, err
	}
	rc := C.gi_paged_gather(p.h, C.int(layer), (*C.int32_t)(dt), C.int(n), dk, dv, 1)
	if err := giErr(rc, "gi_paged_gather"); err != nil {
		return nil, nil, err
	}
	if err := giErr(C.gi_synchronize(p.h), "gi_synchronize"); err != nil {
		return nil, nil, err
	}
	k := make([]float32, n*kvDim)
	v := make([]float32, n*kvDim)
	if err := giErr(C.gi_memcpy_d2h(p.h, unsafe.Pointer(&k[0]), dk, C.size_t(4*len(k))), "gi_memcpy_d2h"); err != nil {
		return nil, nil, err
	}
	if err := giErr(C.gi_memcpy_d2h(p.h, unsafe.Pointer(&v[0]), dv, C.size_t(4*len(v))), "gi_memcpy_d2h"); err != nil {
		return nil, nil, err
	}
	return k, v, nil
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
	rowLen := numHeads * p.HeadDim
	if len(tables) != batch || len(q) != batch*rowLen || len(out) != batch*rowLen {
		return fmt.Errorf("AttentionGQA: %d tables, %d q and %d out values for batch %d x %d",
			len(tables), len(q), len(out), batch, rowLen)
	}
	flat, maxBlocks := flatTables(tables)
	dq, err := p.buf("q", 4*len(q), unsafe.Pointer(&q[0]))
	if err != nil {
		return err
	}
	dout, err := p.buf("out", 4*len(out), nil)
	if err != nil {
		return err
	}
	dbt, err := p.buf("tables", 4*len(flat), unsafe.Pointer(&flat[0]))
	if err != nil {
		return err
	}
	dsl, err := p.buf("lens", 4*batch, unsafe.Pointer(&seqLens[0]))
	if err != nil {
		return err
	}
	// the kernels read the lengths on the device; max_seq_len is not needed
	rc := C.gi_paged_decode_attention(p.h, C.int(layer), C.int(batch), C.int(numHeads),
		(*C.float)(dq), (*C.float)(dout), (*C.int32_t)(dbt), C.int(maxBlocks), (*C.int32_t)(dsl),
		0, C.float(attnScale))
	if err := giErr(rc, "gi_paged_decode_attention"); err != nil {
		return err
	}
	if err := giErr(C.gi_synchronize(p.h), "gi_synchronize"); err != nil {
		return err
	}
	return giErr(C.gi_memcpy_d2h(p.h, unsafe.Pointer(&out[0]), dout, C.size_t(4*len(out))), "gi_memcpy_d2h")
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
	flat, maxBlocks := flatTables(tables)
	dq, err := p.buf("q", 4*n, unsafe.Pointer(&q[0]))
	if err != nil {
		return err
	}
	dout, err := p.buf("out", 4*n, nil)
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
	rc := C.gi_paged_prefill_attention(p.h, C.int(layer), C.int(batch), C.int(chunkLen), C.int(numHeads),
		(*C.float)(dq), (*C.float)(dout), (*C.int32_t)(dbt), C.int(maxBlocks), (*C.int32_t)(dsp),
		C.float(attnScale))
	if err := giErr(rc, "gi_paged_prefill_attention"); err != nil {
		return err
	}
	if err := giErr(C.gi_synchronize(p.h), "gi_synchronize"); err != nil {
		return err
	}
	return giErr(C.gi_memcpy_d2h(p.h, unsafe.Pointer(&out[0]), dout, C.size_t(4*n)), "gi_memcpy_d2h")
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
	rc := C.gi_paged_copy_pages(p.h, C.int(len(src)), (*C.int32_t)(ds), (*C.int32_t)(dd))
	if err := giErr(rc, "gi_paged_copy_pages"); err != nil {
		return err
	}
	return giErr(C.gi_synchronize(p.h), "gi_synchronize")
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
