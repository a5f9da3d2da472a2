//go:build !(linux && cgo && rocm)

// Builds without the HIP library (no cgo, another OS, or no rocm tag) keep
// the same API and report it unavailable, as c_bridge_nocgo.go and
// pkg/metal/metal_fallback.go do; the engine then keeps its CPU loops
// (forward.go:242-267, 547-577).
package engine

import "errors"

// KVTypeF16 stores K/V as fp16 halves truncated by quant.FP32ToFP16
// (pkg/quant/fp16.go:38-69); the reference's own types are kvcache.go:11-15.
const KVTypeF16 KVCacheType = "f16"

var errNoHIP = errors.New("HIP paged KV unavailable (build on linux with cgo and -tags rocm)")

// HIPAvailable reports whether a HIP device is present: never, in this build.
func HIPAvailable() bool {
	return false
}

// HIPDeviceName names the current HIP device: none in this build.
func HIPDeviceName() string {
	return ""
}

// HIPPagedKV is the device page pool of the HIP build; here it cannot be made.
type HIPPagedKV struct {
	Layers   int
	KVHeads  int
	HeadDim  int
	PageSize int
}

// NewHIPPagedKV reports that no device pool exists in this build.
func NewHIPPagedKV(numLayers, numKVHeads, headDim, blockSize, totalBlocks int, t KVCacheType) (*HIPPagedKV, error) {
	return nil, errNoHIP
}

// Write reports that no device pool exists in this build.
func (p *HIPPagedKV) Write(layer int, blockIDs, slots []int32, k, v []float32) error {
	return errNoHIP
}

// Get reports that no device pool exists in this build.
func (p *HIPPagedKV) Get(layer int, table []int32, n int) ([]float32, []float32, error) {
	return nil, nil, errNoHIP
}

// AttentionGQA reports that no device pool exists in this build.
func (p *HIPPagedKV) AttentionGQA(out, q []float32, layer int, tables [][]int32, seqLens []int32,
	numHeads int, attnScale float32) error {
	return errNoHIP
}

// AttentionGQABatch reports that no device pool exists in this build.
func (p *HIPPagedKV) AttentionGQABatch(out, q []float32, layer int, tables [][]int32, startPos []int32,
	numHeads, chunkLen int, attnScale float32) error {
	return errNoHIP
}

// CopyPages reports that no device pool exists in this build.
func (p *HIPPagedKV) CopyPages(src, dst []int32) error {
	return errNoHIP
}

// Close does nothing in this build.
func (p *HIPPagedKV) Close() {}
