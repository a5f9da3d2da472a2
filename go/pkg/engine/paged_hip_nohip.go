//go:build !(linux && cgo && rocm)

// Builds without the HIP library (no cgo, another OS, or no rocm tag) keep
// the same API and report it unavailable, as c_bridge_nocgo.go and
// pkg/metal/metal_fallback.go do; the engine then keeps its CPU loops
// (forward.go:242-267, 547-577) and its own PagedKVManager (paged_kv.go).
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

// DecodeStep reports that no device pool exists in this build.
func (p *HIPPagedKV) DecodeStep(out, q, k, v []float32, layer int, tables [][]int32, seqLens []int32,
	numHeads int, attnScale float32) error {
	return errNoHIP
}

// SetRoPE reports that no device pool exists in this build.
func (p *HIPPagedKV) SetRoPE(theta float32, ropeDim, maxPositions int) error {
	return errNoHIP
}

// RoPEDecodeStep reports that no device pool exists in this build.
func (p *HIPPagedKV) RoPEDecodeStep(out, q, k, v []float32, layer int, tables [][]int32, seqLens []int32,
	numHeads int, attnScale float32) error {
	return errNoHIP
}

// AttentionGQABatch reports that no device pool exists in this build.
func (p *HIPPagedKV) AttentionGQABatch(out, q []float32, layer int, tables [][]int32, startPos []int32,
	numHeads, chunkLen int, attnScale float32) error {
	return errNoHIP
}

// AttentionPlan is gi_attention_plan of the HIP build.
type AttentionPlan struct {
	DecodeKernel      int
	DecodeFallback    bool
	DecodeSplits      int
	DecodeSplitTokens int
	DecodeWaves       int
	DecodeStepFused   bool
	PrefillKernel     int
	PrefillFallback   bool
}

// AttentionPlan reports that no device pool exists in this build.
func (p *HIPPagedKV) AttentionPlan(batch, numHeads, maxSeqLen int) (AttentionPlan, error) {
	return AttentionPlan{}, errNoHIP
}

// CopyPages reports that no device pool exists in this build.
func (p *HIPPagedKV) CopyPages(src, dst []int32) error {
	return errNoHIP
}

// Close does nothing in this build.
func (p *HIPPagedKV) Close() {}

// HIPKVManager is the library's allocator in the HIP build; here the
// engine's own PagedKVManager serves.
type HIPKVManager struct{}

// NewHIPKVManager reports that the library is absent in this build.
func NewHIPKVManager(numLayers, kvDim, totalBlocks, blockSize int) (*HIPKVManager, error) {
	return nil, errNoHIP
}

// AllocateSequence reports that the library is absent in this build.
func (m *HIPKVManager) AllocateSequence() (int, error) {
	return 0, errNoHIP
}

// AppendToken reports that the library is absent in this build.
func (m *HIPKVManager) AppendToken(seqID int) (blockID, slot, copyFrom int32, err error) {
	return 0, 0, -1, errNoHIP
}

// AppendBatch reports that the library is absent in this build.
func (m *HIPKVManager) AppendBatch(seqIDs []int) (blockIDs, slots, copySrc []int32, err error) {
	return nil, nil, nil, errNoHIP
}

// ForkSequence reports that the library is absent in this build.
func (m *HIPKVManager) ForkSequence(src, nTokens int) (int, error) {
	return 0, errNoHIP
}

// FreeSequence reports that the library is absent in this build.
func (m *HIPKVManager) FreeSequence(seqID int) error {
	return errNoHIP
}

// BlockTable reports that the library is absent in this build.
func (m *HIPKVManager) BlockTable(seqID int) ([]int32, int, error) {
	return nil, 0, errNoHIP
}

// BlockRefs reports that the library is absent in this build.
func (m *HIPKVManager) BlockRefs(blockID int32) (int, error) {
	return 0, errNoHIP
}

// Close does nothing in this build.
func (m *HIPKVManager) Close() {}

// HIPPrefixCache is the shared-page prefix cache of the HIP build.
type HIPPrefixCache struct{}

// NewHIPPrefixCache reports that the library is absent in this build.
func NewHIPPrefixCache(m *HIPKVManager, maxSize int) (*HIPPrefixCache, error) {
	return nil, errNoHIP
}

// Store reports that the library is absent in this build.
func (c *HIPPrefixCache) Store(tokens []int32, seqID int) error {
	return errNoHIP
}

// FindLongestPrefix reports that the library is absent in this build.
func (c *HIPPrefixCache) FindLongestPrefix(tokens []int32) (matched, newSeq int, err error) {
	return 0, 0, errNoHIP
}

// Size reports that the library is absent in this build.
func (c *HIPPrefixCache) Size() (int, error) {
	return 0, errNoHIP
}

// Close does nothing in this build.
func (c *HIPPrefixCache) Close() {}

// HIPBatchDecoder is the continuous-batching driver of the HIP build.
type HIPBatchDecoder struct{}

// NewHIPBatchDecoder reports that the library is absent in this build.
func NewHIPBatchDecoder(m *HIPKVManager, p *HIPPagedKV, maxBatch, maxBlocks int) (*HIPBatchDecoder, error) {
	return nil, errNoHIP
}

// Add reports that the library is absent in this build.
func (d *HIPBatchDecoder) Add(seqID int) (int, error) {
	return 0, errNoHIP
}

// Remove reports that the library is absent in this build.
func (d *HIPBatchDecoder) Remove(seqID int) error {
	return errNoHIP
}

// Step reports that the library is absent in this build.
func (d *HIPBatchDecoder) Step() (int, error) {
	return 0, errNoHIP
}

// Rows reports that the library is absent in this build.
func (d *HIPBatchDecoder) Rows() ([]int32, []int32, error) {
	return nil, nil, errNoHIP
}

// DecodeLayer reports that the library is absent in this build.
func (d *HIPBatchDecoder) DecodeLayer(layer, numHeads int, q, k, v, out []float32, attnScale float32, rope bool) error {
	return errNoHIP
}

// Close does nothing in this build.
func (d *HIPBatchDecoder) Close() {}

// HIPWeights is a device weight matrix of the HIP build.
type HIPWeights struct {
	Rows, Cols int
}

// UploadWeights reports that no device pool exists in this build.
func (p *HIPPagedKV) UploadWeights(ggmlType, rows, cols int, raw []byte) (*HIPWeights, error) {
	return nil, errNoHIP
}

// MatMulBatch reports that the library is absent in this build.
func (w *HIPWeights) MatMulBatch(out, x []float32, batch int) error {
	return errNoHIP
}

// Close does nothing in this build.
func (w *HIPWeights) Close() {}
