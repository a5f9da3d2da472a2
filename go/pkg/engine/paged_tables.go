// Block-table layout shared by the HIP build and its no-HIP twin (no build
// tag): the per-sequence tables of PagedKVManager (paged_kv.go:41-46) laid
// out as the [batch][maxBlocks] int32 array the device kernels read.
package engine

import "fmt"

// flatTables lays out tables as [len(tables)][maxBlocks] int32, padding each
// row past its own blocks with -1, an id outside every pool: the kernels skip
// such entries and report them (GI_ERR_BAD_PAGE), where padding with a valid
// id (0) would attend another sequence's page.  need[b] is the number of
// tokens row b is read for (its length, or start + chunk for prefill); a row
// whose blocks cover fewer tokens is refused here.
func flatTables(tables [][]int32, need []int32, pageSize int) ([]int32, int, error) {
	if len(need) != len(tables) {
		return nil, 0, fmt.Errorf("flatTables: %d tables for %d sequences", len(tables), len(need))
	}
	maxBlocks := 1
	for b, t := range tables {
		if len(t) > maxBlocks {
			maxBlocks = len(t)
		}
		if need[b] < 0 || int64(need[b]) > int64(len(t))*int64(pageSize) {
			return nil, 0, fmt.Errorf("flatTables: sequence %d needs %d tokens, its %d blocks of %d hold %d",
				b, need[b], len(t), pageSize, len(t)*pageSize)
		}
	}
	flat := make([]int32, len(tables)*maxBlocks)
	for i := range flat {
		flat[i] = -1
	}
	for i, t := range tables {
		copy(flat[i*maxBlocks:], t)
	}
	return flat, maxBlocks, nil
}
