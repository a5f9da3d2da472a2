package engine

import "testing"

// flatTables runs without the HIP library (no build tag).
func TestFlatTablesPadsWithInvalidIDs(t *testing.T) {
	flat, mb, err := flatTables([][]int32{{7, 3, 9}, {5}}, []int32{40, 16}, 16)
	if err != nil {
		t.Fatal(err)
	}
	want := []int32{7, 3, 9, 5, -1, -1}
	if mb != 3 || len(flat) != len(want) {
		t.Fatalf("maxBlocks %d, %d entries", mb, len(flat))
	}
	for i := range want {
		if flat[i] != want[i] {
			t.Fatalf("entry %d: %d, want %d", i, flat[i], want[i])
		}
	}
}

func TestFlatTablesRefusesLengthsPastTheTable(t *testing.T) {
	// one block of 16 tokens cannot hold 17
	if _, _, err := flatTables([][]int32{{7, 3}, {5}}, []int32{32, 17}, 16); err == nil {
		t.Fatal("a length past the table was accepted")
	}
	if _, _, err := flatTables([][]int32{{7}}, []int32{-1}, 16); err == nil {
		t.Fatal("a negative length was accepted")
	}
	if _, _, err := flatTables([][]int32{{7}}, []int32{1, 2}, 16); err == nil {
		t.Fatal("a length count that differs from the tables was accepted")
	}
	// empty rows need no blocks
	flat, mb, err := flatTables([][]int32{{}, {4}}, []int32{0, 3}, 16)
	if err != nil || mb != 1 || flat[0] != -1 || flat[1] != 4 {
		t.Fatalf("empty row: %v %d %v", flat, mb, err)
	}
}
