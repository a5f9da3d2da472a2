/* A C99 host of the C ABI, compiled the way cgo compiles its preamble
 * (plain C including goinfer_paged.h, linked against libgoinfer_paged.so).
 * It runs the host-only allocator through the reference's own test,
 * pkg/engine/paged_kv_test.go:7-40: sequence ids start at 1, 35 tokens take
 * three 16-token blocks popped from the tail of the free list (the first is
 * block N-1, paged_kv.go:122-123), and freeing returns every block.
 * Exit status 0 on success; a message on stderr otherwise. */
#include "goinfer_paged.h"

#include <stdio.h>

static int fail(const char *what)
{
    fprintf(stderr, "%s: %s\n", what, gi_last_error());
    return 1;
}

int main(void)
{
    gi_kvmgr *m = NULL;
    int seq = 0, n = 0, i;
    int32_t blk = -1, slot = -1, ids[16];
    if (gi_device_count() < 0)
        return fail("gi_device_count");
    if (gi_kvmgr_create(4, 64, 10, 16, &m) != GI_OK)
        return fail("gi_kvmgr_create");
    if (gi_kvmgr_allocate_sequence(m, &seq) != GI_OK || seq != 1)
        return fail("gi_kvmgr_allocate_sequence");
    for (i = 0; i < 35; i++) {
        if (gi_kvmgr_append_token(m, seq, &blk, &slot) != GI_OK)
            return fail("gi_kvmgr_append_token");
        if (slot != i % 16)
            return fail("slot");
    }
    if (gi_kvmgr_block_table(m, seq, ids, 16, &n, &i) != GI_OK || n != 3 || i != 35)
        return fail("gi_kvmgr_block_table");
    if (ids[0] != 9 || ids[1] != 8 || ids[2] != 7)
        return fail("LIFO block order");
    if (gi_kvmgr_append_token(m, 99, &blk, &slot) != GI_ERR_UNKNOWN_SEQ)
        return fail("unknown sequence");
    if (gi_kvmgr_free_sequence(m, seq) != GI_OK)
        return fail("gi_kvmgr_free_sequence");
    if (gi_kvmgr_free_list(m, ids, 16, &n) != GI_OK || n != 10)
        return fail("gi_kvmgr_free_list");
    gi_kvmgr_destroy(m);
    printf("abi_smoke ok\n");
    return 0;
}
