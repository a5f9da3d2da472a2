// Growable device buffers of the HIP translation units.
#pragma once

#include "gi_host.h"

#include <hip/hip_runtime.h>

#include <vector>

namespace gi {

// A device buffer that grows on demand (split-K partials, activation splits).
//
// Growth needs a synchronisation and an allocation, which a stream that is
// capturing a graph cannot take, so devbuf_reserve refuses to grow while the
// stream captures: run one call of the largest shape eagerly first.  Once a
// call on the buffer has been captured, a graph may hold its address, so a
// later (eager) growth keeps the old allocation alive until devbuf_release
// instead of freeing it: replays of that graph stay valid.
struct DevBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    bool captured = false; // some captured call may reference ptr
    std::vector<void *> retired;
};

// Makes b hold at least `need` bytes on the current device (allocating a
// quarter more), noting whether `st` is capturing.  Returns GI_OK or an error
// code with the reason set; `what` names the caller in the message.
int devbuf_reserve(DevBuffer &b, size_t need, hipStream_t st, const char *what);

// Frees b and every allocation it retired (the caller has drained the
// streams that use them).
void devbuf_release(DevBuffer &b);

} // namespace gi
