// Device plumbing of the tbn host runtime: the stream every operator is
// queued on, a caching allocator for HBM buffers, and host<->device copies.
//
// Stream model.  All work of a thread goes to one HIP stream, the thread's
// current stream (the null stream unless set).  Device buffers freed by a
// Tensor go back to a per-device cache and may be handed out again at once:
// that is safe because every later use is queued behind the earlier ones on
// the same stream.  set_current_stream() therefore first waits for the
// previous stream, so no cached buffer is reused across streams while work
// on it is still pending.
#pragma once

#include <cstddef>

namespace tbn {
namespace device {

using Stream = void*;  // a hipStream_t

Stream current_stream();
void set_current_stream(Stream s);

// Device allocation from the caching allocator (throws OutOfMemoryError).
void* allocate(size_t bytes);
void release(void* p) noexcept;
// Returns every cached (free) block to the HIP runtime.
void empty_cache();
size_t cached_bytes();
size_t allocated_bytes();

// Queued on the current stream.  copy_to_device and copy_to_host return
// once the copy is complete (the host buffer may then be reused).
void copy_to_device(void* dst, const void* src, size_t bytes);
void copy_to_host(void* dst, const void* src, size_t bytes);
void copy_on_device(void* dst, const void* src, size_t bytes);
// Waits for the current stream and reports any asynchronous device error.
void synchronize();

}  // namespace device
}  // namespace tbn
