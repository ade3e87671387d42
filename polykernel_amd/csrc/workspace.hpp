// workspace.hpp -- the library-owned scratch of entry points whose reference
// signature has no workspace argument (split-K / split-KV partials, the
// normalised panel of a long-row RMSNorm->MatMul).  Host-only declarations,
// shared by the kernel sources and the runtime's code-object launchers.
#pragma once

#include <cstddef>
#include <memory>
#include <mutex>

namespace pk {

// One buffer per (device, stream): launches on one stream run in order, so
// the next call on that stream may reuse the buffer, and calls on different
// streams never share one (hipStreamPerThread is a different stream on each
// host thread, so it gets a buffer per thread).  The lease holds the slot's
// lock until it is destroyed: the caller enqueues every kernel that touches
// the buffer before another thread can take the same slot, so two threads
// feeding one stream cannot interleave their partial-sum kernels.  A slot
// that must grow gets a new buffer and keeps the old one allocated (kernels
// already queued may still read it); sizes grow by powers of two, so what is
// kept is less than the current buffer.  Nothing here synchronises the device
// or frees memory except release_workspace (pk_release_workspace), which
// waits for the stream and frees its slot: callers that create short-lived
// streams call it before destroying one.
struct WorkspaceLease {
  void *ptr = nullptr;
  std::shared_ptr<void> keep;          // keeps the slot alive while the lock is held
  std::unique_lock<std::mutex> lock;   // destroyed first (members unwind in reverse)
};

// `stream` is the hipStream_t the caller will launch on (nullptr: the null
// stream).  Returns a PK_* status.
int library_workspace(size_t bytes, void *stream, WorkspaceLease &lease);

// Frees the calling device's slot of `stream` after hipStreamSynchronize on
// it; the next call on that stream allocates again.  PK_OK when there is no
// slot.
int release_workspace(void *stream);

}  // namespace pk
