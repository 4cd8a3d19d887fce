// The calling thread's execution context and the scopes generated code opens on it, for whichever machine the
// including header chose as cr::gpu::Machine (cairn_gpu.hpp): HIP, or the host under CAIRN_EMULATE. The spellings
// are the ones CAIRN emits (src/cairn/compiler/lower/execution.py:33-37, header.py:296-304): cr::gpu::here(),
// cr::gpu::use_stream, cr::gpu::Held, cr::gpu::Enqueued, cr::gpu::Lent.
#pragma once
#include "cairn_context.hpp"

namespace cr::gpu {

using reuse::Allocation;
using reuse::Budget;
using reuse::Dir;
using reuse::Scratch;
using reuse::Where;
using Context = reuse::Context<Machine>;
using Lent = reuse::Lent<Machine>;

// The thread's context, made by its first device operation and kept for the thread's life. Its arena grows to the
// largest request met and keeps that size, so a pipeline run again allocates no scratch.
inline Context& here() noexcept {
  thread_local Context mine(Budget{0, reuse::UNBOUNDED});
  return mine;
}

// A stream the C caller owns, for the thread's synchronous device work (after what the caller queued there); null
// gives the thread its own back. What NAME_device_stream calls.
inline void use_stream(void* stream) noexcept {
  if(stream) here().bind(Machine::stream_of(stream));
  else here().unbind();
}

// A run of synchronous device work that waits once, when it ends (or where the host observes device memory first).
class Held final {
 public:
  Held() noexcept { here().hold(); }
  ~Held() noexcept { here().settle(); }
  Held(const Held&) = delete;
  Held& operator=(const Held&) = delete;
};

// An enqueued entry (cq_NAME): its device work queues on the caller's stream and nothing waits for it.
class Enqueued final {
 public:
  explicit Enqueued(void* stream) noexcept { here().enqueue(Machine::stream_of(stream)); }
  ~Enqueued() noexcept { here().leave(); }
  Enqueued(const Enqueued&) = delete;
  Enqueued& operator=(const Enqueued&) = delete;
};

}  // namespace cr::gpu
