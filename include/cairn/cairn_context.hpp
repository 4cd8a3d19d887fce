// The execution context device work runs through, written against a machine (a template parameter): the HIP machine
// of cairn_hip.hpp on a GPU, a counting host machine in the tests. It keeps the semantics CAIRN-emitted code relies on
// (src/cairn/runtime/cairn_reuse.hpp:57-200, cairn_exec.hpp:1-67):
//
//  - synchronous work runs on one lane (a stream and an event) and the call returns once that stream has run it,
//    never by waiting for the whole device;
//  - a caller may bind its own stream: synchronous work then runs there, after what the caller queued;
//  - a held run queues all its synchronous work on one lane and waits once, at its end;
//  - an enqueued call queues on the caller's stream and never waits;
//  - lanes are made on first use and kept: work repeated on a thread makes no stream and allocates nothing.
//
// Misuse (a lane never given back, nested synchronous work on a bound stream, a wait inside an enqueued call) traps.
#pragma once
#include <cstddef>
#include <new>
#include <utility>
#include "cairn_runtime.hpp"

namespace cr::reuse {

template<class Api> class Context final {
public:
  using Stream = typename Api::Stream;
  using Event = typename Api::Event;
  struct Lane {
    Stream stream{};
    Event event{};
    Lane* next = nullptr;
  };

  explicit Context(Api api = Api{}) noexcept : api_(std::move(api)) {}
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;
  ~Context() noexcept {
    if(lent_ || held_ || holding_) trap();  // work nobody waited for
    while(free_) {
      Lane* lane = free_;
      free_ = lane->next;
      api_.destroy_event(lane->event);
      api_.destroy_stream(lane->stream);
      delete lane;
    }
    if(bound_event_) api_.destroy_event(bound_.event);
  }

  // A lane for work about to be queued: for synchronous work the held run's lane, else the bound stream, else a
  // free lane (made if none). Another lane lent while a run is held or a stream bound starts after that work.
  Lane* lend(bool synchronous = false) noexcept {
    if(synchronous && held_) return held_;
    if(synchronous && binding_) {
      if(bound_lent_) trap();
      bound_lent_ = true;
      ++lent_;
      return &bound_;
    }
    Lane* lane = free_;
    if(lane) free_ = lane->next;
    else {
      lane = new(std::nothrow) Lane;
      if(!lane) trap();
      lane->stream = api_.make_stream();
      lane->event = api_.make_event();
      ++made_;
    }
    lane->next = nullptr;
    ++lent_;
    if(held_ || binding_) {
      Lane& before = held_ ? *held_ : bound_;
      api_.record(event_of(before), before.stream);
      api_.wait_event(lane->stream, before.event);
    }
    return lane;
  }
  // Wait for the lane's work (not under an enqueued call, whose stream the caller synchronizes) and keep the lane.
  void give_back(Lane* lane) noexcept {
    if(lane == held_) held_ = nullptr;
    if(!(enqueued_ && lane == &bound_)) api_.sync_stream(lane->stream);
    --lent_;
    if(lane == &bound_) {
      bound_lent_ = false;
      return;
    }
    lane->next = free_;
    free_ = lane;
  }
  // The end of synchronous work: wait now, or in a held run at its end.
  void finish(Lane* lane) noexcept {
    if(holding_) held_ = lane;
    else give_back(lane);
  }

  void bind(Stream stream) noexcept {
    if(bound_lent_ || enqueued_) trap();
    bound_.stream = stream;
    binding_ = true;
  }
  void unbind() noexcept {
    if(bound_lent_ || enqueued_) trap();
    binding_ = false;
  }
  void hold() noexcept { ++holding_; }
  void settle() noexcept {
    if(!holding_) trap();
    if(--holding_ == 0 && held_) give_back(held_);
  }
  void enqueue(Stream stream) noexcept {
    if(enqueued_ || holding_ || bound_lent_) trap();
    saved_binding_ = binding_;
    saved_stream_ = bound_.stream;
    bound_.stream = stream;
    binding_ = enqueued_ = true;
    holding_ = 1;
  }
  void leave() noexcept {
    if(!enqueued_ || holding_ != 1) trap();
    if(held_) give_back(held_);
    holding_ = 0;
    enqueued_ = false;
    binding_ = saved_binding_;
    bound_.stream = saved_stream_;
  }
  // Before the host reads a result: wait for the held run so far. An enqueued call never waits.
  void observed() noexcept {
    if(enqueued_) trap();
    if(held_) give_back(held_);
  }

  std::size_t streams_made() const noexcept { return made_; }
  std::size_t lent() const noexcept { return lent_; }
  bool bound() const noexcept { return binding_; }
  bool enqueued() const noexcept { return enqueued_; }
  Api& api() noexcept { return api_; }

private:
  Event event_of(Lane& lane) noexcept {
    if(&lane == &bound_ && !bound_event_) bound_.event = api_.make_event(), bound_event_ = true;
    return lane.event;
  }

  Api api_;
  Lane* free_ = nullptr;
  std::size_t lent_ = 0, made_ = 0, holding_ = 0;
  Lane bound_{};
  bool binding_ = false, bound_lent_ = false, bound_event_ = false, enqueued_ = false;
  Lane* held_ = nullptr;
  bool saved_binding_ = false;
  Stream saved_stream_{};
};

// Synchronous work: queued on the context's synchronous lane; returns once that lane has run it (at once in a held
// run, whose end waits).
template<class Api, class Q> inline void synchronous(Context<Api>& ctx, Q&& queue) noexcept {
  typename Context<Api>::Lane* lane = ctx.lend(true);
  queue(lane->stream);
  ctx.finish(lane);
}

}  // namespace cr::reuse
