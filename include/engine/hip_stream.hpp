#pragma once
//===----------------------------------------------------------------------===//
// engine/hip_stream.hpp -- move-only RAII streams and events.
//
// HIP counterpart of the reference's CudaStream / CudaEvent
// (include/engine/cuda_stream.hpp:21-124): a stream is non-blocking by
// default, an event records timing by default; both are move-only and
// release their handle in the destructor. Created through the C-ABI
// (eng_stream_* / eng_event_*), always at the default stream priority.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>

#include <hip/hip_runtime_api.h>

namespace engine {

class HipEvent;

class HipStream {
 public:
  HipStream() : HipStream(ENG_STREAM_NON_BLOCKING) {}
  explicit HipStream(unsigned int flags) {
    eng_stream s = nullptr;
    ENGINE_ABI_CHECK(eng_stream_create(&s, flags));
    stream_ = reinterpret_cast<hipStream_t>(s);
  }
  ~HipStream() {
    if (stream_ != nullptr) (void)eng_stream_destroy(stream_);
  }

  HipStream(const HipStream&) = delete;
  HipStream& operator=(const HipStream&) = delete;
  HipStream(HipStream&& o) noexcept : stream_(o.stream_) { o.stream_ = nullptr; }
  HipStream& operator=(HipStream&& o) noexcept {
    if (this != &o) {
      if (stream_ != nullptr) (void)eng_stream_destroy(stream_);
      stream_ = o.stream_;
      o.stream_ = nullptr;
    }
    return *this;
  }

  hipStream_t get() const { return stream_; }
  operator hipStream_t() const { return stream_; }

  void synchronize() const {
    if (stream_ != nullptr) ENGINE_ABI_CHECK(eng_stream_sync(stream_));
  }

  void wait(const HipEvent& event, unsigned int flags = 0) const;

 private:
  hipStream_t stream_ = nullptr;
};

class HipEvent {
 public:
  HipEvent() : HipEvent(ENG_EVENT_DEFAULT) {}
  explicit HipEvent(unsigned int flags) {
    eng_event e = nullptr;
    ENGINE_ABI_CHECK(eng_event_create(&e, flags));
    event_ = reinterpret_cast<hipEvent_t>(e);
  }
  ~HipEvent() {
    if (event_ != nullptr) (void)eng_event_destroy(event_);
  }

  HipEvent(const HipEvent&) = delete;
  HipEvent& operator=(const HipEvent&) = delete;
  HipEvent(HipEvent&& o) noexcept : event_(o.event_) { o.event_ = nullptr; }
  HipEvent& operator=(HipEvent&& o) noexcept {
    if (this != &o) {
      if (event_ != nullptr) (void)eng_event_destroy(event_);
      event_ = o.event_;
      o.event_ = nullptr;
    }
    return *this;
  }

  hipEvent_t get() const { return event_; }
  operator hipEvent_t() const { return event_; }

  void record(hipStream_t stream = nullptr) {
    ENGINE_CHECK(event_ != nullptr, "HipEvent::record called on null event");
    ENGINE_ABI_CHECK(eng_event_record(event_, stream));
  }

  void synchronize() const {
    if (event_ != nullptr) ENGINE_ABI_CHECK(eng_event_sync(event_));
  }

  bool is_complete() const {
    if (event_ == nullptr) return true;
    int done = 0;
    ENGINE_ABI_CHECK(eng_event_query(event_, &done));
    return done != 0;
  }

  static float elapsed_ms(const HipEvent& start, const HipEvent& end) {
    ENGINE_CHECK(start.get() != nullptr && end.get() != nullptr,
                 "HipEvent::elapsed_ms called on uninitialized event");
    float ms = 0.0f;
    ENGINE_ABI_CHECK(eng_event_elapsed_ms(&ms, start.get(), end.get()));
    return ms;
  }

 private:
  hipEvent_t event_ = nullptr;
};

inline void HipStream::wait(const HipEvent& event, unsigned int flags) const {
  ENGINE_CHECK(event.get() != nullptr, "HipStream::wait called on null event");
  ENGINE_ABI_CHECK(eng_stream_wait_event(stream_, event.get(), flags));
}

}  // namespace engine
