// Stream-ordered pool of library scratch buffers for one device.
//
// Kernels of a call that need scratch memory (split-K partials, repacked
// operands, convolution partials, the attention delta) lease one buffer for
// the duration of the call's launches:
//   - a held buffer belongs to its holder alone: a second acquirer, on any
//     thread or stream, gets another buffer;
//   - on release the pool records an event on the holder's stream after the
//     holder's work; a later lease on the same stream needs nothing more
//     (stream order), a lease on another stream first makes that stream wait
//     for the event;
//   - growing never frees a held buffer: idle buffers too small for a request
//     are freed only after their last use has completed (their event), and a
//     new, larger buffer is allocated beside any that are still held.
// The logic is independent of HIP: the backend supplies the allocation,
// event and stream-wait operations, so the ownership rules can be exercised
// on the CPU with a model backend.
#pragma once

#include <cstddef>
#include <memory>
#include <mutex>
#include <vector>

namespace tvk {

// Backend B provides:
//   typedef ... Stream; typedef ... Event;
//   void* alloc(size_t bytes);            nullptr when out of memory
//   void free(void* p);
//   Event make_event();
//   void destroy_event(Event e);
//   void record(Event e, Stream s);       e completes after the work queued on s so far
//   void wait(Stream s, Event e);         work queued on s from now on runs after e
//   void sync(Event e);                   blocks the host until e has completed
template <class B>
class ScratchPool {
public:
    typedef typename B::Stream Stream;
    typedef typename B::Event Event;

    struct Buffer {
        void* ptr = nullptr;
        size_t bytes = 0;
        Event done{};            // recorded on `stream` when the last holder released
        bool recorded = false;
        Stream stream{};
        bool held = false;
    };

    explicit ScratchPool(B& backend, size_t min_bytes = size_t(16) << 20) : b_(backend), min_bytes_(min_bytes) {}
    ScratchPool(const ScratchPool&) = delete;
    ScratchPool& operator=(const ScratchPool&) = delete;

    // A buffer of at least `bytes` for work queued on `s` from now on, or
    // nullptr when no memory can be had.
    Buffer* acquire(size_t bytes, Stream s) {
        std::lock_guard<std::mutex> lk(mu_);
        Buffer* pick = nullptr;
        for (auto& up : bufs_) {
            Buffer* b = up.get();
            if (b->held || b->bytes < bytes) continue;
            // prefer a buffer last used on this stream (no wait), then the smallest
            const bool same = b->recorded && b->stream == s, pick_same = pick && pick->recorded && pick->stream == s;
            if (!pick || (same && !pick_same) || (same == pick_same && b->bytes < pick->bytes)) pick = b;
        }
        if (!pick) {
            retire_idle_locked(bytes);
            const size_t sz = bytes > min_bytes_ ? bytes : min_bytes_;
            void* p = b_.alloc(sz);
            if (!p) {
                retire_idle_locked(~size_t(0));   // give every idle buffer back and retry once
                p = b_.alloc(sz);
                if (!p) return nullptr;
            }
            std::unique_ptr<Buffer> nb(new Buffer());
            nb->ptr = p;
            nb->bytes = sz;
            nb->done = b_.make_event();
            bufs_.push_back(std::move(nb));
            pick = bufs_.back().get();
        } else if (pick->recorded && !(pick->stream == s)) {
            b_.wait(s, pick->done);
        }
        pick->held = true;
        return pick;
    }

    // Ends a lease: the buffer is free for others once the work queued on `s`
    // so far has run.
    void release(Buffer* buf, Stream s) {
        if (!buf) return;
        std::lock_guard<std::mutex> lk(mu_);
        b_.record(buf->done, s);
        buf->recorded = true;
        buf->stream = s;
        buf->held = false;
    }

    // Frees every idle buffer after its last use (held buffers stay).
    void trim() {
        std::lock_guard<std::mutex> lk(mu_);
        retire_idle_locked(~size_t(0));
    }

    size_t buffer_count() {
        std::lock_guard<std::mutex> lk(mu_);
        return bufs_.size();
    }

    // Bytes of every buffer the pool holds (held or idle).
    size_t total_bytes() {
        std::lock_guard<std::mutex> lk(mu_);
        size_t n = 0;
        for (auto& b : bufs_) n += b->bytes;
        return n;
    }

    size_t held_count() {
        std::lock_guard<std::mutex> lk(mu_);
        size_t n = 0;
        for (auto& b : bufs_) n += b->held ? 1 : 0;
        return n;
    }

private:
    // Frees idle buffers smaller than `below`, each after its last use.
    void retire_idle_locked(size_t below) {
        for (size_t i = 0; i < bufs_.size();) {
            Buffer* b = bufs_[i].get();
            if (b->held || b->bytes >= below) {
                ++i;
                continue;
            }
            if (b->recorded) b_.sync(b->done);
            b_.free(b->ptr);
            b_.destroy_event(b->done);
            bufs_.erase(bufs_.begin() + (std::ptrdiff_t)i);
        }
    }

    B& b_;
    const size_t min_bytes_;
    std::mutex mu_;
    std::vector<std::unique_ptr<Buffer>> bufs_;
};

}  // namespace tvk
