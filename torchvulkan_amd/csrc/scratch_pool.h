// Pool of library scratch buffers for one device, ordered by streams.
//
// Kernels of a call that need scratch memory (split-K partials, repacked
// operands, convolution partials, the attention delta) lease one buffer for
// the duration of the call's launches:
//   - a held buffer belongs to its holder alone: a second acquirer, on any
//     thread or stream, gets another buffer;
//   - a buffer keeps the stream its first lease named and is only ever leased
//     again for that stream, where stream order alone puts the next holder's
//     kernels after the previous holder's. Nothing is recorded on the hot path
//     (an event per call would put a barrier packet between every pair of
//     kernels);
//   - buffers are freed only on a slow path (a request larger than every idle
//     buffer of its stream, an allocation failure, trim), after the whole
//     device has drained, so no kernel of any stream can still use them; held
//     buffers are never freed.
// The logic is independent of HIP: the backend supplies allocation and the
// device-wide wait, so the ownership rules can be exercised on the CPU with a
// model backend.
#pragma once

#include <cstddef>
#include <memory>
#include <mutex>
#include <vector>

namespace tvk {

// Backend B provides:
//   typedef ... Stream;
//   void* alloc(size_t bytes);    nullptr when out of memory
//   void free(void* p);
//   void sync_device();           blocks the host until every stream's work has run
template <class B>
class ScratchPool {
public:
    typedef typename B::Stream Stream;

    struct Buffer {
        void* ptr = nullptr;
        size_t bytes = 0;
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
        bool small_idle = false;
        for (auto& up : bufs_) {
            Buffer* b = up.get();
            if (b->held || !(b->stream == s)) continue;
            if (b->bytes < bytes) {
                small_idle = true;
                continue;
            }
            if (!pick || b->bytes < pick->bytes) pick = b;
        }
        if (!pick) {
            // this stream's idle buffers are all too small: replace them
            if (small_idle) retire_idle_locked([&](const Buffer& b) { return b.stream == s && b.bytes < bytes; });
            const size_t sz = bytes > min_bytes_ ? bytes : min_bytes_;
            void* p = b_.alloc(sz);
            if (!p) {
                retire_idle_locked([](const Buffer&) { return true; });   // give every idle buffer back, retry once
                p = b_.alloc(sz);
                if (!p) return nullptr;
            }
            std::unique_ptr<Buffer> nb(new Buffer());
            nb->ptr = p;
            nb->bytes = sz;
            nb->stream = s;
            bufs_.push_back(std::move(nb));
            pick = bufs_.back().get();
        }
        pick->held = true;
        return pick;
    }

    // Ends a lease; the next lease for the same stream may take the buffer.
    void release(Buffer* buf) {
        if (!buf) return;
        std::lock_guard<std::mutex> lk(mu_);
        buf->held = false;
    }

    // Frees every idle buffer (held buffers stay).
    void trim() {
        std::lock_guard<std::mutex> lk(mu_);
        retire_idle_locked([](const Buffer&) { return true; });
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
    // Frees the idle buffers `which` selects, after the device has drained.
    template <class Pred>
    void retire_idle_locked(Pred which) {
        bool any = false;
        for (auto& b : bufs_) any = any || (!b->held && which(*b));
        if (!any) return;
        b_.sync_device();
        for (size_t i = 0; i < bufs_.size();) {
            Buffer* b = bufs_[i].get();
            if (b->held || !which(*b)) {
                ++i;
                continue;
            }
            b_.free(b->ptr);
            bufs_.erase(bufs_.begin() + (std::ptrdiff_t)i);
        }
    }

    B& b_;
    const size_t min_bytes_;
    std::mutex mu_;
    std::vector<std::unique_ptr<Buffer>> bufs_;
};

}  // namespace tvk
