// CPU model of the library's scratch pool (torchvulkan_amd/csrc/scratch_pool.h)
// under a simulated device: streams are queues of operations that run only
// when the model advances them, events complete when the stream reaches the
// position they were recorded at, and every use of a buffer is an operation
// on some stream. The model checks the pool's ownership rules:
//   1. a buffer is never freed while an operation that uses it is pending;
//   2. a buffer handed to stream s2 after use on stream s1 is used on s2 only
//      after s2 waits for s1's last use of it (or that use has run);
//   3. two holders never share a buffer.
// Scenarios: same-stream reuse, cross-stream reuse, growth while another
// lease is held, out-of-memory recovery, and a multi-threaded stress run.
// Prints "ok" and exits 0 on success; any violation aborts with a message.
#include "scratch_pool.h"

#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <random>
#include <set>
#include <thread>
#include <vector>

namespace {

[[noreturn]] void die(const char* what) {
    std::fprintf(stderr, "scratch pool model: %s\n", what);
    std::abort();
}
#define CHECK(c, msg) do { if (!(c)) die(msg); } while (0)

struct Op {
    enum Kind { USE, WAIT } kind;
    void* ptr;         // USE
    int on_stream;     // WAIT: stream waited for
    long on_pos;       // WAIT: position (exclusive) it must have run to
};

struct Model {
    typedef int Stream;
    typedef int Event;

    std::recursive_mutex mu;
    std::map<int, std::vector<Op>> queue;   // stream -> operations
    std::map<int, long> ran;                // stream -> operations run so far
    std::map<int, std::map<int, long>> clock;   // stream -> (stream -> position it is ordered after)
    std::map<int, std::pair<int, long>> events; // event -> (stream, position) recorded
    std::set<void*> live;
    size_t budget = size_t(1) << 40, in_use = 0;
    std::map<void*, size_t> sizes;
    int next_event = 1;
    long allocs = 0, frees = 0, waits = 0;

    // ---- backend interface ----
    void* alloc(size_t bytes) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        if (in_use + bytes > budget) return nullptr;
        void* p = std::malloc(1);
        live.insert(p);
        sizes[p] = bytes;
        in_use += bytes;
        ++allocs;
        return p;
    }
    void free(void* p) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        for (auto& kv : queue)
            for (long i = ran[kv.first]; i < (long)kv.second.size(); ++i)
                if (kv.second[i].kind == Op::USE && kv.second[i].ptr == p) die("a buffer was freed while a use of it was pending");
        CHECK(live.erase(p) == 1, "free of an unknown buffer");
        in_use -= sizes[p];
        sizes.erase(p);
        std::free(p);
        ++frees;
    }
    Event make_event() {
        std::lock_guard<std::recursive_mutex> lk(mu);
        return next_event++;
    }
    void destroy_event(Event e) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        events.erase(e);
    }
    void record(Event e, Stream s) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        events[e] = {s, (long)queue[s].size()};
    }
    void wait(Stream s, Event e) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        auto it = events.find(e);
        CHECK(it != events.end(), "wait on an event never recorded");
        queue[s].push_back(Op{Op::WAIT, nullptr, it->second.first, it->second.second});
        long& c = clock[s][it->second.first];
        c = std::max(c, it->second.second);
        ++waits;
    }
    void sync(Event e) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        auto it = events.find(e);
        CHECK(it != events.end(), "sync on an event never recorded");
        run_until(it->second.first, it->second.second);
    }

    // ---- simulation ----
    // Runs stream s up to position pos (exclusive), running what its waits need first.
    void run_until(int s, long pos) {
        std::vector<Op>& q = queue[s];
        long& r = ran[s];
        while (r < pos && r < (long)q.size()) {
            const Op& op = q[r];
            if (op.kind == Op::WAIT) run_until(op.on_stream, op.on_pos);
            ++r;
        }
    }
    // Queues a use of p on s, checking rule 2 against pending uses on other streams.
    void use(void* p, int s) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        CHECK(live.count(p) == 1, "use of a freed buffer");
        for (auto& kv : queue) {
            const int other = kv.first;
            if (other == s) continue;
            for (long i = ran[other]; i < (long)kv.second.size(); ++i) {
                const Op& op = kv.second[i];
                if (op.kind == Op::USE && op.ptr == p && clock[s][other] <= i)
                    die("a buffer was used on a stream before that stream waited for its pending use on another stream");
            }
        }
        queue[s].push_back(Op{Op::USE, p, 0, 0});
    }
    void run_all() {
        std::lock_guard<std::recursive_mutex> lk(mu);
        for (auto& kv : queue) run_until(kv.first, (long)kv.second.size());
    }
};

typedef tvk::ScratchPool<Model> Pool;

void same_stream_reuse() {
    Model m;
    Pool pool(m, 1024);
    auto* a = pool.acquire(100, 1);
    m.use(a->ptr, 1);
    pool.release(a, 1);
    auto* b = pool.acquire(200, 1);
    CHECK(b == a, "a released buffer big enough is reused on the same stream");
    CHECK(m.waits == 0, "reuse on the same stream needs no wait");
    m.use(b->ptr, 1);
    pool.release(b, 1);
    m.run_all();
    pool.trim();
    CHECK(m.live.empty(), "trim frees every idle buffer");
}

void cross_stream_reuse() {
    Model m;
    Pool pool(m, 1024);
    auto* a = pool.acquire(100, 1);
    m.use(a->ptr, 1);
    pool.release(a, 1);
    auto* b = pool.acquire(100, 2);   // still pending on stream 1
    CHECK(b == a, "an idle buffer is reused across streams");
    CHECK(m.waits == 1, "reuse on another stream waits for the event");
    m.use(b->ptr, 2);                 // checked against the pending use on stream 1
    pool.release(b, 2);
    m.run_all();
    pool.trim();
}

void prefer_same_stream() {
    Model m;
    Pool pool(m, 1024);
    auto* a = pool.acquire(100, 1);
    auto* b = pool.acquire(100, 2);
    CHECK(a != b, "two holders get two buffers");
    m.use(a->ptr, 1);
    m.use(b->ptr, 2);
    pool.release(a, 1);
    pool.release(b, 2);
    auto* c = pool.acquire(100, 2);
    CHECK(c == b, "the buffer last used on the acquiring stream is preferred");
    CHECK(m.waits == 0, "no wait when the same stream's buffer is taken");
    pool.release(c, 2);
    m.run_all();
    pool.trim();
}

void grow_while_held() {
    Model m;
    Pool pool(m, 1024);
    auto* small = pool.acquire(100, 1);   // held by "another thread"
    m.use(small->ptr, 1);
    auto* big = pool.acquire(1 << 20, 2);
    CHECK(big != small && big->bytes >= (1u << 20), "growth allocates beside a held buffer");
    CHECK(m.live.count(small->ptr) == 1, "a held buffer is not freed by growth");
    m.use(big->ptr, 2);
    pool.release(big, 2);
    pool.release(small, 1);               // pending use on stream 1 remains
    // a request larger than every idle buffer retires the small one: only
    // after its last use has run (the model aborts otherwise)
    auto* bigger = pool.acquire(4 << 20, 3);
    CHECK(m.live.size() == 1, "idle buffers too small for a request are retired");
    m.use(bigger->ptr, 3);
    pool.release(bigger, 3);
    m.run_all();
    pool.trim();
    CHECK(m.live.empty() && m.allocs == m.frees, "every buffer freed once");
}

void out_of_memory() {
    Model m;
    m.budget = 3000;
    Pool pool(m, 1024);
    auto* a = pool.acquire(1024, 1);
    auto* b = pool.acquire(1024, 1);
    m.use(a->ptr, 1);
    pool.release(a, 1);
    // 1024 + 1024 in use: a 2000-byte buffer fits only after the idle one is
    // given back (after its pending use has run)
    auto* c = pool.acquire(1900, 2);
    CHECK(c != nullptr, "idle buffers are released to satisfy a request");
    CHECK(pool.acquire(4096, 2) == nullptr, "a request beyond the budget fails cleanly");
    pool.release(c, 2);
    pool.release(b, 1);
    m.run_all();
    pool.trim();
}

void threads() {
    Model m;
    Pool pool(m, 256);
    std::mutex held_mu;
    std::set<void*> held;
    auto worker = [&](int tid) {
        std::mt19937 rng(1234 + tid);
        const int stream = 10 + tid % 3;   // several threads share some streams
        for (int it = 0; it < 3000; ++it) {
            const size_t want = 64u << (rng() % 8);
            auto* buf = pool.acquire(want, stream);
            CHECK(buf && buf->bytes >= want, "acquire returns a large enough buffer");
            {
                std::lock_guard<std::mutex> lk(held_mu);
                CHECK(held.insert(buf->ptr).second, "two holders share a buffer");
            }
            m.use(buf->ptr, stream);
            {
                std::lock_guard<std::mutex> lk(held_mu);
                held.erase(buf->ptr);
            }
            pool.release(buf, stream);
            if (rng() % 64 == 0) {
                std::lock_guard<std::recursive_mutex> lk(m.mu);
                m.run_until(stream, (long)m.queue[stream].size());
            }
        }
    };
    std::vector<std::thread> ts;
    for (int t = 0; t < 6; ++t) ts.emplace_back(worker, t);
    for (auto& t : ts) t.join();
    CHECK(pool.held_count() == 0, "no lease left held");
    m.run_all();
    pool.trim();
    CHECK(m.live.empty(), "every buffer freed after trim");
}

}  // namespace

int main() {
    same_stream_reuse();
    cross_stream_reuse();
    prefer_same_stream();
    grow_while_held();
    out_of_memory();
    threads();
    std::printf("ok\n");
    return 0;
}
