// CPU model of the library's scratch pool (torchvulkan_amd/csrc/scratch_pool.h)
// under a simulated device: streams are queues of operations that run only
// when the model advances them, and every use of a buffer is an operation on
// some stream. The model checks the pool's ownership rules:
//   1. a buffer is never freed while an operation that uses it is pending;
//   2. a buffer is only ever used on one stream (so stream order alone orders
//      its successive holders);
//   3. two holders never share a buffer;
//   4. the hot path (a lease for a stream that has a large enough idle
//      buffer) neither allocates nor drains the device.
// Scenarios: same-stream reuse, several streams, growth while another lease is
// held, out-of-memory recovery, and a multi-threaded stress run.
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

struct Model {
    typedef int Stream;

    std::recursive_mutex mu;
    std::map<int, std::vector<void*>> queue;   // stream -> pending uses
    std::map<void*, int> home;                 // buffer -> the stream it was used on
    std::set<void*> live;
    std::map<void*, size_t> sizes;
    size_t budget = size_t(1) << 40, in_use = 0;
    long allocs = 0, frees = 0, drains = 0;

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
            for (void* u : kv.second)
                if (u == p) die("a buffer was freed while a use of it was pending");
        CHECK(live.erase(p) == 1, "free of an unknown buffer");
        in_use -= sizes[p];
        sizes.erase(p);
        home.erase(p);
        std::free(p);
        ++frees;
    }
    void sync_device() {
        std::lock_guard<std::recursive_mutex> lk(mu);
        for (auto& kv : queue) kv.second.clear();
        ++drains;
    }

    // ---- simulation ----
    void use(void* p, int s) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        CHECK(live.count(p) == 1, "use of a freed buffer");
        auto it = home.find(p);
        if (it == home.end()) home[p] = s;
        else CHECK(it->second == s, "a buffer was used on a second stream");
        queue[s].push_back(p);
    }
    void run_stream(int s) {
        std::lock_guard<std::recursive_mutex> lk(mu);
        queue[s].clear();
    }
};

typedef tvk::ScratchPool<Model> Pool;

void same_stream_reuse() {
    Model m;
    Pool pool(m, 1024);
    auto* a = pool.acquire(100, 1);
    m.use(a->ptr, 1);
    pool.release(a);
    const long allocs = m.allocs, drains = m.drains;
    auto* b = pool.acquire(200, 1);
    CHECK(b == a, "a released buffer big enough is reused on the same stream");
    CHECK(m.allocs == allocs && m.drains == drains, "the hot path neither allocates nor drains");
    m.use(b->ptr, 1);
    pool.release(b);
    pool.trim();
    CHECK(m.live.empty(), "trim frees every idle buffer");
}

void streams_keep_their_buffers() {
    Model m;
    Pool pool(m, 1024);
    auto* a = pool.acquire(100, 1);
    m.use(a->ptr, 1);
    pool.release(a);
    auto* b = pool.acquire(100, 2);   // stream 1's buffer is idle but not stream 2's
    CHECK(b != a, "another stream gets its own buffer");
    m.use(b->ptr, 2);
    pool.release(b);
    auto* c = pool.acquire(100, 1);
    CHECK(c == a, "each stream reuses its own buffer");
    m.use(c->ptr, 1);
    auto* d = pool.acquire(100, 1);
    CHECK(d != c, "two holders on one stream get two buffers");
    m.use(d->ptr, 1);
    pool.release(c);
    pool.release(d);
    pool.trim();
    CHECK(m.live.empty() && m.allocs == m.frees, "every buffer freed once");
}

void grow_while_held() {
    Model m;
    Pool pool(m, 1024);
    auto* small = pool.acquire(100, 1);   // held by "another thread"
    m.use(small->ptr, 1);
    auto* big = pool.acquire(1 << 20, 1);
    CHECK(big != small && big->bytes >= (1u << 20), "growth allocates beside a held buffer");
    CHECK(m.live.count(small->ptr) == 1, "a held buffer is not freed by growth");
    m.use(big->ptr, 1);
    pool.release(big);
    pool.release(small);                  // its use is still pending
    // a request larger than every idle buffer of the stream retires them:
    // only after the device drained (the model aborts otherwise)
    auto* bigger = pool.acquire(4 << 20, 1);
    CHECK(m.live.size() == 1, "idle buffers too small for a request are retired");
    m.use(bigger->ptr, 1);
    pool.release(bigger);
    pool.trim();
    CHECK(m.live.empty() && m.allocs == m.frees, "every buffer freed once");
}

void out_of_memory() {
    Model m;
    m.budget = 3000;
    Pool pool(m, 1024);
    auto* a = pool.acquire(1024, 1);
    auto* b = pool.acquire(1024, 2);
    m.use(a->ptr, 1);
    m.use(b->ptr, 2);
    pool.release(a);
    // 2048 in use: a 1900-byte buffer for stream 3 fits only after the idle
    // one of stream 1 is given back (after the device drained)
    auto* c = pool.acquire(1900, 3);
    CHECK(c != nullptr, "idle buffers of any stream are released to satisfy a request");
    CHECK(pool.acquire(4096, 3) == nullptr, "a request beyond the budget fails cleanly");
    m.use(c->ptr, 3);
    pool.release(c);
    pool.release(b);
    pool.trim();
    CHECK(m.live.empty(), "every buffer freed");
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
            pool.release(buf);
            if (rng() % 64 == 0) m.run_stream(stream);
        }
    };
    std::vector<std::thread> ts;
    for (int t = 0; t < 6; ++t) ts.emplace_back(worker, t);
    for (auto& t : ts) t.join();
    CHECK(pool.held_count() == 0, "no lease left held");
    pool.trim();
    CHECK(m.live.empty(), "every buffer freed after trim");
}

}  // namespace

int main() {
    same_stream_reuse();
    streams_keep_their_buffers();
    grow_while_held();
    out_of_memory();
    threads();
    std::printf("ok\n");
    return 0;
}
