// CopyPool: CPU threads for the host entries' large copies (pqa_api.hip).
// Header-only so that a host-only test can build it with g++.
#pragma once
#include <algorithm>
#include <condition_variable>
#include <cstddef>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace pqa {

// CPU threads that split large copies between pageable and pinned host
// memory: one memcpy per thread (the calling thread takes the first piece).
// A single thread copies ~20 GB/s on the hosts here, below what the PCIe DMA
// of the next stage moves.
struct CopyPool {
    struct Piece {
        char* dst;
        const char* src;
        size_t n;
    };
    std::vector<std::thread> threads;
    std::vector<Piece> pieces;
    std::mutex mu;
    std::condition_variable go, done;
    unsigned gen = 0;
    int pending = 0;
    bool quit = false;

    explicit CopyPool(int workers) : pieces((size_t)workers) {
        for (int i = 0; i < workers; ++i) threads.emplace_back([this, i] { run(i); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> l(mu);
            quit = true;
        }
        go.notify_all();
        for (auto& t : threads) t.join();
    }
    void run(int i) {
        unsigned seen = 0;
        std::unique_lock<std::mutex> l(mu);
        for (;;) {
            go.wait(l, [&] { return quit || gen != seen; });
            if (quit) return;
            seen = gen;
            const Piece p = pieces[(size_t)i];
            l.unlock();
            if (p.n) std::memcpy(p.dst, p.src, p.n);
            l.lock();
            if (--pending == 0) done.notify_one();
        }
    }
    // dst[0, n) = src[0, n)
    void copy(char* dst, const char* src, size_t n) {
        if (threads.empty() || n < (size_t(1) << 20)) {
            std::memcpy(dst, src, n);
            return;
        }
        // parts pieces of per bytes (a multiple of 64) cover [0, n): per is
        // the rounded-up share, so per * parts >= n
        const size_t parts = threads.size() + 1;
        const size_t per = ((n + parts - 1) / parts + 63) & ~size_t(63);
        {
            std::lock_guard<std::mutex> l(mu);
            for (size_t i = 0; i < threads.size(); ++i) {
                const size_t off = std::min(n, per * (i + 1));
                pieces[i] = Piece{dst + off, src + off, std::min(per, n - off)};
            }
            pending = (int)threads.size();
            ++gen;
        }
        go.notify_all();
        std::memcpy(dst, src, std::min(per, n));
        std::unique_lock<std::mutex> l(mu);
        done.wait(l, [&] { return pending == 0; });
    }
};

}  // namespace pqa
