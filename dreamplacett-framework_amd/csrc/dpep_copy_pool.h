// dpep_copy_pool.h -- the shm server's host copy pool: a fixed set of worker
// threads that copy lists of (dst, src, bytes) jobs between the shared-memory
// file and the page-locked staging buffers, with the calling thread taking
// part.  One memcpy thread moves ~10 GB/s, below the host link, so the
// server's uploads and read-backs are split over several.
//
// It serves the reference server's ordering (host/
// density_scatter_ttnn_server_host.cpp:1335-1349, :1785-1815): the positions
// are wholly in the staging buffers before they are uploaded, and the outputs
// wholly in the shm file before DONE is published.  copy() therefore returns
// only when every byte of its jobs has been written AND no worker is still
// inside the round, so the next copy() may rebuild the piece list freely.
//
// Rounds.  A round is open from its publication (under mu_) until the caller
// has run out of pieces and closes it (under mu_).  A worker joins a round
// only while it is open and only once (it remembers the round id), and it
// counts itself in active_ under mu_ before it touches the piece list; copy()
// waits for active_ == 0 after closing.  So:
//   * the piece list and the counters are written only while no worker is
//     active and none can join (the previous round is closed and drained);
//   * a worker that wakes late, after its round closed, sees open_ false and
//     goes back to sleep without reading anything of that round;
//   * every piece is claimed before the caller's own work() returns (it runs
//     until next_ passes the end), and a worker's claimed piece is copied
//     before it leaves active_, so active_ == 0 means every byte is written;
//   * the memcpy writes happen-before copy()'s return through mu_ (the
//     worker's decrement and the caller's wait both hold it).
#pragma once

#include <stddef.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

namespace dpep {

class CopyPool {
  public:
    struct Job {
        void* dst;
        const void* src;
        size_t bytes;
    };
    // Where a worker may be held up: after it woke for a round (before it
    // takes the lock to join it) and before each piece.  A hook is called
    // there when set; tests use it to stall workers at those points.
    enum class At { wake, piece };
    using Hook = void (*)(At);

    explicit CopyPool(int workers, size_t piece_bytes = size_t(1) << 20,
                      Hook hook = nullptr)
        : piece_(piece_bytes ? piece_bytes : 1), hook_(hook)
    {
        for (int i = 0; i < workers; ++i) threads_.emplace_back([this] { run(); });
    }
    ~CopyPool()
    {
        {
            std::lock_guard<std::mutex> g(mu_);
            quit_ = true;
        }
        cv_.notify_all();
        for (auto& t : threads_) t.join();
    }
    CopyPool(const CopyPool&) = delete;
    CopyPool& operator=(const CopyPool&) = delete;

    // Copies every job, split into pieces of at most piece_bytes, and returns
    // when all are written and no worker remains in the round.  One caller
    // at a time.
    void copy(const std::vector<Job>& jobs)
    {
        // no worker is active here: the previous round was closed and
        // drained before the previous copy() returned
        pieces_.clear();
        for (const Job& j : jobs)
            for (size_t o = 0; o < j.bytes; o += piece_)
                pieces_.push_back({(char*)j.dst + o, (const char*)j.src + o,
                                   std::min(piece_, j.bytes - o)});
        if (pieces_.empty()) return;
        {
            std::lock_guard<std::mutex> g(mu_);
            next_.store(0, std::memory_order_relaxed);
            open_ = true;
            ++round_;
        }
        if (pieces_.size() > 1) cv_.notify_all();
        work();
        std::unique_lock<std::mutex> g(mu_);
        open_ = false;
        done_cv_.wait(g, [this] { return active_ == 0; });
    }

  private:
    void work()
    {
        const size_t n = pieces_.size();
        for (;;) {
            const size_t i = next_.fetch_add(1, std::memory_order_relaxed);
            if (i >= n) return;
            if (hook_) hook_(At::piece);
            memcpy(pieces_[i].dst, pieces_[i].src, pieces_[i].bytes);
        }
    }
    void run()
    {
        unsigned long seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return quit_ || (open_ && round_ != seen); });
                if (quit_) return;
                seen = round_;
            }
            // the round may close while this worker is held here; it then
            // must not join it
            if (hook_) hook_(At::wake);
            {
                std::lock_guard<std::mutex> g(mu_);
                if (!open_ || round_ != seen) continue;
                ++active_;
            }
            work();
            {
                std::lock_guard<std::mutex> g(mu_);
                if (--active_ == 0) done_cv_.notify_all();
            }
        }
    }

    const size_t piece_;
    const Hook hook_;
    std::vector<std::thread> threads_;
    std::vector<Job> pieces_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    std::atomic<size_t> next_{0};
    unsigned long round_ = 0;   // under mu_
    int active_ = 0;            // under mu_
    bool open_ = false;         // under mu_
    bool quit_ = false;         // under mu_
};

}  // namespace dpep
