// Stress test of dpep::CopyPool (the shm server's host copy pool), built with
// -fsanitize=thread by tests/test_copy_pool.py.
//
//   copy_pool_stress ROUNDS SEED
//
// Every round copies a random number of jobs of random sizes (so the piece
// count changes from round to round, from none to a few hundred), with
// workers that the pool's hook holds up at random: a yield or a short sleep
// after waking for a round and before pieces.  After each copy() returns,
// every destination byte is checked against its source, and the bytes just
// past each job against a guard value.  ThreadSanitizer reports any data race
// on the piece list or the buffers; a wrong byte exits with status 1.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <random>
#include <thread>
#include <vector>

#include "dpep_copy_pool.h"

namespace {

thread_local std::mt19937 t_rng{std::random_device{}()};

void jitter(dpep::CopyPool::At at)
{
    const unsigned r = t_rng() % 64;
    if (r < 8)
        std::this_thread::yield();
    else if (r == 8)
        usleep(at == dpep::CopyPool::At::wake ? 200 : 20);
}

}  // namespace

int main(int argc, char** argv)
{
    const long rounds = argc > 1 ? atol(argv[1]) : 100000;
    const unsigned seed = argc > 2 ? (unsigned)atol(argv[2]) : 1;
    constexpr size_t kPiece = 64;       // small pieces: many per round
    constexpr size_t kMaxJob = 1024;
    constexpr int kMaxJobs = 6;
    constexpr unsigned char kGuard = 0xA5;
    std::mt19937 rng(seed);
    std::vector<std::vector<unsigned char>> src(kMaxJobs), dst(kMaxJobs);
    for (int j = 0; j < kMaxJobs; ++j) {
        src[j].resize(kMaxJob);
        dst[j].resize(kMaxJob + kPiece);
    }
    long pieces_total = 0;
    {
        dpep::CopyPool pool(7, kPiece, jitter);
        for (long r = 0; r < rounds; ++r) {
            const int nj = (int)(rng() % (kMaxJobs + 1));
            std::vector<dpep::CopyPool::Job> jobs;
            std::vector<size_t> len(nj);
            for (int j = 0; j < nj; ++j) {
                // sizes from 0 to kMaxJob bytes, often not a piece multiple
                len[j] = (rng() % 4 == 0) ? rng() % kPiece : rng() % (kMaxJob + 1);
                const unsigned char tag = (unsigned char)(r * 7 + j);
                for (size_t b = 0; b < len[j]; ++b) src[j][b] = (unsigned char)(tag + b * 13);
                memset(dst[j].data(), kGuard, dst[j].size());
                jobs.push_back({dst[j].data(), src[j].data(), len[j]});
                pieces_total += (long)((len[j] + kPiece - 1) / kPiece);
            }
            pool.copy(jobs);
            for (int j = 0; j < nj; ++j) {
                if (memcmp(dst[j].data(), src[j].data(), len[j]) != 0) {
                    fprintf(stderr, "round %ld job %d: destination differs\n", r, j);
                    return 1;
                }
                for (size_t b = len[j]; b < len[j] + kPiece; ++b)
                    if (dst[j][b] != kGuard) {
                        fprintf(stderr, "round %ld job %d: write past the job\n", r, j);
                        return 1;
                    }
            }
        }
    }
    printf("copy_pool_stress ok: %ld rounds, %ld pieces\n", rounds, pieces_total);
    return 0;
}
