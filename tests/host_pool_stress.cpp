// Stress test of the host thread pool (redukt_amd/csrc/host/host_pool.cpp), built by
// tests/test_host_pool.py with ThreadSanitizer and with AddressSanitizer on the host.
//
// Back-to-back parallel_for jobs with shrinking and growing unit counts, more threads than
// cores, each job's body bound to storage that dies when the job returns.  Every unit must
// run exactly once, inside its own job: a worker that carried one job's body over into the
// next would touch freed storage (ASan), race on it (TSan) or leave a unit count != 1.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <vector>

#include "host_pool.h"

int main(int argc, char** argv) {
    const int jobs = argc > 1 ? std::atoi(argv[1]) : 20000;
    unsigned bad = 0;
    for (int j = 0; j < jobs; ++j) {
        // Counts cycle down and up (like lockstep's active set as files finish and new
        // files are admitted), including 0, 1 and counts below the thread count.
        const size_t count = size_t((j * 7919u) % 97u);
        const unsigned width = unsigned(j % 5 == 0 ? 0 : 1 + j % 40);
        std::unique_ptr<std::atomic<int>[]> hits(new std::atomic<int>[count ? count : 1]);
        for (size_t i = 0; i < count; ++i) hits[i].store(0, std::memory_order_relaxed);
        std::vector<size_t> seen(count, 0);
        const int tag = j;
        redukt_host::parallel_for(count, width, [&, tag](size_t i) {
            if (i >= count || tag != j) {
                std::fprintf(stderr, "job %d: unit %zu outside the job (count %zu, tag %d)\n", j, i, count, tag);
                std::abort();
            }
            hits[i].fetch_add(1, std::memory_order_relaxed);
            seen[i] = i + 1;  // plain writes: each unit owns its element
        });
        for (size_t i = 0; i < count; ++i) {
            if (hits[i].load() != 1 || seen[i] != i + 1) {
                if (bad < 10) std::fprintf(stderr, "job %d: unit %zu ran %d times\n", j, i, hits[i].load());
                ++bad;
            }
        }
    }
    if (bad) {
        std::fprintf(stderr, "%u units ran a wrong number of times\n", bad);
        return 1;
    }
    std::printf("ok: %d jobs on %u threads\n", jobs, redukt_host::pool_threads());
    return 0;
}
