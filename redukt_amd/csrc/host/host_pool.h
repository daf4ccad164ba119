// A persistent pool of host threads for the per-stream work of a lockstep step (CDF
// construction and range coding).  It decides only WHICH thread runs a unit, never how:
// every unit is a pure function of its own inputs, so results do not depend on the thread
// count (the identity rule of src/application/lockstep.rs:16-21).
#pragma once

#include <cstddef>
#include <functional>
#include <utility>

namespace redukt_host {

// Host threads the pool can use (hardware threads, at least 1).
unsigned pool_threads();

// Runs body(i) for i in [0, count) on up to `threads` threads (0 = all of them), the
// calling thread included; returns when every unit has finished.  Calls from several
// threads at once are serialised.
void parallel_for_fn(size_t count, unsigned threads, const std::function<void(size_t)>& body);

template <class F>
inline void parallel_for(size_t count, unsigned threads, F&& body) {
    if (count == 0) return;
    if (count == 1 || threads == 1) {
        for (size_t i = 0; i < count; ++i) body(i);
        return;
    }
    parallel_for_fn(count, threads, std::function<void(size_t)>(std::forward<F>(body)));
}

}  // namespace redukt_host
