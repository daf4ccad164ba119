#include "host_pool.h"

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <thread>
#include <vector>

namespace redukt_host {
namespace {

// Workers sleep on a generation counter; a job is published by bumping it.  Each worker
// with id < job's width claims units through one shared atomic index.  A job ends when
// all of its units have run and no worker that took it is still draining, so a worker
// can never carry one job's body or index over into the next job.
class Pool {
public:
    Pool() {
        unsigned hw = std::thread::hardware_concurrency();
        if (const char* env = std::getenv("REDUKT_HOST_THREADS")) {
            const long v = std::strtol(env, nullptr, 10);
            if (v > 0) hw = unsigned(v);
        }
        threads_ = std::max(1u, hw);
        for (unsigned i = 1; i < threads_; ++i) workers_.emplace_back([this, i] { loop(i); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
            ++gen_;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }
    unsigned threads() const { return threads_; }

    void run(size_t count, unsigned width, const std::function<void(size_t)>& body) {
        std::lock_guard<std::mutex> serial(run_mu_);
        width = std::min<unsigned>(width == 0 ? threads_ : width, threads_);
        width = unsigned(std::min<size_t>(width, count));
        {
            std::lock_guard<std::mutex> g(mu_);
            body_ = &body;
            count_ = count;
            width_ = width;
            next_.store(0, std::memory_order_relaxed);
            done_ = 0;
            ++gen_;
        }
        cv_.notify_all();
        const size_t mine = drain(body, count);
        std::unique_lock<std::mutex> g(mu_);
        done_ += mine;
        // Every unit has run AND every worker that took this job has left drain(): a worker
        // still inside drain() holds `body` and reads next_, so the job (and the next one's
        // reset of next_ and done_) must wait for it.
        done_cv_.wait(g, [&] { return done_ == count_ && busy_ == 0; });
        body_ = nullptr;
    }

private:
    size_t drain(const std::function<void(size_t)>& body, size_t count) {
        size_t n = 0;
        for (size_t i; (i = next_.fetch_add(1, std::memory_order_relaxed)) < count; ++n) body(i);
        return n;
    }

    void loop(unsigned id) {
        uint64_t seen = 0;
        for (;;) {
            const std::function<void(size_t)>* body;
            size_t count;
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return gen_ != seen; });
                seen = gen_;
                if (stop_) return;
                if (id >= width_ || body_ == nullptr) continue;
                body = body_;
                count = count_;
                ++busy_;
            }
            const size_t n = drain(*body, count);
            {
                std::lock_guard<std::mutex> g(mu_);
                done_ += n;
                --busy_;
                if (done_ == count_ && busy_ == 0) done_cv_.notify_all();
            }
        }
    }

    unsigned threads_ = 1;
    std::vector<std::thread> workers_;
    std::mutex run_mu_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    uint64_t gen_ = 0;
    bool stop_ = false;
    const std::function<void(size_t)>* body_ = nullptr;
    size_t count_ = 0, done_ = 0;
    unsigned busy_ = 0;  // workers between taking the current job and leaving drain()
    unsigned width_ = 0;
    std::atomic<size_t> next_{0};
};

Pool& pool() {
    static Pool p;
    return p;
}

}  // namespace

unsigned pool_threads() { return pool().threads(); }

void parallel_for_fn(size_t count, unsigned threads, const std::function<void(size_t)>& body) {
    pool().run(count, threads, body);
}

}  // namespace redukt_host
