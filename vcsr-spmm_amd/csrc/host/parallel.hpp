// parallel.hpp - a small fork-join helper over std::thread.
#pragma once

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <exception>
#include <mutex>
#include <thread>
#include <vector>

namespace vcsr {

// Run body(begin, end) over [0, n) in chunks of `grain`, on up to `nthreads`
// threads, chunks taken dynamically.  The first exception thrown by any chunk
// is rethrown on the calling thread after all workers have stopped.
template <class F>
void parallel_for(int64_t n, int64_t grain, int nthreads, F&& body) {
    if (n <= 0) return;
    if (grain < 1) grain = 1;
    const int64_t nchunks = (n + grain - 1) / grain;
    int nt = (int)std::min<int64_t>(std::max(1, nthreads), nchunks);
    if (nt <= 1) {
        body((int64_t)0, n);
        return;
    }
    std::atomic<int64_t> next{0};
    std::exception_ptr err;
    std::mutex err_mu;
    auto worker = [&]() {
        for (;;) {
            int64_t c = next.fetch_add(1);
            if (c >= nchunks) return;
            int64_t b = c * grain, e = std::min(n, b + grain);
            try {
                body(b, e);
            } catch (...) {
                std::lock_guard<std::mutex> lk(err_mu);
                if (!err) err = std::current_exception();
                next.store(nchunks);
                return;
            }
        }
    };
    std::vector<std::thread> pool;
    pool.reserve((size_t)nt - 1);
    for (int t = 1; t < nt; ++t) pool.emplace_back(worker);
    worker();
    for (auto& th : pool) th.join();
    if (err) std::rethrow_exception(err);
}

}  // namespace vcsr
