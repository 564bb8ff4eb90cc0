// fn(i) for i in [0, n) on up to `threads` host threads (this one among
// them).  Indices are taken in increasing order from a shared counter; when
// several calls throw, the exception of the lowest index is rethrown after
// every thread has finished, so the report matches a sequential loop's.  A
// thread that cannot be started leaves its share to the others.
#pragma once

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <exception>
#include <mutex>
#include <system_error>
#include <thread>
#include <vector>

namespace mslim {

template <class F>
void parallel_indices(size_t n, size_t threads, F fn) {
    std::atomic<size_t> next{0};
    std::mutex m;
    size_t failed = SIZE_MAX;
    std::exception_ptr error;
    auto worker = [&] {
        for (size_t i = next++; i < n; i = next++) {
            try {
                fn(i);
            } catch (...) {
                std::lock_guard<std::mutex> g(m);
                if (i < failed) {
                    failed = i;
                    error = std::current_exception();
                }
            }
        }
    };
    threads = std::max<size_t>(1, std::min(threads, n));
    std::vector<std::thread> pool;
    pool.reserve(threads);
    try {
        for (size_t t = 1; t < threads; ++t) pool.emplace_back(worker);
    } catch (const std::system_error &) {
        // fewer threads than asked: the started ones and this one do it all
    }
    worker();
    for (auto &t : pool) t.join();
    if (error) std::rethrow_exception(error);
}

// Host threads for parallel record work: the machine's, at most 16.
inline size_t host_worker_threads() {
    const unsigned hw = std::thread::hardware_concurrency();
    return std::min<size_t>(16, hw ? hw : 1);
}

}  // namespace mslim
