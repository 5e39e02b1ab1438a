// lhip_pool.h -- the host thread pool of the host-table GEMM path
// (lhip_matmul_host): fp64 <-> fp32 conversions split into parts across a few
// threads.  Plain C++ (no HIP), so that it can be built and checked on its own.
//
// run(parts, fn) calls fn(0) .. fn(parts - 1) once each, on the calling thread
// and on the workers, and returns when every call has returned.  Parts are
// claimed through one 64-bit counter that carries the generation of the run in
// its high half, so a worker that wakes late (after its run has finished and
// another has started) cannot claim a part of the newer run with the older
// run's fn: a claim is a compare-and-swap that only succeeds while the counter
// still carries the worker's generation and an unclaimed index.  The caller
// therefore never waits for workers to wake up, only for the parts they took.
//
// The first `spinners` workers spin (with a pause instruction) for up to
// `spin_us` microseconds after each generation before they block on their own
// condition variable, so that back-to-back small calls find them awake: a
// futex wake-up costs several microseconds, about what a small call's
// conversions take in all.  A run of at most spinners + 1 parts signals only
// the spinners' condition variable; waking every worker for each
// of a small call's runs (and their turns at the mutex) cost ~100 us a call.
// Awake workers read a run's fn and part count through a sequence lock, not
// the mutex.
#pragma once

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace lhip {

class HostPool {
public:
    explicit HostPool(int spinners = 3, int spin_us = 1000) : spinners_(spinners), spin_us_(spin_us) {}

    // How long the spinners (and a caller waiting for workers' parts) spin
    // before they block; 0 makes them block at once.  Takes effect from the
    // next wait of each thread.
    void set_spin_us(int us) { spin_us_.store(us < 0 ? 0 : us, std::memory_order_relaxed); }
    int spin_us() const { return spin_us_.load(std::memory_order_relaxed); }
    ~HostPool() { stop(); }
    HostPool(const HostPool&) = delete;
    HostPool& operator=(const HostPool&) = delete;

    // worker threads + the calling thread
    int threads() const { return static_cast<int>(workers_.size()) + 1; }
    int spinners() const { return std::min(spinners_, static_cast<int>(workers_.size())); }

    void start(int max_threads = kMaxThreads)
    {
        if (!workers_.empty()) return;
        unsigned hw = std::thread::hardware_concurrency();
        int n = static_cast<int>(hw > 0 ? hw : 4);
        if (n > max_threads) n = max_threads;
        {
            std::lock_guard<std::mutex> g(mu_);
            quit_.store(false, std::memory_order_relaxed);
        }
        const unsigned long long g0 = gen_.load(std::memory_order_acquire);   // new workers wait for the next one
        for (int i = 1; i < n; ++i) workers_.emplace_back([this, i, g0] { loop(i - 1, g0); });
    }

    void stop()
    {
        publish(nullptr, 0, true);
        cv_.notify_all();
        spin_cv_.notify_all();
        for (auto& t : workers_) t.join();
        workers_.clear();
    }

    void run(int parts, const std::function<void(int)>& fn)
    {
        if (workers_.empty() || parts <= 1) {
            for (int p = 0; p < parts; ++p) fn(p);
            return;
        }
        const unsigned long long gen = publish(&fn, parts, false);
        spin_cv_.notify_all();
        if (parts > spinners() + 1) cv_.notify_all();
        claim(gen, &fn, parts);
        // the parts that workers took: spin briefly, then block
        const auto t0 = std::chrono::steady_clock::now();
        for (int it = 1; remaining_.load(std::memory_order_acquire) > 0; ++it) {
            cpu_pause();
            if ((it & 255) == 0 && std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(spin_us())) {
                std::unique_lock<std::mutex> g(mu_);
                caller_waits_.store(true);
                done_cv_.wait(g, [&] { return remaining_.load() == 0; });
                caller_waits_.store(false);
                break;
            }
        }
    }

private:
    static constexpr int kMaxThreads = 16;
    static constexpr unsigned long long kIdx = 0xffffffffULL;

    static unsigned long long tag(unsigned long long gen) { return (gen & kIdx) << 32; }

    static void cpu_pause()
    {
#if defined(__x86_64__) || defined(__i386__)
        __builtin_ia32_pause();
#else
        std::this_thread::yield();
#endif
    }

    // gen_ is a sequence lock over fn_, parts_ and quit_: odd while they are
    // written, advanced by two per generation.  The mutex orders the writes
    // with the sleepers' condition-variable waits.
    unsigned long long publish(const std::function<void(int)>* fn, int parts, bool quit)
    {
        std::lock_guard<std::mutex> g(mu_);
        const unsigned long long s = gen_.load(std::memory_order_relaxed);
        gen_.store(s + 1, std::memory_order_relaxed);
        std::atomic_thread_fence(std::memory_order_release);
        remaining_.store(parts, std::memory_order_relaxed);
        next_.store(tag(s + 2), std::memory_order_relaxed);
        parts_.store(parts, std::memory_order_relaxed);
        fn_.store(fn, std::memory_order_relaxed);
        if (quit) quit_.store(true, std::memory_order_relaxed);
        gen_.store(s + 2, std::memory_order_release);
        return s + 2;
    }

    // A consistent (generation, fn, parts, quit) of the latest publish.
    void snapshot(unsigned long long& gen, const std::function<void(int)>*& fn, int& parts, bool& quit) const
    {
        while (true) {
            const unsigned long long s1 = gen_.load(std::memory_order_acquire);
            if (s1 & 1) { cpu_pause(); continue; }
            fn = fn_.load(std::memory_order_relaxed);
            parts = parts_.load(std::memory_order_relaxed);
            quit = quit_.load(std::memory_order_relaxed);
            std::atomic_thread_fence(std::memory_order_acquire);
            if (gen_.load(std::memory_order_relaxed) == s1) { gen = s1; return; }
        }
    }

    // Claim and run parts of generation gen until none is left (or a newer
    // generation has replaced it).
    void claim(unsigned long long gen, const std::function<void(int)>* fn, int parts)
    {
        const unsigned long long t = tag(gen);
        unsigned long long v = next_.load(std::memory_order_acquire);
        while ((v & ~kIdx) == t && static_cast<int>(v & kIdx) < parts) {
            if (!next_.compare_exchange_weak(v, v + 1, std::memory_order_acq_rel, std::memory_order_acquire))
                continue;   // v was reloaded
            (*fn)(static_cast<int>(v & kIdx));
            // the last part: wake the caller if it went to sleep (it sets
            // caller_waits_ before testing remaining_, this tests it after
            // the decrement; sequentially consistent, so one sees the other)
            if (remaining_.fetch_sub(1) == 1 && caller_waits_.load()) {
                std::lock_guard<std::mutex> g(mu_);
                done_cv_.notify_all();
            }
            v = next_.load(std::memory_order_acquire);
        }
    }

    void loop(int idx, unsigned long long seen)
    {
        const bool spinner = idx < spinners_;
        std::condition_variable& cv = spinner ? spin_cv_ : cv_;
        while (true) {
            bool moved = false;
            if (spinner) {
                const auto t0 = std::chrono::steady_clock::now();
                for (int it = 1;; ++it) {
                    if (gen_.load(std::memory_order_acquire) != seen) { moved = true; break; }
                    cpu_pause();
                    if ((it & 255) == 0 &&
                        std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(spin_us()))
                        break;
                }
            }
            if (!moved) {
                std::unique_lock<std::mutex> g(mu_);
                cv.wait(g, [&] { return gen_.load(std::memory_order_relaxed) != seen; });
            }
            unsigned long long gen;
            const std::function<void(int)>* fn;
            int parts;
            bool quit;
            snapshot(gen, fn, parts, quit);
            seen = gen;
            if (quit) return;
            if (fn) claim(gen, fn, parts);
        }
    }

    const int spinners_;
    std::atomic<int> spin_us_;
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, spin_cv_, done_cv_;   // other workers, spinners, the caller
    std::atomic<unsigned long long> gen_{0};           // sequence lock, +2 per generation
    std::atomic<const std::function<void(int)>*> fn_{nullptr};
    std::atomic<int> parts_{0};
    std::atomic<bool> quit_{false};
    std::atomic<unsigned long long> next_{0};          // (generation << 32) | next part
    std::atomic<int> remaining_{0};                    // parts of the current run not yet finished
    std::atomic<bool> caller_waits_{false};
};

}  // namespace lhip
