// Stress check of lhip::HostPool (lanternl_amd/csrc/lhip_pool.h), built and run
// by tests/test_host_pool.py (also under ThreadSanitizer).  Every run() must
// call each part exactly once and return only after all of them returned;
// workers are let fall asleep between some runs (short and long pauses), the
// spin window is switched between 0 and 200 us while they run, and the pool
// is stopped and restarted.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <functional>
#include <random>
#include <thread>
#include <vector>

#include "../../lanternl_amd/csrc/lhip_pool.h"

int main(int argc, char** argv)
{
    const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
    std::mt19937 rng(12345);
    long long bad = 0;
    for (int round = 0; round < 2; ++round) {
        lhip::HostPool pool(3, 200);
        pool.start(8);
        for (int it = 0; it < iters; ++it) {
            const int parts = 1 + static_cast<int>(rng() % 9);
            std::vector<int> hits(parts, 0);          // plain ints: a late or doubled call is a race
            std::vector<long long> out(parts, 0);
            pool.run(parts, [&](int p) {
                hits[p] += 1;
                long long s = 0;
                for (int i = 0; i < 200 * (p + 1); ++i) s += i ^ p;
                out[p] = s;
            });
            for (int p = 0; p < parts; ++p) {
                long long s = 0;
                for (int i = 0; i < 200 * (p + 1); ++i) s += i ^ p;
                if (hits[p] != 1 || out[p] != s) ++bad;
            }
            const unsigned r = rng() % 100;
            if (r < 3) std::this_thread::sleep_for(std::chrono::microseconds(400));   // past the spin window
            else if (r < 8) std::this_thread::sleep_for(std::chrono::microseconds(50));
            // the spin window changed while workers spin or sleep (0: block at once)
            if (r == 50) pool.set_spin_us(0);
            else if (r == 51) pool.set_spin_us(200);
        }
        pool.stop();
        pool.start(4);   // restart, then let the destructor join
        std::vector<int> hits(5, 0);
        pool.run(5, [&](int p) { hits[p] += 1; });
        for (int h : hits)
            if (h != 1) ++bad;
    }
    std::printf("%s bad=%lld\n", bad ? "FAIL" : "ok", bad);
    return bad ? 1 : 0;
}
