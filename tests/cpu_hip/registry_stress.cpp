// Registry stress under ThreadSanitizer, on the CPU: the library's own
// pk_gpu_runtime.hip against the HIP stand-in (cpu_hip.cpp), the loop shape
// of tests/test_gpu_library.py's unregister test.  GEMM threads call the
// host-pointer drop-in with a registered weight (small-M calls also make and
// read its panel) while another thread unregisters and registers it again.
// Every unregister must return PK_GPU_OK or PK_GPU_EBUSY, every GEMM
// PK_GPU_OK, no copy may be freed while queued work reads it (the stand-in
// runs queued work at synchronisation, on whichever thread synchronises;
// ThreadSanitizer reports a free that races with it), and no GEMM thread may
// do device-wide work (the explicit device synchronisation before a resident
// copy is freed runs on the unregistering thread only).
// Prints one JSON line of counts; exit status 0 when all held.
#include "pk_gpu.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

int main(int argc, char** argv)
{
    // at least `target` unregisters that succeed and as many refused as busy,
    // or `limit_s` seconds
    const long target = argc > 1 ? std::atol(argv[1]) : 50;
    const double limit_s = argc > 2 ? std::atof(argv[2]) : 60.0;
    if (pk_gpu_init(0) != PK_GPU_OK) {
        std::fprintf(stderr, "init: %s\n", pk_gpu_last_error());
        return 2;
    }
    const int K = 256, N = 256;
    std::vector<int8_t> W((size_t)K * N, 3);
    if (pk_gpu_register_weight(W.data(), W.size()) != PK_GPU_OK) return 2;

    std::atomic<bool> stop{false};
    std::atomic<long> gemms{0}, bad{0}, ok{0}, busy{0}, other{0};
    std::vector<std::thread> workers;
    for (int t = 0; t < 4; ++t) {
        workers.emplace_back([&, t] {
            cpu_hip_set_role(1);
            const int M = t % 2 ? 16 : 96;            // small-M (panel) and the other path
            std::vector<float> A((size_t)M * K, 1.0f), C((size_t)M * N, 0.0f);
            unsigned seed = 12345u + 977u * t;
            while (!stop.load()) {
                const int rc = pk_gpu_gemm_i8(M, N, K, 1.0f, A.data(), K, W.data(), 0.01f, N, 0.0f, C.data(), N);
                ++gemms;
                if (rc != PK_GPU_OK) {
                    ++bad;
                    std::fprintf(stderr, "gemm: %d %s\n", rc, pk_gpu_last_error());
                }
                seed = seed * 1103515245u + 12345u;       // a pause of 0-1 ms between calls
                std::this_thread::sleep_for(std::chrono::microseconds((seed >> 16) % 1000));
            }
        });
    }
    const auto t0 = std::chrono::steady_clock::now();
    long rounds = 0;
    while ((ok.load() < target || busy.load() < target) &&
           std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < limit_s) {
        ++rounds;
        std::this_thread::sleep_for(std::chrono::microseconds(100));
        const int rc = pk_gpu_unregister_weight(W.data());
        if (rc == PK_GPU_OK) {
            ++ok;
            if (pk_gpu_register_weight(W.data(), W.size()) != PK_GPU_OK) ++other;
        } else if (rc == PK_GPU_EBUSY) {
            ++busy;
        } else {
            ++other;
            std::fprintf(stderr, "unregister: %d %s\n", rc, pk_gpu_last_error());
        }
    }
    stop.store(true);
    for (std::thread& w : workers) w.join();
    const int last = pk_gpu_unregister_weight(W.data());
    pk_gpu_shutdown();
    const long gemm_thread_syncs = cpu_hip_device_syncs(1);
    std::printf("{\"rounds\": %ld, \"gemms\": %ld, \"gemm_errors\": %ld, \"unregistered\": %ld, "
                "\"busy\": %ld, \"other\": %ld, \"final_unregister\": %d, "
                "\"device_syncs_on_gemm_threads\": %ld}\n",
                rounds, gemms.load(), bad.load(), ok.load(), busy.load(), other.load(), last, gemm_thread_syncs);
    return bad.load() == 0 && other.load() == 0 && last == PK_GPU_OK && ok.load() >= target &&
                   busy.load() >= target && gemm_thread_syncs == 0
               ? 0
               : 1;
}
