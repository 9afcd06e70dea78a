// KCMM_* tunables: read from the environment once per process, on first use,
// so launch paths do no getenv (and do not race a setenv elsewhere in the
// process); kcmm_reload_tunables() reads them again (for tests and tuning
// runs; not meant to run concurrently with launches).
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "device_api.hpp"

namespace kcmm {
namespace dev {
namespace {

const char* const kNames[static_cast<int>(Tun::kCount)] = {
    "KCMM_ATTN_WAVES", "KCMM_ATTN_HW",   "KCMM_ATTN_MIN_TILES", "KCMM_ATTN_DEPTH",
    "KCMM_ATTN_GENERIC", "KCMM_GEMM_SPLITS", "KCMM_GEMM_WGS", "KCMM_GEMM_TILED",
    "KCMM_GEMM_TILE", "KCMM_GEMM_WAVES", "KCMM_GEMM_HELPERS"};

std::atomic<int> g_set[static_cast<int>(Tun::kCount)];
std::atomic<int> g_val[static_cast<int>(Tun::kCount)];
std::atomic<bool> g_loaded{false};
std::mutex g_mu;

void read_all() {
    for (int i = 0; i < static_cast<int>(Tun::kCount); ++i) {
        const char* e = std::getenv(kNames[i]);
        g_val[i].store(e ? std::atoi(e) : 0, std::memory_order_relaxed);
        g_set[i].store(e ? 1 : 0, std::memory_order_relaxed);
    }
}

}  // namespace

bool tunable(Tun t, int* value) {
    if (!g_loaded.load(std::memory_order_acquire)) {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_loaded.load(std::memory_order_relaxed)) {
            read_all();
            g_loaded.store(true, std::memory_order_release);
        }
    }
    const int i = static_cast<int>(t);
    if (!g_set[i].load(std::memory_order_relaxed)) return false;
    *value = g_val[i].load(std::memory_order_relaxed);
    return true;
}

int tunable_or(Tun t, int dflt) {
    int v = 0;
    return tunable(t, &v) ? v : dflt;
}

void reload_tunables() {
    std::lock_guard<std::mutex> lk(g_mu);
    read_all();
    g_loaded.store(true, std::memory_order_release);
}

}  // namespace dev
}  // namespace kcmm

extern "C" void kcmm_reload_tunables(void) { kcmm::dev::reload_tunables(); }
