// Device page backing for a KCMM pool on MI355X.
//
//  * HipFlatBacking (the backing pools get): each of the 2*L regions is one
//    hipMalloc of the pool's full capacity.  MI355X carries 288 GB of HBM per
//    GPU, so the configured capacity is committed up front and growth costs
//    nothing.  Block ids and offsets are the reference's either way.
//  * VmmBacking<HipVmmOps>: the reference's CUDA-VMM design (ref
//    src/cache/cuda_vmm.rs:6-234, pool.rs:211-221,287-322) on HIP VMM, one
//    reservation per pool.  Switched off: a process that created and
//    destroyed about a dozen VMM pools saw hipMemSetAccess fail with
//    "invalid argument" and then a crash in pool teardown.  The call
//    sequence breaks none of the API's documented preconditions (checked on
//    the CPU against a mock that enforces them); the cause is not known, so
//    KCMM_BACKING=vmm makes pool creation fail.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <thread>
#include <tuple>
#include <vector>

#include "../device_api.hpp"
#include "../vmm_backing.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

// HIP VMM calls for VmmBacking (vmm_backing.hpp).  Not reachable: the VMM
// backing is switched off (make_backing); kept with the bookkeeping it
// drives, which the host-check build tests with a fault-injecting mock.
struct HipVmmOps {
    using Handle = hipMemGenericAllocationHandle_t;
    hipMemAllocationProp prop;
    explicit HipVmmOps(int device) {
        std::memset(&prop, 0, sizeof(prop));
        prop.type = hipMemAllocationTypePinned;
        prop.location.type = hipMemLocationTypeDevice;
        prop.location.id = device;
    }
    bool granularity(size_t* g, std::string* err) {
        KCMM_HIP_CHECK(hipMemGetAllocationGranularity(g, &prop, hipMemAllocationGranularityMinimum),
                       err);
        return true;
    }
    bool reserve(size_t bytes, size_t align, void** va, std::string* err) {
        KCMM_HIP_CHECK(hipMemAddressReserve(va, bytes, align, nullptr, 0), err);
        return true;
    }
    bool create(size_t bytes, Handle* h, std::string* err) {
        KCMM_HIP_CHECK(hipMemCreate(h, bytes, &prop, 0), err);
        return true;
    }
    bool map(void* at, size_t bytes, Handle h, std::string* err) {
        KCMM_HIP_CHECK(hipMemMap(at, bytes, 0, h, 0), err);
        return true;
    }
    bool set_access(void* at, size_t bytes, std::string* err) {
        hipMemAccessDesc desc;
        std::memset(&desc, 0, sizeof(desc));
        desc.location = prop.location;
        desc.flags = hipMemAccessFlagsProtReadWrite;
        KCMM_HIP_CHECK(hipMemSetAccess(at, bytes, &desc, 1), err);
        return true;
    }
    void unmap(void* at, size_t bytes) { (void)hipMemUnmap(at, bytes); }
    void release(Handle h) { (void)hipMemRelease(h); }
    void free_va(void* va, size_t bytes) { (void)hipMemAddressFree(va, bytes); }
};

[[maybe_unused]] std::unique_ptr<PageBacking> make_vmm_backing(int device) {
    return std::unique_ptr<PageBacking>(new VmmBacking<HipVmmOps>(HipVmmOps(device)));
}

class HipFlatBacking final : public PageBacking {
public:
    ~HipFlatBacking() override { release(); }

    bool reserve(size_t num_regions, size_t region_bytes, std::string* err) override {
        for (size_t r = 0; r < num_regions; ++r) {
            void* p = nullptr;
            KCMM_HIP_CHECK(hipMalloc(&p, region_bytes), err);
            bases_.push_back(p);
        }
        return true;
    }
    uint64_t region_base(size_t r) const override {
        return reinterpret_cast<uint64_t>(bases_[r]);
    }
    bool map_superblock(size_t, std::string*) override { return true; }
    void release() override {
        for (void* b : bases_) (void)hipFree(b);
        bases_.clear();
    }
    int kind() const override { return 1; }

private:
    std::vector<void*> bases_;
};

}  // namespace

__global__ void zero_words(u32x4* p, size_t n) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
        p[i] = u32x4{0, 0, 0, 0};
}

namespace dev {

std::unique_ptr<PageBacking> make_backing(int device, std::string* err) {
    const char* env = std::getenv("KCMM_BACKING");
    if (env != nullptr && std::strcmp(env, "vmm") == 0) {
        // Switched off: in one process that created and destroyed about a
        // dozen VMM pools, hipMemSetAccess began to fail ("invalid argument")
        // and pool teardown crashed; the cause is not known.
        *err = "KCMM_BACKING=vmm: the HIP VMM page backing is disabled in this build "
               "(unexplained hipMemSetAccess failures after repeated pool create/destroy); "
               "unset KCMM_BACKING for the flat backing";
        return nullptr;
    }
    return std::unique_ptr<PageBacking>(new HipFlatBacking());
}

bool set_device(int device, std::string* err) {
    KCMM_HIP_CHECK(hipSetDevice(device), err);
    return true;
}

// Device scratch for split-K partials and arrival counters, one buffer per
// (device, stream, user slot, host thread): launches on different streams
// never share one, and a buffer is only ever handed to the thread that
// grows it, so a growth (which frees the old buffer once its stream has
// drained) cannot free a buffer another thread is about to launch with.
// `zero_fill` buffers start zeroed (their users restore zero).
//
// When a thread exits, its buffers become orphans (no HIP call is made at
// thread exit: the runtime may be shutting down); the next workspace
// allocation on any thread, or a pool destroy, synchronizes their device and
// frees them, so a server whose worker threads come and go holds at most
// the buffers of its live threads plus those of threads that exited since
// the last allocation.
namespace {

struct Ws {
    void* ptr = nullptr;
    size_t bytes = 0;
};
using WsKey = std::tuple<int, uint64_t, int, std::thread::id>;

// Never destroyed, so a thread's exit (including the main thread's, after
// main returns) can always reach them.
std::mutex& ws_mutex() {
    static std::mutex* m = new std::mutex;
    return *m;
}
std::map<WsKey, Ws>& ws_table() {
    static auto* t = new std::map<WsKey, Ws>;
    return *t;
}
std::vector<std::pair<int, void*>>& ws_orphans() {
    static auto* v = new std::vector<std::pair<int, void*>>;
    return *v;
}

struct ThreadWsOwner {
    ~ThreadWsOwner() {
        std::lock_guard<std::mutex> lk(ws_mutex());
        const std::thread::id me = std::this_thread::get_id();
        auto& t = ws_table();
        for (auto it = t.begin(); it != t.end();) {
            if (std::get<3>(it->first) == me) {
                if (it->second.ptr) ws_orphans().emplace_back(std::get<0>(it->first), it->second.ptr);
                it = t.erase(it);
            } else {
                ++it;
            }
        }
    }
};
thread_local ThreadWsOwner t_ws_owner;

// Frees the orphaned buffers; call with ws_mutex() held.
bool free_orphans_locked(std::string* err) {
    auto& o = ws_orphans();
    if (o.empty()) return true;
    int cur = 0;
    KCMM_HIP_CHECK(hipGetDevice(&cur), err);
    while (!o.empty()) {
        const int dev = o.back().first;
        KCMM_HIP_CHECK(hipSetDevice(dev), err);
        KCMM_HIP_CHECK(hipDeviceSynchronize(), err);
        for (size_t i = o.size(); i-- > 0;) {
            if (o[i].first != dev) continue;
            KCMM_HIP_CHECK(hipFree(o[i].second), err);
            o.erase(o.begin() + static_cast<std::ptrdiff_t>(i));
        }
    }
    KCMM_HIP_CHECK(hipSetDevice(cur), err);
    return true;
}

}  // namespace

bool stream_workspace(uint64_t stream, int slot, size_t bytes, void** out, bool zero_fill,
                      std::string* err) {
    (void)&t_ws_owner;   // registers this thread's owner (its destructor runs at thread exit)
    int dev = 0;
    KCMM_HIP_CHECK(hipGetDevice(&dev), err);
    std::lock_guard<std::mutex> lk(ws_mutex());
    Ws& w = ws_table()[std::make_tuple(dev, stream, slot, std::this_thread::get_id())];
    if (w.bytes < bytes) {
        if (!free_orphans_locked(err)) return false;
        if (w.ptr) {
            KCMM_HIP_CHECK(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)), err);
            KCMM_HIP_CHECK(hipFree(w.ptr), err);
            w.ptr = nullptr;
            w.bytes = 0;
        }
        const size_t want = (bytes + bytes / 4 + 255) & ~static_cast<size_t>(255);
        KCMM_HIP_CHECK(hipMalloc(&w.ptr, want), err);
        w.bytes = want;
        if (zero_fill) {
            // a kernel, not hipMemsetAsync: callers may be capturing a graph
            const size_t words = want / 16;
            hipLaunchKernelGGL(zero_words, dim3(static_cast<unsigned>(std::min<size_t>((words + 255) / 256, 4096))),
                               dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                               static_cast<u32x4*>(w.ptr), words);
            KCMM_HIP_CHECK(hipGetLastError(), err);
        }
    }
    *out = w.ptr;
    return true;
}

bool release_orphaned_workspaces(std::string* err) {
    std::lock_guard<std::mutex> lk(ws_mutex());
    return free_orphans_locked(err);
}

size_t orphaned_workspaces() {
    std::lock_guard<std::mutex> lk(ws_mutex());
    return ws_orphans().size();
}

bool synchronize_device(int device, std::string* err) {
    int cur = 0;
    KCMM_HIP_CHECK(hipGetDevice(&cur), err);
    if (cur != device) KCMM_HIP_CHECK(hipSetDevice(device), err);
    KCMM_HIP_CHECK(hipDeviceSynchronize(), err);
    if (cur != device) KCMM_HIP_CHECK(hipSetDevice(cur), err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
