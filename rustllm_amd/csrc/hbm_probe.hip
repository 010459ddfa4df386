// hbm_probe.hip -- the attainable HBM time of a streaming launch on this GPU.
//
//     hbm_probe READ_BYTES:WRITE_BYTES [...]
//
// For each pair, one plain streaming kernel that reads READ_BYTES (one
// stream, non-temporal 16-byte loads) and writes WRITE_BYTES (one stream,
// non-temporal 16-byte stores).  Both streams are spread evenly over the
// grid: block b reads and writes its proportional, contiguous share of each
// stream (as a row kernel does), with up to four 16-byte packs per thread
// and stream, every load issued before the first store.  It is timed as 40
// back-to-back launches over windows of a 4 GiB pool (so that no launch
// reuses what the 256 MB Infinity Cache holds from the previous ones), best
// of 3, and as single launches bracketed by events.  Prints one JSON object:
// {"cases": [{"read": R, "write": W, "us": back-to-back us per launch,
// "us_one": one launch}, ...]}.
//
// The bench compares each kernel of the layer chain with this probe at the
// kernel's own read and write bytes: the probe does no arithmetic and no
// index math, so its time is what HBM, the launch and the drain cost for
// those bytes.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 4;

// Block b of nb covers slots [b * S, (b + 1) * S) of the longer stream
// (S = kThreads * kUnroll) and the matching share of the other:
// packs [first(b), first(b + 1)) with first(b) = b * S * n / n_max.
__device__ inline uint64_t share_first(uint64_t b, uint64_t n, uint64_t n_max) {
    return (b * kThreads * kUnroll * n) / n_max;
}

__global__ __launch_bounds__(kThreads) void k_stream(const f4* __restrict__ src,
                                                     f4* __restrict__ dst, uint64_t n_read,
                                                     uint64_t n_write) {
    const uint64_t n_max = n_read > n_write ? n_read : n_write;
    const uint64_t b = blockIdx.x;
    const uint64_t r0 = share_first(b, n_read, n_max), r1 = share_first(b + 1, n_read, n_max);
    const uint64_t w0 = share_first(b, n_write, n_max), w1 = share_first(b + 1, n_write, n_max);
    const uint64_t r_end = r1 < n_read ? r1 : n_read, w_end = w1 < n_write ? w1 : n_write;
    f4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint64_t i = r0 + uint64_t(u) * kThreads + threadIdx.x;
        v[u] = i < r_end ? __builtin_nontemporal_load(src + i) : f4{1.0f, 2.0f, 3.0f, 4.0f};
    }
    f4 acc = v[0];
#pragma unroll
    for (int u = 1; u < kUnroll; ++u) acc += v[u];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint64_t i = w0 + uint64_t(u) * kThreads + threadIdx.x;
        if (i < w_end) __builtin_nontemporal_store(acc + float(u), dst + i);
    }
}

bool ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    fprintf(stderr, "hbm_probe: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

}  // namespace

int main(int argc, char** argv) {
    struct Case {
        uint64_t read, write;
        double us = 0, us_one = 0;
    };
    std::vector<Case> cases;
    for (int a = 1; a < argc; ++a) {
        const std::string s = argv[a];
        const size_t colon = s.find(':');
        if (colon == std::string::npos) {
            fprintf(stderr, "hbm_probe: expected READ_BYTES:WRITE_BYTES, got %s\n", argv[a]);
            return 2;
        }
        Case c;
        c.read = std::strtoull(s.substr(0, colon).c_str(), nullptr, 10);
        c.write = std::strtoull(s.substr(colon + 1).c_str(), nullptr, 10);
        cases.push_back(c);
    }
    const uint64_t pool_bytes = uint64_t(4) << 30;
    char* pool = nullptr;
    if (!ok(hipMalloc(&pool, pool_bytes), "hipMalloc") ||
        !ok(hipMemset(pool, 0, pool_bytes), "hipMemset"))
        return 1;
    hipEvent_t e0, e1;
    if (!ok(hipEventCreate(&e0), "event") || !ok(hipEventCreate(&e1), "event")) return 1;
    for (Case& c : cases) {
        const uint64_t n_read = c.read / 16, n_write = c.write / 16;
        const uint64_t n = n_read > n_write ? n_read : n_write;
        // windows of [read | write] bytes, each rounded up to 4 KiB
        const uint64_t rbytes = (n_read * 16 + 4095) / 4096 * 4096;
        const uint64_t wbytes = (n_write * 16 + 4095) / 4096 * 4096;
        const uint64_t window = rbytes + wbytes;
        if (n == 0 || window > pool_bytes) {
            fprintf(stderr, "hbm_probe: case %llu:%llu does not fit the pool\n",
                    (unsigned long long)c.read, (unsigned long long)c.write);
            return 2;
        }
        uint64_t windows = pool_bytes / window;
        if (windows > 64) windows = 64;
        const unsigned grid = unsigned((n + uint64_t(kThreads) * kUnroll - 1) /
                                       (uint64_t(kThreads) * kUnroll));
        auto launch = [&](uint64_t i) {
            char* w = pool + (i % windows) * window;
            hipLaunchKernelGGL(k_stream, dim3(grid), dim3(kThreads), 0, 0,
                               reinterpret_cast<const f4*>(w), reinterpret_cast<f4*>(w + rbytes),
                               n_read, n_write);
        };
        for (uint64_t i = 0; i < windows; ++i) launch(i);
        if (!ok(hipDeviceSynchronize(), "warm-up")) return 1;
        float best = 1e30f;
        constexpr int kReps = 40;
        for (int rep = 0; rep < 3; ++rep) {
            if (!ok(hipEventRecord(e0, 0), "event")) return 1;
            for (int i = 0; i < kReps; ++i) launch(uint64_t(rep) * kReps + i);
            if (!ok(hipEventRecord(e1, 0), "event") || !ok(hipEventSynchronize(e1), "timing"))
                return 1;
            float ms = 0;
            if (!ok(hipEventElapsedTime(&ms, e0, e1), "elapsed")) return 1;
            best = ms < best ? ms : best;
        }
        c.us = best * 1e3 / kReps;
        double one = 0;
        for (int i = 0; i < 10; ++i) {
            if (!ok(hipEventRecord(e0, 0), "event")) return 1;
            launch(uint64_t(i) * 7);
            if (!ok(hipEventRecord(e1, 0), "event") || !ok(hipEventSynchronize(e1), "timing"))
                return 1;
            float ms = 0;
            if (!ok(hipEventElapsedTime(&ms, e0, e1), "elapsed")) return 1;
            one += ms * 1e3 / 10;
        }
        c.us_one = one;
    }
    printf("{\"cases\": [");
    for (size_t i = 0; i < cases.size(); ++i)
        printf("%s{\"read\": %llu, \"write\": %llu, \"us\": %.3f, \"us_one\": %.3f}", i ? ", " : "",
               (unsigned long long)cases[i].read, (unsigned long long)cases[i].write, cases[i].us,
               cases[i].us_one);
    printf("]}\n");
    return ok(hipFree(pool), "hipFree") ? 0 : 1;
}
