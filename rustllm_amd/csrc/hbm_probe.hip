// hbm_probe.hip -- the attainable HBM time of a streaming launch on this GPU.
//
//     hbm_probe READ_BYTES:WRITE_BYTES [...]
//
// For each pair, plain streaming kernels that read READ_BYTES (one stream,
// non-temporal 16-byte loads) and write WRITE_BYTES (one stream,
// non-temporal 16-byte stores), four 16-byte packs per thread and stream,
// every load issued before the first store, in two layouts:
//  * phased: thread pack i is loaded if i < reads and stored if i < writes,
//    so the blocks past the shorter stream's end move one stream only;
//  * interleaved: block b moves its proportional, contiguous share of each
//    stream (as a row kernel does).
// Each is timed as 40 back-to-back launches over windows of a 4 GiB pool
// (so that no launch reuses what the 256 MB Infinity Cache holds from the
// previous ones), best of 3, and as single launches bracketed by events.
// Prints one JSON object: {"cases": [{"read": R, "write": W, "us": the
// faster layout's back-to-back us per launch, "us_phased": ..,
// "us_interleaved": .., "us_one": one launch of the faster}, ...]}.
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

__global__ __launch_bounds__(kThreads) void k_phased(const f4* __restrict__ src,
                                                     f4* __restrict__ dst, uint64_t n_read,
                                                     uint64_t n_write) {
    const uint64_t base = uint64_t(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
    f4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint64_t i = base + uint64_t(u) * kThreads;
        v[u] = i < n_read ? __builtin_nontemporal_load(src + i) : f4{1.0f, 2.0f, 3.0f, 4.0f};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint64_t i = base + uint64_t(u) * kThreads;
        if (i < n_write) __builtin_nontemporal_store(v[u], dst + i);
    }
}

// Block b covers slots [b * S, (b + 1) * S) of the longer stream
// (S = kThreads * kUnroll) and packs [first(b), first(b + 1)) of each stream
// of n packs, first(b) = floor(b * S * (n / n_max)) (the ratio in double,
// the last block ending at n); a share is at most S packs.
__device__ inline uint64_t share_first(uint64_t b, double ratio, uint64_t n) {
    if (b >= gridDim.x) return n;
    const uint64_t f = uint64_t(double(b * kThreads * kUnroll) * ratio);
    return f < n ? f : n;
}

__global__ __launch_bounds__(kThreads) void k_interleaved(const f4* __restrict__ src,
                                                          f4* __restrict__ dst, uint64_t n_read,
                                                          uint64_t n_write, double r_ratio,
                                                          double w_ratio) {
    const uint64_t b = blockIdx.x;
    const uint64_t r0 = share_first(b, r_ratio, n_read), r1 = share_first(b + 1, r_ratio, n_read);
    const uint64_t w0 = share_first(b, w_ratio, n_write);
    const uint64_t w1 = share_first(b + 1, w_ratio, n_write);
    f4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint64_t i = r0 + uint64_t(u) * kThreads + threadIdx.x;
        v[u] = i < r1 ? __builtin_nontemporal_load(src + i) : f4{1.0f, 2.0f, 3.0f, 4.0f};
    }
    f4 acc = v[0];
#pragma unroll
    for (int u = 1; u < kUnroll; ++u) acc += v[u];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint64_t i = w0 + uint64_t(u) * kThreads + threadIdx.x;
        if (i < w1) __builtin_nontemporal_store(acc + float(u), dst + i);
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
        double us = 0, us_one = 0, us_phased = 0, us_interleaved = 0;
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
        const double r_ratio = double(n_read) / double(n), w_ratio = double(n_write) / double(n);
        for (int layout = 0; layout < 2; ++layout) {
            auto launch = [&](uint64_t i) {
                char* w = pool + (i % windows) * window;
                const f4* src = reinterpret_cast<const f4*>(w);
                f4* dst = reinterpret_cast<f4*>(w + rbytes);
                if (layout == 0)
                    hipLaunchKernelGGL(k_phased, dim3(grid), dim3(kThreads), 0, 0, src, dst,
                                       n_read, n_write);
                else
                    hipLaunchKernelGGL(k_interleaved, dim3(grid), dim3(kThreads), 0, 0, src, dst,
                                       n_read, n_write, r_ratio, w_ratio);
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
            const double us = best * 1e3 / kReps;
            (layout == 0 ? c.us_phased : c.us_interleaved) = us;
            if (layout == 0 || us < c.us) {
                c.us = us;
                c.us_one = one;
            }
        }
    }
    printf("{\"cases\": [");
    for (size_t i = 0; i < cases.size(); ++i)
        printf("%s{\"read\": %llu, \"write\": %llu, \"us\": %.3f, \"us_phased\": %.3f, "
               "\"us_interleaved\": %.3f, \"us_one\": %.3f}",
               i ? ", " : "", (unsigned long long)cases[i].read,
               (unsigned long long)cases[i].write, cases[i].us, cases[i].us_phased,
               cases[i].us_interleaved, cases[i].us_one);
    printf("]}\n");
    return ok(hipFree(pool), "hipFree") ? 0 : 1;
}
