// common.hpp -- shared pieces of the gfx950 tensor-op library: the context
// struct behind rl_context, error reporting, launch bookkeeping, and the
// device helpers (16-byte packs, f16 conversion, wave64 reductions, fast
// 32-bit division by a runtime constant).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>

#include "rustllm_hip.h"

namespace rl {

// ------------------------------------------------------------------ errors

rl_status fail(rl_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Failures whose TinyError variant carries data: the message is the
// reference's Display text (src/error.rs:56-95) and the fields are kept for
// rl_last_error_payload.
rl_status fail_shape_mismatch(const uint64_t* left, uint32_t left_rank, const uint64_t* right,
                              uint32_t right_rank);
rl_status fail_position_out_of_range(uint64_t start_pos, uint64_t seq_len, uint64_t max_seq_len);
rl_status fail_invalid_token_id(uint32_t token_id, uint64_t vocab_size);

// ------------------------------------------------------------------ pool

// Stream-ordered caching allocator.  All work of a context runs in order on
// one stream, so a block released by the host can be handed to the next
// allocation at once: any kernel that still reads it was enqueued earlier
// and finishes before anything enqueued later touches the block.
struct BufferPool {
    std::multimap<uint64_t, void*> free_blocks;    // size class -> block
    std::unordered_map<void*, uint64_t> block_size;  // every live or free block
    uint64_t reserved_bytes = 0;

    static uint64_t size_class(uint64_t bytes);
    rl_status allocate(uint64_t bytes, void** out);
    void release(void* ptr);
    void trim();
    ~BufferPool();
};

// A streaming op deferred while a graph is recorded: independent ones are
// launched together as one kernel (elementwise.hip: flush_fused).  `kind`
// names the op's body, `blocks` its share of the grid; the byte ranges it
// reads and writes decide which ops may share a launch.
struct FusedOp {
    uint32_t kind = 0;
    uint32_t blocks = 0;
    const void* a = nullptr;
    const void* b = nullptr;
    void* out = nullptr;
    uint64_t n_packs = 0;
    uint32_t tail = 0;       // map: elements after the last pack
    uint32_t div = 1;        // packs per row (bias add, row gather) or per head (repeat_kv)
    uint64_t head_packs = 0;  // repeat_kv
    uint32_t repeats = 0;
    bool small_index = false;
    uint32_t outer_rank = 0;  // row gather / scatter: outer dims, innermost first
    uint32_t outer_dim[4] = {1, 1, 1, 1};
    uint32_t outer_stride[4] = {0, 0, 0, 0};
    uintptr_t read[2][2] = {{0, 0}, {0, 0}};  // [begin, end) of each input
    uintptr_t write[2] = {0, 0};
};
constexpr uint32_t kMaxFused = 16;
constexpr uint32_t kMaxFusedOuterRank = 4;
// Fused kinds (elementwise.hip launches them): maps, bias adds, row
// gathers and repeat_kv.
enum FusedKind : uint32_t {
    kFusedAddF32 = 1, kFusedMulF32, kFusedSiluF32, kFusedSwigluF32,
    kFusedAddF16, kFusedMulF16, kFusedSiluF16, kFusedSwigluF16,
    kFusedCastF32F16, kFusedCastF16F32, kFusedBiasF32, kFusedBiasF16,
    kFusedGatherF32, kFusedGatherF16, kFusedRepeatF32, kFusedRepeatF16,
    kFusedScatterF32, kFusedScatterF16,  // row copies walked in source order
};

}  // namespace rl

struct rl_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool owns_stream = false;
    int num_cus = 256;
    rl::BufferPool pool;

    int active_executions = 0;
    bool capturing = false;

    bool profiling = false;
    rl_profile profile{};
    std::map<std::string, uint64_t> dispatches_by_name;

    // Set by rl_event_time_next_kernel: the next launch records its own
    // start and end in these events.
    hipEvent_t timed_start = nullptr;
    hipEvent_t timed_stop = nullptr;

    // Pinned host staging for small host arrays an op takes by value (the
    // embedding's token ids): copied here, then to device memory in stream
    // order; `staging_done` marks when the last such copy has read it.
    void* staging = nullptr;
    uint64_t staging_bytes = 0;
    hipEvent_t staging_done = nullptr;
    bool staging_pending = false;

    // One counter per (batch, KV head) for the decode attention's split
    // hand-off, one per 256 bytes: zero between launches (the workgroup that
    // draws the last ticket puts it back).  Grown on demand, freed with the
    // context.  ticket_count is in 32-bit words.
    uint32_t* tickets = nullptr;
    uint64_t ticket_count = 0;

    // Streaming ops recorded into a graph but not yet launched (at most
    // kMaxFused, no two touching the same bytes unless both only read them).
    rl::FusedOp fused[rl::kMaxFused];
    uint32_t fused_count = 0;
    bool fuse_recorded = true;  // rl_context_set_fusion
    // A fused launch that failed where no status could be returned (inside
    // RL_LAUNCH): reported by the next after_launch.
    hipError_t fused_error = hipSuccess;
};


namespace rl {
// Launches the deferred streaming ops as one kernel (nothing if there are
// none).  Every other stream operation of a recording context calls it
// first, so the recorded order is the call order.
rl_status flush_fused(rl_context* ctx);
// Adds an op to the deferred ones, launching those first if the op writes
// bytes one of them touches, reads bytes one of them writes, or the batch
// is full.
rl_status defer_fused(rl_context* ctx, const FusedOp& f);
// Whether an op launched now on `ctx` is deferred for a fused launch.
inline bool fusing(const rl_context* ctx) {
    return ctx->capturing && ctx->fuse_recorded && ctx->timed_start == nullptr;
}
}  // namespace rl

// Every kernel launch of the library: on the context's stream, and, when
// armed by rl_event_time_next_kernel, with the kernel's own start/end
// timestamps recorded (hipExtLaunchKernelGGL).
#define RL_LAUNCH(ctx, kernel, grid, block, ...)                                              \
    do {                                                                                      \
        if ((ctx)->fused_count != 0 && rl::flush_fused(ctx) != RL_OK)                         \
            (ctx)->fused_error = hipErrorLaunchFailure; /* reported by after_launch */        \
        if ((ctx)->timed_start != nullptr) {                                                  \
            hipExtLaunchKernelGGL(kernel, grid, block, 0, (ctx)->stream, (ctx)->timed_start,  \
                                  (ctx)->timed_stop, 0, __VA_ARGS__);                         \
            (ctx)->timed_start = nullptr;                                                     \
            (ctx)->timed_stop = nullptr;                                                      \
        } else {                                                                              \
            hipLaunchKernelGGL(kernel, grid, block, 0, (ctx)->stream, __VA_ARGS__);           \
        }                                                                                     \
    } while (0)

namespace rl {

// Common prologue of every op: after validation, a NULL context is reported
// as a device error (validation itself needs no device).
inline rl_status require_context(rl_context* ctx) {
    if (ctx == nullptr) return fail(RL_ERR_DEVICE, "no HIP context (validation passed)");
    return RL_OK;
}

// Makes the context's device current for the calling thread.
rl_status activate(rl_context* ctx);

// Bookkeeping after a kernel launch: launch errors become RL_ERR_DEVICE and
// the dispatch is counted in an active profile.
rl_status after_launch(rl_context* ctx, const char* kernel_name);

// Copies `bytes` of host memory to a pool block in the context's stream
// order (through the pinned staging area) and returns the block in *dev.
// The caller enqueues its readers and then releases the block to the pool.
// Not allowed while recording a graph (the copy would replay stale data).
rl_status stage_to_device(rl_context* ctx, const void* host, uint64_t bytes, void** dev);

// Checks of a KV-cache write of a [1, H, S, D] source view (dims/strides,
// rank 4) into a [1, H, max_seq, D] cache of `es`-byte elements; with
// `exact_source` the source buffer must hold exactly H*S*D elements.
rl_status validate_kv_write(const char* name, const rl_buffer* cache, uint64_t max_seq,
                            const rl_buffer* src, const uint64_t* dims, const uint64_t* strides,
                            uint32_t rank, uint64_t start, uint64_t es, bool exact_source);

inline bool aligned_to(const void* p, uint64_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Buffer checks shared by the ops; messages follow the reference's wording.
rl_status check_buffer(const rl_buffer* b, const char* what);
rl_status check_output(const rl_buffer* out, uint64_t len, uint64_t element_size,
                       const char* op);

// ------------------------------------------------------------ fast divmod

// Division of a 32-bit numerator by a runtime-constant 32-bit divisor with a
// multiply-high, a 64-bit add and a shift (Granlund & Montgomery, "Division
// by invariant integers using multiplication", PLDI 1994, unsigned case with
// a 33-bit magic whose top bit is the explicit "+ n").
struct FastDiv {
    uint32_t divisor;
    uint32_t magic;
    uint32_t shift;

    FastDiv() : divisor(1), magic(1), shift(0) {}
    explicit FastDiv(uint32_t d) : divisor(d) {
        uint32_t s = 0;
        while ((uint64_t(1) << s) < d) ++s;
        shift = s;
        magic = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
    }
    __host__ __device__ inline uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        uint32_t hi = __umulhi(n, magic);
#else
        uint32_t hi = uint32_t((uint64_t(n) * magic) >> 32);
#endif
        return uint32_t((uint64_t(hi) + n) >> shift);
    }
    __host__ __device__ inline void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
        q = div(n);
        r = n - q * divisor;
    }
};

// The row dims of a strided [..., S, D] view (every dim but the innermost D)
// in the order rows are enumerated, fastest first.  Decoding row index r
// gives the source element offset, the sequence position (the coordinate of
// dim `seq_dim`) and the group: the flat index of the other row dims in the
// view's own row-major order (e.g. the head of a [1, H, S, D] view), which
// places the row in a contiguous or cache-shaped destination.
constexpr int kMaxRowRank = 16;
template <int R>
struct RowDimsN {
    uint32_t rank;
    uint32_t seq_dim;
    FastDiv dim[R];
    uint64_t stride[R];
    uint32_t group_mult[R];
};
typedef RowDimsN<kMaxRowRank> RowDims;

// Rows enumerated in the view's memory order (row dims sorted by source
// stride, smallest first), so consecutive rows read consecutive memory where
// the view allows: for the [1, H, S, D] permute of a [1, S, H, D] projection
// the heads of one position come together, reading the projection straight
// through and sharing that position's table row.  dims/strides: outermost
// first, `rank` >= 2 including the innermost dim.
// RowDimsN<R> holds views of up to R row dims (rank <= R + 1).
template <int R = kMaxRowRank>
inline RowDimsN<R> make_row_dims(const uint64_t* dims, const uint64_t* strides, uint32_t rank) {
    RowDimsN<R> rd{};
    const uint32_t n = rank - 1;  // row dims: 0 .. rank - 2; the sequence dim is rank - 2
    uint32_t order[R];
    for (uint32_t i = 0; i < n; ++i) order[i] = n - 1 - i;  // innermost first
    for (uint32_t i = 1; i < n; ++i) {  // stable insertion sort by stride
        const uint32_t v = order[i];
        uint32_t j = i;
        while (j > 0 && strides[order[j - 1]] > strides[v]) {
            order[j] = order[j - 1];
            --j;
        }
        order[j] = v;
    }
    rd.rank = n;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t d = order[i];
        rd.dim[i] = FastDiv(uint32_t(dims[d]));
        rd.stride[i] = strides[d];
        if (d == n - 1) {
            rd.seq_dim = i;
            rd.group_mult[i] = 0;
        } else {
            uint64_t mult = 1;  // row-major over the row dims other than the sequence dim
            for (uint32_t e = d + 1; e < n - 1; ++e) mult *= dims[e];
            rd.group_mult[i] = uint32_t(mult);
        }
    }
    return rd;
}

template <int R>
__device__ inline void decode_row(const RowDimsN<R>& rd, uint32_t row, uint64_t& src_off,
                                  uint32_t& position, uint32_t& group) {
    src_off = 0;
    position = 0;
    group = 0;
    for (uint32_t d = 0; d < rd.rank; ++d) {
        uint32_t q, r;
        rd.dim[d].divmod(row, q, r);
        src_off += uint64_t(r) * rd.stride[d];
        if (d == rd.seq_dim)
            position = r;
        else
            group += r * rd.group_mult[d];
        row = q;
    }
}

}  // namespace rl

// ------------------------------------------------------------ device side

namespace rl {

typedef _Float16 half_t;

// Streamed (non-temporal) loads pay only where a launch reads more than the
// 256 MB MALL keeps between launches: below about 160 MB of reads, plain
// loads find part of the data there (f16 softmax, [15, 2048, 2048] causal:
// 33.7 -> 26.4 us plain; P V, 15 heads x [1024, 4096]: 60 -> 48 us), above it
// streamed loads win by 3-4 %.
constexpr uint64_t kStreamReadBytes = uint64_t(160) << 20;

template <typename T, int N>
struct VecOf {
    typedef T type __attribute__((ext_vector_type(N)));
};

// N elements of T at the alignment of one element: a row of a width that is
// not a multiple of N starts off the 16-byte grid.  gfx950 runs global memory
// in unaligned mode, so a load or store of this type is still one 16-byte
// access (split by the hardware where it crosses a cache line).
template <typename T, int N>
struct VecOfU {
    typedef T type __attribute__((ext_vector_type(N), aligned(sizeof(T))));
};

// One 16-byte pack of T.
template <typename T>
struct Pack16 {
    static constexpr int N = 16 / sizeof(T);
    typedef typename VecOf<T, N>::type type;
};

__device__ inline float to_float(float v) { return v; }
// rope.hip: a plain copy of a [..., S, D] view (unit innermost stride) into
// rows group * group_rows + first_row + s of dst on the row-block kernel;
// false (nothing launched) when the view does not fit that kernel.
template <typename T>
bool launch_copy_rows(rl_context* ctx, const T* src, const uint64_t* dims,
                      const uint64_t* strides, uint32_t rank, T* dst, uint32_t group_rows,
                      uint32_t first_row);

__device__ inline float to_float(half_t v) { return static_cast<float>(v); }

template <typename T>
__device__ inline T from_float(float v);
template <>
__device__ inline float from_float<float>(float v) { return v; }
template <>
__device__ inline half_t from_float<half_t>(float v) { return static_cast<half_t>(v); }  // RNE

template <typename V>
__device__ inline V load_stream(const V* p) {
    return __builtin_nontemporal_load(p);
}

template <typename V>
__device__ inline void store_stream(V* p, V v) {
    __builtin_nontemporal_store(v, p);
}

// The same for N elements of T at the alignment of one element (VecOfU), for
// packs that start off the 16-byte grid.  The builtins see the pointer as
// spelled here, so the access keeps the element alignment; passed through
// load_stream / store_stream the deduced V would drop VecOfU's alignment
// attribute and claim 16.
template <typename T, int N>
__device__ inline typename VecOf<T, N>::type load_stream_u(const T* p) {
    typedef typename VecOfU<T, N>::type U;
    return __builtin_nontemporal_load(reinterpret_cast<const U*>(p));
}

// A plain (cached) load of such a pack.
template <typename T, int N>
__device__ inline typename VecOf<T, N>::type load_u(const T* p) {
    typedef typename VecOfU<T, N>::type U;
    return *reinterpret_cast<const U*>(p);
}

template <typename T, int N>
__device__ inline void store_stream_u(T* p, typename VecOf<T, N>::type v) {
    typedef typename VecOfU<T, N>::type U;
    const U u = v;
    __builtin_nontemporal_store(u, reinterpret_cast<U*>(p));
}

// e^x as 2^(x * log2 e) on the hardware exp2 (v_exp_f32), which returns
// 0 for -inf, inf for +inf and NaN for NaN by itself.  The only error beyond
// the instruction's own ~1 ulp is the rounding of t = x * log2 e, which
// scales the result by 2^(dt) with |dt| <= |t| * 2^-24: a relative error of
// at most |t| * 2^-24 * ln 2, i.e. <= 2.7e-6 over the finite range of e^x
// (|t| < 128) and <= 3e-7 for |x| < 10.
// The instruction flushes results below 2^-126 to zero, so arguments whose
// result would be subnormal are raised by 64 and the result scaled back by
// an exact power of two.
__device__ inline float exp_fast(float x) {
    const float t = x * 1.44269504088896340736f;
    const bool tiny = t < -126.0f;
    const float r = __builtin_amdgcn_exp2f(tiny ? t + 64.0f : t);
    return tiny ? r * 0x1p-64f : r;
}

// 1 / x on the hardware reciprocal (v_rcp_f32, ~1 ulp; subnormal results
// flush to zero, so callers keep the result normal).
__device__ inline float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// SiLU x * (1 / (1 + e^-x)) on the hardware exp2 and reciprocal.  For
// x < -44 the sigmoid can be subnormal (x < -87.3) although x * sigmoid is
// not; the denominator is then scaled by 2^-64 so the reciprocal stays
// normal, and the product is scaled back.  e^-x itself may flush to zero
// for x > 87.3, where 1 + e^-x rounds to 1 anyway.
__device__ inline float silu_fast(float x) {
    const float s = 1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896340736f);
    const bool big = s > 0x1p64f;
    const float r = rcp_fast(big ? s * 0x1p-64f : s);
    return big ? (x * r) * 0x1p-64f : x * r;
}

// Wave-wide max / sum without LDS round trips (a __shfl_xor is an LDS
// permute, ~100 cycles each): four DPP steps reduce every row of 16 lanes
// (lane ^ 1, lane ^ 2, then the mirrors within 8 and within 16 lanes pair
// the halves), and the four row results are read as scalars and combined,
// so the result is the same in every lane.
template <int CTRL>
__device__ inline float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
__device__ inline float lane_value(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ inline float row16_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
    return fmaxf(v, dpp_move<0x140>(v));  // row_mirror
}
__device__ inline float row16_sum(float v) {
    v += dpp_move<0xB1>(v);
    v += dpp_move<0x4E>(v);
    v += dpp_move<0x141>(v);
    return v + dpp_move<0x140>(v);
}
__device__ inline float wave_max_dpp(float v) {
    v = row16_max(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)),
                 fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ inline float wave_sum_dpp(float v) {
    v = row16_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
// Sum over the aligned group of TPR lanes (16, 32 or 64) a lane belongs to,
// the same in every lane of the group.
template <int TPR>
__device__ inline float lane_group_sum_dpp(float v) {
    static_assert(TPR == 16 || TPR == 32 || TPR == 64, "lane groups of 16, 32 or 64");
    v = row16_sum(v);
    if constexpr (TPR == 16) {
        return v;
    } else if constexpr (TPR == 32) {
        const float lo = lane_value(v, 0) + lane_value(v, 16);
        const float hi = lane_value(v, 32) + lane_value(v, 48);
        return (threadIdx.x & 32) ? hi : lo;
    } else {
        return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
    }
}

// wave64 butterfly reductions (every lane ends with the result).
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
    return v;
}

}  // namespace rl
