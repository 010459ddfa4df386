// elementwise.hip -- add, mul, SiLU, SwiGLU, f32<->f16 cast and row-broadcast
// add for gfx950.
//
// Every op here is a pure stream: HBM-bound, a few VALU ops per element.
// Each thread moves one 16-byte pack per operand (float4 / 8 halves; the
// casts use 8-element packs when narrowing and 4-element packs when
// widening, so the wider side is always one contiguous 16-byte access per
// lane), 256 threads per block over a full grid.  One load or store
// instruction of a wave covers 1 KiB of contiguous memory.  Loads are
// non-temporal: nothing is reused, so the data should not displace L2
// contents.  Packs per thread and the store kind are set per op (MapShape
// below); with one pack per thread a 75 MB launch reaches about 71% of peak
// and a 300 MB one 80%, non-temporal loads being worth about 8 points.  The
// few elements past the last whole pack are handled by block 0.
#include "common.hpp"

namespace rl {
namespace {

constexpr int kThreads = 256;

// ------------------------------------------------------------ element ops
// Each is the reference shader's expression, evaluated in float32.

struct AddOp {  // vector_add.metal:11,20
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct MulOp {  // mul.metal:18-19,34-35
    __device__ float operator()(float a, float b) const { return a * b; }
};
// SiLU's exp and reciprocal use the hardware instructions (silu_fast in
// common.hpp): with the IEEE-exact expf and divide (~27 VALU ops per
// element) the op is ALU-bound below HBM speed.  Error <= 3e-6 relative,
// within the 1e-5 bar for f32 and 1 ulp of f16.  The f16 kernel's
// x / (1 + e) and the f32 kernel's x * (1 / (1 + e)) are the same value up
// to that error, so both use one expression.
struct SiluF32Op {  // silu.metal:17-23: x * (1 / (1 + exp(-x)))
    __device__ float operator()(float x, float) const { return silu_fast(x); }
};
// silu.metal:31-35: x / (1 + exp(-x)), rounded to f16.  Without the scaling
// of silu_fast: where the reciprocal of 1 + e^-x would be subnormal
// (x < -87.3) it flushes to zero and the result is -0, and the exact result
// there (|x e^x| < 1e-35) also rounds to -0 in f16.  x = -inf gives NaN, as
// -inf / inf does.  Three fewer VALU operations per element make this
// f16-bandwidth kernel 8% faster.
struct SiluF16Op {
    __device__ float operator()(float x, float) const {
        return x * rcp_fast(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896340736f));
    }
};
// silu.metal:44-45: (g / (1 + exp(-g))) * u, rounded once to f16.  As in
// SiluF16Op the sigmoid is not rescaled: where it flushes to zero
// (g < -87.3) the exact |silu(g) u| is below 2^-100 for every finite half u,
// which rounds to a zero of the same sign in f16.
struct SwigluF16Op {
    __device__ float operator()(float g, float u) const {
        return (g * rcp_fast(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896340736f))) * u;
    }
};
struct SwigluF32Op {  // nn/swiglu.rs:15-37 F32 branch: silu_f32(g) then mul_f32
    __device__ float operator()(float g, float u) const { return SiluF32Op()(g, 0.0f) * u; }
};
struct CopyOp {  // cast.metal:10,18: the conversion happens on store/load
    __device__ float operator()(float x, float) const { return x; }
};

// Launch shape of each op: 16-byte packs per thread and the store kind.
// Measured on [4096, 1536] ([4096, 2560] for f16 SwiGLU) over 128-1024
// threads per block x 1, 2, 4 packs per thread x non-temporal / plain
// stores, two boxes agreeing within 1.5 points: about four loads in flight
// per thread pays where the math is light (f16 add 62% -> 69% of HBM peak,
// f16 -> f32 cast 62% -> 71%, f32 SiLU 67% -> 72%), while the exp/rcp-heavy
// f16 SwiGLU is best at one pack per thread.
template <typename Op, typename TIn, typename TOut>
struct MapShape {
    static constexpr int unroll = 1;
    static constexpr bool nt_store = true;
    static constexpr bool phased = false;  // see k_map
};

template <typename TIn, typename TOut>
struct MapShape<AddOp, TIn, TOut> {  // f32: 72% -> 74%, f16: 62% -> 66-69%
    static constexpr int unroll = sizeof(TIn) == 4 ? 4 : 2;
    static constexpr bool phased = false;
    static constexpr bool nt_store = false;
};
template <typename TIn, typename TOut>
struct MapShape<MulOp, TIn, TOut> {
    static constexpr int unroll = sizeof(TIn) == 4 ? 4 : 2;
    static constexpr bool phased = false;
    static constexpr bool nt_store = false;
};
template <typename TIn, typename TOut>
struct MapShape<SwigluF32Op, TIn, TOut> {  // 70% -> 73%
    static constexpr int unroll = 4;
    static constexpr bool phased = false;
    static constexpr bool nt_store = false;
};
template <typename TIn, typename TOut>
struct MapShape<SiluF32Op, TIn, TOut> {
    static constexpr int unroll = 4;
    static constexpr bool phased = false;
    static constexpr bool nt_store = true;
};
template <typename TIn, typename TOut>
struct MapShape<SiluF16Op, TIn, TOut> {  // phased: 5.8 -> 5.1 us on [4096, 1536]
    static constexpr int unroll = 2;
    static constexpr bool phased = true;
    static constexpr bool nt_store = true;
};
template <>
struct MapShape<CopyOp, half_t, float> {  // widening cast: 8-byte loads
    static constexpr int unroll = 4;
    static constexpr bool phased = false;
    static constexpr bool nt_store = true;
};
template <>
struct MapShape<CopyOp, float, half_t> {
    static constexpr int unroll = 2;
    static constexpr bool phased = false;
    static constexpr bool nt_store = false;
};

// out[i] = op(a[i], b[i]) for ARITY 2, op(a[i]) for ARITY 1.  Block b covers
// packs [b * 256 * UNROLL, (b + 1) * 256 * UNROLL): the grid spans the whole
// array (at most 2^32 elements, so at most 2^22 blocks), with no loop.
template <typename TIn, typename TOut, int N, int UNROLL, int ARITY, bool NTS, bool PHASED,
          typename Op>
__global__ __launch_bounds__(kThreads) void k_map(const TIn* __restrict__ a,
                                                  const TIn* __restrict__ b,
                                                  TOut* __restrict__ out, uint64_t n_packs,
                                                  uint32_t tail, Op op) {
    typedef typename VecOf<TIn, N>::type VI;
    typedef typename VecOf<TOut, N>::type VO;
    const VI* va = reinterpret_cast<const VI*>(a);
    const VI* vb = reinterpret_cast<const VI*>(b);
    VO* vo = reinterpret_cast<VO*>(out);
    const uint64_t base = uint64_t(blockIdx.x) * kThreads * UNROLL + threadIdx.x;
    if constexpr (PHASED) {
        // Three phases: every pack's loads (at indices clamped into the
        // array), every result, then every store (a clamped pack rewrites the
        // last pack's own value).  With per-pack branches the compiler issued
        // pack u + 1's loads only after pack u's store.
        if (n_packs > 0) {
            VI ra[UNROLL], rb[UNROLL];
            VO r[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint64_t i = base + uint64_t(u) * kThreads;
                const uint64_t ic = i < n_packs ? i : n_packs - 1;
                ra[u] = load_stream(va + ic);
                if constexpr (ARITY == 2) rb[u] = load_stream(vb + ic);
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
#pragma unroll
                for (int k = 0; k < N; ++k) {
                    float y = 0.0f;
                    if constexpr (ARITY == 2) y = to_float(rb[u][k]);
                    r[u][k] = from_float<TOut>(op(to_float(ra[u][k]), y));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint64_t i = base + uint64_t(u) * kThreads;
                const uint64_t ic = i < n_packs ? i : n_packs - 1;
                if constexpr (NTS)
                    store_stream(vo + ic, r[u]);
                else
                    vo[ic] = r[u];
            }
        }
    } else {
        VI ra[UNROLL], rb[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_packs) {
                ra[u] = load_stream(va + i);
                if constexpr (ARITY == 2) rb[u] = load_stream(vb + i);
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_packs) {
                VO r;
#pragma unroll
                for (int k = 0; k < N; ++k) {
                    float x = to_float(ra[u][k]);
                    float y = 0.0f;
                    if constexpr (ARITY == 2) y = to_float(rb[u][k]);
                    r[k] = from_float<TOut>(op(x, y));
                }
                if constexpr (NTS)
                    store_stream(vo + i, r);
                else
                    vo[i] = r;
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < tail) {
        uint64_t i = n_packs * N + threadIdx.x;
        float y = 0.0f;
        if constexpr (ARITY == 2) y = to_float(b[i]);
        out[i] = from_float<TOut>(op(to_float(a[i]), y));
    }
}

// out[r, c] = x[r, c] + bias[c] on packs; col_packs = cols / N.
template <typename T, int N, int UNROLL>
__global__ __launch_bounds__(kThreads) void k_add_broadcast(const T* __restrict__ x,
                                                            const T* __restrict__ bias,
                                                            T* __restrict__ out,
                                                            uint64_t n_packs, FastDiv col_packs) {
    typedef typename VecOf<T, N>::type V;
    const V* vx = reinterpret_cast<const V*>(x);
    const V* vbias = reinterpret_cast<const V*>(bias);
    V* vo = reinterpret_cast<V*>(out);
    const uint64_t tile = uint64_t(kThreads) * UNROLL;
    const uint64_t step = uint64_t(gridDim.x) * tile;
    for (uint64_t base = uint64_t(blockIdx.x) * tile + threadIdx.x; base < n_packs;
         base += step) {
        V rx[UNROLL], rb[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_packs) {
                uint32_t row, col;
                col_packs.divmod(uint32_t(i), row, col);
                rx[u] = load_stream(vx + i);
                rb[u] = vbias[col];  // a few KiB, stays in L2
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_packs) {
                V r;
#pragma unroll
                for (int k = 0; k < N; ++k)
                    r[k] = from_float<T>(to_float(rx[u][k]) + to_float(rb[u][k]));
                store_stream(vo + i, r);
            }
        }
    }
}

// out[r, c] = x[r, c] + bias[c] for rows of at most 1024 packs: thread t of
// a block owns column pack t -- its bias pack is loaded once and kept in
// registers -- and adds it to that pack of R consecutive rows (R loads in
// flight per thread, no index division, no bias reloads).  Consecutive
// threads read consecutive packs of a row.
template <typename T, int N, int R>
__global__ __launch_bounds__(1024) void k_add_bias_rows(const T* __restrict__ x,
                                                        const T* __restrict__ bias,
                                                        T* __restrict__ out, uint32_t rows,
                                                        uint32_t col_packs) {
    typedef typename VecOf<T, N>::type V;
    const uint32_t c = threadIdx.x;
    if (c >= col_packs) return;
    const V* vx = reinterpret_cast<const V*>(x);
    V* vo = reinterpret_cast<V*>(out);
    const V b = reinterpret_cast<const V*>(bias)[c];
    const uint32_t r0 = blockIdx.x * R;
    V rx[R];
#pragma unroll
    for (int u = 0; u < R; ++u)
        if (r0 + u < rows) rx[u] = load_stream(vx + uint64_t(r0 + u) * col_packs + c);
#pragma unroll
    for (int u = 0; u < R; ++u) {
        if (r0 + u < rows) {
            V r;
#pragma unroll
            for (int k = 0; k < N; ++k) r[k] = from_float<T>(to_float(rx[u][k]) + to_float(b[k]));
            store_stream(vo + uint64_t(r0 + u) * col_packs + c, r);
        }
    }
}

// Scalar fallback for buffers that are not pack-aligned or too large for
// 32-bit pack indices.
template <typename T>
__global__ __launch_bounds__(kThreads) void k_add_broadcast_scalar(const T* __restrict__ x,
                                                                   const T* __restrict__ bias,
                                                                   T* __restrict__ out,
                                                                   uint64_t n, uint64_t cols) {
    const uint64_t step = uint64_t(gridDim.x) * kThreads;
    for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += step)
        out[i] = from_float<T>(to_float(x[i]) + to_float(bias[i % cols]));
}

// Blocks for a grid-stride stream over `items` work items of `per_block` each.
inline unsigned grid_for(uint64_t items, uint64_t per_block) {
    uint64_t blocks = ceil_div(items, per_block);
    if (blocks < 1) blocks = 1;
    if (blocks > (1u << 30)) blocks = 1u << 30;
    return unsigned(blocks);
}

template <typename TIn, typename TOut, int ARITY, typename Op>
rl_status launch_map(rl_context* ctx, const char* name, const void* a, const void* b, void* out,
                     uint64_t n, Op op) {
    if (n == 0) return RL_OK;
    if (rl_status st = activate(ctx)) return st;
    // 16-byte packs; the widening cast uses 4-element packs so its stores
    // stay 16 B per lane and contiguous across the wave (8-element f32 packs
    // would be two strided 16-byte stores, which costs extra HBM writes).
    constexpr int N = (sizeof(TIn) == 4 && sizeof(TOut) == 4) ? 4 : (sizeof(TOut) == 4 ? 4 : 8);
    constexpr int UNROLL = MapShape<Op, TIn, TOut>::unroll;
    constexpr bool NTS = MapShape<Op, TIn, TOut>::nt_store;
    constexpr bool PHASED = MapShape<Op, TIn, TOut>::phased;
    const bool vec = aligned_to(a, N * sizeof(TIn)) &&
                     (ARITY < 2 || aligned_to(b, N * sizeof(TIn))) &&
                     aligned_to(out, N * sizeof(TOut));
    const TIn* pa = static_cast<const TIn*>(a);
    const TIn* pb = static_cast<const TIn*>(b);
    TOut* po = static_cast<TOut*>(out);
    // The kernel has no grid-stride loop: the grid must cover every pack.
    if (ceil_div(n, uint64_t(kThreads) * UNROLL) > (1u << 30))
        return fail(RL_ERR_INVALID_SHAPE, "%s: %llu elements exceed one launch", name,
                    (unsigned long long)n);
    if (vec) {
        uint64_t n_packs = n / N;
        uint32_t tail = uint32_t(n - n_packs * N);
        RL_LAUNCH(ctx, (k_map<TIn, TOut, N, UNROLL, ARITY, NTS, PHASED, Op>), dim3(grid_for(n_packs, uint64_t(kThreads) * UNROLL)), dim3(kThreads), pa, pb, po, n_packs, tail, op);
    } else {
        RL_LAUNCH(ctx, (k_map<TIn, TOut, 1, UNROLL, ARITY, NTS, PHASED, Op>), dim3(grid_for(n, uint64_t(kThreads) * UNROLL)), dim3(kThreads), pa, pb, po, n, 0u, op);
    }
    return after_launch(ctx, name);
}

template <typename T>
rl_status launch_add_broadcast(rl_context* ctx, const char* name, const rl_buffer* x,
                               const rl_buffer* bias, uint64_t rows, uint64_t cols,
                               const rl_buffer* out) {
    uint64_t n = rows * cols;
    if (n == 0) return RL_OK;
    if (rl_status st = activate(ctx)) return st;
    constexpr int N = 16 / sizeof(T);
    // Four packs per thread: f16 53% -> 56% of peak on [4096, 1536] (same
    // sweep as MapShape).
    constexpr int UNROLL = 4;
    const T* px = static_cast<const T*>(x->data);
    const T* pbias = static_cast<const T*>(bias->data);
    T* po = static_cast<T*>(out->data);
    const bool vec = cols % N == 0 && aligned_to(px, 16) && aligned_to(pbias, 16) &&
                     aligned_to(po, 16) && n / N <= UINT32_MAX;
    const uint64_t col_packs = cols / N;
    if (vec && sizeof(T) == 4 && col_packs <= 1024 && rows <= UINT32_MAX) {
        // f32 rows of up to 1024 packs: a block per 8 rows, a thread per
        // column pack (threads rounded up to whole waves).  [4096, 1536]:
        // 8.7 us (72% of peak) against 10.2 us for the per-pack column
        // division below (4 rows per block: 9.4 us, 2: 10.4 us).  f16 rows
        // (half the bytes per row) measured no gain (5.4-6.7 us against
        // 5.2-5.9 us) and keep that kernel.
        constexpr int R = 8;
        const unsigned threads = unsigned(ceil_div(col_packs, 64) * 64);
        RL_LAUNCH(ctx, (k_add_bias_rows<T, N, R>), dim3(unsigned(ceil_div(rows, R))),
                  dim3(threads), px, pbias, po, uint32_t(rows), uint32_t(col_packs));
    } else if (vec) {
        uint64_t n_packs = n / N;
        RL_LAUNCH(ctx, (k_add_broadcast<T, N, UNROLL>), dim3(grid_for(n_packs, uint64_t(kThreads) * UNROLL)), dim3(kThreads), px, pbias, po, n_packs, FastDiv(uint32_t(cols / N)));
    } else {
        RL_LAUNCH(ctx, (k_add_broadcast_scalar<T>), dim3(grid_for(n, kThreads * 4)), dim3(kThreads), px, pbias, po, n, cols);
    }
    return after_launch(ctx, name);
}

rl_status check_input(const rl_buffer* b, uint64_t element_size, const char* what) {
    if (rl_status st = check_buffer(b, what)) return st;
    if (b->byte_len < b->len * element_size)
        return fail(RL_ERR_INVALID_SHAPE,
                    "%s buffer holds %llu bytes, fewer than %llu elements of %llu bytes", what,
                    (unsigned long long)b->byte_len, (unsigned long long)b->len,
                    (unsigned long long)element_size);
    return RL_OK;
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

// src/ops/add.rs:18-49
rl_status rl_add_f32(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out) {
    if (rl_status st = check_input(a, 4, "left")) return st;
    if (rl_status st = check_input(b, 4, "right")) return st;
    if (a->len != b->len)
        return fail(RL_ERR_INVALID_SHAPE, "add requires equal buffer lengths, got %llu and %llu",
                    (unsigned long long)a->len, (unsigned long long)b->len);
    if (rl_status st = check_output(out, a->len, 4, "add")) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<float, float, 2>(ctx, "add_f32", a->data, b->data, out->data, a->len,
                                       AddOp{});
}

// src/ops/add.rs:61-101
rl_status rl_add_f16(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out) {
    if (rl_status st = check_buffer(a, "left")) return st;
    if (rl_status st = check_buffer(b, "right")) return st;
    if (a->len != b->len || a->byte_len != a->len * 2 || b->byte_len != b->len * 2)
        return fail(RL_ERR_INVALID_SHAPE,
                    "F16 add requires equal F16 buffers, got %llu elements/%llu bytes and %llu "
                    "elements/%llu bytes",
                    (unsigned long long)a->len, (unsigned long long)a->byte_len,
                    (unsigned long long)b->len, (unsigned long long)b->byte_len);
    if (rl_status st = check_output(out, a->len, 2, "add")) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<half_t, half_t, 2>(ctx, "add_f16", a->data, b->data, out->data, a->len,
                                         AddOp{});
}

// src/ops/mul.rs:20-68
rl_status rl_mul_f32(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out) {
    if (rl_status st = check_input(a, 4, "left")) return st;
    if (rl_status st = check_input(b, 4, "right")) return st;
    if (a->len != b->len)
        return fail(RL_ERR_INVALID_SHAPE,
                    "element-wise multiply requires equal buffer lengths, got %llu and %llu",
                    (unsigned long long)a->len, (unsigned long long)b->len);
    if (rl_status st = check_output(out, a->len, 4, "multiply")) return st;
    if (a->len > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "multiply input size exceeds u32");
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<float, float, 2>(ctx, "mul_f32", a->data, b->data, out->data, a->len,
                                       MulOp{});
}

// src/ops/mul.rs:80-119
rl_status rl_mul_f16(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out) {
    if (rl_status st = check_input(a, 2, "left")) return st;
    if (rl_status st = check_input(b, 2, "right")) return st;
    if (a->len != b->len)
        return fail(RL_ERR_INVALID_SHAPE,
                    "element-wise multiply requires equal buffer lengths, got %llu and %llu",
                    (unsigned long long)a->len, (unsigned long long)b->len);
    if (rl_status st = check_output(out, a->len, 2, "multiply")) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<half_t, half_t, 2>(ctx, "mul_f16", a->data, b->data, out->data, a->len,
                                         MulOp{});
}

// src/ops/silu.rs:20-63
rl_status rl_silu_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* out) {
    if (rl_status st = check_input(input, 4, "input")) return st;
    if (input->len == 0) return fail(RL_ERR_INVALID_SHAPE, "SiLU input cannot be empty");
    if (rl_status st = check_output(out, input->len, 4, "SiLU")) return st;
    if (input->len > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "SiLU input size exceeds u32");
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<float, float, 1>(ctx, "silu_f32", input->data, nullptr, out->data,
                                       input->len, SiluF32Op{});
}

// src/ops/silu.rs:75-109
rl_status rl_silu_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* out) {
    if (rl_status st = check_input(input, 2, "input")) return st;
    if (input->len == 0) return fail(RL_ERR_INVALID_SHAPE, "SiLU input cannot be empty");
    if (rl_status st = check_output(out, input->len, 2, "SiLU")) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<half_t, half_t, 1>(ctx, "silu_f16", input->data, nullptr, out->data,
                                         input->len, SiluF16Op{});
}

// src/ops/swiglu.rs:8-34
rl_status rl_swiglu_f16(rl_context* ctx, const rl_buffer* gate, const rl_buffer* up,
                        const rl_buffer* out) {
    if (rl_status st = check_buffer(gate, "gate")) return st;
    if (rl_status st = check_buffer(up, "up")) return st;
    if (gate->len != up->len || gate->byte_len != gate->len * 2 || up->byte_len != up->len * 2)
        return fail(RL_ERR_INVALID_SHAPE, "SwiGLU requires equal F16 buffers");
    if (rl_status st = check_output(out, gate->len, 2, "SwiGLU")) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<half_t, half_t, 2>(ctx, "swiglu_f16", gate->data, up->data, out->data,
                                         gate->len, SwigluF16Op{});
}

// src/nn/swiglu.rs:15-37 (F32: silu_f32 then mul_f32, fused)
rl_status rl_swiglu_f32(rl_context* ctx, const rl_buffer* gate, const rl_buffer* up,
                        const rl_buffer* out) {
    if (rl_status st = check_buffer(gate, "gate")) return st;
    if (rl_status st = check_buffer(up, "up")) return st;
    if (gate->len != up->len || gate->byte_len != gate->len * 4 || up->byte_len != up->len * 4)
        return fail(RL_ERR_INVALID_SHAPE, "SwiGLU requires equal F32 buffers");
    if (gate->len == 0) return fail(RL_ERR_INVALID_SHAPE, "SiLU input cannot be empty");
    if (rl_status st = check_output(out, gate->len, 4, "SwiGLU")) return st;
    if (gate->len > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "SiLU input size exceeds u32");
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<float, float, 2>(ctx, "swiglu_f32", gate->data, up->data, out->data,
                                       gate->len, SwigluF32Op{});
}

// src/ops/cast.rs:28-83
rl_status rl_cast_f32_to_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* out) {
    if (rl_status st = check_input(input, 4, "input")) return st;
    if (rl_status st = check_output(out, input->len, 2, "cast")) return st;
    if (input->len > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "cast element count exceeds u32");
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<float, half_t, 1>(ctx, "cast_f32_to_f16", input->data, nullptr, out->data,
                                        input->len, CopyOp{});
}

rl_status rl_cast_f16_to_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* out) {
    if (rl_status st = check_input(input, 2, "input")) return st;
    if (rl_status st = check_output(out, input->len, 4, "cast")) return st;
    if (input->len > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "cast element count exceeds u32");
    if (rl_status st = require_context(ctx)) return st;
    return launch_map<half_t, float, 1>(ctx, "cast_f16_to_f32", input->data, nullptr, out->data,
                                        input->len, CopyOp{});
}

static rl_status validate_broadcast(const rl_buffer* x, const rl_buffer* bias, uint64_t rows,
                                    uint64_t cols, const rl_buffer* out, uint64_t es) {
    if (rl_status st = check_input(x, es, "input")) return st;
    if (rl_status st = check_input(bias, es, "bias")) return st;
    if (rows == 0 || cols == 0)
        return fail(RL_ERR_INVALID_SHAPE, "shape dimensions must be greater than zero");
    if (rows > UINT64_MAX / cols || x->len != rows * cols)
        return fail(RL_ERR_INVALID_SHAPE, "input has %llu elements, expected %llu x %llu",
                    (unsigned long long)x->len, (unsigned long long)rows,
                    (unsigned long long)cols);
    if (bias->len != cols) {  // [rows, cols] + [bias len]: the shapes the add would see
        const uint64_t left[2] = {rows, cols}, right[1] = {bias->len};
        return fail_shape_mismatch(left, 2, right, 1);
    }
    return check_output(out, x->len, es, "add");
}

rl_status rl_add_broadcast_f32(rl_context* ctx, const rl_buffer* x, const rl_buffer* bias,
                               uint64_t rows, uint64_t cols, const rl_buffer* out) {
    if (rl_status st = validate_broadcast(x, bias, rows, cols, out, 4)) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_add_broadcast<float>(ctx, "add_broadcast_f32", x, bias, rows, cols, out);
}

rl_status rl_add_broadcast_f16(rl_context* ctx, const rl_buffer* x, const rl_buffer* bias,
                               uint64_t rows, uint64_t cols, const rl_buffer* out) {
    if (rl_status st = validate_broadcast(x, bias, rows, cols, out, 2)) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_add_broadcast<half_t>(ctx, "add_broadcast_f16", x, bias, rows, cols, out);
}

}  // extern "C"
