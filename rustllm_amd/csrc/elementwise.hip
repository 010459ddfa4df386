// elementwise.hip -- add, mul, SiLU, SwiGLU, f32<->f16 cast and row-broadcast
// add for gfx950.
//
// Every op here is a pure stream: HBM-bound, a few VALU ops per element.
// Each thread moves one 16-byte pack per operand (float4 / 8 halves; both
// casts use 4-element packs, so the f32 side is always one contiguous
// 16-byte access per lane), 256 threads per block over a full grid.  One load or store
// instruction of a wave covers 1 KiB of contiguous memory.  Loads are
// non-temporal: nothing is reused, so the data should not displace L2
// contents.  Packs per thread and the store kind are set per op (MapShape
// below); with one pack per thread a 75 MB launch reaches about 71% of peak
// and a 300 MB one 80%, non-temporal loads being worth about 8 points.  The
// few elements past the last whole pack are handled by block 0.
#include "common.hpp"
#include "movement_bodies.hpp"

#include <type_traits>

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
// f16-bandwidth kernel 8% faster.  Taking the half x unconverted in both
// products (v_fma_mix_f32, two instructions fewer per element, the same
// results bit for bit) measured no faster ([4096, 1536]: 5.91 against 5.89
// us back to back): the time goes to the exp -> add -> rcp latency, not to
// the instruction count.
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
// stores, two MI355X hosts agreeing within 1.5 points: about four loads in flight
// per thread pays where the math is light (f16 add 62% -> 69% of HBM peak,
// f16 -> f32 cast 62% -> 71%, f32 SiLU 67% -> 72%), while the exp/rcp-heavy
// f16 SwiGLU is best at one pack per thread (below 2^20 packs: MapShapeBig).
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
// Phased (loads, results, stores), four packs a thread: one MI355X, back to
// back, [4096, 1536] 5.84 us at two packs -> 5.55 us (eight: 7.0), [4096,
// 2560] 9.16 -> 8.45 us; storing each pack as soon as it is computed is no
// faster (5.85 at two, 5.44 at four).
template <typename TIn, typename TOut>
struct MapShape<SiluF16Op, TIn, TOut> {
    static constexpr int unroll = 4;
    static constexpr bool phased = true;
    static constexpr bool nt_store = true;
};
// A second launch shape for the large launches of an op, from `from_packs`
// packs on (0: none).  f16 SwiGLU, one MI355X, back to back over 16 rotated
// buffer sets, bit-identical: [4096, 2560] (1,310,720 packs) 12.0 us at one
// pack a thread -> 11.4-11.55 us phased at four packs with plain stores
// (three: 11.8-12.0, six: 12.6, eight: 12.3-12.5; four with streamed stores:
// 12.2-12.3); [4096, 1536] (786,432 packs) 8.1 -> 8.1-8.3 us, so the
// one-pack shape stays below 2^20 packs.
template <typename Op, typename TIn, typename TOut>
struct MapShapeBig {
    static constexpr uint64_t from_packs = 0;
    static constexpr int unroll = 1;
    static constexpr bool nt_store = true;
    static constexpr bool phased = false;
};
template <>
struct MapShapeBig<SwigluF16Op, half_t, half_t> {
    static constexpr uint64_t from_packs = uint64_t(1) << 20;
    static constexpr int unroll = 4;
    static constexpr bool nt_store = false;
    static constexpr bool phased = true;
};
template <>
struct MapShape<CopyOp, half_t, float> {  // widening cast: 8-byte loads
    static constexpr int unroll = 4;
    static constexpr bool phased = false;
    static constexpr bool nt_store = true;
};
// Narrowing cast: packs of 4 (16-byte loads, 8-byte stores), four a thread,
// streamed stores.  With packs of 8 each 16-byte load instruction covers
// every other 16 bytes of 2 KB (a lane's 32 bytes come in two loads);
// [4096, 1536] back to back: 7.9 us (8 a pack, 2 a thread, plain stores)
// -> 7.2 us.
template <>
struct MapShape<CopyOp, float, half_t> {
    static constexpr int unroll = 4;
    static constexpr bool phased = false;
    static constexpr bool nt_store = true;
};

// Launch shape of a map inside the fused launch of recorded ops (below):
// two packs per thread and non-temporal stores for every op.  With 16 ops
// streaming side by side the shapes tuned for one op alone lose; on the
// [4096, 1536] batch of 16 ops one fused launch took 109.3 us with them,
// 103.3 us with non-temporal stores for all, and 95.7 us with two packs per
// thread for every map and one for the bias add (kFusedBiasUnroll; one pack
// for the maps: 97.7 us, four: 97.7 us).
template <typename Op, typename TIn, typename TOut>
struct FusedShape {
    static constexpr int unroll = 2;
    static constexpr bool nt_store = true;
    static constexpr bool phased = MapShape<Op, TIn, TOut>::phased;
};

// Pack size of a map: 16-byte packs; both casts use 4-element packs, so
// that the f32 side moves 16 B per lane contiguous across the wave (with
// 8-element packs a lane's 32 f32 bytes would be two 16-byte accesses each
// covering every other 16 bytes of the wave's span: for the widening cast
// extra HBM writes, for the narrowing one 9% more time).
template <typename TIn, typename TOut>
constexpr int map_pack() {
    return (sizeof(TIn) == 4 || sizeof(TOut) == 4) ? 4 : 8;
}

// out[i] = op(a[i], b[i]) for ARITY 2, op(a[i]) for ARITY 1.  Block blk covers
// packs [blk * 256 * UNROLL, (blk + 1) * 256 * UNROLL): the grid spans the
// whole array (at most 2^32 elements, so at most 2^22 blocks), with no loop.
template <typename TIn, typename TOut, int N, int UNROLL, int ARITY, bool NTS, bool PHASED,
          typename Op>
__device__ inline void map_body(const TIn* __restrict__ a, const TIn* __restrict__ b,
                                TOut* __restrict__ out, uint64_t n_packs, uint32_t tail, Op op,
                                uint32_t blk) {
    typedef typename VecOf<TIn, N>::type VI;
    typedef typename VecOf<TOut, N>::type VO;
    const VI* va = reinterpret_cast<const VI*>(a);
    const VI* vb = reinterpret_cast<const VI*>(b);
    VO* vo = reinterpret_cast<VO*>(out);
    const uint64_t base = uint64_t(blk) * kThreads * UNROLL + threadIdx.x;
    if constexpr (PHASED) {
        // Three phases: every pack's loads (at indices clamped into the
        // array, so no load waits on a branch), every result, then the
        // stores of the packs that are this lane's own.  A clamped lane
        // stores nothing: with out == a (in place) the last pack may already
        // hold its owner's result when a clamped lane reads it.  With
        // per-pack branches around the loads the compiler issued pack
        // u + 1's loads only after pack u's store.
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
                if (i >= n_packs) continue;
                if constexpr (NTS)
                    store_stream(vo + i, r[u]);
                else
                    vo[i] = r[u];
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
    if (blk == 0 && threadIdx.x < tail) {
        uint64_t i = n_packs * N + threadIdx.x;
        float y = 0.0f;
        if constexpr (ARITY == 2) y = to_float(b[i]);
        out[i] = from_float<TOut>(op(to_float(a[i]), y));
    }
}

template <typename TIn, typename TOut, int N, int UNROLL, int ARITY, bool NTS, bool PHASED,
          typename Op>
__global__ __launch_bounds__(kThreads) void k_map(const TIn* __restrict__ a,
                                                  const TIn* __restrict__ b,
                                                  TOut* __restrict__ out, uint64_t n_packs,
                                                  uint32_t tail, Op op) {
    map_body<TIn, TOut, N, UNROLL, ARITY, NTS, PHASED, Op>(a, b, out, n_packs, tail, op,
                                                            blockIdx.x);
}

// out[r, c] = x[r, c] + bias[c] on packs; col_packs = cols / N.  Block blk
// of nblk strides over the packs.
template <typename T, int N, int UNROLL>
__device__ inline void broadcast_body(const T* __restrict__ x, const T* __restrict__ bias,
                                      T* __restrict__ out, uint64_t n_packs, FastDiv col_packs,
                                      uint32_t blk, uint32_t nblk) {
    typedef typename VecOf<T, N>::type V;
    const V* vx = reinterpret_cast<const V*>(x);
    const V* vbias = reinterpret_cast<const V*>(bias);
    V* vo = reinterpret_cast<V*>(out);
    const uint64_t tile = uint64_t(kThreads) * UNROLL;
    const uint64_t step = uint64_t(nblk) * tile;
    for (uint64_t base = uint64_t(blk) * tile + threadIdx.x; base < n_packs; base += step) {
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

template <typename T, int N, int UNROLL>
__global__ __launch_bounds__(kThreads) void k_add_broadcast(const T* __restrict__ x,
                                                            const T* __restrict__ bias,
                                                            T* __restrict__ out,
                                                            uint64_t n_packs, FastDiv col_packs) {
    broadcast_body<T, N, UNROLL>(x, bias, out, n_packs, col_packs, blockIdx.x, gridDim.x);
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

// ----------------------------------------------- streaming ops in one launch

// While a graph is recorded, the maps and bias adds below and the row
// gathers and repeat_kv of movement.hip are not launched one by one: runs of
// them that touch disjoint bytes (or only read the same bytes) are recorded
// as one kernel whose blocks are split among the ops,
// each op's blocks running that op's body on its own share of the grid.
// Successive kernels of one stream run one after another here, each with a
// ramp-up and a drain of ~1.5-2 us; one kernel for a batch of independent
// ops (the reference's ops encoded into one command buffer, which the GPU
// may overlap) streams them as one.  Each op computes exactly what its own
// launch computes (the same body and pack width; only the packs per thread
// and the store kind follow FusedShape).
typedef OuterDimsT<kMaxFusedOuterRank, uint32_t> FusedDims;

struct FusedSeg {
    uint32_t kind;
    uint32_t tail;  // map
    const void* a;
    const void* b;
    void* out;
    uint64_t n_packs;
    uint64_t head_packs;  // repeat_kv
    FastDiv div;          // packs per row (bias add, row gather) or per head (repeat_kv)
    uint32_t repeats;     // repeat_kv
    uint32_t small_index;
    FusedDims outer;      // row gather / scatter
};
struct FusedTable {
    uint32_t first[kMaxFused];  // each op's first block in the fused grid (ascending)
    uint32_t count;
    FusedSeg seg[kMaxFused];
};

constexpr int kBroadcastUnroll = 4;  // packs per thread of the bias add
constexpr int kFusedBiasUnroll = 1;  // the same inside the fused launch (FusedShape)

// The fused kind of a map (0: launched on its own).
template <typename TIn, typename TOut, typename Op>
constexpr uint32_t fused_kind() {
    constexpr bool f32 = sizeof(TIn) == 4 && sizeof(TOut) == 4;
    constexpr bool f16 = sizeof(TIn) == 2 && sizeof(TOut) == 2;
    if constexpr (std::is_same<Op, AddOp>::value) return f32 ? kFusedAddF32 : f16 ? kFusedAddF16 : 0;
    if constexpr (std::is_same<Op, MulOp>::value) return f32 ? kFusedMulF32 : f16 ? kFusedMulF16 : 0;
    if constexpr (std::is_same<Op, SiluF32Op>::value) return f32 ? kFusedSiluF32 : 0;
    if constexpr (std::is_same<Op, SiluF16Op>::value) return f16 ? kFusedSiluF16 : 0;
    if constexpr (std::is_same<Op, SwigluF32Op>::value) return f32 ? kFusedSwigluF32 : 0;
    if constexpr (std::is_same<Op, SwigluF16Op>::value) return f16 ? kFusedSwigluF16 : 0;
    if constexpr (std::is_same<Op, CopyOp>::value)
        return sizeof(TIn) == 4 && sizeof(TOut) == 2   ? kFusedCastF32F16
               : sizeof(TIn) == 2 && sizeof(TOut) == 4 ? kFusedCastF16F32
                                                       : 0;
    return 0;
}

template <typename TIn, typename TOut, int ARITY, typename Op>
__device__ inline void fused_map(const FusedSeg& s, uint32_t blk) {
    typedef FusedShape<Op, TIn, TOut> M;
    map_body<TIn, TOut, map_pack<TIn, TOut>(), M::unroll, ARITY, M::nt_store, M::phased, Op>(
        static_cast<const TIn*>(s.a), static_cast<const TIn*>(s.b), static_cast<TOut*>(s.out),
        s.n_packs, s.tail, Op{}, blk);
}

template <typename T>
__device__ inline void fused_bias(const FusedSeg& s, uint32_t blk, uint32_t nblk) {
    broadcast_body<T, 16 / sizeof(T), kFusedBiasUnroll>(
        static_cast<const T*>(s.a), static_cast<const T*>(s.b), static_cast<T*>(s.out),
        s.n_packs, s.div, blk, nblk);
}

constexpr int kMoveUnroll = 2;  // packs per thread of the row gather and repeat_kv

template <typename T>
__device__ inline void fused_gather(const FusedSeg& s, uint32_t blk, uint32_t nblk) {
    gather_rows_body<T, 16 / sizeof(T), kMoveUnroll>(static_cast<const T*>(s.a),
                                                     static_cast<T*>(s.out), uint32_t(s.n_packs),
                                                     s.div, s.outer, blk, nblk);
}

template <typename T>
__device__ inline void fused_scatter(const FusedSeg& s, uint32_t blk, uint32_t nblk) {
    scatter_rows_body<T, 16 / sizeof(T), kMoveUnroll, sizeof(T) == 2>(
        static_cast<const T*>(s.a), static_cast<T*>(s.out), uint32_t(s.n_packs), s.div, s.outer,
        blk, nblk);
}

template <typename T>
__device__ inline void fused_repeat(const FusedSeg& s, uint32_t blk, uint32_t nblk) {
    repeat_kv_body<T, 16 / sizeof(T), kMoveUnroll>(static_cast<const T*>(s.a),
                                                   static_cast<T*>(s.out), s.n_packs, s.head_packs,
                                                   s.div, s.repeats, s.small_index != 0, blk, nblk);
}

__global__ __launch_bounds__(kThreads) void k_fused(FusedTable t) {
    // the op of this block: the last whose first block is not past it (the
    // firsts are read at once and compared, no dependent loads)
    uint32_t i = 0;
#pragma unroll
    for (uint32_t j = 1; j < kMaxFused; ++j) i += (j < t.count && blockIdx.x >= t.first[j]) ? 1u : 0u;
    const FusedSeg& s = t.seg[i];  // read in place from the kernel arguments
    const uint32_t first = t.first[i];
    const uint32_t blk = blockIdx.x - first;
    const uint32_t nblk = (i + 1 < t.count ? t.first[i + 1] : gridDim.x) - first;
    switch (s.kind) {
        case kFusedAddF32: fused_map<float, float, 2, AddOp>(s, blk); break;
        case kFusedMulF32: fused_map<float, float, 2, MulOp>(s, blk); break;
        case kFusedSiluF32: fused_map<float, float, 1, SiluF32Op>(s, blk); break;
        case kFusedSwigluF32: fused_map<float, float, 2, SwigluF32Op>(s, blk); break;
        case kFusedAddF16: fused_map<half_t, half_t, 2, AddOp>(s, blk); break;
        case kFusedMulF16: fused_map<half_t, half_t, 2, MulOp>(s, blk); break;
        case kFusedSiluF16: fused_map<half_t, half_t, 1, SiluF16Op>(s, blk); break;
        case kFusedSwigluF16: fused_map<half_t, half_t, 2, SwigluF16Op>(s, blk); break;
        case kFusedCastF32F16: fused_map<float, half_t, 1, CopyOp>(s, blk); break;
        case kFusedCastF16F32: fused_map<half_t, float, 1, CopyOp>(s, blk); break;
        case kFusedBiasF32: fused_bias<float>(s, blk, nblk); break;
        case kFusedBiasF16: fused_bias<half_t>(s, blk, nblk); break;
        case kFusedGatherF32: fused_gather<float>(s, blk, nblk); break;
        case kFusedGatherF16: fused_gather<half_t>(s, blk, nblk); break;
        case kFusedRepeatF32: fused_repeat<float>(s, blk, nblk); break;
        case kFusedRepeatF16: fused_repeat<half_t>(s, blk, nblk); break;
        case kFusedScatterF32: fused_scatter<float>(s, blk, nblk); break;
        case kFusedScatterF16: fused_scatter<half_t>(s, blk, nblk); break;
        default: break;
    }
}

inline bool overlaps(const uintptr_t (&r)[2], uintptr_t begin, uintptr_t end) {
    return r[0] < end && begin < r[1];
}

template <typename TIn, typename TOut, int ARITY, typename Op>
rl_status launch_map(rl_context* ctx, const char* name, const void* a, const void* b, void* out,
                     uint64_t n, Op op) {
    if (n == 0) return RL_OK;
    if (rl_status st = activate(ctx)) return st;
    constexpr int N = map_pack<TIn, TOut>();
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
        const unsigned grid = grid_for(n_packs, uint64_t(kThreads) * UNROLL);
        constexpr uint32_t kind = fused_kind<TIn, TOut, Op>();
        if (kind != 0 && fusing(ctx)) {
            FusedOp f;
            f.kind = kind;
            f.blocks = grid_for(n_packs, uint64_t(kThreads) * FusedShape<Op, TIn, TOut>::unroll);
            f.a = pa;
            f.b = pb;
            f.out = po;
            f.n_packs = n_packs;
            f.tail = tail;
            f.read[0][0] = uintptr_t(pa);
            f.read[0][1] = uintptr_t(pa) + n * sizeof(TIn);
            if (ARITY == 2) {
                f.read[1][0] = uintptr_t(pb);
                f.read[1][1] = uintptr_t(pb) + n * sizeof(TIn);
            }
            f.write[0] = uintptr_t(po);
            f.write[1] = uintptr_t(po) + n * sizeof(TOut);
            if (rl_status st = defer_fused(ctx, f)) return st;
            return after_launch(ctx, name);
        }
        using Big = MapShapeBig<Op, TIn, TOut>;
        if constexpr (Big::from_packs != 0) {
            if (n_packs >= Big::from_packs) {
                RL_LAUNCH(ctx, (k_map<TIn, TOut, N, Big::unroll, ARITY, Big::nt_store, Big::phased, Op>), dim3(grid_for(n_packs, uint64_t(kThreads) * Big::unroll)), dim3(kThreads), pa, pb, po, n_packs, tail, op);
                return after_launch(ctx, name);
            }
        }
        RL_LAUNCH(ctx, (k_map<TIn, TOut, N, UNROLL, ARITY, NTS, PHASED, Op>), dim3(grid), dim3(kThreads), pa, pb, po, n_packs, tail, op);
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
    constexpr int UNROLL = kBroadcastUnroll;
    const T* px = static_cast<const T*>(x->data);
    const T* pbias = static_cast<const T*>(bias->data);
    T* po = static_cast<T*>(out->data);
    const bool vec = cols % N == 0 && aligned_to(px, 16) && aligned_to(pbias, 16) &&
                     aligned_to(po, 16) && n / N <= UINT32_MAX;
    const uint64_t col_packs = cols / N;
    if (vec && fusing(ctx)) {
        const uint64_t n_packs = n / N;
        FusedOp f;
        f.kind = sizeof(T) == 4 ? kFusedBiasF32 : kFusedBiasF16;
        f.blocks = grid_for(n_packs, uint64_t(kThreads) * kFusedBiasUnroll);
        f.a = px;
        f.b = pbias;
        f.out = po;
        f.n_packs = n_packs;
        f.div = uint32_t(col_packs);
        f.read[0][0] = uintptr_t(px);
        f.read[0][1] = uintptr_t(px) + n * sizeof(T);
        f.read[1][0] = uintptr_t(pbias);
        f.read[1][1] = uintptr_t(pbias) + cols * sizeof(T);
        f.write[0] = uintptr_t(po);
        f.write[1] = uintptr_t(po) + n * sizeof(T);
        if (rl_status st = defer_fused(ctx, f)) return st;
        return after_launch(ctx, name);
    }
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

rl_status defer_fused(rl_context* ctx, const FusedOp& f) {
    bool clash = ctx->fused_count == kMaxFused;
    uint64_t blocks = f.blocks;
    for (uint32_t i = 0; i < ctx->fused_count && !clash; ++i) {
        const FusedOp& p = ctx->fused[i];
        blocks += p.blocks;
        clash = overlaps(p.write, f.write[0], f.write[1]) ||
                overlaps(p.read[0], f.write[0], f.write[1]) ||
                overlaps(p.read[1], f.write[0], f.write[1]) ||
                overlaps(p.write, f.read[0][0], f.read[0][1]) ||
                overlaps(p.write, f.read[1][0], f.read[1][1]);
    }
    if (clash || blocks > (1u << 30))
        if (rl_status st = flush_fused(ctx)) return st;
    ctx->fused[ctx->fused_count++] = f;
    return RL_OK;
}

rl_status flush_fused(rl_context* ctx) {
    if (ctx->fused_count == 0) return RL_OK;
    FusedTable t{};
    uint32_t first = 0;
    for (uint32_t i = 0; i < ctx->fused_count; ++i) {
        const FusedOp& f = ctx->fused[i];
        t.first[i] = first;
        FusedSeg& g = t.seg[i];
        g.kind = f.kind;
        g.tail = f.tail;
        g.a = f.a;
        g.b = f.b;
        g.out = f.out;
        g.n_packs = f.n_packs;
        g.head_packs = f.head_packs;
        g.div = FastDiv(f.div ? f.div : 1u);
        g.repeats = f.repeats;
        g.small_index = f.small_index ? 1u : 0u;
        g.outer.rank = f.outer_rank;
        for (uint32_t d = 0; d < kMaxFusedOuterRank; ++d) {
            g.outer.dim[d] = FastDiv(f.outer_dim[d] ? f.outer_dim[d] : 1u);
            g.outer.stride[d] = f.outer_stride[d];
        }
        first += f.blocks;
    }
    t.count = ctx->fused_count;
    ctx->fused_count = 0;
    hipLaunchKernelGGL(k_fused, dim3(first), dim3(kThreads), 0, ctx->stream, t);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(RL_ERR_DEVICE, "fused streaming ops: %s", hipGetErrorString(err));
    return RL_OK;
}

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
