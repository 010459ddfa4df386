// movement.hip -- contiguous (strided gather of a view) and repeat_kv for
// gfx950.
//
// contiguous: the view is first simplified on the host (size-1 dims dropped,
// dims whose strides chain are merged).  If the innermost dim has stride 1
// the copy is a gather of rows: each row's source offset is decoded once per
// 16-byte pack with 32-bit multiply-high division, and rows move as whole
// packs, so every wave load covers runs of at least one row (256 B for a
// 64-wide f32 head).  A view that permutes a dense tensor (a transpose of
// head and sequence dims) is walked in source order instead: contiguous
// loads, each row stored whole at its output position.  Anything else falls
// back to a per-element gather.
//
// repeat_kv: each thread reads one pack of the KV input once and writes it
// to the `repeats` query heads that share it, so HBM sees the minimum
// traffic (input once + output once).
#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "movement_bodies.hpp"

namespace rl {
namespace {

constexpr int kThreads = kMoveThreads;
constexpr int kMaxRank = 16;
typedef OuterDimsT<kMaxRank> OuterDims;

template <typename T, int N, int UNROLL>
__global__ __launch_bounds__(kThreads) void k_gather_rows(const T* __restrict__ src,
                                                          T* __restrict__ dst, uint32_t n_packs,
                                                          FastDiv row_packs, OuterDims outer) {
    gather_rows_body<T, N, UNROLL>(src, dst, n_packs, row_packs, outer, blockIdx.x, gridDim.x);
}

// The row copy walked in source order (a view that permutes a dense tensor):
// `outer` = the source's row dims, fastest first, with their output strides.
template <typename T, int N, int UNROLL, bool NT_STORE>
__global__ __launch_bounds__(kThreads) void k_scatter_rows(const T* __restrict__ src,
                                                           T* __restrict__ dst, uint32_t n_packs,
                                                           FastDiv row_packs, OuterDims outer) {
    scatter_rows_body<T, N, UNROLL, NT_STORE>(src, dst, n_packs, row_packs, outer, blockIdx.x,
                                              gridDim.x);
}

// Per-element gather over all dims (innermost first in `dims`).
template <typename T>
__global__ __launch_bounds__(kThreads) void k_gather_elems(const T* __restrict__ src,
                                                           T* __restrict__ dst, uint32_t numel,
                                                           OuterDims dims) {
    const uint64_t step = uint64_t(gridDim.x) * kThreads;
    for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < numel; i += step)
        dst[i] = src[dims.offset(uint32_t(i))];
}

template <typename T, int N, int UNROLL>
__global__ __launch_bounds__(kThreads) void k_repeat_kv(const T* __restrict__ in,
                                                        T* __restrict__ out, uint64_t n_packs,
                                                        uint64_t head_packs, FastDiv head_div,
                                                        uint32_t repeats, bool small_index) {
    repeat_kv_body<T, N, UNROLL>(in, out, n_packs, head_packs, head_div, repeats, small_index,
                                 blockIdx.x, gridDim.x);
}

inline unsigned grid_for(uint64_t items, uint64_t per_block) {
    uint64_t blocks = ceil_div(items, per_block);
    if (blocks < 1) blocks = 1;
    if (blocks > (1u << 30)) blocks = 1u << 30;
    return unsigned(blocks);
}

// A view after dropping size-1 dims and merging dims whose strides chain
// (strides[i] == strides[i+1] * dims[i+1]); iteration order is unchanged.
struct SimpleView {
    std::vector<uint64_t> dims, strides;  // outermost first
};

SimpleView simplify(const uint64_t* dims, const uint64_t* strides, uint32_t rank) {
    SimpleView v;
    for (uint32_t d = 0; d < rank; ++d) {
        if (dims[d] == 1) continue;
        if (!v.dims.empty() && v.strides.back() == strides[d] * dims[d]) {
            v.dims.back() *= dims[d];
            v.strides.back() = strides[d];
        } else {
            v.dims.push_back(dims[d]);
            v.strides.push_back(strides[d]);
        }
    }
    if (v.dims.empty()) {  // a single element
        v.dims.push_back(1);
        v.strides.push_back(1);
    }
    return v;
}

template <typename T>
rl_status launch_contiguous(rl_context* ctx, const char* name, const T* src, T* dst,
                            const SimpleView& v, uint64_t numel) {
    if (rl_status st = activate(ctx)) return st;
    const uint32_t rank = uint32_t(v.dims.size());
    const uint64_t inner = v.dims[rank - 1];
    if (v.strides[rank - 1] == 1) {
        // Largest pack (<= 16 B) dividing the row, every outer stride and
        // both base addresses.
        int n = 16 / int(sizeof(T));
        while (n > 1) {
            bool ok = inner % n == 0 && aligned_to(src, n * sizeof(T)) &&
                      aligned_to(dst, n * sizeof(T));
            for (uint32_t d = 0; d + 1 < rank && ok; ++d) ok = v.strides[d] % n == 0;
            if (ok) break;
            n >>= 1;
        }
        // A view that permutes a dense tensor -- its outer dims sorted by
        // stride have strides inner, inner * dim, ... (so it covers source
        // elements [0, numel) once each) -- is walked in source order; the
        // output strides of view dim d are the product of the dims after it.
        std::vector<uint32_t> by_stride;  // outer view dims, ascending stride
        for (uint32_t d = 0; d + 1 < rank; ++d) by_stride.push_back(d);
        std::sort(by_stride.begin(), by_stride.end(),
                  [&](uint32_t a, uint32_t b) { return v.strides[a] < v.strides[b]; });
        bool dense = rank >= 2;
        uint64_t expect = inner;
        for (uint32_t d : by_stride) {
            if (!dense || v.strides[d] != expect) {
                dense = false;
                break;
            }
            expect *= v.dims[d];
        }
        OuterDims outer{};
        outer.rank = rank - 1;
        if (dense) {
            std::vector<uint64_t> out_stride(rank, 1);
            for (uint32_t d = rank - 1; d-- > 0;) out_stride[d] = out_stride[d + 1] * v.dims[d + 1];
            for (uint32_t k = 0; k + 1 < rank; ++k) {
                outer.dim[k] = FastDiv(uint32_t(v.dims[by_stride[k]]));
                outer.stride[k] = out_stride[by_stride[k]];
            }
        } else {
            for (uint32_t d = 0; d + 1 < rank; ++d) {
                outer.dim[d] = FastDiv(uint32_t(v.dims[rank - 2 - d]));
                outer.stride[d] = v.strides[rank - 2 - d];
            }
        }
        const uint64_t n_packs = numel / n;
        const FastDiv row_packs(uint32_t(inner / n));
        // Two packs per thread: on the [1, 4096, H, 64] -> [1, H, 4096, 64]
        // transpose (9.4-18.9 MB) back-to-back launches take 10-15% less
        // time than with four (fewer, longer waves) and match one.
        constexpr int U = 2;
        const dim3 grid(grid_for(n_packs, uint64_t(kThreads) * U)), block(kThreads);
        if (n == 16 / int(sizeof(T)) && rank - 1 <= kMaxFusedOuterRank && fusing(ctx)) {
            // recorded into a graph: one of the fused streaming ops
            FusedOp f;
            f.kind = dense ? (sizeof(T) == 4 ? kFusedScatterF32 : kFusedScatterF16)
                           : (sizeof(T) == 4 ? kFusedGatherF32 : kFusedGatherF16);
            f.blocks = grid.x;
            f.a = src;
            f.out = dst;
            f.n_packs = n_packs;
            f.div = uint32_t(inner / n);
            f.outer_rank = rank - 1;
            uint64_t last = v.dims[rank - 1] - 1;  // the view's last element in the source
            for (uint32_t d = 0; d + 1 < rank; ++d) {
                f.outer_dim[d] = outer.dim[d].divisor;
                f.outer_stride[d] = uint32_t(outer.stride[d]);
                last += (v.dims[rank - 2 - d] - 1) * v.strides[rank - 2 - d];
            }
            f.read[0][0] = uintptr_t(src);
            f.read[0][1] = uintptr_t(src + last + 1);
            f.write[0] = uintptr_t(dst);
            f.write[1] = uintptr_t(dst + numel);
            if (rl_status st = defer_fused(ctx, f)) return st;
            return after_launch(ctx, name);
        }
        // f16: streamed stores into the 128-byte rows; f32: plain stores
        constexpr bool NT = sizeof(T) == 2;
#define RL_ROWS(N)                                                                                 \
    do {                                                                                           \
        if (dense)                                                                                 \
            RL_LAUNCH(ctx, (k_scatter_rows<T, N, U, NT>), grid, block, src, dst, uint32_t(n_packs), \
                      row_packs, outer);                                                           \
        else                                                                                       \
            RL_LAUNCH(ctx, (k_gather_rows<T, N, U>), grid, block, src, dst, uint32_t(n_packs),    \
                      row_packs, outer);                                                           \
    } while (0)
        switch (n) {
            case 8: RL_ROWS(8); break;
            case 4: RL_ROWS(4); break;
            case 2: RL_ROWS(2); break;
            default: RL_ROWS(1); break;
        }
#undef RL_ROWS
    } else {
        OuterDims all{};
        all.rank = rank;
        for (uint32_t d = 0; d < rank; ++d) {
            all.dim[d] = FastDiv(uint32_t(v.dims[rank - 1 - d]));
            all.stride[d] = v.strides[rank - 1 - d];
        }
        RL_LAUNCH(ctx, (k_gather_elems<T>), dim3(grid_for(numel, kThreads * 4)), dim3(kThreads), src, dst, uint32_t(numel), all);
    }
    return after_launch(ctx, name);
}

// src/ops/contiguous.rs:85-154, in the reference's order, plus two checks
// that keep every read inside the source buffer.
rl_status contiguous_impl(rl_context* ctx, const char* name, const rl_buffer* src,
                          const uint64_t* dims, const uint64_t* strides, uint32_t rank,
                          const rl_buffer* out, uint64_t es) {
    if (rl_status st = check_buffer(src, "source")) return st;
    if (rank == 0) return fail(RL_ERR_INVALID_SHAPE, "shape cannot be empty");
    if (dims == nullptr || strides == nullptr)
        return fail(RL_ERR_INVALID_SHAPE, "shape rank and strides rank differ");
    if (rank > kMaxRank) return fail(RL_ERR_INVALID_SHAPE, "tensor rank exceeds %d", kMaxRank);
    uint64_t numel = 1;
    for (uint32_t d = 0; d < rank; ++d) {
        if (dims[d] == 0)
            return fail(RL_ERR_INVALID_SHAPE, "shape dimensions must be greater than zero");
        if (numel > UINT64_MAX / dims[d])
            return fail(RL_ERR_INVALID_SHAPE, "tensor element count exceeds u32");
        numel *= dims[d];
    }
    // The reference also requires src->len >= numel; that holds for every view
    // its API can form (permute / transpose / narrow of a whole tensor).  The
    // exact bound below replaces it so that stride-0 (broadcast) views, whose
    // storage is smaller than the view, can be materialised too.
    if (src->byte_len != src->len * es)
        return fail(RL_ERR_INVALID_SHAPE,
                    "source buffer does not match contiguous materialization dtype");
    for (uint32_t d = 0; d < rank; ++d)
        if (dims[d] > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "shape dimension exceeds u32");
    for (uint32_t d = 0; d < rank; ++d)
        if (strides[d] > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "stride exceeds u32");
    if (numel > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "tensor element count exceeds u32");
    unsigned __int128 last = 0;
    for (uint32_t d = 0; d < rank; ++d) last += (unsigned __int128)(dims[d] - 1) * strides[d];
    if (last >= src->len)
        return fail(RL_ERR_INVALID_SHAPE,
                    "view reaches element %llu of a %llu-element source buffer",
                    (unsigned long long)(last > UINT64_MAX ? UINT64_MAX : uint64_t(last)),
                    (unsigned long long)src->len);
    if (rl_status st = check_output(out, numel, es, "contiguous")) return st;
    if (rl_status st = require_context(ctx)) return st;
    SimpleView v = simplify(dims, strides, rank);
    if (es == 4)
        return launch_contiguous<float>(ctx, name, static_cast<const float*>(src->data),
                                        static_cast<float*>(out->data), v, numel);
    return launch_contiguous<half_t>(ctx, name, static_cast<const half_t*>(src->data),
                                     static_cast<half_t*>(out->data), v, numel);
}

// src/tensor/repeat_kv.rs:13-130 (buffer level: rank-4 and contiguity are
// the Tensor layer's checks; repeats == 0 is rejected here as there).
rl_status repeat_kv_impl(rl_context* ctx, const char* name, const rl_buffer* in, uint64_t batch,
                         uint64_t kv_heads, uint64_t seq_len, uint64_t head_dim, uint64_t repeats,
                         const rl_buffer* out, uint64_t es) {
    if (rl_status st = check_buffer(in, "input")) return st;
    if (repeats == 0)
        return fail(RL_ERR_MODEL_FORMAT, "repeat_kv repeats must be greater than zero");
    if (batch == 0 || kv_heads == 0 || seq_len == 0 || head_dim == 0)
        return fail(RL_ERR_INVALID_SHAPE, "shape dimensions must be greater than zero");
    if (kv_heads > UINT64_MAX / repeats)
        return fail(RL_ERR_MODEL_FORMAT, "repeat_kv head count overflow");
    const uint64_t dims[4] = {kv_heads, seq_len, head_dim, repeats};
    for (uint64_t d : dims)
        if (d > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "repeat_kv dimension exceeds u32");
    const uint64_t head = seq_len * head_dim;
    const uint64_t in_numel = batch * kv_heads * head;
    if (in->len != in_numel || in->byte_len != in_numel * es)
        return fail(RL_ERR_INVALID_SHAPE, "repeat_kv input has %llu elements, expected %llu",
                    (unsigned long long)in->len, (unsigned long long)in_numel);
    if (rl_status st = check_output(out, in_numel * repeats, es, "repeat_kv")) return st;
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;

    const void* src = in->data;
    void* dst = out->data;
    constexpr int U = 2;
    auto launch = [&](auto tag, auto n_const) {
        typedef decltype(tag) T;
        constexpr int N = decltype(n_const)::value;
        const uint64_t head_packs = head / N;
        const uint64_t n_packs = in_numel / N;
        const bool small = n_packs <= UINT32_MAX && head_packs <= UINT32_MAX;
        if (N * sizeof(T) == 16 && fusing(ctx)) {
            // recorded into a graph: one of the fused streaming ops
            FusedOp f;
            f.kind = sizeof(T) == 4 ? kFusedRepeatF32 : kFusedRepeatF16;
            f.blocks = grid_for(n_packs, kThreads * U);
            f.a = src;
            f.out = dst;
            f.n_packs = n_packs;
            f.head_packs = head_packs;
            f.div = small ? uint32_t(head_packs) : 1u;
            f.repeats = uint32_t(repeats);
            f.small_index = small;
            f.read[0][0] = uintptr_t(src);
            f.read[0][1] = uintptr_t(src) + in_numel * sizeof(T);
            f.write[0] = uintptr_t(dst);
            f.write[1] = uintptr_t(dst) + in_numel * repeats * sizeof(T);
            return rl_status(defer_fused(ctx, f));
        }
        RL_LAUNCH(ctx, (k_repeat_kv<T, N, U>), dim3(grid_for(n_packs, kThreads * U)), dim3(kThreads), static_cast<const T*>(src), static_cast<T*>(dst), n_packs, head_packs, FastDiv(small ? uint32_t(head_packs) : 1u), uint32_t(repeats), small);
        return rl_status(RL_OK);
    };
    const bool aligned16 = aligned_to(src, 16) && aligned_to(dst, 16);
    rl_status st = RL_OK;
    if (es == 4) {
        if (head % 4 == 0 && aligned16)
            st = launch(float(), std::integral_constant<int, 4>());
        else
            st = launch(float(), std::integral_constant<int, 1>());
    } else {
        if (head % 8 == 0 && aligned16)
            st = launch(half_t(), std::integral_constant<int, 8>());
        else
            st = launch(half_t(), std::integral_constant<int, 1>());
    }
    if (st != RL_OK) return st;
    return after_launch(ctx, name);
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_contiguous_f32(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                            const uint64_t* strides, uint32_t rank, const rl_buffer* out) {
    return contiguous_impl(ctx, "contiguous_f32", src, dims, strides, rank, out, 4);
}

rl_status rl_contiguous_f16(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                            const uint64_t* strides, uint32_t rank, const rl_buffer* out) {
    return contiguous_impl(ctx, "contiguous_f16", src, dims, strides, rank, out, 2);
}

rl_status rl_repeat_kv_f32(rl_context* ctx, const rl_buffer* input, uint64_t batch,
                           uint64_t kv_heads, uint64_t seq_len, uint64_t head_dim,
                           uint64_t repeats, const rl_buffer* out) {
    return repeat_kv_impl(ctx, "repeat_kv_f32", input, batch, kv_heads, seq_len, head_dim,
                          repeats, out, 4);
}

rl_status rl_repeat_kv_f16(rl_context* ctx, const rl_buffer* input, uint64_t batch,
                           uint64_t kv_heads, uint64_t seq_len, uint64_t head_dim,
                           uint64_t repeats, const rl_buffer* out) {
    return repeat_kv_impl(ctx, "repeat_kv_f16", input, batch, kv_heads, seq_len, head_dim,
                          repeats, out, 2);
}

}  // extern "C"
