// embedding.hip -- token embedding gather for gfx950.
//
// out[t, :] = weight[ids[t], :] (kernels/embedding.metal:5-54).  The ids
// are validated on the host against the vocabulary (src/ops/embedding.rs:
// 119-149).  Up to 256 of them (decode steps, short prompts) travel in the
// kernel arguments, so the gather is one launch with no copy and no
// dependent id load from memory; more are staged to device memory in
// stream order.  Each thread copies one 16-byte pack of a row; the weight
// row and the output row move as whole packs.
#include "common.hpp"

namespace rl {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kInlineIds = 256;

// Token ids in device memory.
struct DeviceIds {
    const uint32_t* p;
    __device__ uint32_t operator[](uint32_t t) const { return p[t]; }
};

// Token ids in the kernel arguments.
struct InlineIds {
    uint32_t id[kInlineIds];
    __device__ uint32_t operator[](uint32_t t) const { return id[t]; }
};

template <typename T, int N, int UNROLL, typename Ids>
__global__ __launch_bounds__(kThreads) void k_embedding(const T* __restrict__ weight, Ids ids,
                                                        T* __restrict__ out, uint32_t n_items,
                                                        FastDiv packs_per_row) {
    typedef typename VecOf<T, N>::type V;
    const uint64_t tile = uint64_t(kThreads) * UNROLL;
    const uint64_t step = uint64_t(gridDim.x) * tile;
    const uint32_t row_packs = packs_per_row.divisor;
    for (uint64_t base = uint64_t(blockIdx.x) * tile + threadIdx.x; base < n_items;
         base += step) {
        V v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_items) {
                uint32_t token, pp;
                packs_per_row.divmod(uint32_t(i), token, pp);
                const uint64_t src = uint64_t(ids[token]) * row_packs + pp;
                v[u] = reinterpret_cast<const V*>(weight)[src];
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_items) store_stream(reinterpret_cast<V*>(out) + i, v[u]);
        }
    }
}

inline unsigned grid_for(uint64_t items, uint64_t per_block) {
    uint64_t blocks = ceil_div(items, per_block);
    if (blocks < 1) blocks = 1;
    if (blocks > (1u << 30)) blocks = 1u << 30;
    return unsigned(blocks);
}

template <typename T, typename Ids>
void launch_gather(rl_context* ctx, const T* w, const Ids& ids, T* o, uint64_t hidden_size,
                   uint64_t out_elements) {
    constexpr int U = 2;
    int n = 16 / int(sizeof(T));
    while (n > 1 && !(hidden_size % n == 0 && aligned_to(w, n * sizeof(T)) &&
                      aligned_to(o, n * sizeof(T))))
        n >>= 1;
    const uint64_t n_items = out_elements / n;
    const FastDiv ppr(uint32_t(hidden_size / n));
    const dim3 grid(grid_for(n_items, uint64_t(kThreads) * U)), block(kThreads);
    const uint32_t ni = uint32_t(n_items);
    switch (n) {
        case 8:
            RL_LAUNCH(ctx, (k_embedding<T, 8, U, Ids>), grid, block, w, ids, o, ni, ppr);
            break;
        case 4:
            RL_LAUNCH(ctx, (k_embedding<T, 4, U, Ids>), grid, block, w, ids, o, ni, ppr);
            break;
        case 2:
            RL_LAUNCH(ctx, (k_embedding<T, 2, U, Ids>), grid, block, w, ids, o, ni, ppr);
            break;
        default:
            RL_LAUNCH(ctx, (k_embedding<T, 1, U, Ids>), grid, block, w, ids, o, ni, ppr);
            break;
    }
}

// src/ops/embedding.rs:119-149 (validate) and :171-183 (u32 limits), in order.
template <typename T>
rl_status embedding_entry(rl_context* ctx, const char* name, const rl_buffer* weight,
                          uint64_t vocab_size, uint64_t hidden_size, const uint32_t* token_ids,
                          uint64_t n_tokens, const rl_buffer* out) {
    if (rl_status st = check_buffer(weight, "weight")) return st;
    if (n_tokens == 0)
        return fail(RL_ERR_INVALID_SHAPE, "embedding requires at least one token");
    if (token_ids == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "token ids pointer is null");
    const bool size_ok = hidden_size == 0 || vocab_size <= UINT64_MAX / hidden_size;
    if (!size_ok || weight->len != vocab_size * hidden_size ||
        weight->byte_len != weight->len * sizeof(T))
        return fail(RL_ERR_INVALID_SHAPE,
                    "embedding weight has %llu elements (%llu bytes), expected %llu elements of "
                    "%zu bytes for shape [%llu, %llu]",
                    (unsigned long long)weight->len, (unsigned long long)weight->byte_len,
                    (unsigned long long)(size_ok ? vocab_size * hidden_size : 0), sizeof(T),
                    (unsigned long long)vocab_size, (unsigned long long)hidden_size);
    for (uint64_t t = 0; t < n_tokens; ++t)
        if (uint64_t(token_ids[t]) >= vocab_size)
            return fail_invalid_token_id(token_ids[t], vocab_size);
    if (hidden_size == 0 || n_tokens > UINT64_MAX / hidden_size)
        return fail(RL_ERR_INVALID_SHAPE, "embedding dimension exceeds u32");
    const uint64_t out_elements = n_tokens * hidden_size;
    if (hidden_size > UINT32_MAX || out_elements > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "embedding dimension exceeds u32");
    if (rl_status st = check_output(out, out_elements, sizeof(T), "embedding")) return st;
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;

    const T* w = static_cast<const T*>(weight->data);
    T* o = static_cast<T*>(out->data);
    if (n_tokens <= kInlineIds) {
        InlineIds ids{};
        for (uint64_t t = 0; t < n_tokens; ++t) ids.id[t] = token_ids[t];
        launch_gather<T>(ctx, w, ids, o, hidden_size, out_elements);
        return after_launch(ctx, name);
    }
    void* dev_ids = nullptr;
    if (rl_status st = stage_to_device(ctx, token_ids, n_tokens * sizeof(uint32_t), &dev_ids))
        return st;
    launch_gather<T>(ctx, w, DeviceIds{static_cast<const uint32_t*>(dev_ids)}, o, hidden_size,
                     out_elements);
    const rl_status st = after_launch(ctx, name);
    ctx->pool.release(dev_ids);  // stream-ordered: later users run after the gather
    return st;
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_embedding_f32(rl_context* ctx, const rl_buffer* weight, uint64_t vocab_size,
                           uint64_t hidden_size, const uint32_t* token_ids, uint64_t n_tokens,
                           const rl_buffer* out) {
    return embedding_entry<float>(ctx, "embedding_f32", weight, vocab_size, hidden_size,
                                  token_ids, n_tokens, out);
}

rl_status rl_embedding_f16(rl_context* ctx, const rl_buffer* weight, uint64_t vocab_size,
                           uint64_t hidden_size, const uint32_t* token_ids, uint64_t n_tokens,
                           const rl_buffer* out) {
    return embedding_entry<half_t>(ctx, "embedding_f16", weight, vocab_size, hidden_size,
                                   token_ids, n_tokens, out);
}

}  // extern "C"
