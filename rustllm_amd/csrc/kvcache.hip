// kvcache.hip -- KV-cache writes for gfx950.
//
// kv_cache_write (kernels/kv_cache_write.metal:4-36): a [1, H, S, D] source
// goes to rows start .. start + S of each head of a [1, H, max_seq, D]
// cache: cache[(h * max_seq + start + s) * D + d] = src[h, s, d].  The
// reference runs one thread per element with two divisions; here each
// thread moves a 16-byte pack and decodes its row with 32-bit multiply-high
// division.  The source may be a strided view (the [1, H, S, D] permute of
// the [1, S, H*D] projection that LayerKvCache::append_encode first makes
// contiguous, src/model/kv_cache.rs:123-137): the gather and the write are
// then one pass, so the projection is read once and the cache written once.
// Rows of 32-256 bytes go through the RoPE row-block kernel as a copy job
// (launch_copy_rows); other head sizes and alignments through k_kv_write.
#include "common.hpp"

namespace rl {
namespace {

constexpr int kThreads = 256;

template <typename T, int N, int UNROLL>
__global__ __launch_bounds__(kThreads) void k_kv_write(const T* __restrict__ src,
                                                       T* __restrict__ cache, uint32_t n_items,
                                                       FastDiv packs_per_row, RowDims rd,
                                                       uint32_t inner_stride, uint32_t head_dim,
                                                       uint32_t max_seq, uint32_t start) {
    typedef typename VecOf<T, N>::type V;
    const uint64_t tile = uint64_t(kThreads) * UNROLL;
    const uint64_t step = uint64_t(gridDim.x) * tile;
    for (uint64_t base = uint64_t(blockIdx.x) * tile + threadIdx.x; base < n_items;
         base += step) {
        V v[UNROLL];
        uint64_t dst_off[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_items) {
                uint32_t row, pp;
                packs_per_row.divmod(uint32_t(i), row, pp);
                uint64_t src_off;
                uint32_t position, head;
                decode_row(rd, row, src_off, position, head);
                const uint32_t col = pp * N;
                if constexpr (N == 1) {
                    v[u][0] = src[src_off + uint64_t(col) * inner_stride];
                } else {
                    v[u] = *reinterpret_cast<const V*>(src + src_off + col);
                }
                dst_off[u] = (uint64_t(head) * max_seq + start + position) * head_dim + col;
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_items) store_stream(reinterpret_cast<V*>(cache + dst_off[u]), v[u]);
        }
    }
}

inline unsigned grid_for(uint64_t items, uint64_t per_block) {
    uint64_t blocks = ceil_div(items, per_block);
    if (blocks < 1) blocks = 1;
    if (blocks > (1u << 30)) blocks = 1u << 30;
    return unsigned(blocks);
}

// dims = [1, H, S, D] (validated), strides of the source view.
template <typename T>
rl_status launch_kv_write(rl_context* ctx, const char* name, const T* src, const uint64_t* dims,
                          const uint64_t* strides, T* cache, uint64_t max_seq, uint64_t start) {
    if (rl_status st = activate(ctx)) return st;
    // Rows of 32-256 bytes on 16-byte boundaries: the row-block kernel (16
    // bytes a lane, rows decoded branch-free; the [1, 5, 4096, 64] f16 append
    // of a [1, 4096, 5, 64] projection view, graph-replayed back to back:
    // 4.22 us with k_kv_write below, 2.63 us).
    if (strides[3] == 1 &&
        launch_copy_rows<T>(ctx, src, dims, strides, 4, cache, uint32_t(max_seq), uint32_t(start)))
        return after_launch(ctx, name);
    const uint64_t heads = dims[1], seq = dims[2], head_dim = dims[3];
    int n = 16 / int(sizeof(T));
    while (n > 1) {
        const bool ok = strides[3] == 1 && head_dim % n == 0 && strides[1] % n == 0 &&
                        strides[2] % n == 0 && aligned_to(src, n * sizeof(T)) &&
                        aligned_to(cache, n * sizeof(T));
        if (ok) break;
        n >>= 1;
    }
    const RowDims rd = make_row_dims(dims, strides, 4);
    const uint64_t n_items = heads * seq * (head_dim / n);
    const FastDiv ppr(uint32_t(head_dim / n));
    constexpr int U = 1;
    const dim3 grid(grid_for(n_items, uint64_t(kThreads) * U)), block(kThreads);
    const uint32_t ni = uint32_t(n_items), is = uint32_t(strides[3]), hd = uint32_t(head_dim),
                   ms = uint32_t(max_seq), st = uint32_t(start);
    switch (n) {
        case 8:
            RL_LAUNCH(ctx, (k_kv_write<T, 8, U>), grid, block, src, cache, ni, ppr, rd, is, hd, ms, st);
            break;
        case 4:
            RL_LAUNCH(ctx, (k_kv_write<T, 4, U>), grid, block, src, cache, ni, ppr, rd, is, hd, ms, st);
            break;
        case 2:
            RL_LAUNCH(ctx, (k_kv_write<T, 2, U>), grid, block, src, cache, ni, ppr, rd, is, hd, ms, st);
            break;
        default:
            RL_LAUNCH(ctx, (k_kv_write<T, 1, U>), grid, block, src, cache, ni, ppr, rd, is, hd, ms, st);
            break;
    }
    return after_launch(ctx, name);
}

}  // namespace

// kv_cache_write_encode's checks (src/ops/kv_cache_write.rs:71-141) in order
// for a source of dims [1, H, S, D] and a [1, H, max_seq, D] cache buffer,
// plus the view's bounds.  Shared with the fused RoPE entry.
rl_status validate_kv_write(const char* name, const rl_buffer* cache, uint64_t max_seq,
                            const rl_buffer* src, const uint64_t* dims, const uint64_t* strides,
                            uint32_t rank, uint64_t start, uint64_t es, bool exact_source) {
    if (rl_status st = check_buffer(cache, "cache")) return st;
    if (rl_status st = check_buffer(src, "source")) return st;
    if (dims == nullptr || strides == nullptr)
        return fail(RL_ERR_INVALID_ARGUMENT, "dims or strides is null");
    if (cache->byte_len != cache->len * es || src->byte_len < src->len * es)
        return fail(RL_ERR_UNSUPPORTED_DTYPE, "%s expects %s cache and source", name,
                    es == 4 ? "F32" : "F16");
    if (rank != 4) return fail(RL_ERR_INVALID_SHAPE, "invalid KV cache write shape");
    for (uint32_t d = 0; d < 4; ++d)
        if (dims[d] == 0)
            return fail(RL_ERR_INVALID_SHAPE, "shape dimensions must be greater than zero");
    const uint64_t heads = dims[1], seq = dims[2], head_dim = dims[3];
    if (max_seq == 0 || heads > UINT64_MAX / max_seq || heads * max_seq > UINT64_MAX / head_dim)
        return fail(RL_ERR_INVALID_SHAPE, "invalid KV cache write shape");
    if (dims[0] != 1 || cache->len != heads * max_seq * head_dim)
        return fail(RL_ERR_INVALID_SHAPE, "invalid KV cache write shape");
    if (exact_source && (heads > UINT64_MAX / seq || heads * seq > UINT64_MAX / head_dim ||
                         src->len != heads * seq * head_dim))
        return fail(RL_ERR_INVALID_SHAPE, "invalid KV cache write shape");
    if (start > UINT64_MAX - seq || start + seq > max_seq)
        return fail_position_out_of_range(start, seq, max_seq);
    const uint64_t numel = heads * seq * head_dim;
    if (start > UINT32_MAX || seq > UINT32_MAX || max_seq > UINT32_MAX ||
        head_dim > UINT32_MAX || numel > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "KV cache dimension exceeds u32");
    for (uint32_t d = 0; d < 4; ++d)
        if (strides[d] > UINT32_MAX)
            return fail(RL_ERR_INVALID_SHAPE, "KV cache dimension exceeds u32");
    unsigned __int128 last = 0;
    for (uint32_t d = 0; d < 4; ++d) last += (unsigned __int128)(dims[d] - 1) * strides[d];
    if (last >= src->len)
        return fail(RL_ERR_INVALID_SHAPE, "view reaches past the end of its %llu-element buffer",
                    (unsigned long long)src->len);
    return RL_OK;
}

namespace {

template <typename T>
rl_status kv_write_entry(rl_context* ctx, const char* name, const rl_buffer* cache,
                         uint64_t max_seq, const rl_buffer* src, const uint64_t* dims,
                         const uint64_t* strides, uint32_t rank, uint64_t start,
                         bool exact_source) {
    if (rl_status st = validate_kv_write(name, cache, max_seq, src, dims, strides, rank, start,
                                         sizeof(T), exact_source))
        return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_kv_write<T>(ctx, name, static_cast<const T*>(src->data), dims, strides,
                              static_cast<T*>(cache->data), max_seq, start);
}

template <typename T>
rl_status kv_write_contiguous_entry(rl_context* ctx, const char* name, const rl_buffer* cache,
                                    uint64_t kv_heads, uint64_t max_seq, uint64_t head_dim,
                                    const rl_buffer* source, uint64_t seq_len, uint64_t start) {
    // A contiguous source holds exactly [1, H, S, D] (the strides only matter
    // once the dims have been validated).
    const uint64_t dims[4] = {1, kv_heads, seq_len, head_dim};
    const uint64_t strides[4] = {kv_heads * seq_len * head_dim, seq_len * head_dim, head_dim, 1};
    return kv_write_entry<T>(ctx, name, cache, max_seq, source, dims, strides, 4, start, true);
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_kv_cache_write_f32(rl_context* ctx, const rl_buffer* cache, uint64_t kv_heads,
                                uint64_t max_seq, uint64_t head_dim, const rl_buffer* source,
                                uint64_t seq_len, uint64_t start) {
    return kv_write_contiguous_entry<float>(ctx, "kv_cache_write_f32", cache, kv_heads, max_seq,
                                            head_dim, source, seq_len, start);
}

rl_status rl_kv_cache_write_f16(rl_context* ctx, const rl_buffer* cache, uint64_t kv_heads,
                                uint64_t max_seq, uint64_t head_dim, const rl_buffer* source,
                                uint64_t seq_len, uint64_t start) {
    return kv_write_contiguous_entry<half_t>(ctx, "kv_cache_write_f16", cache, kv_heads, max_seq,
                                             head_dim, source, seq_len, start);
}

rl_status rl_kv_cache_write_strided_f32(rl_context* ctx, const rl_buffer* src,
                                        const uint64_t* dims, const uint64_t* strides,
                                        uint32_t rank, const rl_buffer* cache, uint64_t max_seq,
                                        uint64_t start) {
    return kv_write_entry<float>(ctx, "kv_cache_write_f32", cache, max_seq, src, dims, strides,
                                 rank, start, false);
}

rl_status rl_kv_cache_write_strided_f16(rl_context* ctx, const rl_buffer* src,
                                        const uint64_t* dims, const uint64_t* strides,
                                        uint32_t rank, const rl_buffer* cache, uint64_t max_seq,
                                        uint64_t start) {
    return kv_write_entry<half_t>(ctx, "kv_cache_write_f16", cache, max_seq, src, dims, strides,
                                  rank, start, false);
}

}  // extern "C"
