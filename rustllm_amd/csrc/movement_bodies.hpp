// movement_bodies.hpp -- the bodies of the row gather (contiguous of a view
// whose innermost dim has stride 1) and of repeat_kv, shared by their own
// kernels (movement.hip) and the fused launch of recorded streaming ops
// (elementwise.hip).  A body takes its block index and the block count of
// its grid, so that it runs the same whether it owns the grid or a share of
// a fused one.
#pragma once

#include "common.hpp"

namespace rl {

constexpr int kMoveThreads = 256;

// Outer dimensions of a view, innermost first (at most MAXR of them).
template <int MAXR, typename Stride = uint64_t>
struct OuterDimsT {
    uint32_t rank;
    FastDiv dim[MAXR];
    Stride stride[MAXR];

    __device__ inline uint64_t offset(uint32_t index) const {
        uint64_t off = 0;
#pragma unroll 4
        for (uint32_t d = 0; d < rank; ++d) {
            uint32_t q, r;
            dim[d].divmod(index, q, r);
            off += uint64_t(r) * stride[d];
            index = q;
        }
        return off;
    }
};

// dst[i] = src[offset(row) + pack], rows of `row_packs` packs of N elements.
template <typename T, int N, int UNROLL, typename Dims>
__device__ inline void gather_rows_body(const T* __restrict__ src, T* __restrict__ dst,
                                        uint32_t n_packs, FastDiv row_packs, const Dims& outer,
                                        uint32_t blk, uint32_t nblk) {
    typedef typename VecOf<T, N>::type V;
    V* vdst = reinterpret_cast<V*>(dst);
    const uint64_t tile = uint64_t(kMoveThreads) * UNROLL;
    const uint64_t step = uint64_t(nblk) * tile;
    for (uint64_t base = uint64_t(blk) * tile + threadIdx.x; base < n_packs; base += step) {
        V r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kMoveThreads;
            if (i < n_packs) {
                uint32_t row, p;
                row_packs.divmod(uint32_t(i), row, p);
                uint64_t off = outer.offset(row) + uint64_t(p) * N;
                r[u] = *reinterpret_cast<const V*>(src + off);
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kMoveThreads;
            if (i < n_packs) store_stream(vdst + i, r[u]);
        }
    }
}

// The same copy walked in source order, for a view that is a permutation of
// a dense tensor (its rows tile the source with no gaps): src pack i (read
// contiguously) goes to dst[outer.offset(row) + pack], where `outer` lists
// the source's row dims fastest first with each one's stride in the
// (contiguous) output.  A wave then reads 1 KB of consecutive source and
// writes whole rows, where the output-order walk reads rows scattered
// through the source ([1, 4096, 9, 64] -> [1, 9, 4096, 64], back to back:
// f16 3.65 -> 3.28 us, f32 5.45 -> 4.68 us, against 3.1 and 4.5 us for a
// plain copy of the same bytes).  NT_STORE: streamed stores (faster for the
// 128-byte f16 rows there; plain stores for the 256-byte f32 rows).
template <typename T, int N, int UNROLL, bool NT_STORE, typename Dims>
__device__ inline void scatter_rows_body(const T* __restrict__ src, T* __restrict__ dst,
                                         uint32_t n_packs, FastDiv row_packs, const Dims& outer,
                                         uint32_t blk, uint32_t nblk) {
    typedef typename VecOf<T, N>::type V;
    const V* vsrc = reinterpret_cast<const V*>(src);
    const uint64_t tile = uint64_t(kMoveThreads) * UNROLL;
    const uint64_t step = uint64_t(nblk) * tile;
    for (uint64_t base = uint64_t(blk) * tile + threadIdx.x; base < n_packs; base += step) {
        V r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kMoveThreads;
            if (i < n_packs) r[u] = load_stream(vsrc + i);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * kMoveThreads;
            if (i < n_packs) {
                uint32_t row, p;
                row_packs.divmod(uint32_t(i), row, p);
                V* d = reinterpret_cast<V*>(dst + outer.offset(row) + uint64_t(p) * N);
                if constexpr (NT_STORE)
                    store_stream(d, r[u]);
                else
                    *d = r[u];
            }
        }
    }
}

// out[(head * repeats + r) * head_packs + p] = in[head * head_packs + p],
// head = b * kv_heads + kv_head.
template <typename T, int N, int UNROLL>
__device__ inline void repeat_kv_body(const T* __restrict__ in, T* __restrict__ out,
                                      uint64_t n_packs, uint64_t head_packs, FastDiv head_div,
                                      uint32_t repeats, bool small_index, uint32_t blk,
                                      uint32_t nblk) {
    typedef typename VecOf<T, N>::type V;
    const V* vin = reinterpret_cast<const V*>(in);
    V* vout = reinterpret_cast<V*>(out);
    const uint64_t tile = uint64_t(kMoveThreads) * UNROLL;
    const uint64_t step = uint64_t(nblk) * tile;
    for (uint64_t base = uint64_t(blk) * tile + threadIdx.x; base < n_packs; base += step) {
        V r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kMoveThreads;
            if (i < n_packs) r[u] = load_stream(vin + i);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kMoveThreads;
            if (i < n_packs) {
                uint64_t head, p;
                if (small_index) {
                    uint32_t q, rem;
                    head_div.divmod(uint32_t(i), q, rem);
                    head = q;
                    p = rem;
                } else {
                    head = i / head_packs;
                    p = i - head * head_packs;
                }
                V* dst = vout + head * repeats * head_packs + p;
                for (uint32_t k = 0; k < repeats; ++k) store_stream(dst + k * head_packs, r[u]);
            }
        }
    }
}

}  // namespace rl
