// gqa.hip -- the grouped-query matmuls of the attention core for gfx950.
//
// gqa_qk_matmul (src/tensor/gqa_matmul.rs:23-61, kernels/gqa_matmul.metal:
// 7-322): scores[b, h, i, j] = sum_d q[b, h, i, d] * k[b, h / g, j, d] over
// the first kv_len of kv_capacity rows per KV head, f32 accumulation, the f16
// score rounded once.  gqa_pv_matmul (:72-110, metal :323-629):
// out[b, h, i, d] = sum_j p[b, h, i, j] * v[b, h / g, j, d].
//
// In f16 both are bound by HBM (the [B, QH, Q, K] scores are written once
// or read once; Q, K and V are small), in f32 by the f32 matrix cores.  A
// head size of 32..128 in steps of 32 takes the matrix cores
// (v_mfma_f32_32x32x16_f16 for f16):
//  * QK^T computes S^T = K Q^T per wave (32 queries x 128 keys; a
//    workgroup takes 128 queries x 256 keys): the workgroup's 256 key rows are
//    loaded whole into LDS in the order that swaps bits 2 and 3 of the key
//    index, so every lane ends up holding runs of 8 consecutive keys of one
//    query row; each wave stages its score tile in LDS (reusing the key
//    tile's space) and writes 256-byte row segments per 16 lanes, 512 bytes
//    a row per workgroup.  All key tiles of one (head, query tile) run on
//    one XCD.
//  * PV computes O^T = V^T P^T in steps of 128 keys: each wave stages its
//    32 x 128 probabilities in LDS (whole 256-byte row segments per 16
//    lanes), V goes through LDS row-major and its transposed operand comes
//    from ds_read_b64_tr_b16; the next step's loads are in flight meanwhile.
//    Rows on the line grid are walked from a step that differs per
//    workgroup (walk_step), so that the workgroups do not all read one
//    column range at once.
// f32 takes v_mfma_f32_32x32x2_f32 with the same workgroups (the f32
// kernels below); other head sizes take row kernels on the vector ALUs.
#include "common.hpp"
#include "mfma_layout.hpp"

#include <type_traits>

namespace rl {
namespace {

struct GqaParams {
    uint32_t q_heads, group, q_len, kv_len, head_dim;
    uint64_t kv_head_stride;  // elements between KV heads (kv_capacity * head_dim)
    uint32_t q_tiles;         // 128-query tiles per head (MFMA kernels)
    uint32_t k_tiles;         // key tiles per query tile (QK^T: 256 keys in f16, 128 in f32)
    uint32_t k_per_block;     // key tiles one f32 QK^T workgroup computes in turn
    uint32_t k_groups;        // f32 QK^T workgroups per query tile
    uint32_t qk_groups;       // (head, query tile) groups of the f16 QK^T kernel
};

// 16-byte store / load of f16 scores, streamed past the caches (STREAM,
// non-temporal) or plain.  Measured on [15, 4096, kv_len] scores with the
// QK^T key tiles of a query tile on one XCD: QK^T rows that are whole
// 128-byte lines stream (4096 keys: 99 us, plain 122); rows off the line
// grid -- 1000 keys, or 4093 keys, whose rows start off the 16-byte grid --
// store plainly, so the XCD's L2 merges the lines neighbouring key tiles
// share before they reach HBM (1000 keys: 11.7 us; 4093 keys: 126 us,
// streamed 182).  PV reads rows off the line grid plainly (1000 keys 24.6 us,
// streamed 27.1; 4093 keys 124 us).  A template parameter, not a flag: the
// compiler merges the two stores of a run-time choice into one plain store.
template <bool STREAM>
__device__ inline void put_scores(h8* dst, h8 w) {
    if constexpr (STREAM)
        __builtin_nontemporal_store(w, dst);
    else
        *dst = w;
}
template <bool STREAM>
__device__ inline h8 get_scores(const h8* src) {
    if constexpr (STREAM)
        return __builtin_nontemporal_load(src);
    else
        return *src;
}

// The same for 8 scores at any 2-byte alignment: a row of kv_len % 8 != 0
// scores starts (row x kv_len) mod 8 elements past a 16-byte boundary.
// gfx950 runs global memory in unaligned mode, so this is still one 16-byte
// access (split by the hardware where it crosses a line).
typedef half_t h8u __attribute__((ext_vector_type(8), aligned(2)));
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));  // f32 rows off the grid
template <bool STREAM>
__device__ inline void put_scores_u(half_t* dst, h8 w) {
    const h8u v = w;
    if constexpr (STREAM)
        __builtin_nontemporal_store(v, reinterpret_cast<h8u*>(dst));
    else
        *reinterpret_cast<h8u*>(dst) = v;
}
template <bool STREAM>
__device__ inline h8 get_scores_u(const half_t* src) {
    if constexpr (STREAM)
        return __builtin_nontemporal_load(reinterpret_cast<const h8u*>(src));
    else
        return *reinterpret_cast<const h8u*>(src);
}

__device__ inline uint32_t kv_head_of(uint32_t bh, const GqaParams& p) {
    const uint32_t kv_heads = p.q_heads / p.group;
    return (bh / p.q_heads) * kv_heads + (bh % p.q_heads) / p.group;
}

// ------------------------------------------------------------ QK^T, MFMA

// Workgroup = 128 queries x 256 keys of one head; wave w = queries 32 (w % 4)
// .. + 31 x keys 128 (w / 4) .. + 127.  The workgroup writes 128 rows x 512
// bytes of scores: HBM takes the [15, 4096, 4096] tensor in that pattern at
// ~83 us, against ~90 us as 128 rows x 256 bytes (a write-pattern probe of
// the same shapes).  The 256 key rows go to LDS once for the four query
// quarters; after the products the waves stage their score tiles in the
// same LDS (a barrier between), which keeps a workgroup at 70 KB.
// Rows of kv_len % 8 != 0 scores start off the 16-byte grid; their 8-score
// chunks go out as unaligned 16-byte stores (put_scores_u), and a row's last
// partial chunk element by element.
template <int NT, bool STREAM>
__global__ __launch_bounds__(512) void k_gqa_qk_mfma(const half_t* __restrict__ q,
                                                     const half_t* __restrict__ k,
                                                     half_t* __restrict__ out, GqaParams p) {
    constexpr int D = 32 * NT;
    constexpr int DC = D / 16;
    constexpr int TS = 128 + 8;  // LDS row stride (halves) of a wave's 32 x 128 score tile
    constexpr int KS = D + 8;    // LDS row stride (halves) of the key tile
    constexpr int ROW_CHUNKS = D / 8;
    constexpr int KEY_HALVES = 256 * KS;
    constexpr int LDS_HALVES = KEY_HALVES > 8 * 32 * TS ? KEY_HALVES : 8 * 32 * TS;
    __shared__ __align__(16) half_t lds[LDS_HALVES];
    half_t* const ks = lds;  // the key tile, then (after a barrier) the eight score tiles
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t col = lane % 32;
    const uint32_t hs = lane / 32;
    // block = (head, 128-query tile, 256-key tile).  Hardware block b runs on
    // XCD b mod 8.  XCD x takes a contiguous run of (head, query tile) groups
    // -- consecutive heads, which share KV heads -- with all their key tiles:
    // the cache lines that neighbouring key tiles share (rows off the line
    // grid) are merged in one L2, a group's queries and a KV head's keys are
    // fetched into few L2s.  The grid is padded to whole runs per XCD.
    const uint32_t xcd = blockIdx.x % 8, xi = blockIdx.x / 8;
    const uint32_t per_xcd = (p.qk_groups + 7) / 8;
    const uint32_t group = xcd * per_xcd + xi / p.k_tiles;
    if (group >= p.qk_groups) return;  // padding (the whole block)
    const uint32_t kt_blk = xi % p.k_tiles;
    const uint32_t qt = group % p.q_tiles;
    const uint32_t bh = group / p.q_tiles;
    const uint32_t q0 = qt * 128 + (wave % 4) * 32;
    const half_t* kh = k + uint64_t(kv_head_of(bh, p)) * p.kv_head_stride;
    const uint32_t kblock = kt_blk * 256;
    const uint32_t kbase = kblock + (wave / 4) * 128;  // this wave's first key
    // this wave's queries first, so their loads overlap the key tile's; a
    // query past q_len reads row 0 (its scores are not stored)
    const uint32_t qi = q0 + col;
    const bool q_valid = qi < p.q_len;
    h8 qf[DC];
    const half_t* qrow = q + (uint64_t(bh) * p.q_len + (q_valid ? qi : 0)) * D + 8 * hs;
#pragma unroll
    for (int c = 0; c < DC; ++c) qf[c] = *reinterpret_cast<const h8*>(qrow + 16 * c);
    // the block's 256 key rows -> LDS, whole rows per ROW_CHUNKS lanes; key
    // row j goes to LDS row perm32(j) of its 32-row group, so that the S^T
    // operand of lane i is row i.  Keys past kv_len read row kv_len - 1
    // (their scores are not stored).
#pragma unroll
    for (int li = 0; li < 256 * ROW_CHUNKS / 512; ++li) {
        const uint32_t chunk = threadIdx.x + 512 * li;
        const uint32_t j = chunk / ROW_CHUNKS;
        const uint32_t d0 = (chunk % ROW_CHUNKS) * 8;
        const uint32_t key = min(kblock + j, p.kv_len - 1);
        *reinterpret_cast<h8*>(ks + ((j & ~31u) | perm32(j & 31u)) * KS + d0) =
            *reinterpret_cast<const h8*>(kh + uint64_t(key) * D + d0);
    }
    __syncthreads();
    const bool active = q0 < p.q_len && kbase < p.kv_len;
    const uint32_t keys_here = kbase < p.kv_len ? min(128u, p.kv_len - kbase) : 0u;
    // the scores, rounded to f16 as each 32-key tile completes: lane (query
    // col, hs) holds keys 32 t + 16 half + 8 hs + 0..7 in sh[t][half]
    h8 sh[4][2];
    if (active) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // four 32-key tiles
            const half_t* krow = ks + ((wave / 4) * 128 + t * 32 + col) * KS + 8 * hs;
            f32x16 sc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[r] = 0.0f;
#pragma unroll
            for (int c = 0; c < DC; ++c)
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    *reinterpret_cast<const h8*>(krow + 16 * c), qf[c], sc, 0, 0, 0);
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int e = 0; e < 8; ++e) sh[t][half][e] = half_t(sc[8 * half + e]);
        }
    }
    __syncthreads();  // every wave's key reads are done: the LDS takes the score tiles
    if (!active) return;  // (no barrier below)
    half_t* my = lds + wave * 32 * TS;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int half = 0; half < 2; ++half)
            *reinterpret_cast<h8*>(my + col * TS + t * 32 + 16 * half + 8 * hs) = sh[t][half];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // rows of the tile to memory: 16 lanes per 256-byte row segment.  A
    // 16-byte LDS read serves 32 lanes at once over 128 dword banks, so the
    // two rows lanes 0-31 (and 32-63) read must lie 64 dwords apart modulo
    // 128: at a row stride of 68 dwords (136 halves, which keeps the MFMA
    // layout writes above conflict-free) that is rows 16 apart.  Instruction
    // i reads rows 2i, 2i + 16 (lanes 0-31) and 2i + 1, 2i + 17 (lanes 32-63).
    const uint32_t rlane = (lane / 32) + 16 * ((lane / 16) % 2);
    if (keys_here == 128 && q0 + 31 < p.q_len) {
        // A whole tile (the common case): every LDS read, then every store,
        // with no branch between them (under per-store branches the compiler
        // waited for each read before its store).
        h8 w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            w[i] = *reinterpret_cast<const h8*>(my + (2 * i + rlane) * TS + (lane % 16) * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t r = 2 * i + rlane;
            half_t* dst = out + (uint64_t(bh) * p.q_len + q0 + r) * p.kv_len + kbase +
                          (lane % 16) * 8;
            put_scores_u<STREAM>(dst, w[i]);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t r = 2 * i + rlane;  // tile row (query q0 + r)
        const uint32_t c8 = (lane % 16) * 8;   // first key of this lane's 8
        if (q0 + r >= p.q_len || c8 >= keys_here) continue;
        const h8 w = *reinterpret_cast<const h8*>(my + r * TS + c8);
        half_t* dst = out + (uint64_t(bh) * p.q_len + q0 + r) * p.kv_len + kbase + c8;
        if (c8 + 8 <= keys_here) {
            put_scores_u<STREAM>(dst, w);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (c8 + e < keys_here) dst[e] = w[e];
        }
    }
}

// -------------------------------------------------------------- P V, MFMA

// Step i of a P V workgroup's walk over its `steps` key steps.  With ROTATE,
// workgroup b starts at step b mod steps and wraps: in key order every
// resident workgroup reads the same 256-byte column range of its
// probability rows at once, which rows 4 or 8 KB apart (2048 or 4096 f16
// keys) alias onto few HBM channels once about two workgroups a CU are in
// flight ([15, 4096, 4096] x [5, 4096, 64] f16: 100 us in key order, 88 us
// rotated; 32 heads x [2048, 4096]: 120 against 99 us).  Other row strides,
// and grids of fewer workgroups, walk faster in key order (15 heads x
// [2048, 4096]: 60 against 68.5 us; [4608, 4608]: 145 against 165 us).
// Each output is still one fixed-order f32 sum (its order depends only on
// the workgroup), so results repeat exactly from run to run; sums of exactly
// representable products do not depend on the order at all.
template <bool ROTATE>
__device__ inline uint32_t walk_step(uint32_t i, uint32_t steps) {
    if constexpr (!ROTATE) return i;
    const uint32_t s = i + blockIdx.x % steps;
    return s >= steps ? s - steps : s;
}

// Rows of kv_len % 8 != 0 probabilities start off the 16-byte grid; their
// chunks are read as unaligned 16-byte loads (get_scores_u), a row's last
// partial chunk element by element.  STREAM: non-temporal loads (rows on
// the 128-byte line grid only); ROTATE: the staggered walk (walk_step).
template <int NT, bool STREAM, bool ROTATE>
__global__ __launch_bounds__(256) void k_gqa_pv_mfma(const half_t* __restrict__ probs,
                                                     const half_t* __restrict__ v,
                                                     half_t* __restrict__ out, GqaParams p) {
    constexpr int D = 32 * NT;
    constexpr int BN = 128;               // keys per step
    constexpr int PC = BN / 16;           // 16-key slices per step
    constexpr int VS = v_stride_tr(D);    // LDS row stride of V
    constexpr int PS = BN + 8;            // LDS row stride of a wave's 32 x 128 probability tile
    constexpr int LOADS = BN * D / 8 / 256;
    constexpr int ROW_CHUNKS = D / 8;
    __shared__ __align__(16) half_t vs[BN * VS];
    __shared__ __align__(16) half_t pt[4][32 * PS];
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t col = lane % 32;
    const uint32_t hs = lane / 32;
    const uint32_t qt = blockIdx.x % p.q_tiles;
    const uint32_t bh = blockIdx.x / p.q_tiles;
    const uint32_t q0 = qt * 128 + wave * 32;
    const half_t* vh = v + uint64_t(kv_head_of(bh, p)) * p.kv_head_stride;
    const half_t* pbase = probs + uint64_t(bh) * p.q_len * p.kv_len;
    const uint32_t tr_off = (8 * (lane / 32) + (lane % 16) / 4) * VS + 16 * ((lane / 16) % 2) +
                            4 * (lane % 4);
    half_t* my = pt[wave];
    constexpr int P_LOADS = 8;
    // this wave's 32 x 128 probabilities of step blk, whole 256-byte row
    // segments per 16 lanes (rows past q_len and keys past kv_len as zeros)
    auto load_p = [&](uint32_t blk, h8 (&pr)[P_LOADS]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t r = i * 4 + lane / 16;
            const uint32_t kb = blk * BN + (lane % 16) * 8;
            const half_t* src = pbase + uint64_t(q0 + r) * p.kv_len + kb;
            if (q0 + r < p.q_len && kb + 8 <= p.kv_len) {
                pr[i] = get_scores_u<STREAM>(src);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    pr[i][e] = (q0 + r < p.q_len && kb + e < p.kv_len) ? src[e] : half_t(0.0f);
            }
        }
    };
    auto store_p = [&](uint32_t blk, const h8 (&pr)[P_LOADS]) {
        (void)blk;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<h8*>(my + (i * 4 + lane / 16) * PS + (lane % 16) * 8) = pr[i];
    };
    auto load_v = [&](uint32_t blk, h8 (&vr)[LOADS]) {
#pragma unroll
        for (int li = 0; li < LOADS; ++li) {
            const uint32_t chunk = threadIdx.x + 256 * li;
            const uint32_t gk = blk * BN + chunk / ROW_CHUNKS;
            const uint32_t d0 = (chunk % ROW_CHUNKS) * 8;
            const h8 zero = {};
            vr[li] = gk < p.kv_len ? *reinterpret_cast<const h8*>(vh + uint64_t(gk) * D + d0)
                                   : zero;
        }
    };
    auto store_v = [&](const h8 (&vr)[LOADS]) {
#pragma unroll
        for (int li = 0; li < LOADS; ++li) {
            const uint32_t chunk = threadIdx.x + 256 * li;
            *reinterpret_cast<h8*>(vs + (chunk / ROW_CHUNKS) * VS + (chunk % ROW_CHUNKS) * 8) =
                vr[li];
        }
    };

    f32x16 o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;

    const uint32_t blocks = (p.kv_len + BN - 1) / BN;
    h8 pnext[P_LOADS], vnext[LOADS];
    load_p(walk_step<ROTATE>(0, blocks), pnext);
    load_v(walk_step<ROTATE>(0, blocks), vnext);
    store_p(0, pnext);
    store_v(vnext);
    __syncthreads();
    for (uint32_t blk = 0; blk < blocks; ++blk) {
        const bool more = blk + 1 < blocks;
        if (more) {  // next step's operands in flight during this step's products
            load_p(walk_step<ROTATE>(blk + 1, blocks), pnext);
            load_v(walk_step<ROTATE>(blk + 1, blocks), vnext);
        }
#pragma unroll
        for (int c = 0; c < PC; ++c) {
            // P^T operand: keys 16 c + 8 hs + 0..7 of query row col
            const h8 pb = *reinterpret_cast<const h8*>(my + col * PS + 16 * c + 8 * hs);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const half_t* vsrc = vs + tr_off + 16 * c * VS + 32 * t;
                const h4 lo = lds_read_transposed(vsrc);
                const h4 hi = lds_read_transposed(vsrc + 4 * VS);
                const h8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[t], 0, 0, 0);
            }
        }
        if (more) {
            __syncthreads();
            store_p(blk + 1, pnext);
            store_v(vnext);
            __syncthreads();
        }
    }
    const uint32_t qi = q0 + col;
    if (qi < p.q_len) {
        half_t* orow = out + (uint64_t(bh) * p.q_len + qi) * D + 4 * hs;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                h4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = half_t(o[t][4 * g + e]);
                *reinterpret_cast<h4*>(orow + t * 32 + 8 * g) = w;
            }
        }
    }
}

// ----------------------------------------------------- f32, matrix cores

// QK^T in f32 (v_mfma_f32_32x32x2_f32, exact f32 products; bound by the
// f32 matrix cores): workgroup = (head, 128 queries, run of k_per_block
// 128-key tiles), wave = 32 queries.  The queries stay in registers for the
// whole run; key tiles pass through registers into one of two LDS buffers
// (tile t + 1 loads while tile t is multiplied), in key order at a stride of
// 2 mod 64 floats (every operand read on its own bank).  Each lane stores
// its result registers directly, four consecutive keys per 16-byte store: a
// row receives 32-byte pieces that the L2 merges into whole lines.  VEC:
// score rows on the 16-byte grid (kv_len % 4 == 0); otherwise the stores
// are unaligned 16-byte stores, a row's last partial group element-wise.
template <int NT, bool VEC>
__global__ __launch_bounds__(256) void k_gqa_qk_mfma_f32(const float* __restrict__ q,
                                                         const float* __restrict__ k,
                                                         float* __restrict__ out, GqaParams p) {
    constexpr int D = 32 * NT;
    constexpr int DS = D / 2;  // MFMA steps over the head
    constexpr int KS = f32_stride(D, 2);
    constexpr int ROW_CHUNKS = D / 4;
    constexpr int LOADS = 128 * ROW_CHUNKS / 256;  // 16-byte pieces of a key tile per thread
    __shared__ __align__(16) float ks[2][128 * KS];
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t col = lane % 32;
    const uint32_t hs = lane / 32;
    const uint32_t kg = blockIdx.x % p.k_groups;
    const uint32_t rest = blockIdx.x / p.k_groups;
    const uint32_t qt = rest % p.q_tiles;
    const uint32_t bh = rest / p.q_tiles;
    const uint32_t q0 = qt * 128 + wave * 32;
    const float* kh = k + uint64_t(kv_head_of(bh, p)) * p.kv_head_stride;
    const uint32_t t_first = kg * p.k_per_block;
    const uint32_t t_end = min(p.k_tiles, t_first + p.k_per_block);

    // keys past kv_len read row kv_len - 1 (their scores are not stored)
    float4 kreg[LOADS];
    auto load_tile = [&](uint32_t t) {
#pragma unroll
        for (int li = 0; li < LOADS; ++li) {
            const uint32_t chunk = threadIdx.x + 256 * li;
            const uint32_t key = min(t * 128 + chunk / ROW_CHUNKS, p.kv_len - 1);
            kreg[li] = *reinterpret_cast<const float4*>(kh + uint64_t(key) * D +
                                                        (chunk % ROW_CHUNKS) * 4);
        }
    };
    auto store_tile = [&](float* dst) {
#pragma unroll
        for (int li = 0; li < LOADS; ++li) {
            const uint32_t chunk = threadIdx.x + 256 * li;
            float* row = dst + (chunk / ROW_CHUNKS) * KS + (chunk % ROW_CHUNKS) * 4;  // 8-byte aligned
            *reinterpret_cast<float2*>(row) = float2{kreg[li].x, kreg[li].y};
            *reinterpret_cast<float2*>(row + 2) = float2{kreg[li].z, kreg[li].w};
        }
    };
    load_tile(t_first);
    // B operand: lane (col, hs) holds elements 2j + hs of its query
    const uint32_t qi = q0 + col;
    const bool q_valid = qi < p.q_len;
    const float* qrow = q + (uint64_t(bh) * p.q_len + (q_valid ? qi : 0)) * D + hs;
    float qf[DS];
#pragma unroll
    for (int j = 0; j < DS; ++j) qf[j] = q_valid ? qrow[2 * j] : 0.0f;
    store_tile(ks[0]);
    __syncthreads();

    float* orow = out + (uint64_t(bh) * p.q_len + (q_valid ? qi : 0)) * p.kv_len;
    for (uint32_t t = t_first; t < t_end; ++t) {
        const uint32_t buf = (t - t_first) % 2;
        if (t + 1 < t_end) load_tile(t + 1);
        if (q0 < p.q_len) {
#pragma unroll
            for (int st = 0; st < 4; ++st) {  // four 32-key sub-tiles
                const uint32_t k0 = t * 128 + st * 32;
                const float* krow = ks[buf] + (st * 32 + col) * KS + hs;
                f32x16 s;
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
                for (int j = 0; j < DS; ++j)
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(krow[2 * j], qf[j], s, 0, 0, 0);
                if (!q_valid) continue;
                // register 4g + e holds key k0 + 8g + 4hs + e; rows of
                // kv_len % 4 != 0 scores start off the 16-byte grid and take
                // unaligned 16-byte stores
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint32_t key = k0 + 8 * g + 4 * hs;
                    const f32x4 w = {s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]};
                    if constexpr (VEC) {  // kv_len % 4 == 0: a group is whole or past the end
                        if (key < p.kv_len) *reinterpret_cast<f32x4*>(orow + key) = w;
                    } else if (key + 4 <= p.kv_len) {
                        *reinterpret_cast<f32x4u*>(orow + key) = w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (key + e < p.kv_len) orow[key + e] = s[4 * g + e];
                    }
                }
            }
        }
        if (t + 1 < t_end) store_tile(ks[buf ^ 1]);  // read during step t - 1, before its barrier
        __syncthreads();
    }
}

// P V in f32: workgroup = (head, 128 queries), keys in steps of 64.  Each
// wave stages its 32 x 64 probabilities in LDS (whole 256-byte row segments
// per 16 lanes) at a row stride of 2 mod 64, so that lane (col, hs) reads the
// probability of key 2s + hs of its query -- the B operand of the step over
// keys 2s, 2s + 1 -- on its own bank; V rows at 32 mod 64 floats.  The next
// step's operands are in flight during this step's products.  VEC:
// probability rows on the 16-byte grid (streamed loads); otherwise plain
// unaligned 16-byte loads, a row's last partial group element-wise.
template <int NT, bool VEC>
__global__ __launch_bounds__(256) void k_gqa_pv_mfma_f32(const float* __restrict__ probs,
                                                         const float* __restrict__ v,
                                                         float* __restrict__ out, GqaParams p) {
    constexpr int D = 32 * NT;
    constexpr int BN = 64;                      // keys per step
    constexpr int VS = f32_stride(D, 32);       // LDS row stride of V
    constexpr int PS = f32_stride(BN, 2);       // LDS row stride of a wave's probabilities
    constexpr int ROW_CHUNKS = D / 4;
    constexpr int LOADS = BN * ROW_CHUNKS / 256;
    __shared__ __align__(16) float vs[BN * VS];
    __shared__ __align__(16) float pt[4][32 * PS];
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t col = lane % 32;
    const uint32_t hs = lane / 32;
    const uint32_t qt = blockIdx.x % p.q_tiles;
    const uint32_t bh = blockIdx.x / p.q_tiles;
    const uint32_t q0 = qt * 128 + wave * 32;
    const float* vh = v + uint64_t(kv_head_of(bh, p)) * p.kv_head_stride;
    const float* pbase = probs + uint64_t(bh) * p.q_len * p.kv_len;
    float* my = pt[wave];

    // rows past q_len and keys past kv_len as zeros
    auto load_p = [&](uint32_t blk, f32x4 (&pr)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t r = i * 4 + lane / 16;
            const uint32_t kb = blk * BN + (lane % 16) * 4;
            const float* src = pbase + uint64_t(q0 + r) * p.kv_len + kb;
            if constexpr (VEC) {  // kv_len % 4 == 0: a group is whole or past the end
                if (q0 + r < p.q_len && kb < p.kv_len)
                    pr[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src));
                else
                    pr[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            } else if (q0 + r < p.q_len && kb + 4 <= p.kv_len) {
                pr[i] = *reinterpret_cast<const f32x4u*>(src);  // a row off the 16-byte grid
            } else {
                const bool row = q0 + r < p.q_len;
                pr[i] = f32x4{row && kb < p.kv_len ? src[0] : 0.0f,
                              row && kb + 1 < p.kv_len ? src[1] : 0.0f,
                              row && kb + 2 < p.kv_len ? src[2] : 0.0f,
                              row && kb + 3 < p.kv_len ? src[3] : 0.0f};
            }
        }
    };
    auto store_p = [&](const f32x4 (&pr)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float* dst = my + (i * 4 + lane / 16) * PS + (lane % 16) * 4;  // 8-byte aligned
            *reinterpret_cast<float2*>(dst) = float2{pr[i][0], pr[i][1]};
            *reinterpret_cast<float2*>(dst + 2) = float2{pr[i][2], pr[i][3]};
        }
    };
    auto load_v = [&](uint32_t blk, float4 (&vr)[LOADS]) {
#pragma unroll
        for (int li = 0; li < LOADS; ++li) {
            const uint32_t chunk = threadIdx.x + 256 * li;
            const uint32_t gk = blk * BN + chunk / ROW_CHUNKS;
            const uint32_t d0 = (chunk % ROW_CHUNKS) * 4;
            vr[li] = gk < p.kv_len
                         ? *reinterpret_cast<const float4*>(vh + uint64_t(gk) * D + d0)
                         : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    auto store_v = [&](const float4 (&vr)[LOADS]) {
#pragma unroll
        for (int li = 0; li < LOADS; ++li) {
            const uint32_t chunk = threadIdx.x + 256 * li;
            *reinterpret_cast<float4*>(vs + (chunk / ROW_CHUNKS) * VS + (chunk % ROW_CHUNKS) * 4) =
                vr[li];
        }
    };

    f32x16 o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;

    const uint32_t blocks = (p.kv_len + BN - 1) / BN;
    f32x4 pnext[8];
    float4 vnext[LOADS];
    load_p(0, pnext);
    load_v(0, vnext);
    store_p(pnext);
    store_v(vnext);
    __syncthreads();
    for (uint32_t blk = 0; blk < blocks; ++blk) {
        const bool more = blk + 1 < blocks;
        if (more) {
            load_p(blk + 1, pnext);
            load_v(blk + 1, vnext);
        }
        const float* prow = my + col * PS + hs;
        const float* vcol = vs + hs * VS + col;
#pragma unroll
        for (int s = 0; s < BN / 2; ++s) {
            const float pb = prow[2 * s];  // P of key 2s + hs
#pragma unroll
            for (int t = 0; t < NT; ++t)
                o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vcol[2 * s * VS + 32 * t], pb, o[t],
                                                             0, 0, 0);
        }
        if (more) {
            __syncthreads();
            store_p(pnext);
            store_v(vnext);
            __syncthreads();
        }
    }
    const uint32_t qi = q0 + col;
    if (qi < p.q_len) {
        // register r of tile t: element 32t + 8(r / 4) + 4hs + r % 4
        float* orow = out + (uint64_t(bh) * p.q_len + qi) * D + 4 * hs;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(orow + 32 * t + 8 * g) =
                    float4{o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]};
    }
}

// ------------------------------------------------------------ row kernels

// QK^T: one workgroup per (query row, 256 keys); the query row is kept in
// LDS as f32 and each thread forms one dot product in head order.
template <typename T>
__global__ __launch_bounds__(256) void k_gqa_qk_rows(const T* __restrict__ q,
                                                     const T* __restrict__ k,
                                                     T* __restrict__ out, GqaParams p,
                                                     uint32_t key_blocks) {
    extern __shared__ float qs[];
    const uint64_t row = blockIdx.x / key_blocks;  // (b * QH + h) * q_len + i
    const uint32_t key = (blockIdx.x % key_blocks) * 256 + threadIdx.x;
    const uint32_t bh = uint32_t(row / p.q_len);
    const uint32_t D = p.head_dim;
    for (uint32_t d = threadIdx.x; d < D; d += 256) qs[d] = to_float(q[row * D + d]);
    __syncthreads();
    if (key >= p.kv_len) return;
    const T* krow = k + uint64_t(kv_head_of(bh, p)) * p.kv_head_stride + uint64_t(key) * D;
    float sum = 0.0f;
    for (uint32_t d = 0; d < D; ++d) sum += qs[d] * to_float(krow[d]);
    out[row * p.kv_len + key] = from_float<T>(sum);
}

// P V: one workgroup per query row; the probabilities are kept in LDS as
// f32 in chunks of 1024 keys, each thread owns output elements d and sums
// over the keys in order.
template <typename T>
__global__ __launch_bounds__(256) void k_gqa_pv_rows(const T* __restrict__ probs,
                                                     const T* __restrict__ v,
                                                     T* __restrict__ out, GqaParams p) {
    constexpr uint32_t CHUNK = 1024;
    __shared__ float ps[CHUNK];
    const uint64_t row = blockIdx.x;
    const uint32_t bh = uint32_t(row / p.q_len);
    const uint32_t D = p.head_dim;
    const T* vh = v + uint64_t(kv_head_of(bh, p)) * p.kv_head_stride;
    const T* prow = probs + row * p.kv_len;
    constexpr int DMAX = 4;  // head elements per thread (head sizes up to 1024)
    float acc[DMAX] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t c0 = 0; c0 < p.kv_len; c0 += CHUNK) {
        const uint32_t n = min(CHUNK, p.kv_len - c0);
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < n; j += 256) ps[j] = to_float(prow[c0 + j]);
        __syncthreads();
        for (uint32_t j = 0; j < n; ++j) {
            const float pj = ps[j];
            const T* vrow = vh + uint64_t(c0 + j) * D;
#pragma unroll
            for (int e = 0; e < DMAX; ++e) {
                const uint32_t d = threadIdx.x + 256 * e;
                if (d < D) acc[e] += pj * to_float(vrow[d]);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < DMAX; ++e) {
        const uint32_t d = threadIdx.x + 256 * e;
        if (d < D) out[row * D + d] = from_float<T>(acc[e]);
    }
}

// ------------------------------------------------------------ validation

struct GqaShape {
    uint64_t batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity;
};

// gqa_matmul.rs: validate_head_groups (:174-182), then the u32 limits of
// dispatch (:192-212).  Added: non-zero sizes (Shape::new, src/tensor/
// shape.rs:9-23), kv_capacity >= kv_len and exact buffer lengths.
rl_status validate_gqa(const char* op, const rl_buffer* left, const char* left_name,
                       uint64_t left_len, const rl_buffer* right, const GqaShape& s,
                       uint64_t es) {
    if (rl_status st = check_buffer(left, left_name)) return st;
    if (rl_status st = check_buffer(right, op[0] == 'Q' ? "key" : "value")) return st;
    if (s.batch == 0 || s.q_heads == 0 || s.q_len == 0 || s.kv_len == 0 || s.head_dim == 0)
        return fail(RL_ERR_INVALID_SHAPE, "GQA %s dimensions must be greater than zero", op);
    if (s.kv_heads == 0 || s.q_heads % s.kv_heads != 0)
        return fail(RL_ERR_MODEL_FORMAT, "Q heads %llu must be divisible by non-zero KV heads %llu",
                    (unsigned long long)s.q_heads, (unsigned long long)s.kv_heads);
    if (s.q_heads > UINT32_MAX || s.kv_heads > UINT32_MAX || s.q_len > UINT32_MAX ||
        s.kv_len > UINT32_MAX || s.head_dim > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "GQA dimension exceeds u32");
    if (s.kv_capacity > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "GQA KV capacity exceeds u32");
    if (s.batch > UINT64_MAX / s.q_heads)
        return fail(RL_ERR_INVALID_SHAPE, "GQA batch × query-head count overflow");
    if (s.kv_capacity < s.kv_len)
        return fail(RL_ERR_INVALID_SHAPE, "KV capacity %llu is smaller than the key length %llu",
                    (unsigned long long)s.kv_capacity, (unsigned long long)s.kv_len);
    const double kv_elems = double(s.batch) * double(s.kv_heads) * double(s.kv_capacity) *
                            double(s.head_dim);
    if (double(left_len) > double(UINT64_MAX / 16) || kv_elems > double(UINT64_MAX / 16))
        return fail(RL_ERR_INVALID_SHAPE, "GQA %s operands are too large", op);
    const uint64_t kvn = s.batch * s.kv_heads * s.kv_capacity * s.head_dim;
    if (left->len != left_len || left->byte_len != left_len * es)
        return fail(RL_ERR_INVALID_SHAPE, "%s buffer has %llu elements, expected %llu", left_name,
                    (unsigned long long)left->len, (unsigned long long)left_len);
    if (right->len != kvn || right->byte_len != kvn * es)
        return fail(RL_ERR_INVALID_SHAPE, "%s buffer has %llu elements, expected %llu",
                    op[0] == 'Q' ? "key" : "value", (unsigned long long)right->len,
                    (unsigned long long)kvn);
    if (s.batch * s.q_heads * s.q_len > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "GQA row count exceeds u32");
    return RL_OK;
}

GqaParams params_of(const GqaShape& s) {
    GqaParams p{};
    p.q_heads = uint32_t(s.q_heads);
    p.group = uint32_t(s.q_heads / s.kv_heads);
    p.q_len = uint32_t(s.q_len);
    p.kv_len = uint32_t(s.kv_len);
    p.head_dim = uint32_t(s.head_dim);
    p.kv_head_stride = s.kv_capacity * s.head_dim;
    return p;
}

template <typename T>
bool use_mfma(const GqaShape& s, const void* a, const void* b, const void* o) {
    return s.head_dim % 32 == 0 && s.head_dim <= 128 && aligned_to(a, 16) && aligned_to(b, 16) &&
           aligned_to(o, 16);
}

template <typename T>
rl_status qk_entry(rl_context* ctx, const char* name, const rl_buffer* q, const rl_buffer* k,
                   const GqaShape& s, const rl_buffer* out) {
    const uint64_t qn = s.batch * s.q_heads * s.q_len * s.head_dim;
    if (rl_status st = validate_gqa("QK", q, "query", qn, k, s, sizeof(T))) return st;
    const double on = double(s.batch) * double(s.q_heads) * double(s.q_len) * double(s.kv_len);
    if (on > double(UINT64_MAX / 16))
        return fail(RL_ERR_INVALID_SHAPE, "GQA QK output is too large");
    if (rl_status st = check_output(out, s.batch * s.q_heads * s.q_len * s.kv_len, sizeof(T),
                                    "GQA QK"))
        return st;
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    GqaParams p = params_of(s);
    const T* qd = static_cast<const T*>(q->data);
    const T* kd = static_cast<const T*>(k->data);
    T* od = static_cast<T*>(out->data);
    const uint64_t heads = s.batch * s.q_heads;
    if constexpr (std::is_same<T, half_t>::value) {
        if (use_mfma<T>(s, qd, kd, od)) {
            // 128-query x 256-key workgroups; one XCD per (head, query tile)
            // group, the grid padded to 8 runs
            p.q_tiles = uint32_t(ceil_div(s.q_len, 128));
            p.k_tiles = uint32_t(ceil_div(s.kv_len, 256));
            const uint64_t groups = heads * p.q_tiles;
            const uint64_t xgrid = ceil_div(groups, 8) * 8 * p.k_tiles;
            if (xgrid > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "GQA QK grid exceeds u32");
            p.qk_groups = uint32_t(groups);
            const dim3 g(static_cast<unsigned>(xgrid)), b(512);
            const bool lines = s.kv_len % 64 == 0;  // score rows are whole 128-byte lines
#define RL_QK(NT)                                                                      \
    do {                                                                               \
        if (lines)                                                                     \
            RL_LAUNCH(ctx, (k_gqa_qk_mfma<NT, true>), g, b, qd, kd, od, p);            \
        else                                                                           \
            RL_LAUNCH(ctx, (k_gqa_qk_mfma<NT, false>), g, b, qd, kd, od, p);           \
    } while (0)
            switch (s.head_dim / 32) {
                case 1: RL_QK(1); break;
                case 2: RL_QK(2); break;
                case 3: RL_QK(3); break;
                default: RL_QK(4); break;
            }
#undef RL_QK
            return after_launch(ctx, name);
        }
    } else {
        if (use_mfma<T>(s, qd, kd, od)) {
            p.q_tiles = uint32_t(ceil_div(s.q_len, 128));
            p.k_tiles = uint32_t(ceil_div(s.kv_len, 128));
            // Workgroups walk runs of key tiles; a query tile's keys split
            // over several only when the query tiles alone do not fill the
            // resident workgroups (two per CU up to head size 64, one above).
            const uint64_t base = heads * p.q_tiles;
            const uint64_t resident = s.head_dim <= 64 ? 512 : 256;
            const uint64_t groups =
                std::min<uint64_t>(p.k_tiles, std::max<uint64_t>(1, resident / base));
            p.k_per_block = uint32_t(ceil_div(p.k_tiles, groups));
            p.k_groups = uint32_t(ceil_div(p.k_tiles, p.k_per_block));
            const uint64_t grid = base * p.k_groups;
            if (grid > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "GQA QK grid exceeds u32");
            const dim3 g(static_cast<unsigned>(grid)), b(256);
            // score rows on the 16-byte grid (kv_len % 4 == 0) or off it
            const bool vec = s.kv_len % 4 == 0;
#define RL_QK32(NT)                                                                    \
    do {                                                                               \
        if (vec)                                                                       \
            RL_LAUNCH(ctx, (k_gqa_qk_mfma_f32<NT, true>), g, b, qd, kd, od, p);        \
        else                                                                           \
            RL_LAUNCH(ctx, (k_gqa_qk_mfma_f32<NT, false>), g, b, qd, kd, od, p);       \
    } while (0)
            switch (s.head_dim / 32) {
                case 1: RL_QK32(1); break;
                case 2: RL_QK32(2); break;
                case 3: RL_QK32(3); break;
                default: RL_QK32(4); break;
            }
#undef RL_QK32
            return after_launch(ctx, name);
        }
    }
    const uint64_t key_blocks = ceil_div(s.kv_len, 256);
    const uint64_t grid = heads * s.q_len * key_blocks;
    if (grid > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "GQA QK grid exceeds u32");
    if (s.head_dim > 16384) return fail(RL_ERR_INVALID_SHAPE, "GQA QK head size exceeds 16384");
    {
        const dim3 g(static_cast<unsigned>(grid)), b(256);
        const size_t lds = s.head_dim * sizeof(float);
        if (rl_status st = flush_fused(ctx)) return st;
        if (ctx->timed_start != nullptr) {
            hipExtLaunchKernelGGL((k_gqa_qk_rows<T>), g, b, lds, ctx->stream, ctx->timed_start,
                                  ctx->timed_stop, 0, qd, kd, od, p, uint32_t(key_blocks));
            ctx->timed_start = nullptr;
            ctx->timed_stop = nullptr;
        } else {
            hipLaunchKernelGGL((k_gqa_qk_rows<T>), g, b, lds, ctx->stream, qd, kd, od, p,
                               uint32_t(key_blocks));
        }
    }
    return after_launch(ctx, name);
}

template <typename T>
rl_status pv_entry(rl_context* ctx, const char* name, const rl_buffer* probs, const rl_buffer* v,
                   const GqaShape& s, const rl_buffer* out) {
    const double pn = double(s.batch) * double(s.q_heads) * double(s.q_len) * double(s.kv_len);
    if (pn > double(UINT64_MAX / 16))
        return fail(RL_ERR_INVALID_SHAPE, "GQA PV operands are too large");
    const uint64_t plen = s.batch * s.q_heads * s.q_len * s.kv_len;
    if (rl_status st = validate_gqa("PV", probs, "probability", plen, v, s, sizeof(T))) return st;
    if (rl_status st = check_output(out, s.batch * s.q_heads * s.q_len * s.head_dim, sizeof(T),
                                    "GQA PV"))
        return st;
    if (s.head_dim > 1024) return fail(RL_ERR_INVALID_SHAPE, "GQA PV head size exceeds 1024");
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    GqaParams p = params_of(s);
    const T* pd = static_cast<const T*>(probs->data);
    const T* vd = static_cast<const T*>(v->data);
    T* od = static_cast<T*>(out->data);
    const uint64_t heads = s.batch * s.q_heads;
    if constexpr (std::is_same<T, half_t>::value) {
        if (use_mfma<T>(s, pd, vd, od)) {
            p.q_tiles = uint32_t(ceil_div(s.q_len, 128));
            const uint64_t grid = heads * p.q_tiles;
            if (grid > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "GQA PV grid exceeds u32");
            const dim3 g(static_cast<unsigned>(grid)), b(256);
            const bool lines = s.kv_len % 64 == 0;  // probability rows are whole 128-byte lines
            // the staggered walk for rows 4 or 8 KB apart with >= 15/8
            // workgroups a CU; streamed loads for line-grid rows when
            // rotating or past kStreamReadBytes of probabilities (measured
            // over 37 shapes)
            const uint64_t row_bytes = s.kv_len * sizeof(T);
            const bool rotate = lines && (row_bytes == 4096 || row_bytes == 8192) &&
                                grid * 8 >= uint64_t(15) * uint64_t(ctx->num_cus);
            const bool stream = lines && (rotate || plen * sizeof(T) > kStreamReadBytes);
#define RL_PV(NT)                                                                      \
    do {                                                                               \
        if (rotate)                                                                    \
            RL_LAUNCH(ctx, (k_gqa_pv_mfma<NT, true, true>), g, b, pd, vd, od, p);      \
        else if (stream)                                                               \
            RL_LAUNCH(ctx, (k_gqa_pv_mfma<NT, true, false>), g, b, pd, vd, od, p);     \
        else                                                                           \
            RL_LAUNCH(ctx, (k_gqa_pv_mfma<NT, false, false>), g, b, pd, vd, od, p);    \
    } while (0)
            switch (s.head_dim / 32) {
                case 1: RL_PV(1); break;
                case 2: RL_PV(2); break;
                case 3: RL_PV(3); break;
                default: RL_PV(4); break;
            }
#undef RL_PV
            return after_launch(ctx, name);
        }
    } else {
        if (use_mfma<T>(s, pd, vd, od)) {
            p.q_tiles = uint32_t(ceil_div(s.q_len, 128));
            const uint64_t grid = heads * p.q_tiles;
            if (grid > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "GQA PV grid exceeds u32");
            const dim3 g(static_cast<unsigned>(grid)), b(256);
            // probability rows on the 16-byte grid (kv_len % 4 == 0) or off it
            const bool vec = s.kv_len % 4 == 0;
#define RL_PV32(NT)                                                                    \
    do {                                                                               \
        if (vec)                                                                       \
            RL_LAUNCH(ctx, (k_gqa_pv_mfma_f32<NT, true>), g, b, pd, vd, od, p);        \
        else                                                                           \
            RL_LAUNCH(ctx, (k_gqa_pv_mfma_f32<NT, false>), g, b, pd, vd, od, p);       \
    } while (0)
            switch (s.head_dim / 32) {
                case 1: RL_PV32(1); break;
                case 2: RL_PV32(2); break;
                case 3: RL_PV32(3); break;
                default: RL_PV32(4); break;
            }
#undef RL_PV32
            return after_launch(ctx, name);
        }
    }
    RL_LAUNCH(ctx, (k_gqa_pv_rows<T>), dim3(static_cast<unsigned>(heads * s.q_len)), dim3(256),
              pd, vd, od, p);
    return after_launch(ctx, name);
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_gqa_qk_matmul_f32(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out) {
    const GqaShape s{batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity};
    return qk_entry<float>(ctx, "gqa_qk_f32", q, k, s, out);
}

rl_status rl_gqa_qk_matmul_f16(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out) {
    const GqaShape s{batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity};
    return qk_entry<half_t>(ctx, "gqa_qk_f16", q, k, s, out);
}

rl_status rl_gqa_pv_matmul_f32(rl_context* ctx, const rl_buffer* probs, const rl_buffer* v,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out) {
    const GqaShape s{batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity};
    return pv_entry<float>(ctx, "gqa_pv_f32", probs, v, s, out);
}

rl_status rl_gqa_pv_matmul_f16(rl_context* ctx, const rl_buffer* probs, const rl_buffer* v,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out) {
    const GqaShape s{batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity};
    return pv_entry<half_t>(ctx, "gqa_pv_f16", probs, v, s, out);
}

}  // extern "C"
