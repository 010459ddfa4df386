// attention.hip -- the attention core of one layer for gfx950.
//
// SelfAttention::attention_core_encode (src/nn/attention.rs:216-247) runs
// four kernels: scores = Q K^T (gqa_qk_*, or batched_matmul when the head
// counts match), attention_scale_mask, softmax_last_dim, and P V (gqa_pv_*).
// The scores make a [B, QH, Q, K] round trip through memory twice.  Here the
// four are one pass ("flash" attention: Dao et al., 2022): each workgroup
// keeps a tile of queries in registers, streams the keys and values of its
// KV head through LDS in blocks of 64, and folds every block into a running
// (max, sum, output) per query, so the scores never leave the chip.
//
// f16 with a head size that is a multiple of 32 (32..128) takes the matrix
// cores (v_mfma_f32_32x32x16_f16, f32 accumulation): per wave 32 queries,
// S^T = K Q^T so that each lane owns one query column and its row statistics
// need one cross-lane exchange; the keys of a 32-key tile are read in an
// order that swaps bits 2 and 3 of the key index, which leaves each lane
// holding eight consecutive keys of P -- exactly the operand layout of the
// P V product, so P goes from registers to the second MFMA without moving.
// K rows are stored in LDS in that key order; V stays row-major and its
// transposed operand comes from the LDS transpose read (ds_read_b64_tr_b16).  Other shapes (f32, odd
// head sizes, up to 512) take a one-wave-per-query kernel on the vector ALUs.
//
// Arithmetic (both kernels): scores are f32 dot products of the (widened)
// inputs; x * scale in f32 and masking as attention_scale_mask.metal:21-41
// (key > start + query is -inf); softmax in f32 with e^x on the hardware
// exp2; the output is sum_j p_j v_j / sum_j p_j in f32, rounded once to the
// output type.  The reference rounds the scores, the scaled scores and the
// probabilities to f16 in between; this pass does not, so it is closer to
// the exact result than the reference's own four calls (the tests bound both
// against float64).  The MFMA kernel feeds P to the second product as f16
// (relative error 2^-11 per probability, inside the same bound).
#include "common.hpp"

#include <cmath>
#include <type_traits>

namespace rl {
namespace {

typedef half_t h8 __attribute__((ext_vector_type(8)));
typedef half_t h4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.44269504088896340736f;

struct AttnParams {
    uint32_t q_heads;      // query heads per batch entry
    uint32_t group;        // query heads per KV head
    uint32_t q_len;
    uint32_t kv_len;
    uint32_t start;        // absolute position of query 0
    uint32_t tiles;        // query tiles per head (MFMA kernel)
    uint32_t pairs;        // workgroups per head (MFMA kernel)
    uint32_t head_dim;
    uint64_t kv_head_stride;  // elements between KV heads (kv_capacity * head_dim)
    float scale;           // attention scale
    float scale_log2;      // scale * log2(e)
};

// ------------------------------------------------------------- MFMA kernel

constexpr int kBlockKeys = 64;

// Key order inside a 32-key tile: row i of the S^T tile holds key
// perm32(i), bits 2 and 3 of i swapped.  With the 32x32 result layout (lane
// l holds column l % 32, rows 8 * (r / 4) + 4 * (l / 32) + r % 4 in register
// r) register r of lane l then holds key 16 * (r / 8) + 8 * (l / 32) + r % 8.
__device__ inline uint32_t perm32(uint32_t i) {
    return (i & ~12u) | ((i & 4u) << 1) | ((i & 8u) >> 1);
}

// ds_read_b64_tr_b16: in each group of 16 lanes, lanes 4j .. 4j + 3 read 8
// bytes each (row j of a 4 x 16 block of halves); lane i of the group
// receives column i of that block, one half from each row.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ inline h4 lds_read_transposed(const half_t* p) {
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(p));
    return __builtin_bit_cast(h4, r);
}

// Rescaling threshold (log2 units): a query's running max m is only moved
// when a block's max exceeds it by more than this, so most blocks skip the
// rescale of the running sum and output; probabilities exp2(t - m) then stay
// below 2^3, well inside f16 and f32 range.
constexpr float kRescaleSlack = 3.0f;

// QW waves of 32 queries each; KSPLIT groups of such waves split the key
// blocks of the tile between them (group g takes blocks g, g + KSPLIT, ...)
// and merge their partial (max, sum, output) through LDS at the end, so a
// tile keeps KSPLIT x QW waves busy.
template <int NT, int QW, int KSPLIT>
__global__ __launch_bounds__(64 * QW * KSPLIT) void k_flash_attention(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    half_t* __restrict__ out, AttnParams p) {
    constexpr int D = 32 * NT;          // head size
    constexpr int DC = D / 16;          // 16-wide slices of a head (MFMA depth)
    constexpr int BN = kBlockKeys;
    // LDS rows: K at a stride of D + 8 halves (a 16-byte read of 8
    // consecutive rows hits 8 distinct bank quads), V at D + 16 (the four
    // rows a transpose read of 16 lanes touches hit 32 distinct banks).
    constexpr int KS = D + 8;
    constexpr int VS = D + 16;
    constexpr int THREADS = 64 * QW * KSPLIT;
    constexpr int BLOCK_CHUNKS = BN * D / 8;           // 16-byte chunks of one K (or V) block
    constexpr int LOADS = BLOCK_CHUNKS * KSPLIT / THREADS;
    constexpr int ROW_CHUNKS = D / 8;
    constexpr int KV_HALVES = BN * KS + BN * VS;       // one block of K and V
    constexpr int MERGE = NT * 16 + 2;                 // floats a lane hands over
    constexpr int LDS_BYTES = KSPLIT * KV_HALVES * 2 > (KSPLIT - 1) * QW * 64 * MERGE * 4
                                  ? KSPLIT * KV_HALVES * 2
                                  : (KSPLIT - 1) * QW * 64 * MERGE * 4;
    static_assert((BLOCK_CHUNKS * KSPLIT) % THREADS == 0, "blocks must split evenly");
    __shared__ __align__(16) unsigned char lds[LDS_BYTES];
    half_t* const kv_lds = reinterpret_cast<half_t*>(lds);

    const uint32_t bh = blockIdx.x / p.pairs;
    const uint32_t pair = blockIdx.x % p.pairs;
    const uint32_t kv_heads = p.q_heads / p.group;
    const uint32_t kv_head = (bh / p.q_heads) * kv_heads + (bh % p.q_heads) / p.group;
    const half_t* kh = k + uint64_t(kv_head) * p.kv_head_stride;
    const half_t* vh = v + uint64_t(kv_head) * p.kv_head_stride;

    const uint32_t wave = threadIdx.x / 64;
    const uint32_t qw = wave % QW;      // which 32 queries of the tile
    const uint32_t sub = wave / QW;     // which share of the key blocks
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t col = lane % 32;     // query column of this lane
    const uint32_t hs = lane / 32;      // which 8 of 16 in an MFMA slice
    const half_t* ks = kv_lds + sub * KV_HALVES;
    const half_t* vs = ks + BN * KS;
    // Transpose reads of V for the A operand of O^T += V^T P^T: lane
    // 16g + 4j + a reads row 8(g / 2) + j (+ 16c + 4e2 for slice c, half e2)
    // at columns 16(g % 2) + 4a (+ 32t for head tile t); the hardware then
    // hands lane 16g + i the column 16(g % 2) + i of those four rows.
    const uint32_t tr_off = (8 * (lane / 32) + (lane % 16) / 4) * VS + 16 * ((lane / 16) % 2) +
                            4 * (lane % 4);

    // The causal tiles of a head are paired (t, tiles - 1 - t) so that every
    // workgroup streams about the same number of key blocks.
    for (int which = 0; which < 2; ++which) {
        const uint32_t tile = which == 0 ? p.tiles - 1 - pair : pair;
        if (which == 1 && tile >= p.tiles - 1 - pair) break;

        const uint32_t q_first = tile * (32 * QW);
        const uint32_t q_last = min(p.q_len, q_first + 32 * QW) - 1;
        const uint32_t keys = min(p.kv_len, p.start + q_last + 1);
        const uint32_t blocks = (keys + BN - 1) / BN;
        const uint32_t steps = (blocks + KSPLIT - 1) / KSPLIT;

        const uint32_t q0 = q_first + qw * 32;
        const bool wave_active = q0 < p.q_len;
        const uint32_t wave_keys =
            wave_active ? min(p.kv_len, p.start + min(q0 + 31, p.q_len - 1) + 1) : 0;
        const uint32_t qi = q0 + col;
        const bool q_valid = qi < p.q_len;
        // Largest key this lane's query sees (padding columns see a few keys
        // too, so their arithmetic stays finite; they are never stored).
        const uint32_t key_limit = min(p.start + qi, p.kv_len - 1);

        h8 qf[DC];
        {
            const half_t* qrow = q + (uint64_t(bh) * p.q_len + (q_valid ? qi : 0)) * D + 8 * hs;
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                if (q_valid) {
                    qf[c] = *reinterpret_cast<const h8*>(qrow + 16 * c);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) qf[c][e] = half_t(0.0f);
                }
            }
        }

        f32x16 o[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
        float m = -INFINITY;  // running max logit, log2 units
        float l = 0.0f;       // this lane's share of the running sum

        h8 kreg[LOADS], vreg[LOADS];
        auto load_step = [&](uint32_t step) {
#pragma unroll
            for (int li = 0; li < LOADS; ++li) {
                const uint32_t chunk = threadIdx.x + THREADS * li;
                const uint32_t blk = step * KSPLIT + chunk / BLOCK_CHUNKS;
                const uint32_t c = chunk % BLOCK_CHUNKS;
                const uint32_t key = blk * BN + c / ROW_CHUNKS;
                const uint32_t d0 = (c % ROW_CHUNKS) * 8;
                if (key < p.kv_len) {
                    kreg[li] = *reinterpret_cast<const h8*>(kh + uint64_t(key) * D + d0);
                    vreg[li] = *reinterpret_cast<const h8*>(vh + uint64_t(key) * D + d0);
                } else {
                    // rows past kv_len are never read (they may hold anything)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        kreg[li][e] = half_t(0.0f);
                        vreg[li][e] = half_t(0.0f);
                    }
                }
            }
        };
        auto store_step = [&]() {
#pragma unroll
            for (int li = 0; li < LOADS; ++li) {
                const uint32_t chunk = threadIdx.x + THREADS * li;
                const uint32_t c = chunk % BLOCK_CHUNKS;
                half_t* kdst = kv_lds + (chunk / BLOCK_CHUNKS) * KV_HALVES;
                half_t* vdst = kdst + BN * KS;
                const uint32_t key = c / ROW_CHUNKS;
                const uint32_t d0 = (c % ROW_CHUNKS) * 8;
                // K row `key` goes to LDS row perm32(key): the S^T operand of
                // lane i is then LDS row i.
                *reinterpret_cast<h8*>(kdst + perm32(key) * KS + d0) = kreg[li];
                *reinterpret_cast<h8*>(vdst + key * VS + d0) = vreg[li];
            }
        };

        load_step(0);
        __syncthreads();  // the previous tile's LDS use is over
        store_step();
        __syncthreads();

        for (uint32_t step = 0; step < steps; ++step) {
            if (step + 1 < steps) load_step(step + 1);
            const uint32_t blk = step * KSPLIT + sub;
            if (blk < blocks && blk * BN < wave_keys) {
                // S^T = K Q^T for two 32-key tiles.
                f32x16 s[2];
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
                    const half_t* krow = ks + (kt * 32 + col) * KS + 8 * hs;
#pragma unroll
                    for (int c = 0; c < DC; ++c)
                        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            *reinterpret_cast<const h8*>(krow + 16 * c), qf[c], s[kt], 0, 0, 0);
                }
                // mask; the block's max raw score of each query
                const uint32_t kbase = blk * BN;
                if (kbase + BN - 1 > p.start + q0 || kbase + BN > p.kv_len) {
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const uint32_t key = kbase + kt * 32 + 16 * (r >> 3) + 8 * hs + (r & 7);
                            if (key > key_limit) s[kt][r] = -INFINITY;
                        }
                }
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; r += 2)
                        mx = fmaxf(mx, fmaxf(s[kt][r], s[kt][r + 1]));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float mx_log2 = mx * p.scale_log2;
                if (__any(mx_log2 > m + kRescaleSlack)) {
                    const float m_new = fmaxf(m, mx_log2);
                    const float alpha = m_new > m ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
                    m = m_new;
                    l *= alpha;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
                }
                // p = 2^(s * scale * log2 e - m); a query that has seen no key
                // yet (m = -inf) has only -inf scores here, and p = 0.
                const float neg_m = m == -INFINITY ? 0.0f : -m;
                float rs = 0.0f;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float e =
                            __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][r], p.scale_log2, neg_m));
                        s[kt][r] = e;
                        rs += e;
                    }
                }
                l += rs;
                // O^T += V^T P^T, 16 keys per MFMA: lane half hs supplies keys
                // 16c + 8hs .. +7, which it holds in registers 8(c%2) .. +7 of tile c/2.
#pragma unroll
                for (int c = 0; c < BN / 16; ++c) {
                    h8 pb;
#pragma unroll
                    for (int e = 0; e < 8; ++e) pb[e] = half_t(s[c >> 1][8 * (c & 1) + e]);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const half_t* vsrc = vs + tr_off + 16 * c * VS + 32 * t;
                        const h4 lo = lds_read_transposed(vsrc);
                        const h4 hi = lds_read_transposed(vsrc + 4 * VS);
                        const h8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[t], 0, 0, 0);
                    }
                }
            }
            __syncthreads();
            if (step + 1 < steps) store_step();
            __syncthreads();
        }

        if constexpr (KSPLIT > 1) {
            // Groups 1.. hand their (max, sum, output) to group 0 through LDS.
            float* mg = reinterpret_cast<float*>(lds);
            if (sub > 0) {
                float* dst = mg + ((sub - 1) * QW * 64 + qw * 64 + lane) * MERGE;
                dst[0] = m;
                dst[1] = l;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dst[2 + 16 * t + r] = o[t][r];
            }
            __syncthreads();
            if (sub == 0) {
#pragma unroll
                for (int g = 1; g < KSPLIT; ++g) {
                    const float* src = mg + ((g - 1) * QW * 64 + qw * 64 + lane) * MERGE;
                    const float m2 = src[0];
                    const float m_tot = fmaxf(m, m2);
                    const float a1 = m_tot > m ? __builtin_amdgcn_exp2f(m - m_tot) : 1.0f;
                    const float a2 = m_tot > m2 ? __builtin_amdgcn_exp2f(m2 - m_tot) : 1.0f;
                    l = l * a1 + src[1] * a2;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            o[t][r] = o[t][r] * a1 + src[2 + 16 * t + r] * a2;
                    m = m_tot;
                }
            }
            __syncthreads();  // the merge area is free again
        }

        const float total = l + __shfl_xor(l, 32, 64);
        const float inv = 1.0f / total;
        if (q_valid && sub == 0) {
            half_t* orow = out + (uint64_t(bh) * p.q_len + qi) * D + 4 * hs;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    h4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = half_t(o[t][4 * g + e] * inv);
                    *reinterpret_cast<h4*>(orow + t * 32 + 8 * g) = w;
                }
            }
        }
    }
}

// ------------------------------------------------- one wave per query row

// Keys are taken 256 at a time: each lane scores four (a full dot product
// over the head, in order), the wave agrees on the new running max, the
// probabilities go to LDS, and the lanes -- now one per output element --
// accumulate the values of those keys.
template <typename T, int DT>
__global__ __launch_bounds__(64) void k_attention_rows(const T* __restrict__ q,
                                                       const T* __restrict__ k,
                                                       const T* __restrict__ v,
                                                       T* __restrict__ out, AttnParams p) {
    constexpr int KEYS = 256;
    __shared__ float qs[64 * DT];
    __shared__ float ps[KEYS];
    const uint32_t lane = threadIdx.x;
    const uint32_t row = blockIdx.x;  // (b * QH + h) * q_len + qi
    const uint32_t bh = row / p.q_len;
    const uint32_t qi = row % p.q_len;
    const uint32_t kv_heads = p.q_heads / p.group;
    const uint32_t kv_head = (bh / p.q_heads) * kv_heads + (bh % p.q_heads) / p.group;
    const uint32_t D = p.head_dim;
    const T* kh = k + uint64_t(kv_head) * p.kv_head_stride;
    const T* vh = v + uint64_t(kv_head) * p.kv_head_stride;
    const T* qrow = q + uint64_t(row) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        const uint32_t d = lane + 64 * t;
        qs[d] = d < D ? to_float(qrow[d]) : 0.0f;
    }
    __syncthreads();

    const uint32_t key_end = min(p.kv_len, p.start + qi + 1);
    float o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = 0.0f;
    float m = -INFINITY;
    float l = 0.0f;  // this lane's share of the sum
    for (uint32_t base = 0; base < key_end; base += KEYS) {
        float s[KEYS / 64];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < KEYS / 64; ++i) {
            const uint32_t key = base + lane + 64 * i;
            s[i] = -INFINITY;
            if (key < key_end) {
                const T* krow = kh + uint64_t(key) * D;
                float dot = 0.0f;
                for (uint32_t d = 0; d < D; ++d) dot += qs[d] * to_float(krow[d]);
                s[i] = dot * p.scale;
            }
            mx = fmaxf(mx, s[i]);
        }
        mx = wave_max(mx);
        const float m_new = fmaxf(m, mx);
        const float alpha = exp_fast(m - m_new);
        m = m_new;
        l *= alpha;
#pragma unroll
        for (int i = 0; i < KEYS / 64; ++i) {
            const float e = exp_fast(s[i] - m_new);
            ps[lane + 64 * i] = e;
            l += e;
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] *= alpha;
        __syncthreads();
        const uint32_t n = min(uint32_t(KEYS), key_end - base);
        for (uint32_t j = 0; j < n; ++j) {
            const float pj = ps[j];
            const T* vrow = vh + uint64_t(base + j) * D;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const uint32_t d = lane + 64 * t;
                if (d < D) o[t] += pj * to_float(vrow[d]);
            }
        }
        __syncthreads();
    }
    const float inv = 1.0f / wave_sum(l);
    T* orow = out + uint64_t(row) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        const uint32_t d = lane + 64 * t;
        if (d < D) orow[d] = from_float<T>(o[t] * inv);
    }
}

// ------------------------------------------------------------ validation

struct AttnShape {
    uint64_t batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity;
};

// The checks of the four calls attention_core_encode makes, in its order:
// gqa_qk_matmul_encode (src/tensor/gqa_matmul.rs:135-176 head groups, the u32
// limits of :192-212), attention_scale_mask (src/ops/attention_scale_mask.rs:
// 120-161), then the buffers (the reference's Tensor sizes).  Added: every
// size is non-zero (Shape::new rejects zero dims, src/tensor/shape.rs:9-23),
// kv_capacity >= kv_len and exact buffer lengths -- rows past a buffer would
// otherwise be read.
rl_status validate_attention(const rl_buffer* q, const rl_buffer* k, const rl_buffer* v,
                             const AttnShape& s, float scale, uint64_t start, uint64_t es) {
    if (rl_status st = check_buffer(q, "query")) return st;
    if (rl_status st = check_buffer(k, "key")) return st;
    if (rl_status st = check_buffer(v, "value")) return st;
    if (s.batch == 0 || s.q_heads == 0 || s.q_len == 0 || s.kv_len == 0 || s.head_dim == 0)
        return fail(RL_ERR_INVALID_SHAPE, "attention dimensions must be greater than zero");
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
    if (!(scale > 0.0f) || scale == INFINITY)
        return fail(RL_ERR_INVALID_SHAPE, "attention scale must be positive and finite, got %g",
                    double(scale));
    if (start > UINT64_MAX - s.q_len)
        return fail(RL_ERR_INVALID_SHAPE, "attention query position overflow");
    if (start + s.q_len > s.kv_len)
        return fail(RL_ERR_INVALID_SHAPE,
                    "attention query range [%llu, %llu) exceeds key length %llu",
                    (unsigned long long)start, (unsigned long long)(start + s.q_len),
                    (unsigned long long)s.kv_len);
    const double q_elems = double(s.batch) * double(s.q_heads) * double(s.q_len) *
                           double(s.head_dim);
    const double kv_elems = double(s.batch) * double(s.kv_heads) * double(s.kv_capacity) *
                            double(s.head_dim);
    if (q_elems > double(UINT64_MAX / 16) || kv_elems > double(UINT64_MAX / 16))
        return fail(RL_ERR_INVALID_SHAPE, "attention operands are too large");
    const uint64_t qn = s.batch * s.q_heads * s.q_len * s.head_dim;
    const uint64_t kvn = s.batch * s.kv_heads * s.kv_capacity * s.head_dim;
    if (q->len != qn || q->byte_len != qn * es)
        return fail(RL_ERR_INVALID_SHAPE, "query buffer has %llu elements, expected %llu",
                    (unsigned long long)q->len, (unsigned long long)qn);
    if (k->len != kvn || k->byte_len != kvn * es)
        return fail(RL_ERR_INVALID_SHAPE, "key buffer has %llu elements, expected %llu",
                    (unsigned long long)k->len, (unsigned long long)kvn);
    if (v->len != kvn || v->byte_len != kvn * es)
        return fail(RL_ERR_INVALID_SHAPE, "value buffer has %llu elements, expected %llu",
                    (unsigned long long)v->len, (unsigned long long)kvn);
    if (s.batch * s.q_heads * s.q_len > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "attention row count exceeds u32");
    return RL_OK;
}

constexpr int kFlashQueryWaves = 4;
constexpr int kFlashKeySplit = 2;

// Which kernel a shape takes: the MFMA kernel for f16 with a head size of
// 32, 64, 96 or 128 and aligned buffers; the row kernel otherwise (head
// sizes up to 512).
template <typename T>
bool use_flash(const AttnShape& s, const void* q, const void* k, const void* v, const void* o) {
    if constexpr (!std::is_same<T, half_t>::value) {
        return false;
    } else {
        return s.head_dim % 32 == 0 && s.head_dim <= 128 && aligned_to(q, 16) &&
               aligned_to(k, 16) && aligned_to(v, 16) && aligned_to(o, 16);
    }
}

template <typename T>
rl_status attention_entry(rl_context* ctx, const char* name, const rl_buffer* q,
                          const rl_buffer* k, const rl_buffer* v, const AttnShape& s,
                          float scale, uint64_t start, const rl_buffer* out) {
    if (rl_status st = validate_attention(q, k, v, s, scale, start, sizeof(T))) return st;
    if (rl_status st = check_output(out, q->len, sizeof(T), "attention")) return st;
    const bool flash = use_flash<T>(s, q->data, k->data, v->data, out->data);
    if (!flash && s.head_dim > 512)
        return fail(RL_ERR_INVALID_SHAPE, "attention head size %llu exceeds 512",
                    (unsigned long long)s.head_dim);
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;

    AttnParams p{};
    p.q_heads = uint32_t(s.q_heads);
    p.group = uint32_t(s.q_heads / s.kv_heads);
    p.q_len = uint32_t(s.q_len);
    p.kv_len = uint32_t(s.kv_len);
    p.start = uint32_t(start);
    p.head_dim = uint32_t(s.head_dim);
    p.kv_head_stride = s.kv_capacity * s.head_dim;
    p.scale = scale;
    p.scale_log2 = scale * kLog2e;
    const T* qd = static_cast<const T*>(q->data);
    const T* kd = static_cast<const T*>(k->data);
    const T* vd = static_cast<const T*>(v->data);
    T* od = static_cast<T*>(out->data);
    const uint64_t heads = s.batch * s.q_heads;

    if constexpr (std::is_same<T, half_t>::value) {
        if (flash) {
            p.tiles = uint32_t(ceil_div(s.q_len, 32 * kFlashQueryWaves));
            p.pairs = (p.tiles + 1) / 2;
            const uint64_t grid = heads * p.pairs;
            if (grid > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "attention grid exceeds u32");
            constexpr int QW = kFlashQueryWaves, KSPLIT = kFlashKeySplit;
            const dim3 g(static_cast<unsigned>(grid)), b(64 * QW * KSPLIT);
            switch (s.head_dim / 32) {
                case 1: RL_LAUNCH(ctx, (k_flash_attention<1, QW, KSPLIT>), g, b, qd, kd, vd, od, p); break;
                case 2: RL_LAUNCH(ctx, (k_flash_attention<2, QW, KSPLIT>), g, b, qd, kd, vd, od, p); break;
                case 3: RL_LAUNCH(ctx, (k_flash_attention<3, QW, KSPLIT>), g, b, qd, kd, vd, od, p); break;
                default: RL_LAUNCH(ctx, (k_flash_attention<4, QW, KSPLIT>), g, b, qd, kd, vd, od, p); break;
            }
            return after_launch(ctx, name);
        }
    }
    const uint64_t rows = heads * s.q_len;
    const dim3 g(static_cast<unsigned>(rows)), b(64);
    if (s.head_dim <= 64) {
        RL_LAUNCH(ctx, (k_attention_rows<T, 1>), g, b, qd, kd, vd, od, p);
    } else if (s.head_dim <= 128) {
        RL_LAUNCH(ctx, (k_attention_rows<T, 2>), g, b, qd, kd, vd, od, p);
    } else if (s.head_dim <= 256) {
        RL_LAUNCH(ctx, (k_attention_rows<T, 4>), g, b, qd, kd, vd, od, p);
    } else {
        RL_LAUNCH(ctx, (k_attention_rows<T, 8>), g, b, qd, kd, vd, od, p);
    }
    return after_launch(ctx, name);
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_attention_f32(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                           const rl_buffer* v, uint64_t batch, uint64_t q_heads,
                           uint64_t kv_heads, uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                           uint64_t kv_capacity, float scale, uint64_t query_start_pos,
                           const rl_buffer* out) {
    const AttnShape s{batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity};
    return attention_entry<float>(ctx, "attention_f32", q, k, v, s, scale, query_start_pos, out);
}

rl_status rl_attention_f16(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                           const rl_buffer* v, uint64_t batch, uint64_t q_heads,
                           uint64_t kv_heads, uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                           uint64_t kv_capacity, float scale, uint64_t query_start_pos,
                           const rl_buffer* out) {
    const AttnShape s{batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity};
    return attention_entry<half_t>(ctx, "attention_f16", q, k, v, s, scale, query_start_pos,
                                   out);
}

}  // extern "C"
