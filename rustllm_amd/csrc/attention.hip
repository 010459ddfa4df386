// attention.hip -- the attention core of one layer for gfx950.
//
// SelfAttention::attention_core_encode (src/nn/attention.rs:216-247) runs
// four kernels: scores = Q K^T (gqa_qk_*, or batched_matmul when the head
// counts match), attention_scale_mask, softmax_last_dim, and P V (gqa_pv_*).
// The scores make a [B, QH, Q, K] round trip through memory twice.  Here the
// four are one pass ("flash" attention: Dao et al., 2022): each workgroup
// keeps a tile of queries in registers, streams the keys and values of its
// KV head through LDS in blocks of 64 or 128, and folds every block into a
// running (max, sum, output) per query, so the scores never leave the chip.
//
// f16 with a head size that is a multiple of 32 (32..128) takes the matrix
// cores (v_mfma_f32_32x32x16_f16, f32 accumulation): per wave 32 queries,
// S^T = K Q^T so that each lane owns one query column and its row statistics
// need one cross-lane exchange; the keys of a 32-key tile are read in an
// order that swaps bits 2 and 3 of the key index, which leaves each lane
// holding eight consecutive keys of P -- exactly the operand layout of the
// P V product, so P goes from registers to the second MFMA without moving.
// K rows are stored in LDS in that key order; V stays row-major and its
// transposed operand comes from the LDS transpose read (ds_read_b64_tr_b16).
// K and V blocks travel from memory to LDS by DMA (buffer loads into LDS,
// two stages deep), so the next block streams in during this one's compute.
// f32 with the same head sizes takes v_mfma_f32_32x32x2_f32 in the same
// tiling (its own key order, f32 probabilities).  Decode steps (few query
// rows per KV head) split the keys over many workgroups; other head sizes
// (up to 512) take a one-wave-per-query kernel on the vector ALUs.
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
#include "mfma_layout.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

namespace rl {
namespace {

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.693147180559945309417f;

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
    uint32_t kchunks;      // key chunks per query tile (f16 MFMA kernel, PARTIAL)
    float* part;           // PARTIAL: unnormalised outputs, [tile unit][query][head_dim]
    float* part_ml;        // PARTIAL: (max in log2 units, sum) per [tile unit][query]
};

// ------------------------------------------------------------- MFMA kernel

// max over lanes l and l ^ 32 without an LDS permute: v_permlane32_swap
// returns {lower lane's value, upper lane's value} in both lanes.
__device__ inline float max_halves(float v) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// max(a, b, c) in one v_max3_f32.  (fmaxf on a value the compiler cannot
// prove canonical, such as an MFMA result, costs an extra v_max_f32 x, x.)
__device__ inline float max3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Chunk order of the unpadded LDS rows the DMA-fed kernel uses: 16-byte
// chunk c of row r sits at chunk c ^ lds_swizzle(r) of that row.  The MFMA
// operand reads of K (16 rows x one chunk per 16 lanes) and the transpose
// reads of V (4 rows x 4 chunks per 32 lanes) then each fall on 64 distinct
// banks (64 banks of 4 bytes; a row is D / 8 chunks).
template <int NT>
__device__ inline uint32_t lds_swizzle(uint32_t r) {
    if constexpr (NT == 1) return (r >> 2) & 3u;
    else if constexpr (NT == 2) return ((r & 2u) << 1) | ((r >> 2) & 3u);
    else if constexpr (NT == 4) return ((r & 3u) << 2) | ((r >> 2) & 3u);
    else return 0u;
}

// Buffer resource (gfx9 descriptor: base, stride 0, size in bytes, 32-bit
// data format) for raw loads from `base`: a load at or past `bytes` returns
// zeros.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ inline i32x4 raw_buffer(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return i32x4{int(uint32_t(a)), int(uint32_t(a >> 32) & 0xffffu), int(bytes), 0x00020000};
}

// One 16-byte chunk per lane from a raw buffer straight into LDS
// (buffer_load_dwordx4 ... lds): lane l's chunk lands at lds_addr + 16 l.
// The LDS address goes through M0, saved and restored around the load.  In
// assembly so that the compiler's wait counting, which cannot tell the LDS
// stage being filled from the one being read, does not hold every LDS read
// of the step until the transfer lands; the caller waits (vmcnt) before the
// barrier that hands the stage over.
__device__ inline void dma_to_lds(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds_addr), "v"(voffset), "s"(rsrc)
        : "memory");
}

// Rescaling threshold (log2 units): a query's running max m is only moved
// when a block's max exceeds it by more than this, so most blocks skip the
// rescale of the running sum and output; probabilities exp2(t - m) then stay
// below 2^3, well inside f16 and f32 range.
constexpr float kRescaleSlack = 3.0f;

// QW waves of 32 queries each; KSPLIT groups of such waves split the key
// blocks of the tile between them (group g takes blocks g, g + KSPLIT, ...)
// and merge their partial (max, sum, output) through LDS at the end.
//
// DMA: K and V blocks go from memory straight into LDS (buffer_load ... lds,
// no registers), two stages deep, so the next blocks stream in while this
// one is computed; rows are unpadded with the chunk order of lds_swizzle.
// Otherwise blocks pass through registers into rows padded for the bank
// layout (head size 96, whose 12 chunks a row do not swizzle onto 64 banks),
// one block at a time.
template <int NT, int QW, int KSPLIT, int BN, bool DMA, bool PARTIAL = false>
__global__ __launch_bounds__(64 * QW * KSPLIT) void k_flash_attention(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    half_t* __restrict__ out, AttnParams p) {
    constexpr int D = 32 * NT;          // head size
    constexpr int DC = D / 16;          // 16-wide slices of a head (MFMA depth)
    constexpr int KT = BN / 32;         // 32-key tiles per block
    static_assert(!DMA || NT != 3, "no bank-spreading chunk order for 12-chunk rows");
    // LDS rows: with DMA unpadded and swizzled; otherwise K at a stride of
    // D + 8 halves (the 16-byte reads of 16 consecutive rows hit distinct
    // banks), V at v_stride_tr(D).
    constexpr int KS = DMA ? D : D + 8;
    constexpr int VS = DMA ? D : v_stride_tr(D);
    constexpr int NSTAGE = DMA ? 2 : 1;
    constexpr int THREADS = 64 * QW * KSPLIT;
    constexpr int TILE_Q = 32 * QW;                    // queries per tile
    constexpr int BLOCK_CHUNKS = BN * D / 8;           // 16-byte chunks of one K (or V) block
    constexpr int LOADS = BLOCK_CHUNKS * KSPLIT / THREADS;
    constexpr int DMA_LOADS = 2 * LOADS;               // K and V chunks per lane (DMA)
    constexpr int WAVES = THREADS / 64;
    constexpr int ROUNDS = BLOCK_CHUNKS / (64 * WAVES);  // DMA instructions per region
    constexpr int ROW_CHUNKS = D / 8;
    constexpr int KV_HALVES = BN * KS + BN * VS;       // one block of K and V
    constexpr int STAGE_BYTES = KSPLIT * KV_HALVES * 2;
    constexpr int MERGE = NT * 16 + 2;                 // floats a lane hands over
    constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES > (KSPLIT - 1) * QW * 64 * MERGE * 4
                                  ? NSTAGE * STAGE_BYTES
                                  : (KSPLIT - 1) * QW * 64 * MERGE * 4;
    static_assert((BLOCK_CHUNKS * KSPLIT) % THREADS == 0, "blocks must split evenly");
    static_assert(!DMA || BLOCK_CHUNKS % (64 * WAVES) == 0,
                  "every wave's DMA instructions cover whole regions");
    __shared__ __align__(16) unsigned char lds[LDS_BYTES];
    half_t* const kv_lds = reinterpret_cast<half_t*>(lds);

    // PARTIAL: workgroup b takes key chunk b mod kchunks of its tile pair
    // (the chunks of one pair are neighbours in the grid: one KV head)
    const uint32_t chunk = PARTIAL ? blockIdx.x % p.kchunks : 0u;
    const uint32_t unit_blk = PARTIAL ? blockIdx.x / p.kchunks : blockIdx.x;
    const uint32_t bh = unit_blk / p.pairs;
    const uint32_t pair = unit_blk % p.pairs;
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
    // Transpose reads of V for the A operand of O^T += V^T P^T: lane
    // 16g + 4j + a reads row 8(g / 2) + j (+ 16c + 4e2 for slice c, half e2)
    // at columns 16(g % 2) + 4a (+ 32t for head tile t); the hardware then
    // hands lane 16g + i the column 16(g % 2) + i of those four rows.
    // Per lane: offsets of its K operand chunks (row `col`, chunk 2c + hs) and
    // of its V transpose reads (e2 = rows 0-3 or 4-7 of the eight, t = head
    // tile), in the chunk order of the LDS rows.
    uint32_t koff[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c)
        koff[c] = col * KS + 8 * ((2 * c + hs) ^ (DMA ? lds_swizzle<NT>(col) : 0u));
    uint32_t voff[2][NT];
#pragma unroll
    for (int e2 = 0; e2 < 2; ++e2) {
        const uint32_t row = 8 * (lane / 32) + (lane % 16) / 4 + 4 * e2;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t ch = 2 * ((lane / 16) % 2) + (lane % 4) / 2 + 4 * t;
            voff[e2][t] = row * VS + 8 * (ch ^ (DMA ? lds_swizzle<NT>(row) : 0u)) + 4 * (lane % 2);
        }
    }
    // DMA: a stage holds, per key group, the K block then the V block
    // (regions of BLOCK_CHUNKS 16-byte chunks).  Instruction li of a wave
    // fills 64 chunks (lane order) of region li / ROUNDS, so the region --
    // which block, K or V -- is a compile-time fact of li; the lane picks the
    // source chunk that belongs at its place.
    const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
    uint32_t dma_off[DMA_LOADS];
#pragma unroll
    for (int li = 0; li < DMA_LOADS; ++li) {
        const bool is_v = (li / ROUNDS) % 2;
        const uint32_t cf = ((li % ROUNDS) * WAVES + wave) * 64 + lane;  // chunk in the region
        const uint32_t r = cf / ROW_CHUNKS;
        const uint32_t ch = (cf % ROW_CHUNKS) ^ lds_swizzle<NT>(r);
        const uint32_t key = is_v ? r : ((r & ~31u) | perm32(r & 31u));
        dma_off[li] = key * (D * 2) + ch * 16;
    }
    const i32x4 k_rsrc = raw_buffer(kh, p.kv_len * (D * 2));
    const i32x4 v_rsrc = raw_buffer(vh, p.kv_len * (D * 2));
    const uint32_t lds_base = uint32_t(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)(lds)));

    // The causal tiles of a head are paired (t, tiles - 1 - t) so that every
    // workgroup streams about the same number of key blocks.
    for (int which = 0; which < 2; ++which) {
        const uint32_t tile = which == 0 ? p.tiles - 1 - pair : pair;
        if (which == 1 && tile >= p.tiles - 1 - pair) break;

        const uint32_t q_first = tile * TILE_Q;
        const uint32_t q_last = min(p.q_len, q_first + TILE_Q) - 1;
        const uint32_t keys = min(p.kv_len, p.start + q_last + 1);
        const uint32_t blocks = (keys + BN - 1) / BN;
        const uint32_t steps = (blocks + KSPLIT - 1) / KSPLIT;
        // PARTIAL: this workgroup's share of the tile's steps, [s_begin, s_end)
        const uint32_t s_begin = PARTIAL ? uint32_t(uint64_t(steps) * chunk / p.kchunks) : 0u;
        const uint32_t s_end =
            PARTIAL ? uint32_t(uint64_t(steps) * (chunk + 1) / p.kchunks) : steps;

        const uint32_t qw0 = q_first + qw * 32;  // first query of this wave
        const bool wave_active = qw0 < p.q_len;
        const uint32_t wave_keys =
            wave_active ? min(p.kv_len, p.start + min(qw0 + 31, p.q_len - 1) + 1) : 0;

        // B operand of S^T = K Q^T: lane (col, hs) holds elements
        // 16c + 8hs .. + 7 of its query for every slice c
        const uint32_t qi = qw0 + col;
        const bool q_valid = qi < p.q_len;
        // Largest key this lane's query sees (padding columns see a few keys
        // too, so their arithmetic stays finite; never stored).
        const uint32_t key_limit = min(p.start + qi, p.kv_len - 1);
        h8 qf[DC];
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

        f32x16 o[NT];
        float m = -INFINITY, l = 0.0f;  // running max logit (log2 units), this lane's share of the sum
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;

        h8 kreg[LOADS], vreg[LOADS];
        bool vlive[LOADS];
        auto load_step = [&](uint32_t step) {
#pragma unroll
            for (int li = 0; li < LOADS; ++li) {
                const uint32_t chunk = threadIdx.x + THREADS * li;
                const uint32_t blk = step * KSPLIT + chunk / BLOCK_CHUNKS;
                const uint32_t c = chunk % BLOCK_CHUNKS;
                const uint32_t key = blk * BN + c / ROW_CHUNKS;
                const uint32_t d0 = (c % ROW_CHUNKS) * 8;
                // Rows past kv_len are never read (they may hold anything): a
                // key past the end loads row kv_len - 1 instead; its score is
                // masked (selected to -inf) and its value row zeroed, so it
                // adds nothing even if that row is not finite.  (The zeroing
                // happens at the LDS store, after the compute: a select here
                // would make the wave wait for the load now.)
                const uint32_t row = min(key, p.kv_len - 1);
                kreg[li] = *reinterpret_cast<const h8*>(kh + uint64_t(row) * D + d0);
                vreg[li] = *reinterpret_cast<const h8*>(vh + uint64_t(row) * D + d0);
                vlive[li] = key < p.kv_len;
            }
        };
        auto store_step = [&](uint32_t stage) {
#pragma unroll
            for (int li = 0; li < LOADS; ++li) {
                const uint32_t chunk = threadIdx.x + THREADS * li;
                const uint32_t c = chunk % BLOCK_CHUNKS;
                half_t* kdst = kv_lds + (stage * KSPLIT + chunk / BLOCK_CHUNKS) * KV_HALVES;
                half_t* vdst = kdst + BN * KS;
                const uint32_t key = c / ROW_CHUNKS;
                const uint32_t d0 = (c % ROW_CHUNKS) * 8;
                // K row `key` goes to LDS row perm32(key): the S^T operand of
                // lane i is then LDS row i.
                *reinterpret_cast<h8*>(kdst + perm32(key) * KS + d0) = kreg[li];
                const h8 zero = {};
                *reinterpret_cast<h8*>(vdst + key * VS + d0) = vlive[li] ? vreg[li] : zero;
            }
        };

        // DMA of one step's blocks into stage step % 2.  Keys past kv_len
        // read as zeros (the buffer ends at row kv_len): their scores are
        // masked and their value rows add nothing.
        auto issue_step = [&](uint32_t step) {
            // LDS address of the wave's first chunk in this stage
            const uint32_t wave_lds = __builtin_amdgcn_readfirstlane(
                lds_base + (step % 2) * STAGE_BYTES + 16 * 64 * wave_u);
#pragma unroll
            for (int li = 0; li < DMA_LOADS; ++li) {
                constexpr int PER_BLOCK = 2 * ROUNDS;  // instructions per group (K and V)
                const uint32_t blk = step * KSPLIT + li / PER_BLOCK;
                if (blk >= blocks) continue;
                const bool is_v = (li / ROUNDS) % 2;
                const uint32_t region = li / ROUNDS, round = li % ROUNDS;
                dma_to_lds(is_v ? v_rsrc : k_rsrc,
                           wave_lds + 16 * (region * BLOCK_CHUNKS + round * WAVES * 64),
                           dma_off[li] + blk * (BN * D * 2));
            }
        };

        if constexpr (DMA) {
            if (s_begin < s_end) issue_step(s_begin);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        } else {
            load_step(s_begin);
            __syncthreads();  // the previous tile's LDS use is over
            store_step(0);
            __syncthreads();
        }

        // DMA: the blocks of step j + 1 stream into the other stage while
        // step j is computed (one barrier per step).  Otherwise they wait in
        // registers and are stored after the step's compute.
        for (uint32_t step = s_begin; step < s_end; ++step) {
            if constexpr (DMA) {
                if (step + 1 < s_end) issue_step(step + 1);  // nothing past the last block
            } else {
                if (step + 1 < s_end) load_step(step + 1);
            }
            const uint32_t blk = step * KSPLIT + sub;
            const half_t* ks = kv_lds + ((step % NSTAGE) * KSPLIT + sub) * KV_HALVES;
            const half_t* vs = ks + BN * KS;
            if (blk < blocks && blk * BN < wave_keys) {
                // S^T = K Q^T, 32 keys per tile
                f32x16 s[KT];
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
#pragma unroll
                    for (int c = 0; c < DC; ++c) {
                        const h8 ka = *reinterpret_cast<const h8*>(ks + kt * 32 * KS + koff[c]);
                        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[c], s[kt], 0, 0, 0);
                    }
                }
                // mask; the block's max raw score of each query
                const uint32_t kbase = blk * BN;
                if (kbase + BN - 1 > p.start + qw0 || kbase + BN > p.kv_len) {
                    // register r of tile kt holds key kbase + 8hs + (a constant)
                    const int lim = int(key_limit) - int(kbase + 8 * hs);
#pragma unroll
                    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            if (kt * 32 + 16 * (r >> 3) + (r & 7) > lim) s[kt][r] = -INFINITY;
                }
                // two independent max chains, joined at the end
                float mx = -INFINITY, my = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; r += 4) {
                        mx = max3(mx, s[kt][r], s[kt][r + 1]);
                        my = max3(my, s[kt][r + 2], s[kt][r + 3]);
                    }
                mx = fmaxf(mx, my);
                mx = max_halves(mx);
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
                // p = 2^(s * scale * log2 e - m); a query that has seen no
                // key yet (m = -inf) has only -inf scores here, and p = 0.
                const float neg_m = m == -INFINITY ? 0.0f : -m;
                // P as the f16 operand of the P V product: lane half hs
                // supplies keys 16c + 8hs .. +7, which it holds in registers
                // 8(c%2) .. +7 of tile c/2.  The running sum adds the same f16
                // probabilities the product uses (v_dot2_f32_f16 against
                // ones, f32 accumulation).
                const h2 ones = {half_t(1.0f), half_t(1.0f)};
                h8 pb[BN / 16];
#pragma unroll
                for (int c = 0; c < BN / 16; ++c) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        pb[c][e] = half_t(__builtin_amdgcn_exp2f(
                            __builtin_fmaf(s[c >> 1][8 * (c & 1) + e], p.scale_log2, neg_m)));
#pragma unroll
                    for (int e = 0; e < 8; e += 2)
                        l = __builtin_amdgcn_fdot2(h2{pb[c][e], pb[c][e + 1]}, ones, l, false);
                }
                // O^T += V^T P^T, 16 keys per MFMA; each V operand read once.
#pragma unroll
                for (int c = 0; c < BN / 16; ++c) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const h4 lo = lds_read_transposed(vs + 16 * c * VS + voff[0][t]);
                        const h4 hi = lds_read_transposed(vs + 16 * c * VS + voff[1][t]);
                        const h8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[c], o[t], 0, 0, 0);
                    }
                }
            }
            if constexpr (DMA) {
                __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA has landed
            } else {
                __syncthreads();
                if (step + 1 < s_end) store_step(0);
            }
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
                for (int h = 1; h < KSPLIT; ++h) {
                    const float* src = mg + ((h - 1) * QW * 64 + qw * 64 + lane) * MERGE;
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

        if (PARTIAL && sub == 0) {
            // the chunk's (max, sum) and unnormalised f32 output of each query,
            // merged by k_flash_combine
            const float l_row = l + __shfl_xor(l, 32, 64);  // both halves of the query
            if (q_valid) {
                const uint64_t prow =
                    ((uint64_t(bh) * p.tiles + tile) * p.kchunks + chunk) * TILE_Q + (qi - q_first);
                float* po = p.part + prow * D + 4 * hs;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        *reinterpret_cast<f32x4*>(po + t * 32 + 8 * g) =
                            f32x4{o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]};
                if (hs == 0) {
                    p.part_ml[2 * prow] = m;
                    p.part_ml[2 * prow + 1] = l_row;
                }
            }
        } else if (sub == 0) {
            const float inv = 1.0f / (l + __shfl_xor(l, 32, 64));  // both halves of the query
            if (q_valid) {
                // register r of tile t: element 32t + 8(r / 4) + 4hs + r % 4
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
}

// The key chunks of a split launch of k_flash_attention merged, per query:
// every chunk's (max m_c, sum l_c, unnormalised output o_c) rescaled to the
// largest max M, out = sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c (the
// key-share merge of the kernel itself, over kchunks <= kFlashMaxChunks).
// Workgroup = kCombineRows queries of a tile of a head (many workgroups: the
// merge is a short dependent chain of loads per query); thread item =
// (query, 4 head elements), 16-byte pieces of a row on consecutive lanes.
// Every chunk's loads are issued before any is used.  Some chunk holds key
// 0, which every query sees, so M is finite.
constexpr uint32_t kFlashMaxChunks = 16;
constexpr uint32_t kCombineRows = 16;
template <int D, int TILE_Q>
__global__ __launch_bounds__(256) void k_flash_combine(half_t* __restrict__ out, AttnParams p) {
    constexpr uint32_t G = D / 4;
    constexpr uint32_t PARTS = TILE_Q / kCombineRows;
    const uint32_t part = blockIdx.x % PARTS, unit = blockIdx.x / PARTS;
    const uint32_t bh = unit / p.tiles, tile = unit % p.tiles;
    const uint32_t q_first = tile * TILE_Q;
    const uint32_t r0 = part * kCombineRows;
    if (q_first + r0 >= p.q_len) return;
    const uint32_t rows = min(kCombineRows, p.q_len - q_first - r0);
    const uint64_t unit0 = (uint64_t(bh) * p.tiles + tile) * p.kchunks;
    for (uint32_t it = threadIdx.x; it < rows * G; it += 256) {
        const uint32_t r = r0 + it / G, g = it % G;
        float2 ml[kFlashMaxChunks];
        f32x4 oc[kFlashMaxChunks];
#pragma unroll
        for (uint32_t c = 0; c < kFlashMaxChunks; ++c) {
            const uint64_t prow = (unit0 + c) * TILE_Q + r;
            if (c < p.kchunks) {
                ml[c] = *reinterpret_cast<const float2*>(p.part_ml + 2 * prow);
                oc[c] = *reinterpret_cast<const f32x4*>(p.part + prow * D + 4 * g);
            } else {
                ml[c] = make_float2(-INFINITY, 0.0f);
                oc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
        float mmax = -INFINITY;
#pragma unroll
        for (uint32_t c = 0; c < kFlashMaxChunks; ++c) mmax = fmaxf(mmax, ml[c].x);
        float lsum = 0.0f;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t c = 0; c < kFlashMaxChunks; ++c) {
            const float w = mmax > ml[c].x ? __builtin_amdgcn_exp2f(ml[c].x - mmax) : 1.0f;
            lsum += w * ml[c].y;
            acc += w * oc[c];
        }
        const float inv = 1.0f / lsum;
        const h4 o = {half_t(acc[0] * inv), half_t(acc[1] * inv), half_t(acc[2] * inv),
                      half_t(acc[3] * inv)};
        *reinterpret_cast<h4*>(out + (uint64_t(bh) * p.q_len + q_first + r) * D + 4 * g) = o;
    }
}

// ------------------------------------------------- f32 on the matrix cores

// f32 takes v_mfma_f32_32x32x2_f32 (two head elements per step, exact f32
// products) with K rows in the key_row32 order, so each lane's probabilities
// are the B operand of the P V step as they stand; K rows at a stride of
// 2 mod 64 floats and V rows at 32 mod 64 (f32_stride) keep the operand
// reads on 64 distinct banks.
// Same tiling as k_flash_attention (QW waves of 32 queries, KSPLIT key
// shares merged through LDS, causal tiles paired), blocks staged through
// registers; scores, probabilities and the running sum stay in f32.
template <int NT, int QW, int KSPLIT, int BN>
__global__ __launch_bounds__(64 * QW * KSPLIT) void k_flash_attention_f32(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ out, AttnParams p) {
    constexpr int D = 32 * NT;
    constexpr int DS = D / 2;  // MFMA steps over the head
    constexpr int KT = BN / 32;
    constexpr int KS = f32_stride(D, 2);
    constexpr int VS = f32_stride(D, 32);
    constexpr int THREADS = 64 * QW * KSPLIT;
    constexpr int TILE_Q = 32 * QW;
    constexpr int ROW_CHUNKS = D / 4;                   // 16-byte chunks of a row
    constexpr int BLOCK_CHUNKS = BN * ROW_CHUNKS;
    constexpr int LOADS = BLOCK_CHUNKS * KSPLIT / THREADS;
    constexpr int KV_FLOATS = BN * KS + BN * VS;        // one block of K and V
    constexpr int MERGE = NT * 16 + 2;
    constexpr int LDS_FLOATS = KSPLIT * KV_FLOATS > (KSPLIT - 1) * QW * 64 * MERGE
                                   ? KSPLIT * KV_FLOATS
                                   : (KSPLIT - 1) * QW * 64 * MERGE;
    static_assert((BLOCK_CHUNKS * KSPLIT) % THREADS == 0, "blocks must split evenly");
    __shared__ __align__(16) float lds[LDS_FLOATS];

    const uint32_t bh = blockIdx.x / p.pairs;
    const uint32_t pair = blockIdx.x % p.pairs;
    const uint32_t kv_heads = p.q_heads / p.group;
    const uint32_t kv_head = (bh / p.q_heads) * kv_heads + (bh % p.q_heads) / p.group;
    const float* kh = k + uint64_t(kv_head) * p.kv_head_stride;
    const float* vh = v + uint64_t(kv_head) * p.kv_head_stride;
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t qw = wave % QW;
    const uint32_t sub = wave / QW;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t col = lane % 32;
    const uint32_t hs = lane / 32;

    for (int which = 0; which < 2; ++which) {
        const uint32_t tile = which == 0 ? p.tiles - 1 - pair : pair;
        if (which == 1 && tile >= p.tiles - 1 - pair) break;
        const uint32_t q_first = tile * TILE_Q;
        const uint32_t q_last = min(p.q_len, q_first + TILE_Q) - 1;
        const uint32_t keys = min(p.kv_len, p.start + q_last + 1);
        const uint32_t blocks = (keys + BN - 1) / BN;
        const uint32_t steps = (blocks + KSPLIT - 1) / KSPLIT;
        const uint32_t qw0 = q_first + qw * 32;
        const bool wave_active = qw0 < p.q_len;
        const uint32_t wave_keys =
            wave_active ? min(p.kv_len, p.start + min(qw0 + 31, p.q_len - 1) + 1) : 0;

        // B operand of S^T = K Q^T: lane (col, hs) holds elements 2j + hs of
        // its query for every step j.
        const uint32_t qi = qw0 + col;
        const bool q_valid = qi < p.q_len;
        const uint32_t key_limit = min(p.start + qi, p.kv_len - 1);
        float qf[DS];
        const float* qrow = q + (uint64_t(bh) * p.q_len + (q_valid ? qi : 0)) * D + hs;
#pragma unroll
        for (int j = 0; j < DS; ++j) qf[j] = q_valid ? qrow[2 * j] : 0.0f;

        f32x16 o[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
        float m = -INFINITY, l = 0.0f;

        float4 kreg[LOADS], vreg[LOADS];
        bool vlive[LOADS];
        auto load_step = [&](uint32_t step) {
#pragma unroll
            for (int li = 0; li < LOADS; ++li) {
                const uint32_t chunk = threadIdx.x + THREADS * li;
                const uint32_t blk = step * KSPLIT + chunk / BLOCK_CHUNKS;
                const uint32_t c = chunk % BLOCK_CHUNKS;
                const uint32_t key = blk * BN + c / ROW_CHUNKS;
                const uint32_t d0 = (c % ROW_CHUNKS) * 4;
                // rows past kv_len are not read (they may hold anything): a
                // key past the end loads row kv_len - 1, its score is masked
                // and its value row zeroed at the LDS store
                const uint32_t row = min(key, p.kv_len - 1);
                kreg[li] = *reinterpret_cast<const float4*>(kh + uint64_t(row) * D + d0);
                vreg[li] = *reinterpret_cast<const float4*>(vh + uint64_t(row) * D + d0);
                vlive[li] = key < p.kv_len;
            }
        };
        auto store_step = [&]() {
#pragma unroll
            for (int li = 0; li < LOADS; ++li) {
                const uint32_t chunk = threadIdx.x + THREADS * li;
                const uint32_t c = chunk % BLOCK_CHUNKS;
                float* kdst = lds + (chunk / BLOCK_CHUNKS) * KV_FLOATS;
                float* vdst = kdst + BN * KS;
                const uint32_t key = c / ROW_CHUNKS;
                const uint32_t d0 = (c % ROW_CHUNKS) * 4;
                // K rows at the rotated order, 8-byte aligned (stride 2 mod 64)
                float* kr = kdst + ((key & ~31u) | key_row32(key & 31u)) * KS + d0;
                *reinterpret_cast<float2*>(kr) = float2{kreg[li].x, kreg[li].y};
                *reinterpret_cast<float2*>(kr + 2) = float2{kreg[li].z, kreg[li].w};
                // per-component selects: a select of two float4 structs goes
                // through private memory
                const bool live = vlive[li];
                *reinterpret_cast<float4*>(vdst + key * VS + d0) =
                    float4{live ? vreg[li].x : 0.0f, live ? vreg[li].y : 0.0f,
                           live ? vreg[li].z : 0.0f, live ? vreg[li].w : 0.0f};
            }
        };

        load_step(0);
        __syncthreads();  // the previous tile's LDS use is over
        store_step();
        __syncthreads();
        for (uint32_t step = 0; step < steps; ++step) {
            if (step + 1 < steps) load_step(step + 1);
            const uint32_t blk = step * KSPLIT + sub;
            const float* ks = lds + sub * KV_FLOATS;
            const float* vs = ks + BN * KS;
            if (blk < blocks && blk * BN < wave_keys) {
                f32x16 s[KT];
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
                    const float* krow = ks + (kt * 32 + col) * KS + hs;
#pragma unroll
                    for (int j = 0; j < DS; ++j)
                        s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(krow[2 * j], qf[j], s[kt], 0,
                                                                      0, 0);
                }
                // register r of tile kt holds key kbase + 32 kt + 2r + hs
                const uint32_t kbase = blk * BN;
                if (kbase + BN - 1 > p.start + qw0 || kbase + BN > p.kv_len) {
                    const int lim = int(key_limit) - int(kbase + hs);
#pragma unroll
                    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            if (kt * 32 + 2 * r > lim) s[kt][r] = -INFINITY;
                }
                // scores in log2 units first, so that the largest one's
                // probability is exactly 1 (2^(t - m) with t == m)
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[kt][r] *= p.scale_log2;
                float mx = -INFINITY, my = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; r += 4) {
                        mx = max3(mx, s[kt][r], s[kt][r + 1]);
                        my = max3(my, s[kt][r + 2], s[kt][r + 3]);
                    }
                mx = fmaxf(mx, my);
                const float mx_log2 = max_halves(mx);
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
                // p = 2^(t - m), in place; a query that has seen no key yet
                // (m = -inf) has only -inf scores, and p = 0
                const float neg_m = m == -INFINITY ? 0.0f : -m;
                float la = 0.0f, lb = 0.0f;
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        s[kt][r] = __builtin_amdgcn_exp2f(s[kt][r] + neg_m);
                        s[kt][r + 1] = __builtin_amdgcn_exp2f(s[kt][r + 1] + neg_m);
                        la += s[kt][r];
                        lb += s[kt][r + 1];
                    }
                l += la + lb;
                // O^T += V^T P^T over keys 2r, 2r + 1 of each tile: lane
                // (col, hs) supplies V[2r + hs][32t + col] and P of its query
                // at key 2r + hs (register r).
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float* vrow = vs + (kt * 32 + 2 * r + hs) * VS + col;
#pragma unroll
                        for (int t = 0; t < NT; ++t)
                            o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * t], s[kt][r],
                                                                         o[t], 0, 0, 0);
                    }
            }
            __syncthreads();
            if (step + 1 < steps) store_step();
            __syncthreads();
        }

        if constexpr (KSPLIT > 1) {
            // Groups 1.. hand their (max, sum, output) to group 0 through LDS.
            if (sub > 0) {
                float* dst = lds + ((sub - 1) * QW * 64 + qw * 64 + lane) * MERGE;
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
                for (int h = 1; h < KSPLIT; ++h) {
                    const float* src = lds + ((h - 1) * QW * 64 + qw * 64 + lane) * MERGE;
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

        if (sub == 0) {
            const float inv = 1.0f / (l + __shfl_xor(l, 32, 64));  // both halves of the query
            if (q_valid) {
                // register r of tile t: element 32t + 8(r / 4) + 4hs + r % 4
                float* orow = out + (uint64_t(bh) * p.q_len + qi) * D + 4 * hs;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        *reinterpret_cast<float4*>(orow + 32 * t + 8 * g) =
                            float4{o[t][4 * g] * inv, o[t][4 * g + 1] * inv,
                                   o[t][4 * g + 2] * inv, o[t][4 * g + 3] * inv};
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
        mx = wave_max_dpp(mx);
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
    const float inv = 1.0f / wave_sum_dpp(l);
    T* orow = out + uint64_t(row) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        const uint32_t d = lane + 64 * t;
        if (d < D) orow[d] = from_float<T>(o[t] * inv);
    }
}

// ------------------------------------------------- split keys (decode)

// The merge of one KV head's partials by the workgroup that finishes its
// last split: thread (r, d) merges output element d of row r over every
// split, loading kMergeChunk splits' (max, sum, value) at once -- indices
// past the last split are clamped and masked -- and folding them into a
// running max, sum and value.  With up to kMergeChunk splits (4096 keys at
// 256 keys per split) the merge is one memory round trip.
constexpr uint32_t kMaxSplits = 1024;
constexpr int kMergeChunk = 16;

// Agent-coherent store and load of a partial (relaxed atomics at agent
// scope: global_store / global_load with sc1, which write through and read
// past the XCD's own L2).
__device__ inline void publish(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float observe(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ inline void merge_head(const float* part, T* __restrict__ out,
                                  const AttnParams& p, uint32_t b, uint32_t first_head,
                                  uint32_t R, uint32_t splits) {
    const uint32_t D = p.head_dim;
    const uint32_t stride = D + 2;
    for (uint32_t i = threadIdx.x; i < R * D; i += blockDim.x) {
        const uint32_t r = i / D, d = i % D;
        const uint64_t row = (uint64_t(b) * p.q_heads + first_head + r / p.q_len) * p.q_len +
                             r % p.q_len;
        const float* src = part + row * splits * stride;
        float mt = -INFINITY, lt = 0.0f, acc = 0.0f;
        for (uint32_t s0 = 0; s0 < splits; s0 += kMergeChunk) {
            float mv[kMergeChunk], lv[kMergeChunk], ov[kMergeChunk];
#pragma unroll
            for (int j = 0; j < kMergeChunk; ++j) {
                const uint32_t sp = min(s0 + j, splits - 1);
                mv[j] = observe(src + sp * stride);
                lv[j] = observe(src + sp * stride + 1);
                ov[j] = observe(src + sp * stride + 2 + d);
            }
            float mc = mt;
#pragma unroll
            for (int j = 0; j < kMergeChunk; ++j)
                if (s0 + j < splits) mc = fmaxf(mc, mv[j]);
            if (mc == -INFINITY) continue;  // no key seen yet
            const float keep = mt == -INFINITY ? 0.0f : exp_fast(mt - mc);
            lt *= keep;
            acc *= keep;
#pragma unroll
            for (int j = 0; j < kMergeChunk; ++j) {
                const bool use = s0 + j < splits && mv[j] != -INFINITY;
                const float w = use ? exp_fast(mv[j] - mc) : 0.0f;
                lt += lv[j] * w;
                acc += ov[j] * w;
            }
            mt = mc;
        }
        out[row * D + d] = from_float<T>(acc * (1.0f / lt));
    }
}

// A split-key decode workgroup: four waves of 64 keys each.  The hand-off
// counter of KV head i is word i * kTicketStride of the counter array: one
// per 256 bytes, so that the atomics of different heads do not queue on one
// line (the 80 workgroups of a 5-head, 4096-key step: 7.5 -> 7.05 us).
constexpr int kSplitWaves = 4;
constexpr uint32_t kTicketStride = 64;
constexpr int kSplitKeys = 64 * kSplitWaves;   // keys per workgroup
constexpr int kStageBytes = 64 * 256;          // LDS per wave for staged value rows

// The end of a split-key workgroup: its four waves' states (per wave and
// row: max, sum and output row, in LDS) -> one partial per row, stored
// agent-coherent; the workgroup that completes a KV head's last split then
// merges that head's rows.
template <typename T, int RM, int DMAX>
__device__ inline void finish_split(const float (&merge_m)[kSplitWaves][RM],
                                    const float (&merge_l)[kSplitWaves][RM],
                                    const float (&merge_o)[kSplitWaves][RM][DMAX],
                                    float* __restrict__ part, uint32_t* __restrict__ tickets,
                                    T* __restrict__ out, const AttnParams& p, uint32_t b,
                                    uint32_t first_head, uint32_t R, uint32_t kvb,
                                    uint32_t split, uint32_t splits) {
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t D = p.head_dim;
    __syncthreads();  // every wave's state is in LDS
    const uint32_t stride = D + 2;
    for (uint32_t r = wave; r < R; r += kSplitWaves) {
        float mt = -INFINITY;
        for (int w = 0; w < kSplitWaves; ++w) mt = fmaxf(mt, merge_m[w][r]);
        float scale_w[kSplitWaves];
        float lt = 0.0f;
        for (int w = 0; w < kSplitWaves; ++w) {
            scale_w[w] = merge_m[w][r] == -INFINITY ? 0.0f : exp_fast(merge_m[w][r] - mt);
            lt += merge_l[w][r] * scale_w[w];
        }
        const uint64_t row = (uint64_t(b) * p.q_heads + first_head + r / p.q_len) * p.q_len +
                             r % p.q_len;
        float* dst = part + (row * splits + split) * stride;
        for (uint32_t d = lane; d < D; d += 64) {
            float acc = 0.0f;
            for (int w = 0; w < kSplitWaves; ++w) acc += merge_o[w][r][d] * scale_w[w];
            publish(dst + 2 + d, acc);
        }
        if (lane == 0) {
            publish(dst, mt);
            publish(dst + 1, lt);
        }
    }

    // Hand-off: the workgroup that completes a KV head's last split merges
    // that head's rows, so a decode step is one launch.  The partials were
    // stored agent-coherent (publish: written through the XCD's L2), every
    // wave waits for those stores to complete (vmcnt) before the barrier, and
    // only then does one thread draw the ticket -- no L2 write-back, which
    // an agent-scope release fence would make every workgroup pay in turn.
    // This release side rests on the hardware, not on the memory model: the
    // stores are relaxed atomics that gfx950 has completed at the point of
    // coherence (vmcnt 0) before the relaxed fetch_add is issued, which the
    // C++/HIP model alone does not order.  The merging workgroup (one per KV
    // head) takes an agent-scope acquire fence after its ticket, reads the
    // partials agent-coherent as well and puts the ticket back to zero for
    // the next launch.  The back-to-back decode tests guard the hand-off.
    __shared__ uint32_t ticket;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        ticket = __hip_atomic_fetch_add(&tickets[kvb * kTicketStride], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != splits - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (threadIdx.x == 0)
        __hip_atomic_store(&tickets[kvb * kTicketStride], 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    merge_head<T>(part, out, p, b, first_head, R, splits);
}

// Few query rows per KV head (a decode step: R = group * q_len rows): the
// rows of one KV head share every K and V row read.  Workgroup (kv head,
// split) takes 64 keys per wave and writes one partial (max, sum, output
// row) per query row; the workgroup that finishes a KV head's last split
// merges them (one launch per decode step).  A wave's loads
// are issued together -- its 64 value rows (contiguous in the cache) go
// straight to LDS (global_load_lds), its key rows to registers -- so a split
// costs one memory round trip.  RM bounds the rows, DPL the head elements
// per lane (D <= 64 DPL).

template <typename T, int RM, int DPL>
__global__ __launch_bounds__(64 * kSplitWaves) void k_attention_split(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    float* __restrict__ part, uint32_t* __restrict__ tickets, T* __restrict__ out, AttnParams p,
    uint32_t splits, bool vec_rows) {
    constexpr int DMAX = 64 * DPL;
    typedef typename Pack16<T>::type V;
    constexpr int N = Pack16<T>::N;
    __shared__ __align__(16) T qs[RM * DMAX];  // the rows' queries, zero past the head size
    __shared__ float ps[kSplitWaves][RM][64];
    __shared__ __align__(16) unsigned char vstage[kSplitWaves][kStageBytes];
    __shared__ float merge_m[kSplitWaves][RM];
    __shared__ float merge_l[kSplitWaves][RM];
    __shared__ float merge_o[kSplitWaves][RM][DMAX];
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t kvb = blockIdx.x / splits;  // b * kv_heads + kv head
    const uint32_t split = blockIdx.x % splits;
    const uint32_t kv_heads = p.q_heads / p.group;
    const uint32_t b = kvb / kv_heads;
    const uint32_t first_head = (kvb % kv_heads) * p.group;
    const uint32_t R = p.group * p.q_len;
    const uint32_t D = p.head_dim;
    const T* kh = k + uint64_t(kvb) * p.kv_head_stride;
    const T* vh = v + uint64_t(kvb) * p.kv_head_stride;
    const uint32_t base = split * kSplitKeys + wave * 64;
    const uint32_t n = p.kv_len > base ? min(64u, p.kv_len - base) : 0u;  // this wave's keys
    const uint32_t key = base + lane;
    // This thread's query elements first (row r = g * q_len + qi is query qi
    // of head first_head + g), so that their round trip is the key and
    // value loads' one rather than a second one after them.
    constexpr int QPT = (RM * DMAX + 64 * kSplitWaves - 1) / (64 * kSplitWaves);
    T qreg[QPT];
#pragma unroll
    for (int j = 0; j < QPT; ++j) {
        const uint32_t i = threadIdx.x + uint32_t(j) * 64 * kSplitWaves;
        const uint32_t r = i / DMAX, d = i % DMAX;
        T x = T(0.0f);
        if (i < uint32_t(RM * DMAX) && r < R && d < D) {
            const uint64_t row = (uint64_t(b) * p.q_heads + first_head + r / p.q_len) * p.q_len +
                                 r % p.q_len;
            x = q[row * D + d];
        }
        qreg[j] = x;
    }
    // value rows to LDS when 64 of them fit the stage, else read in place
    const bool staged = vec_rows && 64 * D * sizeof(T) <= kStageBytes;
    if (staged) {
        const uint32_t chunks = n * D * sizeof(T) / 16;  // 16-byte pieces of the n rows
        // rows n .. 63 (a wave past the last key): zeros, so that the value
        // reads below need no bounds; written before the copies into rows
        // 0 .. n are issued, which they do not overlap
        const uint32_t all = 64 * D * sizeof(T) / 16;
        for (uint32_t c = chunks + lane; c < all; c += 64)
            *reinterpret_cast<uint4*>(vstage[wave] + c * 16) = uint4{0, 0, 0, 0};
        const unsigned char* src = reinterpret_cast<const unsigned char*>(vh + uint64_t(base) * D);
        for (uint32_t c0 = 0; c0 < chunks; c0 += 64) {
            if (c0 + lane < chunks)
                __builtin_amdgcn_global_load_lds(
                    src + uint64_t(c0 + lane) * 16,
                    (__attribute__((address_space(3))) void*)(vstage[wave] + c0 * 16), 16, 0, 0);
        }
    }
    // key rows (lane = key), every load issued here, before the barrier:
    // unconditional, from a valid row (a lane past the wave's keys reads the
    // last key and its scores are masked below) and a valid pack (packs past
    // the head size read pack 0 and are zeroed), since loads under a branch
    // would be sunk past the barrier into a second round trip
    constexpr int PACKS = DMAX / N;
    V kv[PACKS];
    if (vec_rows) {
        const uint32_t krow_i = lane < n ? key : (p.kv_len > 0 ? p.kv_len - 1 : 0);
        const T* krow = kh + uint64_t(krow_i) * D;
#pragma unroll
        for (int i = 0; i < PACKS; ++i) {
            const bool in = uint32_t(i * N) < D;
            const V x = *reinterpret_cast<const V*>(krow + (in ? i * N : 0));
            kv[i] = in ? x : V{};
        }
    }
#pragma unroll
    for (int j = 0; j < QPT; ++j) {
        const uint32_t i = threadIdx.x + uint32_t(j) * 64 * kSplitWaves;
        if (i < uint32_t(RM * DMAX)) qs[i] = qreg[j];
    }
    __syncthreads();

    float sc[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) sc[r] = 0.0f;
    if (lane < n) {
        if (vec_rows) {
            // per pack: every row's query values read first (one LDS wait
            // per pack, not per read), then the products in f32 -- pairs of
            // f16 products per v_dot2_f32_f16, f32 elements by FMA -- over
            // the whole DMAX (both operands are zero past the head size)
#pragma unroll
            for (int i = 0; i < PACKS; ++i) {
                V qv[RM];
#pragma unroll
                for (int r = 0; r < RM; ++r)
                    qv[r] = *reinterpret_cast<const V*>(qs + r * DMAX + i * N);
#pragma unroll
                for (int r = 0; r < RM; ++r) {
                    if constexpr (std::is_same<T, half_t>::value) {
#pragma unroll
                        for (int e = 0; e < N; e += 2)
                            sc[r] = __builtin_amdgcn_fdot2(h2{qv[r][e], qv[r][e + 1]},
                                                           h2{kv[i][e], kv[i][e + 1]}, sc[r], false);
                    } else {
#pragma unroll
                        for (int e = 0; e < N; ++e) sc[r] = __builtin_fmaf(qv[r][e], kv[i][e], sc[r]);
                    }
                }
            }
        } else {
            const T* krow = kh + uint64_t(key) * D;
            for (uint32_t d = 0; d < D; ++d) {
                const float kd = to_float(krow[d]);
#pragma unroll
                for (int r = 0; r < RM; ++r) sc[r] += to_float(qs[r * DMAX + d]) * kd;
            }
        }
    }
    float m[RM], l[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const uint32_t limit = p.start + uint32_t(r) % p.q_len;  // last key row r sees
        const bool live = uint32_t(r) < R && lane < n && key <= limit;
        const float x = live ? sc[r] * p.scale : -INFINITY;
        m[r] = wave_max_dpp(x);
        const float e = live ? exp_fast(x - m[r]) : 0.0f;
        l[r] = e;  // this lane's share
        ps[wave][r][lane] = e;
    }
    // the staged value rows have landed (vmcnt) and every wave's
    // probabilities are in LDS (barrier)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    float o[RM][DPL];
#pragma unroll
    for (int r = 0; r < RM; ++r)
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[r][e] = 0.0f;
    // eight keys at a time, their reads issued before the arithmetic.  From
    // the LDS stage every read is unconditional -- rows n .. 63 hold zeros and
    // lanes past the head size read other stage bytes into outputs that are
    // never stored -- so the reads are not serialised behind branches; from
    // memory a read past the wave's rows is skipped.  The LDS and the global variant are
    // separate code so that each read is a plain ds_read or global_load (a
    // pointer that may be either would make every read a flat access with a
    // full wait).
    auto pv = [&](const T* vbase, auto from_lds) {
        constexpr bool LDS = decltype(from_lds)::value;
        auto eight_keys = [&](uint32_t j0) {
            float vv[8][DPL];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
#pragma unroll
                for (int e = 0; e < DPL; ++e) {
                    const uint32_t d = lane * DPL + e;
                    if constexpr (LDS) {
                        vv[u][e] = to_float(vbase[(j0 + u) * D + d]);  // inside the stage
                    } else {
                        vv[u][e] = j0 + u < n && d < D
                                       ? to_float(vbase[uint64_t(j0 + u) * D + d]) : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
#pragma unroll
                for (int r = 0; r < RM; ++r) {
                    const float pj = ps[wave][r][j0 + u];  // 0 for keys past n
#pragma unroll
                    for (int e = 0; e < DPL; ++e) o[r][e] += pj * vv[u][e];
                }
            }
        };
        if constexpr (LDS) {
            // all 64 rows (zeros past n), unrolled so that the reads of later
            // keys issue under the products of earlier ones
#pragma unroll
            for (uint32_t j0 = 0; j0 < 64; j0 += 8) eight_keys(j0);
        } else {
            for (uint32_t j0 = 0; j0 < n; j0 += 8) eight_keys(j0);
        }
    };
    if (staged) {
        pv(reinterpret_cast<const T*>(vstage[wave]), std::true_type{});
    } else {
        pv(vh + uint64_t(base) * D, std::false_type{});
    }
    // the four waves' states -> one partial per row
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const float lsum = wave_sum_dpp(l[r]);
        if (lane == 0) {
            merge_m[wave][r] = m[r];
            merge_l[wave][r] = lsum;
        }
#pragma unroll
        for (int e = 0; e < DPL; ++e) merge_o[wave][r][lane * DPL + e] = o[r][e];
    }
    finish_split<T>(merge_m, merge_l, merge_o, part, tickets, out, p, b, first_head, R, kvb,
                    split, splits);
}

// The split-key decode step on the matrix cores (f16, R <= 16 rows per KV
// head, head size D = 64 or 128).  Per wave of 64 keys: S^T = K Q^T as four
// 16-key tiles of v_mfma_f32_16x16x32_f16 (A = key rows loaded straight
// from memory, B = the query rows; a row past R reads row 0 and is masked),
// then O = P V in two 32-key
// steps (A = P from the score registers, B = value columns read from the
// wave's LDS stage by transpose reads).  Row a of score tile m holds key
// key16(m, a), so that lane l's registers of tiles 2t and 2t + 1 hold keys
// 32 t + 8 (l / 16) + 0..7 of query row l % 16: the P operand of step t as
// they stand.  No barrier before the products (every wave reads only its
// own stage and registers); the end is finish_split's, as for
// k_attention_split.
__device__ inline uint32_t key16(uint32_t m, uint32_t a) {
    return 32 * (m / 2) + 8 * (a / 4) + 4 * (m % 2) + a % 4;
}

// max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (one query row's four
// lane groups).  A swap returns {lower lane's value, upper lane's value} in
// both lanes of a pair, so both compute the same result bit for bit.
__device__ inline float rows4_max(float v) {
    auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                              false);
    v = fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
    s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ inline float rows4_sum(float v) {
    auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                              false);
    v = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Chunk swizzle of the decode's value stage (rows of D halves, 16-byte
// chunks): with chunk c of row r at c ^ stage_swizzle<D>(r), the stage
// writes (16 lanes, 16 bytes each, per LDS cycle) and the transpose reads
// (32 lanes, 8 bytes each: rows 8 g + j, four lanes a row) fall on 64
// distinct 4-byte banks; unswizzled, the reads met 4 (D 64) or 8 (D 128)
// lanes a bank.  Row bits 2 and 5 are not used, so rows + 4 and + 32 share
// a row's swizzle.
template <int D>
__device__ inline uint32_t stage_swizzle(uint32_t r) {
    if constexpr (D == 64)
        return (r & 2u) | ((r >> 1) & 4u);
    else
        return ((r & 3u) << 1) | (r & 8u);
}

template <int D>
__global__ __launch_bounds__(64 * kSplitWaves) void k_attention_split_mfma(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    float* __restrict__ part, uint32_t* __restrict__ tickets, half_t* __restrict__ out,
    AttnParams p, uint32_t splits) {
    static_assert(D == 64 || D == 128, "head size 64 or 128");
    constexpr int RM = 16;
    constexpr int KS = D / 32;  // 32-element steps of the scores
    constexpr int NT = D / 16;  // 16-element tiles of the output
    __shared__ __align__(16) half_t vstage[kSplitWaves][64 * D];
    __shared__ float merge_m[kSplitWaves][RM];
    __shared__ float merge_l[kSplitWaves][RM];
    // rows padded by 4 floats: the 64 lanes' writes below (rows 4 g + r,
    // columns 16 nt + lane % 16) then fall on 64 distinct banks
    __shared__ float merge_o[kSplitWaves][RM][D + 4];
    const uint32_t wave = threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t lr = lane % 16;  // query row of the scores and P, column of the outputs
    const uint32_t g = lane / 16;
    const uint32_t kvb = blockIdx.x / splits;  // b * kv_heads + kv head
    const uint32_t split = blockIdx.x % splits;
    const uint32_t kv_heads = p.q_heads / p.group;
    const uint32_t b = kvb / kv_heads;
    const uint32_t first_head = (kvb % kv_heads) * p.group;
    const uint32_t R = p.group * p.q_len;
    const half_t* kh = k + uint64_t(kvb) * p.kv_head_stride;
    const half_t* vh = v + uint64_t(kvb) * p.kv_head_stride;
    const uint32_t base = split * kSplitKeys + wave * 64;
    const uint32_t n = p.kv_len > base ? min(64u, p.kv_len - base) : 0u;  // this wave's keys

    // every load issued before the first use, unconditional (clamped rows,
    // masked afterwards) so that none waits behind a branch or a select: the
    // query row lr (row r = g' * q_len + qi is query qi of head
    // first_head + g'; a row past R reads row 0, its scores are masked),
    // elements 32 s + 8 g .. + 7
    const bool row_live = lr < R;
    const uint32_t qr = row_live ? lr : 0u;
    const uint64_t qrow = (uint64_t(b) * p.q_heads + first_head + qr / p.q_len) * p.q_len +
                          qr % p.q_len;
    h8 qf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = *reinterpret_cast<const h8*>(q + qrow * D + 32 * s + 8 * g);
    // key rows: tile m, row lr holds key base + key16(m, lr) (a row past the
    // last key reads the last key; its scores are masked below)
    h8 kf[4][KS];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t key = min(base + key16(m, lr), p.kv_len - 1);
        const half_t* krow = kh + uint64_t(key) * D;
#pragma unroll
        for (int s = 0; s < KS; ++s) kf[m][s] = *reinterpret_cast<const h8*>(krow + 32 * s + 8 * g);
    }
    // then the 64 value rows (needed last), 16 bytes a lane, to registers:
    // loads of one kind only, so that the products wait for the key rows
    // alone (vmcnt counts in order); rows past the last key copy the last
    // key's row, whose probability is zero
    h8 vf[D / 8];
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
        const uint32_t c = 64 * i + lane;  // 16-byte piece c of the 64 rows
        const uint32_t key = min(base + c / (D / 8), p.kv_len - 1);
        vf[i] = *reinterpret_cast<const h8*>(vh + uint64_t(key) * D + (c % (D / 8)) * 8);
    }
    // all of them issued before the first wait (the scheduler would
    // otherwise place value loads behind the products' waits for key rows)
    __builtin_amdgcn_sched_barrier(0);

    // S^T: lane l holds query row lr's scores of keys key16(m, 4 g + r)
    f32x4 sc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        sc[m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; ++s)
            sc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[m][s], qf[s], sc[m], 0, 0, 0);
    }
    // the row's max over its 64 keys (16 per lane, four lanes per row) in
    // log2 units, probabilities rounded to f16 as the P operand, and their
    // sum.  Row lr sees the wave's keys below min(n, limit + 1 - base) (none
    // past R); key16(m, 4 g + r) - 8 g is a constant, compared with that
    // count less 8 g.
    const uint32_t limit = p.start + lr % p.q_len;  // last key row lr sees
    const uint32_t causal = limit + 1 > base ? limit + 1 - base : 0u;
    const int seen = row_live ? int(min(n, causal)) - int(8 * g) : 0;
    float x[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int kc = 32 * (m / 2) + 4 * (m % 2) + r;
            x[m][r] = kc < seen ? sc[m][r] * p.scale_log2 : -INFINITY;
            mx = fmaxf(mx, x[m][r]);
        }
    mx = rows4_max(mx);
    // 2^(x - mx), 0 for masked keys (x = -inf; mx = -inf only if every key is);
    // results below 2^-126 flush to zero, as they round to zero in f16
    const float ms = mx == -INFINITY ? 0.0f : mx;
    half_t ph[4][4];
    float lsum = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ph[m][r] = static_cast<half_t>(__builtin_amdgcn_exp2f(x[m][r] - ms));
            lsum += static_cast<float>(ph[m][r]);
        }
    lsum = rows4_sum(lsum);

    // the value rows to the wave's LDS stage (read by this wave only: no
    // barrier), 16-byte chunk c of row r at chunk c ^ stage_swizzle<D>(r)
    half_t* stage = vstage[wave];
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
        const uint32_t c = 64 * i + lane, row = c / (D / 8), ch = c % (D / 8);
        *reinterpret_cast<h8*>(stage + row * D + (ch ^ stage_swizzle<D>(row)) * 8) = vf[i];
    }
    // P V: lane 16 g + 4 j + a reads 4 elements of value rows 32 t + 8 g + j
    // and + 4, columns 16 nt + 4 a (chunk 2 nt + a / 2, swizzled by the row;
    // rows 32 t + 8 g + j + 4 h share the swizzle of row 8 g + j); the
    // transpose hands lane 16 g + i column 16 nt + i of those eight rows
    f32x4 o[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t vrow = 8 * g + lr / 4;
    const uint32_t vsw = stage_swizzle<D>(vrow);
    const half_t* tr = stage + vrow * D + 4 * (lr % 2);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const h8 a = {ph[2 * t][0],     ph[2 * t][1],     ph[2 * t][2],     ph[2 * t][3],
                      ph[2 * t + 1][0], ph[2 * t + 1][1], ph[2 * t + 1][2], ph[2 * t + 1][3]};
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const half_t* src = tr + 32 * t * D + ((2 * nt + (lr % 4) / 2) ^ vsw) * 8;
            const h4 lo = lds_read_transposed(src);
            const h4 hi = lds_read_transposed(src + 4 * D);
            const h8 bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv, o[nt], 0, 0, 0);
        }
    }
    // lane l holds rows 4 g + r, column 16 nt + lr of the wave's output
    if (g == 0) {
        merge_m[wave][lr] = mx * kLn2;  // natural units, as finish_split takes them
        merge_l[wave][lr] = lsum;
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) merge_o[wave][4 * g + r][16 * nt + lr] = o[nt][r];
    finish_split<half_t>(merge_m, merge_l, merge_o, part, tickets, out, p, b, first_head, R,
                         kvb, split, splits);
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

// MFMA kernel shape: 4 waves of 32 queries, two key halves (8 waves); key
// blocks of 128 for head sizes up to 64 and of 64 above (two DMA stages of
// K and V then take 64, 128 and 128 KB of LDS for head sizes 32, 64, 128).
constexpr int kFlashMaxBlockKeys = 128;
constexpr int kFlashMaxKeySplit = 4;
// f32 (one MI355X, all launches inside the events): the 32-query tiles win up to
// at least 128 pairs (8 heads x [4096, 4096]: 203 against 308 us), the wide
// tiles at 180 (15 heads x [3072, 3072]: 240 against 281 us)
constexpr uint64_t kFlashFillBlocks = 180;
constexpr uint64_t kFlashFillBlocksF16 = 96;    // f16: wide tiles from here on

// Workgroup shape: 4 query waves x 2 key shares (128-query tiles) while that
// gives enough workgroups (`fill`); otherwise 32-query tiles, so that short
// or few-head prefills spread over more CUs: 1 query wave x 2 key shares, or
// x 4 when the workgroups are still few or the head is large (96, 128: more
// waves per workgroup keep all four SIMDs busy).  f16, one MI355X, all
// launches of a call inside the events: the wide tiles win from about 96
// workgroups (15 heads x [2048, 2048] causal 31.8 -> 28.7 us, [3072, 3072]
// 71.8 -> 37.0, 8 heads x [4096, 4096] 52.1 -> 44.8) and lose below 64
// (15 heads x [1024, 1024]: 19.1 against 14.2 us for 32-query tiles).
enum class FlashShape { kWide, kNarrow2, kNarrow4 };
FlashShape flash_shape(uint64_t heads, uint64_t q_len, uint64_t head_dim, uint64_t fill) {
    if (heads * ((ceil_div(q_len, 128) + 1) / 2) >= fill) return FlashShape::kWide;
    if (head_dim >= 96 || heads * ((ceil_div(q_len, 32) + 1) / 2) < 256) return FlashShape::kNarrow4;
    return FlashShape::kNarrow2;
}

// Key chunks per 128-query tile for the f16 kernel (1 = no split), W the
// wide tile pairs, steps the longest tile's key steps (two blocks each).
// One workgroup a CU fits (its LDS), so chunks beyond 256 / W workgroups
// queue behind the first wave.  One MI355X, every launch of a call inside
// the events, against what the shape took unsplit: with 96 <= W <= 128 and
// at least 16 steps two chunks (8 heads x [4096, 4096] 45.0 -> 39.5 us on the
// wide tiles, 15 heads x 2048 queries after 2048 cached keys 61.3 -> 47.8,
// 32 heads of 128 x 1024 after 3072 105.8 -> 87.6); below 96 pairs only a
// prefill after cached keys, whose every tile is long, splits, up to 256 / W
// chunks of two steps or more (15 heads x 512 queries after 3584 keys: 51.1
// us on 32-query tiles, 25.5 in 8 chunks; 1024 after 3072: 49.1, 34.2 in 4).
// Causal squares with fewer pairs stay on the 32-query tiles (8 heads of 128
// x [2048, 2048]: 31.8 us against 34.0 in 4 chunks; 15 x [1024, 1024]: 14.0
// against 20.1): each chunk writes and merges another f32 copy of the output.
uint32_t flash_key_chunks(uint64_t heads, uint64_t q_len, uint64_t kv_len, uint64_t start,
                          uint64_t head_dim) {
    const uint64_t wide = heads * ((ceil_div(q_len, 128) + 1) / 2);
    const uint64_t bn = head_dim <= 64 ? 128 : 64;
    const uint64_t keys = std::min<uint64_t>(kv_len, start + q_len);  // the longest tile's
    const uint64_t steps = ceil_div(ceil_div(keys, bn), 2);
    if (wide >= kFlashFillBlocksF16) return wide <= 128 && steps >= 16 ? 2 : 1;
    if (start == 0 || steps < 16) return 1;
    const uint64_t chunks = std::min<uint64_t>({256 / wide, 8, steps / 2});
    return uint32_t(std::max<uint64_t>(chunks, 1));
}

// The matrix-core kernels by head size: f16 in key blocks of 128 (head
// size up to 64 with 128-query tiles) or 64 (32 for head size 128 with
// 32-query tiles), from DMA-fed LDS except head size 96; f32 in blocks of
// 64 (up to 64, 128-query tiles) or 32.
template <int QW, int KS>
void launch_flash(rl_context* ctx, dim3 g, uint32_t nt, const half_t* q, const half_t* k,
                  const half_t* v, half_t* o, const AttnParams& p) {
    constexpr int BN = QW == 4 ? 128 : 64;
    constexpr int BN4 = KS == 4 ? 32 : 64;
    const dim3 b(64 * QW * KS);
    if (nt == 1) {
        RL_LAUNCH(ctx, (k_flash_attention<1, QW, KS, BN, true>), g, b, q, k, v, o, p);
    } else if (nt == 2) {
        RL_LAUNCH(ctx, (k_flash_attention<2, QW, KS, BN, true>), g, b, q, k, v, o, p);
    } else if constexpr (!(QW == 1 && KS == 2)) {  // that shape only for head sizes <= 64
        if (nt == 3) {
            RL_LAUNCH(ctx, (k_flash_attention<3, QW, KS, 64, false>), g, b, q, k, v, o, p);
        } else {
            RL_LAUNCH(ctx, (k_flash_attention<4, QW, KS, BN4, true>), g, b, q, k, v, o, p);
        }
    }
}
// The wide f16 kernel over key chunks (PARTIAL), then the merge.
void launch_flash_split(rl_context* ctx, uint64_t heads, uint32_t nt, const half_t* q,
                        const half_t* k, const half_t* v, half_t* o, const AttnParams& p) {
    const dim3 g(static_cast<unsigned>(heads * p.pairs * p.kchunks)), b(64 * 4 * 2);
    const dim3 gc(static_cast<unsigned>(heads * p.tiles * (128 / kCombineRows))), bc(256);
    if (nt == 1) {
        RL_LAUNCH(ctx, (k_flash_attention<1, 4, 2, 128, true, true>), g, b, q, k, v, o, p);
        RL_LAUNCH(ctx, (k_flash_combine<32, 128>), gc, bc, o, p);
    } else if (nt == 2) {
        RL_LAUNCH(ctx, (k_flash_attention<2, 4, 2, 128, true, true>), g, b, q, k, v, o, p);
        RL_LAUNCH(ctx, (k_flash_combine<64, 128>), gc, bc, o, p);
    } else if (nt == 3) {
        RL_LAUNCH(ctx, (k_flash_attention<3, 4, 2, 64, false, true>), g, b, q, k, v, o, p);
        RL_LAUNCH(ctx, (k_flash_combine<96, 128>), gc, bc, o, p);
    } else {
        RL_LAUNCH(ctx, (k_flash_attention<4, 4, 2, 64, true, true>), g, b, q, k, v, o, p);
        RL_LAUNCH(ctx, (k_flash_combine<128, 128>), gc, bc, o, p);
    }
}

template <int QW, int KS>
void launch_flash(rl_context* ctx, dim3 g, uint32_t nt, const float* q, const float* k,
                  const float* v, float* o, const AttnParams& p) {
    constexpr int BN = QW == 4 ? 64 : 32;
    const dim3 b(64 * QW * KS);
    if (nt == 1) {
        RL_LAUNCH(ctx, (k_flash_attention_f32<1, QW, KS, BN>), g, b, q, k, v, o, p);
    } else if (nt == 2) {
        RL_LAUNCH(ctx, (k_flash_attention_f32<2, QW, KS, BN>), g, b, q, k, v, o, p);
    } else if constexpr (!(QW == 1 && KS == 2)) {  // that shape only for head sizes <= 64
        if (nt == 3) {
            RL_LAUNCH(ctx, (k_flash_attention_f32<3, QW, KS, 32>), g, b, q, k, v, o, p);
        } else {
            RL_LAUNCH(ctx, (k_flash_attention_f32<4, QW, KS, 32>), g, b, q, k, v, o, p);
        }
    }
}

// Which kernel a shape takes: the MFMA kernels for a head size of 32, 64,
// 96 or 128 and 16-byte aligned buffers (f16: also byte offsets into one KV
// head, a block past its end included, that fit the 32-bit buffer offsets
// of its loads); the row kernel otherwise (head sizes up to 512).
template <typename T>
bool use_flash(const AttnShape& s, const void* q, const void* k, const void* v, const void* o) {
    const bool shape = s.head_dim % 32 == 0 && s.head_dim <= 128 && aligned_to(q, 16) &&
                       aligned_to(k, 16) && aligned_to(v, 16) && aligned_to(o, 16);
    if constexpr (!std::is_same<T, half_t>::value) {
        return shape;
    } else {
        const uint64_t span = (s.kv_len + uint64_t(kFlashMaxBlockKeys) * kFlashMaxKeySplit) *
                              s.head_dim * sizeof(T);
        return shape && span <= UINT32_MAX;
    }
}

// ---------------------------------------------- allocation-free decode

// The scratch of rl_attention_f16_noalloc: the decode path's hand-off
// counters (the first kScratchTicketBytes) and its per-split partials (the
// rest), in one file-scope device array instead of the context's counters
// and a pool block.  Each GPU holds its own copy from the library's load
// until the process ends.  The counters are zero at load, the set-up below
// clears them once more, and every launch leaves them zero (the merging
// workgroup puts its counter back); the partials need no clearing (a
// launch writes every slot it reads).  All calls on one GPU share the
// array, so calls that overlap on one GPU (other streams, other threads)
// race; calls on one stream are ordered.
constexpr uint64_t kScratchBytes = uint64_t(8) << 20;
constexpr uint64_t kScratchTicketBytes = uint64_t(256) << 10;
constexpr uint64_t kScratchTicketWords = kScratchTicketBytes / sizeof(uint32_t);
constexpr uint64_t kScratchTickets = kScratchTicketWords / kTicketStride;  // 1024 counters
constexpr uint64_t kScratchPartialBytes = kScratchBytes - kScratchTicketBytes;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void k_zero_u32(uint32_t* __restrict__ p, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// The device address of `scratch` on each device, looked up once per device
// with that device current (the array's name is only a host-side stand-in).
constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
    std::once_flag once;
    void* ptr = nullptr;
    hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxScratchDevices];

rl_status scratch_on_device(rl_context* ctx, void** out) {
    *out = nullptr;
    if (ctx->device < 0 || ctx->device >= kMaxScratchDevices)
        return fail(RL_ERR_DEVICE, "device %d has no scratch slot", ctx->device);
    ScratchSlot& slot = g_scratch[ctx->device];
    std::call_once(slot.once, [&] {
        void* ptr = nullptr;
        hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err == hipSuccess) err = flush_fused(ctx) == RL_OK ? hipSuccess : hipErrorLaunchFailure;
        if (err == hipSuccess) {
            hipLaunchKernelGGL(k_zero_u32, dim3(unsigned(kScratchTicketWords / 256)), dim3(256), 0,
                               ctx->stream, static_cast<uint32_t*>(ptr),
                               uint32_t(kScratchTicketWords));
            err = hipGetLastError();
        }
        slot.err = err;
        slot.ptr = err == hipSuccess ? ptr : nullptr;
    });
    if (slot.err != hipSuccess)
        return fail(RL_ERR_DEVICE, "scratch address: %s", hipGetErrorString(slot.err));
    *out = slot.ptr;
    return RL_OK;
}

// The decode hand-off counters: at least n of them (n * kTicketStride
// words), all zero.  Growing waits for the stream (a launch in flight may
// hold the old array).
rl_status ensure_tickets(rl_context* ctx, uint64_t n) {
    const uint64_t words = n * kTicketStride;
    if (ctx->ticket_count >= words) return RL_OK;
    const uint64_t count = std::max<uint64_t>(words, 256 * kTicketStride);
    hipError_t err = hipStreamSynchronize(ctx->stream);
    if (err == hipSuccess && ctx->tickets != nullptr) err = hipFree(ctx->tickets);
    if (err != hipSuccess) return fail(RL_ERR_DEVICE, "ticket array: %s", hipGetErrorString(err));
    ctx->tickets = nullptr;
    ctx->ticket_count = 0;
    void* mem = nullptr;
    err = hipMalloc(&mem, count * sizeof(uint32_t));
    if (err == hipSuccess) err = hipMemsetAsync(mem, 0, count * sizeof(uint32_t), ctx->stream);
    if (err != hipSuccess) {
        if (mem != nullptr) (void)hipFree(mem);
        return fail(RL_ERR_DEVICE, "ticket array: %s", hipGetErrorString(err));
    }
    ctx->tickets = static_cast<uint32_t*>(mem);
    ctx->ticket_count = count;
    return RL_OK;
}

// Where the decode path keeps its partials and hand-off counters: a pool
// block and the context's counters, or the file-scope scratch.
enum class DecodeScratch { kPool, kStatic };

template <typename T>
rl_status attention_entry(rl_context* ctx, const char* name, const rl_buffer* q,
                          const rl_buffer* k, const rl_buffer* v, const AttnShape& s,
                          float scale, uint64_t start, const rl_buffer* out,
                          DecodeScratch mode = DecodeScratch::kPool) {
    if (rl_status st = validate_attention(q, k, v, s, scale, start, sizeof(T))) return st;
    if (rl_status st = check_output(out, q->len, sizeof(T), "attention")) return st;
    const bool flash = use_flash<T>(s, q->data, k->data, v->data, out->data);
    if (!flash && s.head_dim > 512)
        return fail(RL_ERR_INVALID_SHAPE, "attention head size %llu exceeds 512",
                    (unsigned long long)s.head_dim);
    // Few rows per KV head (decode): split the keys over many workgroups.
    const uint64_t heads = s.batch * s.q_heads;
    const uint64_t rows = heads * s.q_len;
    const uint64_t R = s.q_len * (s.q_heads / s.kv_heads);
    const uint64_t dpl = ceil_div(s.head_dim, 64);
    const uint64_t rm = R <= 4 ? 4 : R <= 8 ? 8 : R <= 16 ? 16 : 32;
    const uint64_t needed = std::min<uint64_t>(s.kv_len, start + s.q_len);  // keys any row sees
    const uint64_t splits = ceil_div(needed, uint64_t(kSplitKeys));
    const bool split_shape = R <= 32 && s.head_dim <= 256 && rm * dpl <= 32 && needed >= 512 &&
                             splits <= kMaxSplits;
    const uint64_t part_bytes = rows * splits * (s.head_dim + 2) * sizeof(float);
    if (mode == DecodeScratch::kStatic && split_shape &&
        (part_bytes > kScratchPartialBytes || s.batch * s.kv_heads > kScratchTickets))
        return fail(RL_ERR_INVALID_SHAPE,
                    "decode attention needs %llu bytes of partials and %llu counters; the "
                    "allocation-free entry holds %llu bytes and %llu counters",
                    (unsigned long long)part_bytes, (unsigned long long)(s.batch * s.kv_heads),
                    (unsigned long long)kScratchPartialBytes,
                    (unsigned long long)kScratchTickets);
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

    // The pooled partials are not used while recording a graph: the block is
    // released (and may be reused) once the launch is enqueued.  The static
    // scratch has no such lifetime.
    if (split_shape && (mode == DecodeScratch::kStatic || !ctx->capturing)) {
        const bool vec_rows = s.head_dim % (16 / sizeof(T)) == 0 && aligned_to(kd, 16) &&
                              aligned_to(vd, 16);
        void* part = nullptr;
        uint32_t* tk = nullptr;
        if (mode == DecodeScratch::kStatic) {
            void* base = nullptr;
            if (rl_status st = scratch_on_device(ctx, &base)) return st;
            tk = static_cast<uint32_t*>(base);
            part = static_cast<unsigned char*>(base) + kScratchTicketBytes;
        } else {
            if (rl_status st = ensure_tickets(ctx, s.batch * s.kv_heads)) return st;
            if (rl_status st = ctx->pool.allocate(part_bytes, &part)) return st;
            tk = ctx->tickets;
        }
        const dim3 gs(static_cast<unsigned>(s.batch * s.kv_heads * splits)), bs(64 * kSplitWaves);
        float* pf = static_cast<float*>(part);
        const uint32_t sp = uint32_t(splits);
        // f16 with at most 16 rows per KV head and head size 64 or 128: the
        // matrix-core kernel
        bool on_mfma = false;
        if constexpr (std::is_same<T, half_t>::value) {
            on_mfma = vec_rows && R <= 16 && (s.head_dim == 64 || s.head_dim == 128) &&
                      aligned_to(qd, 16);
            if (on_mfma && s.head_dim == 64)
                RL_LAUNCH(ctx, k_attention_split_mfma<64>, gs, bs, qd, kd, vd, pf, tk, od, p, sp);
            else if (on_mfma)
                RL_LAUNCH(ctx, k_attention_split_mfma<128>, gs, bs, qd, kd, vd, pf, tk, od, p, sp);
        }
#define RL_SPLIT(RMV, DPLV)                                                                    \
    RL_LAUNCH(ctx, (k_attention_split<T, RMV, DPLV>), gs, bs, qd, kd, vd, pf, tk, od, p, sp,   \
              vec_rows)
        if (!on_mfma) {
            if (rm == 4 && dpl == 1) RL_SPLIT(4, 1);
            else if (rm == 4 && dpl == 2) RL_SPLIT(4, 2);
            else if (rm == 4) RL_SPLIT(4, 4);
            else if (rm == 8 && dpl == 1) RL_SPLIT(8, 1);
            else if (rm == 8 && dpl == 2) RL_SPLIT(8, 2);
            else if (rm == 8) RL_SPLIT(8, 4);
            else if (rm == 16 && dpl == 1) RL_SPLIT(16, 1);
            else if (rm == 16) RL_SPLIT(16, 2);
            else RL_SPLIT(32, 1);
        }
#undef RL_SPLIT
        const rl_status st = after_launch(ctx, name);
        if (mode == DecodeScratch::kPool)
            ctx->pool.release(part);  // stream-ordered: later users run after this launch
        return st;
    }
    if (flash) {
        if constexpr (std::is_same<T, half_t>::value) {
            // Too few 128-query tile pairs to fill the CUs: keep the wide
            // tiles and split each tile's key steps over workgroups
            // (chunked prefill, short or few-head prefills), the pool holding
            // the partials (not while a graph records, nor for the
            // allocation-free entry).
            const uint32_t chunks = flash_key_chunks(heads, s.q_len, s.kv_len, start, s.head_dim);
            if (chunks > 1 && mode == DecodeScratch::kPool && !ctx->capturing) {
                p.tiles = uint32_t(ceil_div(s.q_len, 128));
                p.pairs = (p.tiles + 1) / 2;
                p.kchunks = chunks;
                const uint64_t units = heads * p.tiles * chunks * 128;
                void* part = nullptr;
                if (rl_status st = ctx->pool.allocate(units * (s.head_dim + 2) * sizeof(float), &part))
                    return st;
                p.part = static_cast<float*>(part);
                p.part_ml = p.part + units * s.head_dim;
                launch_flash_split(ctx, heads, uint32_t(s.head_dim / 32), qd, kd, vd, od, p);
                const rl_status st = after_launch(ctx, name);
                ctx->pool.release(part);  // stream-ordered: later users run after these launches
                return st;
            }
        }
        const FlashShape shape =
            flash_shape(heads, s.q_len, s.head_dim,
                        sizeof(T) == 2 ? kFlashFillBlocksF16 : kFlashFillBlocks);
        p.tiles = uint32_t(ceil_div(s.q_len, shape == FlashShape::kWide ? 128 : 32));
        p.pairs = (p.tiles + 1) / 2;
        const uint64_t grid = heads * p.pairs;
        if (grid > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "attention grid exceeds u32");
        const dim3 g(static_cast<unsigned>(grid));
        const uint32_t nt = uint32_t(s.head_dim / 32);
        if (shape == FlashShape::kWide) launch_flash<4, 2>(ctx, g, nt, qd, kd, vd, od, p);
        else if (shape == FlashShape::kNarrow2) launch_flash<1, 2>(ctx, g, nt, qd, kd, vd, od, p);
        else launch_flash<1, 4>(ctx, g, nt, qd, kd, vd, od, p);
        return after_launch(ctx, name);
    }
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

rl_status rl_attention_f16_noalloc(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                                   const rl_buffer* v, uint64_t batch, uint64_t q_heads,
                                   uint64_t kv_heads, uint64_t q_len, uint64_t kv_len,
                                   uint64_t head_dim, uint64_t kv_capacity, float scale,
                                   uint64_t query_start_pos, const rl_buffer* out) {
    const AttnShape s{batch, q_heads, kv_heads, q_len, kv_len, head_dim, kv_capacity};
    return attention_entry<half_t>(ctx, "attention_f16", q, k, v, s, scale, query_start_pos,
                                   out, DecodeScratch::kStatic);
}

}  // extern "C"
