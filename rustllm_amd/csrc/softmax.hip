// softmax.hip -- row softmax, attention scale/mask, and the two fused, for
// gfx950.
//
// Softmax (kernels/softmax.metal) reads each row three times through a
// 256-thread group with two 8-barrier shared-memory trees.  Here a row is
// held in VGPRs by a group of TPR = 64, 128 or 256 threads (one to four
// waves) with up to NV 16-byte packs per thread: one HBM read, a max
// reduction, exp in registers, a sum reduction, one write.  Reductions are
// wave64 butterflies of cross-lane shuffles; LDS is used only to combine the
// waves of a group.  A sweep of 64/128/256 threads per row on the causal
// configurations ([9, 2048, 2048] f32, [15, 4096, 4096] f16) found two waves
// per row with four packs per thread best: 73% / 76% of HBM peak, against
// 66% / 71% for one wave per row with eight packs.  Rows longer than
// 256 x 16 packs use a streaming kernel with an online (max, sum) merge and
// a second read.
//
// Scale/mask + softmax fused (the adjacent calls at nn/attention.rs:233-240):
// for query row q the keys past start + q are masked, so their scores are
// never read; the kept scores are scaled (and, for f16, rounded to f16 as
// the scale/mask kernel's output would be) before the softmax.  Masked
// outputs are 0 * (1 / sum): exact zeros, or NaN exactly where the two-op
// composition gives NaN.
//
// The standalone scale/mask op also skips reading masked scores: its output
// there is -inf whatever the input.
//
// exp(x - max) runs on the hardware exp2 (exp_fast in common.hpp, subnormal
// results kept): relative error <= |x - max| * log2(e) * 2^-24 * ln 2 plus
// ~1 ulp, i.e. <= 2e-6 for scores within 40 of the row max, inside the 1e-5
// bar; the IEEE expf would make the f16 rows ALU-bound.  The normaliser is
// one correctly rounded 1 / sum per row.
#include "common.hpp"

namespace rl {
namespace {

constexpr int kThreads = 256;
constexpr int kWave = 64;

struct MaskParams {
    float scale;
    FastDiv query_len;
    uint32_t start;
};

// The scale/mask op's output for a kept score: the f32 product, rounded to
// T.  For f16 the empty asm keeps the product in a register: without it the
// compiler folds the multiply and the rounding into one v_fma_mixlo_f16
// with a +0 addend, which turns the -0 product of a -0 score into +0.
template <typename T>
__device__ inline T scale_to(T raw, float scale) {
    float p = to_float(raw) * scale;
    if constexpr (sizeof(T) == 2) asm volatile("" : "+v"(p));
    return from_float<T>(p);
}

// Score as the scale/mask op would store it, widened back to float.
template <typename T>
__device__ inline float scaled_score(T raw, float scale) {
    return to_float(scale_to<T>(raw, scale));
}

template <typename T>
__device__ inline bool is_f16() {
    return sizeof(T) == 2;
}

// exp(d), d = x - max <= 0, for a row of T outputs p = e * (1 / sum), sum >= 1.
// f32 keeps subnormal e (exp_fast).  For f16 the bare v_exp_f32 suffices:
// where it flushes (e < 2^-126) p < 2^-126 rounds to 0 in f16 either way and
// the sum is unchanged; three VALU operations instead of eight matter here,
// as the f16 rows carry twice the elements per byte.
template <typename T>
__device__ inline float exp_row(float d) {
    if constexpr (sizeof(T) == 2)
        return __builtin_amdgcn_exp2f(d * 1.44269504088896340736f);
    else
        return exp_fast(d);
}

// Number of unmasked keys of a row: keys 0 ..= start + q are kept.
__device__ inline uint32_t kept_keys(uint32_t row, uint32_t width, const MaskParams& mp) {
    uint32_t q, qi;
    mp.query_len.divmod(row, q, qi);
    uint64_t kept = uint64_t(mp.start) + qi + 1;
    return kept < width ? uint32_t(kept) : width;
}

// Max / sum over the TPR threads of a row group (the waves of a group are
// consecutive): DPP within each wave, LDS across its waves.  `lds` holds one slot per wave of the block and is written
// once per call; callers separate consecutive uses by a barrier.
template <int TPR>
__device__ inline float group_max(float v, float* lds) {
    v = wave_max_dpp(v);
    if constexpr (TPR > kWave) {
        constexpr int WPR = TPR / kWave;
        if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = v;
        __syncthreads();
        const int first = (threadIdx.x / TPR) * WPR;
        float r = lds[first];
#pragma unroll
        for (int w = 1; w < WPR; ++w) r = fmaxf(r, lds[first + w]);
        v = r;
    }
    return v;
}

template <int TPR>
__device__ inline float group_sum(float v, float* lds) {
    v = wave_sum_dpp(v);
    if constexpr (TPR > kWave) {
        constexpr int WPR = TPR / kWave;
        if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = v;
        __syncthreads();
        const int first = (threadIdx.x / TPR) * WPR;
        float r = 0.0f;
#pragma unroll
        for (int w = 0; w < WPR; ++w) r += lds[first + w];
        v = r;
    }
    return v;
}

// ------------------------------------------ a row per TPR threads, in VGPRs

// Block b takes rows row_base + b * RPB ... + RPB - 1 (RPB = kThreads / TPR).
// Threads of a group past the last row take part in the barriers with no
// memory accesses.  (One group per block, no grid-stride loop: the loop
// doubled the VGPR count of the masked f16 variant.)
// RAGGED: the width is not a multiple of N, so a row starts off the 16-byte
// grid.  Pack p still holds the row's elements p * N .. p * N + N - 1, read
// and written as unaligned 16-byte accesses (load_stream_u / store_stream_u,
// VecOfU: the element alignment the pointers have); a row's partial last
// pack reads on into the next row (masked) and is written element by
// element.  Only the buffer's last pack can reach past its end: that load
// is moved back inside the buffer and the pack reloaded element by element.
// The buffer holds at least N elements (smaller ones take k_softmax_stream).
// CACHED: rows on the grid read with plain loads (a launch reading less than
// kStreamReadBytes), otherwise streamed.
template <typename T, int N, int NV, int TPR, bool MASK, bool RAGGED, bool CACHED>
__global__ __launch_bounds__(kThreads) void k_softmax_rows(const T* __restrict__ in,
                                                           T* __restrict__ out, uint32_t row_base,
                                                           uint32_t rows, uint32_t width,
                                                           MaskParams mp) {
    typedef typename VecOf<T, N>::type V;
    constexpr int RPB = kThreads / TPR;
    __shared__ float lds_m[kThreads / kWave];
    __shared__ float lds_s[kThreads / kWave];
    const uint32_t lane = threadIdx.x % TPR;
    const uint32_t w_packs = width / N;
    {
        const uint64_t row64 = uint64_t(row_base) + uint64_t(blockIdx.x) * RPB + threadIdx.x / TPR;
        const bool active = row64 < rows;
        const uint32_t row = uint32_t(row64);
        const uint64_t e0 = uint64_t(active ? row : 0) * width;  // the row's first element
        const uint32_t n_packs = RAGGED ? (width + N - 1) / N : w_packs;
        const V* src = reinterpret_cast<const V*>(in + e0);
        V* dst = reinterpret_cast<V*>(out + e0);
        const uint32_t kept = !active ? 0u : MASK ? kept_keys(row, width, mp) : width;

        float v[NV][N];
        float m = -INFINITY;
        {
            // Every lane issues all its loads before using any: a pack past
            // the row's last kept key (or past the row) reloads that last
            // kept pack -- a line the wave reads anyway -- and its elements
            // are masked by a select.  With a branch per pack the compiler
            // waited for each load before issuing the next.
            const uint32_t live = (kept + N - 1) / N;  // packs holding a kept key
            const uint32_t last = live > 0 ? live - 1 : 0u;
            const uint64_t total = uint64_t(rows) * width;
            V raw[NV];
            bool moved[NV];
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const uint32_t p = lane + k * TPR;
                const uint32_t q = p < last ? p : last;
                if constexpr (RAGGED) {
                    const uint64_t off = e0 + uint64_t(q) * N;
                    moved[k] = off + N > total;  // the buffer's last pack
                    raw[k] = load_stream_u<T, N>(in + (moved[k] ? total - N : off));
                } else if constexpr (CACHED) {
                    raw[k] = src[q];
                } else {
                    raw[k] = load_stream(src + q);
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the arithmetic
            if constexpr (RAGGED) {
#pragma unroll
                for (int k = 0; k < NV; ++k) {
                    if (moved[k]) {
                        const uint32_t p = lane + k * TPR;
                        const uint32_t q = p < last ? p : last;
#pragma unroll
                        for (int j = 0; j < N; ++j)
                            raw[k][j] = q * N + j < width ? in[e0 + q * N + j] : T(0.0f);
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const uint32_t p = lane + k * TPR;
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    const float f = MASK ? scaled_score(raw[k][j], mp.scale) : to_float(raw[k][j]);
                    v[k][j] = p * N + j < kept ? f : -INFINITY;
                    m = fmaxf(m, v[k][j]);
                }
            }
        }
        m = group_max<TPR>(m, lds_m);
        // softmax.metal:166-173: an f16 row whose max is -inf is all zeros.
        const bool zero_row = is_f16<T>() && m == -INFINITY;
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const uint32_t p = lane + k * TPR;
            if (!zero_row && p < n_packs && p * N < kept) {
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    float e = exp_row<T>(v[k][j] - m);
                    v[k][j] = e;
                    s += e;
                }
            } else {
#pragma unroll
                for (int j = 0; j < N; ++j) v[k][j] = 0.0f;
            }
        }
        s = group_sum<TPR>(s, lds_s);
        const float inv = zero_row ? 0.0f : 1.0f / s;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const uint32_t p = lane + k * TPR;
            if (!active || p >= n_packs) continue;
            V o;
#pragma unroll
            for (int j = 0; j < N; ++j) o[j] = from_float<T>(v[k][j] * inv);
            if constexpr (RAGGED) {
                if (p * N + N <= width) {
                    store_stream_u<T, N>(out + e0 + uint64_t(p) * N, o);
                } else {  // the row's partial last pack
#pragma unroll
                    for (int j = 0; j < N; ++j)
                        if (p * N + j < width) out[e0 + p * N + j] = o[j];
                }
            } else {
                store_stream(dst + p, o);
            }
        }
    }
}

// ----------------------- f16 rows, the first pass on pairs of halves

// k_softmax_rows for f16 rows whose scale is itself an f16 value (the fused
// scale/mask at 1/8, 1/sqrt(64), ...; 1 for the plain softmax).  On the
// [15, 4096, 4096] causal scores k_softmax_rows keeps the SIMDs' vector ALUs
// ~93% busy (counters: 14 VALU instructions per element), almost all of it
// in the first pass, which widens, scales, rounds, indexes, compares and
// selects every element of every row.  Here that pass works on pairs of
// halves (v_pk_mul_f16, v_pk_max_f16) and masks whole packs:
//  * the scaled score is one f16 multiply: x * scale with x and scale f16
//    values is exact in f32 (11 + 11 significant bits), so rounding it once
//    to f16 gives the scale/mask op's f16 output (f32 product, then RNE);
//  * a pack past the row's last kept key becomes -inf by one select per
//    pair; the one pack of a row that holds its last kept key masks its
//    remaining elements in a branch that only that row's lane takes;
//  * the row max is a max of pairs (NaN scores are ignored, as fmaxf does),
//    widened once.
// exp(x - max) is exp2(x * log2 e - max * log2 e), one FMA with the pair
// element widened in the FMA, where |max| <= 256: the rounding of
// max * log2 e adds at most |max| * 6e-8 relative error (<= 1.6e-5, 0.03 ulp
// of f16); larger maxima take (x - max) * log2 e.  A pack past the row's
// last kept key stores 0 * (1 / sum), computed once per row: +0, or NaN
// where a NaN score made the sum NaN, as in the two-op composition.
typedef half_t h2v __attribute__((ext_vector_type(2)));

template <bool NEAR>
__device__ inline float exp_arg(float x, float m, float mL) {
    constexpr float kLog2e = 1.44269504088896340736f;
    if constexpr (NEAR)
        return fmaf(x, kLog2e, -mL);
    else
        return (x - m) * kLog2e;
}

// exp of the kept packs' scores (ev), and their sum; packs past the last
// kept key are left unset (the store writes them without ev).
template <int NV, bool NEAR>
__device__ inline float exp_packs(const h2v (&s)[NV][4], float (&ev)[NV][8], float m,
                                  uint32_t lane, uint32_t tpr, uint32_t kept) {
    const float mL = m * 1.44269504088896340736f;
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if ((lane + k * tpr) * 8 < kept) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = static_cast<float>(s[k][e / 2][e % 2]);
                ev[k][e] = __builtin_amdgcn_exp2f(exp_arg<NEAR>(x, m, mL));
                sum += ev[k][e];
            }
        }
    }
    return sum;
}

// CACHED: rows on the 16-byte grid read with plain loads (a launch reading
// less than kStreamReadBytes); otherwise streamed.  Ragged rows always load
// plainly.
template <int NV, int TPR, bool MASK, bool RAGGED, bool CACHED>
__global__ __launch_bounds__(kThreads) void k_softmax_rows_h2(const half_t* __restrict__ in,
                                                              half_t* __restrict__ out,
                                                              uint32_t row_base, uint32_t rows,
                                                              uint32_t width, MaskParams mp,
                                                              h2v scale2) {
    constexpr int N = 8;
    typedef typename VecOf<half_t, N>::type V;
    constexpr int RPB = kThreads / TPR;
    __shared__ float lds_m[kThreads / kWave];
    __shared__ float lds_s[kThreads / kWave];
    const uint32_t lane = threadIdx.x % TPR;
    const uint64_t row64 = uint64_t(row_base) + uint64_t(blockIdx.x) * RPB + threadIdx.x / TPR;
    const bool active = row64 < rows;
    const uint32_t row = uint32_t(row64);
    const uint64_t e0 = uint64_t(active ? row : 0) * width;
    const uint32_t n_packs = RAGGED ? (width + N - 1) / N : width / N;
    const V* src = reinterpret_cast<const V*>(in + e0);
    V* dst = reinterpret_cast<V*>(out + e0);
    const uint32_t kept = !active ? 0u : MASK ? kept_keys(row, width, mp) : width;

    // Loads as in k_softmax_rows: all issued first, packs past the last
    // kept one reloading it (their values are replaced by -inf below).
    V raw[NV];
    {
        const uint32_t live = (kept + N - 1) / N;
        const uint32_t last = live > 0 ? live - 1 : 0u;
        const uint64_t total = uint64_t(rows) * width;
        bool moved[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const uint32_t p = lane + k * TPR;
            const uint32_t q = p < last ? p : last;
            if constexpr (RAGGED) {
                // Plain loads: a 1 KB wave load of a ragged row shares its
                // first and last 128-byte lines with the next and previous
                // wave loads, which then hit in L2 ([15, 4093, 4093]
                // 149.6 -> 148.3 us, 4090 keys 139.3 -> 136.7, 4095 keys
                // 151.8 -> 150.1, one MI355X; streamed loads re-fetch them).
                const uint64_t off = e0 + uint64_t(q) * N;
                moved[k] = off + N > total;  // the buffer's last pack
                raw[k] = load_u<half_t, N>(in + (moved[k] ? total - N : off));
            } else if constexpr (CACHED) {
                raw[k] = src[q];
            } else {
                raw[k] = load_stream(src + q);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (RAGGED) {
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                if (moved[k]) {
                    const uint32_t p = lane + k * TPR;
                    const uint32_t q = p < last ? p : last;
#pragma unroll
                    for (int j = 0; j < N; ++j)
                        raw[k][j] = q * N + j < width ? in[e0 + q * N + j] : half_t(0.0f);
                }
            }
        }
    }

    // Masked halves become -inf before the multiply (-inf * scale = -inf),
    // so every operand of the max is a multiply's result: canonical, which
    // spares the max its canonicalising of each operand.
    const h2v ninf2 = {half_t(-INFINITY), half_t(-INFINITY)};
    h2v s[NV][4];
    h2v mx = ninf2;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t b = (lane + k * TPR) * N;  // the pack's first key
        const bool none = b >= kept;
        h2v r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = none ? ninf2 : h2v{raw[k][2 * j], raw[k][2 * j + 1]};
        if (!none && b + N > kept) {  // the pack holding the row's last kept key
#pragma unroll
            for (int e = 0; e < N; ++e)
                if (b + e >= kept) r[e / 2][e % 2] = half_t(-INFINITY);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[k][j] = r[j] * scale2;
            mx = __builtin_elementwise_max(mx, s[k][j]);
        }
    }
    float m = fmaxf(static_cast<float>(mx[0]), static_cast<float>(mx[1]));
    m = group_max<TPR>(m, lds_m);
    // softmax.metal:166-173: an f16 row whose max is -inf is all zeros.
    const bool zero_row = m == -INFINITY;
    float ev[NV][8];
    float sum = 0.0f;
    if (!zero_row) {
        if (fabsf(m) <= 256.0f)
            sum = exp_packs<NV, true>(s, ev, m, lane, TPR, kept);
        else
            sum = exp_packs<NV, false>(s, ev, m, lane, TPR, kept);
    }
    sum = group_sum<TPR>(sum, lds_s);
    const float inv = zero_row ? 0.0f : 1.0f / sum;
    // A pack past the last kept key (or any pack of an all-zero row) holds
    // 0 * (1 / sum) in every element: +0, or NaN where the sum is NaN or 0.
    const half_t fill = from_float<half_t>(0.0f * inv);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t p = lane + k * TPR;
        if (!active || p >= n_packs) continue;
        V o;
        if (zero_row || p * N >= kept) {
#pragma unroll
            for (int e = 0; e < N; ++e) o[e] = fill;
        } else {
#pragma unroll
            for (int e = 0; e < N; ++e) o[e] = from_float<half_t>(ev[k][e] * inv);
        }
        if constexpr (RAGGED) {
            if (p * N + N <= width) {
                store_stream_u<half_t, N>(out + e0 + uint64_t(p) * N, o);
            } else {  // the row's partial last pack
#pragma unroll
                for (int e = 0; e < N; ++e)
                    if (p * N + e < width) out[e0 + p * N + e] = o[e];
            }
        } else {
            store_stream(dst + p, o);
        }
    }
}

// ------------------------------------- streaming rows of any width (2 reads)

// Online merge of (max, sum of exp(x - max)) pairs.
// The new maximum's own term is exp(x - x): 1, or NaN for x = +inf exactly
// as exp(inf - inf) in the reference's sum.
__device__ inline void online_add(float& m, float& s, float x) {
    if (x > m) {
        s = s * exp_fast(m - x) + exp_fast(x - x);
        m = x;
    } else {
        s += exp_fast(x - m);
    }
}

// A pair whose max is still -inf holds s = 0, or NaN if it met a NaN score;
// multiplying by 0 keeps that NaN (the reference's sum is NaN then) without
// forming exp(-inf - -inf).
__device__ inline float rescale(float s, float m, float new_m) {
    return s * ((m == -INFINITY) ? 0.0f : expf(m - new_m));
}

template <typename T, bool MASK>
__global__ __launch_bounds__(kThreads) void k_softmax_stream(const T* __restrict__ in,
                                                             T* __restrict__ out, uint32_t rows,
                                                             uint32_t width, MaskParams mp) {
    __shared__ float lds_m[kThreads / kWave];
    __shared__ float lds_s[kThreads / kWave];
    for (uint32_t row = blockIdx.x; row < rows; row += gridDim.x) {
        __syncthreads();  // the previous row's lds reads are done
        const uint64_t off = uint64_t(row) * width;
        const uint32_t kept = MASK ? kept_keys(row, width, mp) : width;
        auto score = [&](uint32_t i) -> float {
            if constexpr (MASK) return scaled_score(in[off + i], mp.scale);
            return to_float(in[off + i]);
        };
        float m = -INFINITY, s = 0.0f;
        for (uint32_t i = threadIdx.x; i < kept; i += kThreads) {
            float x = score(i);
            // A -inf score adds exp(-inf - m) = 0 once the row max is finite;
            // if the max stays -inf the row is handled as a whole below.
            if (x == -INFINITY) continue;
            online_add(m, s, x);
        }
        for (int offset = 32; offset > 0; offset >>= 1) {
            float om = __shfl_xor(m, offset, 64);
            float os = __shfl_xor(s, offset, 64);
            float nm = fmaxf(m, om);
            s = rescale(s, m, nm) + rescale(os, om, nm);
            m = nm;
        }
        if (threadIdx.x % kWave == 0) {
            lds_m[threadIdx.x / kWave] = m;
            lds_s[threadIdx.x / kWave] = s;
        }
        __syncthreads();
        float gm = -INFINITY;
#pragma unroll
        for (int w = 0; w < kThreads / kWave; ++w) gm = fmaxf(gm, lds_m[w]);
        float gs = 0.0f;
#pragma unroll
        for (int w = 0; w < kThreads / kWave; ++w) gs += rescale(lds_s[w], lds_m[w], gm);
        if (gm == -INFINITY) {
            // Every kept score is -inf: f16 writes zeros (softmax.metal:166-173),
            // f32 yields NaN as exp(-inf - -inf) does in the reference.
            const T fill = from_float<T>(is_f16<T>() ? 0.0f : __builtin_nanf(""));
            for (uint32_t i = threadIdx.x; i < width; i += kThreads) out[off + i] = fill;
            continue;
        }
        // NaN scores make gs NaN, and every output NaN, as in the reference.
        const float inv = 1.0f / gs;
        for (uint32_t i = threadIdx.x; i < width; i += kThreads) {
            float e = (i < kept) ? exp_fast(score(i) - gm) : 0.0f;
            out[off + i] = from_float<T>(e * inv);
        }
    }
}

// ------------------------------------------------------ scale/mask alone

// RAGGED: rows on the buffer's 16-byte pack grid as in k_softmax_rows.
// Plain loads, streamed stores.  Streamed loads never won: level or slower
// with the input cold or just written by a producer's streamed stores, and
// far slower after a producer's plain stores -- how QK^T writes rows off the
// 128-byte line grid ([15, 4093, 4093] f16 171.7 -> 155.7 us, 4088 keys
// 161 -> 140, [15, 2047, 2047] cold 45 -> 35 us).
template <typename T, int N, bool RAGGED>
__global__ __launch_bounds__(kThreads) void k_scale_mask(const T* __restrict__ in,
                                                         T* __restrict__ out, uint32_t rows,
                                                         uint32_t width, MaskParams mp) {
    typedef typename VecOf<T, N>::type V;
    const uint32_t w_packs = width / N;
    for (uint32_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const uint64_t e0 = uint64_t(row) * width;
        const uint32_t lead = RAGGED ? uint32_t(e0 % N) : 0u;
        const uint32_t n_packs = RAGGED ? (lead + width + N - 1) / N : w_packs;
        const V* src = reinterpret_cast<const V*>(in + (e0 - lead));
        V* dst = reinterpret_cast<V*>(out + (e0 - lead));
        const uint32_t kept = kept_keys(row, width, mp);
        for (uint32_t p = threadIdx.x; p < n_packs; p += kThreads) {
            if (RAGGED && (p * N < lead || p * N + N > lead + width)) {
                // a pack shared with a neighbouring row: read whole where it
                // lies in the buffer, this row's elements written one by one
                V raw = {};
                if (e0 - lead + uint64_t(p + 1) * N <= uint64_t(rows) * width) {
                    raw = src[p];
                } else {
#pragma unroll
                    for (int j = 0; j < N; ++j)
                        if (p * N + j >= lead && p * N + j < lead + width)
                            raw[j] = in[e0 + (p * N + j - lead)];
                }
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    const uint32_t pj = p * N + j;
                    if (pj < lead || pj >= lead + width) continue;
                    const uint32_t x = pj - lead;
                    out[e0 + x] = x < kept ? scale_to<T>(raw[j], mp.scale)
                                           : from_float<T>(-INFINITY);
                }
                continue;
            }
            V o;
            if (p * N < kept + lead) {
                V raw = src[p];
#pragma unroll
                for (int j = 0; j < N; ++j)
                    o[j] = (p * N + j < kept + lead) ? scale_to<T>(raw[j], mp.scale)
                                                     : from_float<T>(-INFINITY);
            } else {
#pragma unroll
                for (int j = 0; j < N; ++j) o[j] = from_float<T>(-INFINITY);
            }
            store_stream(dst + p, o);
        }
    }
}

// ---------------------------------------------------------------- launch

// Elements a softmax launch reads: every row's kept keys (query qi of a
// masked row keeps min(width, start + qi + 1)), summed per query_len rows.
inline uint64_t softmax_read_bytes(uint64_t rows, uint64_t width, const MaskParams& mp,
                                   bool mask) {
    if (!mask) return rows * width;
    const uint64_t q = mp.query_len.divisor, a = uint64_t(mp.start) + 1;
    const uint64_t open = a > width ? 0 : std::min<uint64_t>(q, width - a + 1);  // unclamped
    const uint64_t per_group = open * a + open * (open - 1) / 2 + (q - open) * width;
    return (rows / q) * per_group + (rows % q) * width;
}

// Blocks for a grid-stride loop over `items` (rows or row groups).
inline unsigned row_grid(uint64_t items) {
    return unsigned(items < (uint64_t(1) << 20) ? items : (uint64_t(1) << 20));
}

template <typename T, bool MASK>
rl_status launch_softmax(rl_context* ctx, const char* name, const T* in, T* out, uint64_t rows,
                         uint64_t width, MaskParams mp) {
    if (rl_status st = activate(ctx)) return st;
    constexpr int N = 16 / sizeof(T);
    const uint32_t r32 = uint32_t(rows), w32 = uint32_t(width);
    // Rows on the buffer's 16-byte pack grid; a width that is not a multiple
    // of the pack takes the ragged variant, whose rows span at most one pack
    // more (one more per thread).
    // Ragged rows (a width that is not a multiple of the pack) take the
    // same pack counts with unaligned packs; a buffer of fewer than N
    // elements streams.
    const bool packs_ok = aligned_to(in, 16) && aligned_to(out, 16) && rows * width >= uint64_t(N);
    const bool ragged = width % N != 0;
    const uint64_t w_packs = ceil_div(width, N);
    const dim3 block(kThreads);
    // f16 rows whose scale is an f16 value take the first pass on pairs
    // (k_softmax_rows_h2); the plain softmax's scale is 1.  Rows on the
    // 16-byte grid load plainly when the launch reads little (kept keys only;
    // f32 [15, 2048, 2048] causal 63.3 -> 58.9 us, f16 33.7 -> 25.3 us).
    const bool cached = softmax_read_bytes(rows, width, mp, MASK) * sizeof(T) <= kStreamReadBytes;
    bool pairs = false;
    h2v scale2 = {half_t(1.0f), half_t(1.0f)};
    if constexpr (sizeof(T) == 2) {
        const half_t hs = static_cast<half_t>(mp.scale);
        pairs = static_cast<float>(hs) == mp.scale;
        scale2 = h2v{hs, hs};
    }
    // Row chunks of at most 2^30 blocks each (one launch for any real shape).
#define RL_SOFTMAX_ROWS_R(NV, TPR, R)                                                            \
    do {                                                                                         \
        for (uint64_t base = 0; base < rows; base += (uint64_t(1) << 30) * (kThreads / TPR)) { \
            const uint64_t left = ceil_div(rows - base, kThreads / TPR);                         \
            const dim3 grid(unsigned(left < (uint64_t(1) << 30) ? left : (uint64_t(1) << 30)));  \
            if constexpr (sizeof(T) == 2) {                                                      \
                if (pairs && !R && cached) {                                                     \
                    RL_LAUNCH(ctx, (k_softmax_rows_h2<NV, TPR, MASK, R, true>), grid, block, in, \
                              out, uint32_t(base), r32, w32, mp, scale2);                        \
                    continue;                                                                    \
                }                                                                                \
                if (pairs) {                                                                     \
                    RL_LAUNCH(ctx, (k_softmax_rows_h2<NV, TPR, MASK, R, false>), grid, block,    \
                              in, out, uint32_t(base), r32, w32, mp, scale2);                    \
                    continue;                                                                    \
                }                                                                                \
            }                                                                                    \
            if (!R && cached)                                                                    \
                RL_LAUNCH(ctx, (k_softmax_rows<T, N, NV, TPR, MASK, R, true>), grid, block, in,  \
                          out, uint32_t(base), r32, w32, mp);                                    \
            else                                                                                 \
                RL_LAUNCH(ctx, (k_softmax_rows<T, N, NV, TPR, MASK, R, false>), grid, block, in, \
                          out, uint32_t(base), r32, w32, mp);                                    \
        }                                                                                        \
    } while (0)
#define RL_SOFTMAX_ROWS(NV, TPR)                    \
    do {                                            \
        if (ragged)                                 \
            RL_SOFTMAX_ROWS_R(NV, TPR, true);       \
        else                                        \
            RL_SOFTMAX_ROWS_R(NV, TPR, false);      \
    } while (0)
    if (packs_ok && w_packs <= 64)
        RL_SOFTMAX_ROWS(1, 64);
    else if (packs_ok && w_packs <= 128)
        RL_SOFTMAX_ROWS(2, 64);
    else if (packs_ok && w_packs <= 256)
        RL_SOFTMAX_ROWS(4, 64);
    else if (packs_ok && w_packs <= 512)
        RL_SOFTMAX_ROWS(4, 128);
    else if (packs_ok && w_packs <= 1024)
        RL_SOFTMAX_ROWS(4, 256);
    else if (packs_ok && w_packs <= 2048)
        RL_SOFTMAX_ROWS(8, 256);
    else if (packs_ok && w_packs <= 4096)
        RL_SOFTMAX_ROWS(16, 256);
    else
        RL_LAUNCH(ctx, (k_softmax_stream<T, MASK>), dim3(row_grid(rows)), block, in, out, r32,
                  w32, mp);
#undef RL_SOFTMAX_ROWS
#undef RL_SOFTMAX_ROWS_R
    return after_launch(ctx, name);
}

template <typename T>
rl_status launch_scale_mask(rl_context* ctx, const char* name, const T* in, T* out,
                            uint64_t rows, uint64_t width, MaskParams mp) {
    if (rl_status st = activate(ctx)) return st;
    constexpr int N = 16 / sizeof(T);
    const bool packs_ok = aligned_to(in, 16) && aligned_to(out, 16);
    if (packs_ok && width % N == 0)
        RL_LAUNCH(ctx, (k_scale_mask<T, N, false>), dim3(row_grid(rows)), dim3(kThreads), in,
                  out, uint32_t(rows), uint32_t(width), mp);
    else if (packs_ok)
        RL_LAUNCH(ctx, (k_scale_mask<T, N, true>), dim3(row_grid(rows)), dim3(kThreads), in,
                  out, uint32_t(rows), uint32_t(width), mp);
    else
        RL_LAUNCH(ctx, (k_scale_mask<T, 1, false>), dim3(row_grid(rows)), dim3(kThreads), in,
                  out, uint32_t(rows), uint32_t(width), mp);
    return after_launch(ctx, name);
}

// src/ops/softmax.rs:91-108 plus the u32 width check of :130-131.
rl_status validate_softmax(const rl_buffer* input, uint64_t rows, uint64_t width, uint64_t es) {
    if (rl_status st = check_buffer(input, "input")) return st;
    if (rows == 0 || width == 0)
        return fail(RL_ERR_INVALID_SHAPE, "Softmax rows and width must be greater than zero");
    if (rows > UINT64_MAX / width || input->len != rows * width ||
        input->byte_len != input->len * es)
        return fail(RL_ERR_INVALID_SHAPE,
                    "Softmax input has %llu elements (%llu bytes), expected %llu elements of %llu "
                    "bytes",
                    (unsigned long long)input->len, (unsigned long long)input->byte_len,
                    (unsigned long long)(rows > UINT64_MAX / width ? 0 : rows * width),
                    (unsigned long long)es);
    if (width > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "Softmax width exceeds u32");
    if (rows > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "Softmax row count exceeds u32");
    return RL_OK;
}

// src/ops/attention_scale_mask.rs:120-161 plus the u32 checks of :349-352.
rl_status validate_mask(const rl_buffer* input, float scale, uint64_t query_len,
                        uint64_t key_len, uint64_t start, uint64_t es) {
    if (rl_status st = check_buffer(input, "input")) return st;
    if (query_len == 0 || key_len == 0)
        return fail(RL_ERR_INVALID_SHAPE, "attention query/key length cannot be zero");
    if (!(scale > 0.0f) || scale == INFINITY)
        return fail(RL_ERR_INVALID_SHAPE, "attention scale must be positive and finite, got %g",
                    double(scale));
    if (start > UINT64_MAX - query_len)
        return fail(RL_ERR_INVALID_SHAPE, "attention query position overflow");
    const uint64_t query_end = start + query_len;
    if (query_end > key_len)
        return fail(RL_ERR_INVALID_SHAPE,
                    "attention query range [%llu, %llu) exceeds key length %llu",
                    (unsigned long long)start, (unsigned long long)query_end,
                    (unsigned long long)key_len);
    const bool fits = query_len <= UINT64_MAX / key_len;
    if (!fits || input->len % (query_len * key_len) != 0 || input->byte_len != input->len * es)
        return fail(RL_ERR_INVALID_SHAPE,
                    "attention score buffer has %llu elements (%llu bytes), incompatible with "
                    "query_len=%llu, key_len=%llu and %llu byte elements",
                    (unsigned long long)input->len, (unsigned long long)input->byte_len,
                    (unsigned long long)query_len, (unsigned long long)key_len,
                    (unsigned long long)es);
    if (query_len > UINT32_MAX || key_len > UINT32_MAX || start > UINT32_MAX ||
        input->len > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "attention dimension exceeds u32");
    return RL_OK;
}

template <typename T>
rl_status softmax_entry(rl_context* ctx, const char* name, const rl_buffer* input, uint64_t rows,
                        uint64_t width, const rl_buffer* out) {
    if (rl_status st = validate_softmax(input, rows, width, sizeof(T))) return st;
    if (rl_status st = check_output(out, input->len, sizeof(T), "Softmax")) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_softmax<T, false>(ctx, name, static_cast<const T*>(input->data),
                                    static_cast<T*>(out->data), rows, width,
                                    MaskParams{1.0f, FastDiv(1), 0});
}

template <typename T>
rl_status scale_mask_entry(rl_context* ctx, const char* name, const rl_buffer* input,
                           float scale, uint64_t query_len, uint64_t key_len, uint64_t start,
                           const rl_buffer* out, bool fused) {
    if (rl_status st = validate_mask(input, scale, query_len, key_len, start, sizeof(T)))
        return st;
    if (rl_status st = check_output(out, input->len, sizeof(T), "attention")) return st;
    if (rl_status st = require_context(ctx)) return st;
    if (input->len == 0) return RL_OK;
    const uint64_t rows = input->len / key_len;
    const MaskParams mp{scale, FastDiv(uint32_t(query_len)), uint32_t(start)};
    const T* in = static_cast<const T*>(input->data);
    T* o = static_cast<T*>(out->data);
    if (fused) return launch_softmax<T, true>(ctx, name, in, o, rows, key_len, mp);
    return launch_scale_mask<T>(ctx, name, in, o, rows, key_len, mp);
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_softmax_f32(rl_context* ctx, const rl_buffer* input, uint64_t rows, uint64_t width,
                         const rl_buffer* out) {
    return softmax_entry<float>(ctx, "softmax_f32", input, rows, width, out);
}

rl_status rl_softmax_f16(rl_context* ctx, const rl_buffer* input, uint64_t rows, uint64_t width,
                         const rl_buffer* out) {
    return softmax_entry<half_t>(ctx, "softmax_f16", input, rows, width, out);
}

rl_status rl_attention_scale_mask_f32(rl_context* ctx, const rl_buffer* input, float scale,
                                      uint64_t query_len, uint64_t key_len,
                                      uint64_t query_start_pos, const rl_buffer* out) {
    return scale_mask_entry<float>(ctx, "attention_scale_mask_f32", input, scale, query_len,
                                   key_len, query_start_pos, out, false);
}

rl_status rl_attention_scale_mask_f16(rl_context* ctx, const rl_buffer* input, float scale,
                                      uint64_t query_len, uint64_t key_len,
                                      uint64_t query_start_pos, const rl_buffer* out) {
    return scale_mask_entry<half_t>(ctx, "attention_scale_mask_f16", input, scale, query_len,
                                    key_len, query_start_pos, out, false);
}

rl_status rl_attention_softmax_f32(rl_context* ctx, const rl_buffer* input, float scale,
                                   uint64_t query_len, uint64_t key_len,
                                   uint64_t query_start_pos, const rl_buffer* out) {
    return scale_mask_entry<float>(ctx, "attention_softmax_f32", input, scale, query_len,
                                   key_len, query_start_pos, out, true);
}

rl_status rl_attention_softmax_f16(rl_context* ctx, const rl_buffer* input, float scale,
                                   uint64_t query_len, uint64_t key_len,
                                   uint64_t query_start_pos, const rl_buffer* out) {
    return scale_mask_entry<half_t>(ctx, "attention_softmax_f16", input, scale, query_len,
                                    key_len, query_start_pos, out, true);
}

}  // extern "C"
