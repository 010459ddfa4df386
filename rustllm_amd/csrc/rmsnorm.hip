// rmsnorm.hip -- RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// y = x * rsqrt(sum(x^2) / h + eps) * w per row of h elements
// (kernels/rmsnorm.metal:7-126).  The reference gives each row a 256-thread
// group with an 8-barrier shared-memory tree and reads x twice.  Here a
// group of TPR lanes (16, 32 or 64: a quarter, half or whole wave64) owns
// one row: it loads the row once into VGPRs as 16-byte packs, NV packs per
// lane (all loads issued back to back), loads the weight packs (they stay
// L2-resident), reduces the sum of squares with DPP moves inside each row of
// 16 lanes and scalar lane reads across them (no LDS, no barrier) and writes
// y from registers, so x is read from HBM exactly once.  TPR is picked per
// row length so that every lane holds 3-12 packs with few idle lanes: 2-5
// packs per lane left the loads too short to cover HBM latency (f16 rows of
// 576-960 reached 50-63% of peak with a wave per row, 63-73% with 16-32
// lanes per row).  Rows longer than
// 64 x 16 packs fall back to a block per row with an LDS step across its
// four waves and a second (L2-resident) read.
//
// The fused variant first forms s = x + r rounded to the dtype (the add
// kernel's result), writes s and normalises it: the two adjacent calls of
// nn/transformer_block.rs:148-152 in one pass.
#include "common.hpp"

namespace rl {
namespace {

constexpr int kThreads = 256;
constexpr int kWave = 64;

// Pack p of a row, or the row's last pack for p past its end.
__device__ inline uint32_t clamp_pack(uint32_t p, uint32_t h_packs) {
    return p < h_packs ? p : h_packs - 1;
}
// Rows per launch chunk: keeps blocks x threads far below 2^32.
constexpr uint32_t kRowChunk = 1u << 22;

// Rows [row_base, row_base + rows) of the launch chunk; TPR lanes per row,
// kThreads / TPR rows per block.  Lanes of a group stride over the row's
// packs (pack p = lane + k * TPR), so each load instruction covers TPR
// consecutive packs of every row in the wave.
template <typename T, int N, int NV, int TPR, bool ADD, bool WLATE>
__global__ __launch_bounds__(kThreads) void k_rmsnorm_rows(
    const T* __restrict__ x, const T* __restrict__ residual, const T* __restrict__ weight,
    T* __restrict__ sum_out, T* __restrict__ y, uint32_t row_base, uint32_t rows,
    uint32_t h_packs, float hidden, float eps) {
    typedef typename VecOf<T, N>::type V;
    constexpr int kRowsPerBlock = kThreads / TPR;
    const uint32_t lane = threadIdx.x % TPR;
    const uint32_t row = row_base + blockIdx.x * kRowsPerBlock + threadIdx.x / TPR;
    if (row >= rows) return;  // the whole lane group leaves; no block barrier below
    const uint64_t row_off = uint64_t(row) * h_packs;
    const V* xr = reinterpret_cast<const V*>(x) + row_off;
    const V* wr = reinterpret_cast<const V*>(weight);
    V v[NV];
    V w[NV];
    // Every load is issued, at an index clamped into the row (packs past the
    // row are reloads of its last pack, never used): a load under a per-pack
    // branch made the compiler wait for each f16 load before issuing the next.
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = load_stream(xr + clamp_pack(lane + k * TPR, h_packs));
    if constexpr (ADD) {
        const V* rr = reinterpret_cast<const V*>(residual) + row_off;
        V* sr = reinterpret_cast<V*>(sum_out) + row_off;
        V r[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) r[k] = load_stream(rr + clamp_pack(lane + k * TPR, h_packs));
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const uint32_t p = lane + k * TPR;
            V s;
#pragma unroll
            for (int j = 0; j < N; ++j) s[j] = from_float<T>(to_float(v[k][j]) + to_float(r[k][j]));
            v[k] = s;
            if (p < h_packs) store_stream(sr + p, s);
        }
    }
    // The weight (h elements shared by every row) comes from L2.  With two
    // packs per lane its loads go out with the row's, so their latency hides
    // behind the reduction; with three or more (WLATE) every wave of a large
    // launch asking for the same few weight lines at its start slowed the
    // f16 [16384, h] launches by 10-20%, so they follow the reduction there.
    if constexpr (!WLATE) {
#pragma unroll
        for (int k = 0; k < NV; ++k) w[k] = wr[clamp_pack(lane + k * TPR, h_packs)];
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t p = lane + k * TPR;
        if (p < h_packs) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                float f = to_float(v[k][j]);
                ss = fmaf(f, f, ss);
            }
        }
    }
    if constexpr (WLATE) {
#pragma unroll
        for (int k = 0; k < NV; ++k) w[k] = wr[clamp_pack(lane + k * TPR, h_packs)];
    }
    ss = lane_group_sum_dpp<TPR>(ss);  // DPP within rows of 16, scalar reads across
    const float inverse_rms = rsqrtf(ss / hidden + eps);  // rmsnorm.metal:55-60
    V* yr = reinterpret_cast<V*>(y) + row_off;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t p = lane + k * TPR;
        if (p < h_packs) {
            V o;
#pragma unroll
            for (int j = 0; j < N; ++j)
                o[j] = from_float<T>(to_float(v[k][j]) * inverse_rms * to_float(w[k][j]));
            store_stream(yr + p, o);
        }
    }
}

// One 256-thread block per row, any h: pass 1 sums squares (and writes s for
// the fused add), pass 2 re-reads the row (from L2 for these sizes).
template <typename T, bool ADD>
__global__ __launch_bounds__(kThreads) void k_rmsnorm_block(
    const T* __restrict__ x, const T* __restrict__ residual, const T* __restrict__ weight,
    T* __restrict__ sum_out, T* __restrict__ y, uint32_t row_base, uint32_t h, float eps) {
    __shared__ float partial[kThreads / kWave];
    const uint32_t row = row_base + blockIdx.x;
    const uint64_t off = uint64_t(row) * h;
    const T* src = ADD ? sum_out : x;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < h; i += kThreads) {
        float f;
        if constexpr (ADD) {
            T s = from_float<T>(to_float(x[off + i]) + to_float(residual[off + i]));
            sum_out[off + i] = s;
            f = to_float(s);
        } else {
            f = to_float(x[off + i]);
        }
        ss = fmaf(f, f, ss);
    }
    ss = wave_sum(ss);
    if (threadIdx.x % kWave == 0) partial[threadIdx.x / kWave] = ss;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) total += partial[w];
    const float inverse_rms = rsqrtf(total / float(h) + eps);
    // Each thread re-reads only elements it wrote itself in pass 1.
    for (uint32_t i = threadIdx.x; i < h; i += kThreads)
        y[off + i] = from_float<T>(to_float(src[off + i]) * inverse_rms * to_float(weight[i]));
}

// Packs per lane instantiated for each lane-group width.
constexpr int kNv64[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16};
constexpr int kNv32[] = {3, 4, 5, 8, 10, 12};
constexpr int kNv16[] = {3, 4, 5, 8, 9, 12};

template <size_t K>
int smallest_at_least(const int (&set)[K], uint64_t need) {
    for (int v : set)
        if (uint64_t(v) >= need) return v;
    return 0;
}

struct RowPlan {
    int tpr;  // lanes per row
    int nv;   // packs per lane (instantiated, >= ceil(h_packs / tpr))
};

// Lane-group width for `rows` rows of h_packs packs (1 <= h_packs <= 1024):
// prefer 3..12 packs per lane, then the fewest idle lanes, then the wider
// group; then widen the group while the launch would have fewer than 4096
// waves (4 per SIMD), where more, shorter waves hide latency better
// ([4096, 960] f16: 4.4 us with 64 lanes per row, 4.9 us with 32).
RowPlan plan_by_length(uint64_t h_packs, bool narrow_ties);

RowPlan plan_rows(uint64_t h_packs, uint64_t rows, bool narrow_ties) {
    RowPlan plan = plan_by_length(h_packs, narrow_ties);
    while (plan.tpr < 64 && rows * uint64_t(plan.tpr) < 4096ull * kWave) {
        const int tpr = plan.tpr * 2;
        const uint64_t need = ceil_div(h_packs, uint64_t(tpr));
        const int nv = tpr == 64 ? smallest_at_least(kNv64, need) : smallest_at_least(kNv32, need);
        if (nv == 0) break;
        plan = {tpr, nv};
    }
    return plan;
}

// narrow_ties: between groups of equal lane use, take the narrower one (more
// packs per lane) when its instantiated pack count is exactly what the row
// needs: f16 [16384, 960] runs 8% faster on 16 lanes x 8 packs than on
// 32 x 4, while [16384, 768] (96 packs) on 16 x 8 -- two reloads of the last
// pack a lane -- takes 9.6 us against 8.9 on 32 x 3 (16 x 6: 9.0-9.3).  f32
// rows keep the wider group on a tie.
RowPlan plan_by_length(uint64_t h_packs, bool narrow_ties) {
    RowPlan best{0, 0};
    bool best_ok = false;
    uint64_t best_num = 0, best_den = 1;  // lane use = num / den
    for (int tpr : {64, 32, 16}) {
        const uint64_t need = ceil_div(h_packs, uint64_t(tpr));
        const int nv = tpr == 64   ? smallest_at_least(kNv64, need)
                       : tpr == 32 ? smallest_at_least(kNv32, need)
                                   : smallest_at_least(kNv16, need);
        if (nv == 0) continue;
        const bool ok = need >= 3 && need <= 12;
        const uint64_t num = h_packs, den = uint64_t(tpr) * need;
        const bool better_use = num * best_den > best_num * den ||
                                (narrow_ties && num * best_den == best_num * den &&
                                 uint64_t(nv) == need);
        if (best.tpr == 0 || (ok && !best_ok) || (ok == best_ok && better_use)) {
            best = {tpr, nv};
            best_ok = ok;
            best_num = num;
            best_den = den;
        }
    }
    return best;
}

template <typename T, int N, int NV, int TPR, bool ADD>
void launch_rows(rl_context* ctx, const T* x, const T* residual, const T* weight, T* sum_out,
                 T* y, uint32_t rows, uint32_t h_packs, float hidden, float eps) {
    constexpr uint32_t kRowsPerBlock = kThreads / TPR;
    static_assert(kRowChunk % kRowsPerBlock == 0, "chunks must hold whole blocks");
    for (uint32_t base = 0; base < rows; base += kRowChunk) {
        const uint32_t n = rows - base < kRowChunk ? rows - base : kRowChunk;
        const dim3 grid(unsigned(ceil_div(n, kRowsPerBlock))), block(kThreads);
        RL_LAUNCH(ctx, (k_rmsnorm_rows<T, N, NV, TPR, ADD, (NV >= 3)>), grid, block, x,
                  residual, weight, sum_out, y, base, rows, h_packs, hidden, eps);
        if (rows - base <= kRowChunk) break;
    }
}

template <typename T, bool ADD>
rl_status launch_rmsnorm(rl_context* ctx, const char* name, const T* x, const T* residual,
                         const T* weight, T* sum_out, T* y, uint64_t rows, uint64_t hidden,
                         float eps) {
    if (rl_status st = activate(ctx)) return st;
    constexpr int N = 16 / sizeof(T);
    const bool packs_ok = hidden % N == 0 && aligned_to(x, 16) && aligned_to(weight, 16) &&
                          aligned_to(y, 16) && (!ADD || (aligned_to(residual, 16) &&
                                                         aligned_to(sum_out, 16)));
    const uint64_t h_packs = hidden / N;
    const uint32_t r32 = uint32_t(rows);
    if (packs_ok && h_packs <= 16 * kWave) {
        const RowPlan plan = plan_rows(h_packs, rows, sizeof(T) == 2);
        const uint32_t hp = uint32_t(h_packs);
        const float hf = float(hidden);
#define RL_RMS_PLAN(TPR_, NV_)                                                                \
    if (plan.tpr == TPR_ && plan.nv == NV_) {                                                 \
        launch_rows<T, N, NV_, TPR_, ADD>(ctx, x, residual, weight, sum_out, y, r32, hp, hf,  \
                                          eps);                                               \
        return after_launch(ctx, name);                                                       \
    }
        RL_RMS_PLAN(64, 1) RL_RMS_PLAN(64, 2)
        RL_RMS_PLAN(64, 3) RL_RMS_PLAN(64, 4) RL_RMS_PLAN(64, 5) RL_RMS_PLAN(64, 6)
        RL_RMS_PLAN(64, 8) RL_RMS_PLAN(64, 10) RL_RMS_PLAN(64, 12) RL_RMS_PLAN(64, 16)
        RL_RMS_PLAN(32, 3) RL_RMS_PLAN(32, 4) RL_RMS_PLAN(32, 5) RL_RMS_PLAN(32, 8)
        RL_RMS_PLAN(32, 10) RL_RMS_PLAN(32, 12)
        RL_RMS_PLAN(16, 3) RL_RMS_PLAN(16, 4) RL_RMS_PLAN(16, 5) RL_RMS_PLAN(16, 8)
        RL_RMS_PLAN(16, 9) RL_RMS_PLAN(16, 12)
#undef RL_RMS_PLAN
        return fail(RL_ERR_DEVICE, "RMSNorm: no kernel for %d lanes x %d packs per row",
                    plan.tpr, plan.nv);
    }
    for (uint32_t base = 0; base < r32; base += kRowChunk) {
        const uint32_t n = r32 - base < kRowChunk ? r32 - base : kRowChunk;
        RL_LAUNCH(ctx, (k_rmsnorm_block<T, ADD>), dim3(n), dim3(kThreads), x, residual, weight,
                  sum_out, y, base, uint32_t(hidden), eps);
        if (r32 - base <= kRowChunk) break;
    }
    return after_launch(ctx, name);
}

// src/ops/rmsnorm.rs:38-116 / :142-206 in order, plus the byte lengths and
// the row-count limit of the grid.  Any eps is accepted here, as by the
// reference's buffer-level rmsnorm_f32/_f16; the Tensor-level ops::rmsnorm
// (:226-230) checks that it is finite and positive.
rl_status validate(const rl_buffer* input, const rl_buffer* weight, uint64_t rows,
                   uint64_t hidden, float eps, uint64_t es) {
    if (rl_status st = check_buffer(input, "input")) return st;
    if (rl_status st = check_buffer(weight, "weight")) return st;
    if (hidden == 0)
        return fail(RL_ERR_INVALID_SHAPE, "RMSNorm hidden size cannot be zero");
    if (rows > UINT64_MAX / hidden || input->len != rows * hidden)
        return fail(RL_ERR_INVALID_SHAPE, "RMSNorm input has %llu elements, expected %llu",
                    (unsigned long long)input->len,
                    (unsigned long long)(rows > UINT64_MAX / hidden ? 0 : rows * hidden));
    if (weight->len != hidden)
        return fail(RL_ERR_INVALID_SHAPE, "RMSNorm weight has %llu elements, expected %llu",
                    (unsigned long long)weight->len, (unsigned long long)hidden);
    if (input->byte_len < input->len * es || weight->byte_len < weight->len * es)
        return fail(RL_ERR_INVALID_SHAPE, "RMSNorm buffers do not hold %llu-byte elements",
                    (unsigned long long)es);
    if (hidden > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "RMSNorm hidden size exceeds u32");
    if (rows > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "RMSNorm row count exceeds u32");
    return RL_OK;
}

template <typename T>
rl_status rmsnorm_entry(rl_context* ctx, const char* name, const rl_buffer* input,
                        const rl_buffer* weight, uint64_t rows, uint64_t hidden, float eps,
                        const rl_buffer* out) {
    if (rl_status st = validate(input, weight, rows, hidden, eps, sizeof(T))) return st;
    if (rl_status st = check_output(out, input->len, sizeof(T), "RMSNorm")) return st;
    if (rl_status st = require_context(ctx)) return st;
    if (rows == 0) return RL_OK;
    return launch_rmsnorm<T, false>(ctx, name, static_cast<const T*>(input->data), nullptr,
                                    static_cast<const T*>(weight->data), nullptr,
                                    static_cast<T*>(out->data), rows, hidden, eps);
}

template <typename T>
rl_status add_rmsnorm_entry(rl_context* ctx, const char* name, const rl_buffer* x,
                            const rl_buffer* residual, const rl_buffer* weight, uint64_t rows,
                            uint64_t hidden, float eps, const rl_buffer* sum_out,
                            const rl_buffer* norm_out) {
    if (rl_status st = check_buffer(residual, "residual")) return st;
    if (rl_status st = check_buffer(x, "input")) return st;
    if (x->len != residual->len) {  // Tensor::add's check (elementwise.rs:119-124) on lengths
        const uint64_t left[1] = {x->len}, right[1] = {residual->len};
        return fail_shape_mismatch(left, 1, right, 1);
    }
    if (residual->byte_len < residual->len * sizeof(T))
        return fail(RL_ERR_INVALID_SHAPE, "residual buffer does not hold %zu-byte elements",
                    sizeof(T));
    if (rl_status st = validate(x, weight, rows, hidden, eps, sizeof(T))) return st;
    if (rl_status st = check_output(sum_out, x->len, sizeof(T), "add")) return st;
    if (rl_status st = check_output(norm_out, x->len, sizeof(T), "RMSNorm")) return st;
    if (rl_status st = require_context(ctx)) return st;
    if (rows == 0) return RL_OK;
    return launch_rmsnorm<T, true>(ctx, name, static_cast<const T*>(x->data),
                                   static_cast<const T*>(residual->data),
                                   static_cast<const T*>(weight->data),
                                   static_cast<T*>(sum_out->data), static_cast<T*>(norm_out->data),
                                   rows, hidden, eps);
}

}  // namespace
}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_rmsnorm_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* weight,
                         uint64_t rows, uint64_t hidden, float eps, const rl_buffer* out) {
    return rmsnorm_entry<float>(ctx, "rmsnorm_f32", input, weight, rows, hidden, eps, out);
}

rl_status rl_rmsnorm_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* weight,
                         uint64_t rows, uint64_t hidden, float eps, const rl_buffer* out) {
    return rmsnorm_entry<half_t>(ctx, "rmsnorm_f16", input, weight, rows, hidden, eps, out);
}

rl_status rl_add_rmsnorm_f32(rl_context* ctx, const rl_buffer* x, const rl_buffer* residual,
                             const rl_buffer* weight, uint64_t rows, uint64_t hidden, float eps,
                             const rl_buffer* sum_out, const rl_buffer* norm_out) {
    return add_rmsnorm_entry<float>(ctx, "add_rmsnorm_f32", x, residual, weight, rows, hidden,
                                    eps, sum_out, norm_out);
}

rl_status rl_add_rmsnorm_f16(rl_context* ctx, const rl_buffer* x, const rl_buffer* residual,
                             const rl_buffer* weight, uint64_t rows, uint64_t hidden, float eps,
                             const rl_buffer* sum_out, const rl_buffer* norm_out) {
    return add_rmsnorm_entry<half_t>(ctx, "add_rmsnorm_f16", x, residual, weight, rows, hidden,
                                     eps, sum_out, norm_out);
}

}  // extern "C"
