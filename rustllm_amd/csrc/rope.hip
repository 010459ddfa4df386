// rope.hip -- rotary position embedding for gfx950.
//
// For row r of [..., S, D] at position p = (r mod S) + start and pair
// i < D/2: (a, b) = (x[i], x[i + D/2]) -> (a*c - b*s, b*c + a*s) with
// c, s = table[p, i] (kernels/rope.metal:23-63, 82-96).  Each thread rotates
// a pack of N pairs: one 16-byte-or-smaller load from each half of the row
// plus N cos and N sin values.  The f32 tables are [table_rows, D/2] (1 MiB
// for 4096 x 32 x 2) and stay in L2, so HBM traffic is the input and output
// rows only.  Contraction into FMA is off: each product and difference is
// rounded once, as in the reference expression.
//
// The input may be a strided view whose innermost stride is 1 (the
// [1, H, S, D] permute of [1, S, H, D] the attention path rotates): the
// gather that ops::rope_encode does first with contiguous_encode
// (src/ops/rope.rs:345) happens in the same pass, rows being decoded with
// 32-bit multiply-high division.  Rows are taken in the view's memory order:
// for that permute the heads of one position come together, so the
// projection is read straight through and the position's cos/sin row is
// fetched once per wave instead of once per head.
#include "common.hpp"

#pragma clang fp contract(off)

namespace rl {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxRank = kMaxRowRank;

// Output row of input row (g, p) -- g the index over all dims outside the
// sequence dim, p the position -- is g * group_rows + first_row + p: the
// contiguous [..., S, D] result for group_rows = S, first_row = 0, or the
// rows of a [1, H, max_seq, D] KV cache from `start` on for
// group_rows = max_seq, first_row = start.
struct DstRows {
    uint32_t group_rows;
    uint32_t first_row;
};

template <typename T, int N, int UNROLL>
__global__ __launch_bounds__(kThreads) void k_rope(const T* __restrict__ src,
                                                   const float* __restrict__ cos_table,
                                                   const float* __restrict__ sin_table,
                                                   T* __restrict__ out, uint32_t n_items,
                                                   FastDiv packs_per_row, RowDims rd,
                                                   uint32_t half_dim, uint32_t start,
                                                   DstRows dst) {
    typedef typename VecOf<T, N>::type V;
    typedef typename VecOf<float, N>::type VF;
    const uint64_t tile = uint64_t(kThreads) * UNROLL;
    const uint64_t step = uint64_t(gridDim.x) * tile;
    for (uint64_t base = uint64_t(blockIdx.x) * tile + threadIdx.x; base < n_items;
         base += step) {
        V a[UNROLL], b[UNROLL];
        VF c[UNROLL], s[UNROLL];
        uint64_t dst_off[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_items) {
                uint32_t row, pp;
                packs_per_row.divmod(uint32_t(i), row, pp);
                // Rows run in the view's memory order (make_row_dims).
                uint64_t src_off;
                uint32_t position, group;
                decode_row(rd, row, src_off, position, group);
                const uint32_t pair = pp * N;
                const uint64_t t = uint64_t(start + position) * half_dim + pair;
                a[u] = *reinterpret_cast<const V*>(src + src_off + pair);
                b[u] = *reinterpret_cast<const V*>(src + src_off + half_dim + pair);
                c[u] = *reinterpret_cast<const VF*>(cos_table + t);
                s[u] = *reinterpret_cast<const VF*>(sin_table + t);
                const uint64_t dst_row =
                    uint64_t(group) * dst.group_rows + dst.first_row + position;
                dst_off[u] = dst_row * (2 * half_dim) + pair;
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t i = base + uint64_t(u) * kThreads;
            if (i < n_items) {
                V o1, o2;
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    const float first = to_float(a[u][j]);
                    const float second = to_float(b[u][j]);
                    o1[j] = from_float<T>(first * c[u][j] - second * s[u][j]);
                    o2[j] = from_float<T>(second * c[u][j] + first * s[u][j]);
                }
                store_stream(reinterpret_cast<V*>(out + dst_off[u]), o1);
                store_stream(reinterpret_cast<V*>(out + dst_off[u] + half_dim), o2);
            }
        }
    }
}

// ---------------------------------------------- row blocks of 16-byte lanes
//
// The layout for rows of 32, 64, 128 or 256 bytes (head_dim 16..128 in f16,
// 8..64 in f32): L = row bytes / 16 lanes per row, each loading one 16-byte
// pack, so a lane group reads and writes its whole row in one access.  The
// rotation partner of a pack -- the pack half_dim elements away -- sits in
// another lane of the group and comes over with one DPP move per dword:
// quad_perm for L = 2 and 4, row_ror:8 for L = 16, and row_half_mirror for
// L = 8, where lane j >= 4 holds pack 11 - j so that the partners of lanes j
// and 7 - j are each other.  A block serves kThreads / L consecutive rows in
// the view's memory order (make_row_dims), so it reads one contiguous
// stretch of the source, and the heads of one position, coming together in
// a [1, S, H, D] projection, share their cos/sin row.

constexpr int kMaxJobRank = 6;  // row dims of a job's view

// One view rotated (or copied) into `dst` rows
// group * dst_rows.group_rows + dst_rows.first_row + position and, when `rep`
// is set, into rows (group * n_rep + r) * rep_rows + rep_first + position of
// `rep` for r < n_rep.  A null `dst` skips the first write.
struct RowJob {
    const void* src;
    void* dst;
    void* rep;
    RowDimsN<kMaxJobRank> rows;
    DstRows dst_rows;
    uint32_t n_rows;
    uint32_t n_rep;
    uint32_t rep_rows;
    uint32_t rep_first;
    uint32_t first_block;  // blocks [first_block, next job's first_block)
    uint32_t rotate;
};

constexpr int kMaxJobs = 5;
struct RowJobs {
    RowJob job[kMaxJobs];
};

template <int L>
__device__ inline int partner_dword(int v) {
    if constexpr (L == 2)
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
    else if constexpr (L == 4)
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
    else if constexpr (L == 8)
        return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    else
        return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);  // row_ror:8
}

// decode_row over the first R row dims with no branch, so the scalar loads
// of every dim go out together (the views of a launch have at most R row
// dims; R = kMaxJobRank decodes any job).  Dims past rd.rank are
// make_row_dims' zero initialisation -- divisor 1, stride 0, group
// multiplier 0 -- and leave the row, the offset and the group as they are.
template <int R>
__device__ inline void decode_job_row_r(const RowDimsN<kMaxJobRank>& rd, uint32_t row,
                                        uint64_t& src_off, uint32_t& position, uint32_t& group) {
    src_off = 0;
    position = 0;
    group = 0;
#pragma unroll
    for (uint32_t d = 0; d < uint32_t(R); ++d) {
        uint32_t q, r;
        rd.dim[d].divmod(row, q, r);
        src_off += uint64_t(r) * rd.stride[d];
        position = d == rd.seq_dim ? r : position;
        group += r * rd.group_mult[d];
        row = q;
    }
}

// U rows per lane group: the group takes rows first + u * kRows (u < U) of
// its block's kRows * U and issues every row's loads before any arithmetic,
// so a wave has U rows' loads in flight.  A lane and its rotation partner
// need the same cos and sin values: the first-half lane loads cos, the
// second-half lane sin, and each takes the other's over the same DPP move
// as the data (half the table loads, which on the [1, 25, 4096, 64]
// prologue outnumbered the data loads four to one).  A block belongs to one
// job, so a copy job branches around the rotation without divergence.
// R: row dims decoded (3 when every job of the launch has at most 3).
template <typename T, int L, int U, int R>
__global__ __launch_bounds__(kThreads) void k_rope_blocks(RowJobs jobs,
                                                          const float* __restrict__ cos_table,
                                                          const float* __restrict__ sin_table,
                                                          uint32_t start) {
    constexpr int N = 16 / int(sizeof(T));  // elements per lane
    constexpr uint32_t D = uint32_t(L * N);
    constexpr uint32_t kHalf = D / 2;
    constexpr uint32_t kRows = kThreads / L;  // rows per block and row slot
    typedef typename VecOf<T, N>::type V;
    typedef typename VecOf<float, N>::type VF;
    uint32_t k = 0;
#pragma unroll
    for (int t = 1; t < kMaxJobs; ++t) k += blockIdx.x >= jobs.job[t].first_block ? 1u : 0u;
    const RowJob& job = jobs.job[k];
    const bool rotate = job.rotate != 0;
    const uint32_t first = (blockIdx.x - job.first_block) * kRows * U + threadIdx.x / L;
    const uint32_t lane = threadIdx.x % L;
    const uint32_t pack = (L == 8 && lane >= 4) ? 11 - lane : lane;
    const uint32_t pair = (pack % (L / 2)) * N;
    const bool first_half = pack < uint32_t(L / 2);
    const float* own_table = first_half ? cos_table : sin_table;
    V x[U];
    VF tab[U];  // cos (first half) or sin (second half)
    uint32_t pos[U], group[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        uint32_t row = first + uint32_t(u) * kRows;
        live[u] = row < job.n_rows;
        if (!live[u]) row = job.n_rows - 1;  // a valid row: every lane takes part in the DPP moves
        uint64_t src_off;
        decode_job_row_r<R>(job.rows, row, src_off, pos[u], group[u]);
        // The loads go out back to back.  A copy job reads table row 0
        // (valid for every job here) and ignores it, which keeps them
        // branch-free.
        const uint64_t t = rotate ? uint64_t(start + pos[u]) * kHalf + pair : pair;
        tab[u] = *reinterpret_cast<const VF*>(own_table + t);
        x[u] = load_stream(reinterpret_cast<const V*>(static_cast<const T*>(job.src) + src_off +
                                                      pack * N));
    }
    __builtin_amdgcn_sched_barrier(0);  // every load ahead of the first wait
#pragma unroll
    for (int u = 0; u < U; ++u) {
        V o;
        if (!rotate) {
            o = x[u];
        } else {
            int tv[N], pv[N], w[4], m[4];
            __builtin_memcpy(tv, &tab[u], sizeof(VF));
#pragma unroll
            for (int i = 0; i < N; ++i) pv[i] = partner_dword<L>(tv[i]);
            __builtin_memcpy(w, &x[u], 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) m[i] = partner_dword<L>(w[i]);
            VF ptab;
            V other;
            __builtin_memcpy(&ptab, pv, sizeof(VF));
            __builtin_memcpy(&other, m, 16);
            const VF c = first_half ? tab[u] : ptab;
            const VF s = first_half ? ptab : tab[u];
            // First half: first*c - second*s; second half: second*c + first*s.
            // Negating the partner is exact, so each result keeps the
            // reference's two rounded products and one rounded sum.
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const float own = to_float(x[u][j]);
                const float partner = first_half ? -to_float(other[j]) : to_float(other[j]);
                o[j] = from_float<T>(own * c[j] + partner * s[j]);
            }
        }
        if (!live[u]) continue;
        if (job.dst) {
            const uint64_t r =
                uint64_t(group[u]) * job.dst_rows.group_rows + job.dst_rows.first_row + pos[u];
            store_stream(reinterpret_cast<V*>(static_cast<T*>(job.dst) + r * D + pack * N), o);
        }
        if (job.rep) {
            for (uint32_t i = 0; i < job.n_rep; ++i) {
                const uint64_t r =
                    (uint64_t(group[u]) * job.n_rep + i) * job.rep_rows + job.rep_first + pos[u];
                store_stream(reinterpret_cast<V*>(static_cast<T*>(job.rep) + r * D + pack * N),
                             o);
            }
        }
    }
}

// Lanes per row for the row-block kernel, or 0 when the row is not 32, 64,
// 128 or 256 bytes.
template <typename T>
int row_lanes(uint64_t head_dim) {
    switch (head_dim * sizeof(T)) {
        case 32: return 2;
        case 64: return 4;
        case 128: return 8;
        case 256: return 16;
        default: return 0;
    }
}

// A job for a [..., S, D] view, or false when the view does not fit the
// row-block kernel (more row dims than it decodes, a row start off a 16-byte
// boundary, or more than u32 rows).
template <typename T>
bool make_job(RowJob& job, const void* src, const uint64_t* dims, const uint64_t* strides,
              uint32_t rank, void* dst, DstRows dst_rows, bool rotate) {
    constexpr uint64_t N = 16 / sizeof(T);
    if (rank < 2 || rank - 1 > uint32_t(kMaxJobRank) || strides[rank - 1] != 1) return false;
    if (!aligned_to(src, 16) || (dst && !aligned_to(dst, 16))) return false;
    uint64_t rows = 1;
    for (uint32_t d = 0; d + 1 < rank; ++d) {
        if (strides[d] % N != 0 || dims[d] > UINT32_MAX) return false;
        rows *= dims[d];
        if (rows > UINT32_MAX) return false;
    }
    job = RowJob{};
    job.src = src;
    job.dst = dst;
    job.rows = make_row_dims<kMaxJobRank>(dims, strides, rank);
    job.dst_rows = dst_rows;
    job.n_rows = uint32_t(rows);
    job.rotate = rotate ? 1u : 0u;
    return true;
}

// Rows per lane group of a launch of `total_rows` rows of `lanes` lanes
// each: 2 when one row per group would need more waves than the chip holds
// at once (8 per SIMD), so that every wave is resident from the start with
// two rows' loads in flight; else 1.
inline int rows_per_group(const rl_context* ctx, uint64_t total_rows, int lanes) {
    const uint64_t waves = ceil_div(total_rows * uint64_t(lanes), 64);
    return waves > uint64_t(8) * 4 * uint64_t(ctx->num_cus) ? 2 : 1;
}

template <typename T, int L, int R>
void launch_rows_r(rl_context* ctx, int unroll, dim3 grid, const RowJobs& jobs,
                   const float* cos_table, const float* sin_table, uint32_t start) {
    if (unroll == 2)
        RL_LAUNCH(ctx, (k_rope_blocks<T, L, 2, R>), grid, dim3(kThreads), jobs, cos_table,
                  sin_table, start);
    else
        RL_LAUNCH(ctx, (k_rope_blocks<T, L, 1, R>), grid, dim3(kThreads), jobs, cos_table,
                  sin_table, start);
}

template <typename T, int L>
void launch_rows(rl_context* ctx, int unroll, bool rank3, dim3 grid, const RowJobs& jobs,
                 const float* cos_table, const float* sin_table, uint32_t start) {
    if (rank3)
        launch_rows_r<T, L, 3>(ctx, unroll, grid, jobs, cos_table, sin_table, start);
    else
        launch_rows_r<T, L, kMaxJobRank>(ctx, unroll, grid, jobs, cos_table, sin_table, start);
}

// Assigns first blocks to jobs[0 .. n) (jobs with no rows get none) and
// launches; false when the grid would be too large.
template <typename T>
bool launch_jobs(rl_context* ctx, RowJobs& jobs, int n, int lanes, const float* cos_table,
                 const float* sin_table, uint64_t start) {
    uint64_t total_rows = 0;
    bool rank3 = true;  // every job's view has at most 3 row dims
    for (int t = 0; t < n; ++t) {
        total_rows += jobs.job[t].n_rows;
        rank3 = rank3 && jobs.job[t].rows.rank <= 3;
    }
    const int unroll = rows_per_group(ctx, total_rows, lanes);
    const uint64_t rows_per_block = uint64_t(kThreads) / lanes * unroll;
    uint64_t blocks = 0;
    for (int t = 0; t < kMaxJobs; ++t) {
        RowJob& job = jobs.job[t];
        if (t >= n) {
            job.first_block = UINT32_MAX;
            continue;
        }
        job.first_block = uint32_t(blocks);
        blocks += ceil_div(uint64_t(job.n_rows), rows_per_block);
        if (blocks >= (1u << 30)) return false;
    }
    if (blocks == 0) return true;
    const dim3 grid(static_cast<unsigned>(blocks));
    const uint32_t s32 = uint32_t(start);
    switch (lanes) {
        case 2: launch_rows<T, 2>(ctx, unroll, rank3, grid, jobs, cos_table, sin_table, s32); break;
        case 4: launch_rows<T, 4>(ctx, unroll, rank3, grid, jobs, cos_table, sin_table, s32); break;
        case 8: launch_rows<T, 8>(ctx, unroll, rank3, grid, jobs, cos_table, sin_table, s32); break;
        default: launch_rows<T, 16>(ctx, unroll, rank3, grid, jobs, cos_table, sin_table, s32); break;
    }
    return true;
}

inline unsigned grid_for(uint64_t items, uint64_t per_block) {
    uint64_t blocks = ceil_div(items, per_block);
    if (blocks < 1) blocks = 1;
    if (blocks > (1u << 30)) blocks = 1u << 30;
    return unsigned(blocks);
}

// dims/strides: the view, outermost first, rank >= 2, strides[rank-1] == 1.
// dst.group_rows == 0 means the contiguous [dims] output.
template <typename T>
rl_status launch_rope(rl_context* ctx, const char* name, const T* src, const uint64_t* dims,
                      const uint64_t* strides, uint32_t rank, const float* cos_table,
                      const float* sin_table, uint64_t start, T* out,
                      DstRows dst = DstRows{0, 0}) {
    if (rl_status st = activate(ctx)) return st;
    const uint64_t head_dim = dims[rank - 1];
    const uint64_t half = head_dim / 2;
    if (dst.group_rows == 0) dst = DstRows{uint32_t(dims[rank - 2]), 0};
    if (const int lanes = row_lanes<T>(head_dim);
        lanes && aligned_to(cos_table, 64 / sizeof(T)) && aligned_to(sin_table, 64 / sizeof(T))) {
        RowJobs jobs{};
        if (make_job<T>(jobs.job[0], src, dims, strides, rank, out, dst, true) &&
            launch_jobs<T>(ctx, jobs, 1, lanes, cos_table, sin_table, start))
            return after_launch(ctx, name);
    }
    uint64_t rows = 1;
    for (uint32_t d = 0; d + 1 < rank; ++d) rows *= dims[d];
    // Widest pack of pairs (<= 16 B of T, <= 4 or 8 lanes) that keeps every
    // access aligned.
    int n = 16 / int(sizeof(T));
    while (n > 1) {
        bool ok = half % n == 0 && aligned_to(src, n * sizeof(T)) &&
                  aligned_to(out, n * sizeof(T)) && aligned_to(cos_table, n * 4) &&
                  aligned_to(sin_table, n * 4);
        for (uint32_t d = 0; d + 1 < rank && ok; ++d) ok = strides[d] % n == 0;
        if (ok) break;
        n >>= 1;
    }
    const RowDims rd = make_row_dims(dims, strides, rank);
    const uint64_t n_items = rows * (half / n);
    const FastDiv ppr(uint32_t(half / n));
    constexpr int U = 1;
    const dim3 grid(grid_for(n_items, uint64_t(kThreads) * U)), block(kThreads);
    const uint32_t h32 = uint32_t(half), s32 = uint32_t(start), ni = uint32_t(n_items);
    switch (n) {
        case 8:
            RL_LAUNCH(ctx, (k_rope<T, 8, U>), grid, block, src, cos_table, sin_table, out, ni, ppr, rd, h32, s32, dst);
            break;
        case 4:
            RL_LAUNCH(ctx, (k_rope<T, 4, U>), grid, block, src, cos_table, sin_table, out, ni, ppr, rd, h32, s32, dst);
            break;
        case 2:
            RL_LAUNCH(ctx, (k_rope<T, 2, U>), grid, block, src, cos_table, sin_table, out, ni, ppr, rd, h32, s32, dst);
            break;
        default:
            RL_LAUNCH(ctx, (k_rope<T, 1, U>), grid, block, src, cos_table, sin_table, out, ni, ppr, rd, h32, s32, dst);
            break;
    }
    return after_launch(ctx, name);
}

rl_status check_tables(const rl_buffer* cos_table, const rl_buffer* sin_table,
                       uint64_t table_rows, uint64_t half, uint64_t start, uint64_t seq_len) {
    if (rl_status st = check_buffer(cos_table, "cos table")) return st;
    if (rl_status st = check_buffer(sin_table, "sin table")) return st;
    // ops::rope_encode (src/ops/rope.rs:329-343): equal [rows, D/2] f32 tables
    // covering positions start .. start + seq_len.
    if (cos_table->byte_len != cos_table->len * 4 || sin_table->byte_len != sin_table->len * 4)
        return fail(RL_ERR_UNSUPPORTED_DTYPE, "RoPE requires F32 cos/sin tables");
    if (table_rows > UINT64_MAX / half || cos_table->len != table_rows * half ||
        sin_table->len != cos_table->len)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE cos/sin tables must have equal rank-2 shapes");
    if (start > UINT64_MAX - seq_len || start + seq_len > table_rows)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE cos/sin table shape or position range is invalid");
    return RL_OK;
}

// src/ops/rope.rs:38-151 / :177-277 in order, plus the table bounds above.
template <typename T>
rl_status rope_entry(rl_context* ctx, const char* name, const rl_buffer* input,
                     const rl_buffer* cos_table, const rl_buffer* sin_table, uint64_t seq_len,
                     uint64_t head_dim, uint64_t start, const rl_buffer* out) {
    if (rl_status st = check_buffer(input, "input")) return st;
    if (head_dim == 0 || head_dim % 2 != 0)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE head dimension must be positive and even, got %llu",
                    (unsigned long long)head_dim);
    if (seq_len == 0) return fail(RL_ERR_INVALID_SHAPE, "RoPE sequence length cannot be zero");
    if (input->len % head_dim != 0)
        return fail(RL_ERR_INVALID_SHAPE,
                    "RoPE input length %llu is not divisible by head dimension %llu",
                    (unsigned long long)input->len, (unsigned long long)head_dim);
    const uint64_t half = head_dim / 2;
    const uint64_t rows = input->len / head_dim;
    if (rows % seq_len != 0)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE input rows are incompatible with sequence length");
    if (input->byte_len < input->len * sizeof(T))
        return fail(RL_ERR_INVALID_SHAPE, "RoPE input does not hold %zu-byte elements", sizeof(T));
    if (rl_status st = check_output(out, input->len, sizeof(T), "RoPE")) return st;
    if (seq_len > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE sequence length exceeds u32");
    if (head_dim > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "RoPE head dimension exceeds u32");
    if (start > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "RoPE start position exceeds u32");
    if (rows * half > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "RoPE work size exceeds u32");
    const uint64_t table_rows = cos_table ? (cos_table->len / half) : 0;
    if (rl_status st = check_tables(cos_table, sin_table, table_rows, half, start, seq_len))
        return st;
    if (rl_status st = require_context(ctx)) return st;
    if (input->len == 0) return RL_OK;
    const uint64_t dims[3] = {rows / seq_len, seq_len, head_dim};
    const uint64_t strides[3] = {seq_len * head_dim, head_dim, 1};
    return launch_rope<T>(ctx, name, static_cast<const T*>(input->data), dims, strides, 3,
                          static_cast<const float*>(cos_table->data),
                          static_cast<const float*>(sin_table->data), start,
                          static_cast<T*>(out->data));
}

// ops::rope_encode on a view (src/ops/rope.rs:303-370): the Tensor-level
// checks (rank >= 2, even head_dim, tables) and the view's own bounds.
template <typename T>
rl_status rope_strided_entry(rl_context* ctx, const char* name, const rl_buffer* src,
                             const uint64_t* dims, const uint64_t* strides, uint32_t rank,
                             const rl_buffer* cos_table, const rl_buffer* sin_table,
                             uint64_t table_rows, uint64_t start, const rl_buffer* out) {
    if (rl_status st = check_buffer(src, "input")) return st;
    if (dims == nullptr || strides == nullptr)
        return fail(RL_ERR_INVALID_ARGUMENT, "dims or strides is null");
    if (rank < 2)
        return fail(RL_ERR_INVALID_DIMENSION,
                    "RoPE expects [..., sequence, head_dim], got rank %u", rank);
    if (rank > kMaxRank + 1) return fail(RL_ERR_INVALID_SHAPE, "tensor rank exceeds %d", kMaxRank + 1);
    const uint64_t seq_len = dims[rank - 2], head_dim = dims[rank - 1];
    if (head_dim == 0 || head_dim % 2 != 0)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE head dimension must be positive and even, got %llu",
                    (unsigned long long)head_dim);
    const uint64_t half = head_dim / 2;
    uint64_t numel = 1;
    for (uint32_t d = 0; d < rank; ++d) {
        if (dims[d] == 0)
            return fail(RL_ERR_INVALID_SHAPE, "shape dimensions must be greater than zero");
        if (numel > UINT64_MAX / dims[d])
            return fail(RL_ERR_INVALID_SHAPE, "RoPE work size exceeds u32");
        numel *= dims[d];
    }
    if (rl_status st = check_tables(cos_table, sin_table, table_rows, half, start, seq_len))
        return st;
    if (strides[rank - 1] != 1)
        return fail(RL_ERR_NON_CONTIGUOUS, "RoPE view must have a unit innermost stride");
    if (src->byte_len < src->len * sizeof(T))
        return fail(RL_ERR_INVALID_SHAPE, "RoPE input does not hold %zu-byte elements", sizeof(T));
    for (uint32_t d = 0; d < rank; ++d)
        if (dims[d] > UINT32_MAX || strides[d] > UINT32_MAX)
            return fail(RL_ERR_INVALID_SHAPE, "shape dimension exceeds u32");
    if (numel / 2 > UINT32_MAX || start > UINT32_MAX)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE work size exceeds u32");
    unsigned __int128 last = 0;
    for (uint32_t d = 0; d < rank; ++d) last += (unsigned __int128)(dims[d] - 1) * strides[d];
    if (last >= src->len)
        return fail(RL_ERR_INVALID_SHAPE, "view reaches past the end of its %llu-element buffer",
                    (unsigned long long)src->len);
    if (rl_status st = check_output(out, numel, sizeof(T), "RoPE")) return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_rope<T>(ctx, name, static_cast<const T*>(src->data), dims, strides, rank,
                          static_cast<const float*>(cos_table->data),
                          static_cast<const float*>(sin_table->data), start,
                          static_cast<T*>(out->data));
}

// RotaryEmbedding::forward_encode on the [1, H, S, D] key view followed by
// LayerKvCache::append_encode's write of the result into the cache
// (src/nn/attention.rs:202-207 then src/model/kv_cache.rs:112-142): the
// gather, the rotation and the cache write in one pass.  The rotation uses
// positions start .. start + S, the cache rows the same range, as both
// calls take the cache's current length.
template <typename T>
rl_status rope_kv_entry(rl_context* ctx, const char* name, const char* write_name,
                        const rl_buffer* src, const uint64_t* dims, const uint64_t* strides,
                        uint32_t rank, const rl_buffer* cos_table, const rl_buffer* sin_table,
                        uint64_t table_rows, uint64_t start, const rl_buffer* cache,
                        uint64_t max_seq) {
    // The rotation's checks come first, as forward_encode runs before the
    // append; its output would be a contiguous tensor of the view's dims.
    if (rl_status st = check_buffer(src, "input")) return st;
    if (dims == nullptr || strides == nullptr)
        return fail(RL_ERR_INVALID_ARGUMENT, "dims or strides is null");
    if (rank < 2)
        return fail(RL_ERR_INVALID_DIMENSION,
                    "RoPE expects [..., sequence, head_dim], got rank %u", rank);
    if (rank > kMaxRank + 1) return fail(RL_ERR_INVALID_SHAPE, "tensor rank exceeds %d", kMaxRank + 1);
    const uint64_t seq_len = dims[rank - 2], head_dim = dims[rank - 1];
    if (head_dim == 0 || head_dim % 2 != 0)
        return fail(RL_ERR_INVALID_SHAPE, "RoPE head dimension must be positive and even, got %llu",
                    (unsigned long long)head_dim);
    for (uint32_t d = 0; d < rank; ++d)
        if (dims[d] == 0)
            return fail(RL_ERR_INVALID_SHAPE, "shape dimensions must be greater than zero");
    if (rl_status st = check_tables(cos_table, sin_table, table_rows, head_dim / 2, start, seq_len))
        return st;
    if (strides[rank - 1] != 1)
        return fail(RL_ERR_NON_CONTIGUOUS, "RoPE view must have a unit innermost stride");
    // Then the cache write's.
    if (rl_status st = validate_kv_write(write_name, cache, max_seq, src, dims, strides, rank,
                                         start, sizeof(T), false))
        return st;
    if (rl_status st = require_context(ctx)) return st;
    return launch_rope<T>(ctx, name, static_cast<const T*>(src->data), dims, strides, rank,
                          static_cast<const float*>(cos_table->data),
                          static_cast<const float*>(sin_table->data), start,
                          static_cast<T*>(cache->data),
                          DstRows{uint32_t(max_seq), uint32_t(start)});
}

// ------------------------------------------- Q, K and V of a layer, one launch

// One [1, H, S, D] view moved to its destination rows, rotated or copied,
// with the same optional second destination as RowJob.
struct RowTask {
    const void* src;
    void* dst;
    void* rep;
    RowDimsN<3> rd;
    FastDiv packs_per_row;  // packs of pairs per row (half_dim / N)
    DstRows dst_rows;
    uint32_t n_items;       // rows * packs_per_row
    uint32_t n_rep;
    uint32_t rep_rows;
    uint32_t rep_first;
    uint32_t first_block;   // blocks [first_block, next task's first_block)
    uint32_t rotate;
};

struct RowTasks {
    RowTask task[kMaxJobs];
};

// Blocks are split between the tasks; each block serves one task (a
// uniform branch), each thread UNROLL packs of pairs of it.
template <typename T, int N, int UNROLL>
__global__ __launch_bounds__(kThreads) void k_rope_tasks(RowTasks tasks,
                                                         const float* __restrict__ cos_table,
                                                         const float* __restrict__ sin_table,
                                                         uint32_t half_dim, uint32_t start) {
    typedef typename VecOf<T, N>::type V;
    typedef typename VecOf<float, N>::type VF;
    uint32_t k = 0;
#pragma unroll
    for (int t = 1; t < kMaxJobs; ++t) k += blockIdx.x >= tasks.task[t].first_block ? 1u : 0u;
    const RowTask& task = tasks.task[k];
    const T* src = static_cast<const T*>(task.src);
    T* out = static_cast<T*>(task.dst);
    T* rep = static_cast<T*>(task.rep);
    const uint64_t base =
        uint64_t(blockIdx.x - task.first_block) * kThreads * UNROLL + threadIdx.x;
    V a[UNROLL], b[UNROLL];
    VF c[UNROLL], s[UNROLL];
    uint64_t dst_off[UNROLL], rep_off[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
        const uint64_t i = base + uint64_t(u) * kThreads;
        if (i < task.n_items) {
            uint32_t row, pp;
            task.packs_per_row.divmod(uint32_t(i), row, pp);
            uint64_t src_off;
            uint32_t position, group;
            decode_row(task.rd, row, src_off, position, group);
            const uint32_t pair = pp * N;
            a[u] = *reinterpret_cast<const V*>(src + src_off + pair);
            b[u] = *reinterpret_cast<const V*>(src + src_off + half_dim + pair);
            if (task.rotate) {
                const uint64_t t = uint64_t(start + position) * half_dim + pair;
                c[u] = *reinterpret_cast<const VF*>(cos_table + t);
                s[u] = *reinterpret_cast<const VF*>(sin_table + t);
            }
            const uint64_t dst_row =
                uint64_t(group) * task.dst_rows.group_rows + task.dst_rows.first_row + position;
            dst_off[u] = dst_row * (2 * half_dim) + pair;
            rep_off[u] = (uint64_t(group) * task.n_rep * task.rep_rows + task.rep_first +
                          position) * (2 * half_dim) + pair;
        }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
        const uint64_t i = base + uint64_t(u) * kThreads;
        if (i < task.n_items) {
            V o1 = a[u], o2 = b[u];
            if (task.rotate) {
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    const float first = to_float(a[u][j]);
                    const float second = to_float(b[u][j]);
                    o1[j] = from_float<T>(first * c[u][j] - second * s[u][j]);
                    o2[j] = from_float<T>(second * c[u][j] + first * s[u][j]);
                }
            }
            if (out) {
                store_stream(reinterpret_cast<V*>(out + dst_off[u]), o1);
                store_stream(reinterpret_cast<V*>(out + dst_off[u] + half_dim), o2);
            }
            if (rep) {
                const uint64_t step = uint64_t(task.rep_rows) * (2 * half_dim);
                for (uint32_t r = 0; r < task.n_rep; ++r) {
                    store_stream(reinterpret_cast<V*>(rep + rep_off[u] + r * step), o1);
                    store_stream(reinterpret_cast<V*>(rep + rep_off[u] + r * step + half_dim), o2);
                }
            }
        }
    }
}

// A view's checks as an input of this launch: rank 4 [1, H, S, D] with a
// unit innermost stride, within its buffer, u32 sizes.
rl_status check_head_view(const rl_buffer* src, const uint64_t* dims, const uint64_t* strides,
                          uint64_t es, const char* what) {
    if (rl_status st = check_buffer(src, what)) return st;
    if (dims == nullptr || strides == nullptr)
        return fail(RL_ERR_INVALID_ARGUMENT, "%s dims or strides is null", what);
    uint64_t numel = 1;
    for (uint32_t d = 0; d < 4; ++d) {
        if (dims[d] == 0)
            return fail(RL_ERR_INVALID_SHAPE, "shape dimensions must be greater than zero");
        if (dims[d] > UINT32_MAX || strides[d] > UINT32_MAX || numel > UINT64_MAX / dims[d])
            return fail(RL_ERR_INVALID_SHAPE, "shape dimension exceeds u32");
        numel *= dims[d];
    }
    if (numel > UINT32_MAX) return fail(RL_ERR_INVALID_SHAPE, "%s size exceeds u32", what);
    if (strides[3] != 1)
        return fail(RL_ERR_NON_CONTIGUOUS, "%s view must have a unit innermost stride", what);
    if (src->byte_len < src->len * es)
        return fail(RL_ERR_INVALID_SHAPE, "%s does not hold %llu-byte elements", what,
                    (unsigned long long)es);
    unsigned __int128 last = 0;
    for (uint32_t d = 0; d < 4; ++d) last += (unsigned __int128)(dims[d] - 1) * strides[d];
    if (last >= src->len)
        return fail(RL_ERR_INVALID_SHAPE, "%s view reaches past the end of its %llu-element buffer",
                    what, (unsigned long long)src->len);
    return RL_OK;
}

// RotaryEmbedding::forward_encode of Q and of K at start_pos
// (src/nn/attention.rs:202-207), then LayerKvCache::append_encode of K and V
// at the same position (src/model/kv_cache.rs:112-142; the attention calls it
// with cache.len() == start_pos, :304-307), as one launch: Q rotated into a
// contiguous [1, QH, S, D] output, K rotated and V copied into rows start ..
// start + S of their caches.  Checks in the reference's order: RoPE on Q,
// RoPE on K, the append's shape check (ModelFormat), the two cache writes.
//
// With k_rep set, the same launch also writes tensor::repeat_kv of the
// caches' prefix after the append -- rows 0 .. start + S, the cache's key()
// and value() views (kv_cache.rs:87-99) -- as contiguous
// [1, KVH * n_rep, start + S, D] tensors: the new rows straight from the
// registers that hold them, the older rows 0 .. start copied from the cache
// by two more jobs, which read only rows this launch does not write.
// repeat_kv's checks (src/tensor/repeat_kv.rs:13-50) follow the append's.
template <typename T>
rl_status qkv_entry(rl_context* ctx, const char* name, const rl_buffer* q_src,
                    const uint64_t* q_dims, const uint64_t* q_strides, const rl_buffer* k_src,
                    const uint64_t* k_dims, const uint64_t* k_strides, const rl_buffer* v_src,
                    const uint64_t* v_dims, const uint64_t* v_strides,
                    const rl_buffer* cos_table, const rl_buffer* sin_table, uint64_t table_rows,
                    uint64_t start, const rl_buffer* q_out, const rl_buffer* k_cache,
                    const rl_buffer* v_cache, uint64_t max_seq, bool repeat = false,
                    uint64_t n_rep = 0, const rl_buffer* k_rep = nullptr,
                    const rl_buffer* v_rep = nullptr) {
    const char* write_name = sizeof(T) == 4 ? "kv_cache_write_f32" : "kv_cache_write_f16";
    for (int v = 0; v < 2; ++v) {  // Q, then K: RotaryEmbedding::forward_encode
        const rl_buffer* src = v == 0 ? q_src : k_src;
        const uint64_t* dims = v == 0 ? q_dims : k_dims;
        const uint64_t* strides = v == 0 ? q_strides : k_strides;
        if (rl_status st = check_head_view(src, dims, strides, sizeof(T), v == 0 ? "Q" : "K"))
            return st;
        const uint64_t head_dim = dims[3];
        if (head_dim % 2 != 0)
            return fail(RL_ERR_INVALID_SHAPE,
                        "RoPE head dimension must be positive and even, got %llu",
                        (unsigned long long)head_dim);
        if (rl_status st = check_tables(cos_table, sin_table, table_rows, head_dim / 2, start,
                                        dims[2]))
            return st;
    }
    if (rl_status st = check_output(q_out, q_dims[0] * q_dims[1] * q_dims[2] * q_dims[3],
                                    sizeof(T), "RoPE"))
        return st;
    if (rl_status st = check_head_view(v_src, v_dims, v_strides, sizeof(T), "V")) return st;
    // LayerKvCache::validate_append (kv_cache.rs:31-40): K and V of one shape.
    for (uint32_t d = 0; d < 4; ++d)
        if (k_dims[d] != v_dims[d])
            return fail(RL_ERR_MODEL_FORMAT,
                        "KV cache write shape does not match this layer: key and value differ");
    // Q and K of one layout apart from the head count (one sequence, one head_dim).
    if (q_dims[0] != k_dims[0] || q_dims[2] != k_dims[2] || q_dims[3] != k_dims[3])
        return fail(RL_ERR_INVALID_SHAPE, "Q and K must share batch, sequence and head_dim");
    if (rl_status st = validate_kv_write(write_name, k_cache, max_seq, k_src, k_dims, k_strides,
                                         4, start, sizeof(T), false))
        return st;
    if (rl_status st = validate_kv_write(write_name, v_cache, max_seq, v_src, v_dims, v_strides,
                                         4, start, sizeof(T), false))
        return st;
    const uint64_t total = start + k_dims[2];  // cache length after the append
    if (repeat) {
        if (n_rep == 0)
            return fail(RL_ERR_MODEL_FORMAT, "repeat_kv repeats must be greater than zero");
        if (k_dims[1] > UINT64_MAX / n_rep)
            return fail(RL_ERR_MODEL_FORMAT, "repeat_kv head count overflow");
        if (n_rep > UINT32_MAX || k_dims[1] * n_rep > UINT32_MAX || total > UINT32_MAX)
            return fail(RL_ERR_INVALID_SHAPE, "repeat_kv dimension exceeds u32");
        const uint64_t rep_numel = k_dims[0] * k_dims[1] * n_rep * total * k_dims[3];
        if (rl_status st = check_output(k_rep, rep_numel, sizeof(T), "repeat_kv")) return st;
        if (rl_status st = check_output(v_rep, rep_numel, sizeof(T), "repeat_kv")) return st;
    }
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;

    const uint64_t half = q_dims[3] / 2;
    const float* cs = static_cast<const float*>(cos_table->data);
    const float* sn = static_cast<const float*>(sin_table->data);
    const void* srcs[3] = {q_src->data, k_src->data, v_src->data};
    void* dsts[3] = {q_out->data, k_cache->data, v_cache->data};
    const uint64_t* dims[3] = {q_dims, k_dims, v_dims};
    const uint64_t* strides[3] = {q_strides, k_strides, v_strides};
    // Jobs 3 and 4 (with a repeat after a non-empty prefix): cache rows
    // 0 .. start of K and V, a [1, KVH, start, D] view of the cache.
    const int n_jobs = repeat && start > 0 ? 5 : 3;
    const uint64_t kvh = k_dims[1], hd = k_dims[3];
    const uint64_t prefix_dims[4] = {1, kvh, start, hd};
    const uint64_t prefix_strides[4] = {kvh * max_seq * hd, max_seq * hd, hd, 1};
    auto set_rep = [&](auto& job, int t) {
        if (!repeat || t == 0) return;
        job.rep = (t % 2 == 1 ? k_rep : v_rep)->data;
        job.n_rep = uint32_t(n_rep);
        job.rep_rows = uint32_t(total);
        job.rep_first = t < 3 ? uint32_t(start) : 0u;
    };
    if (const int lanes = row_lanes<T>(q_dims[3]);
        lanes && aligned_to(cs, 64 / sizeof(T)) && aligned_to(sn, 64 / sizeof(T)) &&
        (!repeat || (aligned_to(k_rep->data, 16) && aligned_to(v_rep->data, 16)))) {
        RowJobs jobs{};
        bool ok = true;
        for (int t = 0; t < n_jobs && ok; ++t) {
            if (t < 3)
                ok = make_job<T>(jobs.job[t], srcs[t], dims[t], strides[t], 4, dsts[t],
                                 t == 0 ? DstRows{uint32_t(dims[t][2]), 0}
                                        : DstRows{uint32_t(max_seq), uint32_t(start)},
                                 t < 2);
            else
                ok = make_job<T>(jobs.job[t], t == 3 ? k_cache->data : v_cache->data,
                                 prefix_dims, prefix_strides, 4, nullptr, DstRows{0, 0}, false);
            set_rep(jobs.job[t], t);
        }
        if (ok && launch_jobs<T>(ctx, jobs, n_jobs, lanes, cs, sn, start))
            return after_launch(ctx, name);
    }
    int n = 16 / int(sizeof(T));
    while (n > 1) {
        bool ok = half % n == 0 && aligned_to(cs, n * 4) && aligned_to(sn, n * 4);
        for (int t = 0; t < 3 && ok; ++t) {
            ok = aligned_to(srcs[t], n * sizeof(T)) && aligned_to(dsts[t], n * sizeof(T));
            for (uint32_t d = 0; d < 3 && ok; ++d) ok = strides[t][d] % n == 0;
        }
        if (repeat && ok)
            ok = aligned_to(k_rep->data, n * sizeof(T)) && aligned_to(v_rep->data, n * sizeof(T));
        if (ok) break;
        n >>= 1;
    }
    constexpr int U = 1;
    RowTasks tasks{};
    uint64_t blocks = 0;
    for (int t = 0; t < kMaxJobs; ++t) {
        RowTask& task = tasks.task[t];
        if (t >= n_jobs) {
            task.first_block = UINT32_MAX;
            continue;
        }
        const uint64_t* td = t < 3 ? dims[t] : prefix_dims;
        const uint64_t* ts = t < 3 ? strides[t] : prefix_strides;
        task.src = t < 3 ? srcs[t] : (t == 3 ? k_cache->data : v_cache->data);
        task.dst = t < 3 ? dsts[t] : nullptr;
        task.rd = make_row_dims<3>(td, ts, 4);
        task.packs_per_row = FastDiv(uint32_t(half / n));
        task.dst_rows = t == 0 ? DstRows{uint32_t(td[2]), 0}
                               : DstRows{uint32_t(max_seq), uint32_t(start)};
        const uint64_t rows = td[0] * td[1] * td[2];
        task.n_items = uint32_t(rows * (half / n));
        task.first_block = uint32_t(blocks);
        task.rotate = t < 2 ? 1u : 0u;
        set_rep(task, t);
        blocks += ceil_div(task.n_items, uint64_t(kThreads) * U);
    }
    if (blocks > (1u << 30)) return fail(RL_ERR_INVALID_SHAPE, "%s: work exceeds one launch", name);
    const dim3 grid(static_cast<unsigned>(blocks)), block(kThreads);
    const uint32_t h32 = uint32_t(half), s32 = uint32_t(start);
    switch (n) {
        case 8:
            RL_LAUNCH(ctx, (k_rope_tasks<T, 8, U>), grid, block, tasks, cs, sn, h32, s32);
            break;
        case 4:
            RL_LAUNCH(ctx, (k_rope_tasks<T, 4, U>), grid, block, tasks, cs, sn, h32, s32);
            break;
        case 2:
            RL_LAUNCH(ctx, (k_rope_tasks<T, 2, U>), grid, block, tasks, cs, sn, h32, s32);
            break;
        default:
            RL_LAUNCH(ctx, (k_rope_tasks<T, 1, U>), grid, block, tasks, cs, sn, h32, s32);
            break;
    }
    return after_launch(ctx, name);
}

}  // namespace

// A plain copy of a [..., S, D] view into rows group * group_rows +
// first_row + s of dst on the row-block kernel (a copy job, as the layer
// prologue's V append), or false when the view does not fit that kernel.
// A copy job issues its table loads like a rotating one and ignores the
// values (branch-free); they read floats [0, D / 2) of the table pointer,
// i.e. 2D bytes, which the view's first row holds (D elements of >= 2
// bytes, 16-byte aligned: make_job checks), so the source stands in for the
// table.
template <typename T>
bool launch_copy_rows(rl_context* ctx, const T* src, const uint64_t* dims,
                      const uint64_t* strides, uint32_t rank, T* dst, uint32_t group_rows,
                      uint32_t first_row) {
    const int lanes = row_lanes<T>(dims[rank - 1]);
    if (lanes == 0) return false;
    RowJobs jobs{};
    if (!make_job<T>(jobs.job[0], src, dims, strides, rank, dst, DstRows{group_rows, first_row},
                     false))
        return false;
    const float* table = reinterpret_cast<const float*>(src);
    return launch_jobs<T>(ctx, jobs, 1, lanes, table, table, 0);
}
template bool launch_copy_rows<float>(rl_context*, const float*, const uint64_t*, const uint64_t*,
                                      uint32_t, float*, uint32_t, uint32_t);
template bool launch_copy_rows<half_t>(rl_context*, const half_t*, const uint64_t*,
                                       const uint64_t*, uint32_t, half_t*, uint32_t, uint32_t);

}  // namespace rl

using namespace rl;

extern "C" {

rl_status rl_qkv_rope_kv_append_f32(rl_context* ctx, const rl_buffer* q_src,
                                    const uint64_t* q_dims, const uint64_t* q_strides,
                                    const rl_buffer* k_src, const uint64_t* k_dims,
                                    const uint64_t* k_strides, const rl_buffer* v_src,
                                    const uint64_t* v_dims, const uint64_t* v_strides,
                                    const rl_buffer* cos_table, const rl_buffer* sin_table,
                                    uint64_t table_rows, uint64_t start_pos,
                                    const rl_buffer* q_out, const rl_buffer* k_cache,
                                    const rl_buffer* v_cache, uint64_t max_seq) {
    return qkv_entry<float>(ctx, "qkv_rope_kv_append_f32", q_src, q_dims, q_strides, k_src,
                            k_dims, k_strides, v_src, v_dims, v_strides, cos_table, sin_table,
                            table_rows, start_pos, q_out, k_cache, v_cache, max_seq);
}

rl_status rl_qkv_rope_kv_append_f16(rl_context* ctx, const rl_buffer* q_src,
                                    const uint64_t* q_dims, const uint64_t* q_strides,
                                    const rl_buffer* k_src, const uint64_t* k_dims,
                                    const uint64_t* k_strides, const rl_buffer* v_src,
                                    const uint64_t* v_dims, const uint64_t* v_strides,
                                    const rl_buffer* cos_table, const rl_buffer* sin_table,
                                    uint64_t table_rows, uint64_t start_pos,
                                    const rl_buffer* q_out, const rl_buffer* k_cache,
                                    const rl_buffer* v_cache, uint64_t max_seq) {
    return qkv_entry<half_t>(ctx, "qkv_rope_kv_append_f16", q_src, q_dims, q_strides, k_src,
                             k_dims, k_strides, v_src, v_dims, v_strides, cos_table, sin_table,
                             table_rows, start_pos, q_out, k_cache, v_cache, max_seq);
}

rl_status rl_qkv_rope_kv_append_repeat_f32(
    rl_context* ctx, const rl_buffer* q_src, const uint64_t* q_dims, const uint64_t* q_strides,
    const rl_buffer* k_src, const uint64_t* k_dims, const uint64_t* k_strides,
    const rl_buffer* v_src, const uint64_t* v_dims, const uint64_t* v_strides,
    const rl_buffer* cos_table, const rl_buffer* sin_table, uint64_t table_rows,
    uint64_t start_pos, const rl_buffer* q_out, const rl_buffer* k_cache,
    const rl_buffer* v_cache, uint64_t max_seq, uint64_t n_rep, const rl_buffer* k_rep,
    const rl_buffer* v_rep) {
    return qkv_entry<float>(ctx, "qkv_rope_kv_append_repeat_f32", q_src, q_dims, q_strides,
                            k_src, k_dims, k_strides, v_src, v_dims, v_strides, cos_table,
                            sin_table, table_rows, start_pos, q_out, k_cache, v_cache, max_seq,
                            true, n_rep, k_rep, v_rep);
}

rl_status rl_qkv_rope_kv_append_repeat_f16(
    rl_context* ctx, const rl_buffer* q_src, const uint64_t* q_dims, const uint64_t* q_strides,
    const rl_buffer* k_src, const uint64_t* k_dims, const uint64_t* k_strides,
    const rl_buffer* v_src, const uint64_t* v_dims, const uint64_t* v_strides,
    const rl_buffer* cos_table, const rl_buffer* sin_table, uint64_t table_rows,
    uint64_t start_pos, const rl_buffer* q_out, const rl_buffer* k_cache,
    const rl_buffer* v_cache, uint64_t max_seq, uint64_t n_rep, const rl_buffer* k_rep,
    const rl_buffer* v_rep) {
    return qkv_entry<half_t>(ctx, "qkv_rope_kv_append_repeat_f16", q_src, q_dims, q_strides,
                             k_src, k_dims, k_strides, v_src, v_dims, v_strides, cos_table,
                             sin_table, table_rows, start_pos, q_out, k_cache, v_cache, max_seq,
                             true, n_rep, k_rep, v_rep);
}

rl_status rl_rope_kv_cache_write_f32(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                                     const uint64_t* strides, uint32_t rank,
                                     const rl_buffer* cos_table, const rl_buffer* sin_table,
                                     uint64_t table_rows, uint64_t start_pos,
                                     const rl_buffer* cache, uint64_t max_seq) {
    return rope_kv_entry<float>(ctx, "rope_kv_cache_write_f32", "kv_cache_write_f32", src, dims,
                                strides, rank, cos_table, sin_table, table_rows, start_pos, cache,
                                max_seq);
}

rl_status rl_rope_kv_cache_write_f16(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                                     const uint64_t* strides, uint32_t rank,
                                     const rl_buffer* cos_table, const rl_buffer* sin_table,
                                     uint64_t table_rows, uint64_t start_pos,
                                     const rl_buffer* cache, uint64_t max_seq) {
    return rope_kv_entry<half_t>(ctx, "rope_kv_cache_write_f16", "kv_cache_write_f16", src, dims,
                                 strides, rank, cos_table, sin_table, table_rows, start_pos,
                                 cache, max_seq);
}

rl_status rl_rope_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* cos_table,
                      const rl_buffer* sin_table, uint64_t seq_len, uint64_t head_dim,
                      uint64_t start_pos, const rl_buffer* out) {
    return rope_entry<float>(ctx, "rope_f32", input, cos_table, sin_table, seq_len, head_dim,
                             start_pos, out);
}

rl_status rl_rope_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* cos_table,
                      const rl_buffer* sin_table, uint64_t seq_len, uint64_t head_dim,
                      uint64_t start_pos, const rl_buffer* out) {
    return rope_entry<half_t>(ctx, "rope_f16", input, cos_table, sin_table, seq_len, head_dim,
                              start_pos, out);
}

rl_status rl_rope_strided_f32(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                              const uint64_t* strides, uint32_t rank, const rl_buffer* cos_table,
                              const rl_buffer* sin_table, uint64_t table_rows,
                              uint64_t start_pos, const rl_buffer* out) {
    return rope_strided_entry<float>(ctx, "rope_strided_f32", src, dims, strides, rank, cos_table,
                                     sin_table, table_rows, start_pos, out);
}

rl_status rl_rope_strided_f16(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                              const uint64_t* strides, uint32_t rank, const rl_buffer* cos_table,
                              const rl_buffer* sin_table, uint64_t table_rows,
                              uint64_t start_pos, const rl_buffer* out) {
    return rope_strided_entry<half_t>(ctx, "rope_strided_f16", src, dims, strides, rank,
                                      cos_table, sin_table, table_rows, start_pos, out);
}

}  // extern "C"
