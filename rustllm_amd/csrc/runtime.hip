// runtime.hip -- context, stream-ordered buffer pool, execution batching,
// graphs, events, submission counters and error reporting: the HIP
// replacement of src/metal/{context,buffer,execution}.rs.
#include <cstdio>
#include <cstring>

#include "common.hpp"

namespace rl {

static thread_local std::string g_last_error;
static thread_local rl_error_payload g_last_payload{};

rl_status fail(rl_status code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    g_last_payload = rl_error_payload{};
    g_last_payload.code = code;
    return code;
}

void clear_error() {
    g_last_error.clear();
    g_last_payload = rl_error_payload{};
}

static std::string dims_text(const uint64_t* dims, uint32_t rank) {
    std::string s = "[";
    for (uint32_t i = 0; i < rank; ++i) {
        if (i) s += ", ";
        s += std::to_string(dims[i]);
    }
    return s + "]";
}

rl_status fail_shape_mismatch(const uint64_t* left, uint32_t left_rank, const uint64_t* right,
                              uint32_t right_rank) {
    fail(RL_ERR_SHAPE_MISMATCH, "left=%s, right=%s", dims_text(left, left_rank).c_str(),
         dims_text(right, right_rank).c_str());
    g_last_payload.left_rank = left_rank;
    g_last_payload.right_rank = right_rank;
    for (uint32_t i = 0; i < left_rank && i < RL_ERROR_MAX_RANK; ++i)
        g_last_payload.left[i] = left[i];
    for (uint32_t i = 0; i < right_rank && i < RL_ERROR_MAX_RANK; ++i)
        g_last_payload.right[i] = right[i];
    return RL_ERR_SHAPE_MISMATCH;
}

rl_status fail_position_out_of_range(uint64_t start_pos, uint64_t seq_len, uint64_t max_seq_len) {
    // The end is printed as the reference does (start_pos + seq_len); an
    // overflowing sum prints its wrapped value there as well.
    fail(RL_ERR_POSITION_OUT_OF_RANGE, "position range [%llu, %llu) exceeds max sequence length %llu",
         (unsigned long long)start_pos, (unsigned long long)(start_pos + seq_len),
         (unsigned long long)max_seq_len);
    g_last_payload.start_pos = start_pos;
    g_last_payload.seq_len = seq_len;
    g_last_payload.max_seq_len = max_seq_len;
    return RL_ERR_POSITION_OUT_OF_RANGE;
}

rl_status fail_invalid_token_id(uint32_t token_id, uint64_t vocab_size) {
    fail(RL_ERR_INVALID_TOKEN_ID, "invalid token id %u: vocabulary size is %llu", token_id,
         (unsigned long long)vocab_size);
    g_last_payload.token_id = token_id;
    g_last_payload.vocab_size = vocab_size;
    return RL_ERR_INVALID_TOKEN_ID;
}

static rl_status hip_fail(hipError_t err, const char* what) {
    return fail(RL_ERR_DEVICE, "%s: %s", what, hipGetErrorString(err));
}

#define RL_HIP(call, what)                                  \
    do {                                                    \
        hipError_t rl_err_ = (call);                        \
        if (rl_err_ != hipSuccess) return hip_fail(rl_err_, what); \
    } while (0)

// Size classes: multiples of 512 B up to 64 KiB, then eight classes per
// power of two, so a pooled block wastes at most 1/8 of its size.
uint64_t BufferPool::size_class(uint64_t bytes) {
    if (bytes <= 65536) return ceil_div(bytes, 512) * 512;
    uint64_t top = 63 - __builtin_clzll(bytes);  // floor(log2)
    uint64_t step = uint64_t(1) << (top - 3);
    return ceil_div(bytes, step) * step;
}

rl_status BufferPool::allocate(uint64_t bytes, void** out) {
    uint64_t cls = size_class(bytes);
    auto it = free_blocks.find(cls);
    if (it != free_blocks.end()) {
        *out = it->second;
        free_blocks.erase(it);
        return RL_OK;
    }
    void* p = nullptr;
    hipError_t err = hipMalloc(&p, cls);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        trim();
        err = hipMalloc(&p, cls);
        if (err != hipSuccess) return hip_fail(err, "hipMalloc");
    }
    block_size[p] = cls;
    reserved_bytes += cls;
    *out = p;
    return RL_OK;
}

void BufferPool::release(void* ptr) {
    auto it = block_size.find(ptr);
    if (it == block_size.end()) return;  // not a pool block
    free_blocks.emplace(it->second, ptr);
}

void BufferPool::trim() {
    for (auto& kv : free_blocks) {
        auto it = block_size.find(kv.second);
        if (it != block_size.end()) {
            reserved_bytes -= it->second;
            block_size.erase(it);
        }
        (void)hipFree(kv.second);
    }
    free_blocks.clear();
}

BufferPool::~BufferPool() {
    for (auto& kv : block_size) (void)hipFree(kv.first);
    block_size.clear();
    free_blocks.clear();
}

rl_status activate(rl_context* ctx) {
    RL_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return RL_OK;
}

rl_status after_launch(rl_context* ctx, const char* kernel_name) {
    if (ctx->fused_error != hipSuccess) {  // a fused launch this op flushed failed
        const hipError_t fe = ctx->fused_error;
        ctx->fused_error = hipSuccess;
        return hip_fail(fe, "fused streaming ops");
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, kernel_name);
    if (ctx->profiling) {
        // MetalContext::pipeline counts one dispatch and one encoder per op
        // (src/metal/context.rs:95-103).
        ctx->profile.kernel_dispatches += 1;
        ctx->profile.compute_encoders += 1;
        ctx->dispatches_by_name[kernel_name] += 1;
    }
    return RL_OK;
}

rl_status stage_to_device(rl_context* ctx, const void* host, uint64_t bytes, void** dev) {
    *dev = nullptr;
    if (ctx->capturing)
        return fail(RL_ERR_DEVICE, "host arrays cannot be recorded into a graph");
    // The previous staged copy must have read the staging area before it is
    // overwritten (or freed to grow it).
    if (ctx->staging_pending) {
        RL_HIP(hipEventSynchronize(ctx->staging_done), "hipEventSynchronize");
        ctx->staging_pending = false;
    }
    if (bytes > ctx->staging_bytes) {
        uint64_t cap = 4096;
        while (cap < bytes) cap *= 2;
        if (ctx->staging != nullptr) {
            (void)hipHostFree(ctx->staging);
            ctx->staging = nullptr;
            ctx->staging_bytes = 0;
        }
        RL_HIP(hipHostMalloc(&ctx->staging, cap, hipHostMallocDefault), "hipHostMalloc");
        ctx->staging_bytes = cap;
    }
    if (ctx->staging_done == nullptr)
        RL_HIP(hipEventCreateWithFlags(&ctx->staging_done, hipEventDisableTiming),
               "hipEventCreateWithFlags");
    std::memcpy(ctx->staging, host, bytes);
    void* p = nullptr;
    if (rl_status st = ctx->pool.allocate(bytes, &p)) return st;
    hipError_t err = hipMemcpyAsync(p, ctx->staging, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipEventRecord(ctx->staging_done, ctx->stream);
    if (err != hipSuccess) {
        ctx->pool.release(p);
        return hip_fail(err, "staging copy");
    }
    ctx->staging_pending = true;
    *dev = p;
    return RL_OK;
}

rl_status check_buffer(const rl_buffer* b, const char* what) {
    if (b == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "%s buffer is null", what);
    if (b->len > 0 && b->data == nullptr)
        return fail(RL_ERR_INVALID_ARGUMENT, "%s buffer has no device memory", what);
    return RL_OK;
}

rl_status check_output(const rl_buffer* out, uint64_t len, uint64_t element_size,
                       const char* op) {
    if (rl_status st = check_buffer(out, "output")) return st;
    if (out->len != len || out->byte_len != len * element_size)
        return fail(RL_ERR_INVALID_SHAPE,
                    "%s output buffer has %llu elements (%llu bytes), expected %llu elements of "
                    "%llu bytes",
                    op, (unsigned long long)out->len, (unsigned long long)out->byte_len,
                    (unsigned long long)len, (unsigned long long)element_size);
    return RL_OK;
}

}  // namespace rl

using namespace rl;

struct rl_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

struct rl_event {
    hipEvent_t event = nullptr;
};

extern "C" {

const char* rl_last_error_message(void) { return g_last_error.c_str(); }

rl_status rl_last_error_payload(rl_error_payload* out) {
    if (out == nullptr) return RL_OK;
    *out = g_last_payload;
    return g_last_payload.code;
}

const char* rl_version(void) { return "rustllm-hip 0.1.0 (gfx950)"; }

int32_t rl_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

static rl_status create_context(int32_t device, void* stream, rl_context** out) {
    if (out == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "output pointer is null");
    *out = nullptr;
    int count = rl_device_count();
    if (count <= 0)
        return fail(RL_ERR_DEVICE, "no HIP GPU is available; run on a host with an MI355X");
    if (device < 0 || device >= count)
        return fail(RL_ERR_DEVICE, "device %d does not exist (%d visible)", device, count);
    RL_HIP(hipSetDevice(device), "hipSetDevice");
    auto* ctx = new rl_context();
    ctx->device = device;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) ==
            hipSuccess &&
        cus > 0)
        ctx->num_cus = cus;
    if (stream != nullptr) {
        ctx->stream = static_cast<hipStream_t>(stream);
        ctx->owns_stream = false;
    } else {
        // Default priority on purpose: one in-order stream per context.
        hipError_t err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
        if (err != hipSuccess) {
            delete ctx;
            return hip_fail(err, "hipStreamCreateWithFlags");
        }
        ctx->owns_stream = true;
    }
    *out = ctx;
    return RL_OK;
}

rl_status rl_context_create(int32_t device, rl_context** out) {
    return create_context(device, nullptr, out);
}

rl_status rl_context_create_on_stream(int32_t device, void* stream, rl_context** out) {
    if (stream == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "stream is null");
    return create_context(device, stream, out);
}

void rl_context_destroy(rl_context* ctx) {
    if (ctx == nullptr) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->staging != nullptr) (void)hipHostFree(ctx->staging);
    if (ctx->staging_done != nullptr) (void)hipEventDestroy(ctx->staging_done);
    if (ctx->tickets != nullptr) (void)hipFree(ctx->tickets);
    if (ctx->owns_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;  // the pool frees its blocks
}

void* rl_context_stream(const rl_context* ctx) {
    return ctx == nullptr ? nullptr : static_cast<void*>(ctx->stream);
}

rl_status rl_buffer_empty(rl_context* ctx, uint64_t len, uint64_t element_size, rl_buffer* out) {
    if (out == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "output buffer pointer is null");
    *out = rl_buffer{nullptr, 0, 0};
    // MetalBuffer::empty_with_element_size asserts len > 0 && element_size > 0.
    if (len == 0 || element_size == 0)
        return fail(RL_ERR_INVALID_SHAPE, "invalid buffer size: %llu elements of %llu bytes",
                    (unsigned long long)len, (unsigned long long)element_size);
    if (len > UINT64_MAX / element_size)
        return fail(RL_ERR_INVALID_SHAPE, "buffer byte size overflow");
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    uint64_t bytes = len * element_size;
    void* p = nullptr;
    if (rl_status st = ctx->pool.allocate(bytes, &p)) return st;
    *out = rl_buffer{p, len, bytes};
    if (ctx->profiling) {
        ctx->profile.buffer_allocations += 1;
        ctx->profile.allocated_bytes += bytes;
    }
    return RL_OK;
}

rl_status rl_buffer_from_host(rl_context* ctx, const void* host, uint64_t len,
                              uint64_t element_size, rl_buffer* out) {
    if (out == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "output buffer pointer is null");
    *out = rl_buffer{nullptr, 0, 0};
    if (host == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "host pointer is null");
    if (len == 0 || element_size == 0)
        return fail(RL_ERR_INVALID_SHAPE, "cannot create a buffer from empty data");
    if (len > UINT64_MAX / element_size)
        return fail(RL_ERR_INVALID_SHAPE, "buffer byte size overflow");
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    uint64_t bytes = len * element_size;
    void* p = nullptr;
    if (rl_status st = ctx->pool.allocate(bytes, &p)) return st;
    // Stream-ordered, so a recycled block is not overwritten before earlier
    // kernels that read it have run.
    hipError_t err = hipMemcpyAsync(p, host, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    if (err != hipSuccess) {
        ctx->pool.release(p);
        return hip_fail(err, "upload");
    }
    *out = rl_buffer{p, len, bytes};
    return RL_OK;
}

rl_status rl_buffer_to_host(rl_context* ctx, const rl_buffer* buffer, void* host,
                            uint64_t byte_len) {
    if (rl_status st = check_buffer(buffer, "source")) return st;
    if (host == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "host pointer is null");
    if (byte_len > buffer->byte_len)
        return fail(RL_ERR_INVALID_SHAPE, "download of %llu bytes from a %llu-byte buffer",
                    (unsigned long long)byte_len, (unsigned long long)buffer->byte_len);
    if (rl_status st = require_context(ctx)) return st;
    if (ctx->capturing) return fail(RL_ERR_DEVICE, "cannot download while recording a graph");
    if (rl_status st = activate(ctx)) return st;
    if (byte_len == 0) return RL_OK;
    RL_HIP(hipMemcpyAsync(host, buffer->data, byte_len, hipMemcpyDeviceToHost, ctx->stream),
           "download");
    RL_HIP(hipStreamSynchronize(ctx->stream), "download");
    return RL_OK;
}

rl_status rl_buffer_copy(rl_context* ctx, const rl_buffer* src, const rl_buffer* dst,
                         uint64_t byte_len) {
    if (rl_status st = check_buffer(src, "source")) return st;
    if (rl_status st = check_buffer(dst, "destination")) return st;
    if (byte_len > src->byte_len || byte_len > dst->byte_len)
        return fail(RL_ERR_INVALID_SHAPE, "copy of %llu bytes exceeds a buffer",
                    (unsigned long long)byte_len);
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    if (byte_len == 0) return RL_OK;
    if (rl_status st = flush_fused(ctx)) return st;
    RL_HIP(hipMemcpyAsync(dst->data, src->data, byte_len, hipMemcpyDeviceToDevice, ctx->stream),
           "device copy");
    return RL_OK;
}

void rl_buffer_release(rl_context* ctx, rl_buffer* buffer) {
    if (ctx == nullptr || buffer == nullptr || buffer->data == nullptr) return;
    ctx->pool.release(buffer->data);
    *buffer = rl_buffer{nullptr, 0, 0};
}

rl_status rl_context_trim(rl_context* ctx) {
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    RL_HIP(hipStreamSynchronize(ctx->stream), "synchronize");
    ctx->pool.trim();
    return RL_OK;
}

rl_status rl_execution_begin(rl_context* ctx) {
    if (rl_status st = require_context(ctx)) return st;
    ctx->active_executions += 1;
    if (ctx->profiling) ctx->profile.command_buffers += 1;  // execution.rs:11-20
    return RL_OK;
}

rl_status rl_execution_finish(rl_context* ctx) {
    if (rl_status st = require_context(ctx)) return st;
    if (ctx->active_executions > 0) ctx->active_executions -= 1;
    if (ctx->profiling) {  // execution.rs:30-36: one commit and one wait
        ctx->profile.commits += 1;
        ctx->profile.waits += 1;
    }
    if (ctx->capturing) return fail(RL_ERR_DEVICE, "cannot wait while recording a graph");
    if (rl_status st = activate(ctx)) return st;
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "execution");
    RL_HIP(hipStreamSynchronize(ctx->stream), "execution");
    return RL_OK;
}

rl_status rl_graph_capture_begin(rl_context* ctx) {
    if (rl_status st = require_context(ctx)) return st;
    if (ctx->capturing) return fail(RL_ERR_DEVICE, "a graph is already being recorded");
    if (rl_status st = activate(ctx)) return st;
    RL_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal),
           "hipStreamBeginCapture");
    ctx->capturing = true;
    return RL_OK;
}

rl_status rl_context_set_fusion(rl_context* ctx, int32_t enabled) {
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    if (rl_status st = flush_fused(ctx)) return st;  // ops deferred so far keep their batch
    ctx->fuse_recorded = enabled != 0;
    return RL_OK;
}

rl_status rl_graph_capture_end(rl_context* ctx, rl_graph** out) {
    if (out == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "output pointer is null");
    *out = nullptr;
    if (rl_status st = require_context(ctx)) return st;
    if (!ctx->capturing) return fail(RL_ERR_DEVICE, "no graph is being recorded");
    if (rl_status st = activate(ctx)) return st;
    const rl_status flushed = flush_fused(ctx);  // the recording ends even if this fails
    ctx->capturing = false;
    hipGraph_t graph = nullptr;
    RL_HIP(hipStreamEndCapture(ctx->stream, &graph), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    if (flushed != RL_OK) {
        (void)hipGraphDestroy(graph);
        return flushed;
    }
    hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (err != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(err, "hipGraphInstantiate");
    }
    auto* g = new rl_graph();
    g->graph = graph;
    g->exec = exec;
    *out = g;
    return RL_OK;
}

rl_status rl_graph_launch(rl_context* ctx, rl_graph* graph) {
    if (graph == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "graph is null");
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    RL_HIP(hipGraphLaunch(graph->exec, ctx->stream), "hipGraphLaunch");
    return RL_OK;
}

void rl_graph_destroy(rl_graph* graph) {
    if (graph == nullptr) return;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}

rl_status rl_event_create(rl_context* ctx, rl_event** out) {
    if (out == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "output pointer is null");
    *out = nullptr;
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    auto* e = new rl_event();
    hipError_t err = hipEventCreate(&e->event);
    if (err != hipSuccess) {
        delete e;
        return hip_fail(err, "hipEventCreate");
    }
    *out = e;
    return RL_OK;
}

rl_status rl_event_record(rl_context* ctx, rl_event* event) {
    if (event == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "event is null");
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    if (rl_status st = flush_fused(ctx)) return st;
    RL_HIP(hipEventRecord(event->event, ctx->stream), "hipEventRecord");
    return RL_OK;
}

rl_status rl_event_wait(rl_context* ctx, rl_event* event) {
    if (event == nullptr) return fail(RL_ERR_INVALID_ARGUMENT, "event is null");
    if (rl_status st = require_context(ctx)) return st;
    if (rl_status st = activate(ctx)) return st;
    if (rl_status st = flush_fused(ctx)) return st;
    RL_HIP(hipStreamWaitEvent(ctx->stream, event->event, 0), "hipStreamWaitEvent");
    return RL_OK;
}

rl_status rl_event_elapsed_ms(rl_event* start, rl_event* end, float* ms) {
    if (start == nullptr || end == nullptr || ms == nullptr)
        return fail(RL_ERR_INVALID_ARGUMENT, "null event or result pointer");
    RL_HIP(hipEventSynchronize(end->event), "hipEventSynchronize");
    RL_HIP(hipEventElapsedTime(ms, start->event, end->event), "hipEventElapsedTime");
    return RL_OK;
}

rl_status rl_event_time_next_kernel(rl_context* ctx, rl_event* start, rl_event* stop) {
    if (start == nullptr || stop == nullptr)
        return fail(RL_ERR_INVALID_ARGUMENT, "null event");
    if (rl_status st = require_context(ctx)) return st;
    if (ctx->capturing) return fail(RL_ERR_DEVICE, "cannot time a kernel while recording a graph");
    ctx->timed_start = start->event;
    ctx->timed_stop = stop->event;
    return RL_OK;
}

void rl_event_destroy(rl_event* event) {
    if (event == nullptr) return;
    if (event->event) (void)hipEventDestroy(event->event);
    delete event;
}

void rl_profile_begin(rl_context* ctx) {
    if (ctx == nullptr) return;
    ctx->profiling = true;
    ctx->profile = rl_profile{};
    ctx->dispatches_by_name.clear();
}

int32_t rl_profile_take(rl_context* ctx, rl_profile* out) {
    if (ctx == nullptr || !ctx->profiling) return 0;
    if (out != nullptr) *out = ctx->profile;
    ctx->profiling = false;
    return 1;
}

uint64_t rl_profile_dispatches(const rl_context* ctx, const char* kernel_name) {
    if (ctx == nullptr || kernel_name == nullptr) return 0;
    auto it = ctx->dispatches_by_name.find(kernel_name);
    return it == ctx->dispatches_by_name.end() ? 0 : it->second;
}

}  // extern "C"
