// ds5_ctx.hip -- the device context: the HIP implementation of DS5's frozen
// GPU API (src/shared/contracts.zig:374-384 assertGpuApi). The Metal glue it
// replaces is src/metal/metal.zig:103-432; the host-memory twin is
// src/kernels/cpu/ctx.zig:15-68.
//
// One context = one device, one stream, one begin/end event pair. Device
// buffers are owned by the context and released in ds5_hip_deinit, as the
// reference's contexts own theirs (src/engine/forward.zig:272-273).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "ds5_common.hpp"

int ds5_fail(ds5_hip_ctx* ctx, int code, const char* fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->last_error = buf;
    }
    return code;
}

int ds5_hip_status(ds5_hip_ctx* ctx, hipError_t err, const char* what) {
    if (err == hipSuccess) return DS5_OK;
    const int code = (err == hipErrorOutOfMemory) ? DS5_OUT_OF_MEMORY : DS5_DEVICE_FAILURE;
    return ds5_fail(ctx, code, "%s: %s", what, hipGetErrorString(err));
}

int ds5_after_launch(ds5_hip_ctx* ctx, const char* what) {
    return ds5_hip_status(ctx, hipGetLastError(), what);
}

// Grows a context-owned buffer to at least `bytes`. A larger buffer is a new
// allocation; the old one stays owned by the context until deinit, because
// enqueued kernels and captured graphs may still reference it. Growing needs a
// synchronise and an allocation, neither of which a stream capture allows.
static int grow_buffer(ds5_hip_ctx* ctx, size_t bytes, void*& buf, size_t& have, const char* what) {
    if (bytes > have) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        int rc = ds5_hip_status(ctx, hipStreamIsCapturing(ctx->stream, &cap), "workspace capture query");
        if (rc) return rc;
        if (cap != hipStreamCaptureStatusNone)
            return ds5_fail(ctx, DS5_DEVICE_FAILURE,
                            "%s must grow to %zu bytes during a stream capture: run the same call once "
                            "before capturing it", what, bytes);
        rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "workspace sync");
        if (rc) return rc;
        const size_t want = std::max<size_t>(bytes, 4u << 20);
        void* p = nullptr;
        rc = ds5_hip_status(ctx, hipMalloc(&p, want), "workspace alloc");
        if (rc) return rc;
        if (buf) ctx->owned.push_back(buf);
        buf = p;
        have = want;
    }
    return DS5_OK;
}

int ds5_workspace(ds5_hip_ctx* ctx, size_t bytes, void** out) {
    if (ctx->use_scratch) {
        // allocation-free call: the static scratch array, never an allocation
        if (bytes > ctx->scratch_bytes)
            return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "needs %zu bytes of scratch; the allocation-free entry point "
                            "holds at most %zu", bytes, ctx->scratch_bytes);
        *out = ctx->scratch;
        return DS5_OK;
    }
    if (int rc = grow_buffer(ctx, bytes, ctx->workspace, ctx->workspace_bytes, "workspace")) return rc;
    *out = ctx->workspace;
    return DS5_OK;
}

int ds5_aux_workspace(ds5_hip_ctx* ctx, size_t bytes, void** out) {
    if (int rc = grow_buffer(ctx, bytes, ctx->aux, ctx->aux_bytes, "workspace")) return rc;
    *out = ctx->aux;
    return DS5_OK;
}

hipEvent_t ds5_next_event(ds5_hip_ctx* ctx) {
    if (ctx->event_next == ctx->event_pool.size()) {
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        ctx->event_pool.push_back(e);
    }
    return ctx->event_pool[ctx->event_next++];
}

void ds5_timer_record(ds5_hip_ctx* ctx, const char* name, hipEvent_t start, hipEvent_t end) {
    ctx->pending.push_back({name, start, end});
}

int ds5_timers_resolve(ds5_hip_ctx* ctx) {
    if (ctx->pending.empty()) return DS5_OK;
    int rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "timer sync");
    if (rc) return rc;
    for (const auto& p : ctx->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.start, p.end) != hipSuccess) continue;
        auto& slot = ctx->kernel_ns[p.name];
        slot.first += (double)ms * 1.0e6;
        slot.second += 1;
    }
    ctx->pending.clear();
    ctx->event_next = 0;
    return DS5_OK;
}

extern "C" {

int ds5_hip_init(int device_index, ds5_hip_ctx** out) {
    if (!out) return DS5_SHAPE_MISMATCH;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return DS5_DEVICE_FAILURE;
    if (device_index < 0 || device_index >= n) return DS5_DEVICE_FAILURE;
    ds5_hip_ctx* ctx = new (std::nothrow) ds5_hip_ctx();
    if (!ctx) return DS5_OUT_OF_MEMORY;
    ctx->device = device_index;
    int rc = ds5_hip_status(ctx, hipSetDevice(device_index), "hipSetDevice");
    hipDeviceProp_t prop;
    if (!rc) rc = ds5_hip_status(ctx, hipGetDeviceProperties(&prop, device_index), "hipGetDeviceProperties");
    if (!rc) ctx->cu_count = prop.multiProcessorCount;
    if (!rc) rc = ds5_hip_status(ctx, hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate");
    if (!rc) rc = ds5_hip_status(ctx, hipEventCreate(&ctx->ev_begin), "hipEventCreate");
    if (!rc) rc = ds5_hip_status(ctx, hipEventCreate(&ctx->ev_end), "hipEventCreate");
    if (!rc) rc = ds5_scratch_init(ctx);
    if (rc) {
        ds5_hip_deinit(ctx);
        return rc;
    }
    if (const char* s = getenv("DS5_HIP_DECODE_CHUNK")) ctx->decode_chunk = (uint32_t)strtoul(s, nullptr, 10);
    if (const char* s = getenv("DS5_HIP_PLAN_ITEMS")) ctx->plan_items = (uint32_t)strtoul(s, nullptr, 10);
    if (const char* s = getenv("DS5_HIP_MOE_TWO_LAUNCH")) ctx->moe_two_launch = strtoul(s, nullptr, 10) != 0;
    *out = ctx;
    return DS5_OK;
}

void ds5_hip_deinit(ds5_hip_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (void* p : ctx->owned) (void)hipFree(p);
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
    for (hipEvent_t e : ctx->marks) (void)hipEventDestroy(e);
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    if (ctx->aux) (void)hipFree(ctx->aux);
    if (ctx->ev_begin) (void)hipEventDestroy(ctx->ev_begin);
    if (ctx->ev_end) (void)hipEventDestroy(ctx->ev_end);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int ds5_hip_create_buffer(ds5_hip_ctx* ctx, uint64_t len, ds5_buf* out) {
    if (!ctx || !out) return DS5_SHAPE_MISMATCH;
    *out = ds5_buf{nullptr, 0, 0};
    void* p = nullptr;
    // hipMalloc rejects 0 bytes on some runtimes; keep a 1-byte allocation so
    // the handle is still a valid, owned device pointer.
    int rc = ds5_hip_status(ctx, hipMalloc(&p, len ? len : 1), "hipMalloc");
    if (rc) return rc;
    ctx->owned.push_back(p);
    rc = ds5_hip_status(ctx, hipMemsetAsync(p, 0, len ? len : 1, ctx->stream), "hipMemsetAsync");
    if (!rc) rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc) return rc;
    *out = ds5_buf{p, 0, len};
    return DS5_OK;
}

int ds5_hip_buffer_from_bytes(ds5_hip_ctx* ctx, const void* bytes, uint64_t len, ds5_buf* out) {
    int rc = ds5_hip_create_buffer(ctx, len, out);
    if (rc) return rc;
    if (len) rc = ds5_hip_upload(ctx, *out, 0, bytes, len);
    return rc;
}

int ds5_hip_upload(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t offset, const void* bytes, uint64_t len) {
    if (!ctx) return DS5_SHAPE_MISMATCH;
    if (offset + len > buf.len || (len && (!bytes || !buf.handle)))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "upload: %llu bytes at %llu exceed view of %llu",
                        (unsigned long long)len, (unsigned long long)offset, (unsigned long long)buf.len);
    if (!len) return DS5_OK;
    char* dst = (char*)ds5_ptr(buf) + offset;
    int rc = ds5_hip_status(ctx, hipMemcpyAsync(dst, bytes, len, hipMemcpyHostToDevice, ctx->stream), "upload");
    if (!rc) rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "upload sync");
    return rc;
}

int ds5_hip_download(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t offset, void* out, uint64_t len) {
    if (!ctx) return DS5_SHAPE_MISMATCH;
    if (offset + len > buf.len || (len && (!out || !buf.handle)))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "download: %llu bytes at %llu exceed view of %llu",
                        (unsigned long long)len, (unsigned long long)offset, (unsigned long long)buf.len);
    // Drains all enqueued work first (the Metal glue's auto-flush).
    int rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "download sync");
    if (rc || !len) return rc;
    const char* src = (const char*)ds5_ptr(buf) + offset;
    rc = ds5_hip_status(ctx, hipMemcpyAsync(out, src, len, hipMemcpyDeviceToHost, ctx->stream), "download");
    if (!rc) rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "download sync");
    return rc;
}

void ds5_hip_begin(ds5_hip_ctx* ctx) {
    if (!ctx) return;
    if (hipEventRecord(ctx->ev_begin, ctx->stream) == hipSuccess) ctx->batch_open = true;
}

int ds5_hip_submit(ds5_hip_ctx* ctx) {
    if (!ctx) return DS5_SHAPE_MISMATCH;
    if (!ctx->batch_open) return ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "submit sync");
    ctx->batch_open = false;
    int rc = ds5_hip_status(ctx, hipEventRecord(ctx->ev_end, ctx->stream), "hipEventRecord");
    if (!rc) rc = ds5_hip_status(ctx, hipEventSynchronize(ctx->ev_end), "hipEventSynchronize");
    if (rc) return rc;
    float ms = 0.0f;
    rc = ds5_hip_status(ctx, hipEventElapsedTime(&ms, ctx->ev_begin, ctx->ev_end), "hipEventElapsedTime");
    if (rc) return rc;
    ctx->elapsed_ns = (uint64_t)((double)ms * 1.0e6);
    return ds5_timers_resolve(ctx);
}

uint64_t ds5_hip_gpu_elapsed_ns(ds5_hip_ctx* ctx) { return ctx ? ctx->elapsed_ns : 0; }

const char* ds5_hip_last_error(ds5_hip_ctx* ctx) { return ctx ? ctx->last_error.c_str() : "no context"; }

void* ds5_hip_stream(ds5_hip_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int ds5_hip_capture_begin(ds5_hip_ctx* ctx) {
    if (!ctx) return DS5_DEVICE_FAILURE;
    int rc = ds5_timers_resolve(ctx);
    if (rc) return rc;
    if (ctx->kernel_timing) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "capture: disable kernel timing first");
    return ds5_hip_status(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal),
                          "hipStreamBeginCapture");
}

int ds5_hip_capture_end(ds5_hip_ctx* ctx, void** graph_exec) {
    if (!ctx || !graph_exec) return DS5_DEVICE_FAILURE;
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    int rc = ds5_hip_status(ctx, hipStreamEndCapture(ctx->stream, &g), "hipStreamEndCapture");
    if (rc) return rc;
    hipGraphExec_t ge = nullptr;
    rc = ds5_hip_status(ctx, hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc) return rc;
    *graph_exec = (void*)ge;
    return DS5_OK;
}

int ds5_hip_graph_launch(ds5_hip_ctx* ctx, void* graph_exec) {
    if (!ctx || !graph_exec) return DS5_DEVICE_FAILURE;
    return ds5_hip_status(ctx, hipGraphLaunch((hipGraphExec_t)graph_exec, ctx->stream), "hipGraphLaunch");
}

void ds5_hip_graph_destroy(void* graph_exec) {
    if (graph_exec) (void)hipGraphExecDestroy((hipGraphExec_t)graph_exec);
}

int ds5_hip_timing_begin(ds5_hip_ctx* ctx) {
    if (!ctx) return DS5_DEVICE_FAILURE;
    ctx->marks_used = 0;
    return DS5_OK;
}

int ds5_hip_timing_mark(ds5_hip_ctx* ctx) {
    if (!ctx) return DS5_DEVICE_FAILURE;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    int rc = ds5_hip_status(ctx, hipStreamIsCapturing(ctx->stream, &cs), "hipStreamIsCapturing");
    if (rc) return rc;
    if (cs != hipStreamCaptureStatusNone) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "timing_mark: the stream is capturing");
    if (ctx->marks_used == ctx->marks.size()) {
        hipEvent_t e = nullptr;
        rc = ds5_hip_status(ctx, hipEventCreate(&e), "hipEventCreate");
        if (rc) return rc;
        ctx->marks.push_back(e);
    }
    rc = ds5_hip_status(ctx, hipEventRecord(ctx->marks[ctx->marks_used], ctx->stream), "hipEventRecord");
    if (!rc) ctx->marks_used++;
    return rc;
}

int ds5_hip_timing_read(ds5_hip_ctx* ctx, uint64_t* ns, uint32_t max, uint32_t* count) {
    if (!ctx || !count || (max && !ns)) return DS5_SHAPE_MISMATCH;
    *count = 0;
    int rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "timing sync");
    if (rc) return rc;
    const size_t n = ctx->marks_used > 1 ? ctx->marks_used - 1 : 0;
    for (size_t i = 0; i < n && i < max; i++) {
        float ms = 0.0f;
        rc = ds5_hip_status(ctx, hipEventElapsedTime(&ms, ctx->marks[i], ctx->marks[i + 1]), "hipEventElapsedTime");
        if (rc) return rc;
        ns[i] = (uint64_t)((double)ms * 1.0e6);
    }
    *count = (uint32_t)n;
    return DS5_OK;
}

int ds5_hip_set_kernel_timing(ds5_hip_ctx* ctx, int enable) {
    if (!ctx) return DS5_DEVICE_FAILURE;
    int rc = ds5_timers_resolve(ctx);
    ctx->kernel_timing = enable != 0;
    ctx->kernel_ns.clear();
    return rc;
}

int ds5_hip_kernel_time(ds5_hip_ctx* ctx, const char* kernel, uint64_t* launches, double* total_ns) {
    if (!ctx || !kernel || !launches || !total_ns) return DS5_SHAPE_MISMATCH;
    int rc = ds5_timers_resolve(ctx);
    if (rc) return rc;
    auto it = ctx->kernel_ns.find(kernel);
    *launches = it == ctx->kernel_ns.end() ? 0 : it->second.second;
    *total_ns = it == ctx->kernel_ns.end() ? 0.0 : it->second.first;
    return DS5_OK;
}

}  // extern "C"
