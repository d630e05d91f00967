// runtime.hip -- context, device memory, host-boundary copies and the Q8_0
// weight upload (GGUF rows -> split device layout) of the gfx950 library.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <chrono>
#include <cstring>
#include <mutex>

#include "vxm_model.h"

int vxm_fail(vxm_ctx *ctx, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    return code;
}

static std::string g_open_err;

extern "C" int vxm_open(int device, vxm_ctx **out) {
    if (!out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        g_open_err = "no HIP device";
        return VXM_ERR_BACKEND;
    }
    if (device < 0 || device >= n) {
        g_open_err = "device index out of range";
        return VXM_ERR_INVALID_ARG;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        g_open_err = "hipGetDeviceProperties failed";
        return VXM_ERR_BACKEND;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_open_err = std::string("unsupported architecture ") + prop.gcnArchName + " (built for gfx950)";
        return VXM_ERR_UNSUPPORTED_ARCH;
    }
    if (hipSetDevice(device) != hipSuccess) {
        g_open_err = "hipSetDevice failed";
        return VXM_ERR_BACKEND;
    }
    vxm_ctx *ctx = new vxm_ctx();
    ctx->device = device;
    ctx->n_cu = prop.multiProcessorCount;
    // A blocking stream: ordered with work on the legacy default stream, so
    // callers that stage inputs there (torch, hipMemcpy) need no extra sync.
    if (hipStreamCreate(&ctx->stream) != hipSuccess) {
        delete ctx;
        g_open_err = "hipStreamCreate failed";
        return VXM_ERR_BACKEND;
    }
    if (hipMalloc((void **)&ctx->dev_err, 256) != hipSuccess ||
        hipMemsetAsync(ctx->dev_err, 0, 256, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        if (ctx->dev_err) (void)hipFree(ctx->dev_err);
        hipStreamDestroy(ctx->stream);
        delete ctx;
        g_open_err = "device error word allocation failed";
        return VXM_ERR_BACKEND;
    }
    ctx->split_epoch_dev = (uint32_t *)((char *)ctx->dev_err + 64);   // zero: no split launched yet
    vxm_scratch_setup(ctx);   // a failure is reported by the allocation-free entry only
    *out = ctx;
    return VXM_OK;
}

static void forget_stream(vxm_ctx *ctx);

extern "C" int vxm_close(vxm_ctx *ctx) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    forget_stream(ctx);
    if (ctx->act_buf) hipFree(ctx->act_buf);
    if (ctx->split_buf) hipFree(ctx->split_buf);
    if (ctx->split_cnt) hipFree(ctx->split_cnt);
    if (ctx->parts_buf) hipFree(ctx->parts_buf);
    if (ctx->dev_err) hipFree(ctx->dev_err);
    if (ctx->pin_out) hipHostFree(ctx->pin_out);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return VXM_OK;
}

extern "C" int vxm_sync(vxm_ctx *ctx) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->split_launched) {
        // a K-split GEMM since the last check: did every fix-up find its partials?
        ctx->split_launched = false;
        int e = 0;
        VXM_HIP(ctx, hipMemcpy(&e, ctx->dev_err, sizeof e, hipMemcpyDeviceToHost));
        if (e) {
            VXM_HIP(ctx, hipMemset(ctx->dev_err, 0, sizeof e));
            return vxm_fail(ctx, VXM_ERR_BACKEND,
                            "mul_mat: a K-split partial tile never arrived (its outputs were written as NaN)");
        }
    }
    return VXM_OK;
}

extern "C" void *vxm_get_stream(vxm_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

extern "C" const char *vxm_last_error(const vxm_ctx *ctx) {
    return ctx ? ctx->err.c_str() : g_open_err.c_str();
}

extern "C" int vxm_set_quant_variant(vxm_ctx *ctx, int variant) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (variant != VXM_QUANT_REF && variant != VXM_QUANT_X86)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "unknown quantizer variant %d", variant);
    ctx->quant_variant = variant;
    return VXM_OK;
}

extern "C" int vxm_set_path(vxm_ctx *ctx, int path) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (path < VXM_PATH_AUTO || path > VXM_PATH_MFMA_TILED)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "unknown kernel path %d", path);
    ctx->path = path;
    return VXM_OK;
}

static bool capturing(vxm_ctx *ctx) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return st != hipStreamCaptureStatusNone;
}

// A scratch buffer that must grow cannot be replaced under graph capture (the
// free and the allocation would synchronise the stream being recorded).
#define VXM_NO_GROWTH_UNDER_CAPTURE(ctx, what, bytes)                                                    \
    do {                                                                                                 \
        if (capturing(ctx))                                                                              \
            return vxm_fail((ctx), VXM_ERR_INVALID_ARG,                                                  \
                            "%s of %zu bytes would have to grow under graph capture: run the sequence " \
                            "once before capturing it",                                                  \
                            (what), (size_t)(bytes));                                                    \
    } while (0)

// ---- one launch order per device for the single-launch kernels --------------

struct vxm_launch_slot {
    std::mutex mu;
    hipEvent_t ev = nullptr;
    hipStream_t last = nullptr;
};
static vxm_launch_slot g_launch_slots[64];

// Holds the device's slot from begin to end (the launch goes in between).  The
// ordering event is recorded lazily: a launch from another stream records it on the
// stream of the device's last single launch (so it covers that launch and whatever
// that stream queued after it) and waits for it, while launches from one stream,
// ordered by the stream itself, record nothing (a marker after every launch cost
// 3.3 us per decode token: 551.6 against 548.3 us).  A wait binds to the event as
// recorded when the wait is queued, so no cycle of waits can form.  The slot names
// only streams of open contexts: vxm_close clears it.
int vxm_ordered_launch_begin(vxm_ctx *ctx, vxm_launch_slot **slot, bool *cap) {
    *slot = nullptr;
    *cap = false;
    if (ctx->device < 0 || ctx->device >= 64)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "single-launch kernel: device %d beyond the launch table",
                        ctx->device);
    *cap = capturing(ctx);
    vxm_launch_slot &o = g_launch_slots[ctx->device];
    o.mu.lock();
    *slot = &o;
    if (*cap) return VXM_OK;
    hipError_t e = hipSuccess;
    if (o.last && o.last != ctx->stream) {
        if (!o.ev) e = hipEventCreateWithFlags(&o.ev, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventRecord(o.ev, o.last);
        if (e == hipSuccess) e = hipStreamWaitEvent(ctx->stream, o.ev, 0);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        o.mu.unlock();
        *slot = nullptr;
        return vxm_fail(ctx, VXM_ERR_BACKEND, "single-launch kernel: launch ordering failed: %s", hipGetErrorString(e));
    }
    return VXM_OK;
}

int vxm_ordered_launch_end(vxm_ctx *ctx, vxm_launch_slot *slot, bool cap) {
    if (!slot) return VXM_OK;
    if (!cap) slot->last = ctx->stream;
    slot->mu.unlock();
    return VXM_OK;
}

// A closing context's stream leaves the launch table (its work has completed).
static void forget_stream(vxm_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= 64) return;
    vxm_launch_slot &o = g_launch_slots[ctx->device];
    std::lock_guard<std::mutex> g(o.mu);
    if (o.last == ctx->stream) o.last = nullptr;
}

// ---- graph capture of the context's stream ---------------------------------
struct vxm_graph {
    hipGraphExec_t exec = nullptr;
    int device = 0;
};

extern "C" int vxm_capture_begin(vxm_ctx *ctx) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (capturing(ctx)) return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "capture_begin: the stream is already capturing");
    VXM_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return VXM_OK;
}

extern "C" int vxm_capture_end(vxm_ctx *ctx, vxm_graph **out) {
    if (!ctx || !out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    hipGraph_t graph = nullptr;
    VXM_HIP(ctx, hipStreamEndCapture(ctx->stream, &graph));
    if (!graph) return vxm_fail(ctx, VXM_ERR_BACKEND, "capture_end: the capture recorded no graph");
    vxm_graph *g = new vxm_graph();
    g->device = ctx->device;
    const hipError_t e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        delete g;
        return vxm_fail(ctx, VXM_ERR_BACKEND, "capture_end: graph instantiation failed: %s", hipGetErrorString(e));
    }
    *out = g;
    return VXM_OK;
}

extern "C" int vxm_graph_launch(vxm_ctx *ctx, const vxm_graph *g) {
    if (!ctx || !g || !g->exec) return VXM_ERR_INVALID_ARG;
    if (g->device != ctx->device)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "graph_launch: graph of device %d on a context of device %d",
                        g->device, ctx->device);
    VXM_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
    return VXM_OK;
}

extern "C" int vxm_graph_free(vxm_graph *g) {
    if (!g) return VXM_OK;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    delete g;
    return VXM_OK;
}

extern "C" int vxm_malloc(vxm_ctx *ctx, size_t bytes, void **out_dev) {
    if (!ctx || !out_dev) return VXM_ERR_INVALID_ARG;
    *out_dev = nullptr;
    if (bytes == 0) bytes = 256;
    if (hipMalloc(out_dev, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "hipMalloc of %zu bytes failed", bytes);
    }
    return VXM_OK;
}

extern "C" int vxm_free(vxm_ctx *ctx, void *dev) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (dev) VXM_HIP(ctx, hipFree(dev));
    return VXM_OK;
}

extern "C" int vxm_memcpy_h2d(vxm_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes) {
    if (!ctx || (!dst_dev && bytes) || (!src_host && bytes)) return VXM_ERR_INVALID_ARG;
    VXM_HIP(ctx, hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream));
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VXM_OK;
}

// Small device-to-host copies (a decode step's hidden state, 8 KB) go through a
// pinned, device-mapped host buffer that one wave of a copy kernel on the
// context stream writes directly, followed by a sequence number; the host spins
// on that number for a short while (falling back to a stream synchronisation
// when the stream has more work queued) and copies the bytes out.  The DMA copy
// of the same bytes into pageable memory and the stream synchronisation took
// about 20 us per token after the decode launch.
constexpr size_t kPinOutBytes = 64 << 10;
constexpr double kPinSpinUs = 200.0;

__global__ __launch_bounds__(64) void k_copy_out(const uint4 *__restrict__ src, uint4 *__restrict__ dst, int64_t n16,
                                                 unsigned *__restrict__ flag, unsigned seq) {
    for (int64_t i = threadIdx.x; i < n16; i += 64) dst[i] = src[i];
    // every lane's stores reach host memory before the sequence number does
    __threadfence_system();
    if (threadIdx.x == 0) __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

extern "C" int vxm_memcpy_d2h(vxm_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes) {
    if (!ctx || (!dst_host && bytes) || (!src_dev && bytes)) return VXM_ERR_INVALID_ARG;
    if (bytes > 0 && bytes <= kPinOutBytes && (bytes & 15) == 0 && ((uintptr_t)src_dev & 15) == 0 && !capturing(ctx)) {
        if (!ctx->pin_out) {
            void *h = nullptr, *d = nullptr;
            if (hipHostMalloc(&h, kPinOutBytes + 256, hipHostMallocMapped) != hipSuccess ||
                hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
                (void)hipGetLastError();
                if (h) (void)hipHostFree(h);
                return vxm_fail(ctx, VXM_ERR_OOM, "pinned staging of %zu bytes failed", kPinOutBytes);
            }
            *(volatile unsigned *)((char *)h + kPinOutBytes) = 0;
            ctx->pin_out = h;
            ctx->pin_out_dev = d;
            ctx->pin_seq = 0;
        }
        const unsigned seq = ++ctx->pin_seq ? ctx->pin_seq : ++ctx->pin_seq;   // never 0
        hipLaunchKernelGGL(k_copy_out, dim3(1), dim3(64), 0, ctx->stream, (const uint4 *)src_dev,
                           (uint4 *)ctx->pin_out_dev, (int64_t)(bytes / 16),
                           (unsigned *)((char *)ctx->pin_out_dev + kPinOutBytes), seq);
        VXM_CHECK_LAUNCH(ctx);
        volatile unsigned *flag = (volatile unsigned *)((char *)ctx->pin_out + kPinOutBytes);
        const auto t0 = std::chrono::steady_clock::now();
        while (*flag != seq &&
               std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() < kPinSpinUs) {
        }
        if (*flag != seq) {
            // more work ahead of the copy, or a failure: wait for the stream and report it
            VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
            if (*flag != seq) return vxm_fail(ctx, VXM_ERR_BACKEND, "d2h copy: the copy kernel left no data");
        }
        std::atomic_thread_fence(std::memory_order_acquire);
        memcpy(dst_host, ctx->pin_out, bytes);
        return VXM_OK;
    }
    VXM_HIP(ctx, hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VXM_OK;
}

int vxm_ensure_act(vxm_ctx *ctx, size_t bytes) {
    if (ctx->act_bytes >= bytes) return VXM_OK;
    VXM_NO_GROWTH_UNDER_CAPTURE(ctx, "activation scratch", bytes);
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->act_buf) VXM_HIP(ctx, hipFree(ctx->act_buf));
    ctx->act_buf = nullptr;
    ctx->act_bytes = 0;
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (hipMalloc(&ctx->act_buf, want) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "activation scratch of %zu bytes failed", want);
    }
    ctx->act_bytes = want;
    return VXM_OK;
}

int vxm_ensure_parts(vxm_ctx *ctx, size_t bytes) {
    if (ctx->parts_bytes >= bytes) return VXM_OK;
    VXM_NO_GROWTH_UNDER_CAPTURE(ctx, "GEMM slice scratch", bytes);
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->parts_buf) VXM_HIP(ctx, hipFree(ctx->parts_buf));
    ctx->parts_buf = nullptr;
    ctx->parts_bytes = 0;
    if (hipMalloc(&ctx->parts_buf, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "GEMM slice scratch of %zu bytes failed", bytes);
    }
    ctx->parts_bytes = bytes;
    return VXM_OK;
}

int vxm_ensure_split(vxm_ctx *ctx, size_t bytes, size_t n_counters) {
    if (ctx->split_bytes < bytes || ctx->split_ncnt < n_counters)
        VXM_NO_GROWTH_UNDER_CAPTURE(ctx, "GEMM split scratch", bytes);
    if (ctx->split_bytes < bytes) {
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->split_buf) VXM_HIP(ctx, hipFree(ctx->split_buf));
        ctx->split_buf = nullptr;
        ctx->split_bytes = 0;
        if (hipMalloc(&ctx->split_buf, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return vxm_fail(ctx, VXM_ERR_OOM, "GEMM split scratch of %zu bytes failed", bytes);
        }
        // tagged partial words: tag 0 never matches a launch
        VXM_HIP(ctx, hipMemsetAsync(ctx->split_buf, 0, bytes, ctx->stream));
        ctx->split_bytes = bytes;
    }
    if (ctx->split_ncnt < n_counters) {
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->split_cnt) VXM_HIP(ctx, hipFree(ctx->split_cnt));
        ctx->split_cnt = nullptr;
        ctx->split_ncnt = 0;
        const size_t n = n_counters < 4096 ? 4096 : n_counters;
        if (hipMalloc((void **)&ctx->split_cnt, n * sizeof(int)) != hipSuccess) {
            (void)hipGetLastError();
            return vxm_fail(ctx, VXM_ERR_OOM, "GEMM split counters failed");
        }
        VXM_HIP(ctx, hipMemsetAsync(ctx->split_cnt, 0, n * sizeof(int), ctx->stream));
        ctx->split_ncnt = n;
    }
    return VXM_OK;
}

// ---- weight repack --------------------------------------------------------

// One thread per 34-byte block: split into quants / scales / GEMV scales /
// tile-blocked GEMM scales.
__global__ void k_repack_q8_0(const uint16_t *__restrict__ src, int64_t nblocks, int64_t nb,
                              int C, int8_t *__restrict__ qs, uint16_t *__restrict__ d,
                              uint16_t *__restrict__ dg, uint16_t *__restrict__ dt) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint16_t *blk = src + i * 17;   // 34 bytes = 17 half-words, 2-byte aligned
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) w[j] = (uint32_t)blk[1 + 2 * j] | ((uint32_t)blk[2 + 2 * j] << 16);
    uint4 *dst = (uint4 *)(qs + i * 32);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    d[i] = blk[0];
    if (dg) {
        int64_t row = i / nb, b = i % nb;
        int64_t c = b / 32, p = b % 32;
        dg[row * nb + p * C + c] = blk[0];
    }
    if (dt) {
        const int64_t row = i / nb, b = i % nb;
        dt[(((row >> 6) * (nb >> 2) + (b >> 2)) * 64 + (row & 63)) * 4 + (b & 3)] = blk[0];
    }
}

__global__ void k_unpack_q8_0(const int8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                              int64_t nblocks, uint16_t *__restrict__ dst) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint4 *s = (const uint4 *)(qs + i * 32);
    uint4 a = s[0], b = s[1];
    uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint16_t *o = dst + i * 17;
    o[0] = d[i];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        o[1 + 2 * j] = (uint16_t)(w[j] & 0xffffu);
        o[2 + 2 * j] = (uint16_t)(w[j] >> 16);
    }
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

extern "C" int vxm_upload_q8_0(vxm_ctx *ctx, const void *gguf_rows, int64_t n_rows, int64_t k,
                               vxm_weight **out) {
    if (!ctx || !gguf_rows || !out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    if (n_rows <= 0 || k <= 0 || k % VXM_QK != 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                        "Q8_0 tensor needs k %% 32 == 0 and positive sizes (n=%lld k=%lld)",
                        (long long)n_rows, (long long)k);
    const int64_t nb = k / VXM_QK, nblocks = n_rows * nb;
    const size_t raw = (size_t)nblocks * VXM_BLOCK_BYTES;
    const bool gemv_perm = (k % 1024) == 0;
    const bool tile_scales = (k % 256) == 0;
    const size_t qs_b = align256((size_t)n_rows * k);
    const size_t d_b = align256((size_t)nblocks * 2);
    const size_t dt_b = tile_scales ? align256((size_t)((n_rows + 127) / 128) * 128 * nb * 2) : 0;
    const size_t total = qs_b + d_b + (gemv_perm ? d_b : 0) + dt_b;
    vxm_weight *w = new vxm_weight();
    w->n = n_rows;
    w->k = k;
    if (hipMalloc(&w->base, total) != hipSuccess) {
        (void)hipGetLastError();
        delete w;
        return vxm_fail(ctx, VXM_ERR_OOM, "weight allocation of %zu bytes failed", total);
    }
    w->bytes = total;
    w->qs = (int8_t *)w->base;
    w->d = (uint16_t *)((char *)w->base + qs_b);
    w->dg = gemv_perm ? (uint16_t *)((char *)w->base + qs_b + d_b) : nullptr;
    w->dt = tile_scales ? (uint16_t *)((char *)w->base + qs_b + d_b + (gemv_perm ? d_b : 0)) : nullptr;
    void *tmp = nullptr;
    if (hipMalloc(&tmp, raw) != hipSuccess) {
        (void)hipGetLastError();
        hipFree(w->base);
        delete w;
        return vxm_fail(ctx, VXM_ERR_OOM, "staging allocation of %zu bytes failed", raw);
    }
    int rc = VXM_OK;
    if (hipMemcpyAsync(tmp, gguf_rows, raw, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        (w->dt && hipMemsetAsync(w->dt, 0, dt_b, ctx->stream) != hipSuccess)) {   // rows past n: zero scales
        rc = vxm_fail(ctx, VXM_ERR_BACKEND, "weight upload copy failed");
    } else {
        const int threads = 256;
        const int64_t grid = (nblocks + threads - 1) / threads;
        hipLaunchKernelGGL(k_repack_q8_0, dim3((unsigned)grid), dim3(threads), 0, ctx->stream,
                           (const uint16_t *)tmp, nblocks, nb, (int)(k / 1024), w->qs, w->d, w->dg, w->dt);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(ctx->stream) != hipSuccess)
            rc = vxm_fail(ctx, VXM_ERR_BACKEND, "weight repack failed");
    }
    hipFree(tmp);
    if (rc != VXM_OK) {
        hipFree(w->base);
        delete w;
        return rc;
    }
    *out = w;
    return VXM_OK;
}

extern "C" int vxm_download_q8_0(vxm_ctx *ctx, const vxm_weight *w, void *gguf_rows) {
    if (!ctx || !w || !gguf_rows) return VXM_ERR_INVALID_ARG;
    const int64_t nblocks = w->n * (w->k / VXM_QK);
    const size_t raw = (size_t)nblocks * VXM_BLOCK_BYTES;
    void *tmp = nullptr;
    if (hipMalloc(&tmp, raw) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "download staging of %zu bytes failed", raw);
    }
    const int threads = 256;
    const int64_t grid = (nblocks + threads - 1) / threads;
    hipLaunchKernelGGL(k_unpack_q8_0, dim3((unsigned)grid), dim3(threads), 0, ctx->stream, w->qs,
                       w->d, nblocks, (uint16_t *)tmp);
    int rc = VXM_OK;
    if (hipGetLastError() != hipSuccess ||
        hipMemcpyAsync(gguf_rows, tmp, raw, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess)
        rc = vxm_fail(ctx, VXM_ERR_BACKEND, "weight download failed");
    hipFree(tmp);
    return rc;
}

extern "C" int vxm_weight_free(vxm_ctx *ctx, vxm_weight *w) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (!w) return VXM_OK;
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (w->base) VXM_HIP(ctx, hipFree(w->base));
    delete w;
    return VXM_OK;
}

extern "C" int64_t vxm_weight_rows(const vxm_weight *w) { return w ? w->n : -1; }
extern "C" int64_t vxm_weight_cols(const vxm_weight *w) { return w ? w->k : -1; }
