// Context, memory and stream entry points of the C ABI.
// Replaces the reference's wgpu runtime: GpuContext::new (src/gpu/context.rs:22-69)
// and GpuBuffer upload/download (src/gpu/buffers.rs:27-191).
#include <cstring>
#include <mutex>

#include "common.hpp"

namespace {
std::mutex g_init_err_mu;
std::string g_init_err;
}  // namespace

namespace aur {

int set_error(aur_ctx* ctx, int code, const char* fmt, ...) {
  // A failing HIP call also stays behind as the runtime's sticky "last
  // error", which the next launch check (hipGetLastError) would report
  // against an unrelated kernel — a failed hipMalloc would fail the next
  // launch.  Every failure this library reports passes here: consume it.
  (void)hipGetLastError();
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) {
    ctx->last_error = buf;
  } else {
    std::lock_guard<std::mutex> g(g_init_err_mu);
    g_init_err = buf;
  }
  return code;
}

int ensure_workspace(aur_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->ws_bytes) return 0;
  // Growing the workspace synchronises the stream and frees / allocates
  // memory, none of which may happen while the stream is being captured
  // into a HIP graph (the graph would also keep the old pointer).  Work that
  // is captured passes its own Workspace instead.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  AUR_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return set_error(ctx, AUR_EINVAL,
                     "workspace of %zu bytes needed while the stream is captured; pass a Workspace", bytes);
  if (ctx->ws) {
    // The old workspace may still be read by enqueued kernels.
    AUR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    AUR_HIP(ctx, hipFree(ctx->ws));
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
  }
  size_t want = bytes < (size_t(16) << 20) ? (size_t(16) << 20) : bytes;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess)
    return set_error(ctx, AUR_ENOMEM, "workspace of %zu bytes: %s", want,
                     hipGetErrorString(e));
  // No clearing: every user (split-K partial tiles) writes the region it
  // reads back before reading it.
  ctx->ws = p;
  ctx->ws_bytes = want;
  return 0;
}

}  // namespace aur

extern "C" {

int aur_init(int device, aur_ctx** out) {
  if (!out) return aur::set_error(nullptr, AUR_EINVAL, "aur_init: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return aur::set_error(nullptr, e != hipSuccess ? (int)e : AUR_EINVAL,
                          "aur_init: no HIP device (%s)",
                          e != hipSuccess ? hipGetErrorString(e) : "count 0");
  if (device < 0 || device >= n)
    return aur::set_error(nullptr, AUR_EINVAL, "aur_init: device %d of %d", device, n);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess)
    return aur::set_error(nullptr, (int)e, "hipGetDeviceProperties: %s",
                          hipGetErrorString(e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return aur::set_error(nullptr, AUR_EINVAL,
                          "aur_init: device %d is %s, this library is built for gfx950",
                          device, prop.gcnArchName);
  e = hipSetDevice(device);
  if (e != hipSuccess)
    return aur::set_error(nullptr, (int)e, "hipSetDevice: %s", hipGetErrorString(e));
  aur_ctx* ctx = new aur_ctx();
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  aur::noalloc_scratch_init(ctx);
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return aur::set_error(nullptr, (int)e, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  *out = ctx;
  return 0;
}

int aur_destroy(aur_ctx* ctx) {
  if (!ctx) return 0;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  if (ctx->ws) hipFree(ctx->ws);
  hipStreamDestroy(ctx->stream);
  delete ctx;
  return 0;
}

const char* aur_last_error(const aur_ctx* ctx) {
  if (ctx) return ctx->last_error.c_str();
  std::lock_guard<std::mutex> g(g_init_err_mu);
  return g_init_err.c_str();
}

void* aur_stream(aur_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int aur_device_info(aur_ctx* ctx, char* buf, size_t len, int* cu_count) {
  AUR_CHECK_CTX(ctx);
  hipDeviceProp_t prop;
  AUR_HIP(ctx, hipGetDeviceProperties(&prop, ctx->device));
  if (buf && len) snprintf(buf, len, "%s %s", prop.name, prop.gcnArchName);
  if (cu_count) *cu_count = prop.multiProcessorCount;
  return 0;
}

int aur_malloc(aur_ctx* ctx, size_t bytes, void** out) {
  AUR_CHECK_CTX(ctx);
  if (!out) return aur::set_error(ctx, AUR_EINVAL, "aur_malloc: out is NULL");
  *out = nullptr;
  if (bytes == 0) return 0;
  AUR_HIP(ctx, hipMalloc(out, bytes));
  return 0;
}

int aur_free(aur_ctx* ctx, void* ptr) {
  AUR_CHECK_CTX(ctx);
  if (!ptr) return 0;
  // Kernels already enqueued may still use the buffer.
  AUR_HIP(ctx, hipStreamSynchronize(ctx->stream));
  AUR_HIP(ctx, hipFree(ptr));
  return 0;
}

int aur_h2d(aur_ctx* ctx, void* dst, const void* src, size_t bytes) {
  AUR_CHECK_CTX(ctx);
  if (bytes == 0) return 0;
  AUR_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  // The host buffer may be reused by the caller as soon as we return.
  AUR_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return 0;
}

int aur_d2h(aur_ctx* ctx, void* dst, const void* src, size_t bytes) {
  AUR_CHECK_CTX(ctx);
  if (bytes == 0) return 0;
  AUR_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  AUR_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return 0;
}

int aur_d2d(aur_ctx* ctx, void* dst, const void* src, size_t bytes) {
  AUR_CHECK_CTX(ctx);
  if (bytes == 0) return 0;
  AUR_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return 0;
}

int aur_memset0(aur_ctx* ctx, void* dst, size_t bytes) {
  AUR_CHECK_CTX(ctx);
  if (bytes == 0) return 0;
  AUR_HIP(ctx, hipMemsetAsync(dst, 0, bytes, ctx->stream));
  return 0;
}

int aur_sync(aur_ctx* ctx) {
  AUR_CHECK_CTX(ctx);
  AUR_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return 0;
}

int aur_event_create(aur_ctx* ctx, void** ev) {
  AUR_CHECK_CTX(ctx);
  if (!ev) return aur::set_error(ctx, AUR_EINVAL, "aur_event_create: ev is NULL");
  hipEvent_t e;
  AUR_HIP(ctx, hipEventCreate(&e));
  *ev = (void*)e;
  return 0;
}

int aur_event_record(aur_ctx* ctx, void* ev) {
  AUR_CHECK_CTX(ctx);
  AUR_HIP(ctx, hipEventRecord((hipEvent_t)ev, ctx->stream));
  return 0;
}

int aur_event_elapsed_ms(aur_ctx* ctx, void* start, void* stop, float* ms) {
  AUR_CHECK_CTX(ctx);
  if (!ms) return aur::set_error(ctx, AUR_EINVAL, "aur_event_elapsed_ms: ms is NULL");
  AUR_HIP(ctx, hipEventSynchronize((hipEvent_t)stop));
  AUR_HIP(ctx, hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return 0;
}

int aur_event_destroy(aur_ctx* ctx, void* ev) {
  AUR_CHECK_CTX(ctx);
  if (ev) AUR_HIP(ctx, hipEventDestroy((hipEvent_t)ev));
  return 0;
}

}  // extern "C"
