// RHI device of libvdsl.so: devices, buffers, queues (one hipStream_t each), hipGraph capture
// and replay, hipEvent timing, and the thread-local error channel of the C ABI (include/vdsl.h).
//
// The reference has no runtime.  The binding kinds recorded on buffers are the
// `vernon.semantic` vocabulary of VernonToSpirv.cpp:43-56; the device switch stands in for
// `ti.init(arch=...)` (fractal.py:5).

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_set>

#include "common.h"

namespace vdsl {

namespace {

thread_local std::string t_last_error;

// Every live handle is registered here, so a stale or foreign pointer is reported as
// VDSL_ERR_INVALID_HANDLE instead of being dereferenced.
std::mutex g_reg_mu;
std::unordered_set<const void*> g_live;

void reg_add(const void* p) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  g_live.insert(p);
}
bool reg_del(const void* p) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  return g_live.erase(p) != 0;
}
bool reg_has(const void* p) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  return g_live.count(p) != 0;
}

// Allocation-failure injection: the number of further allocations that may succeed; <0 = off.
std::atomic<int64_t> g_fail_alloc_after{-2};  // -2: not yet read from the environment

int64_t fail_alloc_budget() {
  int64_t v = g_fail_alloc_after.load();
  if (v == -2) {
    const char* e = std::getenv("VDSL_FAIL_ALLOC_AFTER");
    int64_t init = e ? std::strtoll(e, nullptr, 10) : -1;
    g_fail_alloc_after.compare_exchange_strong(v, init);
    v = g_fail_alloc_after.load();
  }
  return v;
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, size_t n, uint32_t pattern) {
  size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) p[i] = pattern;
}

}  // namespace

int fail(int status, const std::string& msg) {
  t_last_error = msg;
  return status;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return VDSL_OK;
  // The error is reported here; clear HIP's per-thread last error, or the next launch check
  // would report it again against an unrelated kernel.
  (void)hipGetLastError();
  int st = (e == hipErrorOutOfMemory) ? VDSL_ERR_OUT_OF_MEMORY : VDSL_ERR_DEVICE;
  return fail(st, std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return VDSL_OK;
  return fail(VDSL_ERR_DEVICE, std::string("launch of ") + kernel + " failed: " + hipGetErrorName(e));
}

bool valid_device(vdsl_device d) { return d && reg_has(d) && d->magic == kMagicDevice; }
bool valid_buffer(vdsl_buffer b) { return b && reg_has(b) && b->magic == kMagicBuffer; }
bool valid_queue(vdsl_queue q) { return q && reg_has(q) && q->magic == kMagicQueue; }

int enter_queue(vdsl_queue q) {
  if (!valid_queue(q)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid queue handle");
  // A launch check reads HIP's per-thread last error: drop one left by a call whose failure was
  // ignored or reported earlier, so an op's launch check sees its own launches only.
  (void)hipGetLastError();
  return check_hip(hipSetDevice(q->dev->ordinal), "hipSetDevice");
}

int check_buffer(vdsl_queue q, vdsl_buffer b, size_t bytes, const char* name, bool writable) {
  if (!valid_buffer(b)) return fail(VDSL_ERR_INVALID_HANDLE, std::string("invalid buffer handle: ") + name);
  if (b->dev != q->dev)
    return fail(VDSL_ERR_INVALID_ARG, std::string("buffer ") + name + " belongs to another device");
  if (bytes == kSizeOverflow)
    return fail(VDSL_ERR_SHAPE, std::string("operand ") + name + ": its byte size overflows (extents too large)");
  if (b->bytes < bytes)
    return fail(VDSL_ERR_SHAPE, std::string("buffer ") + name + " holds " + std::to_string(b->bytes) +
                                    " bytes, op needs " + std::to_string(bytes));
  if (writable && b->binding == VDSL_BIND_UNIFORM_CONSTANT)
    return fail(VDSL_ERR_INVALID_ARG, std::string("buffer ") + name + " is uniform_constant (read-only)");
  return VDSL_OK;
}

size_t dtype_size(int dtype) {
  switch (dtype) {
    case VDSL_F32: return 4;
    case VDSL_BF16: return 2;
    case VDSL_I8: return 1;
    case VDSL_I32: return 4;
    default: return 0;
  }
}

}  // namespace vdsl

using namespace vdsl;

extern "C" {

const char* vdsl_last_error(void) { return t_last_error.c_str(); }

int vdsl_abi_version(void) { return VDSL_ABI_VERSION; }

int vdsl_debug_fail_alloc_after(int64_t n) {
  fail_alloc_budget();
  g_fail_alloc_after.store(n < 0 ? -1 : n);
  return VDSL_OK;
}

// ---- devices ---------------------------------------------------------------------------------

int vdsl_device_count(int kind, int* count) {
  if (!count) return fail(VDSL_ERR_INVALID_ARG, "count is null");
  if (kind != VDSL_DEVICE_HIP) return fail(VDSL_ERR_INVALID_ARG, "unknown device kind " + std::to_string(kind));
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) n = 0;
  else if (e != hipSuccess) return check_hip(e, "hipGetDeviceCount");
  *count = n;
  return VDSL_OK;
}

int vdsl_device_open(int kind, int ordinal, vdsl_device* out) {
  if (!out) return fail(VDSL_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  int n = 0;
  VDSL_TRY(vdsl_device_count(kind, &n));
  if (ordinal < 0 || ordinal >= n)
    return fail(VDSL_ERR_NO_DEVICE, "no HIP device with ordinal " + std::to_string(ordinal) + " (" +
                                        std::to_string(n) + " present)");
  VDSL_TRY(check_hip(hipSetDevice(ordinal), "hipSetDevice"));
  auto* d = new vdsl_device_s();
  d->magic = kMagicDevice;
  d->ordinal = ordinal;
  d->live.store(0);
  int st = check_hip(hipGetDeviceProperties(&d->props, ordinal), "hipGetDeviceProperties");
  if (st != VDSL_OK) {
    delete d;
    return st;
  }
  w8a8_noalloc_setup(ordinal);
  reg_add(d);
  *out = d;
  return VDSL_OK;
}

int vdsl_device_close(vdsl_device dev) {
  if (!valid_device(dev)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid device handle");
  const int live = dev->live.load();
  if (live != 0)
    return fail(VDSL_ERR_INVALID_ARG, "device still owns " + std::to_string(live) +
                                          " buffers/queues/graphs/events; release them first");
  reg_del(dev);
  dev->magic = 0;
  delete dev;
  return VDSL_OK;
}

int vdsl_device_get_info(vdsl_device dev, vdsl_device_info* info) {
  if (!valid_device(dev)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid device handle");
  if (!info) return fail(VDSL_ERR_INVALID_ARG, "info is null");
  std::memset(info, 0, sizeof(*info));
  std::snprintf(info->name, sizeof(info->name), "%s", dev->props.name);
  std::snprintf(info->arch, sizeof(info->arch), "%s", dev->props.gcnArchName);
  info->compute_units = dev->props.multiProcessorCount;
  info->clock_khz = dev->props.clockRate;
  info->wavefront_size = dev->props.warpSize;
  info->lds_bytes_per_block = static_cast<int32_t>(dev->props.sharedMemPerBlock);
  info->hbm_bytes = dev->props.totalGlobalMem;
  return VDSL_OK;
}

// ---- buffers ---------------------------------------------------------------------------------

int vdsl_buffer_alloc(vdsl_device dev, size_t bytes, int binding, vdsl_buffer* out) {
  if (!out) return fail(VDSL_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!valid_device(dev)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid device handle");
  if (binding < VDSL_BIND_STORAGE_BUFFER || binding > VDSL_BIND_VARYING)
    return fail(VDSL_ERR_INVALID_ARG, "unknown binding kind " + std::to_string(binding));
  int64_t budget = fail_alloc_budget();
  if (budget == 0) return fail(VDSL_ERR_OUT_OF_MEMORY, "injected allocation failure");
  if (budget > 0) g_fail_alloc_after.fetch_sub(1);
  VDSL_TRY(check_hip(hipSetDevice(dev->ordinal), "hipSetDevice"));
  void* p = nullptr;
  // Zero-byte buffers are legal handles with no storage.
  if (bytes) VDSL_TRY(check_hip(hipMalloc(&p, bytes), "hipMalloc"));
  auto* b = new vdsl_buffer_s();
  b->magic = kMagicBuffer;
  b->dev = dev;
  b->ptr = p;
  b->bytes = bytes;
  b->binding = binding;
  dev->live.fetch_add(1);
  reg_add(b);
  *out = b;
  return VDSL_OK;
}

int vdsl_buffer_free(vdsl_buffer buf) {
  if (!valid_buffer(buf)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid buffer handle");
  reg_del(buf);
  int st = VDSL_OK;
  if (buf->ptr) {
    (void)hipSetDevice(buf->dev->ordinal);
    st = check_hip(hipFree(buf->ptr), "hipFree");
  }
  buf->dev->live.fetch_sub(1);
  buf->magic = 0;
  delete buf;
  return st;
}

int vdsl_buffer_size(vdsl_buffer buf, size_t* bytes) {
  if (!valid_buffer(buf)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid buffer handle");
  if (!bytes) return fail(VDSL_ERR_INVALID_ARG, "bytes is null");
  *bytes = buf->bytes;
  return VDSL_OK;
}

int vdsl_buffer_binding(vdsl_buffer buf, int* binding) {
  if (!valid_buffer(buf)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid buffer handle");
  if (!binding) return fail(VDSL_ERR_INVALID_ARG, "binding is null");
  *binding = buf->binding;
  return VDSL_OK;
}

int vdsl_buffer_device_address(vdsl_buffer buf, uint64_t* address) {
  if (!valid_buffer(buf)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid buffer handle");
  if (!address) return fail(VDSL_ERR_INVALID_ARG, "address is null");
  *address = reinterpret_cast<uint64_t>(buf->ptr);
  return VDSL_OK;
}

static int check_range(vdsl_buffer buf, size_t offset, size_t bytes) {
  if (offset > buf->bytes || bytes > buf->bytes - offset)
    return fail(VDSL_ERR_SHAPE, "range [" + std::to_string(offset) + ", +" + std::to_string(bytes) +
                                    ") exceeds buffer of " + std::to_string(buf->bytes) + " bytes");
  return VDSL_OK;
}

int vdsl_buffer_write(vdsl_queue q, vdsl_buffer buf, size_t offset, const void* src, size_t bytes) {
  VDSL_TRY(enter_queue(q));
  VDSL_TRY(check_buffer(q, buf, 0, "dst", false));
  if (q->capturing) return fail(VDSL_ERR_CAPTURE, "host transfers cannot be recorded into a graph");
  VDSL_TRY(check_range(buf, offset, bytes));
  if (!bytes) return VDSL_OK;
  if (!src) return fail(VDSL_ERR_INVALID_ARG, "src is null");
  VDSL_TRY(check_hip(hipMemcpyAsync(static_cast<char*>(buf->ptr) + offset, src, bytes,
                                    hipMemcpyHostToDevice, q->stream),
                     "hipMemcpyAsync(H2D)"));
  return check_hip(hipStreamSynchronize(q->stream), "hipStreamSynchronize");
}

int vdsl_buffer_read(vdsl_queue q, vdsl_buffer buf, size_t offset, void* dst, size_t bytes) {
  VDSL_TRY(enter_queue(q));
  VDSL_TRY(check_buffer(q, buf, 0, "src", false));
  if (q->capturing) return fail(VDSL_ERR_CAPTURE, "host transfers cannot be recorded into a graph");
  VDSL_TRY(check_range(buf, offset, bytes));
  if (!bytes) return VDSL_OK;
  if (!dst) return fail(VDSL_ERR_INVALID_ARG, "dst is null");
  VDSL_TRY(check_hip(hipMemcpyAsync(dst, static_cast<const char*>(buf->ptr) + offset, bytes,
                                    hipMemcpyDeviceToHost, q->stream),
                     "hipMemcpyAsync(D2H)"));
  return check_hip(hipStreamSynchronize(q->stream), "hipStreamSynchronize");
}

int vdsl_buffer_fill_u32(vdsl_queue q, vdsl_buffer buf, size_t offset, size_t bytes, uint32_t pattern) {
  VDSL_TRY(enter_queue(q));
  VDSL_TRY(check_buffer(q, buf, 0, "dst", true));
  VDSL_TRY(check_range(buf, offset, bytes));
  if ((offset | bytes) & 3u) return fail(VDSL_ERR_INVALID_ARG, "fill offset and size must be multiples of 4");
  size_t n = bytes / 4;
  if (!n) return VDSL_OK;
  size_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(fill_u32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream,
                     reinterpret_cast<uint32_t*>(static_cast<char*>(buf->ptr) + offset), n, pattern);
  return check_launch("fill_u32_kernel");
}

int vdsl_buffer_copy(vdsl_queue q, vdsl_buffer dst, size_t dst_offset, vdsl_buffer src, size_t src_offset,
                     size_t bytes) {
  VDSL_TRY(enter_queue(q));
  VDSL_TRY(check_buffer(q, dst, 0, "dst", true));
  VDSL_TRY(check_buffer(q, src, 0, "src", false));
  VDSL_TRY(check_range(dst, dst_offset, bytes));
  VDSL_TRY(check_range(src, src_offset, bytes));
  if (!bytes) return VDSL_OK;
  return check_hip(hipMemcpyAsync(static_cast<char*>(dst->ptr) + dst_offset,
                                  static_cast<const char*>(src->ptr) + src_offset, bytes,
                                  hipMemcpyDeviceToDevice, q->stream),
                   "hipMemcpyAsync(D2D)");
}

// ---- queues ----------------------------------------------------------------------------------

int vdsl_queue_create(vdsl_device dev, vdsl_queue* out) {
  if (!out) return fail(VDSL_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!valid_device(dev)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid device handle");
  VDSL_TRY(check_hip(hipSetDevice(dev->ordinal), "hipSetDevice"));
  hipStream_t s = nullptr;
  // Default priority, non-blocking with respect to the legacy null stream.
  VDSL_TRY(check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags"));
  auto* q = new vdsl_queue_s();
  q->magic = kMagicQueue;
  q->dev = dev;
  q->stream = s;
  q->capturing = false;
  dev->live.fetch_add(1);
  reg_add(q);
  *out = q;
  return VDSL_OK;
}

int vdsl_queue_destroy(vdsl_queue q) {
  if (!valid_queue(q)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid queue handle");
  if (q->capturing) return fail(VDSL_ERR_CAPTURE, "queue is capturing; end the graph first");
  (void)hipSetDevice(q->dev->ordinal);
  int st = check_hip(hipStreamSynchronize(q->stream), "hipStreamSynchronize");
  (void)hipStreamDestroy(q->stream);
  reg_del(q);
  q->dev->live.fetch_sub(1);
  q->magic = 0;
  delete q;
  return st;
}

int vdsl_queue_sync(vdsl_queue q) {
  VDSL_TRY(enter_queue(q));
  if (q->capturing) return fail(VDSL_ERR_CAPTURE, "cannot synchronize a capturing queue");
  return check_hip(hipStreamSynchronize(q->stream), "hipStreamSynchronize");
}

// ---- graphs ----------------------------------------------------------------------------------

int vdsl_graph_begin(vdsl_queue q) {
  VDSL_TRY(enter_queue(q));
  if (q->capturing) return fail(VDSL_ERR_CAPTURE, "queue is already capturing");
  VDSL_TRY(check_hip(hipStreamBeginCapture(q->stream, hipStreamCaptureModeThreadLocal),
                     "hipStreamBeginCapture"));
  q->capturing = true;
  return VDSL_OK;
}

int vdsl_graph_end(vdsl_queue q, vdsl_graph* out) {
  if (out) *out = nullptr;
  VDSL_TRY(enter_queue(q));
  if (!q->capturing) return fail(VDSL_ERR_CAPTURE, "graph_end without graph_begin");
  q->capturing = false;
  hipGraph_t g = nullptr;
  VDSL_TRY(check_hip(hipStreamEndCapture(q->stream, &g), "hipStreamEndCapture"));
  if (!out) {
    (void)hipGraphDestroy(g);
    return fail(VDSL_ERR_INVALID_ARG, "out is null (recording discarded)");
  }
  hipGraphExec_t exec = nullptr;
  int st = check_hip(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
  if (st != VDSL_OK) {
    (void)hipGraphDestroy(g);
    return st;
  }
  auto* gr = new vdsl_graph_s();
  gr->magic = kMagicGraph;
  gr->dev = q->dev;
  gr->graph = g;
  gr->exec = exec;
  q->dev->live.fetch_add(1);
  reg_add(gr);
  *out = gr;
  return VDSL_OK;
}

int vdsl_graph_launch(vdsl_graph g, vdsl_queue q) {
  if (!g || !reg_has(g) || g->magic != kMagicGraph) return fail(VDSL_ERR_INVALID_HANDLE, "invalid graph handle");
  VDSL_TRY(enter_queue(q));
  if (q->capturing) return fail(VDSL_ERR_CAPTURE, "cannot launch a graph into a capturing queue");
  if (g->dev != q->dev) return fail(VDSL_ERR_INVALID_ARG, "graph and queue are on different devices");
  return check_hip(hipGraphLaunch(g->exec, q->stream), "hipGraphLaunch");
}

int vdsl_graph_destroy(vdsl_graph g) {
  if (!g || !reg_has(g) || g->magic != kMagicGraph) return fail(VDSL_ERR_INVALID_HANDLE, "invalid graph handle");
  (void)hipSetDevice(g->dev->ordinal);
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  reg_del(g);
  g->dev->live.fetch_sub(1);
  g->magic = 0;
  delete g;
  return VDSL_OK;
}

// ---- events ----------------------------------------------------------------------------------

int vdsl_event_create(vdsl_device dev, vdsl_event* out) {
  if (!out) return fail(VDSL_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!valid_device(dev)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid device handle");
  VDSL_TRY(check_hip(hipSetDevice(dev->ordinal), "hipSetDevice"));
  hipEvent_t e = nullptr;
  VDSL_TRY(check_hip(hipEventCreate(&e), "hipEventCreate"));
  auto* ev = new vdsl_event_s();
  ev->magic = kMagicEvent;
  ev->dev = dev;
  ev->ev = e;
  dev->live.fetch_add(1);
  reg_add(ev);
  *out = ev;
  return VDSL_OK;
}

static bool valid_event(vdsl_event e) { return e && reg_has(e) && e->magic == kMagicEvent; }

int vdsl_event_record(vdsl_event ev, vdsl_queue q) {
  if (!valid_event(ev)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid event handle");
  VDSL_TRY(enter_queue(q));
  return check_hip(hipEventRecord(ev->ev, q->stream), "hipEventRecord");
}

int vdsl_event_elapsed_ms(vdsl_event start, vdsl_event end, float* ms) {
  if (!valid_event(start) || !valid_event(end)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid event handle");
  if (!ms) return fail(VDSL_ERR_INVALID_ARG, "ms is null");
  (void)hipSetDevice(end->dev->ordinal);
  VDSL_TRY(check_hip(hipEventSynchronize(end->ev), "hipEventSynchronize"));
  return check_hip(hipEventElapsedTime(ms, start->ev, end->ev), "hipEventElapsedTime");
}

int vdsl_event_destroy(vdsl_event ev) {
  if (!valid_event(ev)) return fail(VDSL_ERR_INVALID_HANDLE, "invalid event handle");
  (void)hipSetDevice(ev->dev->ordinal);
  (void)hipEventDestroy(ev->ev);
  reg_del(ev);
  ev->dev->live.fetch_sub(1);
  ev->magic = 0;
  delete ev;
  return VDSL_OK;
}

}  // extern "C"
