// Runtime wrappers of the C ABI (reference: kernels/drama.cu:1995-2044, src/ffi.rs:13-31).
// Thin HIP calls; the engine never needs HIP headers.
#include "common.hpp"

#include <cstring>
#include <mutex>
#include <new>

using namespace drm;

namespace {
// The error word lives in pinned, mapped host memory (portable to every device), so kernels on
// any GPU can set it and the host reads it with a plain load.  Set up once per process.
uint32_t* g_err_host = nullptr;
uint32_t* g_err_dev = nullptr;
std::once_flag g_err_once;

void err_setup() {
  void* p = nullptr;
  if (hipHostMalloc(&p, 64, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  std::memset(p, 0, 64);
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  g_err_host = static_cast<uint32_t*>(p);
  __atomic_store_n(&g_err_dev, static_cast<uint32_t*>(d), __ATOMIC_RELEASE);
}
// Set up when the library is loaded, if the process sees a device, so that no launcher has to
// allocate (the no-allocation step entry point only reads the word's address); a process that
// loads the library before its device is visible sets it up on the first call of err_word().
__attribute__((constructor)) void err_setup_at_load() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return;
  }
  std::call_once(g_err_once, err_setup);
}
}  // namespace

uint32_t* drm::err_word() {
  std::call_once(g_err_once, err_setup);
  return g_err_dev;
}
uint32_t* drm::err_word_noalloc() { return __atomic_load_n(&g_err_dev, __ATOMIC_ACQUIRE); }
uint32_t drm::err_pending() {
  return g_err_host ? __atomic_load_n(g_err_host, __ATOMIC_ACQUIRE) : 0u;
}

API const char* dr_error_string(int e) {
  if (e == -1) return "unsupported shape";
  if (e == (int)kErrStepTimeout)
    return "fused decode step gave up waiting for its workgroups (not co-resident: another kernel held CUs)";
  if (e == (int)kErrPrefillWait) return "prefill grouped GEMM gave up waiting for an LDS hand-off";
  if (e == (int)kErrRouteWait) return "fused small-batch decode gave up waiting for the router's picks";
  return hipGetErrorString((hipError_t)e);
}
// The runtime's last launch error first; then a pending library error, which this call clears.
API int dr_last_error(void) {
  const int e = (int)hipGetLastError();
  if (e) return e;
  if (!g_err_host) return 0;
  return (int)__atomic_exchange_n(g_err_host, 0u, __ATOMIC_ACQ_REL);
}
API int dr_malloc(void** p, size_t n) {
  (void)err_word();
  return (int)hipMalloc(p, n);
}
API int dr_free(void* p) { return (int)hipFree(p); }
API int dr_host_alloc(void** p, size_t n) { return (int)hipHostMalloc(p, n, hipHostMallocDefault); }
API int dr_host_free(void* p) { return (int)hipHostFree(p); }
API int dr_h2d(void* d, const void* h, size_t n, hipStream_t st) {
  return (int)hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, st);
}
API int dr_d2h(void* h, const void* d, size_t n, hipStream_t st) {
  return (int)hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, st);
}
API int dr_d2d(void* d, const void* s, size_t n, hipStream_t st) {
  return (int)hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, st);
}

// Byte fill as a kernel: graph-capturable without memset nodes.
__global__ void k_fill(uint8_t* __restrict__ d, uint32_t v4, size_t n) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i + 16 <= n && (((uintptr_t)(d + i)) & 15) == 0) {
    *reinterpret_cast<uint4*>(d + i) = make_uint4(v4, v4, v4, v4);
  } else {
    for (size_t j = i; j < i + 16 && j < n; ++j) d[j] = (uint8_t)v4;
  }
}

API int dr_memset(void* d, int v, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  const uint32_t b = (uint32_t)(v & 0xff);
  const uint32_t v4 = b | (b << 8) | (b << 16) | (b << 24);
  // Unaligned heads are handled bytewise by the threads whose 16-byte window is unaligned.
  const size_t chunks = (n + 15) / 16;
  hipLaunchKernelGGL(k_fill, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, (uint8_t*)d, v4, n);
  return (int)hipGetLastError();
}

API int dr_stream_create(hipStream_t* s) {
  (void)err_word();  // set the error word up now, outside any graph capture
  return (int)hipStreamCreateWithFlags(s, hipStreamNonBlocking);
}
// A pending library error (left for dr_last_error to clear) is reported after the wait.
API int dr_stream_sync(hipStream_t s) {
  const int e = (int)hipStreamSynchronize(s);
  return e ? e : (int)err_pending();
}
API int dr_device_sync(void) { return (int)hipDeviceSynchronize(); }
API int dr_mem_info(size_t* free_b, size_t* total_b) { return (int)hipMemGetInfo(free_b, total_b); }

API int dr_graph_begin(hipStream_t s) { return (int)hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal); }
API int dr_graph_end(hipStream_t s, hipGraphExec_t* exec) {
  hipGraph_t g;
  hipError_t e = hipStreamEndCapture(s, &g);
  if (e != hipSuccess) return (int)e;
  e = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  return (int)e;
}
API int dr_graph_launch(hipGraphExec_t exec, hipStream_t s) { return (int)hipGraphLaunch(exec, s); }
API int dr_graph_destroy(hipGraphExec_t exec) { return (int)hipGraphExecDestroy(exec); }

// The engine creates a "BLAS handle" bound to its stream (src/engine.rs, Cublas); here it is
// just the stream for dr_gemm.
struct GemmHandle {
  hipStream_t st;
};
API int dr_cublas_create(void** h, hipStream_t s) {
  GemmHandle* g = new (std::nothrow) GemmHandle{s};
  if (!g) return (int)hipErrorOutOfMemory;
  *h = g;
  return 0;
}
API int dr_cublas_destroy(void* h) {
  delete static_cast<GemmHandle*>(h);
  return 0;
}
hipStream_t gemm_handle_stream(void* h) { return h ? static_cast<GemmHandle*>(h)->st : nullptr; }
