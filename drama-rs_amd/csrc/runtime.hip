// Runtime wrappers of the C ABI (reference: kernels/drama.cu:1995-2044, src/ffi.rs:13-31).
// Thin HIP calls; the engine never needs HIP headers.
#include "common.hpp"

#include <new>

using namespace drm;

API const char* dr_error_string(int e) {
  if (e == -1) return "unsupported shape";
  return hipGetErrorString((hipError_t)e);
}
API int dr_last_error(void) { return (int)hipGetLastError(); }
API int dr_malloc(void** p, size_t n) { return (int)hipMalloc(p, n); }
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

API int dr_stream_create(hipStream_t* s) { return (int)hipStreamCreateWithFlags(s, hipStreamNonBlocking); }
API int dr_stream_sync(hipStream_t s) { return (int)hipStreamSynchronize(s); }
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
hipStream_t gemm_handle_stream(void* h) { return h ? static_cast<GemmHandle*>(h)->st : nullptr; }
