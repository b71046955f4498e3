// The packed float GEMV for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops): trx_gemv_packed_f32 with its workspace (tile counters, the
// blocks' slice sums of x^2, split-K partial sums) in a fixed device array of this library
// instead of a caller's buffer. Each GPU holds its own copy of the array; its address on a
// device is looked up once, on that device's first call, and the counter region is cleared then
// by a fill kernel on the caller's stream (the GEMV leaves the counters zero after every call).
// Calls on one GPU share the array, so calls that overlap on one GPU race.

#include <mutex>

#include "trx_internal.h"
#include "trx_tgemv.h"

namespace trx {

constexpr size_t kScratchBytes = 24u << 20;   // counters + slice sums + up to ~23.4 MB of partial sums

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

__global__ void zero_words_kernel(uint32_t* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

// This device's copy of the scratch array (set up on the device's first call: address lookup,
// counters cleared on stream s).
static int scratch_of_device(void** out, size_t counter_bytes, hipStream_t s) {
  int dev = 0;
  TRX_HIP(hipGetDevice(&dev));
  TRX_CHECK(dev >= 0 && dev < kMaxDevices, TRX_E_INVALID, "no-alloc GEMV: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    TRX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    TRX_CHECK(p != nullptr, TRX_E_HIP, "no-alloc GEMV: scratch array has no device address");
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, s, (uint32_t*)p, counter_bytes / 4);
    TRX_LAUNCHED();
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TRX_OK;
}

int tgemv_f32_noalloc(const uint8_t* packed, int kind, int M, int K, const float* x, const float* norm_w, float eps,
                      float* y, int epi, const float* resid, hipStream_t s) {
  PackGeom g;
  int rc = pack_geom(g, kind, M, K);
  if (rc) return rc;
  TRX_CHECK(g.work_bytes <= kScratchBytes, TRX_E_INVALID,
            "no-alloc GEMV: %d x %d needs %zu bytes of workspace, the fixed array holds %zu", M, K, g.work_bytes,
            kScratchBytes);
  void* work = nullptr;
  if ((rc = scratch_of_device(&work, g.cnt_bytes, s))) return rc;
  return tgemv_f32(packed, kind, M, K, x, norm_w, eps, y, epi, resid, nullptr, work, s);
}

}  // namespace trx

extern "C" __attribute__((visibility("default"))) int trx_gemv_packed_f32_noalloc(
    const uint8_t* packed, int kind, int M, int K, const float* x, const float* norm_w, float eps, float* y,
    int epilogue, const float* resid, trx_stream_t s) {
  TRX_CHECK(epilogue == TRX_EPI_STORE || epilogue == TRX_EPI_RESID || epilogue == TRX_EPI_SWIGLU, TRX_E_INVALID,
            "trx_gemv_packed_f32_noalloc: unknown epilogue %d", epilogue);
  return trx::tgemv_f32_noalloc(packed, kind, M, K, x, norm_w, eps, y, epilogue, resid, (hipStream_t)s);
}
