// Measurement helpers with no counterpart in the reference: capture of a caller's stream work
// into a hipGraph (so a benchmark can time kernels as the decoder's graph replays them), and two
// probe kernels whose timings the benchmark reports beside the decode: a plain streaming read of
// device memory (the practical read ceiling every HBM-bound kernel here is held to) and an empty
// kernel (the fixed cost of one dependent graph node or stream launch).

#include "trx_internal.h"

namespace trx {

// Each thread reads 16-byte vectors grid-stride (non-temporal: the data is used once) and keeps
// a sum so the loads are not dropped; one value per block is stored.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(1024) void stream_read_kernel(const u32x4* __restrict__ p, size_t n, float* out) {
  __shared__ float red[16];
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  const float v = (float)(acc & 0xFFFF);
  const float t = block_sum(v, red);
  if (threadIdx.x == 0) out[blockIdx.x] = t;
}

__global__ void empty_kernel() {}

}  // namespace trx

using namespace trx;

#define TRX_API extern "C" __attribute__((visibility("default")))

TRX_API int trx_graph_begin(trx_stream_t s) {
  TRX_CHECK(s, TRX_E_INVALID, "trx_graph_begin: capture needs a created stream, not the default one");
  TRX_HIP(hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal));
  return TRX_OK;
}

TRX_API int trx_graph_end(trx_stream_t s, void** exec) {
  TRX_CHECK(s && exec, TRX_E_INVALID, "trx_graph_end: null argument");
  hipGraph_t g = nullptr;
  TRX_HIP(hipStreamEndCapture((hipStream_t)s, &g));
  hipGraphExec_t e = nullptr;
  const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
  const hipError_t derr = hipGraphDestroy(g);
  TRX_CHECK(derr == hipSuccess || err != hipSuccess, TRX_E_HIP, "trx_graph_end: destroy: %s", hipGetErrorString(derr));
  TRX_CHECK(err == hipSuccess, TRX_E_HIP, "trx_graph_end: instantiate: %s", hipGetErrorString(err));
  *exec = (void*)e;
  return TRX_OK;
}

TRX_API int trx_graph_launch(void* exec, trx_stream_t s) {
  TRX_CHECK(exec, TRX_E_INVALID, "trx_graph_launch: null graph");
  TRX_HIP(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_graph_destroy(void* exec) {
  if (exec) TRX_HIP(hipGraphExecDestroy((hipGraphExec_t)exec));
  return TRX_OK;
}

TRX_API int trx_probe_stream_read(const void* buf, size_t bytes, float* out, int blocks, int threads,
                                  trx_stream_t s) {
  TRX_CHECK(buf && out && bytes >= 16 && bytes % 16 == 0 && blocks >= 1 && threads >= 64 && threads <= 1024 &&
                threads % 64 == 0,
            TRX_E_INVALID, "trx_probe_stream_read: bad arguments");
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)s, (const u32x4*)buf,
                     bytes / 16, out);
  TRX_LAUNCHED();
  return TRX_OK;
}

TRX_API int trx_probe_empty(trx_stream_t s) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, (hipStream_t)s);
  TRX_LAUNCHED();
  return TRX_OK;
}
