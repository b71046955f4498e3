// The firmware's activation quantizer and its quantized projection (the engine path of
// model/mirror.py:663-678, firmware/infer.c:144 infer_matvec_f):
//   e8 = frexp(max |x|) - 7 (0 for an all-zero x), x8 = clip(lroundf(x * 2^-e8), -127, 127) with
//   lroundf as model/mirror.py:34-35 evaluates it in float32 (floor(x + 0.5) for x >= 0,
//   ceil(x - 0.5) below), mantissas of the largest element in [64, 128);
//   y = float(W x8 through the engine's exact matvec, int32) * 2^(e8 + R - B).

#include "trx_internal.h"

namespace trx {

int gemv_exact(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int B, int R, int32_t* y,
               int32_t* status, hipStream_t s);

constexpr int kQuantThreads = 1024;

__global__ __launch_bounds__(kQuantThreads) void quantize_kernel(const float* x, int K, int8_t* x8, int* e8) {
  __shared__ float red[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float amax = 0.f;
  for (int i = tid; i < K; i += kQuantThreads) amax = fmaxf(amax, fabsf(x[i]));
  amax = wave_max(amax);
  if (lane == 0) red[w] = amax;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < kQuantThreads / 64; ++i) m = fmaxf(m, red[i]);
  int e = 0;
  if (m > 0.f) {
    int ex;
    (void)frexpf(m, &ex);
    e = ex - 7;
  }
  // 2^-e as a float32 (e in [-156, 121] for finite x; the product is exact where it is normal).
  const float sc = ldexpf(1.0f, -e);
  for (int i = tid; i < K; i += kQuantThreads) {
    const float v = x[i] * sc;
    const float r = v >= 0.f ? floorf(v + 0.5f) : ceilf(v - 0.5f);
    x8[i] = (int8_t)fminf(fmaxf(r, -127.f), 127.f);
  }
  if (tid == 0) *e8 = e;
}

__global__ void scale_i32_kernel(const int32_t* yi, const int* e8, int shift, float* y, int M) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  y[i] = (float)yi[i] * ldexpf(1.0f, *e8 + shift);
}

int quantize_f_pow2(const float* x, int K, int8_t* x8, int* e8, hipStream_t s) {
  TRX_CHECK(x && x8 && e8 && K >= 1, TRX_E_INVALID, "quantize: bad arguments");
  hipLaunchKernelGGL(quantize_kernel, dim3(1), dim3(kQuantThreads), 0, s, x, K, x8, e8);
  TRX_LAUNCHED();
  return TRX_OK;
}

int gemv_quantized(const uint8_t* rows, int kind, int M, int K, const float* x, int B, int R, float* y, void* work,
                   int32_t* status, hipStream_t s) {
  TRX_CHECK(rows && x && y && work && status, TRX_E_INVALID, "quantized GEMV: null argument");
  // Workspace: e8 (16 bytes), x8 (K bytes, 16-byte aligned), the int32 results (4 M bytes).
  uint8_t* w = (uint8_t*)work;
  int* e8 = (int*)w;
  int8_t* x8 = (int8_t*)(w + 16);
  int32_t* yi = (int32_t*)(w + 16 + (((size_t)K + 15) / 16) * 16);
  int rc;
  if ((rc = quantize_f_pow2(x, K, x8, e8, s))) return rc;
  if ((rc = gemv_exact(rows, kind, M, K, x8, B, R, yi, status, s))) return rc;
  hipLaunchKernelGGL(scale_i32_kernel, dim3(cdiv(M, 256)), dim3(256), 0, s, yi, e8, R - B, y, M);
  TRX_LAUNCHED();
  return TRX_OK;
}

size_t gemv_quantized_work_bytes(int M, int K) { return 16 + ((size_t)K + 15) / 16 * 16 + 4 * (size_t)M; }

}  // namespace trx

using namespace trx;

#define TRX_API extern "C" __attribute__((visibility("default")))

TRX_API int trx_quantize_f_pow2(const float* x, int K, int8_t* x8, int* e8, trx_stream_t s) {
  return quantize_f_pow2(x, K, x8, e8, (hipStream_t)s);
}

TRX_API int trx_gemv_quantized_geometry(int M, int K, size_t* workspace_bytes) {
  TRX_CHECK(workspace_bytes && M >= 1 && K >= 1, TRX_E_INVALID, "trx_gemv_quantized_geometry: bad arguments");
  *workspace_bytes = gemv_quantized_work_bytes(M, K);
  return TRX_OK;
}

TRX_API int trx_gemv_ternary_quantized(const uint8_t* rows, int kind, int M, int K, const float* x, int B, int R,
                                       float* y, void* workspace, int32_t* status, trx_stream_t s) {
  return gemv_quantized(rows, kind, M, K, x, B, R, y, workspace, status, (hipStream_t)s);
}
