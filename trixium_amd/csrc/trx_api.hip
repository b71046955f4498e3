// C ABI of libtrixium_hip: error reporting, device memory, streams, events, and the GEMV entry
// points (their kernels live in trx_gemv.hip).

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "trx_internal.h"
#include "trx_tgemv.h"

namespace trx {

static thread_local char g_err[1024];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

const char* get_error() { return g_err; }

int gemv_f32(const uint8_t* rows, int kind, int M, int K, const float* x, const float* norm_w,
             float eps, float* y, int epi, const float* resid, int swiglu_F,
             unsigned long long* amax_slot, hipStream_t s, const int* gate_pos, const int* gate_from);
int gemv_exact(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int B, int R,
               int32_t* y, int32_t* status, hipStream_t s);
int gemv_groupsums(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int32_t* gs,
                   hipStream_t s);
int gemv_set_variant(int v);

}  // namespace trx

using namespace trx;

#define TRX_API extern "C" __attribute__((visibility("default")))

TRX_API const char* trx_last_error(void) { return get_error(); }
TRX_API int trx_version(void) { return 1; }

TRX_API int trx_device_count(int* n) {
  TRX_CHECK(n, TRX_E_INVALID, "trx_device_count: null");
  TRX_HIP(hipGetDeviceCount(n));
  return TRX_OK;
}

TRX_API int trx_set_device(int dev) {
  TRX_HIP(hipSetDevice(dev));
  return TRX_OK;
}

TRX_API int trx_device_name(char* buf, int len) {
  TRX_CHECK(buf && len > 0, TRX_E_INVALID, "trx_device_name: bad buffer");
  int dev = 0;
  TRX_HIP(hipGetDevice(&dev));
  hipDeviceProp_t p;
  TRX_HIP(hipGetDeviceProperties(&p, dev));
  snprintf(buf, len, "%s %s cus=%d", p.name, p.gcnArchName, p.multiProcessorCount);
  return TRX_OK;
}

TRX_API int trx_malloc(void** ptr, size_t bytes) {
  TRX_CHECK(ptr, TRX_E_INVALID, "trx_malloc: null");
  *ptr = nullptr;
  hipError_t e = hipMalloc(ptr, bytes + 256);
  if (e != hipSuccess) {
    set_error("trx_malloc(%zu): %s", bytes, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? TRX_E_NOMEM : TRX_E_HIP;
  }
  return TRX_OK;
}

TRX_API int trx_free(void* ptr) {
  if (ptr) TRX_HIP(hipFree(ptr));
  return TRX_OK;
}

TRX_API int trx_memcpy_h2d(void* dst, const void* src, size_t bytes, trx_stream_t s) {
  TRX_CHECK(dst && src, TRX_E_INVALID, "trx_memcpy_h2d: null");
  TRX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_memcpy_d2h(void* dst, const void* src, size_t bytes, trx_stream_t s) {
  TRX_CHECK(dst && src, TRX_E_INVALID, "trx_memcpy_d2h: null");
  TRX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)s));
  TRX_HIP(hipStreamSynchronize((hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_memcpy_d2d(void* dst, const void* src, size_t bytes, trx_stream_t s) {
  TRX_CHECK(dst && src, TRX_E_INVALID, "trx_memcpy_d2d: null");
  TRX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_memset_d8(void* dst, int value, size_t bytes, trx_stream_t s) {
  TRX_CHECK(dst, TRX_E_INVALID, "trx_memset_d8: null");
  TRX_HIP(hipMemsetAsync(dst, value, bytes, (hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_stream_create(trx_stream_t* s) {
  TRX_CHECK(s, TRX_E_INVALID, "trx_stream_create: null");
  hipStream_t h;
  TRX_HIP(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
  *s = (trx_stream_t)h;
  return TRX_OK;
}

TRX_API int trx_stream_destroy(trx_stream_t s) {
  if (s) TRX_HIP(hipStreamDestroy((hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_stream_sync(trx_stream_t s) {
  TRX_HIP(hipStreamSynchronize((hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_event_create(void** ev) {
  TRX_CHECK(ev, TRX_E_INVALID, "trx_event_create: null");
  hipEvent_t e;
  TRX_HIP(hipEventCreate(&e));
  *ev = (void*)e;
  return TRX_OK;
}

TRX_API int trx_event_destroy(void* ev) {
  if (ev) TRX_HIP(hipEventDestroy((hipEvent_t)ev));
  return TRX_OK;
}

TRX_API int trx_event_record(void* ev, trx_stream_t s) {
  TRX_CHECK(ev, TRX_E_INVALID, "trx_event_record: null");
  TRX_HIP(hipEventRecord((hipEvent_t)ev, (hipStream_t)s));
  return TRX_OK;
}

TRX_API int trx_event_elapsed_ms(void* a, void* b, float* ms) {
  TRX_CHECK(a && b && ms, TRX_E_INVALID, "trx_event_elapsed_ms: null");
  TRX_HIP(hipEventSynchronize((hipEvent_t)b));
  TRX_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
  return TRX_OK;
}

TRX_API int trx_gemv_ternary_exact(const uint8_t* rows, int kind, int M, int K, const int8_t* x8,
                                   int B, int R, int32_t* y, int32_t* status, trx_stream_t s) {
  TRX_CHECK(rows, TRX_E_INVALID, "trx_gemv_ternary_exact: null rows");
  return gemv_exact(rows, kind, M, K, x8, B, R, y, status, (hipStream_t)s);
}

TRX_API int trx_gemv_ternary_groupsums(const uint8_t* rows, int kind, int M, int K,
                                       const int8_t* x8, int32_t* gs, trx_stream_t s) {
  TRX_CHECK(rows, TRX_E_INVALID, "trx_gemv_ternary_groupsums: null rows");
  return gemv_groupsums(rows, kind, M, K, x8, gs, (hipStream_t)s);
}

TRX_API int trx_gemv_ternary_f32(const uint8_t* rows, int kind, int M, int K, const float* x,
                                 const float* norm_w, float eps, float* y, int epilogue,
                                 const float* resid, trx_stream_t s) {
  TRX_CHECK(rows, TRX_E_INVALID, "trx_gemv_ternary_f32: null rows");
  TRX_CHECK(epilogue == TRX_EPI_STORE || epilogue == TRX_EPI_RESID || epilogue == TRX_EPI_SWIGLU,
            TRX_E_INVALID, "trx_gemv_ternary_f32: unknown epilogue %d", epilogue);
  return gemv_f32(rows, kind, M, K, x, norm_w, eps, y, epilogue, resid,
                  epilogue == TRX_EPI_SWIGLU ? M / 2 : 0, nullptr, (hipStream_t)s, nullptr, nullptr);
}

TRX_API int trx_gemv_set_variant(int variant) { return gemv_set_variant(variant); }

TRX_API int trx_pack_geometry(int kind, int M, int K, size_t* packed_bytes, size_t* workspace_bytes) {
  TRX_CHECK(packed_bytes && workspace_bytes, TRX_E_INVALID, "trx_pack_geometry: null argument");
  PackGeom g;
  int rc = pack_geom(g, kind, M, K);
  if (rc) return rc;
  *packed_bytes = g.bytes;
  *workspace_bytes = g.work_bytes;
  return TRX_OK;
}

TRX_API int trx_pack_ternary(const uint8_t* rows, int kind, int M, int K, int swiglu, uint8_t* packed,
                             trx_stream_t s) {
  return pack_ternary(rows, kind, M, K, swiglu, packed, (hipStream_t)s);
}

TRX_API int trx_pack_partials_geometry(int kind, int M, int K, int* S, int* rows_p, int* bps) {
  TRX_CHECK(S && rows_p && bps, TRX_E_INVALID, "trx_pack_partials_geometry: null argument");
  PackGeom g;
  int rc = pack_geom(g, kind, M, K);
  if (rc) return rc;
  *S = g.S;
  *rows_p = g.rows_p;
  *bps = g.bps;
  return TRX_OK;
}

TRX_API int trx_gemv_packed_parts_f32(const uint8_t* packed, int kind, int M, int K, const float* x,
                                      const float* norm_w, float eps, float* y, int epilogue,
                                      const float* resid, void* workspace, const trx_partial_sums* parts,
                                      trx_stream_t s) {
  TRX_CHECK(epilogue == TRX_EPI_STORE || epilogue == TRX_EPI_RESID || epilogue == TRX_EPI_SWIGLU,
            TRX_E_INVALID, "trx_gemv_packed_parts_f32: unknown epilogue %d", epilogue);
  PartialSums ps = {};
  if (parts) {
    ps.out = parts->out;
    ps.out_ss = parts->out_ss;
    ps.in = parts->in;
    ps.in_ss = parts->in_ss;
    ps.resid = parts->resid;
    ps.S = parts->S;
    ps.rows_p = parts->rows_p;
    ps.F = parts->F;
    ps.in_K = parts->in_K;
    ps.act = parts->act;
  }
  return tgemv_f32(packed, kind, M, K, x, norm_w, eps, y, epilogue, resid, nullptr, workspace, (hipStream_t)s,
                   nullptr, nullptr, nullptr, parts ? &ps : nullptr);
}

TRX_API int trx_pack_batched_geometry(int kind, int M, int K, int n_mat, size_t* workspace_bytes) {
  TRX_CHECK(workspace_bytes, TRX_E_INVALID, "trx_pack_batched_geometry: null argument");
  PackGeom g;
  return tgemv_batched_geom(kind, M, K, n_mat, g, workspace_bytes);
}

TRX_API int trx_gemv_packed_batched_f32(const uint8_t* packed, size_t mat_stride, int n_mat, int n_copies, int kind,
                                        int M, int K, const float* x, int x_stride, float* y, int y_stride,
                                        void* workspace, trx_stream_t s) {
  return tgemv_f32_batched(packed, mat_stride, n_mat, n_copies, kind, M, K, x, x_stride, y, y_stride,
                           (float*)workspace, (hipStream_t)s);
}

TRX_API int trx_gemv_packed_f32(const uint8_t* packed, int kind, int M, int K, const float* x,
                                const float* norm_w, float eps, float* y, int epilogue,
                                const float* resid, void* workspace, trx_stream_t s) {
  TRX_CHECK(epilogue == TRX_EPI_STORE || epilogue == TRX_EPI_RESID || epilogue == TRX_EPI_SWIGLU,
            TRX_E_INVALID, "trx_gemv_packed_f32: unknown epilogue %d", epilogue);
  return tgemv_f32(packed, kind, M, K, x, norm_w, eps, y, epilogue, resid, nullptr, workspace,
                   (hipStream_t)s);
}
