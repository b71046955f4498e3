// Internal helpers shared by the HIP sources of libtrixium_hip (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/trixium.h"

namespace trx {

// Last error, per host thread. Entry points return TRX_E_* and leave a message here.
void set_error(const char* fmt, ...);
const char* get_error();

#define TRX_HIP(call)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (call);                                                             \
    if (e_ != hipSuccess) {                                                             \
      ::trx::set_error("%s:%d: %s failed: %s", __FILE__, __LINE__, #call,               \
                       hipGetErrorString(e_));                                          \
      return TRX_E_HIP;                                                                 \
    }                                                                                   \
  } while (0)

#define TRX_CHECK(cond, code, ...)                                                      \
  do {                                                                                  \
    if (!(cond)) {                                                                      \
      ::trx::set_error(__VA_ARGS__);                                                    \
      return (code);                                                                    \
    }                                                                                   \
  } while (0)

// Launch check: a launch error is reported by hipGetLastError right after the launch.
#define TRX_LAUNCHED()                                                                  \
  do {                                                                                  \
    hipError_t e_ = hipGetLastError();                                                  \
    if (e_ != hipSuccess) {                                                             \
      ::trx::set_error("%s:%d: kernel launch failed: %s", __FILE__, __LINE__,           \
                       hipGetErrorString(e_));                                          \
      return TRX_E_HIP;                                                                 \
    }                                                                                   \
  } while (0)

constexpr int kBeat = 32;
constexpr int kGroup = 128;
constexpr int kTrit5GroupBytes = 26;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // gfx9-family raw buffer resource

// Geometry of a row-packet tensor (rows back to back, one channel).
struct RowGeom {
  int K;          // columns
  int G;          // 128-groups per row
  int row_bytes;  // bytes per row packet
  int code_off;   // bytes of fp16 scales before the codes (whole beats)
};

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

inline RowGeom row_geom(int kind, int K) {
  RowGeom g;
  g.K = K;
  g.G = K / kGroup;
  g.code_off = kBeat * cdiv(g.G, 16);
  int code_bytes = (kind == TRX_KIND_TERNARY5) ? kBeat * cdiv(kTrit5GroupBytes * g.G, kBeat)
                                                : kBeat * g.G;
  g.row_bytes = g.code_off + code_bytes;
  return g;
}

// Device helpers ------------------------------------------------------------------------------

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           (int)kRsrcWord3);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Cross-lane steps on the DPP path (no LDS round trip), within each row of 16 lanes:
// quad_perm [1,0,3,2] and [2,3,0,1] pair lanes l ^ 1 and l ^ 2, row_half_mirror pairs l and
// 7 - l (within 8), row_mirror pairs l and 15 - l. After the four steps every lane of a row holds
// the row's sum (or maximum).
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140;

// Matrix-core operand and accumulator types (v_mfma_f32_32x32x16_f16).
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  return v;
}
__device__ __forceinline__ int row16_sum_i(int v) {
  v += dpp_i<kDppQuadXor1>(v);
  v += dpp_i<kDppQuadXor2>(v);
  v += dpp_i<kDppRowHalfMirror>(v);
  v += dpp_i<kDppRowMirror>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  return v;
}
// Whole-wave sum through the rows and four lane reads (uniform result; all lanes active).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = row16_sum(v);
  const int b = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
}

// Block-wide sum; `red` is >= 16 floats of shared memory. All threads get the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_sum_dpp(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// A no-op in place of a grid barrier (standalone kernels).
struct NoWait {
  __device__ void operator()() const {}
};

// Loads and stores of vectors that other blocks of the same launch write or read: agent-scope
// (cross-XCD coherent) relaxed atomics when C, plain accesses otherwise.
template <bool C>
__device__ __forceinline__ float ld_vec(const float* p) {
  if (C) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}
template <bool C>
__device__ __forceinline__ void st_vec(float* p, float v) {
  if (C) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

// Float -> ordered unsigned (monotonic), for the packed argmax.
__device__ __forceinline__ uint32_t ordered_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Exact fp16 -> (m11, e16): value = m11 * 2^e16.
__device__ __forceinline__ void fp16_split(uint16_t bits, int& m11, int& e16) {
  int E = (bits >> 10) & 0x1F, frac = bits & 0x3FF;
  int mag = E ? (frac | 0x400) : frac;
  m11 = (bits & 0x8000) ? -mag : mag;
  e16 = E ? E - 25 : -24;
}

}  // namespace trx
