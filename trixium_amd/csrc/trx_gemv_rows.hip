// Multi-row exact ternary GEMV: one pass over a tensor's row packets against up to kRowsMax
// int8 activation vectors (model/bitexact.py:121-125 matvec_ternary_rows, the engine's
// multi-row mode). Every output row is the single-row engine matvec of its x (per-group exact
// sums, fp16 scale split, shift by e16 + B, int48 accumulate, >> R), bit for bit.
//
// Layout of the work: a block (16 waves) stages all n x rows in LDS (n * K bytes); a wave owns a
// weight row at a time. Its 64 lanes take 16 groups per pass, 4 lanes per 128-column group, lane
// q holding columns 32q .. 32q+31 as eight dwords of int8 weights in {-1, 0, 1}:
//   2-bit:  decoded from one 8-byte load;
//   trit5:  lane q decodes code bytes 7q .. 7q+6 (columns 35q .. 35q+34, clipped to the group's
//           26 bytes and 128 columns) into a per-wave LDS tile and reads its 32 columns back.
// Each x row costs two 16-byte LDS reads and eight v_dot4_i32_i8 per lane; a quad shuffle gives
// each group's exact sum, lane q = 0 shifts it into that row's int64 accumulator, and a wave
// reduction ends the weight row.

#include "trx_internal.h"

namespace trx {

int gemv_check(int kind, int M, int K);

constexpr int kRowsThreads = 1024;
constexpr int kRowsWaves = kRowsThreads / 64;
constexpr int kRowsMax = 8;
constexpr int kRowsTile = kRowsWaves * 16 * kGroup;   // decoded trit5 weights, 2 KiB per wave
constexpr int kRowsLds = 144 * 1024 - kRowsTile;     // staged x rows: n * K bytes

struct RowsParams {
  const uint8_t* W;
  const int8_t* x8;     // n rows of K int8, 16-byte aligned
  int32_t* y;           // n rows of M int32
  int32_t* status;
  int M, K, G, row_bytes, code_off, B, R;
};

template <int FMT, int NR>
__global__ __launch_bounds__(kRowsThreads) void gemv_rows_kernel(RowsParams p) {
  extern __shared__ __align__(16) int8_t xs[];
  constexpr bool T5 = (FMT == TRX_KIND_TERNARY5);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane >> 2, q = lane & 3;
  // Per wave: 16 groups of decoded trit5 weights (int8 in {-1, 0, 1}), after the staged x rows.
  int8_t* wd = xs + NR * p.K + wave * 16 * kGroup;

  const int n16 = NR * p.K / 16;
  for (int i = tid; i < n16; i += kRowsThreads) ((int4*)xs)[i] = ((const int4*)p.x8)[i];
  __syncthreads();

  for (int m = blockIdx.x * kRowsWaves + wave; m < p.M; m += gridDim.x * kRowsWaves) {
    const uint8_t* row = p.W + (size_t)m * p.row_bytes;
    const uint16_t* sc = (const uint16_t*)row;
    long long acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0;

    for (int g0 = 0; g0 < p.G; g0 += 16) {
      const int g = g0 + j;
      const bool active = g < p.G;
      // w[k]: this lane's columns 32q + 4k .. 32q + 4k + 3 as packed int8.
      int w[8];
      if (T5) {
        // Lane q decodes code bytes 7q .. 7q+6 (columns 35q + 5i + d) into the wave's tile,
        // then reads back its 32 aligned columns. The fence and wave barrier order the tile's
        // writes before the reads of other lanes, and the previous pass's reads before them.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (active) {
          const uint8_t* cb = row + p.code_off + (size_t)g * kTrit5GroupBytes;
          int8_t* wg = wd + j * kGroup;
#pragma unroll
          for (int i = 0; i < 7; ++i) {
            const int bi = 7 * q + i;
            if (bi < kTrit5GroupBytes) {
              unsigned t = cb[bi];
#pragma unroll
              for (int d = 0; d < 5; ++d) {
                const int col = 5 * bi + d;
                if (col < kGroup) wg[col] = (int8_t)((int)(t % 3u) - 1);
                t /= 3u;
              }
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (active) {
          const int4* src = (const int4*)(wd + j * kGroup + 32 * q);
          const int4 lo = src[0], hi = src[1];
          w[0] = lo.x; w[1] = lo.y; w[2] = lo.z; w[3] = lo.w;
          w[4] = hi.x; w[5] = hi.y; w[6] = hi.z; w[7] = hi.w;
        }
      } else if (active) {
        const uint64_t v = *(const uint64_t*)(row + p.code_off + (size_t)g * kBeat + 8 * q);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          uint32_t d = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            d |= (uint32_t)(uint8_t)(int8_t)((int)((v >> (8 * k + 2 * e)) & 3u) - 1) << (8 * e);
          w[k] = (int)d;
        }
      }
      int part[NR];
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        int s = 0;
        if (active) {
          const int4* xr = (const int4*)(xs + r * p.K + g * kGroup + 32 * q);
          const int4 lo = xr[0], hi = xr[1];
          s = __builtin_amdgcn_sdot4(w[0], lo.x, s, false);
          s = __builtin_amdgcn_sdot4(w[1], lo.y, s, false);
          s = __builtin_amdgcn_sdot4(w[2], lo.z, s, false);
          s = __builtin_amdgcn_sdot4(w[3], lo.w, s, false);
          s = __builtin_amdgcn_sdot4(w[4], hi.x, s, false);
          s = __builtin_amdgcn_sdot4(w[5], hi.y, s, false);
          s = __builtin_amdgcn_sdot4(w[6], hi.z, s, false);
          s = __builtin_amdgcn_sdot4(w[7], hi.w, s, false);
        }
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        part[r] = s;
      }
      if (active && q == 0) {
        int m11, e16;
        fp16_split(sc[g], m11, e16);
        const int sh = e16 + p.B;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const long long prod = (long long)part[r] * (long long)m11;
          long long c;
          if (sh >= 0) c = prod << sh;
          else c = (-sh >= 63) ? (prod < 0 ? -1 : 0) : (prod >> (-sh));
          acc[r] += c;
        }
      }
    }

#pragma unroll
    for (int r = 0; r < NR; ++r) {
      long long v = acc[r];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
      acc[r] = v;
    }
    if (lane == 0) {
      int bad = 0;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const long long v = acc[r];
        const long long res = v >> p.R;
        bad |= ((v >= (1LL << 47)) || (v <= -(1LL << 47))) ? 1 : 0;
        bad |= (res >= (1LL << 31) || res <= -(1LL << 31)) ? 2 : 0;
        p.y[(size_t)r * p.M + m] = (int32_t)res;
      }
      if (bad) atomicOr(p.status, bad);
    }
  }
}

static int rows_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    hipDeviceProp_t prop;
    n = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            ? prop.multiProcessorCount : 256;
  }
  return n;
}

template <int FMT, int NR>
static int launch_rows(const RowsParams& p, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    TRX_HIP(hipFuncSetAttribute((const void*)gemv_rows_kernel<FMT, NR>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, kRowsLds + kRowsTile));
    attr_set = true;
  }
  const int need = cdiv(p.M, kRowsWaves);
  const int nb = need < rows_cus() ? need : rows_cus();
  hipLaunchKernelGGL((gemv_rows_kernel<FMT, NR>), dim3(nb), dim3(kRowsThreads), NR * p.K + kRowsTile, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

template <int FMT>
static int dispatch_rows(const RowsParams& p, int n, hipStream_t s) {
  switch (n) {
    case 1: return launch_rows<FMT, 1>(p, s);
    case 2: return launch_rows<FMT, 2>(p, s);
    case 3: return launch_rows<FMT, 3>(p, s);
    case 4: return launch_rows<FMT, 4>(p, s);
    case 5: return launch_rows<FMT, 5>(p, s);
    case 6: return launch_rows<FMT, 6>(p, s);
    case 7: return launch_rows<FMT, 7>(p, s);
    default: return launch_rows<FMT, 8>(p, s);
  }
}

int gemv_exact(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int B, int R,
               int32_t* y, int32_t* status, hipStream_t s);
constexpr int kRowsSingleMax = 4;

int gemv_exact_rows(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int n, int B,
                    int R, int32_t* y, int32_t* status, hipStream_t s) {
  TRX_CHECK(rows && x8 && y && status, TRX_E_INVALID, "gemv_exact_rows: null argument");
  int rc = gemv_check(kind, M, K);
  if (rc) return rc;
  TRX_CHECK(n >= 1 && n <= kRowsMax, TRX_E_INVALID, "gemv_exact_rows: %d x rows (1..%d)", n, kRowsMax);
  TRX_CHECK((long long)n * K <= kRowsLds, TRX_E_INVALID,
            "gemv_exact_rows: %d x rows of K=%d exceed %d staged bytes", n, K, kRowsLds);
  TRX_CHECK(((uintptr_t)x8 & 15) == 0, TRX_E_INVALID, "gemv_exact_rows: x8 must be 16-byte aligned");
  TRX_CHECK(B >= -48 && B <= 48 && R >= 0 && R < 63, TRX_E_INVALID,
            "gemv_exact_rows: B=%d R=%d out of range", B, R);
  if (n <= kRowsSingleMax) {
    // Few rows: the single-row kernel once per row is faster than one multi-row pass (measured at
    // the 8B gate|up shape: 13.5 us a row against 34.5 us for a one-row pass, even at four rows).
    for (int r = 0; r < n; ++r)
      if ((rc = gemv_exact(rows, kind, M, K, x8 + (size_t)r * K, B, R, y + (size_t)r * M, status, s))) return rc;
    return TRX_OK;
  }
  RowGeom rg = row_geom(kind, K);
  RowsParams p = {};
  p.W = rows;
  p.x8 = x8;
  p.y = y;
  p.status = status;
  p.M = M;
  p.K = K;
  p.G = rg.G;
  p.row_bytes = rg.row_bytes;
  p.code_off = rg.code_off;
  p.B = B;
  p.R = R;
  if (kind == TRX_KIND_TERNARY5) return dispatch_rows<TRX_KIND_TERNARY5>(p, n, s);
  return dispatch_rows<TRX_KIND_TERNARY>(p, n, s);
}

}  // namespace trx

extern "C" __attribute__((visibility("default"))) int trx_gemv_ternary_exact_rows(
    const uint8_t* rows, int kind, int M, int K, const int8_t* x8_rows, int n_rows, int B, int R,
    int32_t* y, int32_t* status, trx_stream_t s) {
  return trx::gemv_exact_rows(rows, kind, M, K, x8_rows, n_rows, B, R, y, status, (hipStream_t)s);
}
