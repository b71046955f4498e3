// Ternary GEMV kernels and their host-side launch (the device code is in trx_gemv_dev.h).

#include "trx_gemv_dev.h"

namespace trx {

template <int FMT, int MODE, int R, int NB, bool SW>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvParams p) {
  // The decode table is static LDS (its base folds into the ds_read offsets); the x layout and
  // staging buffers are dynamic LDS sized by K.
  __shared__ __align__(16) uint64_t lut64[kLutBytes / 8];
  extern __shared__ __align__(16) uint8_t smem[];
  if (p.gate_pos && *p.gate_pos < *p.gate_from) return;        // uniform over the grid
  gemv_body<FMT, MODE, R, NB, SW>(p, (uint8_t*)lut64, smem, blockIdx.x, gridDim.x);
}

// Host side ------------------------------------------------------------------------------------

static int g_num_cus = 0;
static int num_cus() {
  if (!g_num_cus) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 256;
    g_num_cus = prop.multiProcessorCount;
  }
  return g_num_cus;
}

template <int FMT, int MODE, int R, int NB, bool SW>
static int launch_r(GemvParams& p, hipStream_t s) {
  constexpr int kWaves = kGemvThreads / 64;
  static bool attr_set = false;
  if (!attr_set) {
    TRX_HIP(hipFuncSetAttribute((const void*)gemv_kernel<FMT, MODE, R, NB, SW>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, kDynLds));
    attr_set = true;
  }
  p.n_batches = SW ? cdiv(p.n_out, R / 2) : cdiv(p.n_out, R);
  const int per_block = kWaves * (64 / p.LPR);
  const int need = cdiv(p.n_batches, per_block);
  const int nb = need < num_cus() ? need : num_cus();
  hipLaunchKernelGGL((gemv_kernel<FMT, MODE, R, NB, SW>), dim3(nb > 0 ? nb : 1), dim3(kGemvThreads),
                     lds_bytes(p.K, p.G), s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

// Variant selection. g_variant (trx_gemv_set_variant, for tuning) forces rows per item
// (1: R=4, 2: R=2, 3: R=1; SwiGLU takes R=2 for 3); 0 picks the R that minimises
// (grid rounds rounded up) x R, the time of the slowest row group, preferring the larger R.
static int g_variant = 0;

static int pick_rows(const GemvParams& p, bool sw) {
  const int per_block = (kGemvThreads / 64) * (64 / p.LPR);
  const long long slots = (long long)num_cus() * per_block;
  int best_r = sw ? 2 : 1;
  long long best_cost = -1;
  for (int r : {4, 2, 1}) {
    if (sw && r < 2) continue;
    const long long nbat = sw ? cdiv(p.n_out, r / 2) : cdiv(p.n_out, r);
    const long long cost = ((nbat + slots - 1) / slots) * r;
    if (best_cost < 0 || cost < best_cost) { best_cost = cost; best_r = r; }
  }
  return best_r;
}

template <int FMT, int MODE>
static int launch(GemvParams& p, hipStream_t s) {
  const bool sw = (p.epi == TRX_EPI_SWIGLU);
  int r = pick_rows(p, sw);
  if (g_variant == 1) r = 4;
  if (g_variant == 2) r = 2;
  if (g_variant == 3) r = sw ? 2 : 1;
  if (MODE == MODE_F32 && sw) {
    if (r == 4) return launch_r<FMT, MODE, 4, 2, true>(p, s);
    return launch_r<FMT, MODE, 2, 4, true>(p, s);
  }
  if (r == 4) return launch_r<FMT, MODE, 4, 2, false>(p, s);
  if (r == 2) return launch_r<FMT, MODE, 2, 4, false>(p, s);
  return launch_r<FMT, MODE, 1, 6, false>(p, s);
}

int gemv_set_variant(int v) {
  TRX_CHECK(v >= 0 && v <= 3, TRX_E_INVALID, "gemv variant %d", v);
  g_variant = v;
  return TRX_OK;
}

int gemv_check(int kind, int M, int K) {
  TRX_CHECK(kind == TRX_KIND_TERNARY || kind == TRX_KIND_TERNARY5, TRX_E_INVALID,
            "gemv: kind %d is not a ternary kind", kind);
  TRX_CHECK(M > 0 && K > 0 && (K % kGroup) == 0, TRX_E_INVALID,
            "gemv: M=%d K=%d (K must be a positive multiple of 128)", M, K);
  TRX_CHECK(lds_bytes(K, K / kGroup) <= kDynLds && K <= kMaxXRounds * kGemvThreads * 8, TRX_E_INVALID,
            "gemv: K=%d exceeds the LDS budget", K);
  RowGeom rg = row_geom(kind, K);
  TRX_CHECK((unsigned long long)M * rg.row_bytes < 0xFFFF0000ull, TRX_E_INVALID,
            "gemv: tensor of %d rows x %d bytes exceeds 4 GiB", M, rg.row_bytes);
  return TRX_OK;
}

static void fill_geom(GemvParams& p, const uint8_t* rows, int kind, int M, int K) {
  RowGeom rg = row_geom(kind, K);
  p.W = rows;
  p.M = M;
  p.K = K;
  p.G = rg.G;
  p.row_bytes = rg.row_bytes;
  p.code_off = rg.code_off;
  // The last trit5 group of a row may be read 2 bytes past its end: the tensor is followed by a
  // readable 32-byte tail (trx_malloc and the model arena guarantee it).
  p.w_bytes = (uint32_t)((unsigned long long)M * rg.row_bytes + 32);
  p.LPR = pick_lpr(2 * rg.G);
  p.NSLOT = 2 * rg.G / p.LPR;
}

void fill_geom_public(GemvParams& p, const uint8_t* rows, int kind, int M, int K) { fill_geom(p, rows, kind, M, K); }

int gemv_f32(const uint8_t* rows, int kind, int M, int K, const float* x, const float* norm_w,
             float eps, float* y, int epi, const float* resid, int swiglu_F,
             unsigned long long* amax_slot, hipStream_t s, const int* gate_pos, const int* gate_from) {
  int rc = gemv_check(kind, M, K);
  if (rc) return rc;
  TRX_CHECK(x && y, TRX_E_INVALID, "gemv: null x or y");
  TRX_CHECK(((uintptr_t)x & 15) == 0 && (!norm_w || ((uintptr_t)norm_w & 15) == 0), TRX_E_INVALID,
            "gemv: x and the norm gain must be 16-byte aligned");
  TRX_CHECK(epi != TRX_EPI_RESID || resid, TRX_E_INVALID, "gemv: residual epilogue without a residual");
  GemvParams p = {};
  fill_geom(p, rows, kind, M, K);
  p.x = x;
  p.norm_w = norm_w;
  p.eps = eps;
  p.y = y;
  p.epi = epi;
  p.resid = resid;
  p.amax_slot = amax_slot;
  p.gate_pos = gate_pos;
  p.gate_from = gate_from;
  if (epi == TRX_EPI_SWIGLU) {
    TRX_CHECK(swiglu_F > 0 && 2 * swiglu_F == M, TRX_E_INVALID, "gemv: SwiGLU needs M == 2F");
    p.swiglu_F = swiglu_F;
    p.n_out = swiglu_F;
  } else {
    p.n_out = M;
  }
  if (kind == TRX_KIND_TERNARY5) return launch<TRX_KIND_TERNARY5, MODE_F32>(p, s);
  return launch<TRX_KIND_TERNARY, MODE_F32>(p, s);
}

int gemv_exact(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int B, int R,
               int32_t* y, int32_t* status, hipStream_t s) {
  int rc = gemv_check(kind, M, K);
  if (rc) return rc;
  TRX_CHECK(x8 && y && status, TRX_E_INVALID, "gemv_exact: null argument");
  TRX_CHECK(B >= -48 && B <= 48 && R >= 0 && R < 63, TRX_E_INVALID, "gemv_exact: B=%d R=%d out of range", B, R);
  GemvParams p = {};
  fill_geom(p, rows, kind, M, K);
  p.x8 = x8;
  p.yi = y;
  p.B = B;
  p.R = R;
  p.status = status;
  p.epi = TRX_EPI_STORE;
  p.n_out = M;
  if (kind == TRX_KIND_TERNARY5) return launch<TRX_KIND_TERNARY5, MODE_EXACT>(p, s);
  return launch<TRX_KIND_TERNARY, MODE_EXACT>(p, s);
}

int gemv_groupsums(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int32_t* gs,
                   hipStream_t s) {
  int rc = gemv_check(kind, M, K);
  if (rc) return rc;
  TRX_CHECK(x8 && gs, TRX_E_INVALID, "gemv_groupsums: null argument");
  GemvParams p = {};
  fill_geom(p, rows, kind, M, K);
  p.x8 = x8;
  p.yi = gs;
  p.epi = TRX_EPI_STORE;
  p.n_out = M;
  if (kind == TRX_KIND_TERNARY5) return launch<TRX_KIND_TERNARY5, MODE_GSUM>(p, s);
  return launch<TRX_KIND_TERNARY, MODE_GSUM>(p, s);
}

}  // namespace trx
