// Ternary GEMV for gfx950: y = W x over BONS row packets (2-bit or trit5 codes, one fp16 scale
// per 128-group), the hot operation of the batch-1 decode loop.
//
// Numerics (the engine contract of model/bitexact.py:101-119, float form of fastref.py:119-125):
//   per row m and group g:  S[m,g] = sum_{j in g} (code - 1) * x_j     (exact integers)
//   float mode:  x is quantised once per block to int16 per 128-group, x_j ~= q_j * sigma_g;
//                y[m] = sum_g scale[m,g] * sigma_g * S[m,g]            (fp32)
//   exact mode:  x is the caller's int8 vector; y[m] = (sum_g (S*m11) << (e16+B)) >> R  (int32)
//   group sums:  gs[m,g] = S[m,g]
//
// Mapping. A lane owns one 128-group at a time; LPR lanes (power of two dividing G, <= 64)
// cover LPR groups of R rows, and step through the G/LPR group slots of those rows. The x
// values of a group are held in 65 registers in a "dot-ready" form built once per block in
// LDS, and reused across the R rows. No MFMA: the path is a bandwidth-bound GEMV.
//
// Decode. trit5: every code byte b is looked up in an LDS table giving its five base-3 digits
// as four byte lanes (d0..d3, fed to v_dot4 against the int8 planes of x) plus d4 (fed to
// v_dot2 against int16 x). 2-bit: every code byte gives its four 2-bit codes as byte lanes.
// The table is replicated so that the 64 lanes of a wave hit distinct LDS banks; the entry
// address (b << 8 | lane copy) is formed by one v_perm_b32. Since sum (code-1)x =
// sum code*x - sum x, codes are used as unsigned digits and the group's sum of x is
// subtracted once per row.

#include "trx_internal.h"

namespace trx {

enum { MODE_F32 = 0, MODE_EXACT = 1, MODE_GSUM = 2 };

constexpr int kThreads = 512;
constexpr int kLutBytes = 65536;    // 256 entries x 256 bytes
constexpr int kXStride = 68;        // dwords per group in the dot-ready layout (65 used)
constexpr int kXDwords5 = 65;       // trit5: 26 x (hi, lo) + 13 d4 pairs
constexpr int kXDwords2 = 64;       // 2-bit: 32 x (hi, lo)

struct GemvParams {
  const uint8_t* W;
  uint32_t w_bytes;       // bytes addressable from W (bounds of the buffer loads)
  int M;                  // physical rows
  int K, G, row_bytes, code_off;
  int LPR, NSLOT;
  int n_batches;          // batches of R logical rows
  int n_out;              // logical outputs
  int epi;                // TRX_EPI_*
  int swiglu_F;           // SWIGLU: rows [0,F) gate, [F,2F) up
  const float* x;         // float input
  const float* norm_w;    // RMSNorm gain (nullptr: no norm)
  float eps;
  const int8_t* x8;       // int8 input (exact / group sums)
  float* y;
  const float* resid;
  int32_t* yi;            // exact result / group sums
  int B, R;
  int32_t* status;
  unsigned long long* amax_slot;  // argmax epilogue: packed (ordered value, ~index)
};

__device__ __forceinline__ uint32_t trit5_entry_lo(int b) {
  uint32_t v = 0;
  for (int k = 0; k < 4; ++k) { v |= (uint32_t)(b % 3) << (8 * k); b /= 3; }
  return v;
}
__device__ __forceinline__ uint32_t trit5_entry_hi(int b) {
  for (int k = 0; k < 4; ++k) b /= 3;
  return (uint32_t)(b % 3);
}
__device__ __forceinline__ uint32_t code2_entry(int b) {
  uint32_t v = 0;
  for (int k = 0; k < 4; ++k) v |= (uint32_t)((b >> (2 * k)) & 3) << (8 * k);
  return v;
}

// Float -> ordered unsigned (monotonic), for the packed argmax.
__device__ __forceinline__ uint32_t ordered_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int FMT, int MODE, int R>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
  // The decode table is static LDS (its base folds into the ds_read offsets); the x layout and
  // staging buffers are dynamic LDS sized by K.
  __shared__ __align__(16) uint64_t lut64[kLutBytes / 8];
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* lut = (uint8_t*)lut64;
  uint32_t* xl = (uint32_t*)smem;                              // G * kXStride dwords
  int16_t* stage = (int16_t*)(xl + p.G * kXStride);            // K int16
  float* gsig = (float*)(stage + p.K);                         // G: sigma_g
  int32_t* gsum = (int32_t*)(gsig + p.G);                      // G: sum of q over the group
  float* red = (float*)(gsum + p.G);                           // 16

  const int tid = threadIdx.x;
  constexpr bool T5 = (FMT == TRX_KIND_TERNARY5);
  constexpr int NPL = (MODE == MODE_F32) ? 2 : 1;              // int8 planes of x

  // Decode table: 256 entries at a 256-byte stride, lane copies inside an entry.
  if (T5) {
    uint64_t* l64 = (uint64_t*)lut;
    // Copies 0..15 carry d4 in the low half of the high word (even code bytes), copies
    // 16..31 in the high half (odd code bytes), matching the d4 pairs of the x layout.
    for (int i = tid; i < 256 * 32; i += kThreads) {
      int b = i >> 5;
      uint32_t hi = trit5_entry_hi(b) << ((i & 16) ? 16 : 0);
      l64[i] = (uint64_t)trit5_entry_lo(b) | ((uint64_t)hi << 32);
    }
  } else {
    uint32_t* l32 = (uint32_t*)lut;
    for (int i = tid; i < 256 * 64; i += kThreads) l32[i] = code2_entry(i >> 6);
  }

  // x -> int16 per group (float mode) or int8 copy (exact modes), staged in LDS.
  if (MODE == MODE_F32) {
    float rinv = 1.0f;
    if (p.norm_w) {
      float ss = 0.f;
      for (int c = tid * 4; c < p.K; c += kThreads * 4) {
        float4 v = *(const float4*)(p.x + c);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
      ss = block_sum(ss, red);
      rinv = 1.0f / sqrtf(ss / (float)p.K + p.eps);
    }
    // 16 threads per group, 8 columns each.
    for (int c0 = tid * 8; c0 < ((p.K + kThreads * 8 - 1) / (kThreads * 8)) * kThreads * 8; c0 += kThreads * 8) {
      bool live = c0 < p.K;
      float v[8];
      float am = 0.f;
      if (live) {
        float4 a = *(const float4*)(p.x + c0), b = *(const float4*)(p.x + c0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        if (p.norm_w) {
          float4 wa = *(const float4*)(p.norm_w + c0), wb = *(const float4*)(p.norm_w + c0 + 4);
          float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
          for (int k = 0; k < 8; ++k) v[k] = v[k] * rinv * w[k];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) am = fmaxf(am, fabsf(v[k]));
      }
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
      float inv = am > 0.f ? 32767.0f / am : 0.f;
      int s = 0;
      if (live) {
        int q[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) { q[k] = (int)rintf(v[k] * inv); s += q[k]; }
        uint4 pk;
        pk.x = (uint32_t)(uint16_t)q[0] | ((uint32_t)(uint16_t)q[1] << 16);
        pk.y = (uint32_t)(uint16_t)q[2] | ((uint32_t)(uint16_t)q[3] << 16);
        pk.z = (uint32_t)(uint16_t)q[4] | ((uint32_t)(uint16_t)q[5] << 16);
        pk.w = (uint32_t)(uint16_t)q[6] | ((uint32_t)(uint16_t)q[7] << 16);
        *(uint4*)(stage + c0) = pk;
      }
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
      if (live && (tid & 15) == 0) {
        gsig[c0 >> 7] = am / 32767.0f;
        gsum[c0 >> 7] = s;
      }
    }
  } else {
    for (int c = tid; c < p.K; c += kThreads) stage[c] = (int16_t)p.x8[c];
    __syncthreads();
    for (int g = tid; g < p.G; g += kThreads) {
      int s = 0;
      for (int j = 0; j < kGroup; ++j) s += stage[g * kGroup + j];
      gsum[g] = s;
    }
  }
  __syncthreads();

  // Dot-ready layout of every group.
  {
    const int per = T5 ? kXDwords5 : kXDwords2;
    for (int i = tid; i < p.G * per; i += kThreads) {
      int g = i / per, j = i - g * per;
      const int16_t* xs = stage + g * kGroup;
      uint32_t v = 0;
      if (j < (T5 ? 52 : 64)) {
        int byte = j >> 1, plane = j & 1;
        int c0 = T5 ? 5 * byte : 4 * byte;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          int c = c0 + k;
          int q = (c < kGroup) ? xs[c] : 0;
          uint32_t b8 = (NPL == 2) ? (plane == 0 ? (uint32_t)((q >> 8) & 0xFF) : (uint32_t)(q & 0xFF))
                                   : (plane == 0 ? (uint32_t)(q & 0xFF) : 0u);
          v |= b8 << (8 * k);
        }
      } else {
        int pr = j - 52;
        int ca = 5 * (2 * pr) + 4, cb = 5 * (2 * pr + 1) + 4;
        int qa = ca < kGroup ? xs[ca] : 0, qb = cb < kGroup ? xs[cb] : 0;
        v = (uint32_t)(uint16_t)qa | ((uint32_t)(uint16_t)qb << 16);
      }
      xl[g * kXStride + j] = v;
    }
  }
  __syncthreads();

  // Main loop.
  const int lane = tid & 63, wave = tid >> 6;
  const int LPR = p.LPR;
  const int rg = lane / LPR, lg = lane - rg * LPR;
  const int RG = 64 / LPR;
  const int slot = (blockIdx.x * (kThreads / 64) + wave) * RG + rg;
  const int nslots = gridDim.x * (kThreads / 64) * RG;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.W, p.w_bytes);
  // v_perm sources: byte 0 of the result comes from the lane-copy word (selector 0), byte 1
  // from code byte k of the code word (selector 4 + k), bytes 2..3 are zero (selector 0x0c).
  const uint32_t lc_even = T5 ? (uint32_t)((lane & 15) << 3) : (uint32_t)(lane << 2);
  const uint32_t lc_odd = T5 ? (uint32_t)(((lane & 15) | 16) << 3) : lc_even;

  for (int bt = slot; bt < p.n_batches; bt += nslots) {
    int prow[R];
    bool pok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int lr = bt * R + r;
      if (p.epi == TRX_EPI_SWIGLU) {
        int half = R / 2;
        int o = bt * half + (r % half);
        pok[r] = o < p.n_out;
        prow[r] = (r < half) ? o : p.swiglu_F + o;
      } else {
        pok[r] = lr < p.n_out;
        prow[r] = lr;
      }
    }
    float facc[R];
    long long iacc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) { facc[r] = 0.f; iacc[r] = 0; }

    for (int sl = 0; sl < p.NSLOT; ++sl) {
      const int g = sl * LPR + lg;
      // x registers for group g.
      uint32_t xr[T5 ? kXDwords5 : kXDwords2];
      {
        const uint4* src = (const uint4*)(xl + g * kXStride);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          uint4 t = src[i];
          xr[4 * i] = t.x; xr[4 * i + 1] = t.y; xr[4 * i + 2] = t.z; xr[4 * i + 3] = t.w;
        }
        if (T5) xr[64] = xl[g * kXStride + 64];
      }
      const float sig = (MODE == MODE_F32) ? gsig[g] : 0.f;
      const int gsx = gsum[g];
      // Codes (and scales) of the R rows for this group.
      uint32_t cd[R][T5 ? 7 : 8];
      uint32_t sc[R];
      const int shift = T5 ? ((kTrit5GroupBytes * g) & 3) : 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint32_t rowoff = (uint32_t)prow[r] * (uint32_t)p.row_bytes;
        if (!pok[r]) rowoff = p.w_bytes;                      // out of range: loads read 0
        if (T5) {
          // 28 bytes from the dword-aligned start of the group; the last dword is read as two
          // halves so that no access of an in-range row crosses the end of the tensor.
          uint32_t off = rowoff + p.code_off + ((kTrit5GroupBytes * g) & ~3);
          auto a = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
          auto b = __builtin_amdgcn_raw_buffer_load_b64(rs, off + 16, 0, 0);
          uint32_t c0 = __builtin_amdgcn_raw_buffer_load_b16(rs, off + 24, 0, 0);
          uint32_t c1 = __builtin_amdgcn_raw_buffer_load_b16(rs, off + 26, 0, 0);
          cd[r][0] = a[0]; cd[r][1] = a[1]; cd[r][2] = a[2]; cd[r][3] = a[3];
          cd[r][4] = b[0]; cd[r][5] = b[1]; cd[r][6] = c0 | (c1 << 16);
        } else {
          uint32_t off = rowoff + p.code_off + 32 * g;
          auto a = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
          auto b = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0);
          cd[r][0] = a[0]; cd[r][1] = a[1]; cd[r][2] = a[2]; cd[r][3] = a[3];
          cd[r][4] = b[0]; cd[r][5] = b[1]; cd[r][6] = b[2]; cd[r][7] = b[3];
        }
        sc[r] = __builtin_amdgcn_raw_buffer_load_b16(rs, rowoff + 2 * g, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        int accH = 0, acc4 = 0;
        unsigned accL = 0;
        if (T5) {
          uint32_t d[7];
#pragma unroll
          for (int i = 0; i < 6; ++i) d[i] = __builtin_amdgcn_alignbyte(cd[r][i + 1], cd[r][i], shift);
          d[6] = __builtin_amdgcn_alignbyte(0u, cd[r][6], shift);
#pragma unroll
          for (int i = 0; i < 26; ++i) {
            // Entry address: code byte i into bits 8..15, the lane copy into bits 0..7.
            const uint32_t sel = 0x0c0c0400u | ((uint32_t)(i & 3) << 8);
            uint32_t addr = __builtin_amdgcn_perm(d[i >> 2], (i & 1) ? lc_odd : lc_even, sel);
            const uint64_t e64 = *(const uint64_t*)__builtin_assume_aligned(lut + addr, 8);
            const uint2 e = make_uint2((uint32_t)e64, (uint32_t)(e64 >> 32));
            accH = __builtin_amdgcn_sdot4((int)e.x, (int)xr[2 * i], accH, false);
            if (NPL == 2) accL = __builtin_amdgcn_udot4(e.x, xr[2 * i + 1], accL, false);
            typedef short s2 __attribute__((ext_vector_type(2)));
            s2 ea = __builtin_bit_cast(s2, e.y), xa = __builtin_bit_cast(s2, xr[52 + (i >> 1)]);
            acc4 = __builtin_amdgcn_sdot2(ea, xa, acc4, false);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 32; ++i) {
            const uint32_t sel = 0x0c0c0400u | ((uint32_t)(i & 3) << 8);
            uint32_t addr = __builtin_amdgcn_perm(cd[r][i >> 2], lc_even, sel);
            uint32_t e = *(const uint32_t*)__builtin_assume_aligned(lut + addr, 4);
            accH = __builtin_amdgcn_sdot4((int)e, (int)xr[2 * i], accH, false);
            if (NPL == 2) accL = __builtin_amdgcn_udot4(e, xr[2 * i + 1], accL, false);
          }
        }
        int S;
        if (NPL == 2) S = (accH << 8) + (int)accL + acc4 - gsx;
        else S = accH + acc4 - gsx;
        if (MODE == MODE_F32) {
          float s = __half2float(__ushort_as_half((unsigned short)sc[r]));
          facc[r] += (float)S * (s * sig);
        } else if (MODE == MODE_EXACT) {
          int m11, e16;
          fp16_split((uint16_t)sc[r], m11, e16);
          long long prod = (long long)S * (long long)m11;
          int sh = e16 + p.B;
          long long c;
          if (sh >= 0) c = prod << sh;
          else c = (-sh >= 63) ? (prod < 0 ? -1 : 0) : (prod >> (-sh));
          iacc[r] += c;
        } else {
          if (pok[r]) p.yi[(size_t)prow[r] * p.G + g] = S;
        }
      }
    }

    if (MODE == MODE_GSUM) continue;
    // Reduce over the LPR lanes of the row group.
#pragma unroll
    for (int r = 0; r < R; ++r) {
      for (int o = LPR >> 1; o >= 1; o >>= 1) {
        if (MODE == MODE_F32) facc[r] += __shfl_xor(facc[r], o, 64);
        else iacc[r] += __shfl_xor(iacc[r], o, 64);
      }
    }
    if (MODE == MODE_EXACT) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (lg == (r % LPR) && pok[r]) {
          long long a = iacc[r];
          long long res = a >> p.R;
          int bad = ((a >= (1LL << 47)) || (a <= -(1LL << 47))) ? 1 : 0;
          bad |= (res >= (1LL << 31) || res <= -(1LL << 31)) ? 2 : 0;
          if (bad) atomicOr(p.status, bad);
          p.yi[prow[r]] = (int32_t)res;
        }
      }
    } else if (p.epi == TRX_EPI_SWIGLU) {
#pragma unroll
      for (int r = 0; r < R / 2; ++r) {
        if (lg == (r % LPR) && pok[r]) p.y[prow[r]] = silu(facc[r]) * facc[r + R / 2];
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (lg == (r % LPR) && pok[r]) {
          float v = facc[r];
          if (p.epi == TRX_EPI_RESID) v += p.resid[prow[r]];
          p.y[prow[r]] = v;
          if (p.amax_slot) {
            unsigned long long key = ((unsigned long long)ordered_bits(v) << 32) |
                                     (unsigned long long)(0xFFFFFFFFu - (uint32_t)prow[r]);
            atomicMax(p.amax_slot, key);
          }
        }
      }
    }
  }
}

// Host side ------------------------------------------------------------------------------------

static int lds_bytes(int K, int G) {
  return G * kXStride * 4 + K * 2 + G * 8 + 64;
}

static int pick_lpr(int G) {
  int l = 64;
  while (l > 1 && (G % l)) l >>= 1;
  return l;
}

template <int FMT, int MODE, int R>
static int launch(GemvParams& p, int n_blocks, hipStream_t s) {
  int shm = lds_bytes(p.K, p.G);
  static bool attr_set = false;
  if (!attr_set) {
    TRX_HIP(hipFuncSetAttribute((const void*)gemv_kernel<FMT, MODE, R>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - kLutBytes));
    attr_set = true;
  }
  p.n_batches = (p.epi == TRX_EPI_SWIGLU) ? cdiv(p.n_out, R / 2) : cdiv(p.n_out, R);
  int per_block = (kThreads / 64) * (64 / p.LPR);
  int need = cdiv(p.n_batches, per_block);
  int nb = need < n_blocks ? need : n_blocks;
  if (nb < 1) nb = 1;
  hipLaunchKernelGGL((gemv_kernel<FMT, MODE, R>), dim3(nb), dim3(kThreads), shm, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

static int g_num_cus = 0;
static int num_cus() {
  if (!g_num_cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 256;
    g_num_cus = prop.multiProcessorCount;
  }
  return g_num_cus;
}

int gemv_check(int kind, int M, int K) {
  TRX_CHECK(kind == TRX_KIND_TERNARY || kind == TRX_KIND_TERNARY5, TRX_E_INVALID,
            "gemv: kind %d is not a ternary kind", kind);
  TRX_CHECK(M > 0 && K > 0 && (K % kGroup) == 0, TRX_E_INVALID,
            "gemv: M=%d K=%d (K must be a positive multiple of 128)", M, K);
  TRX_CHECK(lds_bytes(K, K / kGroup) <= 160 * 1024 - kLutBytes, TRX_E_INVALID,
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
  p.w_bytes = (uint32_t)((unsigned long long)M * rg.row_bytes);
  p.LPR = pick_lpr(rg.G);
  p.NSLOT = rg.G / p.LPR;
}

int gemv_f32(const uint8_t* rows, int kind, int M, int K, const float* x, const float* norm_w,
             float eps, float* y, int epi, const float* resid, int swiglu_F,
             unsigned long long* amax_slot, hipStream_t s) {
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
  if (epi == TRX_EPI_SWIGLU) {
    TRX_CHECK(swiglu_F > 0 && 2 * swiglu_F == M, TRX_E_INVALID, "gemv: SwiGLU needs M == 2F");
    p.swiglu_F = swiglu_F;
    p.n_out = swiglu_F;
  } else {
    p.n_out = M;
  }
  int nb = num_cus();
  if (kind == TRX_KIND_TERNARY5) return launch<TRX_KIND_TERNARY5, MODE_F32, 4>(p, nb, s);
  return launch<TRX_KIND_TERNARY, MODE_F32, 4>(p, nb, s);
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
  int nb = num_cus();
  if (kind == TRX_KIND_TERNARY5) return launch<TRX_KIND_TERNARY5, MODE_EXACT, 4>(p, nb, s);
  return launch<TRX_KIND_TERNARY, MODE_EXACT, 4>(p, nb, s);
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
  int nb = num_cus();
  if (kind == TRX_KIND_TERNARY5) return launch<TRX_KIND_TERNARY5, MODE_GSUM, 4>(p, nb, s);
  return launch<TRX_KIND_TERNARY, MODE_GSUM, 4>(p, nb, s);
}

}  // namespace trx
