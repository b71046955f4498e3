// Batched prefill kernels: R prompt positions per forward, one weight pass for all of them.
//
// The projections run on the matrix cores (v_mfma_f32_32x32x16_f16): four waves of a block decode
// 256 stored ternary rows into LDS as fp16 weights, 64 columns at a time, while its other four
// multiply 128 (or 64) positions by the previous 64 columns, x split into two fp16 planes (hi,
// lo) so the fp32 accumulation sees x to ~22 bits.
// Attention, the RoPE/KV append and the Gated DeltaNet recurrence are the one-position rules of
// the decode kernels applied to every position of the chunk (the recurrence in order).

#include "trx_internal.h"
#include "trx_prefill.h"

#include <algorithm>
#include <type_traits>

namespace trx {

// GEMM ------------------------------------------------------------------------------------------

constexpr int kGmStage = 256;              // staging threads per block (waves 4-7)
constexpr int kGmThreads = 512;            // waves 0-3 run the MFMAs
constexpr int kGmBM = 256;                 // weight rows per block
constexpr int kGmLd = kGroup / 2 + 8;      // LDS row stride in halves (144 bytes): half a group per step

__device__ __forceinline__ uint32_t pk_mul_h2(uint32_t a, uint32_t s2) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  const h2_t r = __builtin_bit_cast(h2_t, a) * __builtin_bit_cast(h2_t, s2);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t half_bits(float v) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

// Weight row of LDS tile row i: plain tiles take M rows in order; a SwiGLU tile takes 128 gate
// rows f0 .. f0 + 127 (LDS rows 0..127) and the matching up rows F + f0 .. (LDS rows 128..255).
__device__ __forceinline__ int gm_wrow(int epi, int i, int M) {
  if (epi == GM_SWIGLU) {
    const int F = M / 2, f = blockIdx.x * (kGmBM / 2) + (i % (kGmBM / 2));
    return f < F ? (i < kGmBM / 2 ? f : F + f) : M;
  }
  return blockIdx.x * kGmBM + i;
}

template <int KIND>
struct GmRaw {
  uint4 c[KIND == TRX_KIND_Q8 ? 4 : 1];
  uint32_t sc;
};

// NA: position tiles of 32 per wave (2: 128 positions per block; 1: 64, for grids that would
// otherwise leave part of a round of blocks idle).
template <int KIND, int EPI, int NA>
__global__ __launch_bounds__(kGmThreads, 1) void gemm_kernel(GemmParams p) {
  constexpr int BR = 64 * NA;
  // Two buffers of each: a step (64 columns, half a group) is staged into one while the matrix
  // cores read the other.
  __shared__ __align__(16) _Float16 ws[2][kGmBM * kGmLd];
  __shared__ __align__(16) _Float16 xs[2][2][BR * kGmLd];
  __shared__ uint32_t tsel[16];
  __shared__ uint2 tsel27[32];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const bool cw = w < 4;                    // a wave that runs the MFMAs
  const int stid = max(tid - kGmStage, 0);  // staging thread index
  const int r0 = blockIdx.y * BR;
  // K in gridDim.z parts (more than one only for a plain store into p.part): this block's groups
  // g0 .. g0 + G - 1.
  const int G = p.K / kGroup / (int)gridDim.z, g0 = (int)blockIdx.z * G;

  // Weights are decoded by v_perm_b32 from a register pair holding -s, 0, s and 2s as fp16 (s the
  // group's scale): selector half g(c) = 0x0100 + c * 0x0202 picks (c - 1) * s for code c. trit5:
  // a code byte b = lo + 9 hi, tsel[lo] = g(d0) | g(d1) << 16 and tsel27[hi] = {g(d2) | g(d3) <<
  // 16, g(d4)} (hi <= 28 for any byte). 2-bit: tsel[nibble] = g(c0) | g(c1) << 16. No table has
  // more entries than the LDS has banks, so its reads never conflict (a 256-entry table of the
  // decoded bytes stalled the LDS a third of the time).
  if (!cw && stid < 32) {
    auto gsel = [](int c) { return 0x0100u + 0x0202u * (uint32_t)c; };
    const int t = stid;
    if (KIND == TRX_KIND_TERNARY5) {
      if (t < 9) tsel[t] = gsel(t % 3) | gsel(t / 3) << 16;
      tsel27[t] = make_uint2(gsel(t % 3) | gsel(t / 3 % 3) << 16, gsel(t / 9 % 3));
    } else if (KIND == TRX_KIND_TERNARY) {
      if (t < 16) tsel[t] = gsel(t & 3) | gsel(t >> 2) << 16;
    }
  }

  // Staging roles (waves 4-7): staging thread t decodes the 128 codes of LDS row t (two halves
  // of 64), and copies eight 16-byte pieces of the two x planes.
  const int srow = stid;
  const int wrow = gm_wrow(EPI, srow, p.M);
  const bool wvalid = wrow < p.M;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.W, p.w_bytes);
  const uint32_t rbase = (uint32_t)(wvalid ? wrow : 0) * (uint32_t)p.row_bytes;
  const __amdgpu_buffer_rsrc_t rxh = make_rsrc(p.xh, (uint32_t)((size_t)p.R * p.K * 2));
  const __amdgpu_buffer_rsrc_t rxl = make_rsrc(p.xl, (uint32_t)((size_t)p.R * p.K * 2));

  auto load_w = [&](GmRaw<KIND>& raw, int g, int shalf) {
    if (KIND == TRX_KIND_TERNARY5) {
      const uint32_t o = (uint32_t)p.code_off + 26u * (uint32_t)g + (shalf ? 12u : 0u);
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(rw, rbase + (o & ~3u), 0, 0);
      raw.c[0] = make_uint4(a[0], a[1], a[2], a[3]);
      raw.sc = __builtin_amdgcn_raw_buffer_load_b16(rw, rbase + 2u * (uint32_t)g, 0, 0);
    } else if (KIND == TRX_KIND_TERNARY) {
      const uint32_t o = (uint32_t)p.code_off + 32u * (uint32_t)g + 16u * (uint32_t)shalf;
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(rw, rbase + o, 0, 0);
      raw.c[0] = make_uint4(a[0], a[1], a[2], a[3]);
      raw.sc = __builtin_amdgcn_raw_buffer_load_b16(rw, rbase + 2u * (uint32_t)g, 0, 0);
    } else {
      const uint32_t o = (uint32_t)p.code_off + 128u * (uint32_t)g + 64u * (uint32_t)shalf;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(rw, rbase + o + 16u * k, 0, 0);
        raw.c[k] = make_uint4(a[0], a[1], a[2], a[3]);
      }
      // The two 32-column group scales of this half (groups 4g + 2 shalf and the next).
      raw.sc = __builtin_amdgcn_raw_buffer_load_b32(rw, rbase + 2u * (4u * (uint32_t)g + 2u * (uint32_t)shalf), 0, 0);
    }
  };
  constexpr int XQ = BR * 8 / kGmStage;            // 16-byte x pieces per thread, plane and step
  // x of step st (columns 64 st .. + 63): thread t moves pieces t + 256 q (row piece / 8, 8 columns).
  auto load_x = [&](uint4* xr, int st) {
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int piece = stid + kGmStage * q, row = piece >> 3, c8 = piece & 7;
      const uint32_t off = ((uint32_t)(r0 + row) * (uint32_t)p.K + (uint32_t)(64 * st + 8 * c8)) * 2u;
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(rxh, off, 0, 0);
      const auto b = __builtin_amdgcn_raw_buffer_load_b128(rxl, off, 0, 0);
      xr[q] = make_uint4(a[0], a[1], a[2], a[3]);
      xr[XQ + q] = make_uint4(b[0], b[1], b[2], b[3]);
    }
  };
  // Decoded weights of this thread's 64 codes: 32 dwords of fp16 pairs, times the scale (0 for
  // a row past M, whose codes were read from row 0). The half of the group (shc, a compile-time
  // constant) is also the LDS buffer. No branch: one block of code per half.
  auto stage_w = [&](const GmRaw<KIND>& raw, int g, auto shc) {
    constexpr int shalf = decltype(shc)::value, buf = shalf;
    uint32_t D[32];
    const uint32_t sc = wvalid ? raw.sc : 0u;
    if (KIND == TRX_KIND_Q8) {
      // int8 -> fp16 exactly, times the 32-column group's scale in fp16 (fp16(q * s)).
      const uint32_t dw[16] = {raw.c[0].x, raw.c[0].y, raw.c[0].z, raw.c[0].w, raw.c[1].x, raw.c[1].y,
                               raw.c[1].z, raw.c[1].w, raw.c[2].x, raw.c[2].y, raw.c[2].z, raw.c[2].w,
                               raw.c[3].x, raw.c[3].y, raw.c[3].z, raw.c[3].w};
      const uint32_t s0 = sc & 0xFFFFu, s1 = sc >> 16;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        auto q = [&](int b) { return half_bits((float)(int8_t)(uint8_t)(dw[j] >> (8 * b))); };
        const uint32_t s2 = j < 8 ? (s0 | s0 << 16) : (s1 | s1 << 16);
        D[2 * j] = pk_mul_h2(q(0) | q(1) << 16, s2);
        D[2 * j + 1] = pk_mul_h2(q(2) | q(3) << 16, s2);
      }
    } else {
      // The permute pair: bytes 0-3 {-s, 0}, bytes 4-7 {s, 2s} (fp16(1 * s), fp16(2 * s)).
      const uint32_t s16 = sc & 0xFFFFu;
      const uint32_t plo = s16 ^ 0x8000u, phi = pk_mul_h2(s16 | s16 << 16, 0x40003C00u);
      auto wp = [&](uint32_t sel) { return __builtin_amdgcn_perm(phi, plo, sel); };
      if (KIND == TRX_KIND_TERNARY5) {
        const uint32_t o = (uint32_t)p.code_off + 26u * (uint32_t)g + (shalf ? 12u : 0u);
        const uint32_t sh = o & 3u;
        const uint32_t d0 = __builtin_amdgcn_alignbyte(raw.c[0].y, raw.c[0].x, sh);
        const uint32_t d1 = __builtin_amdgcn_alignbyte(raw.c[0].z, raw.c[0].y, sh);
        const uint32_t d2 = __builtin_amdgcn_alignbyte(raw.c[0].w, raw.c[0].z, sh);
        const uint32_t d3 = __builtin_amdgcn_alignbyte(0u, raw.c[0].w, sh);
        const uint32_t dw[4] = {d0, d1, d2, d3};
        // Byte j's selectors: lo pair (d0, d1) and hi {(d2, d3), d4}.
        auto sel = [&](int j, uint32_t& lo, uint2& hi) {
          const uint32_t b = (dw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
          const uint32_t h = (b * 57u) >> 9;          // b / 9 for every byte value
          lo = tsel[b - 9u * h];
          hi = tsel27[h];
        };
        // An even byte's five codes start a dword, the odd byte's five follow: five dwords.
        auto pair5 = [&](int j, uint32_t* out) {
          uint32_t e9, o9;
          uint2 e27, o27;
          sel(j, e9, e27);
          sel(j + 1, o9, o27);
          out[0] = wp(e9);
          out[1] = wp(e27.x);
          out[2] = wp(e27.y | o9 << 16);
          out[3] = wp(__builtin_amdgcn_alignbit(o27.x, o9, 16));
          out[4] = wp(__builtin_amdgcn_alignbit(o27.y, o27.x, 16));
        };
        if constexpr (shalf == 0) {
          // bytes 0..12: codes 0..64, of which 0..63 are this half's
#pragma unroll
          for (int i = 0; i < 6; ++i) pair5(2 * i, D + 5 * i);
          uint32_t e9;
          uint2 e27;
          sel(12, e9, e27);
          D[30] = wp(e9);
          D[31] = wp(e27.x);
        } else {
          // bytes 12..25: codes 60..129; this half takes 64..127
          uint32_t e9, o9;
          uint2 e27, o27;
          sel(0, e9, e27);
          sel(1, o9, o27);
          D[0] = wp(e27.y | o9 << 16);
          D[1] = wp(__builtin_amdgcn_alignbit(o27.x, o9, 16));
          D[2] = wp(__builtin_amdgcn_alignbit(o27.y, o27.x, 16));
#pragma unroll
          for (int i = 1; i < 6; ++i) pair5(2 * i, D + 5 * i - 2);
          uint32_t t[5];
          pair5(12, t);
          D[28] = t[0];
          D[29] = t[1];
          D[30] = t[2];
          D[31] = t[3];
        }
      } else {
        const uint32_t dw[4] = {raw.c[0].x, raw.c[0].y, raw.c[0].z, raw.c[0].w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t b = (dw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
          D[2 * j] = wp(tsel[b & 15u]);
          D[2 * j + 1] = wp(tsel[b >> 4]);
        }
      }
    }
    uint4* dst = (uint4*)(ws[buf] + srow * kGmLd);
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = make_uint4(D[4 * i], D[4 * i + 1], D[4 * i + 2], D[4 * i + 3]);
  };
  auto stage_x = [&](const uint4* xr, int buf) {
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int piece = stid + kGmStage * q, row = piece >> 3, c8 = piece & 7;
      *(uint4*)(xs[buf][0] + row * kGmLd + 8 * c8) = xr[q];
      *(uint4*)(xs[buf][1] + row * kGmLd + 8 * c8) = xr[XQ + q];
    }
  };

  // Wave tiles: positions 64 wr .. + 63 of the block (two tiles of 32); four weight column tiles
  // of 32 (SwiGLU: two gate tiles and the two up tiles of the same features). Per 16-column step a
  // wave reads 4 A and 4 B fragments for 16 MFMAs.
  const int wr = w & 1, wm = w >> 1;
  int ct[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    ct[t] = EPI == GM_SWIGLU ? (t >> 1) * (kGmBM / 2) + 64 * wm + 32 * (t & 1) : 128 * wm + 32 * t;
  const int li = lane & 31, lk = 8 * (lane >> 5);
  f32x16_t acc[NA][4] = {};

  // Steps of 64 columns (st = 2g + half): step st + 1 is staged into the other buffers while the
  // matrix cores take step st, and step st + 3 is loaded into the registers step st + 1 freed (two
  // steps of latency cover). The loop is unrolled by two, so a step's registers and buffers are
  // fixed per half.
  const int NS = 2 * G;
  GmRaw<KIND> raw[2];
  uint4 xr[2][2 * XQ];
  auto load_step = [&](int st, int slot) {
    load_w(raw[slot], g0 + (st >> 1), st & 1);
    load_x(xr[slot], 2 * g0 + st);
  };
  // A step's half is its register slot and LDS buffer: st & 1 == slot.
  auto stage_step = [&](int st, auto slot) {
    stage_w(raw[decltype(slot)::value], g0 + (st >> 1), slot);
    stage_x(xr[decltype(slot)::value], decltype(slot)::value);
  };
  const std::integral_constant<int, 0> I0;
  const std::integral_constant<int, 1> I1;
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < kGroup / 32; ++kk) {
      const int k = 16 * kk + lk;
      half8_t ah[NA], al[NA], b[4];
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        ah[a] = *(const half8_t*)(xs[buf][0] + (32 * NA * wr + 32 * a + li) * kGmLd + k);
        al[a] = *(const half8_t*)(xs[buf][1] + (32 * NA * wr + 32 * a + li) * kGmLd + k);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) b[t] = *(const half8_t*)(ws[buf] + (ct[t] + li) * kGmLd + k);
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[a][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[a], b[t], acc[a][t], 0, 0, 0);
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[a][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[a], b[t], acc[a][t], 0, 0, 0);
    }
  };
  // Waves 0-3 run the MFMAs, waves 4-7 decode and stage the next step meanwhile (with both roles
  // in every wave, all four waves decoded at once and the matrix cores sat idle meanwhile). Each
  // role has a loop of its own, so neither role's registers are live in the other's (two waves
  // per SIMD leave 256 registers a wave), and both pass the same 2 + NS barriers. The loops take
  // two steps a pass with no exit between them: with one, the compiler gave the two halves'
  // accumulators different registers and copied them every pass. A staging thread's loads past
  // the last step repeat it, so its halves have no branch either.
  if (!cw) {
    load_step(0, 0);
    load_step(1, 1);                      // NS >= 2: K is a multiple of 128
    __syncthreads();                      // the code tables are written
    stage_step(0, I0);
    load_step(min(2, NS - 1), 0);
    __syncthreads();
    for (int st = 0; st < NS; st += 2) {
      stage_step(st + 1, I1);
      load_step(min(st + 3, NS - 1), 1);
      __syncthreads();
      stage_step(st + 2, I0);             // the last pass stages a step NS that nothing reads
      load_step(min(st + 4, NS - 1), 0);
      __syncthreads();
    }
    return;
  }
  __syncthreads();
  __syncthreads();
  for (int st = 0; st < NS; st += 2) {
    compute(0);
    __syncthreads();
    compute(1);
    __syncthreads();
  }

  // Accumulator e of lane l holds D[i][j], i = 8 (e / 4) + 4 (l / 32) + e % 4, j = l % 32.
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
    const int r = r0 + 32 * NA * wr + 32 * a + i;
    if (r >= p.R) continue;
    float* yr = (gridDim.z > 1 ? p.part + (size_t)blockIdx.z * p.R * p.ldy : p.y) + (size_t)r * p.ldy;
    const float up = p.xs[r];              // the row's plane scale (a power of two: exact)
    if (EPI == GM_SWIGLU) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int f = blockIdx.x * (kGmBM / 2) + ct[t] + li;
        if (f < p.M / 2) yr[f] = silu(acc[a][t][e] * up) * (acc[a][t + 2][e] * up);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int m = blockIdx.x * kGmBM + ct[t] + li;
        if (m < p.M) {
          if (EPI == GM_RESID) yr[m] += acc[a][t][e] * up;
          else yr[m] = acc[a][t][e] * up;
        }
      }
    }
  }
}

// y[r][m] = sum over z of part[z][r][m], in part order: one block per row.
__global__ __launch_bounds__(256) void gemm_parts_kernel(const float* part, int kp, int R, int M, int ldy, float* y) {
  const int r = blockIdx.x;
  for (int m = threadIdx.x; m < M; m += 256) {
    float v = 0.f;
    for (int z = 0; z < kp; ++z) v += part[((size_t)z * R + r) * ldy + m];
    y[(size_t)r * ldy + m] = v;
  }
}

template <int KIND, int NA>
static void gemm_dispatch(const GemmParams& p, dim3 grid, hipStream_t s) {
  if (p.epi == GM_SWIGLU)
    hipLaunchKernelGGL((gemm_kernel<KIND, GM_SWIGLU, NA>), grid, dim3(kGmThreads), 0, s, p);
  else if (p.epi == GM_RESID)
    hipLaunchKernelGGL((gemm_kernel<KIND, GM_RESID, NA>), grid, dim3(kGmThreads), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_kernel<KIND, GM_STORE, NA>), grid, dim3(kGmThreads), 0, s, p);
}

int launch_gemm(const GemmParams& p, hipStream_t s) {
  TRX_CHECK(p.kind == TRX_KIND_TERNARY || p.kind == TRX_KIND_TERNARY5 || p.kind == TRX_KIND_Q8, TRX_E_INVALID,
            "prefill GEMM: weight kind %d unsupported", p.kind);
  TRX_CHECK(p.M >= 1 && p.K >= kGroup && p.K % kGroup == 0 && p.R >= 1, TRX_E_INVALID,
            "prefill GEMM: M=%d K=%d R=%d", p.M, p.K, p.R);
  TRX_CHECK(p.epi != GM_SWIGLU || p.M % 2 == 0, TRX_E_INVALID, "prefill GEMM: SwiGLU needs an even M");
  TRX_CHECK((size_t)p.R * p.K * 2 < (1ull << 32) && (size_t)p.M * p.row_bytes < (1ull << 32) &&
            (size_t)p.M * p.row_bytes + 16 <= p.w_bytes, TRX_E_INVALID, "prefill GEMM: operands too large");
  const int nx = p.epi == GM_SWIGLU ? cdiv(p.M / 2, kGmBM / 2) : cdiv(p.M, kGmBM);
  // 128 positions per block, or 64 when twice the blocks take fewer rounds of blocks per CU, each
  // round ~0.78 as long: a 64-position block's staging waves decode as many weights for half the
  // products (8B q|k|v, 2048 positions: 768 blocks of 64 in 317 us, 384 of 128 in 271 us).
  int cus = 0, dev = 0;
  TRX_HIP(hipGetDevice(&dev));
  TRX_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const bool small = 0.78 * cdiv(nx * cdiv(p.R, 64), cus) < (double)cdiv(nx * cdiv(p.R, 128), cus);
  // A grid that leaves most CUs idle (a few weight rows, as the DeltaNet beta|alpha rows) splits
  // K into parts when the caller gives room for their sums: the largest divisor of the group
  // count, at most 16, whose blocks still fit one round.
  const int blocks = nx * cdiv(p.R, small ? 64 : 128), G = p.K / kGroup;
  int kp = 1;
  if (p.part && p.epi == GM_STORE && 2 * blocks <= cus)
    for (int d = std::min(16, cus / blocks); d > 1; --d)
      if (G % d == 0 && (size_t)d * p.R * p.ldy <= p.part_floats) {
        kp = d;
        break;
      }
  const dim3 grid(nx, cdiv(p.R, small ? 64 : 128), kp);
  if (p.kind == TRX_KIND_TERNARY5) {
    if (small) gemm_dispatch<TRX_KIND_TERNARY5, 1>(p, grid, s);
    else gemm_dispatch<TRX_KIND_TERNARY5, 2>(p, grid, s);
  } else if (p.kind == TRX_KIND_TERNARY) {
    if (small) gemm_dispatch<TRX_KIND_TERNARY, 1>(p, grid, s);
    else gemm_dispatch<TRX_KIND_TERNARY, 2>(p, grid, s);
  } else {
    if (small) gemm_dispatch<TRX_KIND_Q8, 1>(p, grid, s);
    else gemm_dispatch<TRX_KIND_Q8, 2>(p, grid, s);
  }
  TRX_LAUNCHED();
  if (kp > 1) {
    hipLaunchKernelGGL(gemm_parts_kernel, dim3(p.R), dim3(256), 0, s, p.part, kp, p.R, p.M, p.ldy, p.y);
    TRX_LAUNCHED();
  }
  return TRX_OK;
}

// Input planes ---------------------------------------------------------------------------------

__device__ __forceinline__ void store_hilo(const PrepParams& p, size_t i, float v) {
  const _Float16 h = (_Float16)v;
  p.xh[i] = h;
  p.xl[i] = (_Float16)(v - (float)h);
}

// The power of two 2^e (e >= 0) that brings a row whose values are bounded by `bound` below 2^14
// (fp16 planes stay finite and the low plane keeps its bits), and its inverse.
__device__ __forceinline__ void row_scale(float bound, float& down, float& up) {
  down = up = 1.f;
  if (bound >= 16384.f && bound <= 3.0e38f) {
    int k;
    frexpf(bound, &k);                 // bound < 2^k
    down = ldexpf(1.f, 14 - k);
    up = ldexpf(1.f, k - 14);
  }
}

__device__ __forceinline__ float block_max(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = red[0];
  for (int i = 1; i < nw; ++i) t = fmaxf(t, red[i]);
  return t;
}

// One block of 256 threads per position, no rotation.
__global__ __launch_bounds__(256) void prep_kernel(PrepParams p) {
  __shared__ float red[16];
  const int r = blockIdx.x, t = threadIdx.x;
  const float* x = p.x + (size_t)r * p.ldx;
  float rs = 1.f;
  if (p.norm_w) {
    float ss = 0.f;
    for (int c = t; c < p.K; c += 256) ss += x[c] * x[c];
    rs = 1.0f / sqrtf(block_sum(ss, red) / (float)p.K + p.eps);
  }
  float am = 0.f;
  for (int c = t; c < p.K; c += 256) am = fmaxf(am, fabsf(p.norm_w ? x[c] * rs * p.norm_w[c] : x[c]));
  float down, up;
  row_scale(block_max(am, red), down, up);
  if (t == 0) p.xs[r] = up;
  for (int c = t; c < p.K; c += 256) {
    const float v = p.norm_w ? x[c] * rs * p.norm_w[c] : x[c];
    store_hilo(p, (size_t)r * p.K + c, v * down);
  }
}

// The same with 16-byte loads and 8-byte plane stores (K and the row stride multiples of 4).
__global__ __launch_bounds__(256) void prep_vec_kernel(PrepParams p) {
  __shared__ float red[16];
  const int r = blockIdx.x, t = threadIdx.x, K4 = p.K / 4;
  const float4* x = (const float4*)(p.x + (size_t)r * p.ldx);
  const float4* gw = (const float4*)p.norm_w;
  float rs = 1.f;
  if (gw) {
    float ss = 0.f;
    for (int c = t; c < K4; c += 256) {
      const float4 v = x[c];
      ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    rs = 1.0f / sqrtf(block_sum(ss, red) / (float)p.K + p.eps);
  }
  auto val = [&](int c) {
    float4 v = x[c];
    if (gw) {
      const float4 g = gw[c];
      v = make_float4(v.x * rs * g.x, v.y * rs * g.y, v.z * rs * g.z, v.w * rs * g.w);
    }
    return v;
  };
  float am = 0.f;
  for (int c = t; c < K4; c += 256) {
    const float4 v = val(c);
    am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  float down, up;
  row_scale(block_max(am, red), down, up);
  if (t == 0) p.xs[r] = up;
  uint2* xh = (uint2*)(p.xh + (size_t)r * p.K);
  uint2* xl = (uint2*)(p.xl + (size_t)r * p.K);
  for (int c = t; c < K4; c += 256) {
    const float4 v = val(c);
    const float e[4] = {v.x * down, v.y * down, v.z * down, v.w * down};
    uint32_t hb[4], lb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const _Float16 h = (_Float16)e[i];
      hb[i] = __builtin_bit_cast(uint16_t, h);
      lb[i] = half_bits(e[i] - (float)h);
    }
    xh[c] = make_uint2(hb[0] | hb[1] << 16, hb[2] | hb[3] << 16);
    xl[c] = make_uint2(lb[0] | lb[1] << 16, lb[2] | lb[3] << 16);
  }
}

// Rotated input: one block of B threads per (rotation block, position), as rotate_kernel does for
// one vector (the whole row's sum of squares, the butterflies by shuffles then LDS).
// The rotated input's row statistics, one block of 256 threads per position: the RMSNorm scale
// 1/rms(x) (1 without a norm) and the power of two that keeps the row's planes finite. Every
// output of a rotation block is bounded by scale * B times the row's largest |x * gain| (times
// 1/rms), which sets one scale for all of the row's blocks.
__global__ __launch_bounds__(256) void prep_rot_stats_kernel(PrepParams p) {
  __shared__ float red[16];
  const int r = blockIdx.x, t = threadIdx.x;
  const float* x = p.x + (size_t)r * p.ldx;
  float ss = 0.f, am = 0.f;
  for (int i = t; i < p.K; i += 256) {
    ss += x[i] * x[i];
    am = fmaxf(am, fabsf(p.norm_w ? x[i] * p.norm_w[i] : x[i]));
  }
  const float tot = block_sum(ss, red);
  const float amax = block_max(am, red);
  const float rsn = p.norm_w ? 1.0f / sqrtf(tot / (float)p.K + p.eps) : 1.f;
  float down, up;
  row_scale(fabsf(p.scale) * (float)p.B * amax * rsn, down, up);
  if (t == 0) {
    p.xs[r] = up;
    p.rs[r] = rsn;
  }
}

// Rotated input: one block of B threads per (rotation block, position), as rotate_kernel does for
// one vector (the butterflies by shuffles then LDS), with the row's statistics from above.
__global__ __launch_bounds__(1024) void prep_rot_kernel(PrepParams p) {
  __shared__ float v[1024];
  const int t = threadIdx.x, B = blockDim.x, c = blockIdx.x * B + t, r = blockIdx.y;
  const int lane = t & 63;
  const float* x = p.x + (size_t)r * p.ldx;
  float a = x[c] * p.signs[c];
  if (p.norm_w) a *= p.norm_w[c] * p.rs[r];
  const float down = 1.0f / p.xs[r];               // a power of two: exact
  for (int h = 1; h < 64; h <<= 1) {
    const float o = __shfl_xor(a, h, 64);
    a = (lane & h) ? o - a : a + o;
  }
  for (int h = 64; h < B; h <<= 1) {
    v[t] = a;
    __syncthreads();
    const float o = v[t ^ h];
    __syncthreads();
    a = (t & h) ? o - a : a + o;
  }
  store_hilo(p, (size_t)r * p.K + c, a * p.scale * down);
}

int launch_prep(const PrepParams& p, hipStream_t s) {
  TRX_CHECK(p.R >= 1 && p.K >= 1 && p.ldx >= p.K && p.xs, TRX_E_INVALID, "prefill input: R=%d K=%d", p.R, p.K);
  if (p.signs) {
    TRX_CHECK(p.B >= 64 && p.B <= 1024 && (p.B & (p.B - 1)) == 0 && p.K % p.B == 0, TRX_E_INVALID,
              "prefill input: rotation block %d over %d columns unsupported", p.B, p.K);
    TRX_CHECK(p.rs, TRX_E_INVALID, "prefill input: a rotation needs the row-scale buffer");
    hipLaunchKernelGGL(prep_rot_stats_kernel, dim3(p.R), dim3(256), 0, s, p);
    hipLaunchKernelGGL(prep_rot_kernel, dim3(p.K / p.B, p.R), dim3(p.B), 0, s, p);
  } else if (p.K % 4 == 0 && p.ldx % 4 == 0 && ((uintptr_t)p.x & 15) == 0 && ((uintptr_t)p.norm_w & 15) == 0) {
    hipLaunchKernelGGL(prep_vec_kernel, dim3(p.R), dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL(prep_kernel, dim3(p.R), dim3(256), 0, s, p);
  }
  TRX_LAUNCHED();
  return TRX_OK;
}

// RoPE and the KV append -----------------------------------------------------------------------

// One wave per (position, head): q heads first, then kv heads. HD / 64 elements per lane.
template <int HD>
__global__ __launch_bounds__(64) void rope_kv_kernel(RopeKvParams p) {
  constexpr int E = HD / 64;
  __shared__ float nv_s[HD];
  const int r = blockIdx.x, j = blockIdx.y, lane = threadIdx.x;
  const int pos = p.p0 + r, half = p.rope_n / 2;
  const int qstride = p.gated ? 2 * HD : HD;
  const bool isq = j < p.n_head;
  const int g = j - p.n_head;
  const float* src = p.qkv + (size_t)r * p.ldq + (isq ? (size_t)j * qstride : (size_t)p.n_head * qstride + (size_t)g * HD);
  const float* wn = isq ? p.q_norm : p.k_norm;
  float v[E];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    v[e] = src[lane + 64 * e];
    ss += v[e] * v[e];
  }
  ss = wave_sum(ss);
  const float rr = 1.0f / sqrtf(ss / (float)HD + p.eps);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    v[e] = v[e] * rr * wn[lane + 64 * e];
    nv_s[lane + 64 * e] = v[e];
  }
  __syncthreads();
  float o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    o[e] = v[e];
    if (d < 2 * half) {
      const int i = d < half ? d : d - half;
      float sn, cs;
      if (p.rope_tab) {
        cs = (float)p.rope_tab[(size_t)pos * p.rope_n + i] * (1.0f / 16384.0f);
        sn = (float)p.rope_tab[(size_t)pos * p.rope_n + half + i] * (1.0f / 16384.0f);
      } else if (p.rope_cs) {
        cs = p.rope_cs[(size_t)pos * p.rope_n + i];
        sn = p.rope_cs[(size_t)pos * p.rope_n + half + i];
      } else {
        sincosf((float)pos * p.rope_freq[i], &sn, &cs);
      }
      o[e] = d < half ? v[e] * cs - nv_s[d + half] * sn : nv_s[d - half] * sn + v[e] * cs;
    }
  }
  if (isq) {
    const float post = 1.0f / sqrtf((float)HD);
    float* dst = p.q_out + ((size_t)r * p.n_head + j) * HD;
#pragma unroll
    for (int e = 0; e < E; ++e) dst[lane + 64 * e] = o[e] * post;
  } else {
    const size_t c = ((size_t)g * p.max_ctx + pos) * HD;
    const float* vsrc = p.qkv + (size_t)r * p.ldq + (size_t)p.n_head * qstride + (size_t)p.n_kv * HD + (size_t)g * HD;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      p.kcache[c + lane + 64 * e] = __float2half(o[e]);
      p.vcache[c + lane + 64 * e] = __float2half(vsrc[lane + 64 * e]);
    }
  }
}

int launch_rope_kv(const RopeKvParams& p, hipStream_t s) {
  TRX_CHECK(p.R >= 1 && p.p0 >= 0 && p.p0 + p.R <= p.max_ctx && p.rope_n % 2 == 0 && p.rope_n <= p.hd,
            TRX_E_INVALID, "prefill RoPE: positions %d..%d", p.p0, p.p0 + p.R);
  const dim3 grid(p.R, p.n_head + p.n_kv);
  if (p.hd == 64) hipLaunchKernelGGL(rope_kv_kernel<64>, grid, dim3(64), 0, s, p);
  else if (p.hd == 128) hipLaunchKernelGGL(rope_kv_kernel<128>, grid, dim3(64), 0, s, p);
  else if (p.hd == 256) hipLaunchKernelGGL(rope_kv_kernel<256>, grid, dim3(64), 0, s, p);
  else TRX_CHECK(false, TRX_E_INVALID, "prefill RoPE: head_dim %d unsupported", p.hd);
  TRX_LAUNCHED();
  return TRX_OK;
}

// Causal attention ------------------------------------------------------------------------------
//
// Block (query tile, kv head): the rep q heads of the kv head at QT = 64 / rep positions, one
// query row per 4 threads (row = position offset * rep + head offset). Key tiles of KT cache
// positions in LDS as fp32; each thread scores KT/4 keys, the row's online softmax runs over its
// four lanes (shuffles), and each thread accumulates HD/4 output dims.

template <int HD, int KT>
__global__ __launch_bounds__(256) void attn_prefill_kernel(AttnPrefillParams p) {
  constexpr int KPT = KT / 4, DPT = HD / 4;
  __shared__ __align__(16) float qs[64][HD];
  __shared__ __align__(16) float ks[KT][HD + 4];
  __shared__ __align__(16) float vs[KT][HD + 4];
  __shared__ float ps[64][KT + 1];
  const int tid = threadIdx.x, row = tid >> 2, tq = tid & 3;
  const int rep = p.n_head / p.n_kv, QT = 64 / rep;
  const int g = blockIdx.y, q0 = blockIdx.x * QT;        // chunk offset of the tile's first query
  const int pq = row / rep, jh = row - pq * rep;
  const bool rvalid = pq < QT && q0 + pq < p.R;
  const int qpos = p.p0 + q0 + pq;                        // absolute position of this row
  const int h = g * rep + jh;
  const int last = p.p0 + min(p.R, q0 + QT) - 1;          // last key any row of the tile sees

  for (int i = tid; i < 64 * HD / 4; i += 256) {
    const int rr = i / (HD / 4), d4 = i - rr * (HD / 4);
    const int pq_ = rr / rep, j_ = rr - pq_ * rep;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (pq_ < QT && q0 + pq_ < p.R)
      v = *(const float4*)(p.q + ((size_t)(q0 + pq_) * p.n_head + g * rep + j_) * HD + 4 * d4);
    *(float4*)&qs[rr][4 * d4] = v;
  }
  float acc[DPT];
#pragma unroll
  for (int d = 0; d < DPT; ++d) acc[d] = 0.f;
  float m = -INFINITY, l = 0.f;
  const __half* kc = p.kcache + (size_t)g * p.max_ctx * HD;
  const __half* vc = p.vcache + (size_t)g * p.max_ctx * HD;

  for (int t0 = 0; t0 <= last; t0 += KT) {
    __syncthreads();                                      // previous tile's reads are done
    for (int i = tid; i < KT * HD / 8; i += 256) {
      const int t = i / (HD / 8), d8 = i - t * (HD / 8);
      float kf[8], vf[8];
      if (t0 + t <= last) {
        const uint4 kr = *(const uint4*)(kc + (size_t)(t0 + t) * HD + 8 * d8);
        const uint4 vr = *(const uint4*)(vc + (size_t)(t0 + t) * HD + 8 * d8);
        const __half* kh = (const __half*)&kr;
        const __half* vh = (const __half*)&vr;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          kf[k] = __half2float(kh[k]);
          vf[k] = __half2float(vh[k]);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) kf[k] = vf[k] = 0.f;
      }
      *(float4*)&ks[t][8 * d8] = make_float4(kf[0], kf[1], kf[2], kf[3]);
      *(float4*)&ks[t][8 * d8 + 4] = make_float4(kf[4], kf[5], kf[6], kf[7]);
      *(float4*)&vs[t][8 * d8] = make_float4(vf[0], vf[1], vf[2], vf[3]);
      *(float4*)&vs[t][8 * d8 + 4] = make_float4(vf[4], vf[5], vf[6], vf[7]);
    }
    __syncthreads();
    // Scores of keys t0 + tq * KPT .. + KPT - 1.
    float sc[KPT];
#pragma unroll
    for (int k = 0; k < KPT; ++k) sc[k] = 0.f;
    for (int d = 0; d < HD; d += 4) {
      const float4 qv = *(const float4*)&qs[row][d];
#pragma unroll
      for (int k = 0; k < KPT; ++k) {
        const float4 kv = *(const float4*)&ks[tq * KPT + k][d];
        sc[k] += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      if (t0 + tq * KPT + k > qpos) sc[k] = -INFINITY;
      tmax = fmaxf(tmax, sc[k]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 1, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 2, 64));
    const float mn = fmaxf(m, tmax);
    // A tile past this row's position is all masked: nothing changes (mn stays m).
    const float corr = mn == -INFINITY ? 1.f : __expf(m - mn);
    float psum = 0.f;
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      const float pk = sc[k] == -INFINITY ? 0.f : __expf(sc[k] - mn);
      ps[row][tq * KPT + k] = pk;
      psum += pk;
    }
    psum += __shfl_xor(psum, 1, 64);
    psum += __shfl_xor(psum, 2, 64);
    l = l * corr + psum;
    m = mn;
#pragma unroll
    for (int d = 0; d < DPT; ++d) acc[d] *= corr;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int t = 0; t < KT; ++t) {
      const float pt = ps[row][t];
#pragma unroll
      for (int d = 0; d < DPT; d += 4) {
        const float4 vv = *(const float4*)&vs[t][tq * DPT + d];
        acc[d] += pt * vv.x;
        acc[d + 1] += pt * vv.y;
        acc[d + 2] += pt * vv.z;
        acc[d + 3] += pt * vv.w;
      }
    }
  }
  if (!rvalid) return;
  const float inv = 1.0f / l;
  float* dst = p.out + (size_t)(q0 + pq) * p.n_head * HD + (size_t)h * HD + tq * DPT;
  const float* gate = p.qkv + (size_t)(q0 + pq) * p.ldq + (size_t)h * 2 * HD + HD + tq * DPT;
#pragma unroll
  for (int d = 0; d < DPT; ++d) {
    float o = acc[d] * inv;
    if (p.gated) o *= sigmoidf_(gate[d]);
    dst[d] = o;
  }
}

// The same causal attention on the matrix cores, for head dims 64 and 128. A wave takes 32
// score columns (PW = 32 / rep positions x rep heads of one kv head; rep 6 leaves 2 columns
// idle) and a block four waves; every key tile of 32 cache positions is staged in LDS once per
// block (K row-major, V transposed), as fp16, which is how the cache holds them.
//   S^T = K Q^T   (v_mfma_f32_32x32x16_f16, keys x columns): q enters as two fp16 planes,
//                 q = hi + lo, so each score is the fp32 dot product to ~2^-22 relative;
//   online softmax per column in registers (a lane holds one column: 16 of its 32 keys, the
//                 other 16 in lane l ^ 32);
//   O^T += V^T P^T: the probabilities, again as hi + lo fp16 planes, feed the B operand straight
//                 from the score registers; the K slot order of A (V^T, read from LDS) follows
//                 the score layout (lane half h holds keys 4h..4h+3 and 8+4h..8+4h+3 of each 16).
// Numerics as attn_prefill_kernel's to fp32 rounding (softmax in fp32, __expf).
template <int HD>
__global__ __launch_bounds__(256, HD <= 128 ? 2 : 1) void attn_prefill_mfma_kernel(AttnPrefillParams p) {
  constexpr int NC = HD / 16, NDT = HD / 32;       // q chunks of 16 dims; 32-dim output tiles
  // LDS row strides (halfs). V^T rows of 36 halves (18 dwords, 8-byte aligned): the MFMA lanes'
  // 8-byte reads of rows j spread over every bank, and the staging threads' 8-byte stores to
  // rows 2 dp conflict at most two ways.
  constexpr int KS = HD + 8, VS = 32 + 4;
  // Two buffers of each: the next key tile is stored into one while the waves read the other.
  __shared__ __align__(16) _Float16 ks[2][32 * KS];
  __shared__ __align__(16) _Float16 vt[2][HD * VS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, j = lane & 31;
  const int rep = p.n_head / p.n_kv, PW = 32 / rep, g = blockIdx.y;
  // The causal work of a block grows with its position tile. Blocks b and b + 256 share a CU
  // (blocks go round-robin over the XCDs and their CUs), so the upper half of the kv heads takes
  // the tiles in reverse: a CU holds tiles x and last - x, not two of the longest.
  const int bx = blockIdx.y >= (gridDim.y + 1) / 2 ? gridDim.x - 1 - blockIdx.x : blockIdx.x;
  const int q0 = bx * 4 * PW;                                      // chunk offset of the block
  const int pq = j / rep, jh = j - pq * rep;
  const int qrow = q0 + w * PW + pq;                               // chunk row of this column
  const bool cvalid = pq < PW && qrow < p.R;
  const int qpos = cvalid ? p.p0 + qrow : -1;                      // -1: every key masked
  const int head = g * rep + jh;
  const int wave_last = p.p0 + min(p.R, q0 + (w + 1) * PW) - 1;
  const int wave_first = p.p0 + q0 + w * PW;
  const int block_last = p.p0 + min(p.R, q0 + 4 * PW) - 1;

  // This column's q as fp16 hi/lo planes in the B-operand layout (dims 16c + 8h .. + 7).
  half8_t qh[NC], ql[NC];
  {
    const float* qr = p.q + ((size_t)(cvalid ? qrow : 0) * p.n_head + head) * HD + 8 * h;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 a = cvalid ? *(const float4*)(qr + 16 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 b = cvalid ? *(const float4*)(qr + 16 * c + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const _Float16 hi = (_Float16)v[k];
        qh[c][k] = hi;
        ql[c][k] = (_Float16)(v[k] - (float)hi);
      }
    }
  }
  f32x16_t o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  float m = -INFINITY, l = 0.f;
  const __half* kc = p.kcache + (size_t)g * p.max_ctx * HD;
  const __half* vc = p.vcache + (size_t)g * p.max_ctx * HD;
  // Staging, rows past the block's last query as zeros (their V would otherwise meet probability
  // 0 as garbage). K: thread t moves 16 bytes (8 dims) of key row t / (HD / 8) per pass. V: thread
  // t loads dims 2 dp, 2 dp + 1 (dp = t % (HD / 2)) of KPT consecutive keys, one dword each (a
  // wave reads whole rows), and stores them as KPT keys of V^T rows 2 dp and 2 dp + 1 (8-byte
  // stores, KPT / 4 a row; storing V^T one half at a time put 16 lanes on one bank).
  constexpr int SEG = HD / 8, PASS = 256 / SEG, NPASS = 32 / PASS;
  const int srow = tid / SEG, sd = (tid % SEG) * 8;
  constexpr int KPT = HD / 16;                       // keys per thread for V (4, 8, 16)
  const int dp = tid % (HD / 2), kg = tid / (HD / 2);

  // The next tile's rows are loaded into registers while the waves work on this one, and stored
  // to the other buffer at the top of the next pass: one barrier a tile, and the loads' latency
  // behind the MFMAs. A wave that passed a barrier has finished reading the buffer that barrier's
  // pass did not fill, so the store two passes later is safe.
  uint4 kr[NPASS];
  uint32_t vr[KPT];
  // Buffer loads over the kv head's cache rows; a key past the block's last query gets an offset
  // past the range (zeros, no memory access), so the loads carry no branches.
  const uint32_t head_bytes = (uint32_t)p.max_ctx * HD * 2u, kOut = 0x40000000u;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kc, head_bytes), rv = make_rsrc(vc, head_bytes);
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int kp = t0 + ps * PASS + srow;
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(
          rk, kp <= block_last ? ((uint32_t)kp * HD + sd) * 2u : kOut, 0, 0);
      kr[ps] = make_uint4(a[0], a[1], a[2], a[3]);
    }
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int kp = t0 + kg * KPT + i;
      vr[i] = __builtin_amdgcn_raw_buffer_load_b32(rv, kp <= block_last ? ((uint32_t)kp * HD + 2 * dp) * 2u : kOut, 0, 0);
    }
  };
  load_tile(0);
  for (int t0 = 0, buf = 0; t0 <= block_last; t0 += 32, buf ^= 1) {
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) *(uint4*)(ks[buf] + (ps * PASS + srow) * KS + sd) = kr[ps];
    {
      uint32_t lo[KPT / 2], hi[KPT / 2];             // rows 2 dp and 2 dp + 1, two keys a dword
#pragma unroll
      for (int i = 0; i < KPT / 2; ++i) {
        lo[i] = __builtin_amdgcn_perm(vr[2 * i + 1], vr[2 * i], 0x05040100u);
        hi[i] = __builtin_amdgcn_perm(vr[2 * i + 1], vr[2 * i], 0x07060302u);
      }
      _Float16* v0 = vt[buf] + (2 * dp) * VS + kg * KPT;
#pragma unroll
      for (int i = 0; i < KPT / 2; i += 2) {
        *(uint2*)(v0 + 2 * i) = make_uint2(lo[i], lo[i + 1]);
        *(uint2*)(v0 + VS + 2 * i) = make_uint2(hi[i], hi[i + 1]);
      }
    }
    load_tile(t0 + 32);                               // past the block's last key: zeros, no load
    __syncthreads();
    if (t0 > wave_last) continue;                     // every key past this wave's queries

    // The hi and lo planes' products in two accumulators: two independent MFMA chains.
    f32x16_t s, sl;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = sl[e] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const half8_t a = *(const half8_t*)(ks[buf] + j * KS + 16 * c + 8 * h);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qh[c], s, 0, 0, 0);
      sl = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ql[c], sl, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] += sl[e];
    // Causal mask (only a tile that reaches past the wave's first query needs it; the columns
    // that hold no query are never stored) and the column's running max over its keys.
    if (t0 + 31 > wave_first) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int kp = t0 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (kp > qpos) s[e] = -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // The running max moves only when this tile's exceeds it by more than 8, so a probability
    // stays below e^8 (~2981: its fp16 hi plane finite, hi + lo still ~22 bits) and the output
    // is rescaled in few tiles; o / l is the same whichever max they share.
    const bool raise = mx > m + 8.f;
    const float mn = raise ? mx : m;
    const float corr = raise ? __expf(m - mn) : 1.f;
    float ps_ = 0.f;
    half8_t ph[2], pl[2];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      // A masked score gives exp(-inf) = 0: the running max of a column that holds a query is
      // finite from its first tile on (key 0 is never masked for it); a column that holds none
      // may turn NaN, but it only reaches its own output column, which is never stored.
      const float pe = __expf(s[e] - mn);
      ps_ += pe;
      const _Float16 hi = (_Float16)pe;
      ph[e >> 3][e & 7] = hi;
      pl[e >> 3][e & 7] = (_Float16)(pe - (float)hi);
    }
    ps_ += __shfl_xor(ps_, 32, 64);
    l = l * corr + ps_;
    if (__any(raise)) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= corr;
    }
    m = mn;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        // V^T rows dt * 32 + j, keys 16 kh + 4h .. + 3 and 16 kh + 8 + 4h .. + 3.
        const _Float16* vr0 = vt[buf] + (dt * 32 + j) * VS + 16 * kh + 4 * h;
        const uint2 lo4 = *(const uint2*)vr0, hi4 = *(const uint2*)(vr0 + 8);
        const uint4 av = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
        const half8_t a = __builtin_bit_cast(half8_t, av);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ph[kh], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pl[kh], o[dt], 0, 0, 0);
      }
    }
  }
  if (!cvalid) return;
  const float inv = 1.0f / l;
  float* dst = p.out + (size_t)qrow * p.n_head * HD + (size_t)head * HD;
  const float* gate = p.qkv + (size_t)qrow * p.ldq + (size_t)head * 2 * HD + HD;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      const int d0 = dt * 32 + 8 * a4 + 4 * h;
      float4 v = make_float4(o[dt][4 * a4] * inv, o[dt][4 * a4 + 1] * inv, o[dt][4 * a4 + 2] * inv, o[dt][4 * a4 + 3] * inv);
      if (p.gated) {
        const float4 gv = *(const float4*)(gate + d0);
        v = make_float4(v.x * sigmoidf_(gv.x), v.y * sigmoidf_(gv.y), v.z * sigmoidf_(gv.z), v.w * sigmoidf_(gv.w));
      }
      *(float4*)(dst + d0) = v;
    }
}

int launch_attn_prefill(const AttnPrefillParams& p, hipStream_t s) {
  TRX_CHECK(p.n_kv >= 1 && p.n_head % p.n_kv == 0 && p.n_head / p.n_kv <= 64 && p.R >= 1 &&
            p.p0 + p.R <= p.max_ctx, TRX_E_INVALID, "prefill attention: bad geometry");
  // A kv head's cache rows lie below the offset the loads use for keys past a block's queries.
  TRX_CHECK((size_t)p.max_ctx * p.hd * 2 < 0x40000000u, TRX_E_INVALID, "prefill attention: context %d too long",
            p.max_ctx);
  const int rep = p.n_head / p.n_kv, QT = 64 / rep;
  if ((p.hd == 64 || p.hd == 128 || p.hd == 256) && rep <= 32) {
    const dim3 mgrid(cdiv(p.R, 4 * (32 / rep)), p.n_kv);
    if (p.hd == 64) hipLaunchKernelGGL((attn_prefill_mfma_kernel<64>), mgrid, dim3(256), 0, s, p);
    else if (p.hd == 128) hipLaunchKernelGGL((attn_prefill_mfma_kernel<128>), mgrid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((attn_prefill_mfma_kernel<256>), mgrid, dim3(256), 0, s, p);
    TRX_LAUNCHED();
    return TRX_OK;
  }
  const dim3 grid(cdiv(p.R, QT), p.n_kv);
  if (p.hd == 64) hipLaunchKernelGGL((attn_prefill_kernel<64, 32>), grid, dim3(256), 0, s, p);
  else if (p.hd == 128) hipLaunchKernelGGL((attn_prefill_kernel<128, 32>), grid, dim3(256), 0, s, p);
  else if (p.hd == 256) hipLaunchKernelGGL((attn_prefill_kernel<256, 16>), grid, dim3(256), 0, s, p);
  else TRX_CHECK(false, TRX_E_INVALID, "prefill attention: head_dim %d unsupported", p.hd);
  TRX_LAUNCHED();
  return TRX_OK;
}

// Gated DeltaNet over R positions ---------------------------------------------------------------

// Conv + SiLU (+ the L2 norm of q/k heads) of every position: one block per (head-sized channel
// segment, position). in(rho, c) is the raw projection of chunk row rho, or for rho < 0 the
// state's row Kc - 1 + rho (oldest first).
__global__ void dn_conv_rows_kernel(DnRowsParams p) {
  __shared__ float red[8];
  const int seg = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  const int c = seg * p.hk + t;
  float acc = 0.f;
  for (int i = 0; i < p.Kc; ++i) {
    const int rho = r - (p.Kc - 1) + i;
    const float x = rho >= 0 ? p.io[(size_t)rho * p.ld_io + c] : p.conv_state[(size_t)(p.Kc - 1 + rho) * p.C + c];
    acc += p.taps[c * p.Kc + i] * x;
  }
  float y = silu(acc);
  if (c < 2 * p.nq) {
    const float ss = wave_sum(y * y);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < (blockDim.x + 63) / 64; ++i) tot += red[i];
    y = y / fmaxf(sqrtf(tot), p.eps);
  }
  p.conv_out[(size_t)r * p.C + c] = y;
}

// The window after the chunk: the last Kc - 1 raw rows (older state rows when R < Kc - 1).
__global__ void dn_conv_tail_kernel(DnRowsParams p) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= p.C) return;
  float keep[8];
  for (int i = 0; i < p.Kc - 1; ++i) {
    const int rho = p.R - (p.Kc - 1) + i;
    keep[i] = rho >= 0 ? p.io[(size_t)rho * p.ld_io + c] : p.conv_state[(size_t)(p.Kc - 1 + rho) * p.C + c];
  }
  for (int i = 0; i < p.Kc - 1; ++i) p.conv_state[(size_t)i * p.C + c] = keep[i];
}

// The recurrence of one value head over the chunk, one pass of state rows per block (8 rows at
// HK = 128, 16 at 64; 256 threads): a row's HK columns over HK/4 lanes (a float4 each), row sums by
// DPP. First every block computes its head's decay and beta gates of all the chunk's positions at
// once (into LDS), so the serial loop carries only the state's arithmetic; each position's k, q
// and v are loaded kScanAhead positions ahead. The per-position arithmetic is
// dn_recur_fixed_kernel's.
constexpr int kScanAhead = 4;          // positions whose inputs are in flight ahead of the scan
constexpr int kScanRMax = 8192;        // chunk positions whose gates fit the LDS (64 KB)
template <int HK>
constexpr int scan_rows() { return 4 * (64 / (HK / 4)); }
// Sum over a row's LPR lanes (16 or 32, aligned), every lane getting it: DPP within each 16-lane
// row, then one lane swap between the two rows of a 32-lane row.
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
  static_assert(LPR == 16 || LPR == 32, "row width");
  v = row16_sum(v);
  if (LPR == 32) v += __shfl_xor(v, 16, 64);
  return v;
}
template <int HK>
__global__ __launch_bounds__(256) void dn_scan_kernel(DnRowsParams p) {
  constexpr int LPR = HK / 4, RPW = 64 / LPR, RB = scan_rows<HK>();
  extern __shared__ float gates[];      // [R] decay, then [R] beta
  const int h = blockIdx.x, rb = blockIdx.y, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int sub = lane / LPR, c4 = lane % LPR;
  const int nk = p.nk, kh = h % nk, hv = p.hv;
  const int jr = rb * RB + w * RPW + sub;
  float4* S = (float4*)(p.S + (size_t)h * hv * HK);
  float4 sv = S[jr * LPR + c4];
  const float Ah = p.A[h], dth = p.dt[h];
  for (int r = t; r < p.R; r += 256) {
    const float a = p.ba[(size_t)r * 2 * p.nv + p.nv + h] + dth;
    const float sp = a > 20.f ? a : log1pf(expf(a));
    gates[r] = expf(sp * Ah);
    gates[p.R + r] = sigmoidf_(p.ba[(size_t)r * 2 * p.nv + h]);
  }
  const float qs = 1.0f / sqrtf((float)HK);
  auto ld = [&](int r, float4& k4, float4& q4, float& vj) {
    const float* cr = p.conv_out + (size_t)r * p.C;
    k4 = *(const float4*)(cr + p.nq + kh * HK + 4 * c4);
    q4 = *(const float4*)(cr + kh * HK + 4 * c4);
    vj = cr[2 * p.nq + h * hv + jr];
  };
  // A ring of the next kScanAhead positions' inputs in registers: a position's loads are issued
  // kScanAhead positions before it is used, so their latency is covered by that many steps of the
  // recurrence (one step is shorter than a memory round trip).
  float4 k4[kScanAhead], q4[kScanAhead];
  float vj[kScanAhead];
#pragma unroll
  for (int u = 0; u < kScanAhead; ++u)
    if (u < p.R) ld(u, k4[u], q4[u], vj[u]);
  __syncthreads();
  for (int r0 = 0; r0 < p.R; r0 += kScanAhead)
#pragma unroll
  for (int u = 0; u < kScanAhead; ++u) {
    const int r = r0 + u;
    if (r >= p.R) break;
    const float4 ck = k4[u], cq = q4[u];
    const float cv = vj[u];
    if (r + kScanAhead < p.R) ld(r + kScanAhead, k4[u], q4[u], vj[u]);
    const float decay = gates[r], beta = gates[p.R + r];
    float4 s4 = make_float4(sv.x * decay, sv.y * decay, sv.z * decay, sv.w * decay);
    const float dot = row_sum<LPR>((s4.x * ck.x + s4.y * ck.y) + (s4.z * ck.z + s4.w * ck.w));
    const float delta = (cv - dot) * beta;
    s4 = make_float4(s4.x + delta * ck.x, s4.y + delta * ck.y, s4.z + delta * ck.z, s4.w + delta * ck.w);
    sv = s4;
    const float oq = row_sum<LPR>((s4.x * cq.x + s4.y * cq.y) + (s4.z * cq.z + s4.w * cq.w));
    if (c4 == 0) p.o_raw[(size_t)r * p.nv * hv + (size_t)h * hv + jr] = oq * qs;
  }
  S[jr * LPR + c4] = sv;
}

// Gated RMSNorm of every (position, value head), into the grouped output order.
__global__ void dn_gnorm_rows_kernel(DnRowsParams p) {
  __shared__ float red[16];
  const int h = blockIdx.x, r = blockIdx.y, t = threadIdx.x, hv = p.hv;
  const float* o = p.o_raw + (size_t)r * p.nv * hv + (size_t)h * hv;
  float ss = 0.f;
  for (int i = t; i < hv; i += blockDim.x) ss += o[i] * o[i];
  ss = block_sum(ss, red);
  const float rr = 1.0f / sqrtf(ss / (float)hv + p.eps);
  const int gpos = (h % p.nk) * (p.nv / p.nk) + h / p.nk;
  const float* z = p.io + (size_t)r * p.ld_io + p.C + (size_t)h * hv;
  for (int i = t; i < hv; i += blockDim.x)
    p.out[(size_t)r * p.nv * hv + (size_t)gpos * hv + i] = o[i] * rr * p.norm_w[i] * silu(z[i]);
}

int launch_dn_rows(const DnRowsParams& p, hipStream_t s) {
  const int rb = p.hk == 128 ? scan_rows<128>() : scan_rows<64>();
  TRX_CHECK(p.R >= 1 && p.R <= kScanRMax && p.hk <= 256 && p.C % p.hk == 0 && p.Kc >= 1 && p.Kc <= 9 &&
            p.nv % p.nk == 0 && (p.hk == 64 || p.hk == 128) && p.hv % rb == 0 && p.hv <= 1024, TRX_E_INVALID,
            "prefill DeltaNet: unsupported geometry hk=%d hv=%d Kc=%d (chunk %d)", p.hk, p.hv, p.Kc, p.R);
  hipLaunchKernelGGL(dn_conv_rows_kernel, dim3(p.C / p.hk, p.R), dim3(p.hk), 0, s, p);
  TRX_LAUNCHED();
  if (p.Kc > 1) {
    hipLaunchKernelGGL(dn_conv_tail_kernel, dim3(cdiv(p.C, 256)), dim3(256), 0, s, p);
    TRX_LAUNCHED();
  }
  const dim3 sg(p.nv, p.hv / rb);
  const size_t lds = (size_t)2 * p.R * sizeof(float);
  if (p.hk == 128) hipLaunchKernelGGL(dn_scan_kernel<128>, sg, dim3(256), lds, s, p);
  else hipLaunchKernelGGL(dn_scan_kernel<64>, sg, dim3(256), lds, s, p);
  TRX_LAUNCHED();
  hipLaunchKernelGGL(dn_gnorm_rows_kernel, dim3(p.nv, p.R), dim3(std::min(256, p.hv)), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

__global__ void prefill_ctl_kernel(int* ctl_pos, int* cur_tok, const int* fed, int p_last) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    *ctl_pos = p_last;
    *cur_tok = fed[p_last];
  }
}

int launch_prefill_ctl(int* ctl_pos, int* cur_tok, const int* fed, int p_last, hipStream_t s) {
  hipLaunchKernelGGL(prefill_ctl_kernel, dim3(1), dim3(64), 0, s, ctl_pos, cur_tok, fed, p_last);
  TRX_LAUNCHED();
  return TRX_OK;
}

}  // namespace trx

using namespace trx;

#define TRX_API extern "C" __attribute__((visibility("default")))

TRX_API int trx_gemm_ternary_f32(const uint8_t* rows, int kind, int M, int K, const float* x, int n,
                                 const float* norm_w, float eps, float* y, int epilogue, void* workspace,
                                 trx_stream_t s) {
  TRX_CHECK(rows && x && y && workspace && n >= 1, TRX_E_INVALID, "trx_gemm_ternary_f32: bad arguments");
  TRX_CHECK(epilogue == TRX_EPI_STORE || epilogue == TRX_EPI_RESID || epilogue == TRX_EPI_SWIGLU, TRX_E_INVALID,
            "trx_gemm_ternary_f32: unknown epilogue %d", epilogue);
  TRX_CHECK(K >= kGroup && K % kGroup == 0 && M >= 1, TRX_E_INVALID, "trx_gemm_ternary_f32: M=%d K=%d", M, K);
  const int row_bytes = kind == TRX_KIND_Q8 ? kBeat * cdiv(K / 32, 16) + K : row_geom(kind, K).row_bytes;
  const int code_off = kind == TRX_KIND_Q8 ? kBeat * cdiv(K / 32, 16) : row_geom(kind, K).code_off;
  _Float16* xh = (_Float16*)workspace;
  _Float16* xl = xh + (size_t)n * K;
  float* xs = (float*)(xl + (size_t)n * K);
  PrepParams pp = {};
  pp.x = x;
  pp.ldx = K;
  pp.K = K;
  pp.R = n;
  pp.norm_w = norm_w;
  pp.eps = eps;
  pp.xh = xh;
  pp.xl = xl;
  pp.xs = xs;
  int rc;
  if ((rc = launch_prep(pp, (hipStream_t)s))) return rc;
  GemmParams g = {};
  g.W = rows;
  g.w_bytes = (uint32_t)std::min<size_t>((size_t)M * row_bytes + 16, 0xFFFFFFF0u);
  g.kind = kind;
  g.M = M;
  g.K = K;
  g.row_bytes = row_bytes;
  g.code_off = code_off;
  g.xh = xh;
  g.xl = xl;
  g.xs = xs;
  g.R = n;
  g.epi = epilogue == TRX_EPI_STORE ? GM_STORE : epilogue == TRX_EPI_RESID ? GM_RESID : GM_SWIGLU;
  g.y = y;
  g.ldy = epilogue == TRX_EPI_SWIGLU ? M / 2 : M;
  return launch_gemm(g, (hipStream_t)s);
}
