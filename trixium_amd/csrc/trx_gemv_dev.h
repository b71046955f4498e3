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
// Mapping. A lane owns one half-group (64 columns: 13 trit5 code bytes, or 16 2-bit code bytes)
// at a time; LPR lanes (power of two dividing the 2G half-groups, <= 64) cover LPR half-groups of
// R rows (an "item"), and step through the 2G/LPR slots of those rows. The x values of a
// half-group are held in 33 registers in a "dot-ready" form built once per block in LDS, and
// reused across the R rows. The codes of the next item are loaded while the current one is
// computed. No MFMA: the path is a bandwidth-bound GEMV.
//
// Decode. trit5: every code byte b is looked up in an LDS table giving its base-3 digits d0..d3
// as byte lanes (fed to v_dot4 against the int8 planes of x) and d4 (two bytes' d4 are paired by
// one v_perm and fed to v_dot2 against int16 x). 2-bit: every code byte gives its four 2-bit
// codes as byte lanes. The table is replicated 32x (64x for the 4-byte 2-bit entries) so the
// lanes of a wave hit distinct LDS banks; the entry address (b << 8 | lane copy) is formed by one
// v_perm_b32. Since sum (code-1)x = sum code*x - sum x, codes are used as unsigned digits and
// the half-group's sum of x is subtracted once per row.

#pragma once

#include "trx_internal.h"

namespace trx {

enum { MODE_F32 = 0, MODE_EXACT = 1, MODE_GSUM = 2 };

constexpr int kLutBytes = 65536;    // 256 entries x 256 bytes
constexpr int kMaxXRounds = 3;      // x staged in rounds of 8 columns per thread: K <= 24576
#ifndef GEMV_PRE
#define GEMV_PRE 1                  // ring items fetched before x arrives (capped at NB - 1)
#endif
constexpr int kDynLds = 160 * 1024 - kLutBytes - 512;   // LDS left for the dynamic part
constexpr int kXStride = 36;        // dwords per half-group in the dot-ready layout
constexpr int kXDwords5 = 33;       // trit5: 13 x (hi, lo) + 7 d4 pairs
constexpr int kXDwords2 = 32;       // 2-bit: 16 x (hi, lo)

struct GemvParams {
  const uint8_t* W;
  uint32_t w_bytes;       // bytes addressable from W (tensor + 32-byte tail)
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
  const int* gate_pos;    // when set: the kernel does nothing while *gate_pos < *gate_from
  const int* gate_from;
};


typedef short s2_t __attribute__((ext_vector_type(2)));

template <int FMT, int R>
struct ItemBuf {
  uint32_t cd[R][4];
  uint32_t sc[R];
};

constexpr int kGemvThreads = 1024;

// Decode table replicated into LDS: 4096 chunks of 16 bytes, 16 chunks per entry. Entry b holds
// the digits of code byte b, computed with no memory traffic: trit5 digit k = floor(b / 3^k)
// mod 3 (the reference's decode, model/bons.py:125-130), 2-bit code k = (b >> 2k) & 3.
template <bool T5>
__device__ __forceinline__ void fill_lut(uint8_t* lut) {
  uint4* l = (uint4*)lut;
  for (int i = threadIdx.x; i < kLutBytes / 16; i += blockDim.x) {
    const uint32_t b = (uint32_t)i >> 4;
    uint4 v;
    if (T5) {
      const uint32_t b1 = b / 3, b2 = b1 / 3, b3 = b2 / 3, b4 = b3 / 3;
      const uint32_t lo = (b - 3 * b1) | ((b1 - 3 * b2) << 8) | ((b2 - 3 * b3) << 16) | ((b3 - 3 * b4) << 24);
      const uint32_t hi = b4 - 3 * (b4 / 3);
      v = make_uint4(lo, hi, lo, hi);
    } else {
      const uint32_t c = (b & 3u) | (((b >> 2) & 3u) << 8) | (((b >> 4) & 3u) << 16) | (((b >> 6) & 3u) << 24);
      v = make_uint4(c, c, c, c);
    }
    l[i] = v;
  }
}

// One block's share of a GEMV: rows are dealt to the waves of blocks bid = 0..nblk-1.
// R: rows per item; NB: items held in registers (NB - 1 are in flight while one is computed);
// SW: SwiGLU epilogue (rows [0,F) gate, [F,2F) up; R/2 outputs per item).
// FUSED: the block runs inside a multi-phase kernel: the decode table is already in `lut`, the
// whole ring is fetched before `wait()` (the grid barrier that makes x ready), and x, the
// residual and the outputs are exchanged through agent-scope accesses.
// Uses `lut` (kLutBytes) and `smem` (lds_bytes(K, G)) and every thread of a 1024-thread block.
template <int FMT, int MODE, int R, int NB, bool SW, bool FUSED = false, class Wait = NoWait>
__device__ __forceinline__ void gemv_body(const GemvParams& p, uint8_t* lut_mem, uint8_t* smem, int bid,
                                          int nblk, Wait wait = Wait{}) {
  constexpr int kThreads = kGemvThreads;
  constexpr int kWaves = kThreads / 64;
  constexpr bool T5 = (FMT == TRX_KIND_TERNARY5);
  constexpr int NPL = (MODE == MODE_F32) ? 2 : 1;              // int8 planes of x
  // First column of the second half-group of a group (trit5 bytes 13..25 start at column 65).
  constexpr int kHalfCol = T5 ? 65 : 64;
  const uint8_t* lut = lut_mem;
  uint32_t* xl = (uint32_t*)smem;                              // 2G * kXStride dwords
  int16_t* stage = (int16_t*)(xl + 2 * p.G * kXStride);        // K int16
  float* gsig = (float*)(stage + p.K);                         // G: sigma_g
  int32_t* usum = (int32_t*)(gsig + p.G);                      // 2G: sum of q over a half-group
  float* red = (float*)(usum + 2 * p.G);                       // 16

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int LPR = p.LPR;
  const int rg = lane / LPR, lg = lane - rg * LPR;
  const int RG = 64 / LPR;
  const int first = (bid * kWaves + wave) * RG + rg;
  const int stride = nblk * kWaves * RG;
  const int NSLOT = p.NSLOT;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.W, p.w_bytes);
  // v_perm sources: byte 0 of the address comes from the lane-copy word (selector 0), byte 1
  // from code byte k of the code word (selector 4 + k), bytes 2..3 are zero (selector 0x0c).
  const uint32_t lcopy = T5 ? (uint32_t)((lane & 31) << 3) : (uint32_t)(lane << 2);
  constexpr bool swiglu = SW;
  // Rows of batch bt: plain, bt*R + r; SwiGLU, gate rows bt*R/2 + r and up rows F + bt*R/2 + r.
  const int rows_per_batch = swiglu ? R / 2 : R;
  const uint32_t rb = (uint32_t)p.row_bytes;
  const uint32_t up_off = swiglu ? (uint32_t)p.swiglu_F * rb : 0u;

  auto out_index = [&](int bt, int r) -> int { return bt * rows_per_batch + (swiglu ? (r % (R > 1 ? R / 2 : 1)) : r); };
  auto row_offset = [&](int bt, int r) -> uint32_t {
    const int o = out_index(bt, r);
    if (o >= p.n_out) return p.w_bytes;                          // out of range: loads read 0
    const uint32_t base = (uint32_t)(bt * rows_per_batch) * rb;
    if (!swiglu) return base + (uint32_t)r * rb;
    return (r < R / 2) ? base + (uint32_t)r * rb : base + up_off + (uint32_t)(r - R / 2) * rb;
  };
  // Byte offset of half-group u inside a row's code area.
  auto unit_off = [&](int u) -> uint32_t {
    return T5 ? (uint32_t)(kTrit5GroupBytes * (u >> 1) + 13 * (u & 1)) : (uint32_t)(16 * u);
  };
  auto load_item = [&](ItemBuf<FMT, R>& b, int bt, int sl) {
    const int u = sl * LPR + lg;
    const uint32_t uoff = p.code_off + unit_off(u);
    const uint32_t soff = 2u * (uint32_t)(u >> 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t ro = row_offset(bt, r);
      // trit5: the 16 bytes at the half-group's own (unaligned) offset; the last 3 may be the
      // next half-group's or the row padding (the tensor has a 32-byte tail).
      auto a = __builtin_amdgcn_raw_buffer_load_b128(rs, ro + uoff, 0, 0);
      b.cd[r][0] = a[0]; b.cd[r][1] = a[1]; b.cd[r][2] = a[2]; b.cd[r][3] = a[3];
      b.sc[r] = __builtin_amdgcn_raw_buffer_load_b16(rs, ro + soff, 0, 0);
    }
  };

  // Items of this row group in order: batch bt = first + k*stride, slot sl = 0..NSLOT-1.
  auto advance = [&](int& bt, int& sl) {
    if (++sl == NSLOT) { sl = 0; bt += stride; }
  };

  // The codes do not depend on x. Loads are issued unconditionally (an item past the end reads
  // through the descriptor's bounds check, which returns zeros without touching memory), so the
  // number of loads in flight is static and every wait counts exactly the loads it needs.
  // Standalone, x is fetched first (weight loads issued ahead of it would delay it in the memory
  // pipeline) and kPre items follow; fused, the whole ring goes out before the grid barrier.
  constexpr int kPre = FUSED ? NB - 1 : ((GEMV_PRE < NB - 1) ? GEMV_PRE : NB - 1);
  ItemBuf<FMT, R> buf[NB];
  int lbt = first, lsl = 0;            // next item to fetch
  if (FUSED) {
#pragma unroll
    for (int b = 0; b < kPre; ++b) {
      load_item(buf[b], lbt, lsl);
      advance(lbt, lsl);
    }
    wait();
  }

  // x (and the RMSNorm gain) of this thread's 8 columns per round come first: they gate the
  // prologue, and loads issued after the weight stream would queue behind it.
  const int rounds = (p.K + kThreads * 8 - 1) / (kThreads * 8);
  float xv[kMaxXRounds][8], wv[kMaxXRounds][8];
  uint2 x8v[kMaxXRounds];
#pragma unroll
  for (int rd = 0; rd < kMaxXRounds; ++rd) {
    const int c0 = (rd * kThreads + tid) * 8;
#pragma unroll
    for (int k = 0; k < 8; ++k) { xv[rd][k] = 0.f; wv[rd][k] = 1.f; }
    x8v[rd] = make_uint2(0, 0);
    if (rd < rounds && c0 < p.K) {
      if (MODE == MODE_F32) {
        if (FUSED) {
#pragma unroll
          for (int k = 0; k < 8; ++k) xv[rd][k] = ld_vec<true>(p.x + c0 + k);
        } else {
          const float4 a = *(const float4*)(p.x + c0), b = *(const float4*)(p.x + c0 + 4);
          xv[rd][0] = a.x; xv[rd][1] = a.y; xv[rd][2] = a.z; xv[rd][3] = a.w;
          xv[rd][4] = b.x; xv[rd][5] = b.y; xv[rd][6] = b.z; xv[rd][7] = b.w;
        }
        if (p.norm_w) {
          const float4 c = *(const float4*)(p.norm_w + c0), d = *(const float4*)(p.norm_w + c0 + 4);
          wv[rd][0] = c.x; wv[rd][1] = c.y; wv[rd][2] = c.z; wv[rd][3] = c.w;
          wv[rd][4] = d.x; wv[rd][5] = d.y; wv[rd][6] = d.z; wv[rd][7] = d.w;
        }
      } else {
        x8v[rd] = *(const uint2*)(p.x8 + c0);
      }
    }
  }

  if (!FUSED) {
#pragma unroll
    for (int b = 0; b < kPre; ++b) {
      load_item(buf[b], lbt, lsl);
      advance(lbt, lsl);
    }
    fill_lut<T5>(lut_mem);
  }

  // x -> int16 per group (float mode, sigma_g = amax/32767) or the int8 vector itself (exact
  // modes), staged in LDS, with the sum of the staged values over every half-group.
  {
    // The block sum of x^2 also tells every wave that the whole block's x has arrived.
    float rinv = 1.0f;
    {
      float ss = 0.f;
      if (MODE == MODE_F32) {
#pragma unroll
        for (int rd = 0; rd < kMaxXRounds; ++rd)
#pragma unroll
          for (int k = 0; k < 8; ++k) ss += xv[rd][k] * xv[rd][k];
      } else {
#pragma unroll
        for (int rd = 0; rd < kMaxXRounds; ++rd) ss += (float)(x8v[rd].x & 1u) + (float)(x8v[rd].y & 1u);
      }
      ss = block_sum(ss, red);
      if (MODE == MODE_F32 && p.norm_w) rinv = 1.0f / sqrtf(ss / (float)p.K + p.eps);
    }
    // x has arrived: the rest of the ring goes out now and lands during the staging below.
#pragma unroll
    for (int b = kPre; b < NB - 1; ++b) {
      load_item(buf[b], lbt, lsl);
      advance(lbt, lsl);
    }
    // 16 threads per group, 8 columns each; every thread runs the same number of rounds.
#pragma unroll
    for (int rd = 0; rd < kMaxXRounds; ++rd) {
      if (rd >= rounds) break;
      const int c0 = (rd * kThreads + tid) * 8;
      const bool live = c0 < p.K;
      int q[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      float am = 0.f;
      if (MODE == MODE_F32) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          v[k] = p.norm_w ? xv[rd][k] * rinv * wv[rd][k] : xv[rd][k];
          am = fmaxf(am, fabsf(v[k]));
        }
        am = row16_max(am);               // the 16 lanes of the group
        const float inv = am > 0.f ? 32767.0f / am : 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = (int)rintf(v[k] * inv);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          q[k] = (int)(int8_t)(x8v[rd].x >> (8 * k));
          q[k + 4] = (int)(int8_t)(x8v[rd].y >> (8 * k));
        }
      }
      int s0 = 0, s1 = 0;
      const int lc = c0 & (kGroup - 1);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (lc + k < kHalfCol) s0 += q[k];
        else s1 += q[k];
      }
      if (live) {
        uint4 pk;
        pk.x = (uint32_t)(uint16_t)q[0] | ((uint32_t)(uint16_t)q[1] << 16);
        pk.y = (uint32_t)(uint16_t)q[2] | ((uint32_t)(uint16_t)q[3] << 16);
        pk.z = (uint32_t)(uint16_t)q[4] | ((uint32_t)(uint16_t)q[5] << 16);
        pk.w = (uint32_t)(uint16_t)q[6] | ((uint32_t)(uint16_t)q[7] << 16);
        *(uint4*)(stage + c0) = pk;
      }
      s0 = row16_sum_i(s0);
      s1 = row16_sum_i(s1);
      if (live && (tid & 15) == 0) {
        gsig[c0 >> 7] = am / 32767.0f;
        usum[2 * (c0 >> 7)] = s0;
        usum[2 * (c0 >> 7) + 1] = s1;
      }
    }
  }
  __syncthreads();

  // Dot-ready layout of every half-group u = 2g + h.
  {
    const int per = T5 ? kXDwords5 : kXDwords2;
    for (int i = tid; i < 2 * p.G * per; i += kThreads) {
      const int u = i / per, j = i - u * per;
      const int16_t* xs = stage + (u >> 1) * kGroup;
      const int h = u & 1;
      uint32_t v = 0;
      if (j < (T5 ? 26 : 32)) {
        const int byte = (T5 ? 13 : 16) * h + (j >> 1), plane = j & 1;
        const int c0 = T5 ? 5 * byte : 4 * byte;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int c = c0 + k;
          const int q = (c < kGroup) ? xs[c] : 0;
          const uint32_t b8 = (NPL == 2) ? (plane == 0 ? (uint32_t)((q >> 8) & 0xFF) : (uint32_t)(q & 0xFF))
                                         : (plane == 0 ? (uint32_t)(q & 0xFF) : 0u);
          v |= b8 << (8 * k);
        }
      } else {
        // d4 pair: unit bytes 2pr and 2pr+1 (the 13th byte has no partner).
        const int pr = j - 26;
        const int ba = 13 * h + 2 * pr, bb = ba + 1;
        const int ca = 5 * ba + 4, cb = 5 * bb + 4;
        const int qa = ca < kGroup ? xs[ca] : 0;
        const int qb = (2 * pr + 1 < 13 && cb < kGroup) ? xs[cb] : 0;
        v = (uint32_t)(uint16_t)qa | ((uint32_t)(uint16_t)qb << 16);
      }
      xl[u * kXStride + j] = v;
    }
  }
  __syncthreads();

  uint32_t xr[T5 ? kXDwords5 : kXDwords2];
  auto load_x = [&](int sl) {
    const int u = sl * LPR + lg;
    const uint4* src = (const uint4*)(xl + u * kXStride);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint4 t = src[i];
      xr[4 * i] = t.x; xr[4 * i + 1] = t.y; xr[4 * i + 2] = t.z; xr[4 * i + 3] = t.w;
    }
    if (T5) xr[32] = xl[u * kXStride + 32];
  };

  float facc[R];
  long long iacc[R];
  unsigned long long best = 0;   // argmax epilogue: this lane's best (ordered value, ~row) key
#pragma unroll
  for (int r = 0; r < R; ++r) { facc[r] = 0.f; iacc[r] = 0; }

  auto compute_item = [&](const ItemBuf<FMT, R>& b, int bt, int sl) {
    const int u = sl * LPR + lg;
    const float sig = (MODE == MODE_F32) ? gsig[u >> 1] : 0.f;
    const int usx = usum[u];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int accH = 0, acc4 = 0;
      unsigned accL = 0;
      if (T5) {
        uint32_t d4prev = 0;
#pragma unroll
        for (int i = 0; i < 13; ++i) {
          const uint32_t sel = 0x0c0c0400u | ((uint32_t)(i & 3) << 8);
          const uint32_t addr = __builtin_amdgcn_perm(b.cd[r][i >> 2], lcopy, sel);
          const uint64_t e64 = *(const uint64_t*)__builtin_assume_aligned(lut + addr, 8);
          const uint32_t elo = (uint32_t)e64, ehi = (uint32_t)(e64 >> 32);
          accH = __builtin_amdgcn_sdot4((int)elo, (int)xr[2 * i], accH, false);
          if (NPL == 2) accL = __builtin_amdgcn_udot4(elo, xr[2 * i + 1], accL, false);
          if ((i & 1) || i == 12) {
            // [d4 of byte i-1, d4 of byte i] (or [d4 of byte 12, 0]) as int16 halves, against
            // the x pair of the two bytes.
            const uint32_t pair = (i & 1) ? __builtin_amdgcn_perm(ehi, d4prev, 0x0c040c00u) : ehi;
            acc4 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2_t, pair),
                                          __builtin_bit_cast(s2_t, xr[26 + (i >> 1)]), acc4, false);
          } else {
            d4prev = ehi;
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t sel = 0x0c0c0400u | ((uint32_t)(i & 3) << 8);
          const uint32_t addr = __builtin_amdgcn_perm(b.cd[r][i >> 2], lcopy, sel);
          const uint32_t e = *(const uint32_t*)__builtin_assume_aligned(lut + addr, 4);
          accH = __builtin_amdgcn_sdot4((int)e, (int)xr[2 * i], accH, false);
          if (NPL == 2) accL = __builtin_amdgcn_udot4(e, xr[2 * i + 1], accL, false);
        }
      }
      const int S = (NPL == 2) ? (accH << 8) + (int)accL + acc4 - usx : accH + acc4 - usx;
      if (MODE == MODE_F32) {
        const float s = __half2float(__ushort_as_half((unsigned short)b.sc[r]));
        facc[r] = fmaf((float)S * sig, s, facc[r]);
      } else {
        // The engine shifts whole-group sums (a right shift floors the sum, not each half): the
        // partner lane (lg ^ 1) holds the other half of the group.
        const int Sg = S + __shfl_xor(S, 1, 64);
        if (MODE == MODE_EXACT) {
          if (!(u & 1)) {
            int m11, e16;
            fp16_split((uint16_t)b.sc[r], m11, e16);
            const long long prod = (long long)Sg * (long long)m11;
            const int sh = e16 + p.B;
            long long c;
            if (sh >= 0) c = prod << sh;
            else c = (-sh >= 63) ? (prod < 0 ? -1 : 0) : (prod >> (-sh));
            iacc[r] += c;
          }
        } else {
          const int o = out_index(bt, r);
          if (o < p.n_out && !(u & 1)) p.yi[(size_t)o * p.G + (u >> 1)] = Sg;
        }
      }
    }
  };

  // Cross-lane reduction of the R row sums over the LPR lanes of the row group, by recursive
  // halving (each step sends half of the remaining values). Afterwards every lane holds the full
  // sum of row `held`; the lanes whose low bits (below the halving bits) are zero store it.
  auto finish_batch = [&](int bt) {
    if (MODE == MODE_GSUM) return;
    int held = 0;
    float fv[R];
    long long iv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) { fv[r] = facc[r]; iv[r] = iacc[r]; }
    bool writer;
    const bool halving = (LPR >= R) && !swiglu;
    if (halving) {
      int o = LPR >> 1;
#pragma unroll
      for (int n = R; n > 1; n >>= 1) {
        const bool up = (lg & o) != 0;
#pragma unroll
        for (int i = 0; i < n / 2; ++i) {
          if (MODE == MODE_F32) {
            const float send = up ? fv[i] : fv[i + n / 2];
            const float keep = up ? fv[i + n / 2] : fv[i];
            fv[i] = keep + __shfl_xor(send, o, 64);
          } else {
            const long long send = up ? iv[i] : iv[i + n / 2];
            const long long keep = up ? iv[i + n / 2] : iv[i];
            iv[i] = keep + __shfl_xor(send, o, 64);
          }
        }
        if (up) held += n / 2;
        o >>= 1;
      }
      for (; o >= 1; o >>= 1) {
        if (MODE == MODE_F32) fv[0] += __shfl_xor(fv[0], o, 64);
        else iv[0] += __shfl_xor(iv[0], o, 64);
      }
      writer = (lg & ((LPR / R) - 1)) == 0;
    } else if (!swiglu) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        for (int o = LPR >> 1; o >= 1; o >>= 1) {
          if (MODE == MODE_F32) fv[r] += __shfl_xor(fv[r], o, 64);
          else iv[r] += __shfl_xor(iv[r], o, 64);
        }
      writer = false;
    } else {
      writer = false;
    }
    // One value per writing lane: row `held` (or, for narrow row groups, every row by lane 0).
#pragma unroll
    for (int k = 0; k < R; ++k) {
      if (swiglu) break;
      const int r = halving ? held : k;
      const bool w = halving ? (writer && k == 0) : (lg == 0);
      if (!w) continue;
      const float fval = halving ? fv[0] : fv[k];
      const long long ival = halving ? iv[0] : iv[k];
      const int o = out_index(bt, r);
      if (o >= p.n_out) continue;
      if (MODE == MODE_EXACT) {
        const long long res = ival >> p.R;
        int bad = ((ival >= (1LL << 47)) || (ival <= -(1LL << 47))) ? 1 : 0;
        bad |= (res >= (1LL << 31) || res <= -(1LL << 31)) ? 2 : 0;
        if (bad) atomicOr(p.status, bad);
        p.yi[o] = (int32_t)res;
      } else {
        float v = fval;
        if (p.epi == TRX_EPI_RESID) v += ld_vec<FUSED>(p.resid + o);
        st_vec<FUSED>(p.y + o, v);
        if (p.amax_slot) {
          const unsigned long long key = ((unsigned long long)ordered_bits(v) << 32) |
                                         (unsigned long long)(0xFFFFFFFFu - (uint32_t)o);
          best = key > best ? key : best;
        }
      }
    }
    if (MODE == MODE_F32 && swiglu) {
      // SwiGLU: the gate and up sums of an output sit in different lanes after the halving;
      // a plain butterfly keeps all R sums in every lane.
#pragma unroll
      for (int r = 0; r < R; ++r)
        for (int o = LPR >> 1; o >= 1; o >>= 1) facc[r] += __shfl_xor(facc[r], o, 64);
#pragma unroll
      for (int r = 0; r < R / 2; ++r) {
        const int o = out_index(bt, r);
        if (lg == (r % LPR) && o < p.n_out) st_vec<FUSED>(p.y + o, silu(facc[r]) * facc[r + R / 2]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) { facc[r] = 0.f; iacc[r] = 0; }
  };

  if (NSLOT == 1) load_x(0);
  int cbt = first, csl = 0;            // item being computed
  // A ring of NB register buffers: phase ph computes buf[ph] and refills the buffer consumed
  // one phase earlier with the item NB - 1 ahead.
  while (cbt < p.n_batches) {
#pragma unroll
    for (int ph = 0; ph < NB; ++ph) {
      if (cbt >= p.n_batches) break;
      load_item(buf[(ph + NB - 1) % NB], lbt, lsl);
      advance(lbt, lsl);
      if (NSLOT > 1) load_x(csl);
      compute_item(buf[ph], cbt, csl);
      if (csl == NSLOT - 1) finish_batch(cbt);
      advance(cbt, csl);
    }
  }
  if (MODE == MODE_F32 && p.amax_slot) {
    // One atomic per block: wave maximum, then the block's over its waves.
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const unsigned long long other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    __shared__ unsigned long long wbest[kWaves];
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long b = wbest[0];
      for (int w = 1; w < kWaves; ++w) b = wbest[w] > b ? wbest[w] : b;
      if (b) atomicMax(p.amax_slot, b);
    }
  }
}

static int lds_bytes(int K, int G) { return 2 * G * kXStride * 4 + K * 2 + G * 4 + 2 * G * 4 + 64; }

static int pick_lpr(int G) {
  int l = 64;
  while (l > 1 && (G % l)) l >>= 1;
  return l;
}

}  // namespace trx
