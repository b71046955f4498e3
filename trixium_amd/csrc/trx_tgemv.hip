// Table-lookup ternary GEMV (float path) and the packing of BONS rows into its layout.
// The arithmetic is the float projection of model/fastref.py:119-125 with the fused RMSNorm of
// fastref.py:143-145; the code decode is the reference's (model/bons.py:125-130: trit5 digit k
// of byte b is floor(b / 3^k) mod 3, 2-bit code k is (b >> 2k) & 3; weight = digit - 1).

#include <algorithm>
#include <type_traits>

#include "trx_tgemv.h"

namespace trx {

// Lane roles inside a 16-lane row group ------------------------------------------------------

// Record dword read by lane l16. trit5: lanes 0..5 take group 0's dwords, 8..13 group 1's,
// lanes 6 and 14 the shared dword 12 (group 0's bytes 24..25 at its bytes 0..1, group 1's at
// 2..3); lanes 7 and 15 read dword 12 too but own no byte of it.
__host__ __device__ inline int tg_lane_dword(bool t5, int l16) {
  if (!t5) return l16;
  return l16 < 6 ? l16 : (l16 < 8 ? 12 : (l16 < 14 ? l16 - 2 : 12));
}

// Row order of lane l16's quad: component k of its uint4 holds row k ^ mask. The masks make the
// three reduction steps (row_half_mirror, quad xor 2, quad xor 1) pair equal rows without
// selects; afterwards lane l16 holds row mask(l16) (lanes 0,2,4,6 hold rows 0,1,3,2).
__host__ __device__ inline int tg_lane_mask(int l16) {
  const int i = l16 & 7;
  return (((i >> 2) & 1) << 1) | (((i >> 1) ^ (i >> 2)) & 1);
}

// Group (0, 1; -1 for no byte) and group byte of table position c = 4 * lane + byte of dword.
__host__ __device__ inline void tg_position(bool t5, int c, int& g, int& byte) {
  const int l = c >> 2, jj = c & 3;
  g = -1;
  byte = 0;
  if (!t5) {
    g = l >> 3;
    byte = 4 * (l & 7) + jj;
  } else if (l < 6) {
    g = 0;
    byte = 4 * l + jj;
  } else if (l == 6) {
    if (jj < 2) { g = 0; byte = 24 + jj; }
  } else if (l >= 8 && l < 14) {
    g = 1;
    byte = 4 * (l - 8) + jj;
  } else if (l == 14) {
    if (jj >= 2) { g = 1; byte = 22 + jj; }
  }
}

// Group and group byte of record dword d, byte bi.
__host__ __device__ inline void tg_record_byte(bool t5, int d, int bi, int& g, int& byte) {
  if (!t5) {
    g = d >> 3;
    byte = 4 * (d & 7) + bi;
  } else if (d < 6) {
    g = 0;
    byte = 4 * d + bi;
  } else if (d < 12) {
    g = 1;
    byte = 4 * (d - 6) + bi;
  } else {
    g = bi >> 1;
    byte = 24 + (bi & 1);
  }
}

constexpr int kMaxTilesPerBlock = 128;  // also bounds the tiles of a reduction pass
constexpr int kMaxBatchedTiles = 64;     // row tiles of a batched launch's matrix (16384 rows)
// Tile counters sit 128 bytes apart: the S blocks of a tile count themselves at about the same
// time, and atomics to one line are serialised.
constexpr int kCntStride = 32;
constexpr int kMaxTiles = 4096;          // row tiles of a matrix (4096 x kTileRows rows)
constexpr int kMaxSliceSums = 4096;      // blocks of a launch (one slice sum of x^2 each)

static int cu_count() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      set_error("packed GEMV: cannot query the compute units");
      return 0;
    }
  }
  return cus;
}

int pack_geom(PackGeom& g, int kind, int M, int K) {
  TRX_CHECK(kind == TRX_KIND_TERNARY5 || kind == TRX_KIND_TERNARY, TRX_E_INVALID,
            "packed GEMV: kind %d is not ternary", kind);
  TRX_CHECK(M >= 1 && K >= kGroup && K % kGroup == 0, TRX_E_INVALID,
            "packed GEMV: M=%d K=%d (K must be a positive multiple of 128)", M, K);
  g = PackGeom{};
  g.kind = kind;
  g.M = M;
  g.K = K;
  g.G = K / kGroup;
  g.S = cdiv(g.G, 2);
  g.M4 = cdiv(M, 4) * 4;
  g.Q = g.M4 / 4;
  g.D = kind == TRX_KIND_TERNARY5 ? 13 : 16;
  g.n_tiles = cdiv(g.Q, kTileQuads);
  // Blocks per slice: fill the resident slots (kTgBlocksPerCU per CU), then even out the tiles.
  const int cus = cu_count();
  if (cus <= 0) return TRX_E_HIP;
  int bps = std::max(1, std::min(g.n_tiles, kTgBlocksPerCU * cus / g.S));
  int tpb = std::min(cdiv(g.n_tiles, bps), kMaxTilesPerBlock);
  bps = cdiv(g.n_tiles, tpb);
  g.tpb = cdiv(g.n_tiles, bps);
  g.bps = bps;
  g.rows_p = g.bps * g.tpb * kTileRows;
  g.code_bytes = (size_t)g.S * g.Q * g.D * 16;
  g.scale_off = (g.code_bytes + 255) / 256 * 256;
  // Lanes of a block's partial last tile read up to (bps * tpb * 32 - Q) quads past their
  // slice; the padding keeps those reads inside the allocation for the last slice.
  const size_t over = (size_t)(g.bps * g.tpb * kTileQuads - g.Q) * g.D * 16;
  g.bytes = g.scale_off + (size_t)g.S * g.M4 * 4 + over;
  // The counter region has one size for every matrix, so GEMVs over different matrices can
  // share a workspace (a matrix's partial sums never cover another's counters).
  TRX_CHECK(g.n_tiles <= kMaxTiles, TRX_E_INVALID, "packed GEMV: %d row tiles (at most %d)", g.n_tiles, kMaxTiles);
  g.cnt_bytes = (size_t)kMaxTiles * kCntStride * 4;
  TRX_CHECK(g.bps * g.S <= kMaxSliceSums, TRX_E_INVALID, "packed GEMV: %d blocks (at most %d)", g.bps * g.S, kMaxSliceSums);
  g.ss_bytes = (size_t)kMaxSliceSums * 4;
  g.work_bytes = g.cnt_bytes + g.ss_bytes + (size_t)g.S * g.rows_p * 4;
  TRX_CHECK(g.bytes < (1ull << 32), TRX_E_INVALID, "packed GEMV: %zu bytes exceed 4 GiB", g.bytes);
  return TRX_OK;
}

// Packing -----------------------------------------------------------------------------------

struct PackParams {
  const uint8_t* rows;
  uint8_t* out;
  size_t scale_off;
  int M, G, S, M4, Q, D, row_bytes, code_off, swiglu;
  bool t5;
};

__device__ inline int pack_src_row(const PackParams& p, int prow) {
  if (p.swiglu) {
    const int F = p.M / 2, q = prow >> 2, k = prow & 3;
    const int f = 2 * q + (k & 1);
    if (f >= F) return -1;
    return k < 2 ? f : F + f;
  }
  return prow < p.M ? prow : -1;
}

__global__ void pack_kernel(PackParams p) {
  const long long n = (long long)p.S * p.Q * p.D;
  const int gbytes = p.t5 ? kTrit5GroupBytes : 32;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
       idx += (long long)gridDim.x * blockDim.x) {
    const int d = (int)(idx % p.D);
    const long long r = idx / p.D;
    const int q = (int)(r % p.Q), s = (int)(r / p.Q);
    // The lanes that read dword d share one row order.
    const int owner = p.t5 ? (d < 6 ? d : (d < 12 ? d + 2 : 6)) : d;
    const int msk = tg_lane_mask(owner);
    uint32_t v[4];
    for (int k = 0; k < 4; ++k) {
      const int src = pack_src_row(p, 4 * q + (k ^ msk));
      uint32_t word = 0;
      if (src >= 0) {
        const uint8_t* row = p.rows + (size_t)src * p.row_bytes + p.code_off;
        for (int bi = 0; bi < 4; ++bi) {
          int g, byte;
          tg_record_byte(p.t5, d, bi, g, byte);
          const int ga = 2 * s + g;
          if (ga < p.G) word |= (uint32_t)row[(size_t)gbytes * ga + byte] << (8 * bi);
        }
      }
      v[k] = word;
    }
    ((uint4*)p.out)[idx] = make_uint4(v[0], v[1], v[2], v[3]);
    if (d == 0) {
      uint32_t* sc = (uint32_t*)(p.out + p.scale_off);
      for (int k = 0; k < 4; ++k) {
        const int prow = 4 * q + k;
        const int src = pack_src_row(p, prow);
        uint32_t word = 0;
        if (src >= 0) {
          const uint16_t* rs = (const uint16_t*)(p.rows + (size_t)src * p.row_bytes);
          const uint32_t lo = (2 * s < p.G) ? rs[2 * s] : 0u;
          const uint32_t hi = (2 * s + 1 < p.G) ? rs[2 * s + 1] : 0u;
          word = lo | (hi << 16);
        }
        sc[(size_t)s * p.M4 + prow] = word;
      }
    }
  }
}

int pack_ternary(const uint8_t* rows, int kind, int M, int K, int swiglu, uint8_t* packed,
                 hipStream_t s) {
  PackGeom g;
  int rc = pack_geom(g, kind, M, K);
  if (rc) return rc;
  TRX_CHECK(rows && packed, TRX_E_INVALID, "pack_ternary: null argument");
  TRX_CHECK(!swiglu || (M % 4 == 0), TRX_E_INVALID, "pack_ternary: SwiGLU needs M = 2F with F even (M=%d)", M);
  const RowGeom rg = row_geom(kind, K);
  PackParams p;
  p.rows = rows;
  p.out = packed;
  p.scale_off = g.scale_off;
  p.M = M;
  p.G = g.G;
  p.S = g.S;
  p.M4 = g.M4;
  p.Q = g.Q;
  p.D = g.D;
  p.row_bytes = rg.row_bytes;
  p.code_off = rg.code_off;
  p.swiglu = swiglu ? 1 : 0;
  p.t5 = kind == TRX_KIND_TERNARY5;
  const long long n = (long long)g.S * g.Q * g.D;
  const int blocks = (int)std::min<long long>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(pack_kernel, dim3(blocks), dim3(256), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

// GEMV kernel -------------------------------------------------------------------------------

constexpr int kDppRowRor8 = 0x128;
constexpr int kDppQuadUp2 = 0xEE;      // quad_perm [2,3,2,3]: lanes 0,1 of a quad read lanes 2,3
constexpr int kCpolSc1 = 16;          // buffer cache policy: device (agent) scope
constexpr int kCpolNt = 2;            // buffer cache policy: non-temporal (streaming)
constexpr int kMergeMax = 32;          // attention splits the merging prologue takes
constexpr int kSwiPartMax = 32;        // gate|up slices the SwiGLU prologue takes
constexpr int kResPartMax = 80;        // producer slices the residual prologue takes (68: 17408-wide down)
// Partial-sum prologues load 16 bytes per thread and slice: the SwiGLU one a packed row quad
// (128 per slice, so 8 slices per pass of the block), the residual one 4 columns (64 per slice,
// 16 slices per pass).
constexpr int kSwiSlicesPerPass = kTgThreads / (2 * kSliceCols / 4), kSwiVec = kSwiPartMax / kSwiSlicesPerPass;
constexpr int kResSlicesPerPass = kTgThreads / (kSliceCols / 4), kResVec = kResPartMax / kResSlicesPerPass;
constexpr int kMergeSlicesPerPass = kTgThreads / (kSliceCols / 4), kMergeVec = kMergeMax / kMergeSlicesPerPass;
// Where x comes from: p.x, the attention splits, SwiGLU of gate|up partial sums, or a residual
// plus a producer's partial sums.
constexpr int kXPlain = 0, kXMerge = 1, kXSwiglu = 2, kXResid = 3;

struct TgParams {
  const uint8_t* codes;
  const uint8_t* scales;
  uint32_t code_bytes, scale_bytes;
  int K, M, M4, Q, S, D, n_tiles, bps, tpb, rows_p;
  const float* x;
  const float* norm_w;
  float eps;
  float* y;
  const float* resid;
  int epi, n_out;
  float* part;
  float* ss_out;           // RMSNorm: each block's slice sum of x^2, [bps][S]
  int* cnt;
  unsigned long long* amax_slot;
  const int* gate_pos;
  const int* gate_from;
  AttnMergeSrc merge;      // merge.o != nullptr: x from attention partials
  PartialSums parts;       // parts.out: store the partial sums only; parts.in: x from them
  const float* rot_signs;  // a rotation of x in the prologue (RotSrc), or null
  int rot_B;
  float rot_scale;
  // Several matrices in one launch (blockIdx.y = matrix): matrix i's packed copy at
  // codes/scales + i * mat_bytes, its x at x + i * x_stride, its partial sums of slice s at
  // part + s * part_sstride + i * part_mstride. One matrix: 0, 0, rows_p, 0.
  uint32_t mat_bytes;
  int x_stride, part_sstride, part_mstride;
  int mat_copies;          // > 0: matrix i reads the packed copy i % mat_copies
  int n_mat;               // matrices of a batched launch with one x (the slice-pair kernel)
};

template <bool T5>
struct TgItem {
  uint4 c;            // dword of four rows
  uint32_t sc;        // the two fp16 group scales of this lane's row
};

// The slice's lookup table from its 256 x values: T[b][c] = sum over the digits (codes) k of
// byte b of (digit - 1) * x at table position c's k-th column, at tab[b * kTabCols + c]. T = hi(b)
// + lo(b): lo from the low digits (trit5: b % 9; 2-bit: b & 15), hi from the rest (b / 9; b >> 4).
// Waves w0 .. w0 + NW - 1 of the block build it (the others return at once). A thread owns one
// column: its x values and its lo sums in registers, then whole runs of entries sharing one hi
// (a wave-uniform hi value per run). The per-column set-up is repeated by every building wave,
// so NW = 8 of the 16 waves measured faster than all 16.
template <bool T5, int NW>
__device__ __forceinline__ void tg_build_table(float* tab, const float* xs, int tid, int w0) {
  constexpr int NLO = T5 ? 9 : 16;     // values of the low digits (trit5: 2 digits; 2-bit: 2 codes)
  constexpr int NHI = T5 ? 29 : 16;    // values of the rest (b / 9 <= 28; b >> 4)
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6) - w0;
  if (wv < 0 || wv >= NW) return;
  // Column c's group and byte as tg_position gives them, without branches: every lane loads
  // its digits' x (a clamped index), and a position without a byte or a digit past the group
  // takes 0 by a select.
  const int c = tid & (kTabCols - 1);
  const int l = c >> 2, jj = c & 3, g = l >> 3, ll = l & 7;
  const bool has = !T5 || ll < 6 || (ll == 6 && (g ? jj >= 2 : jj < 2));
  const int byte = !T5 || ll < 6 ? 4 * ll + jj : (g ? 22 + jj : 24 + jj);
  float u[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < (T5 ? 5 : 4); ++k) {
    const int cc = (T5 ? 5 : 4) * byte + k;
    const float v = xs[min(kGroup * g + cc, kSliceCols - 1)];
    u[k] = has && cc < kGroup ? v : 0.f;
  }
  if constexpr (T5) {
    // lo(e) = (e % 3 - 1) u0 + (e / 3 - 1) u1 is one of 0, +-u0, +-u1, +-(u0 + u1), +-(u0 - u1)
    // (every product is exact, and rounding is symmetric in sign).
    const float s01 = u[0] + u[1], d01 = u[0] - u[1];
    for (int h = wv; h < NHI; h += NW) {
      const int h1 = h / 3, h2 = h1 / 3;
      const float hv = (float)(h - 3 * h1 - 1) * u[2] + (float)(h1 - 3 * h2 - 1) * u[3] + (float)(h2 % 3 - 1) * u[4];
      const float t[NLO] = {hv - s01, hv - u[1], hv + d01, hv - u[0], hv, hv + u[0], hv - d01, hv + u[1], hv + s01};
      float* col = tab + h * NLO * kTabCols + c;
#pragma unroll
      for (int e = 0; e < NLO; ++e)
        if (h * NLO + e < 256) col[e * kTabCols] = t[e];
    }
  } else {
    float lo[NLO];
#pragma unroll
    for (int e = 0; e < NLO; ++e) lo[e] = (float)((e & 3) - 1) * u[0] + (float)((e >> 2) - 1) * u[1];
    for (int h = wv; h < NHI; h += NW) {
      const float hv = (float)((h & 3) - 1) * u[2] + (float)((h >> 2) - 1) * u[3];
      float* col = tab + h * NLO * kTabCols + c;
#pragma unroll
      for (int e = 0; e < NLO; ++e) col[e * kTabCols] = lo[e] + hv;
    }
  }
}

// One item's row sums: lane l16 of a row group looks up its four code dwords (16 bytes of four
// rows) in the table at tb (address = v_perm of the code byte and the lane's column: b * 256 +
// col * 4, plus what sel's third byte takes from lw), then the row group's partial sums meet by
// DPP; lane l16 ends with its group's sum of row mask(l16), times its fp16 group scale.
__device__ __forceinline__ float tg_item_sum(const uint4 c, uint32_t scales, uint32_t sshift, const uint32_t* lw,
                                             const uint32_t* sel, const char* tb) {
  float a[4];
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float t4[4];
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const uint32_t addr = __builtin_amdgcn_perm(cw[k], lw[jq], sel[jq]);
      t4[jq] = *(const float*)(tb + addr);
    }
    a[k] = (t4[0] + t4[1]) + (t4[2] + t4[3]);
  }
  a[0] += dpp_f<kDppRowHalfMirror>(a[2]);
  a[1] += dpp_f<kDppRowHalfMirror>(a[3]);
  a[0] += dpp_f<kDppQuadXor2>(a[1]);
  a[0] += dpp_f<kDppQuadXor1>(a[0]);
  return a[0] * __half2float(__ushort_as_half((unsigned short)(scales >> sshift)));
}

// Table-free lookups (TF): a 256-entry table of each code byte's weights (digit - 1) as fp16
// pairs, [w0 w1 | w2 w3 | w4 0 | 0] (trit5) or [w0 w1 | w2 w3 | 0 | 0] (2-bit), built in 4 KB
// of LDS by the first 256 threads; the lane's 4 code positions' x values held in registers as
// fp16 high and low planes (x = hi + lo to ~22 bits), so a code byte costs one LDS read and
// v_dot2 products against both planes, with no per-block table of partial dot products.
typedef _Float16 tf_h2 __attribute__((ext_vector_type(2)));

template <bool T5>
__device__ __forceinline__ void tf_build_lut(uint4* lut, int tid) {
  if (tid >= 256) return;
  int w[6] = {0, 0, 0, 0, 0, 0};
  if (T5) {
    int b = tid;
    for (int k = 0; k < 5; ++k) {
      w[k] = b % 3 - 1;
      b /= 3;
    }
  } else {
    for (int k = 0; k < 4; ++k) w[k] = ((tid >> (2 * k)) & 3) - 1;
  }
  uint32_t d[4];
  for (int k = 0; k < 3; ++k) {
    const tf_h2 v = {(_Float16)w[2 * k], (_Float16)w[2 * k + 1]};
    d[k] = __builtin_bit_cast(uint32_t, v);
  }
  d[3] = 0u;
  lut[tid] = make_uint4(d[0], d[1], d[2], d[3]);
}

// The x values of the lane's four code positions (4 * l16 + jj), digit by digit, split into fp16
// planes: xh[jj][k] = (x of digits 2k, 2k + 1), xl the remainder.
template <bool T5>
__device__ __forceinline__ void tf_lane_x(const float* xs, int l16, tf_h2 (&xh)[4][3], tf_h2 (&xl)[4][3]) {
  constexpr int DPB = T5 ? 5 : 4;                  // digits per code byte
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    int g, byte;
    tg_position(T5, 4 * l16 + jj, g, byte);
    float x[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < DPB; ++k) {
      const int cc = DPB * byte + k;
      if (g >= 0 && cc < kGroup) x[k] = xs[kGroup * g + cc];
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const _Float16 h0 = (_Float16)x[2 * k], h1 = (_Float16)x[2 * k + 1];
      xh[jj][k] = tf_h2{h0, h1};
      xl[jj][k] = tf_h2{(_Float16)(x[2 * k] - (float)h0), (_Float16)(x[2 * k + 1] - (float)h1)};
    }
  }
}

// tg_item_sum with the table-free lookups.
template <bool T5>
__device__ __forceinline__ float tf_item_sum(const uint4 c, uint32_t scales, uint32_t sshift, const uint4* lut,
                                             const tf_h2 (&xh)[4][3], const tf_h2 (&xl)[4][3]) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  // Byte position outer, rows inner: the four rows' lookups are in flight together and their
  // products go to eight independent sums (rows x planes).
  float ah[4] = {0.f, 0.f, 0.f, 0.f}, al[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    uint4 e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) e[k] = lut[(cw[k] >> (8 * jj)) & 255u];
#pragma unroll
    for (int q = 0; q < (T5 ? 3 : 2); ++q) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t ed = q == 0 ? e[k].x : q == 1 ? e[k].y : e[k].z;
        const tf_h2 wv = __builtin_bit_cast(tf_h2, ed);
        ah[k] = __builtin_amdgcn_fdot2(wv, xh[jj][q], ah[k], false);
        al[k] = __builtin_amdgcn_fdot2(wv, xl[jj][q], al[k], false);
      }
    }
  }
  float a[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) a[k] = ah[k] + al[k];
  a[0] += dpp_f<kDppRowHalfMirror>(a[2]);
  a[1] += dpp_f<kDppRowHalfMirror>(a[3]);
  a[0] += dpp_f<kDppQuadXor2>(a[1]);
  a[0] += dpp_f<kDppQuadXor1>(a[0]);
  return a[0] * __half2float(__ushort_as_half((unsigned short)(scales >> sshift)));
}

constexpr int kBuildWaves = 8;           // waves that build the single-slice kernel's table

// HAND: the partial sums go to the next GEMV (parts.out): plain stores, which the kernel's end
// makes visible to the next launch; otherwise agent-scope stores for the tile's reducing block.
template <bool T5, int NB, bool TF, bool HAND>
__global__ __launch_bounds__(kTgThreads, kTgBlocksPerCU) void tgemv_kernel(TgParams p) {
  __shared__ __align__(16) float tab[256 * kTabCols];
  // The prologue's partial-sum groups (their own memory, so the table can be built while the
  // last of them are read).
  __shared__ __align__(16) float scr[16 * kSliceCols];
  __shared__ float xs[kSliceCols];
  __shared__ float red[16];
  __shared__ int todo[kMaxTilesPerBlock];
  __shared__ float amw[kSliceCols / 64][kMergeMax], atot[kSliceCols / 64];
  __shared__ int n_todo;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int s = blockIdx.x % p.S, j = blockIdx.x / p.S;
  const int mi = blockIdx.y;               // the matrix (batched launches)
  const int n_items = p.tpb;               // row tiles of this block
  const int xmode = p.merge.o ? kXMerge : p.parts.in ? (p.parts.F ? kXSwiglu : kXResid) : kXPlain;
  // A gated-off launch does nothing but store the residual it was handed in partials. The gate
  // is read here and tested after the prologue's loads and the first weight loads are issued,
  // so its round trip does not delay them.
  const int gpos = p.gate_pos ? *p.gate_pos : 0, gfrom = p.gate_pos ? *p.gate_from : 0;

  // 1. The slice's 256 x values, or what they are made of. These loads are issued before the
  //    weight stream: vmcnt completes in order, so a wait for them would also wait for weights.
  const int cs = s * kSliceCols + tid;
  float xv = 0.f, wv = 1.f, ssin = 0.f;
  float4 pv[kSwiVec > kResVec ? (kSwiVec > kMergeVec ? kSwiVec : kMergeVec) : (kResVec > kMergeVec ? kResVec : kMergeVec)];
  int h0 = 0, nh = 0, mT = 0;
  float mv = -INFINITY, lv = 0.f, sw0 = 0.f, sw1 = 0.f;
  if (xmode == kXMerge) {
    // The slice's attention output from the split partials: every split's o values and the
    // (m, l) of the slice's heads, none of which waits for the position (the splits holding
    // positions are known once it arrives, after the weight loads are issued).
    const AttnMergeSrc& a = p.merge;
    mT = a.pos[6];                                   // KV slots attended
    h0 = (s * kSliceCols) / a.hd;
    nh = kSliceCols / a.hd;
    // Thread t loads columns 4 (t % 64) .. + 3 of splits t / 64 and t / 64 + 16 (16 bytes each;
    // past n_split a repeat of the last split). A split without positions keeps what an earlier
    // position left, and is dropped by a select, not a zero weight.
    const int c0 = s * kSliceCols + 4 * (tid % (kSliceCols / 4)), sl = tid / (kSliceCols / 4);
    const int h = c0 / a.hd, d = c0 - h * a.hd;
#pragma unroll
    for (int k = 0; k < kMergeVec; ++k)
      pv[k] = c0 < p.K ? *(const float4*)(a.o + ((size_t)h * a.n_split + min(sl + kMergeSlicesPerPass * k, a.n_split - 1)) * a.hd + d)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    // Split statistics of the slice's heads: wave w takes head h0 + w, lane k split k.
    if (w < nh && lane < a.n_split && (h0 + w) * a.hd < p.K) {
      mv = a.m[(size_t)(h0 + w) * a.n_split + lane];
      lv = a.l[(size_t)(h0 + w) * a.n_split + lane];
    }
  } else if (xmode == kXSwiglu) {
    // The gate|up partial sums of this slice's 128 packed row quads ([g 2q, g 2q+1, u 2q,
    // u 2q+1]): thread t loads quad t % 128 of slices t / 128, t / 128 + 8, ...; and the gate|up
    // input's slice sums of squares (its RMSNorm scale multiplies g and u). Slices past S are
    // not loaded (these loads precede the ring prefetch, so the wait for them stays exact).
    const __amdgpu_buffer_rsrc_t rin = make_rsrc(p.parts.in, (uint32_t)((size_t)p.parts.S * p.parts.rows_p * 4));
    const uint32_t off = (uint32_t)(2 * kSliceCols * s + 4 * (tid % (2 * kSliceCols / 4))) * 4u;
    const int sl = tid / (2 * kSliceCols / 4);
#pragma unroll
    for (int k = 0; k < kSwiVec; ++k) {
      pv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (sl + kSwiSlicesPerPass * k < p.parts.S) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(
            rin, off + (uint32_t)(sl + kSwiSlicesPerPass * k) * (uint32_t)p.parts.rows_p * 4u, 0, 0);
        pv[k] = make_float4(__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]));
      }
    }
    if (p.parts.in_ss && tid < p.parts.S) ssin = p.parts.in_ss[tid];
  } else if (xmode == kXResid) {
    // x = resid + the producer's partial sums of this slice's 256 rows: thread t loads columns
    // 4 (t % 64) .. + 3 of slices t / 64, t / 64 + 16, ... Slices past S are not loaded.
    const __amdgpu_buffer_rsrc_t rin = make_rsrc(p.parts.in, (uint32_t)((size_t)p.parts.S * p.parts.rows_p * 4));
    const uint32_t off = (uint32_t)(kSliceCols * s + 4 * (tid % (kSliceCols / 4))) * 4u;
    const int sl = tid / (kSliceCols / 4);
#pragma unroll
    for (int k = 0; k < kResVec; ++k) {
      pv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (sl + kResSlicesPerPass * k < p.parts.S) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(
            rin, off + (uint32_t)(sl + kResSlicesPerPass * k) * (uint32_t)p.parts.rows_p * 4u, 0, 0);
        pv[k] = make_float4(__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]));
      }
    }
    if (tid < kSliceCols && cs < p.K) {
      xv = p.parts.resid[cs];
      if (p.norm_w) wv = p.norm_w[cs];
    }
  } else if (tid < kSliceCols && cs < p.K) {
    xv = p.x[(size_t)mi * p.x_stride + cs];
    if (p.norm_w) wv = p.norm_w[cs];
  }
  // A rotated input: this thread's element of the rotation span holding the slice (the slice
  // itself for blocks of <= 256 columns, else the rotation block containing it), times the gain
  // and its sign.
  const bool rot = p.rot_signs && xmode == kXPlain;
  // A rotation of x taken from partial sums or the attention merge (blocks of <= 256 columns,
  // inside the slice): the slice's signs, loaded with the prologue's other inputs.
  const bool rot_in = p.rot_signs && xmode != kXPlain;
  const float sgn = rot_in && tid < kSliceCols && cs < p.K ? p.rot_signs[cs] : 0.f;
  const int rL = p.rot_B > kSliceCols ? p.rot_B : kSliceCols;
  const int rbase = s * kSliceCols - (s * kSliceCols) % rL;
  float rv = 0.f;
  if (rot && tid < rL) {
    const int c = rbase + tid;
    rv = p.x[c] * p.rot_signs[c];
    if (p.norm_w) rv *= p.norm_w[c];
  }

  // 2. The first NB - 1 items of this lane (they do not depend on x).
  const int rg = lane >> 4, l16 = lane & 15, half = l16 >> 3;
  const int dw = tg_lane_dword(T5, l16), msk = tg_lane_mask(l16);
  const size_t mcopy = p.mat_copies > 0 ? mi % p.mat_copies : mi;
  const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.codes + mcopy * p.mat_bytes, p.code_bytes);
  const __amdgpu_buffer_rsrc_t rsc = make_rsrc(p.scales + mcopy * p.mat_bytes, p.scale_bytes);
  // Item n of this lane is quad quad0 + n * qstep. The lane's offsets stay in fixed VGPRs and
  // the item's step goes in the scalar offset, so no VGPR that an in-flight access reads is
  // rewritten (that would cost a vmcnt wait per item). Only the VGPR offset is relied on for the
  // descriptor's range check: a quad past the matrix (partial last tile) reads zeros or unused
  // bytes of the packed matrix, and prefetches past the block's last item re-read that item.
  constexpr uint32_t kOut = 0x40000000u;     // a VGPR offset past every buffer
  const int quad0 = j * kTileQuads + w * 4 + rg, qstep = p.bps * kTileQuads;
  const uint32_t co0 = (((uint32_t)s * p.Q + (uint32_t)quad0) * p.D + dw) * 16u;
  const uint32_t cstep = (uint32_t)qstep * p.D * 16u;
  const uint32_t so0 = ((uint32_t)s * p.M4 + 4u * (uint32_t)quad0 + msk) * 4u;
  const uint32_t sstep = (uint32_t)qstep * 16u;
  // Partial sums: every lane stores every item (a fixed count of memory events per item keeps
  // the compiler's waits exact); the lanes that hold no row total store past the buffer (dropped
  // by the range check), and the items of a partial last tile land in padding rows.
  const __amdgpu_buffer_rsrc_t rpart = make_rsrc(p.part, (uint32_t)((size_t)p.S * p.part_sstride * 4));
  const uint32_t po0 = (l16 & 9) == 0 ? ((uint32_t)s * p.part_sstride + (uint32_t)mi * p.part_mstride +
                                         4u * (uint32_t)quad0 + msk) * 4u
                                      : kOut;
  const uint32_t pstep = (uint32_t)qstep * 16u;
  // Item n is tile n of the block (loads past the block's last item re-read it); its offsets
  // are scalar, and its partial-sum offset rides with it in the ring. (Non-temporal weight loads
  // measured 0.6% slower in the decode.)
  auto load_next = [&](TgItem<T5>& it, int& pso, int n) {
    const int m = min(n, n_items - 1);
    pso = m * (int)pstep;
    const auto a = __builtin_amdgcn_raw_buffer_load_b128(rc, co0, m * (int)cstep, 0);
    it.c = make_uint4(a[0], a[1], a[2], a[3]);
    it.sc = __builtin_amdgcn_raw_buffer_load_b32(rsc, so0, m * (int)sstep, 0);
  };
  TgItem<T5> buf[NB];
  int rp[NB];
  // Each prefetch is followed by a store that the range check drops: the loop issues a partial-sum
  // store after each item's loads, and with the same pattern on entry the compiler's vmcnt counts
  // at the loop head are those of the loop itself (otherwise the entry path sets them, and every
  // item would also wait for the next item's loads).
#pragma unroll
  for (int b = 0; b < NB - 1; ++b) {
    load_next(buf[b], rp[b], b);
    __builtin_amdgcn_raw_buffer_store_b32(0u, rpart, 0xfffffff0u, 0, 0);
  }
  const bool gated_off = gpos < gfrom;
  if (gated_off && !(xmode == kXResid && j == 0 && p.parts.act)) return;

  // 3. The slice's x (times the RMSNorm gain; 1/rms(x) scales the sums), then the table.
  if (xmode == kXMerge) {
    // The splits holding positions (of the T slots attended), their softmax weights per head, then each
    // thread's two splits weighted, the 16 split groups summed through scr (in group order),
    // then scaled by the heads' 1 / L.
    const int T = mT, chunk = (T + p.merge.n_split - 1) / p.merge.n_split;
    const int ns = min(p.merge.n_split, (T + chunk - 1) / chunk);
    if (w < nh) {
      const bool ok = lane < ns && (h0 + w) * p.merge.hd < p.K;
      const float mk = ok ? mv : -INFINITY;
      const float M = wave_max(mk);
      const float wv = ok ? __expf(mk - M) : 0.f;
      const float L = wave_sum(ok ? lv * wv : 0.f);
      if (lane < kMergeMax) amw[w][lane] = wv;
      if (lane == 0) atot[w] = L;
    }
    __syncthreads();
    {
      constexpr int NQ = kSliceCols / 4;
      const int sl = tid / NQ, hl = (4 * (tid % NQ)) / p.merge.hd;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int k = 0; k < kMergeVec; ++k) {
        const int sp = sl + kMergeSlicesPerPass * k;
        if (sp < ns) {
          const float wk = amw[hl][sp];
          v = make_float4(v.x + pv[k].x * wk, v.y + pv[k].y * wk, v.z + pv[k].z * wk, v.w + pv[k].w * wk);
        }
      }
      *(float4*)(scr + sl * kSliceCols + 4 * (tid % NQ)) = v;
    }
    __syncthreads();
    if (tid < kSliceCols && cs < p.K) {
      const int hl = tid / p.merge.hd, h = h0 + hl;
      float o = 0.f;
#pragma unroll
      for (int i = 0; i < kMergeSlicesPerPass; ++i) o += scr[i * kSliceCols + tid];
      o /= atot[hl];
      if (p.merge.gated) o *= sigmoidf_(p.merge.qkv[(size_t)h * 2 * p.merge.hd + p.merge.hd + (cs - h * p.merge.hd)]);
      xv = o;
    }
  } else if (xmode == kXSwiglu) {
    // Each thread's slices summed, the 8 slice groups through scr (in group
    // order), then per quad x[2q] = silu(r g0) * (r u0), x[2q + 1] = silu(r g1) * (r u1).
    constexpr int NQ = 2 * kSliceCols / 4;
    const int sl = tid / NQ;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < kSwiVec; ++k)
      if (sl + kSwiSlicesPerPass * k < p.parts.S)
        v = make_float4(v.x + pv[k].x, v.y + pv[k].y, v.z + pv[k].z, v.w + pv[k].w);
    *(float4*)(scr + sl * 2 * kSliceCols + 4 * (tid % NQ)) = v;
    if (w == 0) {
      const float t = wave_sum_dpp(ssin);
      if (lane == 0) red[0] = t;
    }
    __syncthreads();
    if (tid < NQ) {
      const float r = p.parts.in_ss ? 1.0f / sqrtf(red[0] / (float)p.parts.in_K + p.eps) : 1.f;
      float4 a = *(const float4*)(scr + 4 * tid);
#pragma unroll
      for (int i = 1; i < kSwiSlicesPerPass; ++i) {
        const float4 b = *(const float4*)(scr + i * 2 * kSliceCols + 4 * tid);
        a = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
      }
      const int fl = 2 * tid, f = s * kSliceCols + fl;
      const float x0 = f < p.K ? silu(r * a.x) * (r * a.z) : 0.f;
      const float x1 = f + 1 < p.K ? silu(r * a.y) * (r * a.w) : 0.f;
      xs[fl] = x0;
      xs[fl + 1] = x1;
      sw0 = x0;
      sw1 = x1;
    }
  } else if (xmode == kXResid) {
    // Each thread's slices summed, then the 16 slice groups through scr (in
    // group order).
    constexpr int NQ = kSliceCols / 4;
    const int sl = tid / NQ;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < kResVec; ++k)
      if (sl + kResSlicesPerPass * k < p.parts.S)
        v = make_float4(v.x + pv[k].x, v.y + pv[k].y, v.z + pv[k].z, v.w + pv[k].w);
    *(float4*)(scr + sl * kSliceCols + 4 * (tid % NQ)) = v;
    __syncthreads();
    if (tid < kSliceCols && cs < p.K) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < kResSlicesPerPass; ++i) a += scr[i * kSliceCols + tid];
      xv += a;
      if (gated_off && j == 0 && p.parts.act) p.parts.act[cs] = xv;
    }
    if (gated_off) return;
  }
  if (rot) {
    // H over each rotation block of the span: butterflies of span < 64 by wave shuffles, the
    // wider ones through the table's memory; then the slice's 256 values, scaled.
    for (int h = 1; h < 64 && h < p.rot_B; h <<= 1) {
      const float o = __shfl_xor(rv, h, 64);
      rv = (lane & h) ? o - rv : rv + o;
    }
    for (int h = 64; h < p.rot_B; h <<= 1) {
      tab[tid] = rv;
      __syncthreads();
      const float o = tab[tid ^ h];
      __syncthreads();
      rv = (tid & h) ? o - rv : rv + o;
    }
    tab[tid] = rv * p.rot_scale;
    __syncthreads();
    if (tid < kSliceCols) xs[tid] = tab[s * kSliceCols - rbase + tid];
  } else if (rot_in) {
    // The slice's x (times the gain), times the signs, through the butterflies of each rotation
    // block (all inside the slice), scaled.
    float r;
    if (xmode == kXSwiglu) {
      __syncthreads();                              // xs complete
      r = tid < kSliceCols ? xs[tid] * sgn : 0.f;
    } else {
      r = tid < kSliceCols && cs < p.K ? (p.norm_w ? xv * wv : xv) * sgn : 0.f;
    }
    for (int h = 1; h < 64 && h < p.rot_B; h <<= 1) {
      const float o = __shfl_xor(r, h, 64);
      r = (lane & h) ? o - r : r + o;
    }
    for (int h = 64; h < p.rot_B; h <<= 1) {
      tab[tid] = r;
      __syncthreads();
      const float o = tab[tid ^ h];
      __syncthreads();
      r = (tid & h) ? o - r : r + o;
    }
    if (tid < kSliceCols) xs[tid] = r * p.rot_scale;
  } else if (xmode != kXSwiglu && tid < kSliceCols) {
    xs[tid] = p.norm_w ? xv * wv : xv;
  }
  // The slice's sum of x^2 (x before the gain), for whoever applies the RMSNorm scale.
  if (p.norm_w && w < kSliceCols / 64) {
    const float q = wave_sum_dpp(xv * xv);
    if (lane == 0) red[w] = q;
  }
  __syncthreads();
  if constexpr (TF) tf_build_lut<T5>((uint4*)tab, tid);
  else tg_build_table<T5, kBuildWaves>(tab, xs, tid, 0);
  __syncthreads();

  // 4. The items: four rows x one dword per lane; sixteen lanes per row group.
  uint32_t lw[4], sel[4];
#pragma unroll
  for (int jq = 0; jq < 4; ++jq) {
    // Byte jj of the dword at step jq; rotating with the row group and half keeps the 64 lanes
    // of an LDS read on 64 different table columns (no bank conflicts).
    const int jj = (jq + rg + 2 * half) & 3;
    lw[jq] = (uint32_t)(4 * l16 + jj) * 4u;
    sel[jq] = 0x0c0c0400u | ((uint32_t)jj << 8);
  }
  const char* tb = (const char*)tab;
  const uint32_t sshift = 16u * (uint32_t)half;       // this lane's group scale in the dword
  tf_h2 xh[4][3], xl[4][3];
  if constexpr (TF) tf_lane_x<T5>(xs, l16, xh, xl);
  auto compute = [&](const TgItem<T5>& it, int pso) {
    float v;
    if constexpr (TF) v = tf_item_sum<T5>(it.c, it.sc, sshift, (const uint4*)tab, xh, xl);
    else v = tg_item_sum(it.c, it.sc, sshift, lw, sel, tb);
    v += dpp_f<kDppRowRor8>(v);                      // the other group (lane l16 ^ 8)
    // Agent-scope store (sc1) when the tile's reducing block (possibly on another XCD) reads it.
    // (One kind of store per kernel: a branch between two kinds would leave the compiler's vmcnt
    // counts short, and every item would also wait for the next item's loads.)
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rpart, po0, pso, HAND ? 0 : kCpolSc1);
  };
  // Whole groups of NB items (a loop with one exit keeps the compiler's vmcnt waits exact: item
  // n waits only for itself), then the remaining < NB items, already in flight.
  // The first group is peeled off the loop: the loop is then entered with the memory operations
  // of one whole group in flight, as at its back edge, so its vmcnt waits are exact (entered from
  // the prologue's many paths, every item would wait for more than its own loads).
  int n = 0;
  const int ngroups = n_items / NB;
  auto group = [&]() {
#pragma unroll
    for (int ph = 0; ph < NB; ++ph) {
      load_next(buf[(ph + NB - 1) % NB], rp[(ph + NB - 1) % NB], n + NB - 1);
      __builtin_amdgcn_sched_barrier(0);     // the prefetch goes out before this item's work
      compute(buf[ph], rp[ph]);
      ++n;
    }
  };
  if (ngroups > 0) {
    group();
    for (int gi = 1; gi < ngroups; ++gi) group();
  }
  const int rem = n_items - n;
#pragma unroll
  for (int ph = 0; ph < NB - 1; ++ph) {
    if (ph < rem) compute(buf[ph], rp[ph]);
  }

  // The prologue's own outputs, stored after the weight stream: a store issued before the table
  // would make its wave's first lookups wait for it (vmcnt completes in order). Block j = 0
  // keeps x (the residual handed on, or the attention output), every block its slice sum of x^2.
  if (j == 0 && tid < kSliceCols) {
    if (xmode == kXMerge && cs < p.K) {
      p.merge.out[cs] = xv;
    } else if (xmode == kXResid && p.parts.act && cs < p.K) {
      p.parts.act[cs] = xv;
    } else if (xmode == kXSwiglu && p.parts.act && tid < kSliceCols / 2) {
      const int f = s * kSliceCols + 2 * tid;
      if (f < p.K) p.parts.act[f] = sw0;
      if (f + 1 < p.K) p.parts.act[f + 1] = sw1;
    }
  }
  if (p.norm_w && tid == 0)
    __hip_atomic_store(p.ss_out + j * p.S + s, (red[0] + red[1]) + (red[2] + red[3]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);

  // The next GEMV reduces the partial sums (their stores complete before the launch ends).
  if (p.parts.out) return;

  // 5. Count this block's tiles done; the last of a tile's S blocks reduces it.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::: "memory");
  if (tid == 0) n_todo = 0;
  __syncthreads();
  if (tid < p.tpb) {
    const int t = j + tid * p.bps;
    if (t < p.n_tiles) {
      const int old = __hip_atomic_fetch_add(p.cnt + t * kCntStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == p.S - 1) {
        __hip_atomic_store(p.cnt + t * kCntStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        todo[atomicAdd(&n_todo, 1)] = t;
      }
    }
  }
  __syncthreads();
  // Reduction: kRedRows rows per thread, kTilesPerPass tiles per pass. The loads carry no
  // branches (a row or slice past the end re-reads a valid partial and is masked), so the
  // kRedRows x kRedChunk loads of a chunk are all in flight together. The S partials of a row
  // are summed in slice order (the same order whichever block reduces). Consecutive threads hold
  // consecutive rows, so a SwiGLU gate row finds its up row two lanes on (quad_perm).
  const int nt = n_todo;
  // The RMSNorm scale from the slice sums the tile's S blocks stored (each wave reads them).
  float rr = 1.f;
  if (p.norm_w && nt > 0) {
    float t = 0.f;
    for (int i = lane; i < p.S; i += 64)
      t += __hip_atomic_load(p.ss_out + j * p.S + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    rr = 1.0f / sqrtf(wave_sum_dpp(t) / (float)p.K + p.eps);
  }
  constexpr int kRedRows = 2, kRedChunk = 16;
  constexpr int kTilesPerPass = kTgThreads * kRedRows / kTileRows;
  static_assert(kTilesPerPass <= kMaxTilesPerBlock, "reduction pass");
  const uint32_t step = (uint32_t)p.part_sstride * 4u;
  for (int i0 = 0; i0 < nt; i0 += kTilesPerPass) {
    float yv[kRedRows];
    int prow[kRedRows];
    bool live[kRedRows];
    uint32_t off[kRedRows];
#pragma unroll
    for (int r = 0; r < kRedRows; ++r) {
      const int idx = tid + r * kTgThreads, i = i0 + idx / kTileRows;
      prow[r] = (i < nt ? todo[i] : todo[0]) * kTileRows + idx % kTileRows;
      live[r] = i < nt && prow[r] < p.M4;
      off[r] = (uint32_t)(live[r] ? prow[r] : 0) * 4u;
      yv[r] = 0.f;
    }
    // Tiles fill row slot 0 first and are kTileRows (4 waves) apart, so the live tests below are
    // uniform per wave (but for a partial last tile), and every load of a branch is consumed in
    // it. Rows of a dead slot issue no load.
    auto chunks = [&](auto nrows) {
      constexpr int NR = decltype(nrows)::value;
      for (int q0 = 0; q0 < p.S; q0 += kRedChunk) {
        float t[NR][kRedChunk];
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
          for (int k = 0; k < kRedChunk; ++k)
            t[r][k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                    rpart, off[r] + (uint32_t)min(q0 + k, p.S - 1) * step, 0, kCpolSc1));
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
          for (int k = 0; k < kRedChunk; ++k) yv[r] += q0 + k < p.S ? t[r][k] : 0.f;
      }
    };
    if (live[0] && live[1]) chunks(std::integral_constant<int, 2>{});
    else if (live[0]) chunks(std::integral_constant<int, 1>{});
#pragma unroll
    for (int r = 0; r < kRedRows; ++r) yv[r] *= rr;
    unsigned long long key = 0;
#pragma unroll
    for (int r = 0; r < kRedRows; ++r) {
      const float up = dpp_f<kDppQuadUp2>(yv[r]);        // row prow + 2 (quad lanes 2, 3)
      if (live[r]) {
        if (p.epi == TRX_EPI_SWIGLU) {
          const int k = prow[r] & 3, f = 2 * (prow[r] >> 2) + k;
          if (k < 2 && f < p.n_out) p.y[f] = silu(yv[r]) * up;
        } else if (prow[r] < p.M) {
          float out = yv[r];
          if (p.epi == TRX_EPI_RESID) out += p.resid[prow[r]];
          p.y[prow[r]] = out;
          const unsigned long long kr =
              ((unsigned long long)ordered_bits(out) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)prow[r]);
          key = kr > key ? kr : key;
        }
      }
    }
    if (p.amax_slot) {
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long other = __shfl_xor(key, o, 64);
        key = other > key ? other : key;
      }
      if (lane == 0 && key) atomicMax(p.amax_slot, key);
    }
  }
}

// Reduction of partial sums over many blocks ------------------------------------------------

constexpr int kRdThreads = 256, kRdBlocks = 256, kRdRowsMax = 4, kRdChunk = 16;

struct RdParams {
  const float* part;
  const float* ss;
  int S, rows_p, M, K, rpb;   // rpb: rows per block
  float eps;
  float* y;
  // Rows of several matrices (mat_rows_p > 0): row r is row r % mat_rows_p of matrix
  // r / mat_rows_p, stored at y[matrix * y_stride + row] when row < mat_M.
  int mat_rows_p, mat_M, y_stride;
  unsigned long long* amax_slot;
  const int* gate_pos;
  const int* gate_from;
};

// Batched matvecs with one x for every matrix (x_stride 0): block (q, y) builds the tables of
// slices 2q and 2q + 1 once, then streams those two slices of its share of the (matrix, tile)
// items (a contiguous run of the n_mat * tpb of them, y-th of ny), summing each row's two slices
// before it stores the partial sum: half the partial sums of one slice per block (their traffic
// to memory costs the batched launch more than their bytes). The two tables sit at LDS addresses
// 0 and 64 KB, so a code byte's lookup address is still one v_perm: the second table's selector
// takes a third address byte (1) from the lane's column word. The partial sums, [S2][n_mat]
// [rows_p] for S2 = ceil(S/2) slice pairs, are for a later launch (plain stores). A missing
// second slice (odd S) re-reads the first and adds nothing.
template <bool T5, int NB>
__global__ __launch_bounds__(kTgThreads, 1) void tgemv_pair_kernel(TgParams p) {
  constexpr int kTab = 256 * kTabCols;          // floats per table
  __shared__ __align__(16) float tab[2 * kTab];
  __shared__ float xs[2 * kSliceCols];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int s = 2 * blockIdx.x;                 // the block's first slice
  const bool two = s + 1 < p.S;
  // The block's items: a contiguous share of the n_mat * tpb (matrix, tile) items.
  const long long tot = (long long)p.n_mat * p.tpb;
  const int i0 = (int)((blockIdx.y * tot) / gridDim.y), i1 = (int)(((blockIdx.y + 1) * tot) / gridDim.y);
  const int n_items = i1 - i0, mi = i0 / p.tpb;

  // 1. The two slices' 512 x values, loaded before the weight stream (vmcnt completes in order).
  const int cx = s * kSliceCols + tid;
  const float xv = tid < 2 * kSliceCols && cx < p.K ? p.x[cx] : 0.f;

  // 2. The first NB - 1 items (they do not depend on x). The next item to load is tile lt of
  //    matrix mi + lm (tiles run through each matrix in turn from the block's first item), read
  //    from copy lc; its second slice lies one slice of codes (scales) further. The offsets stay
  //    in scalar registers.
  const int rg = lane >> 4, l16 = lane & 15, half = l16 >> 3;
  const int dw = tg_lane_dword(T5, l16), msk = tg_lane_mask(l16);
  const uint32_t span = (uint32_t)(p.mat_copies - 1) * p.mat_bytes;
  const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.codes, p.code_bytes + span);
  const __amdgpu_buffer_rsrc_t rsc = make_rsrc(p.scales, p.scale_bytes + span);
  const int quad0 = w * 4 + rg;                 // one block per slice pair covers every tile
  const uint32_t co0 = (((uint32_t)s * p.Q + (uint32_t)quad0) * p.D + dw) * 16u;
  const uint32_t cstep = (uint32_t)kTileQuads * p.D * 16u;
  const uint32_t so0 = ((uint32_t)s * p.M4 + 4u * (uint32_t)quad0 + msk) * 4u;
  const uint32_t sstep = (uint32_t)kTileQuads * 16u;
  const int c2 = two ? (int)(p.Q * p.D * 16u) : 0, s2 = two ? (int)(p.M4 * 4u) : 0;
  constexpr uint32_t kOut = 0x40000000u;
  const int S2 = (p.S + 1) / 2;
  const __amdgpu_buffer_rsrc_t rpart = make_rsrc(p.part, (uint32_t)((size_t)S2 * p.part_sstride * 4));
  const uint32_t po0 = (l16 & 9) == 0 ? ((uint32_t)blockIdx.x * p.part_sstride + 4u * (uint32_t)quad0 + msk) * 4u : kOut;
  const uint32_t pstep = (uint32_t)kTileQuads * 16u;
  struct Item {
    uint4 c0, c1;        // the dwords of four rows in the two slices
    uint32_t s0, s1;     // their fp16 group-scale pairs
  };
  int ln = 0, lt = i0 - mi * p.tpb, lm = 0, lc = mi % p.mat_copies;
  auto load_next = [&](Item& it, int& pso) {
    const int cso = lt * (int)cstep + lc * (int)p.mat_bytes;
    const int sso = lt * (int)sstep + lc * (int)p.mat_bytes;
    pso = lt * (int)pstep + (mi + lm) * p.part_mstride * 4;
    const auto a = __builtin_amdgcn_raw_buffer_load_b128(rc, co0, cso, kCpolNt);
    const auto b = __builtin_amdgcn_raw_buffer_load_b128(rc, co0, cso + c2, kCpolNt);
    it.c0 = make_uint4(a[0], a[1], a[2], a[3]);
    it.c1 = make_uint4(b[0], b[1], b[2], b[3]);
    it.s0 = __builtin_amdgcn_raw_buffer_load_b32(rsc, so0, sso, kCpolNt);
    it.s1 = __builtin_amdgcn_raw_buffer_load_b32(rsc, so0, sso + s2, kCpolNt);
    const int adv = ln < n_items - 1 ? 1 : 0;   // past the last item: re-read it
    const int wrap = adv && lt + 1 == p.tpb ? 1 : 0;
    ln += adv;
    lt = wrap ? 0 : lt + adv;
    lm += wrap;
    lc = wrap && lc + 1 == p.mat_copies ? 0 : lc + wrap;
  };
  Item buf[NB];
  int rp[NB];
  // Each prefetch is followed by a store that the range check drops, as each item's loads are
  // followed by its partial-sum store in the loop (so the loop's vmcnt waits stay exact).
#pragma unroll
  for (int b = 0; b < NB - 1; ++b) {
    load_next(buf[b], rp[b]);
    __builtin_amdgcn_raw_buffer_store_b32(0u, rpart, 0xfffffff0u, 0, 0);
  }

  // 3. The two tables.
  if (tid < 2 * kSliceCols) xs[tid] = xv;
  __syncthreads();
  tg_build_table<T5, kTgThreads / 128>(tab, xs, tid, 0);
  tg_build_table<T5, kTgThreads / 128>(tab + kTab, xs + kSliceCols, tid, kTgThreads / 128);
  __syncthreads();

  // 4. The items (as in the single-slice kernel, once per slice).
  uint32_t lw[4], sel0[4], sel1[4];
#pragma unroll
  for (int jq = 0; jq < 4; ++jq) {
    const int jj = (jq + rg + 2 * half) & 3;
    lw[jq] = (uint32_t)(4 * l16 + jj) * 4u | 0x10000u;      // third byte: the second table
    sel0[jq] = 0x0c0c0400u | ((uint32_t)jj << 8);            // address bytes: col*4, b, 0, 0
    sel1[jq] = 0x0c020400u | ((uint32_t)jj << 8);            // col*4, b, 1, 0
  }
  const char* tb = (const char*)tab;
  const uint32_t sshift = 16u * (uint32_t)half;
  auto compute = [&](const Item& it, int pso) {
    float v0 = tg_item_sum(it.c0, it.s0, sshift, lw, sel0, tb);
    float v1 = tg_item_sum(it.c1, it.s1, sshift, lw, sel1, tb);
    v0 += dpp_f<kDppRowRor8>(v0);               // the slice's other group (lane l16 ^ 8)
    v1 += dpp_f<kDppRowRor8>(v1);
    const float v = two ? v0 + v1 : v0;
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rpart, po0, pso, 0);
  };
  // The first group of NB items peeled off the loop (exact vmcnt waits in the loop), then the
  // remaining < NB items, already in flight.
  int n = 0;
  const int ngroups = n_items / NB;
  auto group = [&]() {
#pragma unroll
    for (int ph = 0; ph < NB; ++ph) {
      load_next(buf[(ph + NB - 1) % NB], rp[(ph + NB - 1) % NB]);
      __builtin_amdgcn_sched_barrier(0);
      compute(buf[ph], rp[ph]);
      ++n;
    }
  };
  if (ngroups > 0) {
    group();
    for (int gi = 1; gi < ngroups; ++gi) group();
  }
  const int rem = n_items - n;
#pragma unroll
  for (int ph = 0; ph < NB - 1; ++ph) {
    if (ph < rem) compute(buf[ph], rp[ph]);
  }
}

__global__ __launch_bounds__(kRdThreads) void tgemv_reduce_kernel(RdParams p) {
  __shared__ unsigned long long kmax[kRdThreads / 64];
  // The gate is read with the partials (a gated-off launch drops them) rather than before them.
  const int gpos = p.gate_pos ? *p.gate_pos : 0, gfrom = p.gate_pos ? *p.gate_from : 0;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r0 = blockIdx.x * p.rpb;
  // Rows q .. q + 3, q = r0 + 4 tid (rpb and rows_p are multiples of 4): one 16-byte load per
  // slice, the slice's offset scalar, every slice of a chunk in flight. A thread past the block's
  // range or M loads zeros (an offset past the buffer) and stores nothing.
  const int q = r0 + kRdRowsMax * tid;
  const bool live = kRdRowsMax * tid < p.rpb && q < p.M;
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.part, (uint32_t)((size_t)p.S * p.rows_p * 4));
  const uint32_t vo = live ? (uint32_t)q * 4u : 0x40000000u;
  float acc[kRdRowsMax] = {};
  for (int q0 = 0; q0 < p.S; q0 += kRdChunk) {
    float v[kRdChunk][kRdRowsMax];
#pragma unroll
    for (int k = 0; k < kRdChunk; ++k) {
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(rp, vo, (uint32_t)min(q0 + k, p.S - 1) * (uint32_t)p.rows_p * 4u, 0);
#pragma unroll
      for (int i = 0; i < kRdRowsMax; ++i) v[k][i] = __uint_as_float(a[i]);
    }
#pragma unroll
    for (int k = 0; k < kRdChunk; ++k)
#pragma unroll
      for (int i = 0; i < kRdRowsMax; ++i) acc[i] += q0 + k < p.S ? v[k][i] : 0.f;
  }
  float rs = 1.f;
  if (p.ss) {
    float t = 0.f;
    for (int i = lane; i < p.S; i += 64) t += p.ss[i];
    rs = rsqrtf(wave_sum_dpp(t) / (float)p.K + p.eps);
  }
  if (gpos < gfrom) return;
  unsigned long long key = 0;
#pragma unroll
  for (int i = 0; i < kRdRowsMax; ++i) {
    const int row = q + i;
    if (!live || row >= p.M) continue;
    const float out = acc[i] * rs;
    if (p.mat_rows_p) {
      const int mt = row / p.mat_rows_p, r = row - mt * p.mat_rows_p;
      if (r < p.mat_M) p.y[(size_t)mt * p.y_stride + r] = out;
      continue;
    }
    p.y[row] = out;
    const unsigned long long kr =
        ((unsigned long long)ordered_bits(out) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)row);
    key = kr > key ? kr : key;
  }
  if (!p.amax_slot) return;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const unsigned long long other = __shfl_xor(key, o, 64);
    key = other > key ? other : key;
  }
  if (lane == 0) kmax[w] = key;
  __syncthreads();
  if (tid == 0) {
    unsigned long long k = kmax[0];
    for (int i = 1; i < kRdThreads / 64; ++i) k = kmax[i] > k ? kmax[i] : k;
    // The slot only grows: a block whose key does not beat the value it reads needs no atomic
    // (same-address atomics from every block serialise).
    if (k && k > __hip_atomic_load(p.amax_slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(p.amax_slot, k);
  }
}

int tgemv_reduce_f32(const float* part, const float* ss, int S, int rows_p, int M, int K, float eps, float* y,
                     unsigned long long* amax_slot, hipStream_t s, const int* gate_pos, const int* gate_from) {
  TRX_CHECK(part && y && S >= 1 && M >= 1 && rows_p >= M && K >= 1, TRX_E_INVALID,
            "partial-sum reduction: bad arguments (S %d, rows %d, M %d)", S, rows_p, M);
  RdParams p;
  p.part = part;
  p.ss = ss;
  p.S = S;
  p.rows_p = rows_p;
  p.M = M;
  p.K = K;
  p.eps = eps;
  p.y = y;
  p.amax_slot = amax_slot;
  p.gate_pos = gate_pos;
  p.gate_from = gate_from;
  p.mat_rows_p = p.mat_M = p.y_stride = 0;
  const int blocks = std::min(kRdBlocks, cdiv(M, kRdThreads));
  p.rpb = cdiv(cdiv(M, blocks), kRdRowsMax) * kRdRowsMax;
  TRX_CHECK(rows_p % kRdRowsMax == 0 && p.rpb <= kRdRowsMax * kRdThreads, TRX_E_INVALID, "partial-sum reduction: %d rows (at most %d)", M,
            kRdBlocks * kRdRowsMax * kRdThreads);
  hipLaunchKernelGGL(tgemv_reduce_kernel, dim3(cdiv(M, p.rpb)), dim3(kRdThreads), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int tgemv_partial_slices_max() { return kSwiPartMax; }
int tgemv_resid_slices_max() { return kResPartMax; }

template <bool T5>
static const void* tg_fn(bool tf, bool hand) {
  if (hand) return tf ? (const void*)tgemv_kernel<T5, 4, true, true> : (const void*)tgemv_kernel<T5, 4, false, true>;
  return tf ? (const void*)tgemv_kernel<T5, 4, true, false> : (const void*)tgemv_kernel<T5, 4, false, false>;
}

int tgemv_f32(const uint8_t* packed, int kind, int M, int K, const float* x, const float* norm_w,
              float eps, float* y, int epi, const float* resid, unsigned long long* amax_slot,
              void* work, hipStream_t s, const int* gate_pos, const int* gate_from,
              const AttnMergeSrc* merge, const PartialSums* parts, const RotSrc* rot, bool tf) {
  PackGeom g;
  int rc = pack_geom(g, kind, M, K);
  if (rc) return rc;
  const bool p_in = parts && parts->in, p_out = parts && parts->out;
  const bool p_swi = p_in && parts->F > 0;
  TRX_CHECK(packed && (x || merge || p_in) && (y || p_out) && work, TRX_E_INVALID, "packed GEMV: null argument");
  TRX_CHECK(!p_in || (!x && !merge && parts->S >= 1 && parts->S <= (p_swi ? kSwiPartMax : kResPartMax) &&
                      parts->rows_p >= (p_swi ? 2 : 1) * K),
            TRX_E_INVALID, "packed GEMV: unsupported partial-sum input (S %d, rows %d, K %d)",
            p_in ? parts->S : 0, p_in ? parts->rows_p : 0, K);
  TRX_CHECK(!p_swi || (parts->F == K && !norm_w && (!parts->in_ss || parts->in_K > 0)), TRX_E_INVALID,
            "packed GEMV: SwiGLU partial-sum input needs F = K, no RMSNorm of its own and in_K");
  TRX_CHECK(!p_in || p_swi || parts->resid, TRX_E_INVALID, "packed GEMV: residual partial-sum input without resid");
  TRX_CHECK(!p_out || (!amax_slot && (!norm_w || parts->out_ss)), TRX_E_INVALID,
            "packed GEMV: partial-sum output with an argmax, or with an RMSNorm but no out_ss");
  TRX_CHECK(((uintptr_t)x & 15) == 0, TRX_E_INVALID, "packed GEMV: x must be 16-byte aligned");
  TRX_CHECK(!norm_w || x || (p_in && !p_swi), TRX_E_INVALID, "packed GEMV: the RMSNorm prologue needs x");
  TRX_CHECK(epi != TRX_EPI_RESID || resid, TRX_E_INVALID, "packed GEMV: residual epilogue without a residual");
  TRX_CHECK(epi != TRX_EPI_SWIGLU || M % 4 == 0, TRX_E_INVALID, "packed GEMV: SwiGLU needs M = 2F, F even");
  TRX_CHECK(epi != TRX_EPI_SWIGLU || !amax_slot, TRX_E_INVALID, "packed GEMV: no argmax with SwiGLU");
  TgParams p;
  p.codes = packed;
  p.scales = packed + g.scale_off;
  p.code_bytes = (uint32_t)g.code_bytes;
  p.scale_bytes = (uint32_t)(g.bytes - g.scale_off);
  p.K = K;
  p.M = M;
  p.M4 = g.M4;
  p.Q = g.Q;
  p.S = g.S;
  p.D = g.D;
  p.n_tiles = g.n_tiles;
  p.bps = g.bps;
  p.tpb = g.tpb;
  p.rows_p = g.rows_p;
  p.x = x;
  p.norm_w = norm_w;
  p.eps = eps;
  p.y = y;
  p.resid = resid;
  p.epi = epi;
  p.n_out = epi == TRX_EPI_SWIGLU ? M / 2 : M;
  p.cnt = (int*)work;
  p.part = p_out ? parts->out : (float*)((uint8_t*)work + g.cnt_bytes + g.ss_bytes);
  p.ss_out = p_out ? parts->out_ss : (float*)((uint8_t*)work + g.cnt_bytes);
  p.amax_slot = amax_slot;
  p.gate_pos = gate_pos;
  p.gate_from = gate_from;
  p.merge = merge ? *merge : AttnMergeSrc{};
  p.parts = parts ? *parts : PartialSums{};
  p.rot_signs = rot ? rot->signs : nullptr;
  p.rot_B = rot ? rot->B : 0;
  p.rot_scale = rot ? rot->scale : 1.f;
  p.mat_bytes = 0;
  p.x_stride = 0;
  p.part_sstride = g.rows_p;
  p.part_mstride = 0;
  TRX_CHECK(!rot || (rot->signs && rot->B >= 1 && rot->B <= kTgThreads && (rot->B & (rot->B - 1)) == 0 &&
                     K % std::max(rot->B, kSliceCols) == 0 && (x || rot->B <= kSliceCols)),
            TRX_E_INVALID, "packed GEMV: rotation of block %d over %d columns unsupported", rot ? rot->B : 0, K);
  const void* fn = kind == TRX_KIND_TERNARY5 ? tg_fn<true>(tf, p_out) : tg_fn<false>(tf, p_out);
  void* args[] = {(void*)&p};
  TRX_HIP(hipLaunchKernel(fn, dim3(g.S * g.bps), dim3(kTgThreads), args, 0, s));
  return TRX_OK;
}

int tgemv_batched_geom(int kind, int M, int K, int n_mat, PackGeom& g, size_t* part_bytes) {
  int rc = pack_geom(g, kind, M, K);
  if (rc) return rc;
  TRX_CHECK(n_mat >= 1 && n_mat <= 65535, TRX_E_INVALID, "batched GEMV: %d matrices (1..65535)", n_mat);
  TRX_CHECK(g.n_tiles <= kMaxBatchedTiles, TRX_E_INVALID, "batched GEMV: %d rows (at most %d)", M,
            kMaxBatchedTiles * kTileRows);
  // One block per (slice, matrix) streams every row of its slice: one table per slice column.
  g.bps = 1;
  g.tpb = g.n_tiles;
  g.rows_p = g.n_tiles * kTileRows;
  const size_t pb = (size_t)g.S * n_mat * g.rows_p * 4;
  TRX_CHECK(pb < (1ull << 32), TRX_E_INVALID, "batched GEMV: %zu bytes of partial sums exceed 4 GiB", pb);
  if (part_bytes) *part_bytes = pb;
  return TRX_OK;
}

int tgemv_f32_batched(const uint8_t* packed, size_t mat_stride, int n_mat, int n_copies, int kind, int M, int K,
                      const float* x, int x_stride, float* y, int y_stride, float* part, hipStream_t s) {
  PackGeom g;
  size_t pb = 0;
  int rc = tgemv_batched_geom(kind, M, K, n_mat, g, &pb);
  if (rc) return rc;
  TRX_CHECK(packed && x && y && part && n_copies >= 1 && n_copies <= n_mat, TRX_E_INVALID,
            "batched GEMV: null argument or %d copies for %d matrices", n_copies, n_mat);
  TRX_CHECK(mat_stride % 256 == 0 && (n_copies == 1 || mat_stride >= g.bytes) && mat_stride < (1ull << 32),
            TRX_E_INVALID, "batched GEMV: matrix stride %zu (a multiple of 256, at least %zu bytes)", mat_stride, g.bytes);
  TRX_CHECK((x_stride == 0 || x_stride >= K) && y_stride >= M && ((uintptr_t)x & 15) == 0 && x_stride % 4 == 0,
            TRX_E_INVALID, "batched GEMV: x stride %d, y stride %d (x 16-byte aligned)", x_stride, y_stride);
  // One x for every matrix: a block takes several matrices with one table (their items in turn).
  const bool multi = x_stride == 0 && n_mat > 1;
  TRX_CHECK(!multi || ((size_t)(n_copies - 1) * mat_stride + g.bytes < (1ull << 31) && pb < (1ull << 31)),
            TRX_E_INVALID, "batched GEMV with one x: %d copies of %zu bytes exceed 2 GiB", n_copies, mat_stride);
  TgParams p = {};
  p.codes = packed;
  p.scales = packed + g.scale_off;
  p.code_bytes = (uint32_t)g.code_bytes;
  p.scale_bytes = (uint32_t)(g.bytes - g.scale_off);
  p.K = K;
  p.M = M;
  p.M4 = g.M4;
  p.Q = g.Q;
  p.S = g.S;
  p.D = g.D;
  p.n_tiles = g.n_tiles;
  p.bps = g.bps;
  p.tpb = g.tpb;
  p.rows_p = g.rows_p;
  p.x = x;
  p.eps = 0.f;
  p.epi = TRX_EPI_STORE;
  p.n_out = M;
  p.part = part;
  p.parts.out = part;
  p.mat_bytes = (uint32_t)mat_stride;
  p.x_stride = x_stride;
  p.part_sstride = n_mat * g.rows_p;
  p.part_mstride = g.rows_p;
  p.mat_copies = n_copies;
  p.n_mat = n_mat;
  int nx = g.S, ny = n_mat;
  const void* fn = kind == TRX_KIND_TERNARY5 ? tg_fn<true>(false, true) : tg_fn<false>(false, true);
  if (multi) {
    // Blocks of slice pairs; the (matrix, tile) items spread evenly over ny groups, ny =
    // cus / gcd(S2, cus) so the grid's S2 * ny blocks fill whole rounds of the GPU (one round
    // when S2 divides the CU count; measured best of one to four rounds).
    const int cus = cu_count();
    if (cus <= 0) return TRX_E_HIP;
    nx = (g.S + 1) / 2;
    int a = nx, b = cus;
    while (b) { const int t = a % b; a = b; b = t; }
    ny = std::max(1, std::min(n_mat * g.tpb, cus / a));
    fn = kind == TRX_KIND_TERNARY5 ? (const void*)tgemv_pair_kernel<true, 4> : (const void*)tgemv_pair_kernel<false, 4>;
  }
  void* args[] = {(void*)&p};
  TRX_HIP(hipLaunchKernel(fn, dim3(nx, ny), dim3(kTgThreads), args, 0, s));
  // The S partial sums of every row of every matrix, reduced over the whole GPU.
  RdParams r = {};
  r.part = part;
  r.S = nx;                      // slices, or slice pairs
  r.rows_p = n_mat * g.rows_p;
  r.M = n_mat * g.rows_p;
  r.K = K;
  r.y = y;
  r.mat_rows_p = g.rows_p;
  r.mat_M = M;
  r.y_stride = y_stride;
  const int blocks = std::min(kRdBlocks, cdiv(r.M, kRdThreads));
  r.rpb = cdiv(cdiv(r.M, blocks), kRdRowsMax) * kRdRowsMax;
  if (r.rpb > kRdRowsMax * kRdThreads) {
    // More rows than one pass of the grid holds: more blocks.
    r.rpb = kRdRowsMax * kRdThreads;
  }
  hipLaunchKernelGGL(tgemv_reduce_kernel, dim3(cdiv(r.M, r.rpb)), dim3(kRdThreads), 0, s, r);
  TRX_LAUNCHED();
  return TRX_OK;
}

}  // namespace trx
