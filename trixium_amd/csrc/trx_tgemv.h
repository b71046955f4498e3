// Table-lookup ternary GEMV over a packed, slice-major weight layout: the float projection of
// the decoder (model/fastref.py:119-125 HybridRef.matmul for one position).
//
// Packed layout of an M x K ternary matrix (built once from BONS row packets by pack_ternary):
//   K is cut into S = ceil(K/256) slices of two 128-groups; rows into Q = ceil(M/4) quads.
//   A (slice, row) record holds the slice's code bytes as D dwords (trit5: 13 = 52 bytes, the
//   two groups' bytes 0..23 in dwords 0..5 and 6..11 and their bytes 24..25 in dword 12; 2-bit:
//   16 = 64 bytes, one group per 8 dwords).
//   codes:  uint4 [S][Q][D]: dword d of the quad's four records, in a per-dword row order (the
//           order the reduction of the lane that owns dword d consumes them in).
//   scales: uint32 [S][4Q] at codes + align256(code bytes): the slice's two fp16 group scales.
//   The bytes per row equal the BONS row's (codes + scales) for trit5 and 2-bit alike.
// SwiGLU matrices ([gate | up], 2F rows) are packed with gate and up rows interleaved per quad:
//   quad q = [gate 2q, gate 2q+1, up 2q, up 2q+1].
//
// Kernel: a block owns one slice and builds in LDS the table T[b][c] = sum_k w_k(b) * xhat[c_k]
// of every code byte value b at every code position c of the slice (64 positions: 16 lanes x
// 4 bytes), so a code byte costs one v_perm (the LDS address), one LDS read and one add. Each
// lane takes one dword of four rows per item; the sixteen lanes of a row reduce over DPP. The
// block writes per-slice partial sums; the block that completes a 32-quad tile last (agent-scope
// counter) adds the S partials in slice order (deterministic) and applies the epilogue
// (store, residual, SwiGLU, or argmax). With the RMSNorm prologue the table is built from
// x * gain and each partial sum is scaled by 1/rms(x) (the block's reduction of sum x^2 then
// overlaps the table build).
#pragma once

#include "trx_internal.h"

namespace trx {

constexpr int kSliceCols = 256;     // columns per K-slice (two 128-groups)
constexpr int kTabCols = 64;        // code positions per slice (16 lanes x 4 bytes)
constexpr int kTgThreads = 1024;    // one block per CU: one 64 KB table per CU
constexpr int kTgBlocksPerCU = 1;
constexpr int kTileQuads = kTgThreads / 16;   // quads per tile: one pass of a block (16 waves x 4 quads)
constexpr int kTileRows = 4 * kTileQuads;

struct PackGeom {
  int kind = 0, M = 0, K = 0, G = 0, S = 0, M4 = 0, Q = 0, D = 0, n_tiles = 0;
  int bps = 0, tpb = 0;       // launch: blocks per slice, tiles per block (tile t -> block t % bps)
  int rows_p = 0;             // partial sums per slice: bps * tpb tiles of kTileRows rows
  size_t code_bytes = 0;      // uint4 [S][Q][D]
  size_t scale_off = 0;       // byte offset of the scales
  size_t bytes = 0;           // packed matrix
  size_t cnt_bytes = 0;       // workspace: tile counters (zero between calls)
  size_t ss_bytes = 0;        // workspace: the blocks' slice sums of x^2 (RMSNorm)
  size_t work_bytes = 0;      // workspace: counters + slice sums + S x rows_p partial sums
};

// Geometry of a packed matrix; TRX_E_INVALID for an unsupported kind or shape.
int pack_geom(PackGeom& g, int kind, int M, int K);

// BONS row packets (M rows back to back) -> packed layout. swiglu: the rows are [gate | up]
// (M = 2F, F even) and are interleaved per quad.
int pack_ternary(const uint8_t* rows, int kind, int M, int K, int swiglu, uint8_t* packed,
                 hipStream_t s);

// y = W xhat with xhat = x (norm_w == nullptr) or x / rms(x) * norm_w, and the epilogue:
//   TRX_EPI_STORE y[m]; TRX_EPI_RESID y[m] = resid[m] + (W xhat)[m]; TRX_EPI_SWIGLU (matrix
//   packed with swiglu=1) y[f] = silu(g[f]) * u[f], f < M/2.
// amax_slot != nullptr: also the packed (ordered value, ~row) maximum of y (atomicMax).
// gate_pos/gate_from: the launch does nothing while *gate_pos < *gate_from.
// work: pack_geom().work_bytes of device memory whose counters are zero (the call leaves them
// zero); matrices may share one workspace of the largest work_bytes (the counters sit in a
// region of one size for all), but calls that share it must not overlap.
// x taken from decode attention's split partials instead (the o projection): x[h*hd + d] =
// sum_sp o[h][sp][d] exp(m[h][sp] - M) / sum_sp l[h][sp] exp(m[h][sp] - M), times
// sigmoid(gate) for gated attention; blocks of the first tile column also store x to `out`.
struct AttnMergeSrc {
  const float* m;          // [n_head][n_split]
  const float* l;
  const float* o;          // [n_head][n_split][hd]
  const int* pos;          // control words: [6] the KV slots attended (the splits' positions)
  int n_split, hd, gated;
  const float* qkv;        // gated: the gate after each q head
  float* out;              // [n_head * hd]
};

// Split-K partial sums handed to the next GEMV instead of reduced in this one. A GEMV given
// `out` stores only its partial sums, part[s * rows_p + r] for slice s and packed row r (every
// slice's partials; pack_geom gives S and rows_p), and skips the tile counting and reduction.
// With an RMSNorm its sums are of W (x * norm_w) (not yet scaled by 1/rms(x)) and each block
// stores its slice's sum of x^2 to out_ss[j * S + s]; the consumer applies the scale.
// A GEMV given `in` takes x from such partials:
//   F > 0 (a SwiGLU-packed gate|up producer): x[f] = silu(r g[f]) * (r u[f]), f < F = K, with
//     g and u the sums over the S slices and r = 1/sqrt(sum(in_ss[0..S)) / in_K + eps) (1 when
//     in_ss is null);
//   F = 0: x = resid + the sums over the S slices (rows of the producer = columns here).
// Blocks of the first tile column store that x to `act` (may be null).
struct PartialSums {
  float* out;              // producer: [S][rows_p]
  float* out_ss;           // producer with an RMSNorm: [bps][S]
  const float* in;         // consumer: the producer's partial sums
  const float* in_ss;      // consumer, SwiGLU input: the producer's out_ss (may be null)
  const float* resid;      // consumer, residual input
  int S, rows_p;           // consumer: the producer's geometry
  int F;                   // consumer: the producer's M / 2 (SwiGLU input) or 0 (residual input)
  int in_K;                // consumer with in_ss: the producer's K
  float* act;              // consumer: x stored here (may be null)
};

// y[m] = r * sum_s part[s * rows_p + m] for m < M (part and ss from a producer GEMV given
// PartialSums.out / out_ss; r = 1/sqrt(sum(ss[0..S)) / K + eps), or 1 without ss), with the
// packed (ordered value, ~row) maximum of y into amax_slot (atomicMax, one per block) when given.
// Spreads the reduction over the whole GPU: the LM head's rows. gate_pos/gate_from as for
// tgemv_f32.
int tgemv_reduce_f32(const float* part, const float* ss, int S, int rows_p, int M, int K, float eps, float* y,
                     unsigned long long* amax_slot, hipStream_t s, const int* gate_pos = nullptr,
                     const int* gate_from = nullptr);

// The most producer slices (K / 256, rounded up) a partial-sum consumer takes (SwiGLU input).
int tgemv_partial_slices_max();
// The same for a residual input.
int tgemv_resid_slices_max();

// A PrismML rotation of the GEMV's input, applied in its prologue: x' = scale * H (signs * xhat)
// per block of B columns (H the +-1 Sylvester matrix; B a power of two <= 1024 with K a multiple
// of max(B, 256)). Each GEMV block transforms the rotation block(s) holding its 256 columns; an x
// taken from a producer's partial sums or the attention merge is rotated for B <= 256 (the
// blocks then lie inside the slice).
struct RotSrc {
  const float* signs;
  int B;
  float scale;
};

// Many independent GEMVs in one launch: y_i = W_i x_i for i < n_mat, matrix i's packed copy at
// packed + (i % n_copies) * mat_stride, x_i at x + i * x_stride, y_i at y + i * y_stride. One
// block per (slice, matrix) streams every row of its slice (one table per slice column); `part`
// holds tgemv_batched_geom's part_bytes of split-K partial sums, reduced by a second launch.
int tgemv_batched_geom(int kind, int M, int K, int n_mat, PackGeom& g, size_t* part_bytes);
int tgemv_f32_batched(const uint8_t* packed, size_t mat_stride, int n_mat, int n_copies, int kind, int M, int K,
                      const float* x, int x_stride, float* y, int y_stride, float* part, hipStream_t s);

// tf: the table-free lookups (a code byte's weights from a 256-entry table, v_dot2 against x
// split into fp16 high and low planes) instead of the per-block table of partial dot products;
// the same results to float32 rounding, cheaper where a block streams few rows.
int tgemv_f32(const uint8_t* packed, int kind, int M, int K, const float* x, const float* norm_w,
              float eps, float* y, int epi, const float* resid, unsigned long long* amax_slot,
              void* work, hipStream_t s, const int* gate_pos = nullptr, const int* gate_from = nullptr,
              const AttnMergeSrc* merge = nullptr, const PartialSums* parts = nullptr,
              const RotSrc* rot = nullptr, bool tf = false);

}  // namespace trx
