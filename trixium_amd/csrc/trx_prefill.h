// Batched prefill: R prompt positions per forward (model/bitexact.py:121-125 matvec_ternary_rows,
// firmware/infer.c:1956-1977 forward_pair: one weight pass for several prompt tokens, no logits).
// Parameter blocks and launchers of the multi-position kernels (trx_prefill.hip).
#pragma once

#include "trx_internal.h"

namespace trx {

// Ternary (or Q8) GEMM on the matrix cores: Y[r][m] = sum_k X[r][k] W[m][k] for R positions.
// W is read as stored (BONS row packets, M rows of row_bytes) and decoded per 128-column group
// into LDS as fp16 weights (code - 1) * scale (2-bit, trit5) or fp16(q * scale) (Q8), which are
// exactly fastref's fp16 weight cache (model/fastref.py:104-116). X comes as two fp16 planes,
// xh = fp16(x') and xl = fp16(x' - xh) of x' = x / xs[r], so that each product of the fp32
// accumulation sees x to ~22 bits (the result is within float32 rounding of the fp32 product);
// xs[r] is a power of two that keeps row r's planes finite (1 for rows below 2^14), multiplied
// back in the epilogue.
enum { GM_STORE = 0, GM_RESID = 1, GM_SWIGLU = 2 };
struct GemmParams {
  const uint8_t* W;        // row packets
  uint32_t w_bytes;        // bytes readable from W (the buffer descriptor's range)
  int kind;                // TRX_KIND_TERNARY, TRX_KIND_TERNARY5 or TRX_KIND_Q8
  int M, K, row_bytes, code_off;
  const _Float16* xh;      // [R][K]
  const _Float16* xl;      // [R][K]
  const float* xs;         // [R] row scales (powers of two)
  int R;
  int epi;
  float* y;                // GM_STORE: y[r*ldy + m] = acc; GM_RESID: y[r*ldy + m] += acc;
  int ldy;                 // GM_SWIGLU (W = [gate; up], M = 2F): y[r*ldy + f] = silu(g[f]) * u[f]
  // GM_STORE with few blocks (a small M): with part != null K may be split over up to 16 parts
  // whose sums go to part[z][R][ldy] (part_floats of room) and are then added in part order.
  float* part;
  size_t part_floats;
};
int launch_gemm(const GemmParams& p, hipStream_t s);

// The GEMM's input planes from fp32 rows: v = x (no norm), or x / rms(x) * norm_w (RMSNorm,
// model/fastref.py:143-144), or a PrismML rotation of that (signs != null: per block of B
// columns v' = scale * H (signs * v), H the +-1 Sylvester matrix); xh = fp16(v / xs), xl =
// fp16(v / xs - xh), with xs[r] the power of two that brings row r below 2^14 (1 for most rows:
// fp16 holds values up to 65504, and a row past that would give inf and NaN products).
struct PrepParams {
  const float* x;
  int ldx, K, R;
  const float* norm_w;
  float eps;
  const float* signs;      // rotation, or null
  int B;
  float scale;
  _Float16* xh;            // [R][K]
  _Float16* xl;
  float* xs;               // [R]
  float* rs;               // [R] a rotated input's 1/rms per row (null without a rotation)
};
int launch_prep(const PrepParams& p, hipStream_t s);

// Per position and head: q and k RMS-normalised (their gains), NEOX RoPE on the first rope_n
// dims at position p0 + r (Q14 table row or theta^(-2i/n)), q scaled by 1/sqrt(hd) into q_out;
// k (post-RoPE) and v appended to the fp16 cache (model/golden.py:385-386).
struct RopeKvParams {
  const float* qkv;        // [R][ldq]: q heads (each [q | gate] when gated), k heads, v heads
  int ldq;
  const float* q_norm;
  const float* k_norm;
  const float* rope_freq;
  const float* rope_cs;    // [max_ctx][rope_n] fp32 cos half, then sin half (or null)
  const int16_t* rope_tab;
  int p0, R;
  __half* kcache;          // [n_kv][max_ctx][hd]
  __half* vcache;
  float* q_out;            // [R][n_head][hd]
  int n_head, n_kv, hd, rope_n, max_ctx, gated;
  float eps;
};
int launch_rope_kv(const RopeKvParams& p, hipStream_t s);

// Causal GQA attention of R query positions p0 .. p0 + R - 1 over the cache positions 0 .. each
// query's own (fastref.py:216-241, attention_fp32:31-43): softmax(q k^T) v in fp32 from the fp16
// cache, times sigmoid(gate) for gated attention.
struct AttnPrefillParams {
  const float* q;          // [R][n_head][hd] (normalised, rotated, scaled)
  const float* qkv;        // gates: qkv[r*ldq + h*2*hd + hd + d]
  int ldq;
  const __half* kcache;
  const __half* vcache;
  float* out;              // [R][n_head*hd]
  int p0, R, n_head, n_kv, hd, max_ctx, gated;
};
int launch_attn_prefill(const AttnPrefillParams& p, hipStream_t s);

// Gated DeltaNet over R positions (fastref.py:182-214, golden.py:400-434):
//   conv rows: conv + SiLU of every position from the raw projections (the window's older rows
//     from the state), q/k heads L2-normalised; then the state keeps the last K-1 raw rows;
//   scan: the recurrence per value head, position by position, rows of the state split over
//     blocks (rows are independent given k, q, beta and the decay);
//   gated norm: rmsnorm(o) * w * silu(z) into the grouped output order.
struct DnRowsParams {
  const float* io;         // [R][ld_io]: qkv (C channels) | z (nv*hv)
  int ld_io;
  const float* taps;       // [C][Kc]
  float* conv_state;       // [Kc-1][C]
  float* conv_out;         // [R][C]
  const float* ba;         // [R][2*nv]: beta then alpha
  const float* A;
  const float* dt;
  const float* norm_w;     // [hv]
  float* S;                // [nv][hv][hk]
  float* o_raw;            // [R][nv*hv]
  float* out;              // [R][nv*hv] grouped order
  int R, C, Kc, nq, nv, nk, hk, hv;
  float eps;
};
int launch_dn_rows(const DnRowsParams& p, hipStream_t s);

// Control words after a prefill of positions .. p_last: pos = p_last, cur_tok = fed[p_last].
int launch_prefill_ctl(int* ctl_pos, int* cur_tok, const int* fed, int p_last, hipStream_t s);

}  // namespace trx
