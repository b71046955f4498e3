// Parameter blocks and launchers of the decode-loop kernels (trx_ops.hip, trx_deltanet.hip).
#pragma once

#include "trx_internal.h"

namespace trx {

enum { EMBED_TABLE = 0, EMBED_TERNARY = 1, EMBED_RESTORE = 2 };

struct EmbedParams {
  int mode;
  int n_embd, vocab;
  const int16_t* mant;     // table mode: [vocab, n_embd]
  const int32_t* exps;     // table mode: [vocab]
  const uint8_t* rows;     // ternary mode: row packets of token_embd
  int kind, row_bytes, code_off;
  int* pos;                // device control words: [0] position of the current token
                           // (incremented here), [5] its KV slot, [6] KV slots attended, [7] the
                           // KV ring's pinned positions (0: no ring)
  const int* n_prompt;     // device
  const int* prompt;       // device ring of prompt_ring fed tokens (position p at p % prompt_ring)
  int prompt_ring;
  int max_ctx;             // KV slots; past them (the ring) the position's RoPE row is computed
  float* rope_cs;          // into row max_ctx of this fp32 cos|sin table (may be null)
  const float* rope_freq;  // [rope_n / 2]
  int rope_n;
  unsigned long long* slot;  // argmax of the previous step (cleared here)
  int* out;                // generated tokens [max_out]
  int max_out;
  int* cur_tok;            // the token embedded this step
  float* x;                // [n_embd]
  const float* signs;      // restore mode: the n_embd width's rotation signs (+-1)
  int hblock;              // restore mode: the rotation block
};

struct AttnParams {
  const float* qkv;        // [n_head*(gated?2:1)*hd | n_kv*hd | n_kv*hd]
  const float* q_norm;
  const float* k_norm;
  const float* rope_freq;  // [rope_n/2]
  const int16_t* rope_tab; // or [max_ctx][rope_n] Q14: cos half, then sin half (null: rope_freq)
  const float* rope_cs;    // [max_ctx + 1][rope_n] fp32 cos half, then sin half (the one-launch
                           // kernel; row max_ctx: the current position's, past the KV slots)
  const int* pos;          // control words: [0] position, [5] its KV slot, [6] KV slots attended
  __half* kcache;          // [n_kv][max_ctx][hd]
  __half* vcache;
  float* part_m;           // [n_head][n_split]
  float* part_l;
  float* part_o;           // [n_head][n_split][hd]
  float* out;              // [n_head*hd]
  int n_head, n_kv, n_rep, hd, rope_n, max_ctx, n_split, gated;
  float eps;
  unsigned* done;          // [n_kv][kDoneStride] split counters of the one-launch kernel (zero
                           // between launches), one per 128-byte line
  // One-launch kernel, non-gated: when set, q|k|v come as the packed GEMV's partial sums
  // ([qkv_S][qkv_rows_p], slice sums of x^2 in qkv_ss, K = qkv_K) instead of qkv.
  const float* qkv_part;
  const float* qkv_ss;
  int qkv_S, qkv_rows_p, qkv_K;
};
constexpr int kDoneStride = 32;
constexpr int kQkvPartMax = 16;    // q|k|v K-slices the attention sums (4096 columns)

struct DenseParams {
  const uint8_t* W;
  int kind;                // TRX_KIND_F16 or TRX_KIND_Q8
  int M, K, row_bytes, code_off;
  const float* x;
  const float* norm_w;
  float eps;
  float* y;
  int sigmoid;
  unsigned long long* amax_slot;
  const int* gate_pos;     // when set: nothing while *gate_pos < *gate_from
  const int* gate_from;
};

struct SynthParams {
  uint8_t* out;
  int kind, rows, cols, row_bytes, code_off;
  uint32_t seed, tensor_id;
  float lo, span;
};

struct DnConvParams {
  float* qkv;              // raw projection [C] (with part: the reduced [qkv | z] is stored here)
  const float* taps;       // [C][Kc]
  float* state;            // [Kc-1][C], oldest row first
  float* out;              // [C]: conv + SiLU, q and k heads L2-normalised
  int C, Kc, nq, hk;
  float eps;
  // When set, [qkv | z] arrives as the packed GEMV's K-slice partial sums ([S][rows_p], S <=
  // kDnPartMax, with its RMSNorm's slice sums of x^2 in part_ss over K columns): each value is
  // r * sum_s part[s] (slices in order, r = 1/sqrt(sum(ss) / K + eps)); the z rows (nz after the
  // C conv channels) are reduced into qkv + C for the recurrence.
  const float* part;
  const float* part_ss;
  int S, rows_p, K, nz;
  float rms_eps;
};
constexpr int kDnPartMax = 32;     // [qkv | z] K-slices the conv kernel sums (8192 columns)

struct DnRecurParams {
  const float* conv;       // [C]: q [nk*hk] | k [nk*hk] | v [nv*hv]
  const float* z;          // [nv*hv]
  const float* ba;         // [2*nv]: beta then alpha (raw projections)
  const float* A;          // [nv]: -exp(A_log)
  const float* dt;         // [nv]
  const float* norm_w;     // [hv]
  float* S;                // [nv][hv][hk] recurrent state of the layer
  float* out;              // [nv*hv], grouped head order
  int nv, nk, hk, hv;
  float eps;
};

// PrismML rotation of a projection input: y = scale * H (s * xhat) per block of B columns (H the
// +-1 Sylvester matrix), xhat = x, or x / rms(x) * norm_w with a norm. y must not alias x.
struct RotParams {
  const float* x;
  const float* norm_w;   // RMSNorm gain, or null
  float eps;
  int K, B;              // columns; block (a power of two in [64, 1024] dividing K)
  const float* signs;    // +-1 per column
  float scale;
  float* y;
};

int launch_rotate(const RotParams& p, hipStream_t s);
int launch_dn_conv(const DnConvParams& p, hipStream_t s);
// The conv and a Q8 GEMV (the beta/alpha rows) in one launch; TRX_E_INVALID for a geometry or
// layout the combined kernel does not take.
int launch_dn_conv_q8(const DnConvParams& cp, const DenseParams& dp, hipStream_t s);
int launch_dn_recur(const DnRecurParams& p, hipStream_t s);
// Sampling of the next token (firmware/infer.c:385-488): the candidates are the maxima of 32 row
// ranges of every channel's vocabulary shard; a repetition penalty over the last `window` tokens,
// then temperature, top-p over the candidates and one xorshift32 draw. The pick replaces the
// argmax in *slot. Nothing on positions before head_from.
struct SampleParams {
  const float* logits;
  int vocab, n_ch, window;
  const int* pos;
  const int* head_from;
  const int* n_prompt;
  const int* prompt;       // ring of prompt_ring fed tokens
  const int* out;
  int max_out;
  const float* cfg;        // temperature, top_p, repetition
  uint32_t* rng;           // xorshift32 state
  unsigned long long* slot;
  unsigned long long* cand;  // [32] the slices' (value bits, token) between the blocks
  unsigned* done;            // blocks finished (zero between launches)
  int prompt_ring;           // the fed tokens' ring: position p at prompt[p % prompt_ring]
};

// The final normed hidden state and the sequence score of one position (model/fastref.py:244-273:
// hidden = rmsnorm(x, out_norm); nll = logsumexp(logits) - logits[next token]). hidden goes to
// hid + row * n (row = *pos when `pos` is set, else 0; rows past max_rows are skipped); nll[*pos]
// is written when the position ran the head (*pos >= *head_from) and a next token was fed
// (*pos + 1 < *n_fed). With logits null only the hidden state is written.
struct ScoreParams {
  const float* x;          // the residual after the last layer
  const float* out_norm;
  float eps;
  int n;
  float* hid;
  int max_rows;
  const float* logits;
  int vocab;
  const int* pos;
  const int* head_from;
  const int* n_fed;
  const int* fed;          // the fed tokens by absolute position
  float* nll;
};
int launch_score(const ScoreParams& p, hipStream_t s);

int launch_embed(const EmbedParams& p, hipStream_t s);
// Prefill: the embeddings of the tokens fed at positions p0 .. p0 + R - 1 into X [R][n_embd]
// (p's control-word fields are not used).
int launch_embed_rows(const EmbedParams& p, const int* fed, int p0, int R, float* X, hipStream_t s);
int launch_sample(const SampleParams& p, hipStream_t s);
int launch_finalize(const int* pos, const int* n_prompt, unsigned long long* slot, int* out, int max_out,
                    hipStream_t s);
int launch_attention(const AttnParams& p, hipStream_t s);
// One-launch attention (trx_attn_fd.hip) for the geometries attention_fd_supported accepts: the
// split partials, merged by the last split block of each kv head when `done` is set (the output
// in `out`), left for the consumer to merge otherwise (attn_merge_into_x, the packed o GEMV).
// The one-launch attention takes the q|k|v GEMV's partial sums (its rotation partner a power-of-two
// number of float4s away).
bool attention_qp_supported(int hd, int rope_n);
bool attention_fd_supported(int rep, int hd, int rope_n, int n_split);
int launch_attention_fd(const AttnParams& p, hipStream_t s);
// The split partials of attention_fd merged by one block per q head (into `out`).
int launch_attention_merge(const AttnParams& p, hipStream_t s);
int attention_splits(int n_kv, int head_dim, int max_ctx);   // -1: the context is too long
int attention_max_chunk(int head_dim);                          // positions one split can hold
int attention_pass_positions(int head_dim);                     // positions one pass of a split block covers
int launch_dense_gemv(const DenseParams& p, hipStream_t s);
int launch_synth_ternary(const SynthParams& p, hipStream_t s);
int launch_synth_f32(float* out, long long n, uint32_t seed, uint32_t tensor_id, float lo, float span,
                     int transform, hipStream_t s);

int gemv_f32(const uint8_t* rows, int kind, int M, int K, const float* x, const float* norm_w,
             float eps, float* y, int epi, const float* resid, int swiglu_F,
             unsigned long long* amax_slot, hipStream_t s, const int* gate_pos = nullptr,
             const int* gate_from = nullptr);

}  // namespace trx
