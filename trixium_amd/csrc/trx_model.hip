// Batch-1 decode runtime: weight arena, KV cache, DeltaNet state, the per-token launch plan and
// its hipGraph. The state semantics follow model/golden.py:FloatModel (reset/forward/generate):
// K cached post-norm and post-RoPE, V raw, the conv window and recurrent matrix per DeltaNet
// layer, one position per forward; the loop contract follows model/mirror.py:1036-1044 (prefill
// one token per forward, logits only from the last prompt position on, no forward after the last
// generated token).

#include <stdio.h>
#include <string.h>
#include <math.h>
#include <map>
#include <vector>
#include <functional>
#include <algorithm>

#include "trx_internal.h"
#include "trx_ops.h"
#include "trx_model.h"
#include "trx_tgemv.h"
#include "trx_prefill.h"

namespace trx {

struct Tensor {
  size_t off = 0;      // byte offset in the arena
  size_t bytes = 0;
  int rows = 0, cols = 0, kind = 0;
  bool loaded = false;
};

// Positions every KV ring keeps past the window at least (firmware/hybrid.c:161 KV_SINKS), and the
// sampler's repetition window (the last 64 tokens, firmware/infer.c:385-488).
constexpr int kKvSinks = 4;
constexpr int kPfPartRow = 16 * 128;   // floats of K-part sums per prefill row
constexpr int kSmpWindow = 64;

// Projections that can run on the packed GEMV (trx_tgemv.h), keyed with their layer.
enum PackedOp { OP_QKV, OP_O, OP_GATE_UP, OP_DOWN, OP_HEAD, OP_DN_QKVZ, OP_DN_OUT };

struct PackedMat {
  uint8_t* buf = nullptr;          // packed copy
  const uint8_t* rows = nullptr;   // BONS row packets in the arena
  int M = 0, K = 0, kind = 0;
  bool swiglu = false;
};

struct Model {
  trx_model_config cfg;
  std::vector<float> rope_freq;
  hipStream_t stream = nullptr;
  uint8_t* arena = nullptr;
  size_t arena_bytes = 0;
  std::map<std::pair<int, int>, Tensor> tensors;   // (role, layer) -> tensor
  // fused groups: (layer) -> offset of [Wq|Wk|Wv] / [Wg|Wu] / [Wqkv|Wz]
  // device state
  __half *kcache = nullptr, *vcache = nullptr;     // per attention layer slice
  float *conv_state = nullptr, *dn_state = nullptr;
  float *x = nullptr, *qkv = nullptr, *attn_out = nullptr, *act = nullptr, *logits = nullptr;
  float *part_m = nullptr, *part_l = nullptr, *part_o = nullptr;
  unsigned* attn_done = nullptr;                   // [n_kv] split counters (one-launch attention)
  float *dn_io = nullptr, *dn_ba = nullptr, *dn_out = nullptr, *rope_dev = nullptr;
  float* rope_cs = nullptr;                        // [max_ctx + 1][rope_n]: cos(pos f_i), then sin
                                                   // (row max_ctx: the position past the window)
  int* ctl = nullptr;  // [0] pos, [1] n_fed, [2] cur_tok, [3] head_from, [4] error, [5] the position's
                       // KV slot, [6] KV slots attended, [7] KV ring pin (0: no ring), [8..] a ring
                       // of fed tokens (prompt_ring), then the generated tokens (max_new)
  int host_pos = -1;   // host mirror of the device position after the enqueued steps
  unsigned long long* slot = nullptr;
  int n_attn = 0, n_dn = 0;
  std::vector<int> attn_index, dn_index;           // per layer: index among attn / dn layers
  int n_split = 0;                                 // attention splits of the per-operation kernels
  // Packed copies of the projections in packed_ops (repacked from the arena after its tensors
  // change), and the workspace their GEMVs share.
  std::map<std::pair<int, int>, PackedMat> packed;
  int packed_ops = 0;
  int tf_ops = 0;                                  // packed projections on the table-free lookups
  bool pack_dirty = true;
  void* pack_work = nullptr;
  // Split-K partial sums handed from a packed GEMV to the next one, which reduces them in its
  // prologue: gate|up -> down (SwiGLU; with gate|up's slice sums of x^2 for its RMSNorm), and the
  // residual producers o and down -> the next packed consumer of the residual (x = resid + sums).
  float* ffn_part = nullptr;
  float* ffn_ss = nullptr;
  int ffn_S = 0, ffn_rows_p = 0;
  float* o_part = nullptr;
  int o_S = 0, o_rows_p = 0;
  float *qkv_part = nullptr, *qkv_ss = nullptr;    // q|k|v partial sums, summed by the attention
  int qkv_S = 0, qkv_rows_p = 0;
  float* down_part = nullptr;
  int down_S = 0, down_rows_p = 0;
  float* dn_out_part = nullptr;                    // DeltaNet out projection -> the FFN's gate|up
  int dn_out_S = 0, dn_out_rows_p = 0;
  float *dnz_part = nullptr, *dnz_ss = nullptr;    // DeltaNet [qkv|z] -> the conv kernel, which sums them
  int dnz_S = 0, dnz_rows_p = 0;
  float* head_part = nullptr;                      // LM head: partial sums reduced by many blocks
  float* head_ss = nullptr;
  int head_S = 0, head_rows_p = 0;
  float* x2 = nullptr;                             // second residual buffer (x alternates)
  float* xrot = nullptr;                           // a rotated model's projection input
  // Sampling (trx_model_set_sampling): temperature, top_p, repetition, then the xorshift32 state.
  float* smp = nullptr;
  unsigned long long* smp_cand = nullptr;          // [32] slice candidates, then the counter
  bool sampling = false;
  int smp_channels = 1;
  float* hidden = nullptr;                         // the residual after the last layer
  // Scoring (trx_model_score): per position the normed hidden state and the next token's NLL.
  bool scoring = false;
  float* hid_rows = nullptr;                       // [max_ctx][n_embd]
  float* nll = nullptr;                            // [max_ctx]
  float* hid_last = nullptr;                       // [n_embd]: TRX_READ_HIDDEN
  float* proj_x = nullptr;                         // [n_embd], [vocab]: trx_model_project_head
  float* proj_y = nullptr;
  // Batched prefill (trx_model_prefill): buffers for chunks of up to pf_rows positions.
  int pf_rows = 0;
  float *pf_x = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_att = nullptr, *pf_act = nullptr;
  float *pf_ba = nullptr, *pf_conv = nullptr, *pf_oraw = nullptr;
  // [pf_rows][kPfPartRow] the sums of a small GEMM's K parts (launch_gemm splits the K of a grid
  // that leaves most CUs idle, as the DeltaNet beta|alpha rows': up to 16 parts of 128 columns).
  float* pf_part = nullptr;
  _Float16 *pf_h = nullptr, *pf_l = nullptr;
  float* pf_xs = nullptr;                          // [pf_rows] row scales of the input planes
  float* pf_rs = nullptr;                          // [pf_rows] a rotated input's 1/rms per row
  int host_n_fed = 0, host_head_from = 0;          // host copies of the control words
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  // KV ring past the window (trx_model_set_kv_ring; firmware/hybrid.c:156-181): enabled (1), off
  // (0) or the default (-1: on for a model with DeltaNet layers), the pinned positions the next
  // reset applies, and the pinned positions in effect since the last reset (0: no ring).
  int kv_ring = -1;
  int kv_pin_next = kKvSinks;
  int kv_pin = 0;
  int prompt_ring = 0;                             // fed tokens kept: position p at p % prompt_ring
  // Decode-state checkpoint (trx_model_checkpoint): device copy of the control words, the argmax
  // slot, the sampler and the DeltaNet state; host copies of the host mirrors.
  uint8_t* ckpt = nullptr;
  size_t ckpt_bytes = 0;
  bool ckpt_valid = false;
  int ck_pos = -1, ck_n_fed = 0, ck_head_from = 0, ck_kv_pin = 0;
  int ck_lowest = 0x7fffffff;                      // lowest position a forward ran at since then
  size_t dev_bytes = 0;
  std::vector<void*> allocs;

  bool is_dn(int l) const { return (cfg.layer_types[l >> 6] >> (l & 63)) & 1ull; }
  int* pos() { return ctl; }
  int* n_prompt() { return ctl + 1; }
  int* cur_tok() { return ctl + 2; }
  int* head_from() { return ctl + 3; }
  int* prompt() { return ctl + 8; }
  int* out() { return ctl + 8 + prompt_ring; }
  int* err() { return ctl + 4; }                   // set by a kernel whose bounded wait timed out
};

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

static int row_bytes_of(int kind, int cols) {
  if (kind == TRX_KIND_TERNARY || kind == TRX_KIND_TERNARY5) return row_geom(kind, cols).row_bytes;
  if (kind == TRX_KIND_Q8) return kBeat * cdiv(cols / 32, 16) + cols;
  if (kind == TRX_KIND_F16 || kind == TRX_KIND_NORM16) return 2 * cols;
  return 4 * cols;  // F32
}

// Arena plan ----------------------------------------------------------------------------------

static void plan_tensor(Model& m, size_t& cur, int role, int layer, int kind, int rows, int cols,
                        bool pad = true) {
  Tensor t;
  t.rows = rows;
  t.cols = cols;
  t.kind = kind;
  t.bytes = (size_t)rows * row_bytes_of(kind, cols);
  t.off = cur;
  cur += t.bytes;
  if (pad) cur = align_up(cur + 64, 256);  // readable tail past every tensor
  m.tensors[{role, layer}] = t;
}

static void plan_arena(Model& m, size_t& cur) {
  const trx_model_config& c = m.cfg;
  const int E = c.n_embd, hd = c.head_dim, F = c.ffn_dim;
  const int qrows = c.n_head * hd * (c.attn_gated ? 2 : 1), kvrows = c.n_kv_head * hd;
  const int wk = c.weight_kind;
  const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
  const int C = 2 * nq + nvh;
  for (int l = 0; l < c.n_layer; ++l) {
    plan_tensor(m, cur, TRX_ROLE_ATTN_NORM, l, TRX_KIND_F32, 1, E);
    if (m.is_dn(l)) {
      // [Wqkv | Wz] adjacent: one GEMV launch.
      plan_tensor(m, cur, TRX_ROLE_ATTN_QKV, l, wk, C, E, false);
      plan_tensor(m, cur, TRX_ROLE_ATTN_ZGATE, l, wk, nvh, E);
      plan_tensor(m, cur, TRX_ROLE_SSM_BETA, l, TRX_KIND_Q8, c.dn_num_v_heads, E, false);
      plan_tensor(m, cur, TRX_ROLE_SSM_ALPHA, l, TRX_KIND_Q8, c.dn_num_v_heads, E);
      plan_tensor(m, cur, TRX_ROLE_SSM_CONV, l, TRX_KIND_F32, C, c.dn_conv_kernel);
      plan_tensor(m, cur, TRX_ROLE_SSM_A, l, TRX_KIND_F32, 1, c.dn_num_v_heads);
      plan_tensor(m, cur, TRX_ROLE_SSM_DT, l, TRX_KIND_F32, 1, c.dn_num_v_heads);
      plan_tensor(m, cur, TRX_ROLE_SSM_NORM, l, TRX_KIND_F32, 1, c.dn_v_head_dim);
      plan_tensor(m, cur, TRX_ROLE_SSM_OUT, l, wk, E, nvh);
    } else {
      // [Wq | Wk | Wv] adjacent: one GEMV launch.
      plan_tensor(m, cur, TRX_ROLE_ATTN_Q, l, wk, qrows, E, false);
      plan_tensor(m, cur, TRX_ROLE_ATTN_K, l, wk, kvrows, E, false);
      plan_tensor(m, cur, TRX_ROLE_ATTN_V, l, wk, kvrows, E);
      plan_tensor(m, cur, TRX_ROLE_ATTN_Q_NORM, l, TRX_KIND_F32, 1, hd);
      plan_tensor(m, cur, TRX_ROLE_ATTN_K_NORM, l, TRX_KIND_F32, 1, hd);
      plan_tensor(m, cur, TRX_ROLE_ATTN_OUT, l, wk, E, c.n_head * hd);
    }
    plan_tensor(m, cur, TRX_ROLE_FFN_NORM, l, TRX_KIND_F32, 1, E);
    plan_tensor(m, cur, TRX_ROLE_FFN_GATE, l, wk, F, E, false);
    plan_tensor(m, cur, TRX_ROLE_FFN_UP, l, wk, F, E);
    plan_tensor(m, cur, TRX_ROLE_FFN_DOWN, l, wk, E, F);
  }
  plan_tensor(m, cur, TRX_ROLE_OUT_NORM, 0, TRX_KIND_F32, 1, E);
  if (c.emb_mode == 0) {
    plan_tensor(m, cur, TRX_ROLE_TOK_EMB16, 0, TRX_KIND_NORM16, c.vocab, E);
    plan_tensor(m, cur, TRX_ROLE_TOK_EMB16_EXP, 0, TRX_KIND_F32, 1, c.vocab);  // int32 exponents
  }
  if (c.emb_mode != 0 || c.head_tied) plan_tensor(m, cur, TRX_ROLE_TOK_EMB, 0, c.emb_kind, c.vocab, E);
  if (!c.head_tied) plan_tensor(m, cur, TRX_ROLE_LM_HEAD, 0, c.head_kind, c.vocab, E);
  if (c.hadamard_block)
    for (int i = 0; i < 4; ++i)
      if (c.hadamard_widths[i]) plan_tensor(m, cur, TRX_ROLE_HADAMARD, i, TRX_KIND_F32, 1, c.hadamard_widths[i]);
  if (c.rope_table && m.n_attn)
    plan_tensor(m, cur, TRX_ROLE_ROPE_TAB, 0, TRX_KIND_NORM16, c.max_ctx, c.rope_dims ? c.rope_dims : c.head_dim);
}

static int dalloc(Model& m, void** p, size_t bytes);
static uint8_t* P(Model& m, int role, int layer);

// Packed copies: the projections selected by packed_ops (TRX_PACK_AUTO: the packed GEMV where it
// is the faster kernel for the weight kind), one device allocation for all of them, and the
// largest workspace any of them needs.
// The library's default table_free_ops.
constexpr int kTableFreeAuto = 0;

static int plan_packed(Model& m) {
  const trx_model_config& c = m.cfg;
  int ops = c.packed_ops;
  // Measured: the packed GEMV is the faster kernel for every attention-layer projection and the
  // head at the 8B shape, in both code formats, and for the DeltaNet qkv|z and out projections
  // at the 27B hybrid's widths.
  if (ops == TRX_PACK_AUTO) ops = TRX_PACK_ALL;
  TRX_CHECK(ops >= 0 && (ops & ~TRX_PACK_ALL) == 0, TRX_E_INVALID, "packed_ops %d has unknown bits", c.packed_ops);
  const int E = c.n_embd, hd = c.head_dim, F = c.ffn_dim, wk = c.weight_kind;
  const int qrows = c.n_head * hd * (c.attn_gated ? 2 : 1), kvrows = c.n_kv_head * hd;
  const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
  std::vector<std::pair<std::pair<int, int>, PackedMat>> list;
  auto add = [&](int op, int l, int role, int kind, int M, int K, bool swiglu) {
    PackedMat pm;
    pm.rows = P(m, role, l);
    pm.kind = kind;
    pm.M = M;
    pm.K = K;
    pm.swiglu = swiglu;
    list.push_back({{op, l}, pm});
  };
  for (int l = 0; l < c.n_layer; ++l) {
    if (m.is_dn(l)) {
      if (ops & TRX_PACK_DN) {
        add(OP_DN_QKVZ, l, TRX_ROLE_ATTN_QKV, wk, 2 * nq + 2 * nvh, E, false);
        add(OP_DN_OUT, l, TRX_ROLE_SSM_OUT, wk, E, nvh, false);
      }
    } else {
      if (ops & TRX_PACK_QKV) add(OP_QKV, l, TRX_ROLE_ATTN_Q, wk, qrows + 2 * kvrows, E, false);
      if (ops & TRX_PACK_O) add(OP_O, l, TRX_ROLE_ATTN_OUT, wk, E, c.n_head * hd, false);
    }
    if (ops & TRX_PACK_GATE_UP) add(OP_GATE_UP, l, TRX_ROLE_FFN_GATE, wk, 2 * F, E, true);
    if (ops & TRX_PACK_DOWN) add(OP_DOWN, l, TRX_ROLE_FFN_DOWN, wk, E, F, false);
  }
  const int head_role = c.head_tied ? TRX_ROLE_TOK_EMB : TRX_ROLE_LM_HEAD;
  const int head_kind = c.head_tied ? c.emb_kind : c.head_kind;
  if ((ops & TRX_PACK_HEAD) && (head_kind == TRX_KIND_TERNARY || head_kind == TRX_KIND_TERNARY5))
    add(OP_HEAD, 0, head_role, head_kind, c.vocab, E, false);
  size_t total = 0, work = 0;
  std::vector<size_t> offs;
  for (auto& e : list) {
    PackGeom g;
    int rc = pack_geom(g, e.second.kind, e.second.M, e.second.K);
    if (rc) return rc;
    offs.push_back(total);
    total += (g.bytes + 255) / 256 * 256;
    work = std::max(work, g.work_bytes);
  }
  m.packed_ops = ops;
  {
    // Measured choice: the table-free lookups where a block streams little (see the measurement
    // notes); every bit must be a packed projection.
    int tf = c.table_free_ops == TRX_PACK_AUTO ? kTableFreeAuto : c.table_free_ops;
    TRX_CHECK(tf >= 0 && (tf & ~TRX_PACK_ALL) == 0, TRX_E_INVALID, "table_free_ops %d has unknown bits",
              c.table_free_ops);
    m.tf_ops = tf & ops;
  }
  if (list.empty()) return TRX_OK;
  uint8_t* buf = nullptr;
  int rc;
  if ((rc = dalloc(m, (void**)&buf, total))) return rc;
  if ((rc = dalloc(m, &m.pack_work, work))) return rc;   // zeroed: the tile counters start at 0
  // Partial-sum buffers of the producers that hand their sums on.
  auto part_buf = [&](int M, int K, float** buf, int* S, int* rows_p, float** ss, int kind) -> int {
    PackGeom g;
    int rc2 = pack_geom(g, kind, M, K);
    if (rc2) return rc2;
    if ((rc2 = dalloc(m, (void**)buf, (size_t)g.S * g.rows_p * 4))) return rc2;
    if (ss && (rc2 = dalloc(m, (void**)ss, (size_t)g.bps * g.S * 4))) return rc2;
    *S = g.S;
    *rows_p = g.rows_p;
    return TRX_OK;
  };
  if ((ops & TRX_PACK_GATE_UP) && (ops & TRX_PACK_DOWN) && cdiv(E, kSliceCols) <= tgemv_partial_slices_max())
    if ((rc = part_buf(2 * F, E, &m.ffn_part, &m.ffn_S, &m.ffn_rows_p, &m.ffn_ss, wk))) return rc;
  if ((ops & TRX_PACK_O) && (ops & TRX_PACK_GATE_UP) && m.n_attn > 0 &&
      cdiv(c.n_head * hd, kSliceCols) <= tgemv_resid_slices_max())
    if ((rc = part_buf(E, c.n_head * hd, &m.o_part, &m.o_S, &m.o_rows_p, nullptr, wk))) return rc;
  if ((ops & TRX_PACK_QKV) && m.n_attn > 0 && !c.attn_gated && cdiv(E, kSliceCols) <= kQkvPartMax)
    if ((rc = part_buf(c.n_head * hd + 2 * c.n_kv_head * hd, E, &m.qkv_part, &m.qkv_S, &m.qkv_rows_p, &m.qkv_ss,
                       wk))) return rc;
  if ((ops & TRX_PACK_DOWN) && cdiv(F, kSliceCols) <= tgemv_resid_slices_max())
    if ((rc = part_buf(E, F, &m.down_part, &m.down_S, &m.down_rows_p, nullptr, wk))) return rc;
  if ((ops & TRX_PACK_DN) && (ops & TRX_PACK_GATE_UP) && m.n_dn > 0 && cdiv(nvh, kSliceCols) <= tgemv_resid_slices_max())
    if ((rc = part_buf(E, nvh, &m.dn_out_part, &m.dn_out_S, &m.dn_out_rows_p, nullptr, wk))) return rc;
  if ((ops & TRX_PACK_DN) && m.n_dn > 0 && cdiv(E, kSliceCols) <= kDnPartMax)
    if ((rc = part_buf(2 * nq + 2 * nvh, E, &m.dnz_part, &m.dnz_S, &m.dnz_rows_p, &m.dnz_ss, wk))) return rc;
  for (auto& e : list)
    if (e.first.first == OP_HEAD &&
        (rc = part_buf(c.vocab, E, &m.head_part, &m.head_S, &m.head_rows_p, &m.head_ss, e.second.kind)))
      return rc;
  for (size_t i = 0; i < list.size(); ++i) {
    list[i].second.buf = buf + offs[i];
    m.packed[list[i].first] = list[i].second;
  }
  return TRX_OK;
}

// Rebuild the packed copies after the arena's tensors changed.
static int ensure_packed(Model& m) {
  if (!m.pack_dirty) return TRX_OK;
  for (auto& kv : m.packed) {
    const PackedMat& pm = kv.second;
    int rc = pack_ternary(pm.rows, pm.kind, pm.M, pm.K, pm.swiglu ? 1 : 0, pm.buf, m.stream);
    if (rc) return rc;
  }
  TRX_HIP(hipStreamSynchronize(m.stream));
  m.pack_dirty = false;
  return TRX_OK;
}

static int dalloc(Model& m, void** p, size_t bytes) {
  hipError_t e = hipMalloc(p, bytes + 256);
  if (e != hipSuccess) {
    set_error("device allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? TRX_E_NOMEM : TRX_E_HIP;
  }
  m.allocs.push_back(*p);
  m.dev_bytes += bytes;
  TRX_HIP(hipMemset(*p, 0, bytes + 256));
  return TRX_OK;
}

// Plan of one decode position -----------------------------------------------------------------

static const Tensor& T(Model& m, int role, int layer) { return m.tensors[{role, layer}]; }
static uint8_t* P(Model& m, int role, int layer) { return m.arena + T(m, role, layer).off; }
static float* PF(Model& m, int role, int layer) { return (float*)P(m, role, layer); }

// One ternary projection: the packed GEMV when the model holds a packed copy of it, otherwise the
// row-packet kernel. In a rotated model the input (normalised first, with a norm) goes through
// the width's rotation into xrot, and the GEMV takes that.
// Whether projection `op` runs the packed GEMV's table-free lookups (config table_free_ops).
static bool tf_op(const Model& m, int op) {
  static const int bit[] = {TRX_PACK_QKV, TRX_PACK_O, TRX_PACK_GATE_UP, TRX_PACK_DOWN, TRX_PACK_HEAD, TRX_PACK_DN,
                            TRX_PACK_DN};
  return (m.tf_ops & bit[op]) != 0;
}

static int projection(Model& m, int op, int l, const uint8_t* rows, int kind, int M, int K, const float* x,
                      const float* norm_w, float* y, int epi, const float* resid, hipStream_t s,
                      unsigned long long* amax = nullptr, const int* gate_pos = nullptr,
                      const int* gate_from = nullptr) {
  auto it = m.packed.find({op, l});
  if (m.cfg.hadamard_block) {
    int wi = 0;
    while (wi < 4 && m.cfg.hadamard_widths[wi] != K) ++wi;
    TRX_CHECK(wi < 4, TRX_E_INVALID, "rotated model: no rotation for input width %d", K);
    const float* signs = PF(m, TRX_ROLE_HADAMARD, wi);
    const int B = m.cfg.hadamard_block;
    if (it != m.packed.end() && K % std::max(B, kSliceCols) == 0) {
      // The packed GEMV rotates its own slice of x in its prologue.
      const RotSrc rs = {signs, B, m.cfg.hadamard_scale};
      return tgemv_f32(it->second.buf, kind, M, K, x, norm_w, m.cfg.rms_eps, y, epi, resid, amax, m.pack_work, s,
                       gate_pos, gate_from, nullptr, nullptr, &rs, tf_op(m, op));
    }
    RotParams rp = {x, norm_w, m.cfg.rms_eps, K, B, signs, m.cfg.hadamard_scale, m.xrot};
    int rc;
    if ((rc = launch_rotate(rp, s))) return rc;
    x = m.xrot;
    norm_w = nullptr;
  }
  if (it != m.packed.end())
    return tgemv_f32(it->second.buf, kind, M, K, x, norm_w, m.cfg.rms_eps, y, epi, resid, amax, m.pack_work, s,
                     gate_pos, gate_from, nullptr, nullptr, nullptr, tf_op(m, op));
  return gemv_f32(rows, kind, M, K, x, norm_w, m.cfg.rms_eps, y, epi, resid, epi == TRX_EPI_SWIGLU ? M / 2 : 0,
                  amax, s, gate_pos, gate_from);
}

// The rotation of a projection input of width K (null for a plain model), held in rots.
static const RotSrc* rotation_of(Model& m, int K, RotSrc* rots) {
  const trx_model_config& c = m.cfg;
  if (!c.hadamard_block) return nullptr;
  for (int wi = 0; wi < 4; ++wi)
    if (c.hadamard_widths[wi] == K) {
      rots[wi] = {PF(m, TRX_ROLE_HADAMARD, wi), c.hadamard_block, c.hadamard_scale};
      return &rots[wi];
    }
  return nullptr;
}

// Gated DeltaNet layer: [qkv|z] GEMV and the beta/alpha Q8 GEMV (both with the attention
// RMSNorm), conv, recurrence with the gated norm, then the out projection with the residual.
// With the packed [qkv|z] and out GEMVs (pz, pdo): [qkv|z] reads x = xin, or xres + the partial
// sums pp (its prologue stores that x to xres for the Q8 GEMV); the out projection adds into
// m.x from xres, or (hand) stores its partial sums to dn_out_part. Otherwise x is m.x.
int dn_layer_launch(Model& m, int l, hipStream_t s, const PackedMat* pz = nullptr, const PackedMat* pdo = nullptr,
                    const float* xin = nullptr, const PartialSums* pp = nullptr, const float* xres = nullptr,
                    bool hand = false) {
  const trx_model_config& c = m.cfg;
  const int E = c.n_embd;
  const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
  const int C = 2 * nq + nvh;
  const int di = m.dn_index[l];
  RotSrc rots[4];
  int rc;
  float* io = m.dn_io;                  // [C + nvh] projections
  float* conv_out = m.dn_io + C + nvh;  // [C]
  const float* x = pz ? xres : m.x;
  DenseParams dp = {};
  dp.W = P(m, TRX_ROLE_SSM_BETA, l);
  dp.kind = TRX_KIND_Q8;
  dp.M = 2 * c.dn_num_v_heads;
  dp.K = E;
  dp.row_bytes = kBeat * cdiv(E / 32, 16) + E;
  dp.code_off = kBeat * cdiv(E / 32, 16);
  dp.x = x;
  dp.norm_w = PF(m, TRX_ROLE_ATTN_NORM, l);
  dp.eps = c.rms_eps;
  dp.y = m.dn_ba;
  DnConvParams cp = {};
  cp.qkv = io;
  cp.taps = PF(m, TRX_ROLE_SSM_CONV, l);
  cp.state = m.conv_state + (size_t)di * (c.dn_conv_kernel - 1) * C;
  cp.out = conv_out;
  cp.C = C;
  cp.Kc = c.dn_conv_kernel;
  cp.nq = nq;
  cp.hk = c.dn_k_head_dim;
  cp.eps = c.rms_eps;
  // One launch for both when the combined kernel takes them (aligned Q8 rows), else two.
  const bool fused = c.dn_k_head_dim <= 256 && C % c.dn_k_head_dim == 0 && E % 32 == 0 && dp.code_off % 16 == 0 &&
                     dp.row_bytes % 16 == 0 && ((uintptr_t)dp.W | (uintptr_t)dp.x | (uintptr_t)dp.norm_w) % 16 == 0;
  // The packed [qkv|z] GEMV hands its K-slice partial sums to the combined kernel, whose blocks
  // sum the values they take (no tile reduction in the GEMV); otherwise it stores [qkv | z].
  const bool qz_hand = pz && fused && m.dnz_part;
  if (qz_hand) {
    PartialSums qz = pp ? *pp : PartialSums{};
    qz.out = m.dnz_part;
    qz.out_ss = m.dnz_ss;
    if ((rc = tgemv_f32(pz->buf, c.weight_kind, C + nvh, E, xin, PF(m, TRX_ROLE_ATTN_NORM, l), c.rms_eps, nullptr,
                        TRX_EPI_STORE, nullptr, nullptr, m.pack_work, s, nullptr, nullptr, nullptr, &qz,
                        rotation_of(m, E, rots), tf_op(m, OP_DN_QKVZ)))) return rc;
    cp.part = m.dnz_part;
    cp.part_ss = m.dnz_ss;
    cp.S = m.dnz_S;
    cp.rows_p = m.dnz_rows_p;
    cp.K = E;
    cp.nz = nvh;
    cp.rms_eps = c.rms_eps;
  } else if (pz) {
    if ((rc = tgemv_f32(pz->buf, c.weight_kind, C + nvh, E, xin, PF(m, TRX_ROLE_ATTN_NORM, l), c.rms_eps, io,
                        TRX_EPI_STORE, nullptr, nullptr, m.pack_work, s, nullptr, nullptr, nullptr, pp,
                        rotation_of(m, E, rots), tf_op(m, OP_DN_QKVZ)))) return rc;
  } else if ((rc = projection(m, OP_DN_QKVZ, l, P(m, TRX_ROLE_ATTN_QKV, l), c.weight_kind, C + nvh, E, m.x,
                               PF(m, TRX_ROLE_ATTN_NORM, l), io, TRX_EPI_STORE, nullptr, s))) {
    return rc;
  }
  if (fused) {
    if ((rc = launch_dn_conv_q8(cp, dp, s))) return rc;
  } else if ((rc = launch_dense_gemv(dp, s)) || (rc = launch_dn_conv(cp, s))) {
    return rc;
  }
  DnRecurParams rp = {};
  rp.conv = conv_out;
  rp.z = io + C;
  rp.ba = m.dn_ba;
  rp.A = PF(m, TRX_ROLE_SSM_A, l);
  rp.dt = PF(m, TRX_ROLE_SSM_DT, l);
  rp.norm_w = PF(m, TRX_ROLE_SSM_NORM, l);
  rp.S = m.dn_state + (size_t)di * nvh * c.dn_k_head_dim;
  rp.out = m.dn_out;
  rp.nv = c.dn_num_v_heads;
  rp.nk = c.dn_num_k_heads;
  rp.hk = c.dn_k_head_dim;
  rp.hv = c.dn_v_head_dim;
  rp.eps = c.rms_eps;
  if ((rc = launch_dn_recur(rp, s))) return rc;
  if (pdo && hand) {
    PartialSums out = {};
    out.out = m.dn_out_part;
    return tgemv_f32(pdo->buf, c.weight_kind, E, nvh, m.dn_out, nullptr, c.rms_eps, nullptr, TRX_EPI_STORE, nullptr,
                     nullptr, m.pack_work, s, nullptr, nullptr, nullptr, &out, rotation_of(m, nvh, rots),
                     tf_op(m, OP_DN_OUT));
  }
  if (pdo)
    return tgemv_f32(pdo->buf, c.weight_kind, E, nvh, m.dn_out, nullptr, c.rms_eps, m.x, TRX_EPI_RESID, xres, nullptr,
                     m.pack_work, s, nullptr, nullptr, nullptr, nullptr, rotation_of(m, nvh, rots), tf_op(m, OP_DN_OUT));
  return projection(m, OP_DN_OUT, l, P(m, TRX_ROLE_SSM_OUT, l), c.weight_kind, E, nvh, m.dn_out, nullptr,
                    m.x, TRX_EPI_RESID, m.x, s);
}

static int run_step(Model& m, hipStream_t s) {
  const trx_model_config& c = m.cfg;
  const int E = c.n_embd, hd = c.head_dim, F = c.ffn_dim;
  const int qrows = c.n_head * hd * (c.attn_gated ? 2 : 1), kvrows = c.n_kv_head * hd;
  const int wk = c.weight_kind;
  int rc;
  // Embedding of this position's token.
  EmbedParams ep = {};
  ep.mode = c.emb_mode == 0 ? EMBED_TABLE : c.emb_mode == 1 ? EMBED_TERNARY : EMBED_RESTORE;
  ep.n_embd = E;
  ep.vocab = c.vocab;
  if (c.emb_mode == 2) {
    int wi = 0;
    while (wi < 4 && c.hadamard_widths[wi] != E) ++wi;
    ep.signs = PF(m, TRX_ROLE_HADAMARD, wi);
    ep.hblock = c.hadamard_block;
  }
  if (c.emb_mode == 0) {
    ep.mant = (const int16_t*)P(m, TRX_ROLE_TOK_EMB16, 0);
    ep.exps = (const int32_t*)P(m, TRX_ROLE_TOK_EMB16_EXP, 0);
  } else {
    ep.rows = P(m, TRX_ROLE_TOK_EMB, 0);
    ep.kind = c.emb_kind;
    ep.row_bytes = row_bytes_of(c.emb_kind, E);
    ep.code_off = row_geom(c.emb_kind, E).code_off;
  }
  ep.pos = m.pos();
  ep.n_prompt = m.n_prompt();
  ep.prompt = m.prompt();
  ep.prompt_ring = m.prompt_ring;
  ep.max_ctx = c.max_ctx;
  ep.rope_cs = m.rope_cs;
  ep.rope_freq = m.rope_dev;
  ep.rope_n = c.rope_dims ? c.rope_dims : c.head_dim;
  ep.slot = m.slot;
  ep.out = m.out();
  ep.max_out = c.max_new;
  ep.cur_tok = m.cur_tok();
  ep.x = m.x;
  if ((rc = launch_embed(ep, s))) return rc;

  // The residual stream between kernels is x = *xc, plus the sums of a producer's partials while
  // pend.in is set: a packed consumer adds them in its prologue and stores x to the other buffer.
  // A producer hands on partial sums only when the next consumer is a packed GEMV; otherwise it
  // reduces them into m.x (the DeltaNet kernels read m.x).
  float* xc = m.x;
  PartialSums pend = {};
  auto other = [&](const float* p) { return p == m.x ? m.x2 : m.x; };
  PartialSums pin;
  // Input of a packed consumer: sets x (or nullptr) and returns its partial-sum input (or null).
  auto take = [&](const float*& x) -> PartialSums* {
    pin = {};
    if (!pend.in) {
      x = xc;
      return nullptr;
    }
    pin.in = pend.in;
    pin.resid = xc;
    pin.S = pend.S;
    pin.rows_p = pend.rows_p;
    xc = other(xc);
    pin.act = xc;
    pend = {};
    x = nullptr;
    return &pin;
  };
  // The packed GEMV's own launches below (partial-sum handoffs, the attention merge in o's
  // prologue) rotate their input in the prologue when the model is rotated with blocks of at most
  // 256 columns (each block inside a GEMV's K-slice); a model with wider rotation blocks runs
  // every projection through projection().
  auto packed = [&](int op, int l) -> const PackedMat* {
    if (c.hadamard_block > kSliceCols) return nullptr;
    auto it = m.packed.find({op, l});
    return it == m.packed.end() ? nullptr : &it->second;
  };
  RotSrc rots[4];
  auto rot_for = [&](int K) { return rotation_of(m, K, rots); };
  // Whether the residual after layer l goes to a packed GEMV that takes the producer's S slices.
  auto next_packed = [&](int l, int S) {
    if (S > tgemv_resid_slices_max()) return false;
    if (l + 1 < c.n_layer) return packed(m.is_dn(l + 1) ? OP_DN_QKVZ : OP_QKV, l + 1) != nullptr;
    return packed(OP_HEAD, 0) != nullptr;
  };

  for (int l = 0; l < c.n_layer; ++l) {
    if (m.is_dn(l) && packed(OP_DN_QKVZ, l) && packed(OP_DN_OUT, l)) {
      // Gated DeltaNet mixer on the packed GEMVs: [qkv|z] takes the residual (or the previous
      // down's partial sums added to it), and the out projection hands its partial sums to the
      // FFN's gate|up when that is packed too.
      const float* xin;
      const PartialSums* pp = take(xin);
      const PackedMat* pdo = packed(OP_DN_OUT, l);
      const bool hand = m.dn_out_part && packed(OP_GATE_UP, l);
      if ((rc = dn_layer_launch(m, l, s, packed(OP_DN_QKVZ, l), pdo, xin, pp, xc, hand))) return rc;
      if (hand) {
        pend.in = m.dn_out_part;
        pend.S = m.dn_out_S;
        pend.rows_p = m.dn_out_rows_p;
      } else {
        xc = m.x;
      }
    } else if (m.is_dn(l)) {
      if ((rc = dn_layer_launch(m, l, s))) return rc;
    } else {
      // q|k|v with the attention RMSNorm fused in the prologue; its partial sums go to the
      // one-launch attention when that kernel takes them (non-gated), else it reduces them.
      const int rope_n = c.rope_dims ? c.rope_dims : hd;
      const bool fd_ok = attention_fd_supported(c.n_head / c.n_kv_head, hd, rope_n, m.n_split);
      const bool qkv_hand = fd_ok && attention_qp_supported(hd, rope_n) && m.qkv_part && m.qkv_rows_p % 4 == 0 &&
                            packed(OP_QKV, l);
      if (const PackedMat* pq = packed(OP_QKV, l)) {
        const float* xin;
        const PartialSums* pp = take(xin);
        PartialSums qp = pp ? *pp : PartialSums{};
        if (qkv_hand) {
          qp.out = m.qkv_part;
          qp.out_ss = m.qkv_ss;
        }
        if ((rc = tgemv_f32(pq->buf, wk, qrows + 2 * kvrows, E, xin, PF(m, TRX_ROLE_ATTN_NORM, l), c.rms_eps,
                            qkv_hand ? nullptr : m.qkv, TRX_EPI_STORE, nullptr, nullptr, m.pack_work, s, nullptr,
                            nullptr, nullptr, pp || qkv_hand ? &qp : nullptr, rot_for(E), tf_op(m, OP_QKV))))
          return rc;
      } else if ((rc = projection(m, OP_QKV, l, P(m, TRX_ROLE_ATTN_Q, l), wk, qrows + 2 * kvrows, E, xc,
                                   PF(m, TRX_ROLE_ATTN_NORM, l), m.qkv, TRX_EPI_STORE, nullptr, s))) {
        return rc;
      }
      AttnParams ap = {};
      ap.qkv = m.qkv;
      ap.q_norm = PF(m, TRX_ROLE_ATTN_Q_NORM, l);
      ap.k_norm = PF(m, TRX_ROLE_ATTN_K_NORM, l);
      ap.rope_freq = m.rope_dev;
      ap.rope_cs = m.rope_cs;
      ap.rope_tab = m.cfg.rope_table ? (const int16_t*)P(m, TRX_ROLE_ROPE_TAB, 0) : nullptr;
      ap.pos = m.pos();
      const size_t per = (size_t)c.n_kv_head * c.max_ctx * hd;
      ap.kcache = m.kcache + (size_t)m.attn_index[l] * per;
      ap.vcache = m.vcache + (size_t)m.attn_index[l] * per;
      ap.part_m = m.part_m;
      ap.part_l = m.part_l;
      ap.part_o = m.part_o;
      ap.out = m.attn_out;
      ap.n_head = c.n_head;
      ap.n_kv = c.n_kv_head;
      ap.n_rep = c.n_head / c.n_kv_head;
      ap.hd = hd;
      ap.rope_n = c.rope_dims ? c.rope_dims : hd;
      ap.max_ctx = c.max_ctx;
      ap.n_split = m.n_split;
      ap.gated = c.attn_gated;
      ap.eps = c.rms_eps;
      if (qkv_hand) {
        ap.qkv_part = m.qkv_part;
        ap.qkv_ss = m.qkv_ss;
        ap.qkv_S = m.qkv_S;
        ap.qkv_rows_p = m.qkv_rows_p;
        ap.qkv_K = E;
      }
      // One-launch attention; with a packed o projection the splits are merged in that GEMV's
      // prologue (each of its blocks merges the heads of its column slice).
      const bool fd = attention_fd_supported(ap.n_rep, hd, ap.rope_n, ap.n_split);
      const PackedMat* po = packed(OP_O, l);
      const bool merge_in_o = fd && po && ap.n_split <= 32 && kSliceCols % hd == 0;
      // Otherwise the splits are merged by the last split block of each kv head, or, when that
      // block would read many partials alone, by a merge launch with one block per q head.
      const bool merge_apart = !merge_in_o && ap.n_split * ap.n_rep * hd > 8192;
      ap.done = merge_in_o || merge_apart ? nullptr : m.attn_done;
      if (fd) {
        if ((rc = launch_attention_fd(ap, s))) return rc;
        if (merge_apart && (rc = launch_attention_merge(ap, s))) return rc;
      } else if ((rc = launch_attention(ap, s))) {
        return rc;
      }
      if (merge_in_o) {
        AttnMergeSrc ms = {ap.part_m, ap.part_l, ap.part_o, ap.pos, ap.n_split, hd, ap.gated, ap.qkv, m.attn_out};
        if (m.o_part && packed(OP_GATE_UP, l)) {
          // The o projection's partial sums go to gate|up, which adds them to the residual.
          PartialSums out = {};
          out.out = m.o_part;
          if ((rc = tgemv_f32(po->buf, wk, E, c.n_head * hd, nullptr, nullptr, c.rms_eps, nullptr, TRX_EPI_STORE,
                              nullptr, nullptr, m.pack_work, s, nullptr, nullptr, &ms, &out,
                              rot_for(c.n_head * hd), tf_op(m, OP_O)))) return rc;
          pend.in = m.o_part;
          pend.S = m.o_S;
          pend.rows_p = m.o_rows_p;
        } else {
          if ((rc = tgemv_f32(po->buf, wk, E, c.n_head * hd, nullptr, nullptr, c.rms_eps, m.x, TRX_EPI_RESID, xc,
                              nullptr, m.pack_work, s, nullptr, nullptr, &ms, nullptr, rot_for(c.n_head * hd),
                              tf_op(m, OP_O))))
            return rc;
          xc = m.x;
        }
      } else {
        if ((rc = projection(m, OP_O, l, P(m, TRX_ROLE_ATTN_OUT, l), wk, E, c.n_head * hd, m.attn_out, nullptr,
                             m.x, TRX_EPI_RESID, xc, s))) return rc;
        xc = m.x;
      }
    }
    // SwiGLU FFN: gate|up with the FFN RMSNorm, then down with the residual add.
    const PackedMat* pg = packed(OP_GATE_UP, l);
    const PackedMat* pd = packed(OP_DOWN, l);
    if (pg && pd && m.ffn_part) {
      // gate|up stores its partial sums (and slice sums of x^2); down's prologue reduces them,
      // applies the RMSNorm scale and SwiGLU.
      const float* xin;
      PartialSums* pp = take(xin);
      PartialSums gu = pp ? *pp : PartialSums{};
      gu.out = m.ffn_part;
      gu.out_ss = m.ffn_ss;
      if ((rc = tgemv_f32(pg->buf, wk, 2 * F, E, xin, PF(m, TRX_ROLE_FFN_NORM, l), c.rms_eps, nullptr, TRX_EPI_SWIGLU,
                          nullptr, nullptr, m.pack_work, s, nullptr, nullptr, nullptr, &gu, rot_for(E),
                          tf_op(m, OP_GATE_UP)))) return rc;
      PartialSums dn = {};
      dn.in = m.ffn_part;
      dn.in_ss = m.ffn_ss;
      dn.S = m.ffn_S;
      dn.rows_p = m.ffn_rows_p;
      dn.F = F;
      dn.in_K = E;
      dn.act = m.act;
      if (m.down_part && next_packed(l, m.down_S)) {
        dn.out = m.down_part;
        if ((rc = tgemv_f32(pd->buf, wk, E, F, nullptr, nullptr, c.rms_eps, nullptr, TRX_EPI_STORE, nullptr, nullptr,
                            m.pack_work, s, nullptr, nullptr, nullptr, &dn, rot_for(F), tf_op(m, OP_DOWN)))) return rc;
        pend.in = m.down_part;
        pend.S = m.down_S;
        pend.rows_p = m.down_rows_p;
      } else {
        if ((rc = tgemv_f32(pd->buf, wk, E, F, nullptr, nullptr, c.rms_eps, m.x, TRX_EPI_RESID, xc, nullptr,
                            m.pack_work, s, nullptr, nullptr, nullptr, &dn, rot_for(F), tf_op(m, OP_DOWN)))) return rc;
        xc = m.x;
      }
      continue;
    }
    if (pg) {
      const float* xin;
      const PartialSums* pp = take(xin);
      if ((rc = tgemv_f32(pg->buf, wk, 2 * F, E, xin, PF(m, TRX_ROLE_FFN_NORM, l), c.rms_eps, m.act, TRX_EPI_SWIGLU,
                          nullptr, nullptr, m.pack_work, s, nullptr, nullptr, nullptr, pp, rot_for(E),
                          tf_op(m, OP_GATE_UP)))) return rc;
    } else if ((rc = projection(m, OP_GATE_UP, l, P(m, TRX_ROLE_FFN_GATE, l), wk, 2 * F, E, xc,
                                 PF(m, TRX_ROLE_FFN_NORM, l), m.act, TRX_EPI_SWIGLU, nullptr, s))) {
      return rc;
    }
    if (pd && m.down_part && next_packed(l, m.down_S)) {
      PartialSums out = {};
      out.out = m.down_part;
      if ((rc = tgemv_f32(pd->buf, wk, E, F, m.act, nullptr, c.rms_eps, nullptr, TRX_EPI_STORE, nullptr, nullptr,
                          m.pack_work, s, nullptr, nullptr, nullptr, &out, rot_for(F), tf_op(m, OP_DOWN)))) return rc;
      pend.in = m.down_part;
      pend.S = m.down_S;
      pend.rows_p = m.down_rows_p;
    } else {
      if ((rc = projection(m, OP_DOWN, l, P(m, TRX_ROLE_FFN_DOWN, l), wk, E, F, m.act, nullptr, m.x, TRX_EPI_RESID,
                           xc, s))) return rc;
      xc = m.x;
    }
  }
  // LM head with the output RMSNorm and the greedy argmax; skipped (by the kernel, reading the
  // position) on prefill positions before head_from.
  const int head_role = c.head_tied ? TRX_ROLE_TOK_EMB : TRX_ROLE_LM_HEAD;
  const int head_kind = c.head_tied ? c.emb_kind : c.head_kind;
  if (const PackedMat* ph = packed(OP_HEAD, 0)) {
    // The head GEMV stores its partial sums; a second launch spreads their reduction (and the
    // argmax) over the whole GPU instead of the tile columns' last blocks.
    const float* xin;
    const PartialSums* pp = take(xin);
    PartialSums hp = pp ? *pp : PartialSums{};
    hp.out = m.head_part;
    hp.out_ss = m.head_ss;
    if ((rc = tgemv_f32(ph->buf, head_kind, c.vocab, E, xin, PF(m, TRX_ROLE_OUT_NORM, 0), c.rms_eps, nullptr,
                        TRX_EPI_STORE, nullptr, nullptr, m.pack_work, s, m.pos(), m.head_from(), nullptr, &hp,
                        rot_for(E), tf_op(m, OP_HEAD))))
      return rc;
    if ((rc = tgemv_reduce_f32(m.head_part, m.head_ss, m.head_S, m.head_rows_p, c.vocab, E, c.rms_eps, m.logits,
                               m.slot, s, m.pos(), m.head_from())))
      return rc;
  } else if (head_kind == TRX_KIND_F16) {
    DenseParams dp = {};
    dp.W = P(m, head_role, 0);
    dp.kind = TRX_KIND_F16;
    dp.M = c.vocab;
    dp.K = E;
    dp.row_bytes = 2 * E;
    dp.x = xc;
    dp.norm_w = PF(m, TRX_ROLE_OUT_NORM, 0);
    dp.eps = c.rms_eps;
    dp.y = m.logits;
    dp.amax_slot = m.slot;
    dp.gate_pos = m.pos();
    dp.gate_from = m.head_from();
    if ((rc = launch_dense_gemv(dp, s))) return rc;
  } else {
    if ((rc = projection(m, OP_HEAD, 0, P(m, head_role, 0), head_kind, c.vocab, E, xc,
                          PF(m, TRX_ROLE_OUT_NORM, 0), m.logits, TRX_EPI_STORE, nullptr, s, m.slot, m.pos(),
                          m.head_from()))) return rc;
  }
  if (m.sampling) {
    SampleParams sp = {m.logits, c.vocab, m.smp_channels, kSmpWindow, m.pos(), m.head_from(), m.n_prompt(),
                       m.prompt(), m.out(), c.max_new, m.smp, (uint32_t*)(m.smp + 3), m.slot, m.smp_cand,
                       (unsigned*)(m.smp_cand + 32), m.prompt_ring};
    if ((rc = launch_sample(sp, s))) return rc;
  }
  m.hidden = xc;
  if (m.scoring) {
    ScoreParams sp = {xc, PF(m, TRX_ROLE_OUT_NORM, 0), c.rms_eps, E, m.hid_rows, c.max_ctx, m.logits, c.vocab,
                      m.pos(), m.head_from(), m.n_prompt(), m.prompt(), m.nll};
    if ((rc = launch_score(sp, s))) return rc;
  }
  return TRX_OK;
}

// Batched prefill of positions p0 .. p0 + R - 1 --------------------------------------------------

// The input planes of a projection of width K: RMSNorm (norm_w), and a rotated model's rotation of
// that width unless `plain` (the DeltaNet beta/alpha take the unrotated input).
static int pf_prep(Model& m, const float* x, int ldx, int K, int R, const float* norm_w, bool plain, hipStream_t s) {
  PrepParams pp = {};
  pp.x = x;
  pp.ldx = ldx;
  pp.K = K;
  pp.R = R;
  pp.norm_w = norm_w;
  pp.eps = m.cfg.rms_eps;
  pp.xh = m.pf_h;
  pp.xl = m.pf_l;
  pp.xs = m.pf_xs;
  pp.rs = m.pf_rs;
  if (m.cfg.hadamard_block && !plain) {
    int wi = 0;
    while (wi < 4 && m.cfg.hadamard_widths[wi] != K) ++wi;
    TRX_CHECK(wi < 4, TRX_E_INVALID, "rotated model: no rotation for input width %d", K);
    pp.signs = PF(m, TRX_ROLE_HADAMARD, wi);
    pp.B = m.cfg.hadamard_block;
    pp.scale = m.cfg.hadamard_scale;
  }
  return launch_prep(pp, s);
}

// One GEMM over the planes pf_prep left: W's rows (role, layer; the fused group starting there).
static int pf_gemm(Model& m, int role, int l, int kind, int M, int K, int R, int epi, float* y, int ldy,
                   hipStream_t s) {
  const Tensor& t = T(m, role, l);
  GemmParams g = {};
  g.W = m.arena + t.off;
  g.w_bytes = (uint32_t)std::min<size_t>(m.arena_bytes - t.off, 0xFFFFFFF0u);
  g.kind = kind;
  g.M = M;
  g.K = K;
  g.row_bytes = row_bytes_of(kind, K);
  g.code_off = kind == TRX_KIND_Q8 ? kBeat * cdiv(K / 32, 16) : row_geom(kind, K).code_off;
  g.xh = m.pf_h;
  g.xl = m.pf_l;
  g.xs = m.pf_xs;
  g.R = R;
  g.epi = epi;
  g.y = y;
  g.ldy = ldy;
  g.part = m.pf_part;
  g.part_floats = (size_t)kPfPartRow * m.pf_rows;
  return launch_gemm(g, s);
}

// Frees one of the model's device allocations (the stream must be idle for it).
static int dfree(Model& m, void* p, size_t bytes) {
  if (!p) return TRX_OK;
  auto it = std::find(m.allocs.begin(), m.allocs.end(), p);
  if (it != m.allocs.end()) m.allocs.erase(it);
  m.dev_bytes -= bytes;
  TRX_HIP(hipFree(p));
  return TRX_OK;
}

// Prefill buffers for chunks of up to R positions. Capacities grow in powers of two (at least
// 64 rows); the smaller buffers are freed when they grow, so prompts of growing length hold
// at most twice the largest chunk.
static int pf_alloc(Model& m, int R) {
  if (R <= m.pf_rows) return TRX_OK;
  const trx_model_config& c = m.cfg;
  const int E = c.n_embd, F = c.ffn_dim, hd = c.head_dim;
  const int qrows = c.n_head * hd * (c.attn_gated ? 2 : 1), kvrows = c.n_kv_head * hd;
  const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
  const int C = 2 * nq + nvh;
  const int kmax = std::max({E, F, c.n_head * hd, nvh});
  const int io = std::max(m.n_attn ? qrows + 2 * kvrows : 0, m.n_dn ? C + nvh : 0);
  const int att = std::max(c.n_head * hd, nvh);
  // (buffer, bytes per row) of every prefill buffer.
  const std::vector<std::pair<void**, size_t>> bufs = {
      {(void**)&m.pf_x, (size_t)E * 4},
      {(void**)&m.pf_h, (size_t)kmax * 2},
      {(void**)&m.pf_l, (size_t)kmax * 2},
      {(void**)&m.pf_xs, 4},
      {(void**)&m.pf_rs, 4},
      {(void**)&m.pf_qkv, (size_t)io * 4},
      {(void**)&m.pf_att, (size_t)att * 4},
      {(void**)&m.pf_act, (size_t)F * 4},
      {(void**)&m.pf_q, m.n_attn ? (size_t)c.n_head * hd * 4 : 0},
      {(void**)&m.pf_ba, m.n_dn ? (size_t)2 * c.dn_num_v_heads * 4 : 0},
      {(void**)&m.pf_conv, m.n_dn ? (size_t)C * 4 : 0},
      {(void**)&m.pf_oraw, m.n_dn ? (size_t)nvh * 4 : 0},
      {(void**)&m.pf_part, (size_t)kPfPartRow * 4}};
  int rc;
  if (m.pf_rows > 0) {
    TRX_HIP(hipStreamSynchronize(m.stream));
    for (auto& b : bufs) {
      if ((rc = dfree(m, *b.first, b.second * (size_t)m.pf_rows))) return rc;
      *b.first = nullptr;
    }
    m.pf_rows = 0;
  }
  int cap = 64;
  while (cap < R) cap *= 2;
  for (auto& b : bufs)
    if (b.second && (rc = dalloc(m, b.first, b.second * (size_t)cap))) return rc;
  m.pf_rows = cap;
  return TRX_OK;
}

static int run_prefill(Model& m, int p0, int R, hipStream_t s) {
  const trx_model_config& c = m.cfg;
  const int E = c.n_embd, hd = c.head_dim, F = c.ffn_dim, wk = c.weight_kind;
  const int qrows = c.n_head * hd * (c.attn_gated ? 2 : 1), kvrows = c.n_kv_head * hd;
  int rc;
  EmbedParams ep = {};
  ep.mode = c.emb_mode == 0 ? EMBED_TABLE : c.emb_mode == 1 ? EMBED_TERNARY : EMBED_RESTORE;
  ep.n_embd = E;
  ep.vocab = c.vocab;
  if (c.emb_mode == 2) {
    int wi = 0;
    while (wi < 4 && c.hadamard_widths[wi] != E) ++wi;
    ep.signs = PF(m, TRX_ROLE_HADAMARD, wi);
    ep.hblock = c.hadamard_block;
  }
  if (c.emb_mode == 0) {
    ep.mant = (const int16_t*)P(m, TRX_ROLE_TOK_EMB16, 0);
    ep.exps = (const int32_t*)P(m, TRX_ROLE_TOK_EMB16_EXP, 0);
  } else {
    ep.rows = P(m, TRX_ROLE_TOK_EMB, 0);
    ep.kind = c.emb_kind;
    ep.row_bytes = row_bytes_of(c.emb_kind, E);
    ep.code_off = row_geom(c.emb_kind, E).code_off;
  }
  if ((rc = launch_embed_rows(ep, m.prompt(), p0, R, m.pf_x, s))) return rc;

  for (int l = 0; l < c.n_layer; ++l) {
    if (m.is_dn(l)) {
      const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
      const int C = 2 * nq + nvh, nv = c.dn_num_v_heads;
      // beta|alpha (Q8) from the unrotated normed input, then qkv|z.
      if ((rc = pf_prep(m, m.pf_x, E, E, R, PF(m, TRX_ROLE_ATTN_NORM, l), true, s))) return rc;
      if ((rc = pf_gemm(m, TRX_ROLE_SSM_BETA, l, TRX_KIND_Q8, 2 * nv, E, R, GM_STORE, m.pf_ba, 2 * nv, s))) return rc;
      if (c.hadamard_block && (rc = pf_prep(m, m.pf_x, E, E, R, PF(m, TRX_ROLE_ATTN_NORM, l), false, s))) return rc;
      if ((rc = pf_gemm(m, TRX_ROLE_ATTN_QKV, l, wk, C + nvh, E, R, GM_STORE, m.pf_qkv, C + nvh, s))) return rc;
      DnRowsParams dp = {};
      dp.io = m.pf_qkv;
      dp.ld_io = C + nvh;
      dp.taps = PF(m, TRX_ROLE_SSM_CONV, l);
      dp.conv_state = m.conv_state + (size_t)m.dn_index[l] * (c.dn_conv_kernel - 1) * C;
      dp.conv_out = m.pf_conv;
      dp.ba = m.pf_ba;
      dp.A = PF(m, TRX_ROLE_SSM_A, l);
      dp.dt = PF(m, TRX_ROLE_SSM_DT, l);
      dp.norm_w = PF(m, TRX_ROLE_SSM_NORM, l);
      dp.S = m.dn_state + (size_t)m.dn_index[l] * nvh * c.dn_k_head_dim;
      dp.o_raw = m.pf_oraw;
      dp.out = m.pf_att;
      dp.R = R;
      dp.C = C;
      dp.Kc = c.dn_conv_kernel;
      dp.nq = nq;
      dp.nv = nv;
      dp.nk = c.dn_num_k_heads;
      dp.hk = c.dn_k_head_dim;
      dp.hv = c.dn_v_head_dim;
      dp.eps = c.rms_eps;
      if ((rc = launch_dn_rows(dp, s))) return rc;
      if ((rc = pf_prep(m, m.pf_att, nvh, nvh, R, nullptr, false, s))) return rc;
      if ((rc = pf_gemm(m, TRX_ROLE_SSM_OUT, l, wk, E, nvh, R, GM_RESID, m.pf_x, E, s))) return rc;
    } else {
      const int M = qrows + 2 * kvrows;
      if ((rc = pf_prep(m, m.pf_x, E, E, R, PF(m, TRX_ROLE_ATTN_NORM, l), false, s))) return rc;
      if ((rc = pf_gemm(m, TRX_ROLE_ATTN_Q, l, wk, M, E, R, GM_STORE, m.pf_qkv, M, s))) return rc;
      const size_t per = (size_t)c.n_kv_head * c.max_ctx * hd;
      RopeKvParams rp = {};
      rp.qkv = m.pf_qkv;
      rp.ldq = M;
      rp.q_norm = PF(m, TRX_ROLE_ATTN_Q_NORM, l);
      rp.k_norm = PF(m, TRX_ROLE_ATTN_K_NORM, l);
      rp.rope_freq = m.rope_dev;
      rp.rope_cs = m.rope_cs;
      rp.rope_tab = c.rope_table ? (const int16_t*)P(m, TRX_ROLE_ROPE_TAB, 0) : nullptr;
      rp.p0 = p0;
      rp.R = R;
      rp.kcache = m.kcache + (size_t)m.attn_index[l] * per;
      rp.vcache = m.vcache + (size_t)m.attn_index[l] * per;
      rp.q_out = m.pf_q;
      rp.n_head = c.n_head;
      rp.n_kv = c.n_kv_head;
      rp.hd = hd;
      rp.rope_n = c.rope_dims ? c.rope_dims : hd;
      rp.max_ctx = c.max_ctx;
      rp.gated = c.attn_gated;
      rp.eps = c.rms_eps;
      if ((rc = launch_rope_kv(rp, s))) return rc;
      AttnPrefillParams ap = {};
      ap.q = m.pf_q;
      ap.qkv = m.pf_qkv;
      ap.ldq = M;
      ap.kcache = rp.kcache;
      ap.vcache = rp.vcache;
      ap.out = m.pf_att;
      ap.p0 = p0;
      ap.R = R;
      ap.n_head = c.n_head;
      ap.n_kv = c.n_kv_head;
      ap.hd = hd;
      ap.max_ctx = c.max_ctx;
      ap.gated = c.attn_gated;
      if ((rc = launch_attn_prefill(ap, s))) return rc;
      if ((rc = pf_prep(m, m.pf_att, c.n_head * hd, c.n_head * hd, R, nullptr, false, s))) return rc;
      if ((rc = pf_gemm(m, TRX_ROLE_ATTN_OUT, l, wk, E, c.n_head * hd, R, GM_RESID, m.pf_x, E, s))) return rc;
    }
    if ((rc = pf_prep(m, m.pf_x, E, E, R, PF(m, TRX_ROLE_FFN_NORM, l), false, s))) return rc;
    if ((rc = pf_gemm(m, TRX_ROLE_FFN_GATE, l, wk, 2 * F, E, R, GM_SWIGLU, m.pf_act, F, s))) return rc;
    if ((rc = pf_prep(m, m.pf_act, F, F, R, nullptr, false, s))) return rc;
    if ((rc = pf_gemm(m, TRX_ROLE_FFN_DOWN, l, wk, E, F, R, GM_RESID, m.pf_x, E, s))) return rc;
  }
  // The last position's residual is readable as the last forward's (TRX_READ_RESIDUAL), and the
  // control words move on.
  TRX_HIP(hipMemcpyAsync(m.hidden, m.pf_x + (size_t)(R - 1) * E, (size_t)E * 4, hipMemcpyDeviceToDevice, s));
  return launch_prefill_ctl(m.pos(), m.cur_tok(), m.prompt(), p0 + R - 1, s);
}

}  // namespace trx

using namespace trx;

#define TRX_API extern "C" __attribute__((visibility("default")))

struct trx_model {
  Model m;
};

TRX_API int trx_model_create(const trx_model_config* cfg, const float* rope_freq, trx_model** out) {
  TRX_CHECK(cfg && out && rope_freq, TRX_E_INVALID, "trx_model_create: null argument");
  *out = nullptr;
  const trx_model_config& c = *cfg;
  TRX_CHECK(c.n_layer > 0 && c.n_layer <= 128 && c.n_embd % 128 == 0 && c.ffn_dim % 128 == 0 &&
            c.head_dim > 0 && c.n_head % (c.n_kv_head ? c.n_kv_head : 1) == 0 && c.vocab > 0 &&
            c.max_ctx > 0 && c.max_new > 0, TRX_E_INVALID,
            "trx_model_create: unsupported geometry");
  TRX_CHECK(c.weight_kind == TRX_KIND_TERNARY || c.weight_kind == TRX_KIND_TERNARY5, TRX_E_INVALID,
            "trx_model_create: weight_kind must be ternary");
  TRX_CHECK(c.emb_mode >= 0 && c.emb_mode <= 2, TRX_E_INVALID, "trx_model_create: emb_mode %d", c.emb_mode);
  if (c.emb_mode == 2) {
    bool has = false;
    for (int i = 0; i < 4; ++i) has = has || (c.hadamard_block && c.hadamard_widths[i] == c.n_embd);
    TRX_CHECK(has && c.n_embd <= 8192 && (c.emb_kind == TRX_KIND_TERNARY || c.emb_kind == TRX_KIND_TERNARY5),
              TRX_E_INVALID, "trx_model_create: the embedding restore needs a rotated n_embd width (<= 8192) and ternary rows");
  }
  if (c.hadamard_block) {
    const int B = c.hadamard_block;
    TRX_CHECK(B >= 64 && B <= 1024 && (B & (B - 1)) == 0 && c.hadamard_scale > 0.f, TRX_E_INVALID,
              "trx_model_create: Hadamard block %d unsupported", B);
    TRX_CHECK(c.head_tied || c.head_kind != TRX_KIND_F16, TRX_E_INVALID,
              "trx_model_create: a rotated model runs one kernel per operation with a ternary head");
    for (int i = 0; i < 4; ++i)
      TRX_CHECK(c.hadamard_widths[i] >= 0 && c.hadamard_widths[i] % B == 0, TRX_E_INVALID,
                "trx_model_create: rotation width %d is not a multiple of the block", c.hadamard_widths[i]);
  }
  trx_model* h = new trx_model();
  Model& m = h->m;
  m.cfg = c;
  const int rope_n = c.rope_dims ? c.rope_dims : c.head_dim;
  m.rope_freq.assign(rope_freq, rope_freq + rope_n / 2);
  for (int l = 0; l < c.n_layer; ++l) {
    m.attn_index.push_back(m.is_dn(l) ? -1 : m.n_attn);
    m.dn_index.push_back(m.is_dn(l) ? m.n_dn : -1);
    if (m.is_dn(l)) ++m.n_dn; else ++m.n_attn;
  }
  size_t cur = 0;
  plan_arena(m, cur);
  m.arena_bytes = cur;
  int rc;
  auto fail = [&](int code) { trx_model_destroy(h); return code; };
  if ((rc = dalloc(m, (void**)&m.arena, m.arena_bytes))) return fail(rc);
  if ((rc = plan_packed(m))) return fail(rc);
  const int hd = c.head_dim;
  m.n_split = attention_splits(c.n_kv_head, c.head_dim, c.max_ctx);
  if (m.n_split < 0) {
    set_error("trx_model_create: context %d is too long for the attention kernel", c.max_ctx);
    return fail(TRX_E_INVALID);
  }
  const int splits = m.n_split;
  const size_t kv = (size_t)m.n_attn * c.n_kv_head * c.max_ctx * hd;
  if (m.n_attn) {
    if ((rc = dalloc(m, (void**)&m.kcache, kv * 2))) return fail(rc);
    if ((rc = dalloc(m, (void**)&m.vcache, kv * 2))) return fail(rc);
  }
  const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
  const int C = 2 * nq + nvh;
  if (m.n_dn) {
    if ((rc = dalloc(m, (void**)&m.conv_state, (size_t)m.n_dn * (c.dn_conv_kernel - 1) * C * 4))) return fail(rc);
    if ((rc = dalloc(m, (void**)&m.dn_state, (size_t)m.n_dn * c.dn_num_v_heads * c.dn_v_head_dim * c.dn_k_head_dim * 4))) return fail(rc);
    if ((rc = dalloc(m, (void**)&m.dn_io, (size_t)(C + nvh) * 4 * 2))) return fail(rc);
    if ((rc = dalloc(m, (void**)&m.dn_ba, (size_t)c.dn_num_v_heads * 2 * 4))) return fail(rc);
    if ((rc = dalloc(m, (void**)&m.dn_out, (size_t)nvh * 4))) return fail(rc);
  }
  const int qrows = c.n_head * hd * (c.attn_gated ? 2 : 1);
  if ((rc = dalloc(m, (void**)&m.x, (size_t)c.n_embd * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.x2, (size_t)c.n_embd * 4))) return fail(rc);
  if (c.hadamard_block) {
    const int wmax = std::max({c.hadamard_widths[0], c.hadamard_widths[1], c.hadamard_widths[2],
                               c.hadamard_widths[3]});
    if ((rc = dalloc(m, (void**)&m.xrot, (size_t)wmax * 4))) return fail(rc);
  }
  m.hidden = m.x;
  if ((rc = dalloc(m, (void**)&m.qkv, (size_t)(qrows + 2 * c.n_kv_head * hd) * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.attn_out, (size_t)c.n_head * hd * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.act, (size_t)c.ffn_dim * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.logits, (size_t)c.vocab * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.hid_last, (size_t)c.n_embd * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.part_m, (size_t)c.n_head * splits * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.part_l, (size_t)c.n_head * splits * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.part_o, (size_t)c.n_head * splits * hd * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.attn_done, (size_t)std::max(c.n_kv_head, 1) * kDoneStride * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.rope_dev, (size_t)rope_n * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.rope_cs, (size_t)(c.max_ctx + 1) * rope_n * 4))) return fail(rc);
  m.prompt_ring = c.max_ctx + kSmpWindow;
  if ((rc = dalloc(m, (void**)&m.ctl, (size_t)(8 + m.prompt_ring + c.max_new) * 4))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.slot, 8))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.smp, 16))) return fail(rc);
  if ((rc = dalloc(m, (void**)&m.smp_cand, 33 * 8))) return fail(rc);
  TRX_HIP(hipMemset(m.smp_cand, 0, 33 * 8));
  {
    const float cfg0[4] = {0.f, 1.f, 1.f, 0.f};
    const uint32_t rng0 = 0x9E3779B9u;         // the firmware's initial stream
    TRX_HIP(hipMemcpy(m.smp, cfg0, 16, hipMemcpyHostToDevice));
    TRX_HIP(hipMemcpy(m.smp + 3, &rng0, 4, hipMemcpyHostToDevice));
  }
  TRX_HIP(hipMemcpy(m.rope_dev, m.rope_freq.data(), m.rope_freq.size() * 4, hipMemcpyHostToDevice));
  {
    // cos and sin of the float32 angle pos * f_i (the product rounded as fastref's float32
    // angles are, model/fastref.py:62-63,229-235), each evaluated in double and rounded once.
    const int half = rope_n / 2;
    std::vector<float> tab((size_t)c.max_ctx * rope_n);
    for (int pos = 0; pos < c.max_ctx; ++pos)
      for (int i = 0; i < half; ++i) {
        const float ang = (float)pos * m.rope_freq[i];
        tab[(size_t)pos * rope_n + i] = (float)cos((double)ang);
        tab[(size_t)pos * rope_n + half + i] = (float)sin((double)ang);
      }
    TRX_HIP(hipMemcpy(m.rope_cs, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
  }
  {
    hipError_t e = hipStreamCreateWithFlags(&m.stream, hipStreamNonBlocking);
    if (e != hipSuccess) { set_error("stream: %s", hipGetErrorString(e)); return fail(TRX_E_HIP); }
  }
  *out = h;
  return trx_model_reset(h);
}

TRX_API int trx_model_destroy(trx_model* h) {
  if (!h) return TRX_OK;
  Model& m = h->m;
  // Teardown is best effort: errors here have no caller to act on them.
  if (m.graph_exec) (void)hipGraphExecDestroy(m.graph_exec);
  if (m.graph) (void)hipGraphDestroy(m.graph);
  if (m.stream) (void)hipStreamSynchronize(m.stream);
  for (void* p : m.allocs) (void)hipFree(p);
  if (m.stream) (void)hipStreamDestroy(m.stream);
  delete h;
  return TRX_OK;
}

TRX_API int trx_model_set_sampling(trx_model* h, float temperature, float top_p, float repetition,
                                   uint32_t seed, int n_channels) {
  TRX_CHECK(h && n_channels >= 1, TRX_E_INVALID, "trx_model_set_sampling: bad argument");
  Model& m = h->m;
  // firmware/infer.c:401-407: a negative temperature is 0, top_p outside (0, 1] is 1, a
  // repetition below 1 is 1, seed 0 keeps the stream.
  const float cfg[3] = {temperature < 0.f ? 0.f : temperature, (top_p <= 0.f || top_p > 1.f) ? 1.f : top_p,
                        repetition < 1.f ? 1.f : repetition};
  TRX_HIP(hipStreamSynchronize(m.stream));
  TRX_HIP(hipMemcpy(m.smp, cfg, 12, hipMemcpyHostToDevice));
  if (seed) TRX_HIP(hipMemcpy(m.smp + 3, &seed, 4, hipMemcpyHostToDevice));
  const bool on = cfg[0] > 0.f || cfg[2] > 1.f;
  if (on != m.sampling || n_channels != m.smp_channels) {
    // The captured position has (or lacks) the sampling launch: capture again.
    if (m.graph_exec) (void)hipGraphExecDestroy(m.graph_exec);
    if (m.graph) (void)hipGraphDestroy(m.graph);
    m.graph_exec = nullptr;
    m.graph = nullptr;
  }
  m.sampling = on;
  m.smp_channels = n_channels;
  return TRX_OK;
}

TRX_API int trx_model_set_tensor(trx_model* h, int role, int layer, const void* data, size_t bytes) {
  TRX_CHECK(h && data, TRX_E_INVALID, "trx_model_set_tensor: null argument");
  Model& m = h->m;
  auto it = m.tensors.find({role, layer});
  TRX_CHECK(it != m.tensors.end(), TRX_E_INVALID, "model has no tensor role=%d layer=%d", role, layer);
  TRX_CHECK(bytes == it->second.bytes, TRX_E_INVALID,
            "tensor role=%d layer=%d: %zu bytes given, %zu expected (%d x %d, kind %d)", role, layer,
            bytes, it->second.bytes, it->second.rows, it->second.cols, it->second.kind);
  TRX_HIP(hipMemcpy(m.arena + it->second.off, data, bytes, hipMemcpyHostToDevice));
  it->second.loaded = true;
  m.pack_dirty = true;
  return TRX_OK;
}

TRX_API int trx_model_synthesize(trx_model* h, uint32_t seed, const float* ranges) {
  // ranges: {scale_lo, scale_span, norm_lo, norm_span} as float32 (computed by the caller the
  // way the host generator computes them, so both sides round alike).
  TRX_CHECK(h && ranges, TRX_E_INVALID, "trx_model_synthesize: null argument");
  Model& m = h->m;
  int rc;
  for (auto& kv : m.tensors) {
    const int role = kv.first.first, layer = kv.first.second;
    Tensor& t = kv.second;
    const uint32_t tid = (uint32_t)(layer * 32 + role);
    if (t.kind == TRX_KIND_TERNARY || t.kind == TRX_KIND_TERNARY5) {
      SynthParams sp = {};
      sp.out = m.arena + t.off;
      sp.kind = t.kind;
      sp.rows = t.rows;
      sp.cols = t.cols;
      sp.row_bytes = row_bytes_of(t.kind, t.cols);
      sp.code_off = row_geom(t.kind, t.cols).code_off;
      sp.seed = seed;
      sp.tensor_id = tid;
      sp.lo = ranges[0];
      sp.span = ranges[1];
      if ((rc = launch_synth_ternary(sp, m.stream))) return rc;
      t.loaded = true;
    } else if (t.kind == TRX_KIND_F32 && role != TRX_ROLE_TOK_EMB16_EXP) {
      float lo = ranges[2], span = ranges[3];
      int transform = 0;
      if (role == TRX_ROLE_SSM_CONV) { lo = -0.5f; span = 1.0f; }
      if (role == TRX_ROLE_SSM_A) { lo = -1.5f; span = 2.0f; transform = 1; }
      if (role == TRX_ROLE_SSM_DT) { lo = -2.0f; span = 2.5f; }
      if ((rc = launch_synth_f32((float*)(m.arena + t.off), (long long)t.rows * t.cols, seed, tid, lo,
                                 span, transform, m.stream))) return rc;
      t.loaded = true;
    } else if (t.kind != TRX_KIND_Q8) {
      TRX_CHECK(false, TRX_E_INVALID, "synthesize: tensor role=%d kind=%d has no generator", role, t.kind);
    }
    // Q8 rows (the DeltaNet beta|alpha, a few KB a layer) are left to the caller's
    // trx_model_set_tensor; a step refuses to run while any tensor is unset.
  }
  TRX_HIP(hipStreamSynchronize(m.stream));
  m.pack_dirty = true;
  return TRX_OK;
}

TRX_API int trx_model_reset(trx_model* h) {
  TRX_CHECK(h, TRX_E_INVALID, "trx_model_reset: null");
  Model& m = h->m;
  const trx_model_config& c = m.cfg;
  // The KV ring of this generation (firmware/hybrid.c:1148-1150): the pinned positions asked for,
  // at least the sinks and at most a quarter of the window, and the ring only where the window holds
  // more than twice them (kv_ring_on, hybrid.c:170-173). The request lasts one reset.
  const bool ring = m.kv_ring > 0 || (m.kv_ring < 0 && m.n_dn > 0);
  const int pin = std::max(kKvSinks, std::min(m.kv_pin_next, c.max_ctx / 4));
  m.kv_pin = ring && !c.rope_table && c.max_ctx > 2 * pin ? pin : 0;
  m.kv_pin_next = kKvSinks;
  int init[8] = {-1, 0, 0, 0, 0, -1, 0, m.kv_pin};
  m.host_pos = -1;
  m.host_n_fed = 0;
  m.host_head_from = 0;
  TRX_HIP(hipMemcpyAsync(m.ctl, init, sizeof init, hipMemcpyHostToDevice, m.stream));
  TRX_HIP(hipMemsetAsync(m.slot, 0, 8, m.stream));
  if (m.n_dn) {
    const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
    TRX_HIP(hipMemsetAsync(m.conv_state, 0, (size_t)m.n_dn * (c.dn_conv_kernel - 1) * (2 * nq + nvh) * 4, m.stream));
    TRX_HIP(hipMemsetAsync(m.dn_state, 0, (size_t)m.n_dn * nvh * c.dn_k_head_dim * 4, m.stream));
  }
  TRX_HIP(hipStreamSynchronize(m.stream));
  return TRX_OK;
}

// The device regions a forward reads and rewrites from one position to the next: the control words
// with the fed and generated tokens, the argmax slot, the sampler's settings, stream and candidates,
// and every DeltaNet layer's conv window and recurrent matrix. The KV rows are not among them: a
// forward appends the row of its own position, so rows past a restored position are written again
// before any forward reads them.
struct StateRegion {
  void* p;
  size_t bytes;
};
static std::vector<StateRegion> state_regions(Model& m) {
  const trx_model_config& c = m.cfg;
  std::vector<StateRegion> r = {{m.ctl, (size_t)(8 + m.prompt_ring + c.max_new) * 4},
                                {m.slot, 8},
                                {m.smp, 16},
                                {m.smp_cand, 33 * 8}};
  if (m.n_dn) {
    const int nq = c.dn_num_k_heads * c.dn_k_head_dim, nvh = c.dn_num_v_heads * c.dn_v_head_dim;
    r.push_back({m.conv_state, (size_t)m.n_dn * (c.dn_conv_kernel - 1) * (2 * nq + nvh) * 4});
    r.push_back({m.dn_state, (size_t)m.n_dn * nvh * c.dn_k_head_dim * 4});
  }
  return r;
}

TRX_API int trx_model_checkpoint(trx_model* h, int op) {
  // firmware/infer.c:1926-1960 forward_checked with hybrid.c:2904-2930 hybrid_ckpt_save/restore:
  // save the state after the forwards enqueued so far; restore puts it back, so the next forwards
  // run again from there and give the same results.
  TRX_CHECK(h && (op == TRX_CKPT_SAVE || op == TRX_CKPT_RESTORE), TRX_E_INVALID,
            "trx_model_checkpoint: bad arguments");
  Model& m = h->m;
  const std::vector<StateRegion> regs = state_regions(m);
  size_t total = 0;
  for (const StateRegion& s : regs) total += (s.bytes + 255) / 256 * 256;
  if (op == TRX_CKPT_SAVE) {
    if (!m.ckpt) {
      int rc;
      if ((rc = dalloc(m, (void**)&m.ckpt, total))) return rc;
      m.ckpt_bytes = total;
    }
    TRX_CHECK(m.ckpt_bytes == total, TRX_E_STATE, "trx_model_checkpoint: state size changed");
    size_t off = 0;
    for (const StateRegion& s : regs) {
      TRX_HIP(hipMemcpyAsync(m.ckpt + off, s.p, s.bytes, hipMemcpyDeviceToDevice, m.stream));
      off += (s.bytes + 255) / 256 * 256;
    }
    m.ck_pos = m.host_pos;
    m.ck_n_fed = m.host_n_fed;
    m.ck_head_from = m.host_head_from;
    m.ck_kv_pin = m.kv_pin;
    m.ck_lowest = 0x7fffffff;
    m.ckpt_valid = true;
    return TRX_OK;
  }
  TRX_CHECK(m.ckpt_valid, TRX_E_STATE, "trx_model_checkpoint: no checkpoint saved");
  // The KV rows are not in the checkpoint: a forward since then at or below its position (after a
  // reset) rewrote rows the restored state reads.
  TRX_CHECK(m.ck_lowest > m.ck_pos, TRX_E_STATE,
            "trx_model_checkpoint: a forward at position %d since the checkpoint at %d rewrote its KV rows",
            m.ck_lowest, m.ck_pos);
  // Past the window a forward at position q writes the KV ring slot of position q - (max_ctx -
  // pin), which the forwards from the checkpoint on still read until they reach q: after one
  // forward that slot's position has left the window anyway (the firmware re-runs one forward),
  // after more the restored state would attend to rows written by the forwards it undoes.
  TRX_CHECK(!m.ck_kv_pin || m.host_pos < std::max(m.cfg.max_ctx, m.ck_pos + 2), TRX_E_STATE,
            "trx_model_checkpoint: %d forwards past the KV window since the checkpoint at position %d "
            "(at most one can be undone there)", m.host_pos - m.ck_pos, m.ck_pos);
  size_t off = 0;
  for (const StateRegion& s : regs) {
    TRX_HIP(hipMemcpyAsync(s.p, m.ckpt + off, s.bytes, hipMemcpyDeviceToDevice, m.stream));
    off += (s.bytes + 255) / 256 * 256;
  }
  m.host_pos = m.ck_pos;
  m.host_n_fed = m.ck_n_fed;
  m.host_head_from = m.ck_head_from;
  m.kv_pin = m.ck_kv_pin;
  m.ck_lowest = 0x7fffffff;
  return TRX_OK;
}

TRX_API int trx_model_set_kv_ring(trx_model* h, int enable, int pin) {
  // The console's `kvring on|off` and hybrid_set_pin (firmware/hybrid.c:156-168): both take effect
  // at the next reset.
  TRX_CHECK(h && enable >= -1 && enable <= 1 && pin >= 0, TRX_E_INVALID, "trx_model_set_kv_ring: bad arguments");
  Model& m = h->m;
  TRX_CHECK(enable <= 0 || !m.cfg.rope_table, TRX_E_INVALID,
            "trx_model_set_kv_ring: the image's RoPE table has no rows past max_ctx");
  m.kv_ring = enable;
  m.kv_pin_next = pin;
  return TRX_OK;
}

static int check_loaded(Model& m) {
  for (auto& kv : m.tensors)
    TRX_CHECK(kv.second.loaded, TRX_E_STATE, "tensor role=%d layer=%d was never set", kv.first.first, kv.first.second);
  return TRX_OK;
}

TRX_API int trx_model_set_prompt(trx_model* h, const int32_t* tokens, int n, int head_from) {
  // Feeds tokens at the next n positions (after the steps already enqueued); logits are produced
  // from absolute position head_from on (-1: the last fed token).
  TRX_CHECK(h && tokens && n > 0, TRX_E_INVALID, "trx_model_set_prompt: bad arguments");
  Model& m = h->m;
  const int first = m.host_pos + 1;
  // With the KV ring the positions go on past the window; a call feeds at most a window's worth.
  TRX_CHECK(m.kv_pin > 0 ? n <= m.cfg.max_ctx : first + n <= m.cfg.max_ctx, TRX_E_STATE,
            "%d tokens after position %d exceed max_ctx %d", n, m.host_pos, m.cfg.max_ctx);
  for (int i = 0; i < n; ++i)
    TRX_CHECK(tokens[i] >= 0 && tokens[i] < m.cfg.vocab, TRX_E_INVALID, "token %d out of range", tokens[i]);
  const int n_fed = first + n, hf = head_from < 0 ? first + n - 1 : head_from;
  // The fed tokens' ring holds max_ctx + 64 positions: n <= max_ctx new ones leave the 64 before
  // them, which the sampler's repetition window reads, in place.
  const int i0 = first % m.prompt_ring, n1 = std::min(n, m.prompt_ring - i0);
  TRX_HIP(hipMemcpyAsync(m.prompt() + i0, tokens, (size_t)n1 * 4, hipMemcpyHostToDevice, m.stream));
  if (n1 < n)
    TRX_HIP(hipMemcpyAsync(m.prompt(), tokens + n1, (size_t)(n - n1) * 4, hipMemcpyHostToDevice, m.stream));
  TRX_HIP(hipMemcpyAsync(m.ctl + 1, &n_fed, 4, hipMemcpyHostToDevice, m.stream));
  TRX_HIP(hipMemcpyAsync(m.ctl + 3, &hf, 4, hipMemcpyHostToDevice, m.stream));
  TRX_HIP(hipStreamSynchronize(m.stream));
  m.host_n_fed = n_fed;
  m.host_head_from = hf;
  return TRX_OK;
}

TRX_API int trx_model_step(trx_model* h, int n_steps, int use_graph) {
  TRX_CHECK(h && n_steps >= 0, TRX_E_INVALID, "trx_model_step: bad arguments");
  Model& m = h->m;
  int rc;
  if ((rc = check_loaded(m))) return rc;
  if ((rc = ensure_packed(m))) return rc;
  if (use_graph && !m.graph_exec) {
    TRX_HIP(hipStreamBeginCapture(m.stream, hipStreamCaptureModeThreadLocal));
    rc = run_step(m, m.stream);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(m.stream, &g);
    if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
    TRX_CHECK(e == hipSuccess, TRX_E_HIP, "graph capture: %s", hipGetErrorString(e));
    m.graph = g;
    TRX_HIP(hipGraphInstantiate(&m.graph_exec, m.graph, nullptr, nullptr, 0));
  }
  TRX_CHECK(m.kv_pin > 0 || m.host_pos + n_steps < m.cfg.max_ctx, TRX_E_STATE,
            "%d steps after position %d exceed max_ctx %d", n_steps, m.host_pos, m.cfg.max_ctx);
  if (n_steps > 0) m.ck_lowest = std::min(m.ck_lowest, m.host_pos + 1);
  for (int i = 0; i < n_steps; ++i) {
    ++m.host_pos;
    if (use_graph) {
      TRX_HIP(hipGraphLaunch(m.graph_exec, m.stream));
    } else if ((rc = run_step(m, m.stream))) {
      return rc;
    }
  }
  return TRX_OK;
}

TRX_API int trx_model_prefill(trx_model* h, int n, int chunk) {
  TRX_CHECK(h && n >= 0, TRX_E_INVALID, "trx_model_prefill: bad arguments");
  Model& m = h->m;
  int rc;
  if ((rc = check_loaded(m))) return rc;
  const int first = m.host_pos + 1;
  TRX_CHECK(first + n <= m.host_n_fed, TRX_E_STATE, "trx_model_prefill: positions %d..%d were not fed (%d fed)",
            first, first + n - 1, m.host_n_fed);
  TRX_CHECK(first + n <= m.host_head_from, TRX_E_STATE,
            "trx_model_prefill: position %d computes logits (head_from %d); step it instead", first + n - 1,
            m.host_head_from);
  if (n == 0) return TRX_OK;
  m.ck_lowest = std::min(m.ck_lowest, first);
  // Positions past the window (the KV ring) run one forward each.
  const int n_in = std::max(0, std::min(n, m.cfg.max_ctx - first));
  if (n_in > 0) {
    if (chunk <= 0) chunk = 1024;
    chunk = std::min(chunk, n_in);
    if ((rc = pf_alloc(m, chunk))) return rc;
    for (int p0 = first; p0 < first + n_in; p0 += chunk) {
      const int R = std::min(chunk, first + n_in - p0);
      if ((rc = run_prefill(m, p0, R, m.stream))) return rc;
    }
    m.host_pos = first + n_in - 1;
  }
  if (n_in < n) return trx_model_step(h, n - n_in, m.graph_exec != nullptr);
  return TRX_OK;
}

TRX_API int trx_model_finalize(trx_model* h) {
  TRX_CHECK(h, TRX_E_INVALID, "trx_model_finalize: null");
  Model& m = h->m;
  return launch_finalize(m.pos(), m.n_prompt(), m.slot, m.out(), m.cfg.max_new, m.stream);
}

// After the stream has drained: a kernel whose bounded wait timed out left garbage.
static int check_err(Model& m) {
  int e = 0;
  TRX_HIP(hipMemcpy(&e, m.err(), 4, hipMemcpyDeviceToHost));
  if (e) {
    const int zero = 0;
    TRX_HIP(hipMemcpy(m.err(), &zero, 4, hipMemcpyHostToDevice));
    TRX_CHECK(false, TRX_E_HIP, "a bounded wait timed out on the device (results of this call are invalid)");
  }
  return TRX_OK;
}

TRX_API int trx_model_sync(trx_model* h) {
  TRX_CHECK(h, TRX_E_INVALID, "trx_model_sync: null");
  TRX_HIP(hipStreamSynchronize(h->m.stream));
  return check_err(h->m);
}

TRX_API int trx_model_generate(trx_model* h, const int32_t* prompt, int n_prompt, int n_new,
                               int32_t* out, int use_graph) {
  TRX_CHECK(h && prompt && out && n_prompt > 0 && n_new > 0, TRX_E_INVALID, "trx_model_generate: bad arguments");
  Model& m = h->m;
  TRX_CHECK(n_new <= m.cfg.max_new, TRX_E_INVALID, "n_new %d exceeds max_new %d", n_new, m.cfg.max_new);
  TRX_CHECK(n_prompt <= m.cfg.max_ctx, TRX_E_INVALID, "prompt of %d tokens exceeds max_ctx", n_prompt);
  int rc;
  if ((rc = trx_model_reset(h))) return rc;
  TRX_CHECK(m.kv_pin > 0 || n_prompt + n_new - 1 <= m.cfg.max_ctx, TRX_E_STATE,
            "context of %d positions exceeds max_ctx %d", n_prompt + n_new - 1, m.cfg.max_ctx);
  if ((rc = trx_model_set_prompt(h, prompt, n_prompt, -1))) return rc;
  const int pre = m.cfg.prefill_chunk > 0 ? n_prompt - 1 : 0;
  if (pre && (rc = trx_model_prefill(h, pre, m.cfg.prefill_chunk))) return rc;
  if ((rc = trx_model_step(h, n_prompt - pre + n_new - 1, use_graph))) return rc;
  if ((rc = trx_model_finalize(h))) return rc;
  TRX_HIP(hipMemcpyAsync(out, m.out(), (size_t)n_new * 4, hipMemcpyDeviceToHost, m.stream));
  TRX_HIP(hipStreamSynchronize(m.stream));
  return check_err(m);
}

TRX_API int trx_model_score(trx_model* h, const int32_t* tokens, int n, float* nll, float* hidden) {
  TRX_CHECK(h && tokens && n >= 1, TRX_E_INVALID, "trx_model_score: bad arguments");
  Model& m = h->m;
  const trx_model_config& c = m.cfg;
  TRX_CHECK(n <= c.max_ctx, TRX_E_STATE, "trx_model_score: %d tokens exceed max_ctx %d", n, c.max_ctx);
  int rc;
  if (!m.nll) {
    if ((rc = dalloc(m, (void**)&m.nll, (size_t)c.max_ctx * 4))) return rc;
    if ((rc = dalloc(m, (void**)&m.hid_rows, (size_t)c.max_ctx * c.n_embd * 4))) return rc;
  }
  if ((rc = trx_model_reset(h))) return rc;
  if ((rc = trx_model_set_prompt(h, tokens, n, 0))) return rc;
  // Every position runs the head and the score launch; the captured graph has no score launch,
  // so these positions run eagerly.
  m.scoring = true;
  rc = trx_model_step(h, n, 0);
  m.scoring = false;
  if (rc) return rc;
  TRX_HIP(hipStreamSynchronize(m.stream));
  if ((rc = check_err(m))) return rc;
  if (nll && n > 1) TRX_HIP(hipMemcpy(nll, m.nll, (size_t)(n - 1) * 4, hipMemcpyDeviceToHost));
  if (hidden) TRX_HIP(hipMemcpy(hidden, m.hid_rows, (size_t)n * c.n_embd * 4, hipMemcpyDeviceToHost));
  return TRX_OK;
}

TRX_API int trx_model_project_head(trx_model* h, const float* hidden, int n, float* logits) {
  TRX_CHECK(h && hidden && logits && n >= 0, TRX_E_INVALID, "trx_model_project_head: bad arguments");
  Model& m = h->m;
  const trx_model_config& c = m.cfg;
  int rc;
  if ((rc = check_loaded(m))) return rc;
  if ((rc = ensure_packed(m))) return rc;
  if (!m.proj_x) {
    if ((rc = dalloc(m, (void**)&m.proj_x, (size_t)c.n_embd * 4))) return rc;
    if ((rc = dalloc(m, (void**)&m.proj_y, (size_t)c.vocab * 4))) return rc;
  }
  const int head_role = c.head_tied ? TRX_ROLE_TOK_EMB : TRX_ROLE_LM_HEAD;
  const int head_kind = c.head_tied ? c.emb_kind : c.head_kind;
  for (int i = 0; i < n; ++i) {
    TRX_HIP(hipMemcpyAsync(m.proj_x, hidden + (size_t)i * c.n_embd, (size_t)c.n_embd * 4, hipMemcpyHostToDevice,
                           m.stream));
    if (head_kind == TRX_KIND_F16) {
      DenseParams dp = {};
      dp.W = P(m, head_role, 0);
      dp.kind = TRX_KIND_F16;
      dp.M = c.vocab;
      dp.K = c.n_embd;
      dp.row_bytes = 2 * c.n_embd;
      dp.x = m.proj_x;
      dp.eps = c.rms_eps;
      dp.y = m.proj_y;
      if ((rc = launch_dense_gemv(dp, m.stream))) return rc;
    } else if ((rc = projection(m, OP_HEAD, 0, P(m, head_role, 0), head_kind, c.vocab, c.n_embd, m.proj_x, nullptr,
                                m.proj_y, TRX_EPI_STORE, nullptr, m.stream))) {
      return rc;
    }
    TRX_HIP(hipMemcpyAsync(logits + (size_t)i * c.vocab, m.proj_y, (size_t)c.vocab * 4, hipMemcpyDeviceToHost,
                           m.stream));
  }
  TRX_HIP(hipStreamSynchronize(m.stream));
  return TRX_OK;
}

TRX_API int trx_model_read(trx_model* h, int what, void* host, size_t bytes) {
  TRX_CHECK(h && host, TRX_E_INVALID, "trx_model_read: null argument");
  Model& m = h->m;
  int rc;
  const trx_model_config& c = m.cfg;
  const void* src = nullptr;
  size_t n = 0;
  switch (what) {
    case TRX_READ_LOGITS: src = m.logits; n = (size_t)c.vocab * 4; break;
    case TRX_READ_HIDDEN: src = m.hid_last; n = (size_t)c.n_embd * 4; break;
    case TRX_READ_RESIDUAL: src = m.hidden; n = (size_t)c.n_embd * 4; break;
    case TRX_READ_POSITION: src = m.pos(); n = 4; break;
    case TRX_READ_TOKEN: src = m.cur_tok(); n = 4; break;
    case TRX_READ_OUT: src = m.out(); n = (size_t)c.max_new * 4; break;
    case TRX_READ_SLOT: src = m.slot; n = 8; break;
    case TRX_READ_QKV:
      src = m.qkv;
      n = (size_t)(c.n_head * c.head_dim * (c.attn_gated ? 2 : 1) + 2 * c.n_kv_head * c.head_dim) * 4;
      break;
    case TRX_READ_ATTN: src = m.attn_out; n = (size_t)c.n_head * c.head_dim * 4; break;
    case TRX_READ_ACT: src = m.act; n = (size_t)c.ffn_dim * 4; break;
    default: TRX_CHECK(false, TRX_E_INVALID, "trx_model_read: unknown item %d", what);
  }
  TRX_CHECK(bytes <= n, TRX_E_INVALID, "trx_model_read: %zu bytes requested, %zu available", bytes, n);
  if (what == TRX_READ_HIDDEN) {
    // fastref's hidden state: the residual through the output RMSNorm (fastref.py:258).
    ScoreParams sp = {};
    sp.x = m.hidden;
    sp.out_norm = PF(m, TRX_ROLE_OUT_NORM, 0);
    sp.eps = c.rms_eps;
    sp.n = c.n_embd;
    sp.hid = m.hid_last;
    sp.max_rows = 1;
    if ((rc = launch_score(sp, m.stream))) return rc;
  }
  TRX_HIP(hipStreamSynchronize(m.stream));
  if ((rc = check_err(m))) return rc;
  TRX_HIP(hipMemcpy(host, src, bytes, hipMemcpyDeviceToHost));
  return TRX_OK;
}

TRX_API int trx_model_info(trx_model* h, int what, int64_t* value) {
  TRX_CHECK(h && value, TRX_E_INVALID, "trx_model_info: null argument");
  Model& m = h->m;
  switch (what) {
    case TRX_INFO_ARENA_BYTES: *value = (int64_t)m.arena_bytes; break;
    case TRX_INFO_DEVICE_BYTES: *value = (int64_t)m.dev_bytes; break;
    case TRX_INFO_STREAM: *value = (int64_t)(intptr_t)m.stream; break;
    case TRX_INFO_ATTN_SPLITS: *value = m.n_split; break;
    case TRX_INFO_ATTN_PASS: *value = attention_pass_positions(m.cfg.head_dim); break;
    case TRX_INFO_TABLE_FREE_OPS: *value = m.tf_ops; break;
    case TRX_INFO_KV_PIN: *value = m.kv_pin; break;
    case TRX_INFO_PACKED_OPS: *value = m.packed_ops; break;
    case TRX_INFO_WEIGHT_BYTES: {
      int64_t s = 0;
      for (auto& kv : m.tensors) s += (int64_t)kv.second.bytes;
      *value = s;
      break;
    }
    default: TRX_CHECK(false, TRX_E_INVALID, "trx_model_info: unknown item %d", what);
  }
  return TRX_OK;
}

TRX_API int trx_model_packed_ptr(trx_model* h, int op, int layer, void** packed, void** workspace) {
  TRX_CHECK(h && packed && workspace, TRX_E_INVALID, "trx_model_packed_ptr: null argument");
  Model& m = h->m;
  int rc;
  if ((rc = ensure_packed(m))) return rc;
  const int ids[] = {TRX_PACK_QKV, TRX_PACK_O, TRX_PACK_GATE_UP, TRX_PACK_DOWN, TRX_PACK_HEAD};
  int id = -1;
  for (int i = 0; i < 5; ++i) if (op == ids[i]) id = i;
  TRX_CHECK(id >= 0, TRX_E_INVALID, "trx_model_packed_ptr: op %d is not one TRX_PACK_* bit of a layer projection", op);
  auto it = m.packed.find({id, layer});
  TRX_CHECK(it != m.packed.end(), TRX_E_INVALID, "projection %d of layer %d is not packed", op, layer);
  *packed = it->second.buf;
  *workspace = m.pack_work;
  return TRX_OK;
}

TRX_API int trx_model_tensor_ptr(trx_model* h, int role, int layer, void** ptr, int64_t* bytes) {
  TRX_CHECK(h && ptr && bytes, TRX_E_INVALID, "trx_model_tensor_ptr: null argument");
  Model& m = h->m;
  auto it = m.tensors.find({role, layer});
  TRX_CHECK(it != m.tensors.end(), TRX_E_INVALID, "model has no tensor role=%d layer=%d", role, layer);
  *ptr = m.arena + it->second.off;
  *bytes = (int64_t)it->second.bytes;
  return TRX_OK;
}
