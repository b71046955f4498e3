/* libtrixium_hip: MI355X (gfx950) batch-1 ternary decode, C ABI.
 *
 * Every entry point returns 0 (TRX_OK) or a negative TRX_E_* code and leaves a message for
 * trx_last_error(). Buffers are device pointers owned by the caller unless stated; work is
 * enqueued on the given stream (NULL = the default stream) and is asynchronous unless stated.
 * No C++ exception crosses this boundary. Reference citations name the interface of
 * enjoy-digital/trixium each entry point stands in for.
 */
#ifndef TRIXIUM_H
#define TRIXIUM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRX_OK 0
#define TRX_E_INVALID (-1)   /* bad argument: null pointer, unsupported shape or kind */
#define TRX_E_HIP (-2)       /* HIP runtime error */
#define TRX_E_OVERFLOW (-3)  /* exact matvec: int48 accumulator or int32 result overflow */
#define TRX_E_NOMEM (-4)     /* device allocation failed */
#define TRX_E_STATE (-5)     /* call out of order (position past max_ctx, missing tensor) */

/* Tensor kinds (model/layout.py:45-54). */
#define TRX_KIND_TERNARY 0   /* 2-bit codes {0,1,2}, one fp16 scale per 128 */
#define TRX_KIND_Q8 1        /* int8, one fp16 scale per 32 */
#define TRX_KIND_F16 2
#define TRX_KIND_F32 3
#define TRX_KIND_NORM16 4
#define TRX_KIND_TERNARY5 5  /* the same trits, 5 per byte (26 bytes per 128-group) */

/* GEMV epilogues. */
#define TRX_EPI_STORE 0      /* y[m] = (W x)[m] */
#define TRX_EPI_RESID 1      /* y[m] = resid[m] + (W x)[m]   (resid may alias y) */
#define TRX_EPI_SWIGLU 2     /* rows [0,F) gate, [F,2F) up: y[m] = silu(g[m]) * u[m], m < F */

typedef void* trx_stream_t; /* a hipStream_t */

const char* trx_last_error(void);
int trx_version(void);

/* Device, memory, streams, events ---------------------------------------------------------- */
int trx_device_count(int* n);
int trx_set_device(int dev);
int trx_device_name(char* buf, int len);
/* Device allocation; every allocation is followed by 256 readable guard bytes. */
int trx_malloc(void** ptr, size_t bytes);
int trx_free(void* ptr);
int trx_memcpy_h2d(void* dst, const void* src, size_t bytes, trx_stream_t s);
int trx_memcpy_d2h(void* dst, const void* src, size_t bytes, trx_stream_t s);
int trx_memcpy_d2d(void* dst, const void* src, size_t bytes, trx_stream_t s);
int trx_memset_d8(void* dst, int value, size_t bytes, trx_stream_t s);
int trx_stream_create(trx_stream_t* s);
int trx_stream_destroy(trx_stream_t s);
int trx_stream_sync(trx_stream_t s);
int trx_event_create(void** ev);
int trx_event_destroy(void* ev);
int trx_event_record(void* ev, trx_stream_t s);
int trx_event_elapsed_ms(void* start, void* stop, float* ms);

/* Ternary GEMV -------------------------------------------------------------------------------
 * `rows` holds M row packets of a BONS tensor back to back (one channel): per row
 * ceil(G/16)*32 bytes of fp16 group scales, then the codes (2-bit: 32 bytes per group; trit5:
 * 26 bytes per group, the row padded to 32 bytes) (model/layout.py:184-217). K % 128 == 0. */

/* Exact engine matvec: int8 x, per-tensor B/R, int32 result (model/bitexact.py:101-119
 * matvec_ternary; the firmware's engine op 0, firmware/engine.h:40-70 + engine.c:238
 * engine_run). *status (device int32) is OR-ed with 1 when the int48 accumulator overflows and
 * with 2 when the int32 result does (where the reference asserts); the caller zeroes it. */
int trx_gemv_ternary_exact(const uint8_t* rows, int kind, int M, int K, const int8_t* x8, int B,
                           int R, int32_t* y, int32_t* status, trx_stream_t s);

/* Multi-row exact engine matvec (model/bitexact.py:121-125 matvec_ternary_rows): one pass over
 * the rows against n_rows (1..8) int8 vectors x8_rows[n_rows][K] (16-byte aligned,
 * n_rows * K <= 114688), y[n_rows][M]; row r equals trx_gemv_ternary_exact on x8_rows[r], and
 * *status is OR-ed the same way. Up to 4 rows run the single-row kernel once per row (faster at
 * that count); 5..8 rows share one pass over the weights. */
int trx_gemv_ternary_exact_rows(const uint8_t* rows, int kind, int M, int K, const int8_t* x8_rows,
                                int n_rows, int B, int R, int32_t* y, int32_t* status,
                                trx_stream_t s);

/* The firmware's activation quantizer (model/mirror.py:45-51 _quantize_f_pow2, firmware/infer.c:144
 * quantize_f_pow2): *e8 = frexp(max |x|) - 7 (0 for an all-zero x), x8[i] = clip(lroundf(x[i] *
 * 2^-e8), -127, 127), lroundf evaluated in float32 as model/mirror.py:34-35 does. One block;
 * K >= 1. */
int trx_quantize_f_pow2(const float* x, int K, int8_t* x8, int* e8, trx_stream_t s);

/* The projection through the engine, as the firmware runs it (model/mirror.py:663-678, the
 * non-exact matvec_f; firmware/infer_float.c:350 infer_matvec_f): x quantized by
 * trx_quantize_f_pow2, the exact engine matvec of trx_gemv_ternary_exact with the tensor's B and
 * R, y[m] = (float)result[m] * 2^(e8 + R - B) (float32). `workspace` holds
 * trx_gemv_quantized_geometry's bytes; *status is OR-ed as for trx_gemv_ternary_exact. */
int trx_gemv_quantized_geometry(int M, int K, size_t* workspace_bytes);
int trx_gemv_ternary_quantized(const uint8_t* rows, int kind, int M, int K, const float* x, int B, int R,
                               float* y, void* workspace, int32_t* status, trx_stream_t s);

/* Exact per-group sums gs[m*G + g] = sum (code-1)*x8 over group g (the engine's adder-tree
 * output, model/bitexact.py:110; debug form of engine op 0). */
int trx_gemv_ternary_groupsums(const uint8_t* rows, int kind, int M, int K, const int8_t* x8,
                               int32_t* gs, trx_stream_t s);

/* Float GEMV (the projection of model/fastref.py:119-125 HybridRef.matmul for one position):
 * fp32 x, optional fused RMSNorm prologue (norm_w != NULL: x <- x / rms(x) * norm_w,
 * fastref.py:143-145), fp32 y with an epilogue. x is quantised to int16 per 128-group inside
 * the kernel. x and norm_w must be 16-byte aligned. */
int trx_gemv_ternary_f32(const uint8_t* rows, int kind, int M, int K, const float* x,
                         const float* norm_w, float eps, float* y, int epilogue,
                         const float* resid, trx_stream_t s);

/* Multi-position float projection, the batched prefill's GEMM (the float counterpart of
 * model/bitexact.py:121-125 matvec_ternary_rows, one weight pass for many rows): y[r] = W xhat_r
 * for n rows x_r of K floats (xhat = x, or x / rms(x) * norm_w with norm_w != NULL), on the matrix
 * cores. W's rows are decoded to fp16 weights exactly as fastref's fp16 weight cache holds them
 * (model/fastref.py:104-116: (code - 1) * scale, or fp16(q * scale) for Q8) and xhat is split
 * into fp16 hi and lo planes, so each product is fp32-accurate. kind: TRX_KIND_TERNARY,
 * TRX_KIND_TERNARY5 or TRX_KIND_Q8. Epilogues: TRX_EPI_STORE y [n][M]; TRX_EPI_RESID y [n][M] +=;
 * TRX_EPI_SWIGLU (rows [0,F) gate, [F,2F) up) y [n][M/2]. A row of xhat at or above 2^14 in
 * magnitude is scaled by a power of two for the planes and back in the result (exact), so large
 * inputs stay finite. rows must be followed by 16 readable bytes; workspace holds 4*n*(K+1)
 * bytes. */
int trx_gemm_ternary_f32(const uint8_t* rows, int kind, int M, int K, const float* x, int n,
                         const float* norm_w, float eps, float* y, int epilogue, void* workspace,
                         trx_stream_t s);

/* Packed float GEMV: the decoder's projection (the same arithmetic as trx_gemv_ternary_f32, with
 * x kept in fp32) over a GPU-native copy of the rows. The copy cuts K into 256-column slices
 * (two 128-groups) and stores, per slice, the rows' code bytes and fp16 scales slice-major in
 * the order the kernel reads them; it holds the same bytes per row as the BONS packets. A block
 * of the kernel builds, for its slice, the table of every code byte's partial dot product with x
 * in LDS, so a code byte costs one LDS read and one add; per-slice partial sums are combined in
 * slice order (deterministic) by the block that completes a tile of rows last.
 *
 * trx_pack_geometry: bytes of the packed copy and of the workspace the GEMV needs.
 * trx_pack_ternary: rows (as for trx_gemv_ternary_f32) -> packed copy. swiglu = 1 packs a
 *   [gate | up] matrix (M = 2F, F even) for TRX_EPI_SWIGLU.
 * trx_gemv_packed_f32: y = W xhat, xhat = x or x / rms(x) * norm_w (fastref.py:119-125,143-145)
 *   with the epilogue; `workspace` holds trx_pack_geometry's workspace bytes, zeroed once before
 *   its first use (every call leaves it ready for the next); calls sharing a workspace must not
 *   overlap. x must be 16-byte aligned. */
int trx_pack_geometry(int kind, int M, int K, size_t* packed_bytes, size_t* workspace_bytes);
int trx_pack_ternary(const uint8_t* rows, int kind, int M, int K, int swiglu, uint8_t* packed,
                     trx_stream_t s);
int trx_gemv_packed_f32(const uint8_t* packed, int kind, int M, int K, const float* x,
                        const float* norm_w, float eps, float* y, int epilogue,
                        const float* resid, void* workspace, trx_stream_t s);

/* trx_gemv_packed_f32 without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The workspace is a fixed 24 MiB device array of the library (one
 * per GPU, held until the process ends), so the matrix's workspace (trx_pack_geometry) must fit
 * in it: TRX_E_INVALID otherwise (the 151936 x 4096 LM head fits). Calls on one GPU share the
 * array: calls that overlap on one GPU race. */
int trx_gemv_packed_f32_noalloc(const uint8_t* packed, int kind, int M, int K, const float* x,
                                const float* norm_w, float eps, float* y, int epilogue,
                                const float* resid, trx_stream_t s);

/* Many independent packed GEMVs in one dispatch (no counterpart in the reference, whose engine
 * runs one matvec op per submit, firmware/engine.c:111-238; for callers with many matrices and
 * vectors, such as the isolated matvec benchmark): y_i = W_i x_i, i < n_mat (<= 65535), matrix
 * i's packed copy (trx_pack_ternary) at packed + (i % n_copies) * mat_stride (a multiple of 256,
 * at least trx_pack_geometry's packed bytes; 1 <= n_copies <= n_mat), x_i at x + i * x_stride
 * (x 16-byte aligned, x_stride a multiple of 4 and >= K, or 0: one x for every matrix, whose
 * tables a block then reuses over several matrices, two K-slices per block; the copies must then
 * span under 2 GiB, and a row's slices are summed in pairs: within rounding of, not bit for bit
 * equal to, trx_gemv_packed_f32), y_i at y + i * y_stride. M <= 16384.
 * `workspace` holds trx_pack_batched_geometry's bytes of split-K partial sums (no zeroing
 * needed). */
int trx_pack_batched_geometry(int kind, int M, int K, int n_mat, size_t* workspace_bytes);
int trx_gemv_packed_batched_f32(const uint8_t* packed, size_t mat_stride, int n_mat, int n_copies, int kind,
                                int M, int K, const float* x, int x_stride, float* y, int y_stride,
                                void* workspace, trx_stream_t s);

/* Split-K partial sums handed from one packed GEMV to the next, as the decoder chains its
 * projections (no counterpart in the reference: its engine returns whole results; these let a
 * caller skip the per-GEMV reduction the same way).
 * trx_pack_partials_geometry: S (slices), rows_p (partial rows per slice) and bps (blocks per
 *   slice) of a matrix: a producer's partial buffer holds S * rows_p floats, its slice-sum
 *   buffer bps * S floats.
 * trx_gemv_packed_parts_f32: trx_gemv_packed_f32 with the partial-sum fields of `parts`
 *   (null: none). out != null: store the partial sums (part[s * rows_p + r] for slice s, packed
 *   row r) instead of y and skip the reduction; with norm_w the sums are of W (x * norm_w), not
 *   yet scaled by 1/rms(x), and each block stores its slice's sum of x^2 to out_ss. in != null:
 *   x is taken from a producer's partials (x must be null): F > 0 for a SwiGLU-packed gate|up
 *   producer (x[f] = silu(r g[f]) * (r u[f]), f < F = K, r from in_ss and in_K, or 1 without
 *   in_ss; no norm_w); F = 0 for a residual (x = resid + the slice sums, S <= 64). act != null:
 *   that x is also stored there. */
typedef struct trx_partial_sums {
  float* out;
  float* out_ss;
  const float* in;
  const float* in_ss;
  const float* resid;
  int S, rows_p, F, in_K;
  float* act;
} trx_partial_sums;
int trx_pack_partials_geometry(int kind, int M, int K, int* S, int* rows_p, int* bps);
int trx_gemv_packed_parts_f32(const uint8_t* packed, int kind, int M, int K, const float* x,
                              const float* norm_w, float eps, float* y, int epilogue,
                              const float* resid, void* workspace, const trx_partial_sums* parts,
                              trx_stream_t s);

/* Decoder ----------------------------------------------------------------------------------------
 * A batch-1 greedy decoder over a BONS model held on the GPU: the GPU counterpart of
 * model/golden.py:FloatModel (reset/forward/generate, golden.py:304-320,436-470) with the
 * arithmetic of model/fastref.py:HybridRef (fastref.py:143-273), and of the firmware loop
 * firmware/infer.c:2001 infer_generate (one position per forward, argmax on the device). */

/* Tensor roles (model/layout.py:95-115). */
#define TRX_ROLE_TOK_EMB 0
#define TRX_ROLE_OUT_NORM 1
#define TRX_ROLE_LM_HEAD 2
#define TRX_ROLE_ATTN_NORM 3
#define TRX_ROLE_ATTN_Q 4
#define TRX_ROLE_ATTN_K 5
#define TRX_ROLE_ATTN_V 6
#define TRX_ROLE_ATTN_OUT 7
#define TRX_ROLE_ATTN_Q_NORM 8
#define TRX_ROLE_ATTN_K_NORM 9
#define TRX_ROLE_FFN_NORM 10
#define TRX_ROLE_FFN_GATE 11
#define TRX_ROLE_FFN_UP 12
#define TRX_ROLE_FFN_DOWN 13
#define TRX_ROLE_ROPE_TAB 14   /* int16 Q14 [max_ctx][rope_dims]: cos half, then sin half */
#define TRX_ROLE_TOK_EMB16 15
#define TRX_ROLE_TOK_EMB16_EXP 16
#define TRX_ROLE_ATTN_QKV 17
#define TRX_ROLE_ATTN_ZGATE 18
#define TRX_ROLE_SSM_OUT 19
#define TRX_ROLE_SSM_BETA 20
#define TRX_ROLE_SSM_ALPHA 21
#define TRX_ROLE_SSM_CONV 22
#define TRX_ROLE_SSM_A 23
#define TRX_ROLE_SSM_DT 24
#define TRX_ROLE_SSM_NORM 25
#define TRX_ROLE_HADAMARD 26   /* model tensor (role, layer = width index): that input width's
                                  PrismML rotation signs, float32 +-1 (trx_model_set_tensor) */

typedef struct {
  int n_layer, n_embd, n_head, n_kv_head, head_dim, ffn_dim, vocab, max_ctx;
  float rms_eps;
  int rope_dims;               /* rotated dims per head, 0 = head_dim */
  int attn_gated;              /* q projection carries [q | gate] per head */
  int dn_num_v_heads, dn_num_k_heads, dn_k_head_dim, dn_v_head_dim, dn_conv_kernel;
  uint64_t layer_types[2];     /* bit l set: layer l is Gated DeltaNet */
  int weight_kind;             /* kind of every layer matrix: TRX_KIND_TERNARY5 or _TERNARY */
  int head_kind;               /* untied LM head: a ternary kind or TRX_KIND_F16 */
  int head_tied;               /* the LM head is the ternary token embedding */
  int emb_mode;                /* 0: int16 BFP lookup table; 1: ternary token_embd rows (the
                                  table's integer rule evaluated on the row); 2: rotated
                                  ternary token_embd rows restored to the plain basis in
                                  integers (model/bons.py:262-295 restored_row_exact; needs the
                                  n_embd width among the rotated widths) */
  int emb_kind;                /* kind of token_embd rows (emb_mode 1 or 2, or a tied head) */
  int max_new;                 /* capacity of the generated-token buffer */
  int packed_ops;              /* projections run by the packed GEMV (trx_gemv_packed_f32) over
                                  a packed copy of their rows, as TRX_PACK_* bits; the others run
                                  trx_gemv_ternary_f32's kernel. TRX_PACK_AUTO: the library's
                                  choice (every projection: q|k|v, o, gate|up, down, the ternary
                                  LM head, the DeltaNet qkv|z and out). */
  /* PrismML's rotated weight basis (model/golden.py:250-289, model/fastref.py:127-140): every
     ternary projection but the DeltaNet beta/alpha takes x' = hadamard_scale * H (s * xhat)
     blockwise over hadamard_block columns (H the +-1 Sylvester matrix, s the width's signs,
     xhat the normalised input), computed by a fast Walsh-Hadamard transform before the GEMV.
     0 = plain basis. A rotated model runs one kernel per operation: its
     projections take the rotated input as a plain vector, on the packed GEMV where packed_ops
     selects it, without the partial-sum handoffs between packed GEMVs. */
  int hadamard_block;          /* 0, or a power of two in [64, 1024] dividing every width */
  float hadamard_scale;        /* the rotation tensors' scale (a power of two) */
  int hadamard_widths[4];      /* the rotated input widths (0 = unused); signs per width as
                                  model tensors TRX_ROLE_HADAMARD, layer = index here */
  int rope_table;              /* 1: RoPE cos/sin per position from the model tensor
                                  TRX_ROLE_ROPE_TAB (the image's int16 Q14 rows [cos | sin] of
                                  rope_dims values, max_ctx rows; model/bons.py:356-367, read as
                                  model/mirror.py:478-483 does), which is how YaRN scaling
                                  reaches the decoder; 0: angles pos * rope_freq[i] */
  int prefill_chunk;           /* trx_model_generate runs the prompt (all but its last token)
                                  through trx_model_prefill in chunks of this many positions;
                                  0: one position per forward, as the firmware's loop */
  int table_free_ops;          /* packed projections (TRX_PACK_* bits, among packed_ops) whose
                                  GEMV looks each code byte's weights up in a 256-entry table and
                                  multiplies them into x held as fp16 high and low planes (v_dot2),
                                  instead of building the per-block table of partial dot products:
                                  the same results to float32 rounding, faster where a block
                                  streams few rows. TRX_PACK_AUTO: the library's choice. */
} trx_model_config;

#define TRX_PACK_QKV 1         /* attention q|k|v */
#define TRX_PACK_O 2           /* attention output */
#define TRX_PACK_GATE_UP 4     /* FFN gate|up with SwiGLU */
#define TRX_PACK_DOWN 8        /* FFN down */
#define TRX_PACK_HEAD 16       /* ternary LM head (with the argmax) */
#define TRX_PACK_DN 32         /* Gated DeltaNet qkv|z and out projections */
#define TRX_PACK_ALL 63
#define TRX_PACK_AUTO (-1)

typedef struct trx_model trx_model;

/* rope_freq: rope_dims/2 float32 frequencies theta^(-2i/rope_dims) (fastref.py:62-63). */
int trx_model_create(const trx_model_config* cfg, const float* rope_freq, trx_model** out);
/* Sampling instead of the greedy argmax (firmware/infer.c:385-488, infer_set_sampling): the
   candidates are the maxima of 32 row ranges of each of n_channels vocabulary shards (the
   image's channel count reproduces the FPGA's candidate set); a repetition penalty
   (logit / repetition above zero, logit * repetition below) on candidates among the last 64
   tokens; then softmax(logit / temperature), the smallest top_p prefix of the sorted mass, one
   xorshift32 draw (seed 0 keeps the stream). temperature 0 with repetition 1 is the greedy
   argmax (no extra launch). */
int trx_model_set_sampling(trx_model* m, float temperature, float top_p, float repetition, uint32_t seed,
                           int n_channels);
int trx_model_destroy(trx_model* m);
/* Upload one tensor (synchronous). Ternary and Q8: BONS row packets of the model's kind; F32:
 * float32 values; F16 head: fp16 values; TOK_EMB16: int16 [vocab, n_embd]; TOK_EMB16_EXP: int32
 * [vocab]. The fused groups (q|k|v, gate|up, qkv|z, beta|alpha) are laid out adjacent. */
int trx_model_set_tensor(trx_model* m, int role, int layer, const void* data, size_t bytes);
/* Fill every tensor from the counter-based generator (trixium_amd/synth.py's hash) but the Q8
 * rows (a hybrid's DeltaNet beta|alpha), which the caller sets with trx_model_set_tensor. ranges:
 * float32 {scale_lo, scale_span, gain_lo, gain_span}. */
int trx_model_synthesize(trx_model* m, uint32_t seed, const float* ranges);
/* Clear the position, the argmax slot and the DeltaNet state (golden.py:304-320). */
int trx_model_reset(trx_model* m);
/* Checkpoint of the decode state, so that forwards can be run again from it: the firmware's
 * forward_checked (firmware/infer.c:1926-1960), which re-runs a forward from the state that
 * hybrid_ckpt_save kept (firmware/hybrid.c:2904-2930). TRX_CKPT_SAVE copies the state after the
 * work enqueued so far (position, fed and generated tokens, argmax slot, sampler stream, every
 * DeltaNet layer's conv window and recurrent matrix) into a buffer of the model (allocated on the
 * first save: the DeltaNet state's size, 151 MB at the 27B hybrid's shape); TRX_CKPT_RESTORE
 * enqueues the copy back, and the next forwards give the results they gave after the save. The KV
 * rows are not copied: a forward writes its own position's row, so rows past the restored
 * position are rewritten before they are read. Outputs of the last forward (logits, taps) are not
 * state and are not restored. Asynchronous on the model's stream; TRX_E_STATE restores with no
 * checkpoint saved. With the KV ring past the window (trx_model_set_kv_ring) a forward there
 * overwrites the ring slot of the position that leaves the window, so a restore there undoes at
 * most one forward, as the firmware's retry does (TRX_E_STATE after more). */
#define TRX_CKPT_SAVE 0
#define TRX_CKPT_RESTORE 1
int trx_model_checkpoint(trx_model* m, int op);
/* KV ring past the window (firmware/hybrid.c:156-181, the console's `kvring` and hybrid_set_pin):
 * with the ring on, forwards go on past max_ctx. Position p < max_ctx keeps KV slot p; past it the
 * first `pin` positions stay (at least 4 sinks, at most max_ctx / 4) and position p takes slot
 * pin + (p - pin) % (max_ctx - pin), so the attention reads every slot: the pinned positions and
 * the most recent max_ctx - pin, K rotated at their own positions. enable: 1 on, 0 off, -1 the
 * default (on for a model with DeltaNet layers, as the firmware's hybrid; off otherwise, which
 * stops at max_ctx as the firmware's Qwen3 loop does). Both take effect at the next reset, and the
 * pin lasts one reset (then 4 again); the ring stays off where max_ctx <= 2 pin. A model whose
 * image carries a RoPE table (no rows past max_ctx) cannot turn it on: TRX_E_INVALID. Positions
 * past the window run one position per forward (trx_model_prefill steps them). */
int trx_model_set_kv_ring(trx_model* m, int enable, int pin);
/* Feed tokens at the next n positions (after the forwards already enqueued); logits are computed
 * from absolute position head_from on (-1: the last fed token). */
int trx_model_set_prompt(trx_model* m, const int32_t* tokens, int n, int head_from);
/* Enqueue n forwards of one position each (eagerly, or as replays of one captured hipGraph). */
int trx_model_step(trx_model* m, int n_steps, int use_graph);
/* Batched prefill (model/bitexact.py:121-125 matvec_ternary_rows; firmware/infer.c:1956-1977
 * forward_pair, which runs two prompt tokens per weight pass): the next n fed positions in
 * chunks of up to `chunk` positions (<= 0: 1024), one weight pass per chunk. Every projection is
 * a GEMM over the chunk on the matrix cores, attention is causal over the cache, the DeltaNet
 * recurrence runs over the chunk's positions in order. The positions must precede head_from (no
 * logits); afterwards the KV cache, the DeltaNet state and the position are those of n
 * one-position forwards, and the next trx_model_step continues from there. */
int trx_model_prefill(trx_model* m, int n, int chunk);
/* Resolve the argmax of the last forward into the output buffer. */
int trx_model_finalize(trx_model* m);
int trx_model_sync(trx_model* m);
/* Greedy decode: n_prompt + n_new - 1 forwards, then the generated ids (FloatModel.generate,
 * golden.py:462-470, with the firmware's no-final-forward contract, mirror.py:1040-1043). */
int trx_model_generate(trx_model* m, const int32_t* prompt, int n_prompt, int n_new, int32_t* out,
                       int use_graph);
#define TRX_READ_LOGITS 0      /* float32 [vocab] of the last forward that ran the head */
#define TRX_READ_HIDDEN 1      /* float32 [n_embd]: the final normed hidden state of the last
                                  forward, rmsnorm(residual, output norm) (fastref.py:244-258) */
#define TRX_READ_POSITION 2    /* int32 */
#define TRX_READ_TOKEN 3       /* int32: the token of the last forward */
#define TRX_READ_OUT 4         /* int32 [max_new]: generated tokens */
#define TRX_READ_SLOT 5        /* uint64: packed argmax */
#define TRX_READ_QKV 6         /* float32: q|k|v projection of the last attention layer run */
#define TRX_READ_ATTN 7        /* float32 [n_head*head_dim]: its attention output */
#define TRX_READ_ACT 8         /* float32 [ffn_dim]: the last layer's SwiGLU activation */
#define TRX_READ_RESIDUAL 9    /* float32 [n_embd]: the residual stream after the last layer */
int trx_model_read(trx_model* m, int what, void* host, size_t bytes);
/* Teacher-forced scoring of a sequence from position 0 (model/fastref.py:263-273 score; resets
 * the model): nll[i] = logsumexp(logits_i) - logits_i[tokens[i + 1]] for i < n - 1 (host float32,
 * may be NULL), and the final normed hidden states hidden[n][n_embd] (host, may be NULL,
 * fastref.py:244-258 hidden). Synchronous; every position runs the LM head. */
int trx_model_score(trx_model* m, const int32_t* tokens, int n, float* nll, float* hidden);
/* The LM head applied to n given hidden states (host float32 [n][n_embd] -> [n][vocab]):
 * model/fastref.py:260-261 logits (the rotation of a rotated model included, no norm).
 * Synchronous. */
int trx_model_project_head(trx_model* m, const float* hidden, int n, float* logits);
#define TRX_INFO_ARENA_BYTES 0
#define TRX_INFO_DEVICE_BYTES 1
#define TRX_INFO_STREAM 2
#define TRX_INFO_WEIGHT_BYTES 3
#define TRX_INFO_PACKED_OPS 5     /* TRX_PACK_* bits in effect */
#define TRX_INFO_ATTN_SPLITS 6    /* decode attention: blocks (position splits) per kv head */
#define TRX_INFO_ATTN_PASS 7      /* decode attention: positions one pass of a split block covers
                                     (a split of c positions takes ceil(c / this) passes) */
#define TRX_INFO_TABLE_FREE_OPS 8 /* TRX_PACK_* bits on the table-free lookups */
#define TRX_INFO_KV_PIN 9         /* positions the KV ring keeps past the window since the last
                                     reset (0: no ring, forwards stop at max_ctx) */
int trx_model_info(trx_model* m, int what, int64_t* value);
/* Device address and size of one resident tensor (for benchmarks and tests). */
int trx_model_tensor_ptr(trx_model* m, int role, int layer, void** ptr, int64_t* bytes);
/* Packed copy of one projection (op: TRX_PACK_QKV, _O, _GATE_UP, _DOWN or _HEAD with layer 0) and
 * the workspace the model's packed GEMVs share, for trx_gemv_packed_f32 (benchmarks and tests;
 * do not overlap with the model's own work). */
int trx_model_packed_ptr(trx_model* m, int op, int layer, void** packed, void** workspace);

/* Measurement (no counterpart in the reference; for benchmarks and tests) -------------------------
 * trx_graph_begin / trx_graph_end: capture the work a caller enqueues on stream s (a created
 *   stream) into a hipGraph and instantiate it (*exec); trx_graph_launch replays it on a stream;
 *   trx_graph_destroy frees it. Library calls made between begin and end are captured, not run.
 * trx_probe_stream_read: a plain streaming read of `bytes` (a multiple of 16) of device memory by
 *   `blocks` blocks of `threads` threads (16-byte non-temporal loads, grid-stride), one float per
 *   block to out: the read rate any HBM-bound kernel here can reach.
 * trx_probe_empty: an empty kernel (one block of 64 threads): the fixed cost of a launch or of a
 *   dependent graph node. */
int trx_graph_begin(trx_stream_t s);
int trx_graph_end(trx_stream_t s, void** exec);
int trx_graph_launch(void* exec, trx_stream_t s);
int trx_graph_destroy(void* exec);
int trx_probe_stream_read(const void* buf, size_t bytes, float* out, int blocks, int threads, trx_stream_t s);
int trx_probe_empty(trx_stream_t s);

/* Tuning: force the GEMV rows per item (0 = automatic; 1: 4 rows, 2: 2 rows, 3: 1 row, 2 for
 * SwiGLU). Process-wide; for benchmarks and tests. No counterpart in the reference. */
int trx_gemv_set_variant(int variant);

#ifdef __cplusplus
}
#endif
#endif /* TRIXIUM_H */
