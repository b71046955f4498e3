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

#ifdef __cplusplus
}
#endif
#endif /* TRIXIUM_H */
