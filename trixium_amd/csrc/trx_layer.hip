// Fused decoder layer: one kernel runs a whole full-attention layer for one position,
//   A  q|k|v GEMV (attention RMSNorm fused)            -> qkv
//   B  attention splits (K/V rows fetched before the barrier)   -> split partials, KV append
//   C  merge of the partials (+ output gate)           -> attention output
//   D  o GEMV + residual                               -> x
//   E  gate|up GEMV (FFN RMSNorm, SwiGLU)              -> act
//   F  down GEMV + residual                            -> x
// with a grid barrier between consecutive phases (the layer's arithmetic is that of the
// per-operation kernels: model/fastref.py:216-261 for one position). One block per CU, all
// resident; before every barrier each block fetches the next phase's weight rows (or K/V rows)
// into registers, so the stream of weights overlaps the barrier and the exchange of the small
// activation vectors, which go through agent-scope (cross-XCD coherent) accesses.
//
// Barrier: hierarchical over the XCDs. A block counts itself in its XCD's counter; the XCD's
// last block counts the XCD in the global counter; every block waits for the global count.
// Counters are 64-bit and never reset during a sequence: the n-th barrier of a launch for
// position `pos` waits for epoch (pos * layers + layer) * 5 + n, so graph replays need no
// resetting. A wait that exceeds 20 ms sets an error flag and gives up rather than hang.

#include <algorithm>

#include "trx_layer.h"
#include "trx_attn_dev.h"

namespace trx {

constexpr int kLayerBarriers = 5;
constexpr int kBarStride = 32;                 // 256-byte lines between counters
constexpr unsigned long long kSpinTicks = 2000000ull;   // 20 ms of the 100 MHz realtime clock

__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xFu;
}

struct GridBarrier {
  unsigned long long* bar;          // [16 XCD counters][global], kBarStride apart
  const unsigned* xcc_blocks;       // blocks of this grid on every XCD
  unsigned long long epoch;
  unsigned n_xcc;
  int* err;
  __device__ void operator()() const {
    // This phase's outputs went out as agent-scope stores: wait until they have completed
    // before counting the block in.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned x = xcc_id();
      const unsigned long long nx = xcc_blocks[x];
      const unsigned long long old =
          __hip_atomic_fetch_add(bar + x * kBarStride, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old + 1 == epoch * nx)
        __hip_atomic_fetch_add(bar + 16 * kBarStride, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned long long target = epoch * n_xcc;
      const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
      unsigned spins = 0;
      while (__hip_atomic_load(bar + 16 * kBarStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        // Give up after 20 ms, or at once when another barrier already has (no further wait of
        // this sequence can succeed).
        if ((++spins & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
        if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
          atomicOr(err, 1);
          break;
        }
      }
    }
    __syncthreads();
  }
};

template <int FMT, int REP, int HD>
__global__ __launch_bounds__(kGemvThreads) void layer_kernel(LayerParams lp) {
  __shared__ __align__(16) uint64_t lut64[kLutBytes / 8];
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* lut = (uint8_t*)lut64;
  const int bid = blockIdx.x, nblk = gridDim.x;
  const unsigned long long launch = (unsigned long long)(*lp.pos) * lp.n_layers + lp.layer_slot;
  auto barrier = [&](int k) {
    return GridBarrier{lp.bar, lp.xcc_blocks, launch * kLayerBarriers + (unsigned long long)k, lp.n_xcc, lp.err};
  };
  fill_lut<FMT == TRX_KIND_TERNARY5>(lut);      // visible after the first phase's staging sync
  // A: q|k|v (x comes from the previous kernel).
  gemv_body<FMT, MODE_F32, 2, 4, false, true>(lp.qkv, lut, smem, bid, nblk, NoWait{});
  // B: attention splits; their K/V rows are fetched before the barrier.
  attn_split_body<REP, HD, true>(lp.attn, bid, barrier(1));
  // C: merge, one block per q head.
  barrier(2)();
  if (bid < lp.attn.n_head) attn_merge_body<true>(lp.attn, bid);
  // D: o projection + residual, E: gate|up + SwiGLU, F: down + residual.
  gemv_body<FMT, MODE_F32, 1, 6, false, true>(lp.o, lut, smem, bid, nblk, barrier(3));
  gemv_body<FMT, MODE_F32, 2, 4, true, true>(lp.gu, lut, smem, bid, nblk, barrier(4));
  gemv_body<FMT, MODE_F32, 1, 6, false, true>(lp.down, lut, smem, bid, nblk, barrier(5));
}

__global__ void count_xcc_kernel(unsigned* xcc_blocks) {
  if (threadIdx.x == 0) atomicAdd(&xcc_blocks[xcc_id()], 1u);
}

// Instantiated layer geometries: (q heads per kv head, head dim).
template <int FMT>
static const void* layer_fn(int rep, int hd) {
  if (rep == 2 && hd == 64) return (const void*)layer_kernel<FMT, 2, 64>;
  if (rep == 4 && hd == 64) return (const void*)layer_kernel<FMT, 4, 64>;
  if (rep == 2 && hd == 128) return (const void*)layer_kernel<FMT, 2, 128>;
  if (rep == 4 && hd == 128) return (const void*)layer_kernel<FMT, 4, 128>;
  return nullptr;
}

static const void* layer_kernel_fn(int kind, int rep, int hd) {
  if (kind == TRX_KIND_TERNARY5) return layer_fn<TRX_KIND_TERNARY5>(rep, hd);
  if (kind == TRX_KIND_TERNARY) return layer_fn<TRX_KIND_TERNARY>(rep, hd);
  return nullptr;
}

int layer_lds_bytes(int E, int qdim, int F) {
  int b = 0;
  for (int K : {E, qdim, F}) b = std::max(b, lds_bytes(K, K / kGroup));
  return b;
}

int layer_prepare(LayerSetup& ls, int kind, int rep, int hd, int E, int qdim, int F, unsigned* xcc_blocks_dev) {
  ls.ok = false;
  const void* fn = layer_kernel_fn(kind, rep, hd);
  if (!fn) return TRX_OK;                      // geometry not instantiated: per-operation kernels
  int dev = 0;
  hipDeviceProp_t prop;
  TRX_HIP(hipGetDevice(&dev));
  TRX_HIP(hipGetDeviceProperties(&prop, dev));
  const int lds = layer_lds_bytes(E, qdim, F);
  TRX_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kGemvThreads, lds) != hipSuccess || per_cu < 1) {
    (void)hipGetLastError();
    return TRX_OK;                             // does not fit one CU: per-operation kernels
  }
  // Every block must be resident at once: one block per CU, exactly one per CU.
  ls.blocks = prop.multiProcessorCount;
  ls.lds = lds;
  ls.fn = fn;
  // Blocks of this grid per XCD (the hardware deals workgroups over the XCDs).
  TRX_HIP(hipMemset(xcc_blocks_dev, 0, 16 * sizeof(unsigned)));
  hipLaunchKernelGGL(count_xcc_kernel, dim3(ls.blocks), dim3(kGemvThreads), 0, 0, xcc_blocks_dev);
  TRX_LAUNCHED();
  TRX_HIP(hipDeviceSynchronize());
  unsigned h[16];
  TRX_HIP(hipMemcpy(h, xcc_blocks_dev, sizeof h, hipMemcpyDeviceToHost));
  ls.n_xcc = 0;
  for (int i = 0; i < 16; ++i) ls.n_xcc += h[i] ? 1 : 0;
  ls.ok = ls.n_xcc > 0;
  return TRX_OK;
}

int launch_layer(const LayerSetup& ls, const LayerParams& lp, hipStream_t s) {
  TRX_CHECK(ls.ok && ls.fn, TRX_E_STATE, "fused layer kernel not prepared");
  void* args[] = {(void*)&lp};
  TRX_HIP(hipLaunchKernel(ls.fn, dim3(ls.blocks), dim3(kGemvThreads), args, ls.lds, s));
  return TRX_OK;
}

// GemvParams of one fused phase (rows per item fixed by the phase: see layer_kernel).
int layer_gemv_params(GemvParams& p, const uint8_t* rows, int kind, int M, int K, const float* x,
                      const float* norm_w, float eps, float* y, int epi, const float* resid, int rows_per_item) {
  int rc = gemv_check(kind, M, K);
  if (rc) return rc;
  p = GemvParams{};
  fill_geom_public(p, rows, kind, M, K);
  p.x = x;
  p.norm_w = norm_w;
  p.eps = eps;
  p.y = y;
  p.epi = epi;
  p.resid = resid;
  if (epi == TRX_EPI_SWIGLU) {
    p.swiglu_F = M / 2;
    p.n_out = M / 2;
    p.n_batches = cdiv(p.n_out, rows_per_item / 2);
  } else {
    p.n_out = M;
    p.n_batches = cdiv(p.n_out, rows_per_item);
  }
  return TRX_OK;
}

}  // namespace trx
