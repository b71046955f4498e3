// Decode-loop kernels other than the ternary GEMV: token embedding, split-K GQA decode attention
// over an fp16 KV cache (QK-RMSNorm, RoPE and the KV append fused in), the split combine, a
// dense fp16 / Q8 GEMV (small heads and the DeltaNet beta/alpha projections), the greedy
// token resolve, and the on-device synthetic weight generator.

#include "trx_internal.h"
#include "trx_ops.h"
#include "trx_dense_dev.h"
#include "trx_attn_dev.h"

namespace trx {

// Token control ---------------------------------------------------------------------------------
//
// Per step: pos += 1; the token is prompt[pos] while pos < n_prompt, otherwise the argmax of
// the previous step (packed (ordered logit, ~row) in *slot, ties to the smallest row), which is
// also recorded as generated token pos - n_prompt. The slot is cleared for this step's head.

__device__ __forceinline__ int slot_token(unsigned long long key) {
  return (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}

__device__ __forceinline__ float bfp_scale(int e) { return ldexpf(1.0f, e); }

// Embedding of one token into x (fp32 [n_embd]).
//   table mode: x = mant[tok] * 2^exp[tok]                                (model/fastref.py:158-172)
//   ternary mode: the integer BFP rule of the int16 table, evaluated on the row (model/bons.py:
//   204-236): every group's (code-1)*m11 aligned to the row's smallest exponent (capped at 20),
//   the live absmax normalised into [2^14, 2^15), truncated to int16.
constexpr int kMaxEmbedGroups = 128;
constexpr int kEmbedRowMax = 32 * (kMaxEmbedGroups / 16 + kMaxEmbedGroups);   // 2-bit row bytes
constexpr int kEmbedVecs = kEmbedRowMax / 16;
constexpr int kEmbedThreads = 1024;       // 16 waves: the row's columns over a whole CU

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

// Restore mode (model/bons.py:262-295 restored_row_exact, the firmware's embed_row_restore):
// the rotated ternary row in integers, v = (code - 1) * m11 << (e16 - e16min); the natural-order
// Walsh-Hadamard butterflies per block of hblock columns (int64 in LDS); y = sign * v; the absmax
// normalised into [2^14, 2^15) with a round-half-even right shift; exponent e16min - floor(log2
// hblock / 2) + shift.
constexpr int kRestoreMax = 8192;

__device__ __forceinline__ long long rne_shift_ll(long long mag, int r) {
  const long long q = mag >> r, rem = mag & ((1ll << r) - 1), half = 1ll << (r - 1);
  return q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
}

// The embedding of token `tok` into x (n_embd floats); a whole block of kEmbedThreads.
__device__ void embed_token(const EmbedParams& p, int tok, float* x) {
  __shared__ int s_red[kEmbedThreads / 64];
  __shared__ __align__(16) uint8_t s_row[kEmbedRowMax];
  const int tid = threadIdx.x;
  if (p.mode == EMBED_TABLE) {
    // Every load of a chunk is issued before its stores (x could alias the table as far as the
    // compiler knows, so a plain loop would wait out each load in turn).
    constexpr int U = 4;
    const float sc = bfp_scale(p.exps[tok]);
    const int16_t* m = p.mant + (size_t)tok * p.n_embd;
    for (int c0 = 0; c0 < p.n_embd; c0 += U * kEmbedThreads) {
      int16_t v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * kEmbedThreads + tid;
        v[u] = c < p.n_embd ? m[c] : (int16_t)0;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * kEmbedThreads + tid;
        if (c < p.n_embd) x[c] = (float)v[u] * sc;
      }
    }
    return;
  }
  // Ternary row: scales at the head of the row packet, codes after code_off. The whole packet
  // comes into LDS with one 16-byte load per thread; every later read is from LDS.
  __shared__ int s_live[kMaxEmbedGroups];
  __shared__ long long s_lred[kEmbedThreads / 64];
  {
    const uint4* src = (const uint4*)(p.rows + (size_t)tok * p.row_bytes);
    const int nvec = p.row_bytes / 16;
#pragma unroll
    for (int k = 0; k < (kEmbedVecs + kEmbedThreads - 1) / kEmbedThreads; ++k) {
      const int i = min(tid + kEmbedThreads * k, nvec - 1);
      ((uint4*)s_row)[i] = src[i];
    }
  }
  __syncthreads();
  const uint8_t* row = s_row;
  const uint16_t* sc = (const uint16_t*)row;
  const int G = p.n_embd / kGroup;
  auto code_of = [&](int c) -> int {
    if (p.kind == TRX_KIND_TERNARY5) {
      const int g = c >> 7, j = c & 127, byte = j / 5, k = j - 5 * byte;
      const int b = row[p.code_off + kTrit5GroupBytes * g + byte];
      const int d = k == 0 ? b : k == 1 ? b / 3 : k == 2 ? b / 9 : k == 3 ? b / 27 : b / 81;
      return d % 3;
    }
    return (row[p.code_off + (c >> 2)] >> (2 * (c & 3))) & 3;
  };
  // Smallest scale exponent of the row, and which groups hold a nonzero weight.
  int emin = 1 << 20;
  for (int g = tid; g < G; g += kEmbedThreads) {
    int m11, e16;
    fp16_split(sc[g], m11, e16);
    emin = min(emin, e16);
    s_live[g] = 0;
  }
  emin = wave_min_i(emin);
  if ((tid & 63) == 0) s_red[tid >> 6] = emin;
  __syncthreads();
  emin = s_red[0];
  for (int i = 1; i < kEmbedThreads / 64; ++i) emin = min(emin, s_red[i]);
  for (int c = tid; c < p.n_embd; c += kEmbedThreads)
    if (code_of(c) != 1) s_live[c >> 7] = 1;
  __syncthreads();
  // Largest aligned |m11| over the live groups.
  long long amax = 0;
  for (int g = tid; g < G; g += kEmbedThreads) {
    if (!s_live[g]) continue;
    int m11, e16;
    fp16_split(sc[g], m11, e16);
    const long long v = (long long)(m11 < 0 ? -m11 : m11) << min(e16 - emin, 20);
    amax = v > amax ? v : amax;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const long long other = __shfl_xor(amax, o, 64);
    amax = other > amax ? other : amax;
  }
  if ((tid & 63) == 0) s_lred[tid >> 6] = amax;
  __syncthreads();
  amax = s_lred[0];
  for (int i = 1; i < kEmbedThreads / 64; ++i) amax = s_lred[i] > amax ? s_lred[i] : amax;
  if (p.mode == EMBED_RESTORE) {
    __shared__ long long s_v[kRestoreMax];
    for (int c = tid; c < p.n_embd; c += kEmbedThreads) {
      int m11, e16;
      fp16_split(sc[c >> 7], m11, e16);
      s_v[c] = (long long)(code_of(c) - 1) * (long long)m11 * (1ll << (e16 - emin));
    }
    for (int h = 1; h < p.hblock; h <<= 1) {
      __syncthreads();
      for (int i2 = tid; i2 < p.n_embd / 2; i2 += kEmbedThreads) {
        const int i = (i2 / h) * 2 * h + (i2 % h);
        const long long a = s_v[i], b = s_v[i + h];
        s_v[i] = a + b;
        s_v[i + h] = a - b;
      }
    }
    __syncthreads();
    long long ym = 0;
    for (int c = tid; c < p.n_embd; c += kEmbedThreads) {
      const long long y = p.signs[c] < 0.f ? -s_v[c] : s_v[c];
      s_v[c] = y;
      const long long a = y < 0 ? -y : y;
      ym = a > ym ? a : ym;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const long long other = __shfl_xor(ym, o, 64);
      ym = other > ym ? other : ym;
    }
    __syncthreads();
    if ((tid & 63) == 0) s_lred[tid >> 6] = ym;
    __syncthreads();
    ym = s_lred[0];
    for (int i = 1; i < kEmbedThreads / 64; ++i) ym = s_lred[i] > ym ? s_lred[i] : ym;
    int lg = 0;
    while ((1 << (lg + 1)) <= p.hblock) ++lg;
    const int bits = ym ? 64 - __clzll(ym) : 0;
    const int r = bits - 15;
    const float sc2 = ym ? bfp_scale(emin - lg / 2 + r) : 0.f;
    for (int c = tid; c < p.n_embd; c += kEmbedThreads) {
      const long long y = s_v[c], a = y < 0 ? -y : y;
      long long mag = r > 0 ? rne_shift_ll(a, r) : (a << (-r));
      mag = mag > 32767 ? 32767 : mag;
      x[c] = (float)(y < 0 ? -mag : mag) * sc2;
    }
    return;
  }
  int bl = 0;
  while (bl < 63 && (amax >> bl) != 0) ++bl;
  const int k2 = bl - 15;
  const float scale = bfp_scale(emin + k2);
  for (int c = tid; c < p.n_embd; c += kEmbedThreads) {
    int m11, e16;
    fp16_split(sc[c >> 7], m11, e16);
    const int sh = min(e16 - emin, 20) - k2;
    const long long v = (long long)(code_of(c) - 1) * m11;
    const long long w = sh >= 0 ? (v << sh) : (v >> (-sh));
    x[c] = (float)(int16_t)(w & 0xFFFF) * scale;
  }
}

__global__ __launch_bounds__(kEmbedThreads) void embed_kernel(EmbedParams p) {
  __shared__ int s_tok, s_pos;
  const int tid = threadIdx.x;
  if (tid == 0) {
    // The control words are read together (one round trip), before the position is written.
    const int pos0 = *p.pos, np = *p.n_prompt, pin = p.pos[7];
    const unsigned long long key = *p.slot;
    const int pos = pos0 + 1;
    *p.pos = pos;
    // The position's KV slot and the slots the attention reads (firmware/hybrid.c:170-181,2483):
    // inside the window the position itself and pos + 1 slots; past it, with the ring on (pin > 0),
    // the first pin positions stay and the others share the rest of the window as a ring, all
    // max_ctx slots attended.
    int slot = pos, nslots = pos + 1;
    if (pos >= p.max_ctx && pin > 0) {
      slot = pin + (pos - pin) % (p.max_ctx - pin);
      nslots = p.max_ctx;
    }
    p.pos[5] = slot;
    p.pos[6] = nslots;
    s_pos = pos;
    int tok;
    if (pos < np) {
      tok = p.prompt[pos % p.prompt_ring];
    } else {
      tok = slot_token(key);
      const int k = pos - np;
      if (k < p.max_out) p.out[k] = tok;
    }
    if (tok < 0 || tok >= p.vocab) tok = 0;
    *p.slot = 0ull;
    *p.cur_tok = tok;
    s_tok = tok;
  }
  __syncthreads();
  // Past the window the RoPE table has no row for the position: row max_ctx gets its cos and sin
  // of the float32 angle pos * f_i, evaluated in double and rounded once (as the table's rows).
  const int pos = s_pos, half = p.rope_n / 2;
  if (pos >= p.max_ctx && p.rope_cs && tid < half) {
    const double ang = (double)((float)pos * p.rope_freq[tid]);
    float* row = p.rope_cs + (size_t)p.max_ctx * p.rope_n;
    row[tid] = (float)cos(ang);
    row[half + tid] = (float)sin(ang);
  }
  embed_token(p, s_tok, p.x);
}

// Prefill: the tokens fed at positions p0 .. p0 + gridDim.x - 1 into rows of X.
__global__ __launch_bounds__(kEmbedThreads) void embed_rows_kernel(EmbedParams p, const int* fed, int p0, float* X) {
  int tok = fed[p0 + blockIdx.x];
  if (tok < 0 || tok >= p.vocab) tok = 0;
  embed_token(p, tok, X + (size_t)blockIdx.x * p.n_embd);
}

// Resolve the last generated token (after the final step): out[pos + 1 - n_prompt].
__global__ void finalize_kernel(const int* pos, const int* n_prompt, unsigned long long* slot, int* out,
                                int max_out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int k = *pos + 1 - *n_prompt;
    if (k >= 0 && k < max_out) out[k] = slot_token(*slot);
  }
}

// Dense GEMV over fp16 or Q8 row packets: y[m] = sum_k w[m,k] x[k] (optional RMSNorm of x),
// optional argmax slot. One wave per row; x staged in LDS as fp32.
__global__ __launch_bounds__(256) void dense_gemv_kernel(DenseParams p) {
  extern __shared__ float xs[];
  __shared__ float red[8];
  if (p.gate_pos && *p.gate_pos < *p.gate_from) return;
  const int tid = threadIdx.x;
  float rinv = 1.0f;
  if (p.norm_w) {
    float ss = 0.f;
    for (int c = tid; c < p.K; c += 256) ss += p.x[c] * p.x[c];
    ss = block_sum(ss, red);
    rinv = 1.0f / sqrtf(ss / (float)p.K + p.eps);
  }
  for (int c = tid; c < p.K; c += 256) xs[c] = p.norm_w ? p.x[c] * rinv * p.norm_w[c] : p.x[c];
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  unsigned long long best = 0;   // lane 0: best (ordered value, ~row) key of this wave's rows
  for (int m = blockIdx.x * 4 + wave; m < p.M; m += gridDim.x * 4) {
    const uint8_t* row = p.W + (size_t)m * p.row_bytes;
    float acc = 0.f;
    if (p.kind == TRX_KIND_F16) {
      const __half* w = (const __half*)row;
      for (int c = lane * 2; c < p.K; c += 128) {
        const __half2 v = *(const __half2*)(w + c);
        acc += __half2float(v.x) * xs[c] + __half2float(v.y) * xs[c + 1];
      }
    } else {  // Q8: fp16 scales per 32, then int8 codes
      // The weight q*s is rounded to fp16 as the float reference caches every dequantised
      // matrix in fp16 (model/fastref.py:46,104-116); q*s itself is exact in fp32.
      const uint16_t* sc = (const uint16_t*)row;
      const int8_t* q = (const int8_t*)(row + p.code_off);
      for (int c = lane; c < p.K; c += 64) {
        const float s = __half2float(__ushort_as_half(sc[c >> 5]));
        acc += __half2float(__float2half((float)q[c] * s)) * xs[c];
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      float v = acc;
      if (p.sigmoid) v = sigmoidf_(v);
      p.y[m] = v;
      if (p.amax_slot) {
        uint32_t u = __float_as_uint(v);
        u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        const unsigned long long key = ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)m);
        best = key > best ? key : best;
      }
    }
  }
  if (p.amax_slot && lane == 0 && best) atomicMax(p.amax_slot, best);
}

// Q8 GEMV for a few rows (the DeltaNet beta|alpha head projections): one block per row, thread t
// takes the 32-column groups t, t + 256, ... whole (two 16-byte code loads, its scale, x and the
// gain from global memory), every load issued before the products. With a norm the row's sum is
// scaled by 1/rms(x) at the end: x^2 and the products reduce together. The weight q*s is rounded
// to fp16 as the float reference caches every dequantised matrix in fp16.
__global__ __launch_bounds__(256) void q8_gemv_kernel(DenseParams p) {
  __shared__ float red[2][4];
  if (p.gate_pos && *p.gate_pos < *p.gate_from) return;
  q8_row_dot(p, blockIdx.x, threadIdx.x, red);
}

// Synthetic weights (csrc side of trixium_amd/synth.py's counter-based generator) ---------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t synth_key(uint32_t seed, uint32_t tid, uint32_t stream) {
  return splitmix64(((uint64_t)seed << 32) | ((uint64_t)(tid & 0xFFFFFF) << 8) | stream);
}

__device__ __forceinline__ float synth_uniform(uint64_t key, uint64_t idx, float lo, float span) {
  // lo + span*u with two roundings (the host generator's numpy float32 arithmetic): no FMA.
#pragma clang fp contract(off)
  const uint64_t h = splitmix64(idx ^ key);
  const float u = (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
  const float su = span * u;
  return lo + su;
}

// One thread per (row, 4-column quad) writes the codes; threads with quad < G also write the
// row's fp16 scale of group `quad`.
__global__ void synth_ternary_kernel(SynthParams p) {
  const long long nq = (long long)p.cols / 4;
  const long long total = (long long)p.rows * nq;
  const uint64_t kc = synth_key(p.seed, p.tensor_id, 1), ks = synth_key(p.seed, p.tensor_id, 2);
  const int G = p.cols / kGroup;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / nq;
    const int q = (int)(i - r * nq);
    uint8_t* row = p.out + (size_t)r * p.row_bytes;
    const uint64_t h = splitmix64((uint64_t)i ^ kc);
    int c[4];
    for (int k = 0; k < 4; ++k) {
      const uint32_t u = (uint32_t)(h >> (16 * k)) & 0xFFFFu;
      c[k] = u < 19661u ? 0 : (u < 45875u ? 1 : 2);
    }
    if (p.kind == TRX_KIND_TERNARY) {
      row[p.code_off + q] = (uint8_t)(c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6));
    } else {
      // trit5: columns 4q..4q+3 go to (byte, digit) positions; bytes are assembled by the
      // thread owning the byte's first column (column 5*byte) from the hashes of its quads.
      for (int k = 0; k < 4; ++k) {
        const int col = 4 * q + k, g = col >> 7, j = col & 127;
        if (j % 5) continue;
        const int byte = j / 5;
        int v = 0, p3 = 1;
        for (int d = 0; d < 5; ++d) {
          const int jj = j + d;
          int cd = 0;
          if (jj < 128) {
            const long long cc = (long long)g * 128 + jj;
            const uint64_t hh = splitmix64((uint64_t)(r * nq + cc / 4) ^ kc);
            const uint32_t u = (uint32_t)(hh >> (16 * (cc & 3))) & 0xFFFFu;
            cd = u < 19661u ? 0 : (u < 45875u ? 1 : 2);
          }
          v += cd * p3;
          p3 *= 3;
        }
        row[p.code_off + kTrit5GroupBytes * g + byte] = (uint8_t)v;
      }
    }
    if (q < G) {
      const float s = synth_uniform(ks, (uint64_t)(r * G + q), p.lo, p.span);
      ((__half*)row)[q] = __float2half(s);
    }
  }
}

__global__ void synth_f32_kernel(float* out, long long n, uint32_t seed, uint32_t tensor_id,
                                 float lo, float span, int transform) {
  const uint64_t k = synth_key(seed, tensor_id, 3);
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x) {
    float v = synth_uniform(k, (uint64_t)i, lo, span);
    if (transform == 1) v = -expf(v);
    out[i] = v;
  }
}

// Sampling ----------------------------------------------------------------------------------------

constexpr int kSmpSlices = 32, kSmpWindowMax = 960;

// One block per slice: its maximum over every channel's rows of the slice (first maximum in
// channel-major order, i.e. the smallest token) into cand; the block that finishes last (an
// agent-scope counter) picks among the 32.
__global__ __launch_bounds__(1024) void sample_kernel(SampleParams p) {
  __shared__ float cval[kSmpSlices], wv[16];
  __shared__ int ctok[kSmpSlices], wi[16];
  __shared__ int win[kSmpWindowMax];
  __shared__ float lg[kSmpSlices], pr[kSmpSlices];
  __shared__ int tk[kSmpSlices], ord[kSmpSlices], seen[kSmpSlices], n_s;
  __shared__ bool last;
  const int pos = *p.pos;
  if (pos < *p.head_from) return;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, k = blockIdx.x;
  const int rpc = (p.vocab + p.n_ch - 1) / p.n_ch, srows = (rpc + kSmpSlices - 1) / kSmpSlices;
  const int r0 = k * srows, rows = max(0, min(srows, rpc - r0));
  float best = -INFINITY;
  int btok = 0x7FFFFFFF;
  for (int c = 0; c < p.n_ch; ++c) {
    const int base = c * rpc + r0;
    for (int i0 = 0; i0 < rows; i0 += 4 * 1024) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * 1024 + t, tok = base + i;
        v[u] = i < rows && tok < p.vocab ? p.logits[tok] : -INFINITY;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int tok = base + i0 + u * 1024 + t;
        if (v[u] > best || (v[u] == best && v[u] > -INFINITY && tok < btok)) best = v[u], btok = tok;
      }
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int ot = __shfl_xor(btok, o, 64);
    if (ob > best || (ob == best && ot < btok)) best = ob, btok = ot;
  }
  if (lane == 0) {
    wv[w] = best;
    wi[w] = btok;
  }
  __syncthreads();
  if (t == 0) {
    for (int i = 1; i < 16; ++i)
      if (wv[i] > wv[0] || (wv[i] == wv[0] && wi[i] < wi[0])) wv[0] = wv[i], wi[0] = wi[i];
    __hip_atomic_store(p.cand + k, ((unsigned long long)__float_as_uint(wv[0]) << 32) |
                                       (unsigned)(wi[0] == 0x7FFFFFFF ? 0xFFFFFFFFu : (unsigned)wi[0]),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_thread_fence(__ATOMIC_RELEASE);
    const unsigned old = __hip_atomic_fetch_add(p.done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = old == kSmpSlices - 1;
    if (last) __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  // The candidates and the token window staged by the block's threads (one load each); the
  // penalty's membership tests and the sort ranks in parallel; the sums and the draw on thread 0
  // in the firmware's order (the same float rounding).
  const int np = *p.n_prompt, j0 = max(0, pos + 1 - p.window), nwin = pos + 1 - j0;
  if (t < kSmpSlices) {
    const unsigned long long c = __hip_atomic_load(p.cand + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    cval[t] = __uint_as_float((uint32_t)(c >> 32));
    ctok[t] = (uint32_t)c == 0xFFFFFFFFu ? -1 : (int)(uint32_t)c;
    seen[t] = 0;
  } else if (t >= 64 && t - 64 < nwin) {
    const int j = j0 + t - 64, g = j - np;   // position j: a prompt token or generated token g
    win[t - 64] = j < np ? p.prompt[j % p.prompt_ring] : (g < p.max_out ? p.out[g] : -1);
  }
  __syncthreads();
  const float temp = p.cfg[0], top_p = p.cfg[1], rep = p.cfg[2];
  if (rep > 1.0f)
    for (int idx = t; idx < kSmpSlices * nwin; idx += 1024) {
      const int q = idx / nwin;
      if (ctok[q] >= 0 && win[idx - q * nwin] == ctok[q]) seen[q] = 1;
    }
  __syncthreads();
  if (t == 0) {
    int n = 0, bi = 0;
    for (int q = 0; q < kSmpSlices; ++q) {
      if (ctok[q] < 0) continue;
      float v = cval[q];
      if (rep > 1.0f && seen[q]) v = v > 0.f ? v / rep : v * rep;
      lg[n] = v;
      tk[n] = ctok[q];
      if (v > lg[bi]) bi = n;
      ++n;
    }
    n_s = n;
    if (n == 0) {
      n_s = -1;
    } else if (temp <= 0.0f) {
      n_s = -1;
      *p.slot = (1ull << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)tk[bi]);
    }
  }
  __syncthreads();
  const int n = n_s;
  if (n <= 0) return;
  if (t < n) {
    // Rank in the stable descending order: the larger values, then the equal ones before it.
    const float v = lg[t];
    int r = 0;
    for (int i = 0; i < n; ++i) r += lg[i] > v || (lg[i] == v && i < t);
    ord[r] = t;
  }
  __syncthreads();
  if (t < n) pr[t] = expf((lg[ord[t]] - lg[ord[0]]) / temp);
  __syncthreads();
  if (t != 0) return;
  float sum = 0.f;
  for (int i = 0; i < n; ++i) sum += pr[i];
  float acc = 0.f;
  const float cut = top_p * sum;
  int keep = n;
  for (int i = 0; i < n; ++i) {              // the smallest prefix holding top_p of the mass
    acc += pr[i];
    if (acc >= cut) {
      keep = i + 1;
      break;
    }
  }
  uint32_t x = *p.rng;
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  *p.rng = x;
  const float r = (float)(x >> 8) * (1.0f / 16777216.0f) * acc;
  float c = 0.f;
  int pick = tk[ord[keep - 1]];
  for (int i = 0; i < keep; ++i) {
    c += pr[i];
    if (r < c) {
      pick = tk[ord[i]];
      break;
    }
  }
  *p.slot = (1ull << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)pick);
}

// PrismML rotation ------------------------------------------------------------------------------

// One workgroup of B threads per block of columns. With a norm every workgroup sums x^2 over the
// whole vector (K <= a few tens of thousands: a few KB from L2 each). The butterflies of span
// below 64 exchange within a wave by shuffles, the wider ones through LDS; the natural-order
// butterfly (a + b, a - b) over spans 1, 2, 4, ... yields H v with H[i][j] = (-1)^popcount(i & j).
__global__ __launch_bounds__(1024) void rotate_kernel(RotParams p) {
  __shared__ float v[1024];
  __shared__ float red[16];
  const int t = threadIdx.x, B = blockDim.x, c = blockIdx.x * B + t;
  const int lane = t & 63, w = t >> 6;
  float a = p.x[c] * p.signs[c];
  if (p.norm_w) {
    float ss = 0.f;
    for (int i = t; i < p.K; i += B) {
      const float e = p.x[i];
      ss += e * e;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[w] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int k = 0; k < B / 64; ++k) tot += red[k];
    a *= p.norm_w[c] / sqrtf(tot / (float)p.K + p.eps);
  }
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
  p.y[c] = a * p.scale;
}

// Launchers ------------------------------------------------------------------------------------

int launch_sample(const SampleParams& p, hipStream_t s) {
  TRX_CHECK(p.n_ch >= 1 && p.vocab > 0 && p.window >= 0 && p.window <= kSmpWindowMax, TRX_E_INVALID,
            "sampling: bad parameters");
  hipLaunchKernelGGL(sample_kernel, dim3(kSmpSlices), dim3(1024), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_rotate(const RotParams& p, hipStream_t s) {
  TRX_CHECK(p.B >= 64 && p.B <= 1024 && (p.B & (p.B - 1)) == 0 && p.K > 0 && p.K % p.B == 0 && p.x != p.y,
            TRX_E_INVALID, "rotation: block %d over %d columns unsupported", p.B, p.K);
  hipLaunchKernelGGL(rotate_kernel, dim3(p.K / p.B), dim3(p.B), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_embed_rows(const EmbedParams& p, const int* fed, int p0, int R, float* X, hipStream_t s) {
  TRX_CHECK(p.n_embd % kGroup == 0 && p.n_embd / kGroup <= kMaxEmbedGroups && R >= 1, TRX_E_INVALID,
            "embedding: n_embd %d unsupported", p.n_embd);
  TRX_CHECK(p.mode == EMBED_TABLE || (p.row_bytes % 16 == 0 && p.row_bytes <= kEmbedRowMax), TRX_E_INVALID,
            "embedding: row of %d bytes unsupported", p.row_bytes);
  TRX_CHECK(p.mode != EMBED_RESTORE || (p.signs && p.hblock >= 1 && p.n_embd % p.hblock == 0 &&
                                        p.n_embd <= kRestoreMax), TRX_E_INVALID,
            "embedding: restore of %d columns in blocks of %d unsupported", p.n_embd, p.hblock);
  hipLaunchKernelGGL(embed_rows_kernel, dim3(R), dim3(kEmbedThreads), 0, s, p, fed, p0, X);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_embed(const EmbedParams& p, hipStream_t s) {
  TRX_CHECK(p.n_embd % kGroup == 0 && p.n_embd / kGroup <= kMaxEmbedGroups, TRX_E_INVALID,
            "embedding: n_embd %d unsupported", p.n_embd);
  TRX_CHECK(p.mode == EMBED_TABLE || (p.row_bytes % 16 == 0 && p.row_bytes <= kEmbedRowMax), TRX_E_INVALID,
            "embedding: row of %d bytes unsupported", p.row_bytes);
  TRX_CHECK(p.mode != EMBED_RESTORE || (p.signs && p.hblock >= 1 && p.n_embd % p.hblock == 0 &&
                                        p.n_embd <= kRestoreMax), TRX_E_INVALID,
            "embedding: restore of %d columns in blocks of %d unsupported", p.n_embd, p.hblock);
  hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(kEmbedThreads), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

// Score ------------------------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void score_kernel(ScoreParams p) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  const int pos = p.pos ? *p.pos : 0;
  // The normed hidden state (fastref.py:143-145 with the output norm, fastref.py:258).
  float ss = 0.f;
  for (int i = tid; i < p.n; i += 1024) ss += p.x[i] * p.x[i];
  const float r = 1.0f / sqrtf(block_sum(ss, red) / (float)p.n + p.eps);
  if (p.hid && pos < p.max_rows)
    for (int i = tid; i < p.n; i += 1024) p.hid[(size_t)pos * p.n + i] = p.x[i] * r * p.out_norm[i];
  if (!p.logits || pos < *p.head_from || pos + 1 >= *p.n_fed) return;
  // log-sum-exp over the vocabulary, then the next token's negative log-likelihood
  // (fastref.py:267-272).
  float mx = -INFINITY;
  for (int i = tid; i < p.vocab; i += 1024) mx = fmaxf(mx, p.logits[i]);
  mx = wave_max(mx);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < 16; ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  float se = 0.f;
  for (int i = tid; i < p.vocab; i += 1024) se += expf(p.logits[i] - m);
  se = block_sum(se, red);
  if (tid == 0) p.nll[pos] = (m + logf(se)) - p.logits[p.fed[pos + 1]];
}

int launch_score(const ScoreParams& p, hipStream_t s) {
  TRX_CHECK(p.x && p.out_norm && p.n > 0 && (!p.logits || (p.nll && p.pos && p.head_from && p.n_fed && p.fed)),
            TRX_E_INVALID, "score: bad arguments");
  hipLaunchKernelGGL(score_kernel, dim3(1), dim3(1024), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_finalize(const int* pos, const int* n_prompt, unsigned long long* slot, int* out, int max_out,
                    hipStream_t s) {
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(64), 0, s, pos, n_prompt, slot, out, max_out);
  TRX_LAUNCHED();
  return TRX_OK;
}

// Attention (the device code is in trx_attn_dev.h) --------------------------------------------

template <int REP, int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnParams p) {
  attn_split_body<REP, HD>(p, blockIdx.x);
}

__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p) { attn_merge_body<false>(p, blockIdx.x); }

int attention_max_chunk(int head_dim) {
  return head_dim == 64 ? attn_max_chunk<64>() : head_dim == 128 ? attn_max_chunk<128>() : attn_max_chunk<256>();
}

int attention_pass_positions(int head_dim) { return kFdThreads / (head_dim / 8); }

int attention_splits(int n_kv, int head_dim, int max_ctx) {
  // Enough blocks to cover the CUs, but at most 32 (the splits the o projection's prologue
  // merges, saving a merge launch) unless the register-held positions per block need more.
  int cap = head_dim == 64 ? attn_max_chunk<64>() : head_dim == 128 ? attn_max_chunk<128>()
                                                                      : attn_max_chunk<256>();
  int s = min(cdiv(256, n_kv > 0 ? n_kv : 1), 32);
  if (cdiv(max_ctx, s) > cap) s = cdiv(max_ctx, cap);
  return s > 64 ? -1 : s;
}

static int hd_threads(int hd) { return hd < 256 ? (hd < 64 ? 64 : hd) : 256; }

template <int REP>
static int launch_attn_rep(const AttnParams& p, hipStream_t s) {
  const dim3 grid(p.n_kv * p.n_split), block(kAttnThreads);
  switch (p.hd) {
    case 64: hipLaunchKernelGGL((attn_decode_kernel<REP, 64>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((attn_decode_kernel<REP, 128>), grid, block, 0, s, p); break;
    case 256: hipLaunchKernelGGL((attn_decode_kernel<REP, 256>), grid, block, 0, s, p); break;
    default: TRX_CHECK(false, TRX_E_INVALID, "attention: head_dim %d unsupported", p.hd);
  }
  TRX_LAUNCHED();
  hipLaunchKernelGGL(attn_merge_kernel, dim3(p.n_head), dim3(hd_threads(p.hd)), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_attention_merge(const AttnParams& p, hipStream_t s) {
  hipLaunchKernelGGL(attn_merge_kernel, dim3(p.n_head), dim3(hd_threads(p.hd)), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_attention(const AttnParams& p, hipStream_t s) {
  const int cap = p.hd == 64 ? attn_max_chunk<64>() : p.hd == 128 ? attn_max_chunk<128>() : attn_max_chunk<256>();
  TRX_CHECK(p.rope_n <= p.hd && p.rope_n % 2 == 0, TRX_E_INVALID, "attention: rope dims %d", p.rope_n);
  TRX_CHECK(p.n_split >= 1 && p.n_split <= kMaxSplits && cdiv(p.max_ctx, p.n_split) <= cap,
            TRX_E_INVALID, "attention: %d splits for context %d", p.n_split, p.max_ctx);
  switch (p.n_rep) {
    case 1: return launch_attn_rep<1>(p, s);
    case 2: return launch_attn_rep<2>(p, s);
    case 4: return launch_attn_rep<4>(p, s);
    case 6: return launch_attn_rep<6>(p, s);
    case 8: return launch_attn_rep<8>(p, s);
    default: TRX_CHECK(false, TRX_E_INVALID, "attention: %d q heads per kv head unsupported", p.n_rep);
  }
}

int launch_dense_gemv(const DenseParams& p, hipStream_t s) {
  if (p.kind == TRX_KIND_Q8 && !p.amax_slot && p.K % 32 == 0 && p.code_off % 16 == 0 && p.row_bytes % 16 == 0 &&
      ((uintptr_t)p.W | (uintptr_t)p.x | (uintptr_t)p.norm_w) % 16 == 0) {
    hipLaunchKernelGGL(q8_gemv_kernel, dim3(p.M), dim3(256), 0, s, p);
    TRX_LAUNCHED();
    return TRX_OK;
  }
  int blocks = (p.M + 3) / 4;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(dense_gemv_kernel, dim3(blocks), dim3(256), p.K * sizeof(float), s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_synth_ternary(const SynthParams& p, hipStream_t s) {
  hipLaunchKernelGGL(synth_ternary_kernel, dim3(4096), dim3(256), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_synth_f32(float* out, long long n, uint32_t seed, uint32_t tensor_id, float lo, float span,
                     int transform, hipStream_t s) {
  hipLaunchKernelGGL(synth_f32_kernel, dim3(256), dim3(256), 0, s, out, n, seed, tensor_id, lo, span, transform);
  TRX_LAUNCHED();
  return TRX_OK;
}

}  // namespace trx
