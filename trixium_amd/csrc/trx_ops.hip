// Decode-loop kernels other than the ternary GEMV: token embedding, split-K GQA decode attention
// over an fp16 KV cache (QK-RMSNorm, RoPE and the KV append fused in), the split combine, a
// dense fp16 / Q8 GEMV (small heads and the DeltaNet beta/alpha projections), the greedy
// token resolve, and the on-device synthetic weight generator.

#include "trx_internal.h"
#include "trx_ops.h"

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
__global__ __launch_bounds__(256) void embed_kernel(EmbedParams p) {
  __shared__ int s_tok;
  __shared__ int s_red[8];
  __shared__ int s_emin, s_k2;
  const int tid = threadIdx.x;
  if (tid == 0) {
    int pos = *p.pos + 1;
    *p.pos = pos;
    int tok;
    if (pos < *p.n_prompt) {
      tok = p.prompt[pos];
    } else {
      tok = slot_token(*p.slot);
      const int k = pos - *p.n_prompt;
      if (k < p.max_out) p.out[k] = tok;
    }
    if (tok < 0 || tok >= p.vocab) tok = 0;
    *p.slot = 0ull;
    *p.cur_tok = tok;
    s_tok = tok;
  }
  __syncthreads();
  const int tok = s_tok;
  if (p.mode == EMBED_TABLE) {
    const float sc = bfp_scale(p.exps[tok]);
    const int16_t* m = p.mant + (size_t)tok * p.n_embd;
    for (int c = tid; c < p.n_embd; c += 256) p.x[c] = (float)m[c] * sc;
    return;
  }
  // Ternary row: scales at the head of the row packet, codes after code_off.
  const uint8_t* row = p.rows + (size_t)tok * p.row_bytes;
  const uint16_t* sc = (const uint16_t*)row;
  const int G = p.n_embd / kGroup;
  // Pass 1: smallest exponent over the row, live absmax of aligned |m11|.
  int emin = 1 << 20;
  for (int g = tid; g < G; g += 256) {
    int m11, e16;
    fp16_split(sc[g], m11, e16);
    emin = min(emin, e16);
  }
  for (int o = 32; o >= 1; o >>= 1) emin = min(emin, __shfl_xor(emin, o, 64));
  if ((tid & 63) == 0) s_red[tid >> 6] = emin;
  __syncthreads();
  if (tid == 0) {
    int m = s_red[0];
    for (int i = 1; i < 4; ++i) m = min(m, s_red[i]);
    s_emin = m;
  }
  __syncthreads();
  emin = s_emin;
  // codes of column c
  auto code_of = [&](int c) -> int {
    if (p.kind == TRX_KIND_TERNARY5) {
      const int g = c >> 7, j = c & 127, byte = j / 5, k = j - 5 * byte;
      int b = row[p.code_off + kTrit5GroupBytes * g + byte];
      for (int i = 0; i < k; ++i) b /= 3;
      return b % 3;
    }
    return (row[p.code_off + (c >> 2)] >> (2 * (c & 3))) & 3;
  };
  long long amax = 0;
  for (int g = 0; g < G; ++g) {
    int live = 0;
    for (int j = tid; j < kGroup; j += 256) live |= (code_of(g * kGroup + j) != 1);
    live = __syncthreads_or(live);
    if (live && tid == 0) {
      int m11, e16;
      fp16_split(sc[g], m11, e16);
      int sh = min(e16 - emin, 20);
      long long v = (long long)(m11 < 0 ? -m11 : m11) << sh;
      if (v > amax) amax = v;
    }
  }
  if (tid == 0) {
    int bl = 0;
    while (bl < 63 && (amax >> bl) != 0) ++bl;
    s_k2 = bl - 15;
  }
  __syncthreads();
  const int k2 = s_k2;
  const float scale = bfp_scale(emin + k2);
  for (int c = tid; c < p.n_embd; c += 256) {
    int m11, e16;
    fp16_split(sc[c >> 7], m11, e16);
    const int sh = min(e16 - emin, 20) - k2;
    const long long v = (long long)(code_of(c) - 1) * m11;
    const long long w = sh >= 0 ? (v << sh) : (v >> (-sh));
    p.x[c] = (float)(int16_t)(w & 0xFFFF) * scale;
  }
}

// Resolve the last generated token (after the final step): out[pos + 1 - n_prompt].
__global__ void finalize_kernel(const int* pos, const int* n_prompt, unsigned long long* slot, int* out,
                                int max_out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int k = *pos + 1 - *n_prompt;
    if (k >= 0 && k < max_out) out[k] = slot_token(*slot);
  }
}

// Attention -------------------------------------------------------------------------------------
//
// One block per (kv head, split of `chunk` positions). q of the n_rep heads sharing the kv head
// and (in the split holding the current position) the new k are RMS-normalised per head and
// rotated (NEOX pairs on the first rope_n dims, angle = pos * freq in fp32; model/fastref.py:
// 216-241); the new k (post-RoPE) and v are appended to the fp16 cache at pos. Each block writes
// its split's softmax partials (max, sum, unnormalised output) per q head.

constexpr int kAttnThreads = 256;
constexpr int kMaxHd = 256;
constexpr int kMaxRep = 8;

__device__ void head_norm_rope(float* v, const float* w, const float* freq, int hd, int rope_n,
                               float eps, int pos, float post_scale, float* red, int tid, int nthreads) {
  // v: one head in LDS (hd floats), normalised and rotated in place by the block.
  float ss = 0.f;
  for (int d = tid; d < hd; d += nthreads) ss += v[d] * v[d];
  ss = wave_sum(ss);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < (nthreads + 63) / 64; ++i) tot += red[i];
  const float r = 1.0f / sqrtf(tot / (float)hd + eps);
  float nv[2] = {0.f, 0.f};
  int nd = 0;
  for (int d = tid; d < hd; d += nthreads) nv[nd++] = v[d] * r * w[d];
  __syncthreads();
  nd = 0;
  for (int d = tid; d < hd; d += nthreads) v[d] = nv[nd++];
  __syncthreads();
  const int half = rope_n / 2;
  for (int i = tid; i < half; i += nthreads) {
    const float ang = (float)pos * freq[i];
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const float x0 = v[i], x1 = v[i + half];
    v[i] = x0 * cs - x1 * sn;
    v[i + half] = x0 * sn + x1 * cs;
  }
  __syncthreads();
  if (post_scale != 1.0f)
    for (int d = tid; d < hd; d += nthreads) v[d] *= post_scale;
  __syncthreads();
}

__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(AttnParams p) {
  __shared__ float q_s[kMaxRep][kMaxHd];
  __shared__ float kn_s[kMaxHd];
  __shared__ float vn_s[kMaxHd];
  __shared__ float sc_s[kMaxRep][64];
  __shared__ float red[8];
  const int tid = threadIdx.x;
  const int h = blockIdx.x / p.n_split, sp = blockIdx.x - h * p.n_split;
  const int pos = *p.pos;
  const int T = pos + 1;
  const int p0 = sp * p.chunk;
  if (p0 >= T) return;
  const int p1 = min(p0 + p.chunk, T);
  const int hd = p.hd, rep = p.n_rep;
  const int qstride = p.gated ? 2 * hd : hd;
  const float qscale = 1.0f / sqrtf((float)hd);
  // q heads of this group (raw projection rows) -> LDS, normalised and rotated.
  for (int j = 0; j < rep; ++j) {
    const float* src = p.qkv + (size_t)(h * rep + j) * qstride;
    for (int d = tid; d < hd; d += kAttnThreads) q_s[j][d] = src[d];
    __syncthreads();
    head_norm_rope(q_s[j], p.q_norm, p.rope_freq, hd, p.rope_n, p.eps, pos, qscale, red, tid, kAttnThreads);
  }
  const bool has_new = (pos >= p0 && pos < p1);
  if (has_new) {
    const float* ksrc = p.qkv + (size_t)p.n_head * qstride + (size_t)h * hd;
    const float* vsrc = p.qkv + (size_t)p.n_head * qstride + (size_t)p.n_kv * hd + (size_t)h * hd;
    for (int d = tid; d < hd; d += kAttnThreads) { kn_s[d] = ksrc[d]; vn_s[d] = vsrc[d]; }
    __syncthreads();
    head_norm_rope(kn_s, p.k_norm, p.rope_freq, hd, p.rope_n, p.eps, pos, 1.0f, red, tid, kAttnThreads);
    if (sp == pos / p.chunk) {
      __half* kc = p.kcache + ((size_t)h * p.max_ctx + pos) * hd;
      __half* vc = p.vcache + ((size_t)h * p.max_ctx + pos) * hd;
      for (int d = tid; d < hd; d += kAttnThreads) { kc[d] = __float2half(kn_s[d]); vc[d] = __float2half(vn_s[d]); }
    }
  }
  // Scores: one position per 64/ (hd/8)... each wave handles positions; lanes split hd.
  const int n = p1 - p0;
  const int lane = tid & 63, wave = tid >> 6;
  const int lpp = hd / 8;                    // lanes per position (8 dims each)
  const int ppw = 64 / lpp;                  // positions per wave step
  const int sub = lane / lpp, li = lane - sub * lpp;
  for (int t0 = wave * ppw; t0 < n; t0 += (kAttnThreads / 64) * ppw) {
    const int t = t0 + sub;
    float kv[8];
    const bool ok = t < n;
    if (ok) {
      const int ap = p0 + t;
      if (has_new && ap == pos) {
        for (int k = 0; k < 8; ++k) kv[k] = __half2float(__float2half(kn_s[li * 8 + k]));
      } else {
        const uint4 raw = *(const uint4*)(p.kcache + ((size_t)h * p.max_ctx + ap) * hd + li * 8);
        const __half* hh = (const __half*)&raw;
        for (int k = 0; k < 8; ++k) kv[k] = __half2float(hh[k]);
      }
    } else {
      for (int k = 0; k < 8; ++k) kv[k] = 0.f;
    }
    for (int j = 0; j < rep; ++j) {
      float s = 0.f;
      for (int k = 0; k < 8; ++k) s += q_s[j][li * 8 + k] * kv[k];
      for (int o = lpp >> 1; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
      if (ok && li == 0) sc_s[j][t] = s;
    }
  }
  __syncthreads();
  // Softmax partials per q head (one wave per head while heads remain).
  for (int j = wave; j < rep; j += kAttnThreads / 64) {
    float m = -INFINITY;
    for (int t = lane; t < n; t += 64) m = fmaxf(m, sc_s[j][t]);
    m = wave_max(m);
    float l = 0.f;
    for (int t = lane; t < n; t += 64) {
      const float e = __expf(sc_s[j][t] - m);
      sc_s[j][t] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      const size_t idx = (size_t)(h * rep + j) * p.n_split + sp;
      p.part_m[idx] = m;
      p.part_l[idx] = l;
    }
  }
  __syncthreads();
  // Unnormalised outputs: thread per (head, dim).
  for (int od = tid; od < rep * hd; od += kAttnThreads) {
    const int j = od / hd, d = od - j * hd;
    float acc = 0.f;
    for (int t = 0; t < n; ++t) {
      const int ap = p0 + t;
      float v;
      if (has_new && ap == pos) v = __half2float(__float2half(vn_s[d]));
      else v = __half2float(p.vcache[((size_t)h * p.max_ctx + ap) * hd + d]);
      acc += sc_s[j][t] * v;
    }
    p.part_o[((size_t)(h * rep + j) * p.n_split + sp) * hd + d] = acc;
  }
}

// Combine the split partials of every q head; gated attention multiplies by sigmoid(gate).
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
  const int qh = blockIdx.x;
  const int T = *p.pos + 1;
  const int ns = (T + p.chunk - 1) / p.chunk;
  const int hd = p.hd;
  const float* pm = p.part_m + (size_t)qh * p.n_split;
  const float* pl = p.part_l + (size_t)qh * p.n_split;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, pm[s]);
  float L = 0.f;
  for (int s = 0; s < ns; ++s) L += pl[s] * __expf(pm[s] - M);
  const float invL = 1.0f / L;
  for (int d = threadIdx.x; d < hd; d += 256) {
    float acc = 0.f;
    for (int s = 0; s < ns; ++s) acc += p.part_o[((size_t)qh * p.n_split + s) * hd + d] * __expf(pm[s] - M);
    float o = acc * invL;
    if (p.gated) {
      const float g = p.qkv[(size_t)qh * 2 * hd + hd + d];
      o *= sigmoidf_(g);
    }
    p.out[(size_t)qh * hd + d] = o;
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
        atomicMax(p.amax_slot, ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)m));
      }
    }
  }
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

// Launchers ------------------------------------------------------------------------------------

int launch_embed(const EmbedParams& p, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(256), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_finalize(const int* pos, const int* n_prompt, unsigned long long* slot, int* out, int max_out,
                    hipStream_t s) {
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(64), 0, s, pos, n_prompt, slot, out, max_out);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_attention(const AttnParams& p, hipStream_t s) {
  TRX_CHECK(p.hd % 8 == 0 && p.hd <= kMaxHd && 64 % (p.hd / 8) == 0 && p.n_rep <= kMaxRep &&
            p.chunk <= 64, TRX_E_INVALID, "attention: unsupported geometry hd=%d rep=%d", p.hd, p.n_rep);
  hipLaunchKernelGGL(attn_split_kernel, dim3(p.n_kv * p.n_split), dim3(kAttnThreads), 0, s, p);
  TRX_LAUNCHED();
  hipLaunchKernelGGL(attn_combine_kernel, dim3(p.n_head), dim3(256), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_dense_gemv(const DenseParams& p, hipStream_t s) {
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
