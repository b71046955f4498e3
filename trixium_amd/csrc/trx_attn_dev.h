// Device code of decode attention for the split kernel and the merge kernel (trx_ops.hip).
//
// Split body: the work of one (kv head g, split sp) pair. It owns the positions
// [sp*chunk, (sp+1)*chunk) of the T = pos + 1 cached ones (chunk = ceil(T / n_split)), for the
// REP q heads sharing g (model/fastref.py:216-241):
//   - the split's K and V rows are loaded into registers first (16-byte loads, HD/8 lanes per
//     position), so one memory round trip overlaps the rest of the prologue;
//   - q: RMS-normalised per head, rotated (NEOX pairs on the first rope_n dims, angle =
//     pos * freq in fp32, or the cos/sin of the model's Q14 table row) and scaled by 1/sqrt(hd); the block holding `pos` does the same for
//     the new k and appends k (post-RoPE) and v to the fp16 cache;
//   - scores, softmax over the split, the unnormalised V sum; the split's (max, sum, output) go
//     to the partials.
// The first kAttnThreads threads of the block do the work; every thread of the block reaches
// its barriers.
// Merge body: one q head's partials merged, the output gate of gated attention applied.
#pragma once

#include "trx_internal.h"
#include "trx_ops.h"

namespace trx {

constexpr int kAttnThreads = 256;
constexpr int kFdThreads = 256;            // threads of the one-launch kernel's blocks
constexpr int kMaxRep = 8;
constexpr int kMaxPass = 8;                 // register-held positions per thread
constexpr int kMaxChunk = 128;

template <int HD>
__host__ __device__ constexpr int attn_max_chunk() {
  // positions per pass = threads / (HD/8); at most kMaxPass passes and kMaxChunk positions.
  return (kMaxPass * (kAttnThreads / (HD / 8))) < kMaxChunk ? kMaxPass * (kAttnThreads / (HD / 8)) : kMaxChunk;
}

__device__ __forceinline__ void h8_to_f(const uint4 raw, float* out) {
  const __half* hh = (const __half*)&raw;
#pragma unroll
  for (int k = 0; k < 8; ++k) out[k] = __half2float(hh[k]);
}

template <int REP, int HD, bool FUSED = false, class Wait = NoWait>
__device__ __forceinline__ void attn_split_body(const AttnParams& p, int bid, Wait wait = Wait{}) {
  constexpr int LPP = HD / 8;                          // lanes per position
  constexpr int PPW = 64 / LPP;                        // positions per wave per pass
  constexpr int PPP = PPW * (kAttnThreads / 64);       // positions per pass
  constexpr int NH = REP + 1;                          // q heads + the new k
  __shared__ float hv[NH + 1][HD];                     // q heads, k, v (normalised / rotated)
  __shared__ float cs_s[HD / 2], sn_s[HD / 2];
  __shared__ float sc_s[REP][kMaxChunk];
  __shared__ float vred[kAttnThreads / 64][REP][HD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool worker = tid < kAttnThreads;              // whole waves
  const int S = p.n_split;
  const int g = bid / S, sp = bid - g * S;
  const bool active = g < p.n_kv;
  // The position (RoPE), the KV slot its k and v go to, and the T slots attended (the position
  // and pos + 1 inside the window, the KV ring's slot and every slot past it).
  const int pos = p.pos[0], slot = p.pos[5], T = p.pos[6];
  const int chunk = (T + S - 1) / S;
  const int p0 = sp * chunk, p1 = min(T, p0 + chunk), n = active ? max(0, p1 - p0) : 0;
  const int qstride = p.gated ? 2 * HD : HD;
  const size_t cache0 = (size_t)g * p.max_ctx * HD;
  const bool owner = n > 0 && slot >= p0 && slot < p1;
  const int li = lane % LPP, sub = lane / LPP;
  const int npass = (n + PPP - 1) / PPP;

  // 1. K and V rows of the split into registers (the position being added is not cached yet:
  //    its row is taken from LDS below).
  uint4 kr[kMaxPass], vr[kMaxPass];
#pragma unroll
  for (int ps = 0; ps < kMaxPass; ++ps) {
    const int t = ps * PPP + wave * PPW + sub;
    if (worker && ps < npass && t < n && p0 + t != slot) {
      const size_t off = cache0 + (size_t)(p0 + t) * HD + li * 8;
      kr[ps] = *(const uint4*)(p.kcache + off);
      vr[ps] = *(const uint4*)(p.vcache + off);
    } else {
      kr[ps] = make_uint4(0, 0, 0, 0);
      vr[ps] = make_uint4(0, 0, 0, 0);
    }
  }
  if (FUSED) wait();

  if (n > 0) {
    // 2. q heads (and k, v for the owner) into LDS; rotation table.
    const float* kraw = p.qkv + (size_t)p.n_head * qstride + (size_t)g * HD;
    const int half = p.rope_n / 2;
    if (worker) {
      for (int i = tid; i < NH * HD; i += kAttnThreads) {
        const int j = i / HD, d = i - j * HD;
        if (j < REP) hv[j][d] = ld_vec<FUSED>(p.qkv + (size_t)(g * REP + j) * qstride + d);
        else if (owner) hv[REP][d] = ld_vec<FUSED>(kraw + d);
      }
      if (owner)
        for (int d = tid; d < HD; d += kAttnThreads) hv[REP + 1][d] = ld_vec<FUSED>(kraw + (size_t)p.n_kv * HD + d);
      for (int i = tid; i < half; i += kAttnThreads) {
        float sn, cs;
        if (p.rope_tab) {
          cs = (float)p.rope_tab[(size_t)pos * p.rope_n + i] * (1.0f / 16384.0f);
          sn = (float)p.rope_tab[(size_t)pos * p.rope_n + half + i] * (1.0f / 16384.0f);
        } else {
          sincosf((float)pos * p.rope_freq[i], &sn, &cs);
        }
        cs_s[i] = cs;
        sn_s[i] = sn;
      }
    }
    __syncthreads();
    // 3. RMSNorm per head (a wave per head) and RoPE, in place.
    if (worker) {
      for (int j = wave; j < NH; j += kAttnThreads / 64) {
        if (j == REP && !owner) continue;
        const float* w = (j < REP) ? p.q_norm : p.k_norm;
        float ss = 0.f;
        for (int d = lane; d < HD; d += 64) ss += hv[j][d] * hv[j][d];
        ss = wave_sum(ss);
        const float r = 1.0f / sqrtf(ss / (float)HD + p.eps);
        const float post = (j < REP) ? 1.0f / sqrtf((float)HD) : 1.0f;
        float nv[(HD + 63) / 64];
#pragma unroll
        for (int k = 0; k < (HD + 63) / 64; ++k) {
          const int d = lane + 64 * k;
          nv[k] = d < HD ? hv[j][d] * r * w[d] : 0.f;
        }
        // Rotation: pair (i, i + half) for i < half; dims past rope_n pass through.
        float ov[(HD + 63) / 64];
#pragma unroll
        for (int k = 0; k < (HD + 63) / 64; ++k) ov[k] = nv[k];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < (HD + 63) / 64; ++k)
          if (lane + 64 * k < HD) hv[j][lane + 64 * k] = nv[k];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int k = 0; k < (HD + 63) / 64; ++k) {
          const int d = lane + 64 * k;
          if (d < half) ov[k] = nv[k] * cs_s[d] - hv[j][d + half] * sn_s[d];
          else if (d < 2 * half) ov[k] = hv[j][d - half] * sn_s[d - half] + nv[k] * cs_s[d - half];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < (HD + 63) / 64; ++k)
          if (lane + 64 * k < HD) hv[j][lane + 64 * k] = ov[k] * post;
      }
    }
    __syncthreads();
    if (owner && tid < HD) {
      const __half kh = __float2half(hv[REP][tid]), vh = __float2half(hv[REP + 1][tid]);
      p.kcache[cache0 + (size_t)slot * HD + tid] = kh;
      p.vcache[cache0 + (size_t)slot * HD + tid] = vh;
      hv[REP][tid] = __half2float(kh);
      hv[REP + 1][tid] = __half2float(vh);
    }
    __syncthreads();
    // 4. Scores.
    if (worker) {
      float qr[REP][8];
#pragma unroll
      for (int j = 0; j < REP; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) qr[j][k] = hv[j][li * 8 + k];
#pragma unroll
      for (int ps = 0; ps < kMaxPass; ++ps) {
        if (ps >= npass) break;
        const int t = ps * PPP + wave * PPW + sub;
        float kv[8];
        if (owner && p0 + t == slot) {
#pragma unroll
          for (int k = 0; k < 8; ++k) kv[k] = hv[REP][li * 8 + k];
        } else {
          h8_to_f(kr[ps], kv);
        }
#pragma unroll
        for (int j = 0; j < REP; ++j) {
          float sdot = 0.f;
#pragma unroll
          for (int k = 0; k < 8; ++k) sdot += qr[j][k] * kv[k];
#pragma unroll
          for (int o = LPP >> 1; o >= 1; o >>= 1) sdot += __shfl_xor(sdot, o, 64);
          if (t < n && li == 0) sc_s[j][t] = sdot;
        }
      }
    }
    __syncthreads();
    // 5. Softmax over the split, a wave per head.
    if (worker) {
      for (int j = wave; j < REP; j += kAttnThreads / 64) {
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
          st_vec<FUSED>(p.part_m + (size_t)(g * REP + j) * S + sp, m);
          st_vec<FUSED>(p.part_l + (size_t)(g * REP + j) * S + sp, l);
        }
      }
    }
    __syncthreads();
    // 6. V: every thread sums its register-held positions, then over the wave's position slots
    //    (lanes li, li + LPP, ...) and over the waves.
    if (worker) {
      float acc[REP][8];
#pragma unroll
      for (int j = 0; j < REP; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[j][k] = 0.f;
#pragma unroll
      for (int ps = 0; ps < kMaxPass; ++ps) {
        if (ps >= npass) break;
        const int t = ps * PPP + wave * PPW + sub;
        if (t >= n) continue;
        float v[8];
        if (owner && p0 + t == slot) {
#pragma unroll
          for (int k = 0; k < 8; ++k) v[k] = hv[REP + 1][li * 8 + k];
        } else {
          h8_to_f(vr[ps], v);
        }
#pragma unroll
        for (int j = 0; j < REP; ++j) {
          const float pj = sc_s[j][t];
#pragma unroll
          for (int k = 0; k < 8; ++k) acc[j][k] += pj * v[k];
        }
      }
#pragma unroll
      for (int j = 0; j < REP; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          float a = acc[j][k];
#pragma unroll
          for (int o = LPP; o < 64; o <<= 1) a += __shfl_xor(a, o, 64);
          acc[j][k] = a;
        }
      if (sub == 0) {
#pragma unroll
        for (int j = 0; j < REP; ++j)
#pragma unroll
          for (int k = 0; k < 8; ++k) vred[wave][j][li * 8 + k] = acc[j][k];
      }
    }
    __syncthreads();
    if (worker) {
      for (int i = tid; i < REP * HD; i += kAttnThreads) {
        const int j = i / HD, d = i - j * HD;
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnThreads / 64; ++w) o += vred[w][j][d];
        st_vec<FUSED>(p.part_o + ((size_t)(g * REP + j) * S + sp) * HD + d, o);
      }
    }
  } else if (active) {
    // An empty split contributes nothing to the merge.
    if (tid < REP) {
      st_vec<FUSED>(p.part_m + (size_t)(g * REP + tid) * S + sp, -INFINITY);
      st_vec<FUSED>(p.part_l + (size_t)(g * REP + tid) * S + sp, 0.f);
    }
  }
}

constexpr int kMaxSplits = 256;

// Merge of the split partials of q head qh (any block size >= 64; at most kMaxSplits splits).
template <bool FUSED = false>
__device__ __forceinline__ void attn_merge_body(const AttnParams& p, int qh) {
  __shared__ float wsp[kMaxSplits];
  const int tid = threadIdx.x;
  const int S = p.n_split, hd = p.hd;
  const int T = p.pos[6];                               // KV slots attended
  const int chunk = (T + S - 1) / S;
  const int ns = min(S, (T + chunk - 1) / chunk);      // splits holding positions
  const float* pm = p.part_m + (size_t)qh * S;
  const float* pl = p.part_l + (size_t)qh * S;
  if (tid < 64) {
    float mv[kMaxSplits / 64], lv[kMaxSplits / 64];
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMaxSplits / 64; ++k) {
      const int s2 = tid + 64 * k;
      mv[k] = s2 < ns ? ld_vec<FUSED>(pm + s2) : -INFINITY;
      lv[k] = s2 < ns ? ld_vec<FUSED>(pl + s2) : 0.f;
      M = fmaxf(M, mv[k]);
    }
    M = wave_max(M);
    float L = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxSplits / 64; ++k) {
      mv[k] = tid + 64 * k < ns ? __expf(mv[k] - M) : 0.f;
      L += lv[k] * mv[k];
    }
    L = wave_sum(L);
#pragma unroll
    for (int k = 0; k < kMaxSplits / 64; ++k) wsp[tid + 64 * k] = mv[k] / L;
  }
  __syncthreads();
  const float* po = p.part_o + (size_t)qh * S * hd;
  for (int d = tid; d < hd; d += blockDim.x) {
    float o = 0.f;
    // 32 independent loads per round: 64 splits in two round trips.
    for (int s0 = 0; s0 < ns; s0 += 32) {
      float v[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) v[k] = (s0 + k < ns) ? ld_vec<FUSED>(po + (size_t)(s0 + k) * hd + d) : 0.f;
#pragma unroll
      for (int k = 0; k < 32; ++k) o += (s0 + k < ns) ? v[k] * wsp[s0 + k] : 0.f;
    }
    if (p.gated) o *= sigmoidf_(ld_vec<FUSED>(p.qkv + (size_t)qh * 2 * hd + hd + d));
    st_vec<FUSED>(p.out + (size_t)qh * hd + d, o);
  }
}

}  // namespace trx
