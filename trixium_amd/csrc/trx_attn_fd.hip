// Decode attention for one position in one launch (flash decoding): a block per (kv head, split)
// of the T = pos + 1 cached positions, the split's partial (max, sum, output) per q head, and the
// merge of a kv head's splits by the block that finishes last. The arithmetic is that of
// model/fastref.py:216-241 for one position: q and k RMS-normalised per head, NEOX RoPE on the
// first rope_n dims (angle = pos * freq in fp32, or the model's Q14 cos/sin table row), q scaled by 1/sqrt(hd), k (post-RoPE) and v
// appended to the fp16 cache and read back rounded, softmax over the positions, the output gate
// of gated attention.
//
// Lanes: a position is handled by LPP = hd/8 lanes (8 dims each), a "group"; a block of 256
// threads has 256/LPP groups. The split's K and V rows are loaded into registers first. q (and
// the new k, v) are normalised and rotated once per block in LDS, then every group reads q.
// Each group computes the scores of its positions, then their max, sum of exponentials and
// weighted V; the groups are combined through LDS once.

#include "trx_internal.h"
#include "trx_ops.h"
#include "trx_attn_dev.h"

namespace trx {

constexpr int kFdMaxSplits = 64;
constexpr int kCpolSc1 = 16;           // buffer cache policy: device (agent) scope

// Sum over the LPP lanes of a position group (every lane gets the sum).
template <int LPP>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  if (LPP >= 4) v += dpp_f<kDppQuadXor2>(v);
  if (LPP >= 8) v += dpp_f<kDppRowHalfMirror>(v);
  if (LPP >= 16) v += dpp_f<kDppRowMirror>(v);
  if (LPP >= 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// QPS > 0 (QP): q, k and v arrive as the q|k|v GEMV's K-slice partial sums (p.qkv_part,
// [S][rows_p], S <= QPS, with its RMSNorm's slice sums of x^2 in p.qkv_ss), summed here in slice
// order: y = r * sum_s part[s], r = 1/sqrt(sum(ss) / K + eps). QPS is 8 or 16, the smallest that
// holds S, so a GEMV of 8 slices does not load each partial twice.
// The q heads and the new k are normalised and rotated once per block, not by every position
// group.
template <int REP, int HD, int QPS>
__global__ __launch_bounds__(kFdThreads) void attn_fd_kernel(AttnParams p) {
  constexpr bool QP = QPS > 0;
  constexpr int LPP = HD / 8;                         // lanes per position
  constexpr int PPW = 64 / LPP;                       // groups per wave
  constexpr int NG = kFdThreads / LPP;              // groups per block
  constexpr int PPP = NG;                             // positions per pass
  __shared__ float gm[NG][REP], gl[NG][REP];
  __shared__ __align__(16) float go[NG][REP][HD];
  __shared__ float wgt[REP][kFdMaxSplits > NG ? kFdMaxSplits : NG];
  __shared__ float lsp[REP][kFdMaxSplits];
  __shared__ float tot[REP];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = p.n_split;
  const int g = blockIdx.x / S, sp = blockIdx.x - g * S;
  const int li = lane % LPP, grp = wave * PPW + lane / LPP;
  const size_t cache0 = (size_t)g * p.max_ctx * HD;
  const int qstride = p.gated ? 2 * HD : HD;
  const int half = p.rope_n / 2;

  // 1. The prologue's inputs first, none of which depends on the position, so they are in flight
  //    while the position is read, and a later wait for them does not cover the K/V stream.
  const float* kraw = p.qkv + (size_t)p.n_head * qstride + (size_t)g * HD;
  constexpr int NST = REP + 4, STV = NST * HD / 4;                 // rows, float4s staged
  constexpr int SPT = (STV + kFdThreads - 1) / kFdThreads;     // float4s per thread
  __shared__ __align__(16) float stg[NST][HD];
  // QP: thread t holds float4 e = t + 256 k of the REP + 2 rows (q heads, k, v), RW threads a row
  // (a row never straddles a wave): every slice's partial of it and its norm gain.
  constexpr int RW = HD / 4, NQE = (REP + 2) * RW;
  constexpr int SPQ = (NQE + kFdThreads - 1) / kFdThreads;
  constexpr int NPS = QP ? QPS : 1;
  // With QP the control words are read first: scalar loads, which the memory barrier below would
  // otherwise turn into vector loads queued behind the partial sums.
  const int pos_qp = QP ? p.pos[0] : 0, slot_qp = QP ? p.pos[5] : 0, T_qp = QP ? p.pos[6] : 0;
  float4 sv[QP ? SPQ : SPT];
  float4 pv[QP ? SPQ : 1][NPS];
  float ssl = 0.f;
  if constexpr (QP) {
    constexpr uint32_t kOutQ = 0x40000000u;        // a buffer offset past every buffer
    const __amdgpu_buffer_rsrc_t rqp = make_rsrc(p.qkv_part, (uint32_t)((size_t)p.qkv_S * p.qkv_rows_p * 4));
#pragma unroll
    for (int k = 0; k < SPQ; ++k) {
      const int e = tid + k * kFdThreads, row = e / RW, d = 4 * (e - row * RW);
      const uint32_t qi = row < REP ? (uint32_t)((g * REP + row) * HD + d)
                          : (uint32_t)(p.n_head * HD + ((row - REP) * p.n_kv + g) * HD + d);
      // Past the rows: an offset past the buffer (zeros, no memory access); past S a repeat of
      // the last slice that gets no weight.
      const uint32_t off0 = e < NQE ? qi * 4u : kOutQ;
#pragma unroll
      for (int q = 0; q < NPS; ++q) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(
            rqp, off0 + (uint32_t)min(q, p.qkv_S - 1) * (uint32_t)p.qkv_rows_p * 4u, 0, 0);
        pv[k][q] = make_float4(__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]));
      }
      sv[k] = *(const float4*)((row == REP ? p.k_norm : p.q_norm) + (e < NQE ? d : 0));
    }
    // Lane i holds slice i's sum of squares (a vector load: counted with the partials, not the
    // position; past S the buffer's range check gives 0).
    ssl = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
              make_rsrc(p.qkv_ss, (uint32_t)p.qkv_S * 4u), (uint32_t)lane * 4u, 0, 0));
    // Keeps these loads ahead of the position's and the K/V rows' (the scheduler would otherwise
    // issue them after the K/V stream, and the scalar ones after its waits).
    asm volatile("" ::: "memory");
  } else {
    // The q heads, the new k and v and the two norm gains, loaded once by the block (every
    // position group uses the same values).
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int e = min(tid + k * kFdThreads, STV - 1);            // past the end: a repeat
      const int row = 4 * e / HD, d = 4 * e - row * HD;
      const float* src = row < REP ? p.qkv + (size_t)(g * REP + row) * qstride + d
                         : row == REP ? kraw + d
                         : row == REP + 1 ? kraw + (size_t)p.n_kv * HD + d
                         : row == REP + 2 ? p.q_norm + d : p.k_norm + d;
      sv[k] = *(const float4*)src;
    }
  }

  // The position (for RoPE), the KV slot its k and v go to and the T slots attended: the slot is
  // the position and T = pos + 1 inside the window, the KV ring's past it.
  const int pos = QP ? pos_qp : p.pos[0], slot = QP ? slot_qp : p.pos[5], T = QP ? T_qp : p.pos[6];
  const int rrow = min(pos, p.max_ctx);               // the fp32 table's row of the position
  const int chunk = (T + S - 1) / S;
  const int p0 = sp * chunk, p1 = min(T, p0 + chunk), n = max(0, p1 - p0);
  const bool owner = n > 0 && slot >= p0 && slot < p1;
  const int npass = (n + PPP - 1) / PPP;

  // The RoPE cos/sin at pos, from the model's table (fp32, or the image's Q14 rows), loaded
  // before the K/V rows: QP, of this thread's four elements (d .. d + 3, one side of the
  // rotation); otherwise of this lane's elements (d = lane + 64 i) when a wave holds a vector.
  constexpr int EPL = HD / 64;
  constexpr int NRC = QP ? 4 * SPQ : EPL;
  float rc[NRC], rsn[NRC];
#pragma unroll
  for (int i = 0; i < NRC; ++i) {
    const int d = QP ? 4 * ((tid + (i / 4) * kFdThreads) % RW) + (i % 4) : lane + 64 * i;
    const int ri = d < half ? d : d - half;
    rc[i] = 1.f;
    rsn[i] = 0.f;
    if (d < 2 * half) {
      if (p.rope_tab) {
        rc[i] = (float)p.rope_tab[(size_t)pos * p.rope_n + ri] * (1.0f / 16384.0f);
        rsn[i] = (float)p.rope_tab[(size_t)pos * p.rope_n + half + ri] * (1.0f / 16384.0f);
      } else {
        rc[i] = p.rope_cs[(size_t)rrow * p.rope_n + ri];
        rsn[i] = p.rope_cs[(size_t)rrow * p.rope_n + half + ri];
      }
    }
  }

  // 2. The split's K and V rows (the new position's come from the projection above).
  //    Every pass issues its loads: a position outside the split (or the new one) gets an offset
  //    past the buffer, which the range check turns into zeros without a memory access. With no
  //    branch around them the compiler's wait for the prologue's inputs counts these loads
  //    exactly (after a conditional load it would also wait for some of them).
  constexpr uint32_t kOut = 0x40000000u;
  const uint32_t head_bytes = (uint32_t)p.max_ctx * HD * 2u;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.kcache + cache0, head_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.vcache + cache0, head_bytes);
  uint4 kr[kMaxPass], vr[kMaxPass];
#pragma unroll
  for (int ps = 0; ps < kMaxPass; ++ps) {
    const int t = ps * PPP + grp;
    const bool ok = ps < npass && t < n && p0 + t != slot;
    const uint32_t off = ok ? ((uint32_t)(p0 + t) * HD + li * 8) * 2u : kOut;
    const auto a = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
    const auto b = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
    kr[ps] = make_uint4(a[0], a[1], a[2], a[3]);
    vr[ps] = make_uint4(b[0], b[1], b[2], b[3]);
  }

  const float qpost = 1.0f / sqrtf((float)HD);
  if constexpr (QP) {
    // The slices added in slice order, times the q|k|v GEMV's RMSNorm scale; then each q head
    // and k RMS-normalised over its row's RW threads (DPP and lane swaps), times its gain, and
    // rotated with the partner element d +- half from the thread half / 4 lanes away; q scaled by
    // 1/sqrt(hd); k and v rounded to fp16 (the cache's values, which the score of this position
    // uses too) and stored to the cache by the block that holds the position. No LDS round trip
    // and no barrier before the rows go to stg.
    const float rs = 1.0f / sqrtf(wave_sum_dpp(ssl) / (float)p.qkv_K + p.eps);
#pragma unroll
    for (int k = 0; k < SPQ; ++k) {
      const int e = tid + k * kFdThreads, row = e / RW, d = 4 * (e - row * RW);
      float4 a = pv[k][0];
#pragma unroll
      for (int q = 1; q < NPS; ++q)
        if (q < p.qkv_S) { a.x += pv[k][q].x; a.y += pv[k][q].y; a.z += pv[k][q].z; a.w += pv[k][q].w; }
      const float x[4] = {a.x * rs, a.y * rs, a.z * rs, a.w * rs};
      // The first split block of each kv head keeps its q, k and v rows in p.qkv, as the GEMV
      // would have stored them (the q|k|v tap of the last attention layer).
      if (sp == 0 && e < NQE) {
        const size_t qi = row < REP ? (size_t)(g * REP + row) * HD + d
                          : (size_t)p.n_head * HD + (size_t)((row - REP) * p.n_kv + g) * HD + d;
        *(float4*)(p.qkv + qi) = make_float4(x[0], x[1], x[2], x[3]);
      }
      float ss = (x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]);
      ss = row16_sum(ss);
      if (RW >= 32) ss += __shfl_xor(ss, 16, 64);
      if (RW >= 64) ss += __shfl_xor(ss, 32, 64);
      const float r = rsqrtf(ss / (float)HD + p.eps);
      const float gw[4] = {sv[k].x, sv[k].y, sv[k].z, sv[k].w};
      float xn[4], pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xn[i] = x[i] * r * gw[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = __shfl_xor(xn[i], half / 4, 64);
      if (e < NQE) {
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float c = rc[4 * k + i], sn = rsn[4 * k + i];
          y[i] = d < half ? xn[i] * c - pr[i] * sn : d < 2 * half ? pr[i] * sn + xn[i] * c : xn[i];
        }
        if (row < REP) {
          *(float4*)&stg[row][d] = make_float4(y[0] * qpost, y[1] * qpost, y[2] * qpost, y[3] * qpost);
        } else {
          // k (normalised, rotated) or v (as it came).
          const float* src = row == REP ? y : x;
          __half h[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) h[i] = __float2half(src[i]);
          *(float4*)&stg[row][d] = make_float4(__half2float(h[0]), __half2float(h[1]), __half2float(h[2]), __half2float(h[3]));
          if (owner) {
            __half* dst = (row == REP ? p.kcache : p.vcache) + cache0 + (size_t)slot * HD + d;
            *(uint2*)dst = make_uint2(__builtin_bit_cast(uint32_t, __halves2half2(h[0], h[1])),
                                      __builtin_bit_cast(uint32_t, __halves2half2(h[2], h[3])));
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int e = min(tid + k * kFdThreads, STV - 1);
      *(float4*)(&stg[0][0] + 4 * e) = sv[k];
    }
  }
  float q[REP][8], kn[8], vn[8];
  if (n > 0) {
    __syncthreads();
    if constexpr (!QP) {
      // The q heads and the new k normalised and rotated once per block: wave w takes vectors w,
      // w + 4, ... (lane l holds elements l + 64 i). The rotation partner (d +- half) is read back
      // from nrm, which only this wave writes for its vector. q is scaled by 1/sqrt(hd); k and v
      // are rounded to fp16 (the cache's values, which the score of this position uses too) and
      // stored to the cache by the block that holds the position.
      __shared__ float nrm[REP + 1][HD];
      for (int v = wave; v <= REP; v += kFdThreads / 64) {
        const float* gw = stg[v < REP ? REP + 2 : REP + 3];
        float x[EPL], ss = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          x[i] = stg[v][lane + 64 * i];
          ss += x[i] * x[i];
        }
        const float r = rsqrtf(wave_sum_dpp(ss) / (float)HD + p.eps);
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          x[i] = x[i] * r * gw[lane + 64 * i];
          nrm[v][lane + 64 * i] = x[i];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's stores before its reads
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          const int d = lane + 64 * i;
          float y = x[i];
          if (d < half) y = x[i] * rc[i] - nrm[v][d + half] * rsn[i];
          else if (d < 2 * half) y = nrm[v][d - half] * rsn[i] + x[i] * rc[i];
          if (v < REP) {
            stg[v][d] = y * qpost;
          } else {
            const __half kh = __float2half(y), vh = __float2half(stg[REP + 1][d]);
            stg[REP][d] = __half2float(kh);
            stg[REP + 1][d] = __half2float(vh);
            if (owner) {
              p.kcache[cache0 + (size_t)slot * HD + d] = kh;
              p.vcache[cache0 + (size_t)slot * HD + d] = vh;
            }
          }
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma unroll
      for (int j = 0; j < REP; ++j) q[j][k] = stg[j][li * 8 + k];
      kn[k] = stg[REP][li * 8 + k];
      vn[k] = stg[REP + 1][li * 8 + k];
    }

    // 3. This group's positions: every score, then the softmax pieces (max, sum, weighted V).
    float sc[kMaxPass][REP];
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ++ps) {
#pragma unroll
      for (int j = 0; j < REP; ++j) sc[ps][j] = -INFINITY;
      if (ps >= npass) continue;
      const int t = ps * PPP + grp;
      float kv[8];
      if (owner && p0 + t == slot) {
#pragma unroll
        for (int k = 0; k < 8; ++k) kv[k] = kn[k];
      } else {
        h8_to_f(kr[ps], kv);
      }
#pragma unroll
      for (int j = 0; j < REP; ++j) {
        float d = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) d += q[j][k] * kv[k];
        d = group_sum<LPP>(d);
        if (t < n) sc[ps][j] = d;
      }
    }
    float m[REP], l[REP], acc[REP][8];
#pragma unroll
    for (int j = 0; j < REP; ++j) {
      m[j] = -INFINITY;
#pragma unroll
      for (int ps = 0; ps < kMaxPass; ++ps) m[j] = fmaxf(m[j], sc[ps][j]);
      l[j] = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[j][k] = 0.f;
    }
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ++ps) {
      if (ps >= npass) break;
      const int t = ps * PPP + grp;
      if (t >= n) continue;
      float vv[8];
      if (owner && p0 + t == slot) {
#pragma unroll
        for (int k = 0; k < 8; ++k) vv[k] = vn[k];
      } else {
        h8_to_f(vr[ps], vv);
      }
#pragma unroll
      for (int j = 0; j < REP; ++j) {
        const float e = __expf(sc[ps][j] - m[j]);
        l[j] += e;
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[j][k] += e * vv[k];
      }
    }

    // 4. The block's groups combined into the split's partial.
#pragma unroll
    for (int j = 0; j < REP; ++j) {
      if (li == 0) { gm[grp][j] = m[j]; gl[grp][j] = l[j]; }
#pragma unroll
      for (int k = 0; k < 8; ++k) go[grp][j][li * 8 + k] = acc[j][k];
    }
    __syncthreads();
    // Wave w combines q heads w, w + 4, ...: lane i holds group i's (max, sum) of the head.
    static_assert(NG <= 64, "one lane per group");
    for (int j = wave; j < REP; j += kFdThreads / 64) {
      const float gmv = lane < NG ? gm[lane][j] : -INFINITY;
      const float glv = lane < NG ? gl[lane][j] : 0.f;
      const float M = wave_max(gmv);
      const float w = glv > 0.f ? __expf(gmv - M) : 0.f;
      if (lane < NG) wgt[j][lane] = w;
      const float L = wave_sum(glv * w);
      if (lane == 0) {
        // Agent-scope stores when the last split block of this launch merges them; plain stores
        // when the next kernel does (the launch's end makes them visible).
        float* pm = p.part_m + (size_t)(g * REP + j) * S + sp;
        float* pl = p.part_l + (size_t)(g * REP + j) * S + sp;
        if (p.done) {
          st_vec<true>(pm, M);
          st_vec<true>(pl, L);
        } else {
          *pm = M;
          *pl = L;
        }
      }
    }
    __syncthreads();
    for (int i = tid; i < REP * HD; i += kFdThreads) {
      const int j = i / HD, d = i - j * HD;
      float o = 0.f;
#pragma unroll
      for (int k = 0; k < NG; ++k) o += go[k][j][d] * wgt[j][k];
      float* po = p.part_o + ((size_t)(g * REP + j) * S + sp) * HD + d;
      if (p.done) st_vec<true>(po, o);
      else *po = o;
    }
  }

  // 5. The last of kv head g's S blocks merges its splits (the others are done, their partials
  //    written by agent-scope stores that completed before they counted themselves). Without
  //    counters the next kernel merges (the packed o projection, trx_tgemv.hip).
  if (!p.done) return;
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(p.done + g * kDoneStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == (unsigned)(S - 1);
    if (last) __hip_atomic_store(p.done + g * kDoneStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  // Agent-scope (sc1) buffer loads: plain loads could hit stale lines of this XCD's L2, and
  // atomic loads would be issued one at a time.
  const int ns = min(S, (T + chunk - 1) / chunk);     // splits holding positions
  const uint32_t nb = (uint32_t)((size_t)p.n_head * S * 4);
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(p.part_m, nb), rl = make_rsrc(p.part_l, nb);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.part_o, nb * (uint32_t)HD);
  for (int i = tid; i < REP * ns; i += kFdThreads) {
    const int j = i / ns, k = i - j * ns;
    const uint32_t off = (uint32_t)(((g * REP + j) * S + k) * 4);
    wgt[j][k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, off, 0, kCpolSc1));
    lsp[j][k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, off, 0, kCpolSc1));
  }
  __syncthreads();
  if (tid < REP) {
    float M = -INFINITY;
    for (int i = 0; i < ns; ++i) M = fmaxf(M, wgt[tid][i]);
    float L = 0.f;
    for (int i = 0; i < ns; ++i) {
      const float w = __expf(wgt[tid][i] - M);
      wgt[tid][i] = w;
      L += lsp[tid][i] * w;
    }
    tot[tid] = L;
  }
  __syncthreads();
  for (int i = tid; i < REP * HD; i += kFdThreads) {
    const int j = i / HD, d = i - j * HD, qh = g * REP + j;
    const uint32_t base = (uint32_t)(((size_t)qh * S * HD + d) * 4), step = (uint32_t)HD * 4u;
    float o = 0.f;
    for (int s0 = 0; s0 < ns; s0 += 32) {
      float v[32];
#pragma unroll
      for (int k = 0; k < 32; ++k)       // past ns: reads of the buffer that get weight 0
        v[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ro, base + min(s0 + k, ns - 1) * step, 0, kCpolSc1));
#pragma unroll
      for (int k = 0; k < 32; ++k) o += s0 + k < ns ? v[k] * wgt[j][s0 + k] : 0.f;
    }
    o /= tot[j];
    if (p.gated) o *= sigmoidf_(p.qkv[(size_t)qh * 2 * HD + HD + d]);
    p.out[(size_t)qh * HD + d] = o;
  }
}

bool attention_qp_supported(int hd, int rope_n) {
  // The partial-sum prologue swaps a thread's four elements with the thread half / 4 lanes away.
  const int half = rope_n / 2, q = half / 4;
  return half >= 4 && half % 4 == 0 && (q & (q - 1)) == 0 && 2 * half <= hd;
}

bool attention_fd_supported(int rep, int hd, int rope_n, int n_split) {
  const int half = rope_n / 2;
  const bool rope_ok = half >= 1 && 2 * half <= hd;
  const bool rep_ok = rep == 1 || rep == 2 || rep == 4 || rep == 6 || rep == 8;
  return rope_ok && rep_ok && (hd == 64 || hd == 128 || hd == 256) && n_split <= kFdMaxSplits;
}

template <int REP, int QPS>
static int launch_fd_qp(const AttnParams& p, hipStream_t s) {
  const dim3 grid(p.n_kv * p.n_split), block(kFdThreads);
  switch (p.hd) {
    case 64: hipLaunchKernelGGL((attn_fd_kernel<REP, 64, QPS>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((attn_fd_kernel<REP, 128, QPS>), grid, block, 0, s, p); break;
    case 256: hipLaunchKernelGGL((attn_fd_kernel<REP, 256, QPS>), grid, block, 0, s, p); break;
    default: TRX_CHECK(false, TRX_E_INVALID, "attention: head_dim %d unsupported", p.hd);
  }
  TRX_LAUNCHED();
  return TRX_OK;
}

template <int REP>
static int launch_fd_rep(const AttnParams& p, hipStream_t s) {
  if (!p.qkv_part) return launch_fd_qp<REP, 0>(p, s);
  static_assert(kQkvPartMax == 16, "the partial-sum prologue takes 8 or 16 slices");
  return p.qkv_S <= 8 ? launch_fd_qp<REP, 8>(p, s) : launch_fd_qp<REP, 16>(p, s);
}

int launch_attention_fd(const AttnParams& p, hipStream_t s) {
  TRX_CHECK(attention_fd_supported(p.n_rep, p.hd, p.rope_n, p.n_split), TRX_E_INVALID,
            "attention: rep %d hd %d rope %d splits %d unsupported", p.n_rep, p.hd, p.rope_n, p.n_split);
  TRX_CHECK(!p.qkv_part || (p.qkv_ss && !p.gated && attention_qp_supported(p.hd, p.rope_n) && p.qkv_S >= 1 && p.qkv_S <= kQkvPartMax &&
                            p.qkv_rows_p % 4 == 0 && p.qkv_K > 0 &&
                            p.qkv_rows_p >= (p.n_head + 2 * p.n_kv) * p.hd),
            TRX_E_INVALID, "attention: unsupported q|k|v partial sums (S %d, rows %d)", p.qkv_S, p.qkv_rows_p);
  const int cap = attention_max_chunk(p.hd);
  TRX_CHECK(p.n_split >= 1 && (p.max_ctx + p.n_split - 1) / p.n_split <= cap, TRX_E_INVALID,
            "attention: %d splits for context %d", p.n_split, p.max_ctx);
  switch (p.n_rep) {
    case 1: return launch_fd_rep<1>(p, s);
    case 2: return launch_fd_rep<2>(p, s);
    case 4: return launch_fd_rep<4>(p, s);
    case 6: return launch_fd_rep<6>(p, s);
    case 8: return launch_fd_rep<8>(p, s);
  }
  return TRX_E_INVALID;
}

}  // namespace trx
