// Gated DeltaNet decode step for the hybrid models (one position per call). The rule is
// model/fastref.py:182-214 (= model/golden.py:400-434 with the grouped output order):
//   conv  = causal depthwise conv over the window [state (K-1 rows, oldest first) | qkv], SiLU
//   q, k  = L2-normalised per key head; v per value head (value head h uses key head h % nk)
//   M_h  *= exp(softplus(alpha_h + dt_h) * A_h);  delta = (v - M_h k) * sigmoid(beta_h)
//   M_h  += delta (x) k;  o_h = (M_h q) / sqrt(hk)
//   out[gpos(h)] = rmsnorm(o_h) * w * silu(z_h),   gpos = (h % nk) * (nv / nk) + h / nk

#include "trx_internal.h"
#include "trx_ops.h"
#include "trx_dense_dev.h"

namespace trx {

// Conv of one head-sized segment of the qkv channels (q heads, then k heads, then v heads): thread
// t < hk takes channel seg * hk + t; every thread of the block (blockDim >= hk, a multiple of 64)
// calls this, the ones past hk only for the L2 norm's barrier.
// [qkv | z] value i from the GEMV's K-slice partial sums: r * the slices' sum in slice order.
__device__ __forceinline__ float dn_part_value(const DnConvParams& p, int i) {
  float ss = 0.f;
  for (int k = 0; k < p.S; ++k) ss += p.part_ss[k];
  const float r = 1.0f / sqrtf(ss / (float)p.K + p.rms_eps);
  float v[kDnPartMax];
#pragma unroll
  for (int k = 0; k < kDnPartMax; ++k) v[k] = k < p.S ? p.part[(size_t)k * p.rows_p + i] : 0.f;
  float a = v[0];
#pragma unroll
  for (int k = 1; k < kDnPartMax; ++k)
    if (k < p.S) a += v[k];
  return a * r;
}

__device__ __forceinline__ void dn_conv_seg(const DnConvParams& p, int seg, int t, float* red) {
  const bool on = t < p.hk;
  const int c = seg * p.hk + (on ? t : 0);
  float y = 0.f;
  if (on) {
    const float x = p.part ? dn_part_value(p, c) : p.qkv[c];
    float acc = 0.f;
    for (int i = 0; i < p.Kc - 1; ++i) acc += p.taps[c * p.Kc + i] * p.state[(size_t)i * p.C + c];
    acc += p.taps[c * p.Kc + p.Kc - 1] * x;
    for (int i = 0; i + 1 < p.Kc - 1; ++i) p.state[(size_t)i * p.C + c] = p.state[(size_t)(i + 1) * p.C + c];
    if (p.Kc > 1) p.state[(size_t)(p.Kc - 2) * p.C + c] = x;
    y = silu(acc);
  }
  if (seg * p.hk < 2 * p.nq) {
    // L2 norm over the key/query head (x / max(|x|, eps), fastref.py:146-148).
    float ss = wave_sum(y * y);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < (int)(blockDim.x + 63) / 64; ++i) tot += red[i];
    y = y / fmaxf(sqrtf(tot), p.eps);
  }
  if (on) p.out[c] = y;
}

// One block per head-sized segment of the qkv channels.
__global__ void dn_conv_kernel(DnConvParams p) {
  extern __shared__ float red[];
  dn_conv_seg(p, blockIdx.x, threadIdx.x, red);
}

// The conv segments and the beta/alpha rows in one launch (both read only the [qkv|z] GEMV's
// output and the residual): blocks below n_seg take a conv segment, the next dp.M a Q8 row each;
// with partial sums (cp.part) the last blocks reduce the z rows, 256 values each.
__global__ __launch_bounds__(256) void dn_conv_q8_kernel(DnConvParams cp, DenseParams dp, int n_seg) {
  __shared__ float red[2][4];
  const int b = blockIdx.x;
  if (b < n_seg) {
    dn_conv_seg(cp, b, threadIdx.x, red[0]);
  } else if (b < n_seg + dp.M) {
    q8_row_dot(dp, b - n_seg, threadIdx.x, red);
  } else {
    const int i = (b - n_seg - dp.M) * 256 + (int)threadIdx.x;
    if (i < cp.nz) cp.qkv[cp.C + i] = dn_part_value(cp, cp.C + i);
  }
}

// One block per value head; threads split the head's rows (hv) and columns (hk).
__global__ __launch_bounds__(256) void dn_recur_kernel(DnRecurParams p) {
  __shared__ float kq[2][512];
  __shared__ float o_s[512];
  __shared__ float red[8];
  const int h = blockIdx.x, t = threadIdx.x;
  const int nk = p.nk, hk = p.hk, hv = p.hv, nq = nk * hk;
  const int kh = h % nk;
  for (int i = t; i < hk; i += 256) {
    kq[0][i] = p.conv[nq + kh * hk + i];   // k
    kq[1][i] = p.conv[kh * hk + i];        // q
  }
  __syncthreads();
  const float a = p.ba[p.nv + h] + p.dt[h];
  const float sp = a > 20.f ? a : log1pf(expf(a));
  const float decay = expf(sp * p.A[h]);
  const float beta = sigmoidf_(p.ba[h]);
  const int tpr = 256 / hv;                  // threads per row
  const int cpt = hk / tpr;                  // columns per thread
  const int j = t / tpr, part = t - j * tpr;
  float* Srow = p.S + ((size_t)h * hv + j) * hk + part * cpt;
  // The row slice stays in registers: the loops are unrolled to the 64-column maximum and
  // predicated on cpt, so the array is never indexed dynamically.
  float s[64];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    if (i < cpt) {
      s[i] = Srow[i] * decay;
      dot += s[i] * kq[0][part * cpt + i];
    }
  }
  for (int o = tpr >> 1; o >= 1; o >>= 1) dot += __shfl_xor(dot, o, 64);
  const float delta = (p.conv[2 * nq + h * hv + j] - dot) * beta;
  float oq = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    if (i < cpt) {
      s[i] += delta * kq[0][part * cpt + i];
      Srow[i] = s[i];
      oq += s[i] * kq[1][part * cpt + i];
    }
  }
  for (int o = tpr >> 1; o >= 1; o >>= 1) oq += __shfl_xor(oq, o, 64);
  const float ov = oq * (1.0f / sqrtf((float)hk));
  if (part == 0) o_s[j] = ov;
  __syncthreads();
  // Gated RMSNorm over the head, then the grouped output position.
  float ss = 0.f;
  for (int i = t; i < hv; i += 256) ss += o_s[i] * o_s[i];
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)hv + p.eps);
  const int rep = p.nv / nk;
  const int gpos = kh * rep + h / nk;
  for (int i = t; i < hv; i += 256)
    p.out[(size_t)gpos * hv + i] = o_s[i] * r * p.norm_w[i] * silu(p.z[(size_t)h * hv + i]);
}

// The same recurrence for head geometries known at compile time: a row's HK columns across HK/4
// lanes (one float4 each), 64/(HK/4) rows per wave pass, so a load instruction covers whole
// consecutive rows; each thread keeps its HV/(4*rows per pass) float4 of the state in registers.
// Row sums (S k and S q) by shuffles within the row's lanes. NW waves per head: more state
// loads in flight per CU (the grid has only one block per value head).
template <int HK, int HV, int NW>
__global__ __launch_bounds__(NW * 64) void dn_recur_fixed_kernel(DnRecurParams p) {
  constexpr int LPR = HK / 4, RPP = 64 / LPR, NIT = HV / (NW * RPP);
  static_assert(HK % 4 == 0 && 64 % LPR == 0 && NIT >= 1 && HV % (NW * RPP) == 0, "head geometry");
  __shared__ float o_s[HV];
  __shared__ float red[NW];
  const int h = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int sub = lane / LPR, c4 = lane % LPR;
  const int nk = p.nk, nq = nk * HK, kh = h % nk;
  const float4 k4 = *(const float4*)(p.conv + nq + kh * HK + 4 * c4);
  const float4 q4 = *(const float4*)(p.conv + kh * HK + 4 * c4);
  float4* S = (float4*)(p.S + (size_t)h * HV * HK);
  float4 sv[NIT];
  float vj[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int j = (it * NW + w) * RPP + sub;
    sv[it] = S[j * LPR + c4];
    vj[it] = p.conv[2 * nq + h * HV + j];
  }
  const float a = p.ba[p.nv + h] + p.dt[h];
  const float sp = a > 20.f ? a : log1pf(expf(a));
  const float decay = expf(sp * p.A[h]);
  const float beta = sigmoidf_(p.ba[h]);
  const float qs = 1.0f / sqrtf((float)HK);
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int j = (it * NW + w) * RPP + sub;
    float4 s4 = make_float4(sv[it].x * decay, sv[it].y * decay, sv[it].z * decay, sv[it].w * decay);
    float dot = (s4.x * k4.x + s4.y * k4.y) + (s4.z * k4.z + s4.w * k4.w);
#pragma unroll
    for (int o = LPR >> 1; o >= 1; o >>= 1) dot += __shfl_xor(dot, o, 64);
    const float delta = (vj[it] - dot) * beta;
    s4 = make_float4(s4.x + delta * k4.x, s4.y + delta * k4.y, s4.z + delta * k4.z, s4.w + delta * k4.w);
    S[j * LPR + c4] = s4;
    float oq = (s4.x * q4.x + s4.y * q4.y) + (s4.z * q4.z + s4.w * q4.w);
#pragma unroll
    for (int o = LPR >> 1; o >= 1; o >>= 1) oq += __shfl_xor(oq, o, 64);
    if (c4 == 0) o_s[j] = oq * qs;
  }
  __syncthreads();
  // Gated RMSNorm over the head, then the grouped output position.
  float ss = 0.f;
  for (int i = t; i < HV; i += NW * 64) ss += o_s[i] * o_s[i];
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)HV + p.eps);
  const int gpos = kh * (p.nv / nk) + h / nk;
  for (int i = t; i < HV; i += NW * 64)
    p.out[(size_t)gpos * HV + i] = o_s[i] * r * p.norm_w[i] * silu(p.z[(size_t)h * HV + i]);
}

int launch_dn_conv(const DnConvParams& p, hipStream_t s) {
  TRX_CHECK(p.hk <= 256 && p.C % p.hk == 0, TRX_E_INVALID, "deltanet conv: head dim %d", p.hk);
  hipLaunchKernelGGL(dn_conv_kernel, dim3(p.C / p.hk), dim3(p.hk), 8 * sizeof(float), s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_dn_conv_q8(const DnConvParams& cp, const DenseParams& dp, hipStream_t s) {
  TRX_CHECK(cp.hk <= 256 && cp.C % cp.hk == 0 && dp.kind == TRX_KIND_Q8 && !dp.amax_slot && !dp.gate_pos &&
            dp.K % 32 == 0 && dp.code_off % 16 == 0 && dp.row_bytes % 16 == 0 &&
            ((uintptr_t)dp.W | (uintptr_t)dp.x | (uintptr_t)dp.norm_w) % 16 == 0,
            TRX_E_INVALID, "deltanet conv + beta/alpha: unsupported geometry");
  TRX_CHECK(!cp.part || (cp.part_ss && cp.S >= 1 && cp.S <= kDnPartMax && cp.rows_p >= cp.C + cp.nz && cp.K > 0),
            TRX_E_INVALID, "deltanet conv: partial sums of %d slices unsupported", cp.S);
  const int n_seg = cp.C / cp.hk, n_z = cp.part ? cdiv(cp.nz, 256) : 0;
  hipLaunchKernelGGL(dn_conv_q8_kernel, dim3(n_seg + dp.M + n_z), dim3(256), 0, s, cp, dp, n_seg);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_dn_recur(const DnRecurParams& p, hipStream_t s) {
  TRX_CHECK(p.hv <= 256 && 256 % p.hv == 0 && p.hk % (256 / p.hv) == 0 && p.hk / (256 / p.hv) <= 64 &&
            p.hk <= 512 && p.hv <= 512 && p.nv % p.nk == 0, TRX_E_INVALID,
            "deltanet recurrence: unsupported head geometry hk=%d hv=%d", p.hk, p.hv);
  const bool aligned = ((uintptr_t)p.S | (uintptr_t)p.conv) % 16 == 0 && (p.nk * p.hk) % 4 == 0;
  if (aligned && p.hk == 128 && p.hv == 128)
    hipLaunchKernelGGL((dn_recur_fixed_kernel<128, 128, 16>), dim3(p.nv), dim3(1024), 0, s, p);
  else if (aligned && p.hk == 64 && p.hv == 64)
    hipLaunchKernelGGL((dn_recur_fixed_kernel<64, 64, 16>), dim3(p.nv), dim3(1024), 0, s, p);
  else
    hipLaunchKernelGGL(dn_recur_kernel, dim3(p.nv), dim3(256), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

}  // namespace trx
