// Gated DeltaNet decode step for the hybrid models (one position per call). The rule is
// model/fastref.py:182-214 (= model/golden.py:400-434 with the grouped output order):
//   conv  = causal depthwise conv over the window [state (K-1 rows, oldest first) | qkv], SiLU
//   q, k  = L2-normalised per key head; v per value head (value head h uses key head h % nk)
//   M_h  *= exp(softplus(alpha_h + dt_h) * A_h);  delta = (v - M_h k) * sigmoid(beta_h)
//   M_h  += delta (x) k;  o_h = (M_h q) / sqrt(hk)
//   out[gpos(h)] = rmsnorm(o_h) * w * silu(z_h),   gpos = (h % nk) * (nv / nk) + h / nk

#include "trx_internal.h"
#include "trx_ops.h"

namespace trx {

// One block per head-sized segment of the qkv channels (q heads, then k heads, then v heads).
__global__ void dn_conv_kernel(DnConvParams p) {
  extern __shared__ float red[];
  const int seg = blockIdx.x, t = threadIdx.x;
  const int c = seg * p.hk + t;
  const float x = p.qkv[c];
  float acc = 0.f;
  for (int i = 0; i < p.Kc - 1; ++i) acc += p.taps[c * p.Kc + i] * p.state[(size_t)i * p.C + c];
  acc += p.taps[c * p.Kc + p.Kc - 1] * x;
  for (int i = 0; i + 1 < p.Kc - 1; ++i) p.state[(size_t)i * p.C + c] = p.state[(size_t)(i + 1) * p.C + c];
  if (p.Kc > 1) p.state[(size_t)(p.Kc - 2) * p.C + c] = x;
  float y = silu(acc);
  if (c < 2 * p.nq) {
    // L2 norm over the key/query head (x / max(|x|, eps), fastref.py:146-148).
    float ss = wave_sum(y * y);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < (blockDim.x + 63) / 64; ++i) tot += red[i];
    y = y / fmaxf(sqrtf(tot), p.eps);
  }
  p.out[c] = y;
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

int launch_dn_conv(const DnConvParams& p, hipStream_t s) {
  TRX_CHECK(p.hk <= 256 && p.C % p.hk == 0, TRX_E_INVALID, "deltanet conv: head dim %d", p.hk);
  hipLaunchKernelGGL(dn_conv_kernel, dim3(p.C / p.hk), dim3(p.hk), 8 * sizeof(float), s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

int launch_dn_recur(const DnRecurParams& p, hipStream_t s) {
  TRX_CHECK(p.hv <= 256 && 256 % p.hv == 0 && p.hk % (256 / p.hv) == 0 && p.hk / (256 / p.hv) <= 64 &&
            p.hk <= 512 && p.hv <= 512 && p.nv % p.nk == 0, TRX_E_INVALID,
            "deltanet recurrence: unsupported head geometry hk=%d hv=%d", p.hk, p.hv);
  hipLaunchKernelGGL(dn_recur_kernel, dim3(p.nv), dim3(256), 0, s, p);
  TRX_LAUNCHED();
  return TRX_OK;
}

}  // namespace trx
