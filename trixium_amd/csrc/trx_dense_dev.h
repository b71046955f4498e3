// Device body of the Q8 row dot product (one 256-thread block per output row), shared by the
// dense GEMV launch and the DeltaNet conv + beta/alpha launch.
#pragma once

#include "trx_internal.h"
#include "trx_ops.h"

namespace trx {

// y[m] = (W_m . (x * norm_w)) / rms(x) (without norm_w: W_m . x), sigmoid if asked. W row m: fp16
// scales of its 32-wide groups at the row's start, int8 codes at code_off; each product is the
// fp16-rounded dequantised weight times x. Every thread of the 256-thread block calls this.
__device__ __forceinline__ void q8_row_dot(const DenseParams& p, int m, int t, float (*red)[4]) {
  const int lane = t & 63, w = t >> 6;
  const uint8_t* row = p.W + (size_t)m * p.row_bytes;
  const uint16_t* sc = (const uint16_t*)row;
  const int8_t* q = (const int8_t*)(row + p.code_off);
  float acc = 0.f, ss = 0.f;
  for (int g = t; g < p.K / 32; g += 256) {
    const int4 c4[2] = {*(const int4*)(q + 32 * g), *(const int4*)(q + 32 * g + 16)};
    const float s = __half2float(__ushort_as_half(sc[g]));
    const float4* xv = (const float4*)(p.x + 32 * g);
    const float4* gv = p.norm_w ? (const float4*)(p.norm_w + 32 * g) : nullptr;
    const int8_t* cb = (const int8_t*)c4;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 x4 = xv[k];
      const float4 g4 = gv ? gv[k] : make_float4(1.f, 1.f, 1.f, 1.f);
      const float xs[4] = {x4.x, x4.y, x4.z, x4.w}, gs[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ss += xs[i] * xs[i];
        acc += __half2float(__float2half((float)cb[4 * k + i] * s)) * (xs[i] * gs[i]);
      }
    }
  }
  acc = wave_sum(acc);
  ss = wave_sum(ss);
  if (lane == 0) {
    red[0][w] = acc;
    red[1][w] = ss;
  }
  __syncthreads();
  if (t == 0) {
    float v = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    if (p.norm_w) v *= 1.0f / sqrtf(((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) / (float)p.K + p.eps);
    if (p.sigmoid) v = sigmoidf_(v);
    p.y[m] = v;
  }
}

}  // namespace trx
