// Fused full-attention decoder layer (trx_layer.hip): parameters and host entry points.
#pragma once

#include "trx_internal.h"
#include "trx_ops.h"
#include "trx_gemv_dev.h"

namespace trx {

struct LayerParams {
  GemvParams qkv, o, gu, down;      // the layer's four projections, rows per item 2, 1, 2, 1
  AttnParams attn;                  // n_split = blocks / n_kv
  unsigned long long* bar;          // barrier counters (zero at the start of a sequence)
  const unsigned* xcc_blocks;       // blocks of the grid per XCD
  const int* pos;                   // device position of this forward
  int n_layers;                     // fused layers per position (epoch stride)
  int layer_slot;                   // this layer's index among them
  unsigned n_xcc;
  int* err;                         // set to 1 when a barrier wait times out
};

struct LayerSetup {
  bool ok = false;
  int blocks = 0, lds = 0;
  unsigned n_xcc = 0;
  const void* fn = nullptr;
};

// Checks whether the geometry has a fused kernel that fits one block per CU, and measures the
// grid's blocks per XCD. ls.ok = false leaves the model on per-operation kernels.
int layer_prepare(LayerSetup& ls, int kind, int rep, int hd, int E, int qdim, int F, unsigned* xcc_blocks_dev);
int layer_gemv_params(GemvParams& p, const uint8_t* rows, int kind, int M, int K, const float* x,
                      const float* norm_w, float eps, float* y, int epi, const float* resid, int rows_per_item);
int launch_layer(const LayerSetup& ls, const LayerParams& lp, hipStream_t s);

// From trx_gemv.hip.
int gemv_check(int kind, int M, int K);
void fill_geom_public(GemvParams& p, const uint8_t* rows, int kind, int M, int K);

}  // namespace trx
