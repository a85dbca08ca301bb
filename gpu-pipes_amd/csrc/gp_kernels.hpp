// Host-side launch interface between the C ABI (capi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gp {

// One MGN-shaped MLP call: x[M,K] -> Linear(K,128)+ReLU -> Linear(128,128)+ReLU
// -> Linear(128,128) [-> LayerNorm(128) when gamma != nullptr] -> out[M,128].
// All tensors fp16, row-major, weights stored [K, N] (nn.Linear.weight.t()).
struct MgnArgs {
  int64_t M;
  int64_t K;
  const void* x;
  const void* w1;
  const void* b1;
  const void* w2;
  const void* b2;
  const void* w3;
  const void* b3;
  const void* gamma;  // nullptr: no LayerNorm (mgn_linears)
  const void* beta;
  float eps;
  void* out;
};

// Persistent fused kernel (all layers in one workgroup per CU).
hipError_t mgn_fused_launch(const MgnArgs& a, int num_cus, hipStream_t stream);

}  // namespace gp
