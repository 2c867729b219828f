// SwiGLU of the fp16 MLP (solution/silu_mul.py:26-44): values are computed in fp32 from the
// fp16 inputs and rounded to fp16 once, in the kernel's order, with no fused multiply-adds
// (the contract pragma), so the only rounding differences from a plain fp32 evaluation are
// those of expf.  Shared by the elementwise kernels (swiglu.hip) and the GEMM epilogues that
// apply it to a tile (nf4_gemm.hip).
#pragma once

#include "common.h"

namespace mxs {

// out = fp16(up * (g * sigmoid(g))), sigmoid(g) = 1 / (1 + exp(-g))
__device__ __forceinline__ _Float16 swiglu_fwd(float g, float u) {
#pragma clang fp contract(off)
  const float s = 1.0f / (1.0f + expf(-g));
  const float silu = g * s;
  return (_Float16)(u * silu);
}

// For the incoming d(out) = dh: d(gate) = fp16((dh * up) * (s + silu * (1 - s))),
// d(up) = fp16(dh * silu)
__device__ __forceinline__ void swiglu_bwd(float dh, float g, float u, _Float16& d_gate,
                                           _Float16& d_up) {
#pragma clang fp contract(off)
  const float s = 1.0f / (1.0f + expf(-g));
  const float silu = g * s;
  d_gate = (_Float16)((dh * u) * (s + silu * (1.0f - s)));
  d_up = (_Float16)(dh * silu);
}

}  // namespace mxs
