// SwiGLU of the fp16 MLP (solution/silu_mul.py:26-44): values are computed in fp32 from the
// fp16 inputs and rounded to fp16 once, in the kernel's order, with no fused multiply-adds
// (the contract pragma; the last product is kept in fp32 before its fp16 cast, f16_of).  sigmoid(g) = 1 / (1 + exp(-g)) uses the hardware's exp2 and
// reciprocal (v_exp_f32 on log2(e) * x, v_rcp_f32: each within about 1 ulp), the class of
// approximation the reference's tl.sigmoid compiles to (approximate exp2 and division).  An
// accurate expf and an IEEE division take about four times the vector instructions (forward
// 30 against 8 per element, backward 35 against 13, on gfx950), which the GEMM epilogues that
// apply this to a whole tile pay on one CU.  Against an fp32 evaluation with
// libm's expf the fp16 results differ only where the fp32 value sits within a few ulp of an
// fp16 rounding boundary.  Shared by the elementwise kernels (swiglu.hip) and the GEMM
// epilogues (nf4_gemm.hip), so the two give the same bits.
#pragma once

#include "common.h"

namespace mxs {

__device__ __forceinline__ float sigmoid_hw(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// out = fp16(up * (g * sigmoid(g)))
__device__ __forceinline__ _Float16 swiglu_fwd(float g, float u) {
#pragma clang fp contract(off)
  const float s = sigmoid_hw(g);
  const float silu = g * s;
  return f16_of(u * silu);
}

// For the incoming d(out) = dh: d(gate) = fp16((dh * up) * (s + silu * (1 - s))),
// d(up) = fp16(dh * silu)
__device__ __forceinline__ void swiglu_bwd(float dh, float g, float u, _Float16& d_gate,
                                           _Float16& d_up) {
#pragma clang fp contract(off)
  const float s = sigmoid_hw(g);
  const float silu = g * s;
  d_gate = f16_of((dh * u) * (s + silu * (1.0f - s)));
  d_up = f16_of(dh * silu);
}

}  // namespace mxs
