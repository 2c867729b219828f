// SwiGLU of the fp16 MLP on gfx950: silu(gate) * up and its in-place backward, the kernel of
// solution/silu_mul.py (silu_mul_kernel, :26-44; SiluMulInPlace, :52-71).  HBM-bound
// elementwise work: 6 bytes per element forward (gate, up in; out), 10 backward (grad, gate,
// up in; d(gate), d(up) written over gate and up).  Each lane takes 8 consecutive elements per
// 16-byte access; a grid-stride loop covers any size, the tail (and unaligned buffers) take the
// scalar form.
#include "common.h"
#include "mxs_nf4.h"
#include "swiglu.h"

namespace mxs {

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void k_silu_mul(const _Float16* __restrict__ gate,
                                                  const _Float16* __restrict__ up,
                                                  _Float16* __restrict__ out, int64_t n,
                                                  int vec) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    for (int64_t c = t; c < n / 8; c += stride) {
      const half8v g = reinterpret_cast<const half8v*>(gate)[c];
      const half8v u = reinterpret_cast<const half8v*>(up)[c];
      half8v o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = swiglu_fwd((float)g[e], (float)u[e]);
      reinterpret_cast<half8v*>(out)[c] = o;
    }
    for (int64_t i = n / 8 * 8 + t; i < n; i += stride)
      out[i] = swiglu_fwd((float)gate[i], (float)up[i]);
  } else {
    for (int64_t i = t; i < n; i += stride) out[i] = swiglu_fwd((float)gate[i], (float)up[i]);
  }
}

__global__ __launch_bounds__(256) void k_silu_mul_bwd(const _Float16* __restrict__ grad,
                                                      _Float16* __restrict__ gate,
                                                      _Float16* __restrict__ up, int64_t n,
                                                      int vec) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    for (int64_t c = t; c < n / 8; c += stride) {
      const half8v d = reinterpret_cast<const half8v*>(grad)[c];
      const half8v g = reinterpret_cast<const half8v*>(gate)[c];
      const half8v u = reinterpret_cast<const half8v*>(up)[c];
      half8v dg, du;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        _Float16 a, b;
        swiglu_bwd((float)d[e], (float)g[e], (float)u[e], a, b);
        dg[e] = a;
        du[e] = b;
      }
      reinterpret_cast<half8v*>(gate)[c] = dg;
      reinterpret_cast<half8v*>(up)[c] = du;
    }
    for (int64_t i = n / 8 * 8 + t; i < n; i += stride)
      swiglu_bwd((float)grad[i], (float)gate[i], (float)up[i], gate[i], up[i]);
  } else {
    for (int64_t i = t; i < n; i += stride)
      swiglu_bwd((float)grad[i], (float)gate[i], (float)up[i], gate[i], up[i]);
  }
}

// Workgroups for n elements: one 8-element chunk per lane and pass, at most 8 per CU of 256
// lanes in flight (a grid-stride loop covers the rest).
static unsigned silu_grid(int64_t n) {
  const int64_t chunks = (n + 7) / 8;
  int64_t wg = (chunks + 255) / 256;
  if (wg > 4096) wg = 4096;
  return (unsigned)(wg < 1 ? 1 : wg);
}

static bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

}  // namespace mxs

using namespace mxs;

extern "C" {

int mxs_silu_mul(const void* gate, const void* up, void* out, int64_t n, hipStream_t stream) {
  if (n < 0) return MXS_ERR_ARG;
  if (n == 0) return MXS_OK;
  if (!gate || !up || !out) return MXS_ERR_ARG;
  const int vec = aligned16(gate) && aligned16(up) && aligned16(out);
  hipLaunchKernelGGL(k_silu_mul, dim3(silu_grid(n)), dim3(256), 0, stream,
                     static_cast<const _Float16*>(gate), static_cast<const _Float16*>(up),
                     static_cast<_Float16*>(out), n, vec);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

int mxs_silu_mul_bwd(const void* grad, void* gate, void* up, int64_t n, hipStream_t stream) {
  if (n < 0) return MXS_ERR_ARG;
  if (n == 0) return MXS_OK;
  if (!grad || !gate || !up) return MXS_ERR_ARG;
  const int vec = aligned16(grad) && aligned16(gate) && aligned16(up);
  hipLaunchKernelGGL(k_silu_mul_bwd, dim3(silu_grid(n)), dim3(256), 0, stream,
                     static_cast<const _Float16*>(grad), static_cast<_Float16*>(gate),
                     static_cast<_Float16*>(up), n, vec);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

}  // extern "C"
