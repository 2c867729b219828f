// q/k/v of Qwen2 attention on gfx950: the LoRA add, the rotary position embedding of q and k,
// and the cast, in one launch each way (solution/attention.py:28-82 qkv_rope_kernel; without
// the add and v it is solution/rope.py:41-66 rope_kernel).  HBM-bound elementwise work: per
// position, every head of 128 values is read once (twice with a LoRA term) and written once;
// cos / sin rows (512 B each) are shared by the position's heads through the caches.
//
// One head is 64 rotation pairs (x[j], x[j + 64]); a lane takes eight adjacent pairs, so 8
// lanes cover a head and a 256-lane workgroup 32 heads, each access 16 bytes (fp16; two of 16
// for fp32).  Tensors are [B, H, T, 128] views with any (b, h, t) strides and unit stride along
// the head: the projections' [B, T, H * 128] output seen per head, or attention's gradients.
// Arithmetic in fp32, each product and sum one rounding (no contraction), one rounding to the
// output type:
//   x = a (+ b * scale);  forward  y1 = x1 * c1 - x2 * s1,  y2 = x2 * c2 + x1 * s2
//                         backward y1 = x1 * c1 + x2 * s2,  y2 = x2 * c2 - x1 * s1
// (q and k rotated; v only added and cast).
#include "common.h"
#include "mxs_nf4.h"

namespace mxs {

struct RopeArgs {
  const void* in[5];      // q_a, q_b, k, v_a, v_b (q_b, v_a, v_b may be null)
  void* out[3];           // q, k, v (v null when v_a is)
  int64_t stride[8][3];   // (b, h, t) element strides of in[0..4], out[0..2]
  const float* cos;
  const float* sin;
  int64_t cs_b, cs_t;     // cos / sin strides (b may be 0: one row set for the batch)
  int batch, n_tokens, n_q, n_kv, heads;
  float q_scale, v_scale;
};

// eight elements: one 16-byte access for fp16, two for fp32
__device__ __forceinline__ void load8(const _Float16* p, float (&x)[8]) {
  const half8_t h = *reinterpret_cast<const half8_t*>(p);
#pragma unroll
  for (int e = 0; e < 8; e++) x[e] = (float)h[e];
}
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
  const float4_t u = *reinterpret_cast<const float4_t*>(p);
  const float4_t v = *reinterpret_cast<const float4_t*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    x[e] = u[e];
    x[4 + e] = v[e];
  }
}
__device__ __forceinline__ void store8(_Float16* p, const float (&y)[8]) {
  half8_t h;
#pragma unroll
  for (int e = 0; e < 8; e++) h[e] = (_Float16)y[e];
  *reinterpret_cast<half8_t*>(p) = h;
}
__device__ __forceinline__ void store8(float* p, const float (&y)[8]) {
  *reinterpret_cast<float4_t*>(p) = (float4_t){y[0], y[1], y[2], y[3]};
  *reinterpret_cast<float4_t*>(p + 4) = (float4_t){y[4], y[5], y[6], y[7]};
}

template <typename TI, typename TO, bool BWD>
__global__ __launch_bounds__(256) void k_qkv_rope(RopeArgs a) {
#pragma clang fp contract(off)
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  constexpr int P = 8;              // pairs per lane
  const int64_t item = gid >> 3;  // (position, head)
  const int d = (int)(gid & 7) * P;
  if (item >= (int64_t)a.batch * a.n_tokens * a.heads) return;
  const int h = (int)(item % a.heads);
  const int64_t pos = item / a.heads;
  const int b = (int)(pos / a.n_tokens), t = (int)(pos % a.n_tokens);
  // heads in order: q (n_q), k (n_kv), v (n_kv)
  const int kind = h < a.n_q ? 0 : (h < a.n_q + a.n_kv ? 1 : 2);
  const int hh = kind == 0 ? h : (kind == 1 ? h - a.n_q : h - a.n_q - a.n_kv);
  const int ia = kind == 0 ? 0 : (kind == 1 ? 2 : 3);
  const int ib = kind == 0 ? 1 : 4;
  const int64_t* sa = a.stride[ia];
  const TI* pa = static_cast<const TI*>(a.in[ia]) + b * sa[0] + hh * sa[1] + t * sa[2] + d;
  float x1[P], x2[P];
  load8(pa, x1);
  load8(pa + 64, x2);
  if (kind != 1 && a.in[ib]) {
    const int64_t* sb = a.stride[ib];
    const TI* pb = static_cast<const TI*>(a.in[ib]) + b * sb[0] + hh * sb[1] + t * sb[2] + d;
    const float scale = kind == 0 ? a.q_scale : a.v_scale;
    float y1[P], y2[P];
    load8(pb, y1);
    load8(pb + 64, y2);
#pragma unroll
    for (int e = 0; e < P; e++) {
      x1[e] = x1[e] + y1[e] * scale;
      x2[e] = x2[e] + y2[e] * scale;
    }
  }
  float o1[P], o2[P];
  if (kind != 2) {
    const int64_t cr = b * a.cs_b + t * a.cs_t + d;
    float c1[P], c2[P], s1[P], s2[P];
    load8(a.cos + cr, c1);
    load8(a.cos + cr + 64, c2);
    load8(a.sin + cr, s1);
    load8(a.sin + cr + 64, s2);
#pragma unroll
    for (int e = 0; e < P; e++) {
      const float p = BWD ? s2[e] : -s1[e];
      const float r = BWD ? -s1[e] : s2[e];
      o1[e] = x1[e] * c1[e] + x2[e] * p;
      o2[e] = x2[e] * c2[e] + x1[e] * r;
    }
  } else {
#pragma unroll
    for (int e = 0; e < P; e++) {
      o1[e] = x1[e];
      o2[e] = x2[e];
    }
  }
  const int64_t* so = a.stride[5 + kind];
  TO* po = static_cast<TO*>(a.out[kind]) + b * so[0] + hh * so[1] + t * so[2] + d;
  store8(po, o1);
  store8(po + 64, o2);
}

template <typename TI, typename TO>
static int launch_rope(const RopeArgs& a, bool bwd, hipStream_t stream) {
  const int64_t threads = (int64_t)a.batch * a.n_tokens * a.heads * 8;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (bwd)
    hipLaunchKernelGGL((k_qkv_rope<TI, TO, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((k_qkv_rope<TI, TO, false>), grid, dim3(256), 0, stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

}  // namespace mxs

using namespace mxs;

extern "C" {

int mxs_qkv_rope(const void* const tensors[8], const int64_t strides[24], const float* cos,
                 const float* sin, int64_t cos_stride_b, int64_t cos_stride_t, int batch,
                 int n_tokens, int n_q, int n_kv, int in_f32, int out_f32, int backward,
                 float q_scale, float v_scale, hipStream_t stream) {
  if (!tensors || !strides || batch < 0 || n_tokens < 0 || n_q < 0 || n_kv < 0)
    return MXS_ERR_ARG;
  RopeArgs a{};
  for (int i = 0; i < 5; i++) a.in[i] = tensors[i];
  for (int i = 0; i < 3; i++) a.out[i] = const_cast<void*>(tensors[5 + i]);
  for (int i = 0; i < 8; i++)
    for (int j = 0; j < 3; j++) a.stride[i][j] = strides[3 * i + j];
  a.cos = cos;
  a.sin = sin;
  a.cs_b = cos_stride_b;
  a.cs_t = cos_stride_t;
  a.batch = batch;
  a.n_tokens = n_tokens;
  a.n_q = n_q;
  a.n_kv = n_kv;
  a.heads = n_q + n_kv + (tensors[3] ? n_kv : 0);
  a.q_scale = q_scale;
  a.v_scale = v_scale;
  if ((int64_t)batch * n_tokens * a.heads == 0) return MXS_OK;
  // required operands: q and k in and out, cos / sin (rotated heads); v in and out together
  if ((n_q && (!a.in[0] || !a.out[0])) || (n_kv && (!a.in[2] || !a.out[1])) || !cos || !sin ||
      (!a.in[3]) != (!a.out[2]) || (a.in[4] && !a.in[3]))
    return MXS_ERR_ARG;
  // 8-element accesses (16 bytes): every used base pointer and stride a multiple of 8
  // elements (fp16) or 4 (fp32)
  const size_t in_sz = in_f32 ? 4 : 2, out_sz = out_f32 ? 4 : 2;
  for (int i = 0; i < 8; i++) {
    const void* p = i < 5 ? a.in[i] : a.out[i - 5];
    if (!p) continue;
    const size_t sz = i < 5 ? in_sz : out_sz;
    const int64_t q = (int64_t)(16 / sz);
    if ((uintptr_t)p % 16 != 0) return MXS_ERR_ALIGN;
    for (int j = 0; j < 3; j++)
      if (a.stride[i][j] % q != 0) return MXS_ERR_ALIGN;
  }
  if ((uintptr_t)cos % 16 || (uintptr_t)sin % 16 || cos_stride_b % 4 || cos_stride_t % 4)
    return MXS_ERR_ALIGN;
  const bool bwd = backward != 0;
  if (in_f32)
    return out_f32 ? launch_rope<float, float>(a, bwd, stream)
                   : launch_rope<float, _Float16>(a, bwd, stream);
  return out_f32 ? launch_rope<_Float16, float>(a, bwd, stream)
                 : launch_rope<_Float16, _Float16>(a, bwd, stream);
}

}  // extern "C"
