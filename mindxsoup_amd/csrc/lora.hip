// LoRA side branch of the NF4 projection on gfx950: the small GEMMs around the fused main GEMM.
//
// peft's branch (restated at solution/attention.py:197-199, solution/test_unpad.py:28-29) with
// the reference's dropout semantics (solution/dropout.py:33-35: keep ? fp16(fp32(x) * 1/(1-p))
// : 0) and scaling s = alpha / r:
//   forward   Hs  = fp16(s * drop(X) . A^T)        [M, r]   (also written transposed [r, M])
//   backward  dHs = fp16(s * dY . B)               [M, r]   (also transposed)
//             dA  = dHs^T . drop(X)                [r, K]   fp32
//             dB  = dY^T . Hs                      [N, r]   fp32
// Hs and dHs carry the factor s, so the main GEMM's epilogue adds Hs . B^T (= s * B(A(drop x)))
// and dHs . A (= the LoRA part of dX before the dropout mask) without another multiply, and
// dB = s * dY^T . H = dY^T . Hs.
//
// Reductions over the hidden dims (Hs, dHs) use v_mfma_f32_16x16x32_f16 with 16 tokens per
// workgroup and the reduction split over 8 waves (LDS sum).  Reductions over tokens (dA, dB)
// need operands contiguous along tokens: each lane loads an 8 token x 8 column block of row-major
// fp16 and regroups it in registers into 8 MFMA operands (one per column), so a wave covers 128
// columns per 32-token step without a transpose in memory.
#include "common.h"
#include "mxs_nf4.h"

namespace mxs {

constexpr int kLoraWaves = 8;

__device__ __forceinline__ _Float16 drop1(_Float16 x, uint8_t keep, float scale) {
  return keep ? (_Float16)((float)x * scale) : (_Float16)0.0f;
}

// out[m][r] = s * sum_k P[m][k] * R(r, k), P fp16 [M, K] row-major (optionally dropped out with
// mask/scale), R(r, k) = R[r * r_stride_r + k * r_stride_k].  One workgroup per 16 rows; the
// r dimension in blocks of 16.  Writes out [M, r] and outT [r, ldt] (fp16; ldt >= M, the
// columns M..ldt-1 of outT are written as zeros).
__global__ __launch_bounds__(64 * kLoraWaves) void k_lora_rows(
    const _Float16* __restrict__ P, int M, int K, const uint8_t* __restrict__ mask, float mscale,
    const _Float16* __restrict__ R, int64_t r_stride_r, int64_t r_stride_k, int r, float s,
    _Float16* __restrict__ out, _Float16* __restrict__ outT, int ldt) {
  __shared__ float red[kLoraWaves][16][17];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m0 = blockIdx.x * 16;
  const int r0 = blockIdx.y * 16;
  const int row = m0 + (lane & 15);
  const int kg = 8 * (lane >> 4);  // k offset of this lane inside a 32-step
  const int rr = r0 + (lane & 15);
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int steps = K / 32;
  for (int st = wave; st < steps; st += kLoraWaves) {
    const int k = st * 32 + kg;
    half8_t a = {};
    if (row < M) {
      a = *reinterpret_cast<const half8_t*>(P + (int64_t)row * K + k);
      if (mask) {
        const u32x2 mk = *reinterpret_cast<const u32x2*>(mask + (int64_t)row * K + k);
#pragma unroll
        for (int e = 0; e < 8; e++)
          a[e] = drop1(a[e], (uint8_t)(mk[e >> 2] >> (8 * (e & 3))), mscale);
      }
    }
    half8_t b;
    if (r_stride_k == 1) {
      b = *reinterpret_cast<const half8_t*>(R + (int64_t)rr * r_stride_r + k);
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) b[e] = R[(int64_t)rr * r_stride_r + (int64_t)(k + e) * r_stride_k];
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
  }
  // acc[v] = C[row 4*(lane/16)+v][col lane%16]
#pragma unroll
  for (int v = 0; v < 4; v++) red[wave][4 * (lane >> 4) + v][lane & 15] = acc[v];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int i = threadIdx.x >> 4, j = threadIdx.x & 15;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kLoraWaves; w++) sum += red[w][i][j];
    const int m = m0 + i;
    if (m < M) {
      const _Float16 h = (_Float16)(s * sum);
      out[(int64_t)m * r + r0 + j] = h;
      outT[(int64_t)(r0 + j) * ldt + m] = h;
    } else if (m < ldt) {
      outT[(int64_t)(r0 + j) * ldt + m] = (_Float16)0.0f;
    }
  }
}

// out[n][j] (or out[j][n] with out_rn) = sum_m PT[j][m] * Q[m][n], PT fp16 [r, ldt] (transposed
// LoRA activations, ldt a multiple of 8), Q fp16 [M, Nq] row-major (optionally dropped out),
// fp32 result.  Workgroup: 128 columns x 16 r-values; 8 waves split the tokens; the 8 partial
// sums are combined in a fixed order in LDS.
__global__ __launch_bounds__(64 * kLoraWaves) void k_lora_cols(
    const _Float16* __restrict__ PT, int M, int ldt, const _Float16* __restrict__ Q, int Nq,
    const uint8_t* __restrict__ mask, float mscale, int r, float* __restrict__ out,
    int out_rn) {
  __shared__ float red[4][16][129];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nb = blockIdx.x * 128;
  const int r0 = blockIdx.y * 16;
  const int ln = lane & 15;        // column group: columns nb + 8*ln .. +8
  const int lg = lane >> 4;        // token group: tokens m + 8*lg .. +8
  const int col = nb + 8 * ln;
  float4_t acc[8];
#pragma unroll
  for (int c = 0; c < 8; c++) acc[c] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const int steps = (M + 31) / 32;
  for (int st = wave; st < steps; st += kLoraWaves) {
    const int mb = st * 32 + 8 * lg;
    // A operand: PT[r0 + lane%16][mb .. mb+8]
    half8_t a = {};
    if (mb < M) a = *reinterpret_cast<const half8_t*>(PT + (int64_t)(r0 + ln) * ldt + mb);
    // 8 tokens x 8 columns of Q
    u32x4 rows[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int m = mb + e;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M && col < Nq) {
        v = *reinterpret_cast<const u32x4*>(Q + (int64_t)m * Nq + col);
        if (mask) {
          const u32x2 mk = *reinterpret_cast<const u32x2*>(mask + (int64_t)m * Nq + col);
          half8_t h = __builtin_bit_cast(half8_t, v);
#pragma unroll
          for (int c = 0; c < 8; c++) h[c] = drop1(h[c], (uint8_t)(mk[c >> 2] >> (8 * (c & 3))), mscale);
          v = __builtin_bit_cast(u32x4, h);
        }
      }
      rows[e] = v;
    }
#pragma unroll
    for (int c = 0; c < 8; c++) {
      // B operand for column col + c: the 8 tokens' values of that column
      half8_t b;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const half8_t h = __builtin_bit_cast(half8_t, rows[e]);
        b[e] = h[c];
      }
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
    }
  }
  // acc[c][v] = C[r = 4*lg + v][j = ln] for column nb + 8*ln + c.  Waves 4..7 store, waves
  // 0..3 add theirs (slot w = wave w + wave w+4), then the 4 slots are summed.
  static_assert(kLoraWaves == 8, "two-stage LDS sum assumes 8 waves");
  if (wave >= 4) {
#pragma unroll
    for (int c = 0; c < 8; c++)
#pragma unroll
      for (int v = 0; v < 4; v++) red[wave - 4][4 * lg + v][8 * ln + c] = acc[c][v];
  }
  __syncthreads();
  if (wave < 4) {
#pragma unroll
    for (int c = 0; c < 8; c++)
#pragma unroll
      for (int v = 0; v < 4; v++) red[wave][4 * lg + v][8 * ln + c] += acc[c][v];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 16 * 128; idx += 64 * kLoraWaves) {
    const int i = idx >> 7, j = idx & 127;
    const float sum = (red[0][i][j] + red[1][i][j]) + (red[2][i][j] + red[3][i][j]);
    const int n = nb + j;
    if (n < Nq) {
      if (out_rn) out[(int64_t)(r0 + i) * Nq + n] = sum;
      else out[(int64_t)n * r + r0 + i] = sum;
    }
  }
}

static int check_launch() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

}  // namespace mxs

using namespace mxs;

extern "C" {

int mxs_lora_h(const void* x, int M, int K, const void* lora_a, int r, const void* mask,
               float mask_scale, float s, void* h, void* ht, int ldt, hipStream_t stream) {
  if (M < 0 || K < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!x || !lora_a || !h || !ht) return MXS_ERR_ARG;
  if (r % 16 || K % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)x % 16) || ((uintptr_t)lora_a % 16) || (mask && ((uintptr_t)mask % 8)))
    return MXS_ERR_ALIGN;
  hipLaunchKernelGGL(k_lora_rows, dim3((ldt + 15) / 16, r / 16), dim3(64 * kLoraWaves), 0, stream,
                     static_cast<const _Float16*>(x), M, K, static_cast<const uint8_t*>(mask),
                     mask_scale, static_cast<const _Float16*>(lora_a), (int64_t)K, (int64_t)1, r,
                     s, static_cast<_Float16*>(h), static_cast<_Float16*>(ht), ldt);
  return check_launch();
}

int mxs_lora_dh(const void* dy, int M, int N, const void* lora_b, int r, float s, void* dh,
                void* dht, int ldt, hipStream_t stream) {
  if (M < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!dy || !lora_b || !dh || !dht) return MXS_ERR_ARG;
  if (r % 16 || N % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if ((uintptr_t)dy % 16) return MXS_ERR_ALIGN;
  hipLaunchKernelGGL(k_lora_rows, dim3((ldt + 15) / 16, r / 16), dim3(64 * kLoraWaves), 0, stream,
                     static_cast<const _Float16*>(dy), M, N, nullptr, 1.0f,
                     static_cast<const _Float16*>(lora_b), (int64_t)1, (int64_t)r, r, s,
                     static_cast<_Float16*>(dh), static_cast<_Float16*>(dht), ldt);
  return check_launch();
}

int mxs_lora_grad_a(const void* dht, int ldt, const void* x, int M, int K, int r,
                    const void* mask, float mask_scale, float* da, hipStream_t stream) {
  if (M < 0 || K < 0 || r <= 0) return MXS_ERR_ARG;
  if (!dht || !x || !da) return MXS_ERR_ARG;
  if (r % 16 || K % 8 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)x % 16) || (mask && ((uintptr_t)mask % 8)) || ((uintptr_t)dht % 16))
    return MXS_ERR_ALIGN;
  if (K == 0) return MXS_OK;
  hipLaunchKernelGGL(k_lora_cols, dim3((K + 127) / 128, r / 16), dim3(64 * kLoraWaves), 0, stream,
                     static_cast<const _Float16*>(dht), M, ldt, static_cast<const _Float16*>(x), K,
                     static_cast<const uint8_t*>(mask), mask_scale, r, da, 1);
  return check_launch();
}

int mxs_lora_grad_b(const void* ht, int ldt, const void* dy, int M, int N, int r, float* db,
                    hipStream_t stream) {
  if (M < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (!ht || !dy || !db) return MXS_ERR_ARG;
  if (r % 16 || N % 8 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)dy % 16) || ((uintptr_t)ht % 16)) return MXS_ERR_ALIGN;
  if (N == 0) return MXS_OK;
  hipLaunchKernelGGL(k_lora_cols, dim3((N + 127) / 128, r / 16), dim3(64 * kLoraWaves), 0, stream,
                     static_cast<const _Float16*>(ht), M, ldt, static_cast<const _Float16*>(dy), N,
                     nullptr, 1.0f, r, db, 0);
  return check_launch();
}

}  // extern "C"
