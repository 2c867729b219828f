// LoRA side branch of the NF4 projection on gfx950: the small GEMMs around the fused main GEMM.
//
// peft's branch (restated at solution/attention.py:197-199, solution/test_unpad.py:28-29) with
// the reference's dropout semantics (solution/dropout.py:33-35: keep ? fp16(fp32(x) * 1/(1-p))
// : 0) and scaling s = alpha / r:
//   forward   Hs  = fp16(s * drop(X) . A^T)        [M, r]   (also written transposed [r, ldt])
//   backward  dHs = fp16(s * dY . B)               [M, r]   (also transposed)
//             dA  = dHs^T . drop(X)                [r, K]   fp32
//             dB  = dY^T . Hs                      [N, r]   fp32
// Hs and dHs carry the factor s, so the main GEMM's epilogue adds Hs . B^T (= s * B(A(drop x)))
// and dHs . A (= the LoRA part of dX before the dropout mask) without another multiply, and
// dB = s * dY^T . H = dY^T . Hs.
//
// These products are thin (r = 16) and read a few MB each, so they are spread over many
// workgroups: each computes a partial over one slice of the reduction with
// v_mfma_f32_16x16x32_f16 and writes it to a workspace, and a small second kernel sums the slices
// in a fixed order (deterministic) and writes the results.  (Summing in the last-arriving
// workgroup instead needs agent-scope fences, which on the multi-XCD gfx950 write back and
// invalidate whole L2s; measured, that cost more than the second launch.)
//   rows kernel (Hs, dHs): workgroup = 16 tokens x one reduction slice, 4 waves in LDS sum.
//   cols kernel (dA and dB in one launch):  reduction over tokens; each lane loads an 8-token x 8-column block
//     of the row-major fp16 input and regroups it in registers into 8 MFMA operands (one per
//     column), so a wave covers 128 columns per 32-token step without a transpose in memory.
#include "common.h"
#include "mxs_nf4.h"

namespace mxs {

constexpr int kRowsWaves = 4;     // waves per rows-kernel workgroup
constexpr int kRowsUnroll = 4;    // 32-wide reduction steps per wave and slice
constexpr int kColsRows = 64;     // tokens per cols-kernel workgroup (2 waves x 32)

__device__ __forceinline__ _Float16 drop1(_Float16 x, uint8_t keep, float scale) {
  return keep ? (_Float16)((float)x * scale) : (_Float16)0.0f;
}

// Reduction slice length (multiple of 32) for the rows kernel.
constexpr int kRowsSlice = 32 * kRowsWaves * kRowsUnroll;
static int rows_slices(int K) { return (K + kRowsSlice - 1) / kRowsSlice; }

struct RowsArgs {
  const _Float16* P;       // [M, K] row-major
  int M, K;
  const uint8_t* mask;     // [M, K] keep mask or null
  float mscale;
  const _Float16* R;       // R(c, k) = R[c * rs_r + k * rs_k]
  int64_t rs_r, rs_k;
  int r, ldt;
  float s;
  _Float16* out;           // [M, r]
  _Float16* outT;          // [r, ldt], zeros past M
  _Float16* rt;            // optional [K, r]: R transposed (rs_k == 1 only)
  float* ws;               // [slices][ldt][r]
};

// Partial of out[m][c] = s * sum_k P[m][k] * R(c, k) over reduction slice blockIdx.y, for the 16
// rows of blockIdx.x: ws[slice][m][c] fp32.
__global__ __launch_bounds__(64 * kRowsWaves) void k_lora_rows(RowsArgs a) {
  __shared__ float red[kRowsWaves][16][17];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m0 = blockIdx.x * 16;
  const int slice = blockIdx.y;
  const int row = m0 + (lane & 15);
  const int kg = 8 * (lane >> 4);
  const int kbase = slice * kRowsSlice + wave * 32 * kRowsUnroll;
  for (int r0 = 0; r0 < a.r; r0 += 16) {
    const int rr = r0 + (lane & 15);
    half8_t av[kRowsUnroll], bv[kRowsUnroll];
#pragma unroll
    for (int u = 0; u < kRowsUnroll; u++) {
      const int k = kbase + u * 32 + kg;
      half8_t x = {}, y = {};
      if (k < a.K) {
        if (row < a.M) {
          x = *reinterpret_cast<const half8_t*>(a.P + (int64_t)row * a.K + k);
          if (a.mask) {
            const u32x2 mk = *reinterpret_cast<const u32x2*>(a.mask + (int64_t)row * a.K + k);
#pragma unroll
            for (int e = 0; e < 8; e++)
              x[e] = drop1(x[e], (uint8_t)(mk[e >> 2] >> (8 * (e & 3))), a.mscale);
          }
        }
        if (a.rs_k == 1) {
          y = *reinterpret_cast<const half8_t*>(a.R + (int64_t)rr * a.rs_r + k);
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++) y[e] = a.R[(int64_t)rr * a.rs_r + (int64_t)(k + e) * a.rs_k];
        }
      }
      av[u] = x;
      bv[u] = y;
    }
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kRowsUnroll; u++)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u], bv[u], acc, 0, 0, 0);
    // acc[v] = C[row 4*(lane/16)+v][col lane%16]
#pragma unroll
    for (int v = 0; v < 4; v++) red[wave][4 * (lane >> 4) + v][lane & 15] = acc[v];
    __syncthreads();
    const int i = threadIdx.x >> 4, j = threadIdx.x & 15;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kRowsWaves; w++) sum += red[w][i][j];
    if (m0 + i < a.ldt) a.ws[((int64_t)slice * a.ldt + m0 + i) * a.r + r0 + j] = sum;
    __syncthreads();
  }
  // the first row block also writes this slice of R transposed
  if (a.rt && blockIdx.x == 0) {
    for (int idx = threadIdx.x; idx < kRowsSlice * a.r; idx += 64 * kRowsWaves) {
      const int k = slice * kRowsSlice + idx / a.r, c = idx % a.r;
      if (k < a.K) a.rt[(int64_t)k * a.r + c] = a.R[(int64_t)c * a.rs_r + k];
    }
  }
}

// out[m][c] = fp16(s * sum over slices of ws) for m < M; outT [r, ldt] with zeros past M.
__global__ __launch_bounds__(256) void k_lora_rows_finish(RowsArgs a, int slices) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.ldt * a.r) return;
  const int m = idx / a.r, c = idx % a.r;
  float sum = 0.f;
  for (int z = 0; z < slices; z++) sum += a.ws[((int64_t)z * a.ldt + m) * a.r + c];
  const _Float16 h = m < a.M ? (_Float16)(a.s * sum) : (_Float16)0.0f;
  if (m < a.M) a.out[(int64_t)m * a.r + c] = h;
  a.outT[(int64_t)c * a.ldt + m] = h;
}

struct ColsProblem {
  const _Float16* PT;      // [r, ldt] (transposed LoRA activations)
  const _Float16* Q;       // [M, Nq] row-major
  const uint8_t* mask;     // [M, Nq] keep mask or null
  float mscale;
  int Nq;
  float* out;              // [r, Nq] (out_rn) or [Nq, r]
  int out_rn;
  float* ws;               // [token blocks][r][Nq]
};

// Partial of out[j][n] = sum_m PT[j][m] * Q[m][n] over the 64 tokens of blockIdx.y, for problem
// blockIdx.z (dA and dB share the launch): workgroup = 128 columns, 2 waves of 32 tokens, LDS
// sum; ws[token block][j][n] fp32.
__global__ __launch_bounds__(128) void k_lora_cols(ColsProblem p0, ColsProblem p1, int M, int ldt,
                                                  int r) {
  __shared__ float red[16][129];
  const ColsProblem a = blockIdx.z == 0 ? p0 : p1;
  const int nb = blockIdx.x * 128;
  if (nb >= a.Nq) return;  // whole workgroup (the wider problem sets the grid)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int mblk = blockIdx.y;
  const int ln = lane & 15;  // columns nb + 8*ln .. +8
  const int lg = lane >> 4;  // tokens mb .. +8
  const int col = nb + 8 * ln;
  const int mb = mblk * kColsRows + wave * 32 + 8 * lg;
  u32x4 rows[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int m = mb + e;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < M && col < a.Nq) {
      v = *reinterpret_cast<const u32x4*>(a.Q + (int64_t)m * a.Nq + col);
      if (a.mask) {
        const u32x2 mk = *reinterpret_cast<const u32x2*>(a.mask + (int64_t)m * a.Nq + col);
        half8_t h = __builtin_bit_cast(half8_t, v);
#pragma unroll
        for (int c = 0; c < 8; c++)
          h[c] = drop1(h[c], (uint8_t)(mk[c >> 2] >> (8 * (c & 3))), a.mscale);
        v = __builtin_bit_cast(u32x4, h);
      }
    }
    rows[e] = v;
  }
  for (int r0 = 0; r0 < r; r0 += 16) {
    half8_t av = {};
    if (mb < ldt) av = *reinterpret_cast<const half8_t*>(a.PT + (int64_t)(r0 + ln) * ldt + mb);
    float4_t acc[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
      half8_t b;
#pragma unroll
      for (int e = 0; e < 8; e++) b[e] = __builtin_bit_cast(half8_t, rows[e])[c];
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, (float4_t){0.f, 0.f, 0.f, 0.f}, 0,
                                                      0, 0);
    }
    // acc[c][v] = C[j = 4*lg + v][column nb + 8*ln + c]; wave 1 stores, wave 0 adds
    if (wave == 1) {
#pragma unroll
      for (int c = 0; c < 8; c++)
#pragma unroll
        for (int v = 0; v < 4; v++) red[4 * lg + v][8 * ln + c] = acc[c][v];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < 8; c++)
#pragma unroll
        for (int v = 0; v < 4; v++) red[4 * lg + v][8 * ln + c] += acc[c][v];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < 16 * 128; idx += 128) {
      const int i = idx >> 7, j = idx & 127;
      const int n = nb + j;
      if (n < a.Nq) a.ws[((int64_t)mblk * r + r0 + i) * a.Nq + n] = red[i][j];
    }
    __syncthreads();
  }
}

// out = sum over token blocks of ws, laid out [r, Nq] (out_rn) or [Nq, r]; problem blockIdx.y.
__global__ __launch_bounds__(256) void k_lora_cols_finish(ColsProblem p0, ColsProblem p1,
                                                         int blocks, int r) {
  const ColsProblem a = blockIdx.y == 0 ? p0 : p1;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= r * a.Nq) return;
  const int j = idx / a.Nq, n = idx % a.Nq;
  float sum = 0.f;
  for (int z = 0; z < blocks; z++) sum += a.ws[((int64_t)z * r + j) * a.Nq + n];
  if (a.out_rn) a.out[(int64_t)j * a.Nq + n] = sum;
  else a.out[(int64_t)n * r + j] = sum;
}

// dst[0, n) = 0 (a kernel, not hipMemsetAsync, so that the call can be captured in a graph).
__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = 0.f;
}

static int zero_f32(float* dst, int64_t n, hipStream_t stream) {
  if (n <= 0) return MXS_OK;
  hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, dst, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

// dst [cols, rows] = src [rows, cols]^T (fp16).
__global__ __launch_bounds__(256) void k_transpose_f16(const _Float16* __restrict__ src,
                                                      int rows, int cols,
                                                      _Float16* __restrict__ dst) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)rows * cols) return;
  const int c = (int)(idx / rows), rr = (int)(idx % rows);
  dst[idx] = src[(int64_t)rr * cols + c];
}

static int check_launch() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

static int64_t rows_ws_bytes(int K, int ldt, int r) {
  return (int64_t)rows_slices(K) * ldt * r * (int64_t)sizeof(float);
}

static int64_t cols_ws_bytes(int M, int N, int r) {
  const int blocks = (M + kColsRows - 1) / kColsRows;
  return (int64_t)blocks * r * N * (int64_t)sizeof(float);
}

static int rows_launch(RowsArgs a, void* workspace, hipStream_t stream) {
  a.ws = static_cast<float*>(workspace);
  const int slices = rows_slices(a.K);
  hipLaunchKernelGGL(k_lora_rows, dim3((a.ldt + 15) / 16, slices), dim3(64 * kRowsWaves), 0,
                     stream, a);
  hipLaunchKernelGGL(k_lora_rows_finish, dim3((a.ldt * a.r + 255) / 256), dim3(256), 0, stream, a,
                     slices);
  return check_launch();
}

// Partial and finish launches for one or two cols problems (p1 ignored when nprob == 1).
static int cols_launch(ColsProblem p0, ColsProblem p1, int nprob, int M, int ldt, int r,
                       void* workspace, hipStream_t stream) {
  const int blocks = (M + kColsRows - 1) / kColsRows;
  const int cb0 = (p0.Nq + 127) / 128, cb1 = nprob > 1 ? (p1.Nq + 127) / 128 : 0;
  p0.ws = static_cast<float*>(workspace);
  if (nprob > 1) {
    p1.ws = p0.ws + (int64_t)blocks * r * p0.Nq;
  } else {
    p1 = p0;
  }
  hipLaunchKernelGGL(k_lora_cols, dim3(cb0 > cb1 ? cb0 : cb1, blocks, nprob), dim3(128), 0,
                     stream, p0, p1, M, ldt, r);
  const int nmax = p0.Nq > p1.Nq ? p0.Nq : p1.Nq;
  hipLaunchKernelGGL(k_lora_cols_finish, dim3((r * nmax + 255) / 256, nprob), dim3(256), 0, stream,
                     p0, p1, blocks, r);
  return check_launch();
}

}  // namespace mxs

using namespace mxs;

extern "C" {

int64_t mxs_lora_workspace_bytes(int M, int K, int N, int r) {
  const int ldt = (M + 7) / 8 * 8;
  int64_t b = rows_ws_bytes(K, ldt, r);
  const int64_t b2 = rows_ws_bytes(N, ldt, r);
  if (b2 > b) b = b2;
  const int64_t c = cols_ws_bytes(M, K, r) + cols_ws_bytes(M, N, r);
  if (c > b) b = c;
  return b;
}

int mxs_lora_h(const void* x, int M, int K, const void* lora_a, int r, const void* mask,
               float mask_scale, float s, void* h, void* ht, int ldt, void* at, void* workspace,
               hipStream_t stream) {
  if (M < 0 || K < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!x || !lora_a || !h || !ht || !workspace) return MXS_ERR_ARG;
  if (r % 16 || K % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)x % 16) || ((uintptr_t)lora_a % 16) || (mask && ((uintptr_t)mask % 8)))
    return MXS_ERR_ALIGN;
  RowsArgs a{};
  a.P = static_cast<const _Float16*>(x);
  a.M = M;
  a.K = K;
  a.mask = static_cast<const uint8_t*>(mask);
  a.mscale = mask_scale;
  a.R = static_cast<const _Float16*>(lora_a);
  a.rs_r = K;
  a.rs_k = 1;
  a.r = r;
  a.ldt = ldt;
  a.s = s;
  a.out = static_cast<_Float16*>(h);
  a.outT = static_cast<_Float16*>(ht);
  a.rt = static_cast<_Float16*>(at);
  return rows_launch(a, workspace, stream);
}

int mxs_lora_dh(const void* dy, int M, int N, const void* lora_b, int r, float s, void* dh,
                void* dht, int ldt, void* workspace, hipStream_t stream) {
  if (M < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!dy || !lora_b || !dh || !dht || !workspace) return MXS_ERR_ARG;
  if (r % 16 || N % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if ((uintptr_t)dy % 16) return MXS_ERR_ALIGN;
  RowsArgs a{};
  a.P = static_cast<const _Float16*>(dy);
  a.M = M;
  a.K = N;
  a.mscale = 1.0f;
  a.R = static_cast<const _Float16*>(lora_b);
  a.rs_r = 1;
  a.rs_k = r;
  a.r = r;
  a.ldt = ldt;
  a.s = s;
  a.out = static_cast<_Float16*>(dh);
  a.outT = static_cast<_Float16*>(dht);
  return rows_launch(a, workspace, stream);
}

int mxs_lora_grads(const void* dht, const void* ht, int ldt, const void* x, const void* dy, int M,
                   int K, int N, int r, const void* mask, float mask_scale, float* da, float* db,
                   void* workspace, hipStream_t stream) {
  if (M < 0 || K < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (!da && !db) return MXS_ERR_ARG;
  if (M == 0) {  // empty reduction: zero gradients
    const int e = da ? zero_f32(da, (int64_t)r * K, stream) : MXS_OK;
    if (e != MXS_OK) return e;
    return db ? zero_f32(db, (int64_t)N * r, stream) : MXS_OK;
  }
  if ((da && (!dht || !x)) || (db && (!ht || !dy)) || !workspace) return MXS_ERR_ARG;
  if (r % 16 || K % 8 || N % 8 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if ((x && ((uintptr_t)x % 16)) || (dy && ((uintptr_t)dy % 16)) ||
      (mask && ((uintptr_t)mask % 8)) || (dht && ((uintptr_t)dht % 16)) ||
      (ht && ((uintptr_t)ht % 16)))
    return MXS_ERR_ALIGN;
  ColsProblem pa{}, pb{};
  pa.PT = static_cast<const _Float16*>(dht);
  pa.Q = static_cast<const _Float16*>(x);
  pa.mask = static_cast<const uint8_t*>(mask);
  pa.mscale = mask_scale;
  pa.Nq = K;
  pa.out = da;
  pa.out_rn = 1;
  pb.PT = static_cast<const _Float16*>(ht);
  pb.Q = static_cast<const _Float16*>(dy);
  pb.mscale = 1.0f;
  pb.Nq = N;
  pb.out = db;
  pb.out_rn = 0;
  const bool a_on = da && K > 0, b_on = db && N > 0;
  if (a_on && b_on) return cols_launch(pa, pb, 2, M, ldt, r, workspace, stream);
  if (a_on) return cols_launch(pa, pa, 1, M, ldt, r, workspace, stream);
  if (b_on) return cols_launch(pb, pb, 1, M, ldt, r, workspace, stream);
  return MXS_OK;
}

int mxs_lora_grad_a(const void* dht, int ldt, const void* x, int M, int K, int r,
                    const void* mask, float mask_scale, float* da, void* workspace,
                    hipStream_t stream) {
  return mxs_lora_grads(dht, nullptr, ldt, x, nullptr, M, K, 0, r, mask, mask_scale, da, nullptr,
                        workspace, stream);
}

int mxs_lora_grad_b(const void* ht, int ldt, const void* dy, int M, int N, int r, float* db,
                    void* workspace, hipStream_t stream) {
  return mxs_lora_grads(nullptr, ht, ldt, nullptr, dy, M, 0, N, r, nullptr, 1.0f, nullptr, db,
                        workspace, stream);
}

int mxs_transpose_f16(const void* src, int rows, int cols, void* dst, hipStream_t stream) {
  if (rows < 0 || cols < 0) return MXS_ERR_ARG;
  const int64_t total = (int64_t)rows * cols;
  if (total == 0) return MXS_OK;
  if (!src || !dst) return MXS_ERR_ARG;
  hipLaunchKernelGGL(k_transpose_f16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     stream, static_cast<const _Float16*>(src), rows, cols,
                     static_cast<_Float16*>(dst));
  return check_launch();
}

}  // extern "C"
