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
// These products are thin (r = 16) and read a few MB each; each is ONE launch with no partial
// sums in memory: a workgroup owns a block of output rows (Hs, dHs: 16 tokens) or columns
// (dA, dB: 32-128 columns) and splits the reduction over up to 16 waves, which add their
// v_mfma_f32_16x16x32_f16 accumulators in LDS in a fixed order (deterministic).  Summing partials
// across workgroups would need a second launch or agent-scope fences (on the multi-XCD gfx950,
// write-back and invalidation of whole L2s): both measured slower than these kernels.
//   rows kernel: lane (row l%16, k-group l/16) loads 16-byte fragments of X (plus a keep byte)
//     and of the r x K operand (lora_A, or lora_B transposed), four 32-wide chunks in flight.
//   cols kernel: each lane loads an 8-token x CPL-column block of the row-major fp16 input and
//     regroups it in registers into CPL MFMA operands (one per column), so a wave covers 16*CPL
//     columns per 32-token step without a transpose in memory; dA and dB share one grid.
//   The forward rows kernel also writes lora_A^T [K, r] and lora_B^T [r, N] for the backward
//     (the dX epilogue's operand and the dHs kernel's operand), spread over its workgroups.
#include "common.h"
#include "lora_cols.h"
#include "mxs_nf4.h"

namespace mxs {

constexpr int kMaxRB = 8;            // r <= 128 (r / 16 accumulator blocks)

// 32-wide reduction chunks each wave of the rows kernel loads per iteration: 4 with one 16-row
// block per workgroup, 3 with two (their loads share one register budget).
template <int TB>
constexpr int rows_chunks_in_flight() { return TB == 1 ? 4 : 3; }

// 8 consecutive values through the dropout: bit e of `keep` set keeps value e (times scale).
// R2: each product rounded to fp32 and then to fp16 (scale_round2), else in one mixed-precision
// FMA (where that is the same: round_once_exact).
template <bool R2>
__device__ __forceinline__ half8_t drop8(half8_t x, uint32_t keep, float scale) {
#pragma unroll
  for (int e = 0; e < 8; e++)
    x[e] = ((keep >> e) & 1u) ? (R2 ? scale_round2(x[e], scale) : (_Float16)((float)x[e] * scale))
                              : (_Float16)0.0f;
  return x;
}

struct RowsArgs {
  const _Float16* P;      // [M, K] row-major
  int M, K;
  const uint8_t* mask;    // keep bits of [M, K] (keep_row_bytes(K) per row) or null
  float mscale;
  int round2;             // dropout rounded twice (round_once_exact(mscale) is false)
  const _Float16* R;      // [r, K] row-major
  int r, ldt;
  float s;
  _Float16* out;          // [M, r]
  _Float16* outT;         // [r, ldt], zeros past M
  _Float16* rt;           // optional [K, r] = R^T
  const _Float16* B;      // optional [N, r]; with bt, bt [r, N] = B^T
  int N;
  _Float16* bt;
  float* ws;              // fp32 partials [slices][ldt][r], times s (sliced or partial mode)
  int partial_out;        // write the partials even for one slice; no final fp16 outputs
  // fp32 LoRA weights (the rows kernel's W32 form): R32 [r, K] and B32 [N, r] are read in place
  // of R / B and rounded to fp16 (nearest even) where they are used, so the results are those of
  // R and B cast first; b16 (optional) receives that fp16 copy of B [N, r].
  const float* R32;
  const float* B32;
  _Float16* b16;
};

// 8 consecutive fp32 weights rounded to fp16 (round to nearest even, as a cast would).
__device__ __forceinline__ half8_t f32x8_to_f16(const float* p) {
  const float4_t lo = *reinterpret_cast<const float4_t*>(p);
  const float4_t hi = *reinterpret_cast<const float4_t*>(p + 4);
  half8_t h;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    h[e] = (_Float16)lo[e];
    h[4 + e] = (_Float16)hi[e];
  }
  return h;
}

// out[m][c] = fp16(s * sum_k drop(P)[m][k] * R[c][k]) for the 16*TB rows of row block rb, over
// reduction slice `slice` of `slices`.  Waves [0, nw) reduce; any waves past nw (a grouped
// launch sized for another problem) only take part in the barrier and the stores, so the result
// is the same bits as a launch of exactly nw waves.  wg of n_wg places the side outputs.
// W32: the weights come as fp32 (R32, B32).  TB: 16-row blocks per workgroup; each R fragment
// a wave loads feeds TB multiplies, so TB = 2 halves the re-reads of R (every row block reads
// all of its slice of R).  Wave w takes chunks c_beg + w, c_beg + w + nw, ... and adds them in
// that order whatever TB, so TB does not change the bits.  RB: the accumulator blocks compiled in
// (1 for r = 16, kMaxRB for any r up to 128).  MASK: a.mask is set (the dropout applies).  R2:
// the dropout rounds twice (a kernel of its own, so that the other keeps its registers).
template <bool W32, int TB, int RB, bool MASK, bool R2>
__device__ __forceinline__ void rows_block(const RowsArgs& a, int rb, int slice, int slices,
                                           int nw, int wg, int n_wg, float* red) {
  constexpr int CIF = rows_chunks_in_flight<TB>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: chunk tests below
  const int m0 = rb * 16 * TB;
  const int g = lane >> 4;
  const int rbn = a.r >> 4;
  const int chunks = a.K >> 5;
  // reduction slice of this workgroup: chunks [c_beg, c_end)
  const int cps = (chunks + slices - 1) / slices;
  const int c_beg = slice * cps;
  const int c_end = min(chunks, c_beg + cps);
  bool row_ok[TB];
  int64_t prow[TB], krow[TB];  // the lane's first value and its keep byte (chunk 0)
#pragma unroll
  for (int t = 0; t < TB; t++) {
    const int row = m0 + 16 * t + (lane & 15);
    row_ok[t] = row < a.M;
    prow[t] = (int64_t)(row_ok[t] ? row : 0) * a.K + 8 * g;
    krow[t] = (int64_t)(row_ok[t] ? row : 0) * keep_row_bytes(a.K) + g;
  }
  float4_t acc[TB][RB];
#pragma unroll
  for (int t = 0; t < TB; t++)
#pragma unroll
    for (int b = 0; b < RB; b++) acc[t][b] = (float4_t){0.f, 0.f, 0.f, 0.f};
  for (int c0 = c_beg + wave; wave < nw && c0 < c_end; c0 += CIF * nw) {
    // A batch's loads come first, each chunk's under its own wave-uniform test (rows past M are
    // clamped to row 0 and zeroed after), and nothing uses a loaded value before the last load:
    // one round trip per batch.  (A chunk's dropout right after its own load split the batch
    // into a round trip per chunk.)
    half8_t x[CIF][TB], y[CIF];
    uint32_t kb[CIF][TB];
    auto load_r = [&](int b) {
      const int64_t roff = (int64_t)(16 * b + (lane & 15)) * a.K + 8 * g;
#pragma unroll
      for (int u = 0; u < CIF; u++) {
        const int c = c0 + u * nw;
        y[u] = (half8_t){};
        if (c < c_end) {
          if constexpr (W32)
            y[u] = f32x8_to_f16(a.R32 + roff + 32 * c);
          else
            y[u] = *reinterpret_cast<const half8_t*>(a.R + roff + 32 * c);
        }
      }
    };
#pragma unroll
    for (int u = 0; u < CIF; u++) {
      const int c = c0 + u * nw;
#pragma unroll
      for (int t = 0; t < TB; t++) {
        x[u][t] = (half8_t){};
        kb[u][t] = 0;
        if (c < c_end) {
          x[u][t] = *reinterpret_cast<const half8_t*>(a.P + prow[t] + 32 * c);
          if constexpr (MASK) kb[u][t] = a.mask[krow[t] + 4 * c];
        }
      }
    }
    load_r(0);
#pragma unroll
    for (int u = 0; u < CIF; u++)
#pragma unroll
      for (int t = 0; t < TB; t++) {
        half8_t v = x[u][t];
        if constexpr (MASK) v = drop8<R2>(v, kb[u][t], a.mscale);
        x[u][t] = row_ok[t] ? v : (half8_t){};
      }
#pragma unroll
    for (int b = 0; b < RB; b++) {
      if (b >= rbn) break;
      if (b > 0) load_r(b);
#pragma unroll
      for (int u = 0; u < CIF; u++)
#pragma unroll
        for (int t = 0; t < TB; t++)
          acc[t][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[u][t], y[u], acc[t][b], 0, 0, 0);
    }
  }
  // acc[t][b][v] = C[row 16*t + 4*g + v][column 16*b + lane%16]
  const int ld = a.r + 1;
#pragma unroll
  for (int b = 0; b < RB; b++) {
    if (b >= rbn || wave >= nw) break;
#pragma unroll
    for (int t = 0; t < TB; t++)
#pragma unroll
      for (int v = 0; v < 4; v++)
        red[(wave * 16 * TB + 16 * t + 4 * g + v) * ld + 16 * b + (lane & 15)] = acc[t][b][v];
  }
  // side outputs, spread over the workgroups: R^T [K, r], B^T [r, N] and (W32) fp16 B [N, r]
  if (a.rt) {
    const int span = ((a.K + n_wg - 1) / n_wg + 7) & ~7;
    const int k_beg = wg * span, k_end = min(a.K, k_beg + span);
    for (int i = threadIdx.x; i < (k_end - k_beg) * a.r; i += blockDim.x) {
      const int k = k_beg + i / a.r, c = i % a.r;
      if constexpr (W32)
        a.rt[(int64_t)k * a.r + c] = (_Float16)a.R32[(int64_t)c * a.K + k];
      else
        a.rt[(int64_t)k * a.r + c] = a.R[(int64_t)c * a.K + k];
    }
  }
  if (a.bt || (W32 && a.b16)) {
    const int span = ((a.N + n_wg - 1) / n_wg + 7) & ~7;
    const int n_beg = wg * span, n_end = min(a.N, n_beg + span);
    for (int i = threadIdx.x; i < (n_end - n_beg) * a.r; i += blockDim.x) {
      const int n = n_beg + i / a.r, c = i % a.r;
      const int64_t src = (int64_t)n * a.r + c;
      _Float16 v;
      if constexpr (W32) {
        v = (_Float16)a.B32[src];
        if (a.b16) a.b16[src] = v;
      } else {
        v = a.B[src];
      }
      if (a.bt) a.bt[(int64_t)c * a.N + n] = v;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 16 * TB * a.r; i += blockDim.x) {
    // consecutive threads: consecutive m of one outT row
    const int c = i / (16 * TB), rr = i % (16 * TB);
    const int m = m0 + rr;
    if (m >= a.ldt) continue;
    float sum = 0.f;
    for (int w = 0; w < nw; w++) sum += red[(w * 16 * TB + rr) * ld + c];
    if (slices > 1 || a.partial_out) {  // this slice's partial, times s
      a.ws[((int64_t)slice * a.ldt + m) * a.r + c] = a.s * sum;
      continue;
    }
    const _Float16 h = m < a.M ? (_Float16)(a.s * sum) : (_Float16)0.0f;
    if (m < a.M) a.out[(int64_t)m * a.r + c] = h;
    a.outT[(int64_t)c * a.ldt + m] = h;
  }
}

template <int TB, int RB, bool R2>
__global__ __launch_bounds__(1024) void k_lora_rows(RowsArgs a) {
  extern __shared__ float red[];  // [waves][16 * TB][r + 1]
  const int wg = (int)(blockIdx.y * gridDim.x + blockIdx.x), n_wg = (int)(gridDim.x * gridDim.y);
  if (a.mask)
    rows_block<false, TB, RB, true, R2>(a, (int)blockIdx.x, (int)blockIdx.y, (int)gridDim.y,
                                        (int)blockDim.x >> 6, wg, n_wg, red);
  else
    rows_block<false, TB, RB, false, false>(a, (int)blockIdx.x, (int)blockIdx.y, (int)gridDim.y,
                                            (int)blockDim.x >> 6, wg, n_wg, red);
}

// Several rows problems over the same tokens in one launch (the q/k/v or gate/up projections
// share their input; their output gradients arrive together): problem i owns workgroups
// [start[i], start[i+1]), laid out as its own launch's grid, with its own slices and waves.
constexpr int kMaxGroup = 4;
struct RowsGroup {
  RowsArgs p[kMaxGroup];
  int start[kMaxGroup + 1];
  int rbs[kMaxGroup], slices[kMaxGroup], nw[kMaxGroup];  // rbs: blocks of 16 * TB rows
  int n;
};

template <bool W32, int TB, int RB, bool R2>
__global__ __launch_bounds__(1024) void k_lora_rows_group(RowsGroup g) {
  extern __shared__ float red[];  // [waves][16 * TB][r + 1]
  const int bid = (int)blockIdx.x;
  int i = 0;
  while (i + 1 < g.n && bid >= g.start[i + 1]) i++;
  const int local = bid - g.start[i];
  if (g.p[i].mask)
    rows_block<W32, TB, RB, true, R2>(g.p[i], local % g.rbs[i], local / g.rbs[i], g.slices[i],
                                  g.nw[i], local, g.start[i + 1] - g.start[i], red);
  else
    rows_block<W32, TB, RB, false, false>(g.p[i], local % g.rbs[i], local / g.rbs[i], g.slices[i],
                                   g.nw[i], local, g.start[i + 1] - g.start[i], red);
}

// out[m][c] = fp16(sum of the slices' partials, in slice order) for m < M; outT [r, ldt]
// with zeros past M.  One thread per row m: its partials and its out row are contiguous, and
// consecutive threads write consecutive m of each outT row.
__global__ __launch_bounds__(64) void k_lora_rows_finish(RowsArgs a, int slices) {
  const int m = blockIdx.x * 64 + threadIdx.x;
  if (m >= a.ldt) return;
  for (int c0 = 0; c0 < a.r; c0 += 16) {
    float4_t v[4][4];  // [slice][quad of columns]; all loads before the first add
#pragma unroll
    for (int z = 0; z < 4; z++)
#pragma unroll
      for (int q = 0; q < 4; q++)
        v[z][q] = z < slices
                      ? *reinterpret_cast<const float4_t*>(a.ws + ((int64_t)z * a.ldt + m) * a.r + c0 + 4 * q)
                      : (float4_t){0.f, 0.f, 0.f, 0.f};
    half8_t h[2];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float4_t sum = v[0][q];
#pragma unroll
      for (int z = 1; z < 4; z++)
        if (z < slices) sum += v[z][q];
#pragma unroll
      for (int e = 0; e < 4; e++)
        h[q >> 1][4 * (q & 1) + e] = m < a.M ? (_Float16)sum[e] : (_Float16)0.0f;
    }
    if (m < a.M && a.out) {
      *reinterpret_cast<half8_t*>(a.out + (int64_t)m * a.r + c0) = h[0];
      *reinterpret_cast<half8_t*>(a.out + (int64_t)m * a.r + c0 + 8) = h[1];
    }
#pragma unroll
    for (int c = 0; c < 16; c++) a.outT[(int64_t)(c0 + c) * a.ldt + m] = h[c >> 3][c & 7];
  }
}




template <int CPL>
__global__ __launch_bounds__(64 * cols_max_waves<CPL>()) void k_lora_cols(ColsProblem p0, ColsProblem p1, int cb0, int M,
                                                   int ldt, int r) {
  extern __shared__ float red[];  // [waves][r][16 * CPL + 1]
  lora_cols_block<CPL>(p0, p1, cb0, M, ldt, r, (int)blockIdx.x, (int)blockDim.x >> 6, red);
}

// dA / dB of several projections in one launch (ColsGroup).
template <int CPL>
__global__ __launch_bounds__(64 * cols_max_waves<CPL>()) void k_lora_cols_group(ColsGroup g, int M,
                                                                               int ldt, int r) {
  extern __shared__ float red[];  // [waves][r][16 * CPL + 1]
  lora_cols_group_block<CPL>(g, M, ldt, r, (int)blockIdx.x, (int)blockDim.x >> 6, red);
}

// Keep bits from a byte keep mask [M, K] (nonzero = kept; the reference's int8 `keep`): one
// thread per 32-bit word, its 32 source bytes contiguous, consecutive threads' words contiguous.
__global__ __launch_bounds__(256) void k_keep_pack(const uint8_t* __restrict__ keep, int M, int K,
                                                  uint32_t* __restrict__ bits) {
  const int kw = keep_words(K);
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * kw) return;
  const int m = (int)(i / kw), w = (int)(i % kw);
  const uint8_t* src = keep + (int64_t)m * K + 32 * w;
  const int n = min(32, K - 32 * w);
  uint32_t v = 0;
  if (n == 32 && ((uintptr_t)src % 16) == 0) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(src);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(src + 16);
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v |= (((lo[d] >> (8 * e)) & 0xffu) ? 1u : 0u) << (4 * d + e);
        v |= (((hi[d] >> (8 * e)) & 0xffu) ? 1u : 0u) << (16 + 4 * d + e);
      }
  } else {
    for (int e = 0; e < n; e++) v |= (src[e] ? 1u : 0u) << e;
  }
  bits[i] = v;
}

// dst[0, n) = 0 (a kernel, not hipMemsetAsync, so that the call can be captured in a graph).
__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = 0.f;
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

static int zero_f32(float* dst, int64_t n, hipStream_t stream) {
  if (n <= 0) return MXS_OK;
  hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, dst, n);
  return check_launch();
}

// Waves for a reduction of `steps` units: about three units per wave, 4..16 waves.
static int waves_for(int steps) {
  int w = (steps + 2) / 3;
  return w < 4 ? 4 : w > kMaxWaves ? kMaxWaves : w;
}

// Reduction slices for the rows kernel: one (a single launch) unless the reduction is long
// (>= 1024) and a workspace is given; then enough slices for about 256 workgroups, at most 4.
static int rows_slices(int K, int ldt) {
  if (K < 1024) return 1;
  const int row_blocks = (ldt + 15) / 16;
  int sl = 256 / row_blocks;
  return sl < 1 ? 1 : sl > 4 ? 4 : sl;
}

// Slices and waves of one rows problem.  The workspace size query assumes ldt = M rounded up
// to 8; any other ldt runs unsliced.  In partial mode the caller sized the partials by
// mxs_lora_slices(M, K) for its ldt.
static void rows_plan(const RowsArgs& a, bool have_ws, int* slices, int* nw) {
  const bool ws_ok = have_ws && (a.partial_out || a.ldt == (a.M + 7) / 8 * 8);
  *slices = ws_ok ? rows_slices(a.K, (a.M + 7) / 8 * 8) : 1;
  int w = waves_for(a.K / 32 / *slices);
  while (w > 1 && (size_t)w * 16 * (a.r + 1) * sizeof(float) > (size_t)kColsLds) w--;
  *nw = w;
}

// 16-row blocks per rows workgroup: two where r = 16 and the launch still has at least 256
// workgroups and 16 waves per CU with them (each R fragment then feeds two multiplies; measured
// at 1024 tokens: gate/up's dHs over N = 8960, 256 workgroups of 16 waves, 14.8 -> 12.4 us,
// while the short reductions of K = 1536, 4 waves per workgroup, got slower), else one.  The
// choice does not change the bits (rows_block).
static int rows_tb(int r, int64_t workgroups_at_two, int64_t waves_at_two) {
  return r == 16 && workgroups_at_two >= 256 && waves_at_two >= 16 * 256 ? 2 : 1;
}

// The row-product kernel with the dropout rounding the launch needs: twice (R2) where some
// problem has a keep mask and rounding once is not the same for its scale.
static bool rows_round2(const RowsArgs& a) { return a.mask && !round_once_exact(a.mscale); }

template <int TB, int RB>
static void launch_rows_k(bool r2, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                          const RowsArgs& a) {
  if (r2)
    hipLaunchKernelGGL((k_lora_rows<TB, RB, true>), grid, block, lds, stream, a);
  else
    hipLaunchKernelGGL((k_lora_rows<TB, RB, false>), grid, block, lds, stream, a);
}

template <bool W32, int TB, int RB>
static void launch_rows_group_k(bool r2, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                                const RowsGroup& g) {
  if (r2)
    hipLaunchKernelGGL((k_lora_rows_group<W32, TB, RB, true>), grid, block, lds, stream, g);
  else
    hipLaunchKernelGGL((k_lora_rows_group<W32, TB, RB, false>), grid, block, lds, stream, g);
}

static int rows_launch(RowsArgs a, void* workspace, hipStream_t stream) {
  int slices, nw;
  rows_plan(a, workspace != nullptr, &slices, &nw);
  a.ws = static_cast<float*>(workspace);
  const int64_t at_two = (int64_t)((a.ldt + 31) / 32) * slices;
  const int tb = rows_tb(a.r, at_two, at_two * nw);
  const size_t lds = (size_t)nw * 16 * tb * (a.r + 1) * sizeof(float);
  const dim3 grid((a.ldt + 16 * tb - 1) / (16 * tb), slices);
  const bool r2 = rows_round2(a);
  if (a.r != 16)
    launch_rows_k<1, kMaxRB>(r2, grid, dim3(64 * nw), lds, stream, a);
  else if (tb == 2)
    launch_rows_k<2, 1>(r2, grid, dim3(64 * nw), lds, stream, a);
  else
    launch_rows_k<1, 1>(r2, grid, dim3(64 * nw), lds, stream, a);
  if (slices > 1 && !a.partial_out)
    hipLaunchKernelGGL(k_lora_rows_finish, dim3((a.ldt + 63) / 64), dim3(64), 0, stream, a,
                       slices);
  return check_launch();
}

// One launch for n rows problems: partial mode (a.ws = the problem's partials, sliced as a
// single launch with that workspace would be) or finished mode (a.ws null: one slice, fp16
// out / outT), each as its own launch would run.  w32: every problem's weights are fp32.
static int rows_group_launch(const RowsArgs* probs, int n, hipStream_t stream, bool w32 = false) {
  if (n < 1 || n > kMaxGroup) return MXS_ERR_ARG;
  RowsGroup g{};
  g.n = n;
  int nw_max = 1;
  int64_t at_two = 0, waves_at_two = 0;
  const int r = probs[0].r;
  for (int i = 0; i < n; i++) {
    g.p[i] = probs[i];
    rows_plan(g.p[i], g.p[i].ws != nullptr, &g.slices[i], &g.nw[i]);
    const int64_t wgs = (int64_t)((g.p[i].ldt + 31) / 32) * g.slices[i];
    at_two += wgs;
    waves_at_two += wgs * g.nw[i];
    nw_max = g.nw[i] > nw_max ? g.nw[i] : nw_max;
  }
  const int tb = rows_tb(r, at_two, waves_at_two);
  int total = 0;
  for (int i = 0; i < n; i++) {
    g.rbs[i] = (g.p[i].ldt + 16 * tb - 1) / (16 * tb);
    g.start[i] = total;
    total += g.rbs[i] * g.slices[i];
  }
  g.start[n] = total;
  const size_t lds = (size_t)nw_max * 16 * tb * (r + 1) * sizeof(float);
  const dim3 grid(total), block(64 * nw_max);
  bool r2 = false;
  for (int i = 0; i < n; i++) r2 = r2 || rows_round2(g.p[i]);
  if (w32) {
    if (r != 16)
      launch_rows_group_k<true, 1, kMaxRB>(r2, grid, block, lds, stream, g);
    else if (tb == 2)
      launch_rows_group_k<true, 2, 1>(r2, grid, block, lds, stream, g);
    else
      launch_rows_group_k<true, 1, 1>(r2, grid, block, lds, stream, g);
  } else {
    if (r != 16)
      launch_rows_group_k<false, 1, kMaxRB>(r2, grid, block, lds, stream, g);
    else if (tb == 2)
      launch_rows_group_k<false, 2, 1>(r2, grid, block, lds, stream, g);
    else
      launch_rows_group_k<false, 1, 1>(r2, grid, block, lds, stream, g);
  }
  return check_launch();
}

template <int CPL>
static int cols_launch_t(const ColsProblem& p0, const ColsProblem& p1, int nprob, int M, int ldt,
                         int r, hipStream_t stream) {
  constexpr int WC = 16 * CPL;
  const int cb0 = (p0.Nq + WC - 1) / WC, cb1 = nprob > 1 ? (p1.Nq + WC - 1) / WC : 0;
  const int nw = cols_waves(M, r, CPL, cols_max_waves<CPL>());
  const int per_wave = r * (WC + 1) * (int)sizeof(float);
  if (nw * per_wave > kColsLds) return MXS_ERR_SIZE;
  hipLaunchKernelGGL(k_lora_cols<CPL>, dim3(cb0 + cb1), dim3(64 * nw), (size_t)nw * per_wave,
                     stream, p0, p1, cb0, M, ldt, r);
  return check_launch();
}

template <int CPL>
static int cols_group_launch_t(ColsGroup g, int M, int ldt, int r, hipStream_t stream) {
  constexpr int WC = 16 * CPL;
  const int total = cols_group_layout(g, CPL);
  const int nw = cols_waves(M, r, CPL, cols_max_waves<CPL>());
  const int per_wave = r * (WC + 1) * (int)sizeof(float);
  if (nw * per_wave > kColsLds) return MXS_ERR_SIZE;
  hipLaunchKernelGGL(k_lora_cols_group<CPL>, dim3(total), dim3(64 * nw), (size_t)nw * per_wave,
                     stream, g, M, ldt, r);
  return check_launch();
}

// One launch for one or two cols problems (p1 ignored when nprob == 1).  Columns per lane: the
// widest that still gives the launch enough workgroups.
static int cols_launch(const ColsProblem& p0, const ColsProblem& p1, int nprob, int M, int ldt,
                       int r, hipStream_t stream) {
  const int cpl = cols_cpl(p0.Nq + (nprob > 1 ? p1.Nq : 0));
  if (cpl == 8) return cols_launch_t<8>(p0, p1, nprob, M, ldt, r, stream);
  if (cpl == 4) return cols_launch_t<4>(p0, p1, nprob, M, ldt, r, stream);
  return cols_launch_t<2>(p0, p1, nprob, M, ldt, r, stream);
}

}  // namespace mxs

using namespace mxs;

extern "C" {

int mxs_keep_pack(const void* keep, int M, int K, void* bits, hipStream_t stream) {
  if (M < 0 || K < 0) return MXS_ERR_ARG;
  if ((int64_t)M * K == 0) return MXS_OK;
  if (!keep || !bits) return MXS_ERR_ARG;
  if ((uintptr_t)bits % 4) return MXS_ERR_ALIGN;
  const int64_t words = (int64_t)M * keep_words(K);
  hipLaunchKernelGGL(k_keep_pack, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(keep), M, K, static_cast<uint32_t*>(bits));
  return check_launch();
}

int64_t mxs_lora_workspace_bytes(int M, int K, int N, int r) {
  const int ldt = (M + 7) / 8 * 8;
  const int sk = rows_slices(K, ldt), sn = rows_slices(N, ldt);
  const int sl = sk > sn ? sk : sn;
  return sl > 1 ? (int64_t)sl * ldt * r * (int64_t)sizeof(float) : 0;
}

int mxs_lora_h(const void* x, int M, int K, const void* lora_a, int r, const void* mask,
               float mask_scale, float s, void* h, void* ht, int ldt, void* at,
               const void* lora_b, int N, void* bt, void* workspace, hipStream_t stream) {
  if (M < 0 || K < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!x || !lora_a || !h || !ht || (bt && !lora_b)) return MXS_ERR_ARG;
  if (r % 16 || r > 16 * kMaxRB || K % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)x % 16) || ((uintptr_t)lora_a % 16) || (mask && ((uintptr_t)mask % 4)))
    return MXS_ERR_ALIGN;
  RowsArgs a{};
  a.P = static_cast<const _Float16*>(x);
  a.M = M;
  a.K = K;
  a.mask = static_cast<const uint8_t*>(mask);
  a.mscale = mask_scale;
  a.R = static_cast<const _Float16*>(lora_a);
  a.r = r;
  a.ldt = ldt;
  a.s = s;
  a.out = static_cast<_Float16*>(h);
  a.outT = static_cast<_Float16*>(ht);
  a.rt = static_cast<_Float16*>(at);
  a.B = static_cast<const _Float16*>(lora_b);
  a.N = N;
  a.bt = static_cast<_Float16*>(bt);
  return rows_launch(a, workspace, stream);
}

int mxs_lora_dh(const void* dy, int M, int N, const void* lora_bt, int r, float s, void* dh,
                void* dht, int ldt, void* workspace, hipStream_t stream) {
  if (M < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!dy || !lora_bt || !dh || !dht) return MXS_ERR_ARG;
  if (r % 16 || r > 16 * kMaxRB || N % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)dy % 16) || ((uintptr_t)lora_bt % 16)) return MXS_ERR_ALIGN;
  RowsArgs a{};
  a.P = static_cast<const _Float16*>(dy);
  a.M = M;
  a.K = N;
  a.mscale = 1.0f;
  a.R = static_cast<const _Float16*>(lora_bt);
  a.r = r;
  a.ldt = ldt;
  a.s = s;
  a.out = static_cast<_Float16*>(dh);
  a.outT = static_cast<_Float16*>(dht);
  return rows_launch(a, workspace, stream);
}

int mxs_lora_slices(int M, int Kr) {
  if (M <= 0 || Kr <= 0) return 1;
  return rows_slices(Kr, (M + 7) / 8 * 8);
}

int mxs_lora_h_partials(const void* x, int M, int K, const void* lora_a, int r, const void* mask,
                        float mask_scale, float s, int ldt, void* at, const void* lora_b, int N,
                        void* bt, float* partials, hipStream_t stream) {
  if (M < 0 || K < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!x || !lora_a || !partials || (bt && !lora_b)) return MXS_ERR_ARG;
  if (r % 16 || r > 16 * kMaxRB || K % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)x % 16) || ((uintptr_t)lora_a % 16) || (mask && ((uintptr_t)mask % 4)))
    return MXS_ERR_ALIGN;
  RowsArgs a{};
  a.P = static_cast<const _Float16*>(x);
  a.M = M;
  a.K = K;
  a.mask = static_cast<const uint8_t*>(mask);
  a.mscale = mask_scale;
  a.R = static_cast<const _Float16*>(lora_a);
  a.r = r;
  a.ldt = ldt;
  a.s = s;
  a.rt = static_cast<_Float16*>(at);
  a.B = static_cast<const _Float16*>(lora_b);
  a.N = N;
  a.bt = static_cast<_Float16*>(bt);
  a.partial_out = 1;
  return rows_launch(a, partials, stream);
}

int mxs_lora_dh_partials(const void* dy, int M, int N, const void* lora_bt, int r, float s,
                         int ldt, float* partials, hipStream_t stream) {
  if (M < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!dy || !lora_bt || !partials) return MXS_ERR_ARG;
  if (r % 16 || r > 16 * kMaxRB || N % 32 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)dy % 16) || ((uintptr_t)lora_bt % 16)) return MXS_ERR_ALIGN;
  RowsArgs a{};
  a.P = static_cast<const _Float16*>(dy);
  a.M = M;
  a.K = N;
  a.mscale = 1.0f;
  a.R = static_cast<const _Float16*>(lora_bt);
  a.r = r;
  a.ldt = ldt;
  a.s = s;
  a.partial_out = 1;
  return rows_launch(a, partials, stream);
}

int mxs_lora_h_partials_group(int n, const void* const x[], int M, const int K[],
                              const void* const lora_a[], int r, const void* const mask[],
                              float mask_scale, float s, int ldt, void* const at[],
                              const void* const lora_b[], const int N[], void* const bt[],
                              float* const partials[], hipStream_t stream) {
  if (n < 1 || n > kMaxGroup || M < 0 || r <= 0 || !x || !K || !lora_a || !partials)
    return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (r % 16 || r > 16 * kMaxRB || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  RowsArgs probs[kMaxGroup];
  for (int i = 0; i < n; i++) {
    const void* mk = mask ? mask[i] : nullptr;
    void* at_i = at ? at[i] : nullptr;
    const void* b_i = lora_b ? lora_b[i] : nullptr;
    void* bt_i = bt ? bt[i] : nullptr;
    const int n_i = N ? N[i] : 0;
    if (K[i] < 0 || n_i < 0) return MXS_ERR_ARG;
    if (!x[i] || !lora_a[i] || !partials[i] || (bt_i && !b_i)) return MXS_ERR_ARG;
    if (K[i] % 32) return MXS_ERR_SIZE;
    if (((uintptr_t)x[i] % 16) || ((uintptr_t)lora_a[i] % 16) || (mk && ((uintptr_t)mk % 4)))
      return MXS_ERR_ALIGN;
    RowsArgs a{};
    a.P = static_cast<const _Float16*>(x[i]);
    a.M = M;
    a.K = K[i];
    a.mask = static_cast<const uint8_t*>(mk);
    a.mscale = mask_scale;
    a.R = static_cast<const _Float16*>(lora_a[i]);
    a.r = r;
    a.ldt = ldt;
    a.s = s;
    a.rt = static_cast<_Float16*>(at_i);
    a.B = static_cast<const _Float16*>(b_i);
    a.N = n_i;
    a.bt = static_cast<_Float16*>(bt_i);
    a.partial_out = 1;
    a.ws = partials[i];
    probs[i] = a;
  }
  return rows_group_launch(probs, n, stream);
}

int mxs_lora_h_partials_group_w32(int n, const void* const x[], int M, const int K[],
                                  const float* const lora_a[], int r, const void* const mask[],
                                  float mask_scale, float s, int ldt, void* const at[],
                                  const float* const lora_b[], const int N[], void* const bt[],
                                  void* const b16[], float* const partials[],
                                  hipStream_t stream) {
  if (n < 1 || n > kMaxGroup || M < 0 || r <= 0 || !x || !K || !lora_a || !partials)
    return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (r % 16 || r > 16 * kMaxRB || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  RowsArgs probs[kMaxGroup];
  for (int i = 0; i < n; i++) {
    const void* mk = mask ? mask[i] : nullptr;
    void* at_i = at ? at[i] : nullptr;
    const float* b_i = lora_b ? lora_b[i] : nullptr;
    void* bt_i = bt ? bt[i] : nullptr;
    void* b16_i = b16 ? b16[i] : nullptr;
    const int n_i = N ? N[i] : 0;
    if (K[i] < 0 || n_i < 0) return MXS_ERR_ARG;
    if (!x[i] || !lora_a[i] || !partials[i] || ((bt_i || b16_i) && !b_i)) return MXS_ERR_ARG;
    if (K[i] % 32) return MXS_ERR_SIZE;
    if (((uintptr_t)x[i] % 16) || ((uintptr_t)lora_a[i] % 16) || (mk && ((uintptr_t)mk % 4)))
      return MXS_ERR_ALIGN;
    RowsArgs a{};
    a.P = static_cast<const _Float16*>(x[i]);
    a.M = M;
    a.K = K[i];
    a.mask = static_cast<const uint8_t*>(mk);
    a.mscale = mask_scale;
    a.R32 = lora_a[i];
    a.r = r;
    a.ldt = ldt;
    a.s = s;
    a.rt = static_cast<_Float16*>(at_i);
    a.B32 = b_i;
    a.N = n_i;
    a.bt = static_cast<_Float16*>(bt_i);
    a.b16 = static_cast<_Float16*>(b16_i);
    a.partial_out = 1;
    a.ws = partials[i];
    probs[i] = a;
  }
  return rows_group_launch(probs, n, stream, true);
}

int mxs_lora_dh_partials_group(int n, const void* const dy[], int M, const int N[],
                               const void* const lora_bt[], int r, float s, int ldt,
                               float* const partials[], hipStream_t stream) {
  if (n < 1 || n > kMaxGroup || M < 0 || r <= 0 || !dy || !N || !lora_bt || !partials)
    return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (r % 16 || r > 16 * kMaxRB || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  RowsArgs probs[kMaxGroup];
  for (int i = 0; i < n; i++) {
    if (N[i] < 0 || !dy[i] || !lora_bt[i] || !partials[i]) return MXS_ERR_ARG;
    if (N[i] % 32) return MXS_ERR_SIZE;
    if (((uintptr_t)dy[i] % 16) || ((uintptr_t)lora_bt[i] % 16)) return MXS_ERR_ALIGN;
    RowsArgs a{};
    a.P = static_cast<const _Float16*>(dy[i]);
    a.M = M;
    a.K = N[i];
    a.mscale = 1.0f;
    a.R = static_cast<const _Float16*>(lora_bt[i]);
    a.r = r;
    a.ldt = ldt;
    a.s = s;
    a.partial_out = 1;
    a.ws = partials[i];
    probs[i] = a;
  }
  return rows_group_launch(probs, n, stream);
}

int mxs_lora_dh_group(int n, const void* const dy[], int M, const int N[],
                      const void* const lora_bt[], int r, float s, int ldt, void* const dh[],
                      void* const dht[], hipStream_t stream) {
  if (n < 1 || n > kMaxGroup || M < 0 || r <= 0 || !dy || !N || !lora_bt || !dh || !dht)
    return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (r % 16 || r > 16 * kMaxRB || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  RowsArgs probs[kMaxGroup];
  for (int i = 0; i < n; i++) {
    if (N[i] < 0 || !dy[i] || !lora_bt[i] || !dh[i] || !dht[i]) return MXS_ERR_ARG;
    if (N[i] % 32) return MXS_ERR_SIZE;
    if (((uintptr_t)dy[i] % 16) || ((uintptr_t)lora_bt[i] % 16)) return MXS_ERR_ALIGN;
    RowsArgs a{};
    a.P = static_cast<const _Float16*>(dy[i]);
    a.M = M;
    a.K = N[i];
    a.mscale = 1.0f;
    a.R = static_cast<const _Float16*>(lora_bt[i]);
    a.r = r;
    a.ldt = ldt;
    a.s = s;
    a.out = static_cast<_Float16*>(dh[i]);
    a.outT = static_cast<_Float16*>(dht[i]);
    probs[i] = a;
  }
  return rows_group_launch(probs, n, stream);
}

int mxs_lora_finish(const float* partials, int slices, int M, int r, int ldt, void* out,
                    void* outT, hipStream_t stream) {
  if (M < 0 || r <= 0 || slices < 1 || slices > 4) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!partials || !outT) return MXS_ERR_ARG;
  if (r % 16 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)partials % 16) || (out && ((uintptr_t)out % 16))) return MXS_ERR_ALIGN;
  RowsArgs a{};
  a.M = M;
  a.r = r;
  a.ldt = ldt;
  a.ws = const_cast<float*>(partials);
  a.out = static_cast<_Float16*>(out);
  a.outT = static_cast<_Float16*>(outT);
  hipLaunchKernelGGL(k_lora_rows_finish, dim3((ldt + 63) / 64), dim3(64), 0, stream, a, slices);
  return (int)hipGetLastError();
}

int mxs_lora_grads(const void* dht, const void* ht, int ldt, const void* x, const void* dy, int M,
                   int K, int N, int r, const void* mask, float mask_scale, float* da, float* db,
                   void* workspace, hipStream_t stream) {
  (void)workspace;
  if (M < 0 || K < 0 || N < 0 || r <= 0) return MXS_ERR_ARG;
  if (!da && !db) return MXS_ERR_ARG;
  if (r % 16 || r > 16 * kMaxRB) return MXS_ERR_SIZE;
  if (M == 0) {  // empty reduction: zero gradients
    const int e = da ? zero_f32(da, (int64_t)r * K, stream) : MXS_OK;
    if (e != MXS_OK) return e;
    return db ? zero_f32(db, (int64_t)N * r, stream) : MXS_OK;
  }
  if ((da && (!dht || !x)) || (db && (!ht || !dy))) return MXS_ERR_ARG;
  if ((da && K % 8) || (db && N % 8) || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if ((da && ((uintptr_t)x % 16 || (uintptr_t)dht % 16)) ||
      (db && ((uintptr_t)dy % 16 || (uintptr_t)ht % 16)) || (mask && ((uintptr_t)mask % 4)))
    return MXS_ERR_ALIGN;
  ColsProblem pa{}, pb{};
  pa.PT = static_cast<const _Float16*>(dht);
  pa.Q = static_cast<const _Float16*>(x);
  pa.mask = static_cast<const uint8_t*>(mask);
  pa.mscale = mask_scale;
  pa.round2 = mask && !round_once_exact(mask_scale);
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
  if (a_on && b_on) return cols_launch(pa, pb, 2, M, ldt, r, stream);
  if (a_on) return cols_launch(pa, pa, 1, M, ldt, r, stream);
  if (b_on) return cols_launch(pb, pb, 1, M, ldt, r, stream);
  return MXS_OK;
}

int mxs_lora_grads_group(int n, const void* const dht[], const void* const ht[], int ldt,
                         const void* const x[], const void* const dy[], int M, const int K[],
                         const int N[], int r, const void* const mask[], float mask_scale,
                         float* const da[], float* const db[], hipStream_t stream) {
  if (n < 1 || n > kMaxGroup || M < 0 || r <= 0 || !dht || !ht || !x || !dy || !K || !N || !da ||
      !db)
    return MXS_ERR_ARG;
  if (r % 16 || r > 16 * kMaxRB) return MXS_ERR_SIZE;
  if (M == 0) {  // empty reductions: zero gradients
    for (int i = 0; i < n; i++) {
      const int e = mxs_lora_grads(nullptr, nullptr, ldt, nullptr, nullptr, 0, K[i], N[i], r,
                                   nullptr, mask_scale, da[i], db[i], nullptr, stream);
      if (e != MXS_OK) return e;
    }
    return MXS_OK;
  }
  ColsGroup g{};
  g.n = n;
  const int cpl = cols_cpl(K[0] + N[0]);
  for (int i = 0; i < n; i++) {
    const int e = cols_group_set(g, i, dht[i], ht[i], ldt, x[i], dy[i], M, K[i], N[i],
                                 mask ? mask[i] : nullptr, mask_scale, da[i], db[i]);
    if (e != MXS_OK) return e;
    if (cols_cpl(K[i] + N[i]) != cpl) return MXS_ERR_SIZE;
  }
  if (cpl == 8) return cols_group_launch_t<8>(g, M, ldt, r, stream);
  if (cpl == 4) return cols_group_launch_t<4>(g, M, ldt, r, stream);
  return cols_group_launch_t<2>(g, M, ldt, r, stream);
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
