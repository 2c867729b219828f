// Fused NF4-dequant GEMMs for gfx950: the frozen Linear4bit forward and its input gradient.
//
//   forward  (solution/linear4bit.py:47-49):  Y[M,N]  = X[M,K] . W[N,K]^T  (+ bias) (+ LoRA)
//   backward (solution/linear4bit.py:51-57):  dX[M,K] = dY[M,N] . W[N,K]            (+ LoRA)
//
// Both are one kernel, C[M,Nc] = A[M,Kr] . B[Nc,Kr]^T with B decoded from NF4 on the fly:
//   forward:  B = W   (Nc = N, Kr = K; NF4 contiguous along B's reduction dim)
//   backward: B = W^T (Nc = K, Kr = N; NF4 contiguous along B's output dim)
// Each K-step of 64 reduction indices stages A (fp16, straight copy) and B (NF4 decoded to the
// exact fp16 the standalone dequant writes) into LDS, double buffered, and feeds
// v_mfma_f32_32x32x16_f16 with fp32 accumulation.  The NF4 bytes of the next K-step are loaded
// while the current one multiplies.  LDS rows are 64 fp16 (128 B) with the 16-byte segments
// XOR-swizzled by the row index, so MFMA operand reads and the tile writes are bank-conflict
// free.
//
// The accumulators start at bias + the LoRA term (one more MFMA per 32x32 tile with K = r; in
// the input gradient masked by the dropout keep mask), computed before the main loop; the
// epilogue stores fp16.  With split-K (gridDim.z > 1) each split writes fp32 partials and
// k_splitk_reduce sums them (split 0 carries bias and LoRA).
#include <atomic>
#include <functional>
#include <mutex>
#include <queue>
#include <type_traits>
#include <vector>

#include "common.h"
#include "lora_cols.h"
#include "swiglu.h"
#include "mxs_nf4.h"

namespace mxs {

constexpr int kBK = 64;           // reduction indices per K-step (one NF4 block in forward)

struct GemmArgs {
  const _Float16* A;        // [M, lda]
  int64_t lda;
  const uint8_t* packed;    // NF4 W [Nw, Kw] (Nw = out_features, Kw = in_features)
  const uint8_t* absmax8;
  const float* code;
  const float* absmax2;
  const float* offset;
  int M, Nc, Kr;            // C is [M, Nc], reduction Kr
  int Kw;                   // in_features (row length of W)
  // epilogue
  const _Float16* bias;     // [Nc] (forward) or null
  const _Float16* lora_h;   // [M, r]: s*H (forward) or s*dH (backward), or null
  const _Float16* lora_w;   // [Nc, r]: forward lora_B; backward lora_A transposed
  int r;
  const uint8_t* mask;      // backward: dropout keep bits of [M, Nc] (keep_words(Nc) per row) or null
  float mask_scale;         // 1 / (1 - p)
  // LoRA activations given as fp32 partial sums instead of lora_h: [hp_slices][ldt][r], already
  // times s; the GEMM adds them in slice order and rounds to fp16 (the same value lora_h holds)
  const float* lora_hp;
  int hp_slices;
  _Float16* lora_ht;        // optional out: that fp16 operand transposed, [r, ldt], zeros past M
  int ldt;
  _Float16* C;              // [M, ldc]
  int64_t ldc;
  float* ws;                // split-K partials [splits, M, Nc]
  int steps_per_split;
  int zf;                   // grid z of this problem's first split (0, or the second problem's
                            // first plane in a launch of two, k_nf4_gemm_ws_pair)
  int unsplit;              // one split although gridDim.z > 1 (the z planes are problems): fp16
                            // stores, no partials
  // backward: the LoRA gradients dA (cp0) and dB (cp1), computed by cols_blocks extra
  // workgroups of the same launch in grid rows past the GEMM's (0: none).  They depend on
  // nothing the GEMM tiles write, so they run on the CUs the tiles leave idle.
  ColsProblem cp0, cp1;
  int cols_blocks, cols_cb0, cols_ldt, cols_nw;  // cols_nw: waves summing (cols_waves)
  // SwiGLU of the MLP applied to the fp16 output tile (buffers [M, ldc] like C):
  //   glu 1 (up projection forward): C as usual, and glu_h = silu(glu_g) * C;
  //   glu 2 (down projection backward): the output is d(hidden) and is not stored; glu_g and
  //   glu_u (gate, up) are read and overwritten with d(gate) and d(up).
  int glu;
  _Float16* glu_g;
  _Float16* glu_u;
  _Float16* glu_h;
  // RoPE of attention's q / k on the fp16 output (forward, grouped launch; null: none): every
  // 128-column head rotated by the (cos, sin) row of the output row's position, row m being
  // token m % rope_T of sequence m / rope_T; cos / sin fp32 with unit stride along the head
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_cs_b, rope_cs_t;
  int rope_T;
};

// Column order of a RoPE tile: within each 128-column head, bits 5 and 6 of the column index
// swap.  A consumer wave's 32-column blocks j = 0 and 1 (tile columns c and c + 32 of its
// share) then hold head columns d and d + 64, the two halves one rotation pairs, in the same
// lane and accumulator element.  Applied to the tile's column coordinate wherever it addresses
// a column (the NF4 rows, lora_B's rows, the bias, the stores).
__device__ __forceinline__ int rope_col(int v) {
  return (v & ~96) | ((v & 32) << 1) | ((v & 64) >> 1);
}

// Columns per lane of the gradient workgroups inside the backward GEMM launch.
constexpr int kFusedColsCPL = 2;


// LDS offset (in halfs) of 16-byte segment `seg` (0..7) of row `row` in a [rows][64] tile.
// Physical segment = seg ^ ((row >> 1) & 7).  A 128-byte row is half of the 64 four-byte banks,
// so rows of one parity share banks: the MFMA operand reads (16 lanes = 16 consecutive rows, one
// segment) see 8 rows of each parity on 8 different segments, and the decoded-tile stores (16
// lanes = 8 consecutive rows, segments 4h + d or 2h + d) see each parity's rows on distinct
// segments too, so neither conflicts.
__device__ __forceinline__ int lds_off(int row, int seg) {
  return row * kBK + (((seg ^ (row >> 1)) & 7) << 3);
}

template <int BM, int BN, int WAVES_M, int WAVES_N_, bool BWD>
struct Tile {
  static constexpr int WAVES_N = WAVES_N_;
  static constexpr int NT = 64 * WAVES_M * WAVES_N;  // threads per workgroup
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int TM = WM / 32;               // 32x32 MFMA tiles per wave along M
  static constexpr int TN = WN / 32;
  static constexpr int A_ITEMS = BM * 8 / NT;      // 16-byte A segments per thread
  // B work items: forward (row, half) = 32 NF4 values; backward 4 W rows x 8 cols.  Handed to
  // threads 0..B_TOTAL-1 (B_TOTAL a multiple of 64, so whole waves take or skip them).
  static constexpr int B_TOTAL = BWD ? (BN / 8) * (kBK / 4) : BN * 2;
  static constexpr int B_ITEMS = (B_TOTAL + NT - 1) / NT;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile");
  static_assert(A_ITEMS >= 1 && BM * 8 % NT == 0, "A tile vs threads");
  static_assert(B_TOTAL % 64 == 0, "B items in whole waves");
  static constexpr int LDS_A = BM * kBK;            // halfs per buffer
  static constexpr int LDS_B = BN * kBK;
};

// Accumulator layout of one wave's TM x TN tiles of 32x32 at output rows mb.., columns nb...:
// the MFMAs take the W fragment as their first operand, so each tile is held transposed: lane l
// keeps row m = mb + 32i + l%32 and, in register group g (4 registers), the 4 consecutive
// columns n = nb + 32j + 8g + 4(l/32) .. +3.
//
// Accumulator start value: the terms that do not depend on the reduction: bias, and the LoRA
// term as one MFMA per tile per 16 ranks (masked by the dropout keep mask and scaled in the
// backward pass).  Only the first split of a split-K launch carries them; the others start at
// zero.  load() prefetches the bias of narrow tiles; the kernels call it before anything else so
// that it shares the first round trip to memory with the first tiles' loads.  finish() builds
// the accumulators.  The LoRA operands and the keep mask come either from LDS areas that the
// warp-specialized kernel's producers staged (`ls`: [rows][16] fp16 operand of the workgroup's
// rows then [cols][16] of lora_w, r = 16; `kls`: the workgroup's keep bits, row stride `kst`
// bytes, a 32-bit word per 32 columns)
// or straight from memory.
template <int TM, int TN, bool BWD, bool ROPE = false>
struct AccStart {
  // the bias is prefetched only for narrow wave tiles (register budget of the wide ones)
  static constexpr bool kBiasPre = !BWD && TN <= 2;
  half4_t bias[kBiasPre ? TN : 1][4];  // 4 bias values per register group
  bool swap = false;                   // ROPE kernels: the tile's columns in rope_col order

  // output column of tile column coordinate n
  __device__ __forceinline__ int col(int n) const {
    if constexpr (ROPE) return swap ? rope_col(n) : n;
    else return n;
  }

  __device__ static __forceinline__ half4_t load_bias(const GemmArgs& a, int n) {
    half4_t b;
    if (((uintptr_t)a.bias % 8) == 0 && n + 3 < a.Nc) {
      b = *reinterpret_cast<const half4_t*>(a.bias + n);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) b[e] = n + e < a.Nc ? a.bias[n + e] : (_Float16)0.0f;
    }
    return b;
  }

  __device__ __forceinline__ void load(const GemmArgs& a, int nb, int lseg) {
    if constexpr (kBiasPre) {
      if ((int)blockIdx.z == a.zf && a.bias) {
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int g = 0; g < 4; g++)
            bias[j][g] = load_bias(a, col(nb + j * 32 + 8 * g + 4 * lseg));
      }
    }
  }

  // start value of tile column j before the LoRA products: the bias (forward) or zero
  __device__ __forceinline__ float16_t base(const GemmArgs& a, int j, int nb, int lseg) const {
    float16_t c = {};
    if constexpr (!BWD) {
      if ((int)blockIdx.z == a.zf && a.bias) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
          half4_t b;
          if constexpr (kBiasPre) b = bias[j][g];
          else b = load_bias(a, col(nb + j * 32 + 8 * g + 4 * lseg));
#pragma unroll
          for (int e = 0; e < 4; e++) c[4 * g + e] = (float)b[e];
        }
      }
    }
    return c;
  }

  // LoRA operand (ranks r0..r0+15) of output row m, straight from memory: the fp16 operand, or
  // the fp32 partial sums added in slice order and rounded to fp16
  __device__ static __forceinline__ half8_t lora_row(const GemmArgs& a, int m, int r0, int lseg) {
    half8_t hf = {};
    if (m >= a.M) return hf;
    if (a.lora_hp) {
      float4_t q0[4], q1[4];  // all slices' loads before the first add (<= 4 slices)
#pragma unroll
      for (int z = 0; z < 4; z++) {
        const float* src = a.lora_hp + ((int64_t)z * a.ldt + m) * a.r + r0 + 8 * lseg;
        q0[z] = z < a.hp_slices ? *reinterpret_cast<const float4_t*>(src) : (float4_t){};
        q1[z] = z < a.hp_slices ? *reinterpret_cast<const float4_t*>(src + 4) : (float4_t){};
      }
      float4_t s0 = q0[0], s1 = q1[0];
#pragma unroll
      for (int z = 1; z < 4; z++)
        if (z < a.hp_slices) {
          s0 += q0[z];
          s1 += q1[z];
        }
#pragma unroll
      for (int e = 0; e < 4; e++) {
        hf[e] = (_Float16)s0[e];
        hf[4 + e] = (_Float16)s1[e];
      }
    } else {
      hf = *reinterpret_cast<const half8_t*>(a.lora_h + (int64_t)m * a.r + r0 + 8 * lseg);
    }
    return hf;
  }

  // the 32 keep bits of row m, columns n..n+31 (n a multiple of 32), from memory
  __device__ static __forceinline__ uint32_t keep_mem(const GemmArgs& a, int m, int n) {
    if (m >= a.M || n >= a.Nc) return 0u;
    return reinterpret_cast<const uint32_t*>(a.mask)[(int64_t)m * keep_words(a.Nc) + (n >> 5)];
  }

  // acc (tile i, j) times the dropout: keep bits `kb` of the tile's 32 columns (bit c for column
  // c of the tile; the lane's columns are 8g + 4 lseg + e) scaled by mask_scale, else 0
  __device__ static __forceinline__ void drop_tile(const GemmArgs& a, float16_t& t, uint32_t kb,
                                                   int lseg) {
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        t[4 * g + e] = ((kb >> (8 * g + 4 * lseg + e)) & 1u) ? t[4 * g + e] * a.mask_scale : 0.0f;
  }

  // Each tile's accumulator is born from its first LoRA MFMA (or its base value).  The first
  // column tile's waves that own the first columns write the fp16 LoRA operand transposed.
  // wr0 / wc0: the wave's first row / column within the workgroup tile (for the LDS areas).
  __device__ __forceinline__ void finish(const GemmArgs& a, float16_t (&acc)[TM][TN], int mb,
                                         int nb, int lrow, int lseg, int wr0, int wc0,
                                         const _Float16* ls = nullptr, int ls_cols = 0,
                                         const uint8_t* kls = nullptr, int kst = 0) {
    if ((int)blockIdx.z != a.zf || !(a.lora_h || a.lora_hp)) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = base(a, j, nb, lseg);
      return;
    }
    // lora_w is [Nc, r] in both directions (the backward pass gets lora_A transposed), so the
    // W-side operand is one 16-byte load per tile and 16 ranks
    const bool write_t = a.lora_hp && a.lora_ht && nb == 0;  // first column tile
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int m = mb + i * 32 + lrow;
      for (int r0 = 0; r0 < a.r; r0 += 16) {
        const half8_t hf =
            ls ? *reinterpret_cast<const half8_t*>(ls + (wr0 + i * 32 + lrow) * 16 + 8 * lseg)
               : lora_row(a, m, r0, lseg);
        if (write_t && m < a.ldt) {
#pragma unroll
          for (int e = 0; e < 8; e++) a.lora_ht[(int64_t)(r0 + 8 * lseg + e) * a.ldt + m] = hf[e];
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
          half8_t wf;
          if (ls) {
            wf = *reinterpret_cast<const half8_t*>(ls + (ls_cols + wc0 + j * 32 + lrow) * 16 +
                                                   8 * lseg);
          } else {
            const int ncol = col(nb + j * 32 + lrow);
            wf = ncol < a.Nc
                ? *reinterpret_cast<const half8_t*>(a.lora_w + (int64_t)ncol * a.r + r0 + 8 * lseg)
                : (half8_t){};
          }
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              wf, hf, r0 == 0 ? base(a, j, nb, lseg) : acc[i][j], 0, 0, 0);
        }
      }
      if constexpr (BWD) {
        if (a.mask) {
#pragma unroll
          for (int j = 0; j < TN; j++) {
            const uint32_t kb =
                kls ? *reinterpret_cast<const uint32_t*>(kls + (wr0 + i * 32 + lrow) * kst +
                                                         (wc0 + j * 32) / 8)
                    : keep_mem(a, m, nb + j * 32);
            drop_tile(a, acc[i][j], kb, lseg);
          }
        }
      }
    }
  }

  // finish() for operands staged in LDS (first split, r = 16): straight-line LDS reads and one
  // MFMA per tile; `ls`: [rows][16] operand then (at row ls_cols) [cols][16] of lora_w; `kls`
  // (backward, may be null): keep bits, row stride kst bytes.
  __device__ __forceinline__ void finish_staged(const GemmArgs& a, float16_t (&acc)[TM][TN],
                                                int mb, int nb, int lrow, int lseg, int wr0,
                                                int wc0, const _Float16* ls, int ls_cols,
                                                const uint8_t* kls, int kst) {
    half8_t wf[TN];
#pragma unroll
    for (int j = 0; j < TN; j++)
      wf[j] = *reinterpret_cast<const half8_t*>(ls + (ls_cols + wc0 + j * 32 + lrow) * 16 + 8 * lseg);
    const bool write_t = a.lora_hp && a.lora_ht && nb == 0;  // first column tile
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const half8_t hf =
          *reinterpret_cast<const half8_t*>(ls + (wr0 + i * 32 + lrow) * 16 + 8 * lseg);
#pragma unroll
      for (int j = 0; j < TN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[j], hf, base(a, j, nb, lseg), 0, 0, 0);
      if (write_t) {
        const int m = mb + i * 32 + lrow;
        if (m < a.ldt) {
#pragma unroll
          for (int e = 0; e < 8; e++) a.lora_ht[(int64_t)(8 * lseg + e) * a.ldt + m] = hf[e];
        }
      }
      if constexpr (BWD) {
        if (kls) {
#pragma unroll
          for (int j = 0; j < TN; j++)
            drop_tile(a, acc[i][j],
                      *reinterpret_cast<const uint32_t*>(kls + (wr0 + i * 32 + lrow) * kst +
                                                         (wc0 + j * 32) / 8),
                      lseg);
        }
      }
    }
  }
};

// The backward pass's dropout keep bits of the warp-specialized kernel's BM x BN tile, staged by
// its producers in LDS: BN / 32 words per row at a row stride of an odd number of words, so the
// consumers' word reads of one 32-column block over 32 rows hit distinct banks.  Producer thread
// p loads words p, p + NTP, ... of the tile (row-major).
template <int BM, int BN, int NTP>
struct MaskStage {
  static_assert(BN % 32 == 0, "whole keep words per tile row");
  static constexpr int KW = BN / 32;                   // keep words per tile row
  static constexpr int KST = 4 * (KW | 1);             // LDS row stride, bytes
  static constexpr int N = (BM * KW + NTP - 1) / NTP;  // words per producer thread
  uint32_t v[N];

  __device__ __forceinline__ void issue(const GemmArgs& a, int p, int m0, int n0) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.mask);
    const int kw = keep_words(a.Nc);
#pragma unroll
    for (int u = 0; u < N; u++) {
      const int c = p + NTP * u;
      const int m = m0 + c / KW, n = n0 + 32 * (c % KW);
      v[u] = c < BM * KW && m < a.M && n < a.Nc ? src[(int64_t)m * kw + (n >> 5)] : 0u;
    }
  }

  __device__ __forceinline__ void commit(uint8_t* kls, int p) const {
#pragma unroll
    for (int u = 0; u < N; u++) {
      const int c = p + NTP * u;
      if (c >= BM * KW) break;
      *reinterpret_cast<uint32_t*>(kls + (c / KW) * KST + 4 * (c % KW)) = v[u];
    }
  }
};

// LoRA operands of the warp-specialized kernel staged by its producers (r = 16): the fp16
// operand of the workgroup's BM rows (partial sums added in slice order and rounded, as
// AccStart::lora_row does) and lora_w's BN rows, 32 bytes per row, into [BM][16] and [BN][16],
// by the NTP producer threads.
// The source blocks are contiguous (BM rows x 16 ranks per slice), so they are read as 16-byte
// chunks in lane order: every load instruction covers 1 KB of consecutive memory.  Thread p
// takes chunks p, p + NTP, ...; a chunk is 4 ranks of one row (fp32) or 8 ranks (fp16).  The
// loads are issued before the first tiles' so that they share one round trip.
template <int BM, int BN, int NTP>
struct LoraStage {
  static constexpr int NP = BM * 4 / NTP;              // fp32 chunks per slice per thread
  static constexpr int NH = (BM * 2 + NTP - 1) / NTP;  // fp16-operand chunks per thread
  static constexpr int NW = (BN * 2 + NTP - 1) / NTP;  // lora_w chunks per thread
  static_assert(BM * 4 % NTP == 0, "whole fp32 chunk rounds");
  float4_t q[4][NP];  // partial sums: slice z, chunk p + NTP u
  u32x4 hv[NH];       // or the fp16 operand
  u32x4 w[NW];

  // swap: the tile's columns in rope_col order (lora_B's rows follow them)
  __device__ __forceinline__ void issue(const GemmArgs& a, int p, int m0, int n0,
                                        bool swap = false) {
    if (a.lora_hp) {
#pragma unroll
      for (int z = 0; z < 4; z++) {
        const float4_t* src =
            reinterpret_cast<const float4_t*>(a.lora_hp + ((int64_t)z * a.ldt + m0) * 16);
#pragma unroll
        for (int u = 0; u < NP; u++) {
          const int c = p + NTP * u;
          const bool ok = z < a.hp_slices && m0 + c / 4 < a.M;
          q[z][u] = ok ? src[c] : (float4_t){};
        }
      }
    } else {
      const u32x4* src = reinterpret_cast<const u32x4*>(a.lora_h + (int64_t)m0 * 16);
#pragma unroll
      for (int u = 0; u < NH; u++) {
        const int c = p + NTP * u;
        hv[u] = c < BM * 2 && m0 + c / 2 < a.M ? src[c] : (u32x4){};
      }
    }
    if (swap) {
#pragma unroll
      for (int u = 0; u < NW; u++) {
        const int c = p + NTP * u;
        const int n = rope_col(n0 + c / 2);
        w[u] = c < BN * 2 && n < a.Nc
            ? *reinterpret_cast<const u32x4*>(a.lora_w + (int64_t)n * 16 + 8 * (c & 1))
            : (u32x4){};
      }
    } else {
      const u32x4* wsrc = reinterpret_cast<const u32x4*>(a.lora_w + (int64_t)n0 * 16);
#pragma unroll
      for (int u = 0; u < NW; u++) {
        const int c = p + NTP * u;
        w[u] = c < BN * 2 && n0 + c / 2 < a.Nc ? wsrc[c] : (u32x4){};
      }
    }
  }

  // after the loads have landed: rows into the LDS area `ls`
  __device__ __forceinline__ void commit(const GemmArgs& a, _Float16* ls, int p) const {
    if (a.lora_hp) {
#pragma unroll
      for (int u = 0; u < NP; u++) {
        const int c = p + NTP * u;
        float4_t sum = q[0][u];  // slices added in order
#pragma unroll
        for (int z = 1; z < 4; z++)
          if (z < a.hp_slices) sum += q[z][u];
        const u32x2 h = {pack_f16x2(sum[0], sum[1]), pack_f16x2(sum[2], sum[3])};
        *reinterpret_cast<u32x2*>(ls + 4 * c) = h;  // row c/4, ranks 4(c%4)..+3
      }
    } else {
#pragma unroll
      for (int u = 0; u < NH; u++) {
        const int c = p + NTP * u;
        if (c < BM * 2) *reinterpret_cast<u32x4*>(ls + 8 * c) = hv[u];
      }
    }
#pragma unroll
    for (int u = 0; u < NW; u++) {
      const int c = p + NTP * u;
      if (c < BN * 2) *reinterpret_cast<u32x4*>(ls + BM * 16 + 8 * c) = w[u];
    }
  }
};

template <int TM, int TN, bool BWD>
__device__ __forceinline__ void init_acc(const GemmArgs& a, float16_t (&acc)[TM][TN], int mb,
                                         int nb, int lrow, int lseg) {
  AccStart<TM, TN, BWD> st;
  st.load(a, nb, lseg);
  st.finish(a, acc, mb, nb, lrow, lseg, 0, 0);
}

// Epilogue: fp16 stores of the tiles (one 8-byte store per register group), or with split-K
// fp32 partials (16 bytes per group) to the workspace.
template <int TM, int TN, bool BWD>
__device__ __forceinline__ void epilogue(const GemmArgs& a, float16_t (&acc)[TM][TN], int mb,
                                         int nb, int lrow, int lseg) {
  const bool split = gridDim.z > 1 && !a.unsplit;
  const bool vec = (a.Nc % 4) == 0 && (a.ldc % 4) == 0;
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int m = mb + i * 32 + lrow;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < TN; j++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int n = nb + j * 32 + 8 * g + 4 * lseg;
        if (n >= a.Nc) continue;
        float4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                      acc[i][j][4 * g + 3]};
        const bool full = vec && n + 3 < a.Nc;
        if (split) {
          float* w = a.ws + ((int64_t)blockIdx.z * a.M + m) * a.Nc + n;
          if (full) {
            *reinterpret_cast<float4_t*>(w) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
              if (n + e < a.Nc) w[e] = v[e];
          }
        } else {
          _Float16* c = a.C + (int64_t)m * a.ldc + n;
          if (full) {
            *reinterpret_cast<half4_t*>(c) = __builtin_convertvector(v, half4_t);
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
              if (n + e < a.Nc) c[e] = (_Float16)v[e];
          }
        }
      }
    }
  }
}

// Split-K: C = fp16(sum over the split planes of ws), summed in split order (deterministic).
// Epilogue through LDS (warp-specialized kernel): a wave's accumulators leave in 32-row slices.
// The slice is written to the wave's own LDS area in the accumulator layout (8-byte fp16 or
// 16-byte fp32 items; row stride padded to 2 x odd (fp16) or 4 x odd (fp32) dwords, so the 32
// rows of one write hit distinct banks), read back row-major, and stored 16 contiguous bytes
// per lane, so every store instruction writes whole cache lines instead of 16 bytes in each of
// 32 rows.  Only the writing wave touches its area, so no barrier is needed between slices;
// LDS instructions of one wave complete in order.  `area` holds 32 * stride dwords.
template <int TM, int TN>
struct StagedStore {
  static constexpr int WN = TN * 32;
  static constexpr int S16 = WN / 2 + 2;  // fp16 row stride in dwords
  static constexpr int S32 = WN + 4;      // fp32 row stride in dwords
  static constexpr int AREA_DWORDS = 32 * S32;
};

// RoPE of one lane's accumulators before the fp16 store (ROPE kernels): output row m, blocks
// j = 0 / 1 holding head columns d / d + 64 (rope_col order; nb the wave's column coordinate).
// Each value is first rounded to fp16, the unrotated projection output, then rotated in fp32
// with every product and sum rounded once (no contraction): k_qkv_rope's arithmetic on that
// output, so the stored fp16 has the bits of the projection followed by the rotation launch.
// The cos / sin are read here, when every tile of the launch reaches its epilogue: staging them
// in LDS earlier (in the prologue, or copied during the main loop by the producer waves without
// NF4 items) measured no faster, the extra traffic then slowing the K-steps instead.
template <int TN>
__device__ __forceinline__ void rope_rotate(const GemmArgs& a, float16_t (&acc)[TN], int m,
                                            int nb, int lseg) {
#pragma clang fp contract(off)
  static_assert(TN == 2, "a lane holds both halves of its head columns");
  if (m >= a.M) return;
  const int b = m / a.rope_T, t = m - b * a.rope_T;
  const int64_t cr = (int64_t)b * a.rope_cs_b + (int64_t)t * a.rope_cs_t;
  const int d0 = rope_col(nb) & 127;  // head column of block 0's first column (< 64)
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int d = d0 + 8 * g + 4 * lseg;
    const float4_t c1 = *reinterpret_cast<const float4_t*>(a.rope_cos + cr + d);
    const float4_t c2 = *reinterpret_cast<const float4_t*>(a.rope_cos + cr + d + 64);
    const float4_t s1 = *reinterpret_cast<const float4_t*>(a.rope_sin + cr + d);
    const float4_t s2 = *reinterpret_cast<const float4_t*>(a.rope_sin + cr + d + 64);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float x1 = (float)(_Float16)acc[0][4 * g + e];
      const float x2 = (float)(_Float16)acc[1][4 * g + e];
      acc[0][4 * g + e] = x1 * c1[e] + x2 * -s1[e];
      acc[1][4 * g + e] = x2 * c2[e] + x1 * s2[e];
    }
  }
}

template <int TM, int TN, bool ROPE = false>
__device__ __forceinline__ void epilogue_staged(const GemmArgs& a, float16_t (&acc)[TM][TN],
                                                int mb, int nb, int lane, float* area) {
  using SS = StagedStore<TM, TN>;
  constexpr int WN = SS::WN;
  const int lrow = lane & 31, lseg = lane >> 5;
  const bool split = gridDim.z > 1 && !a.unsplit;
  // whole 16-byte chunks can be stored when rows keep 16-byte alignment
  const bool vec = split ? (a.Nc % 4) == 0 : ((a.Nc % 8) == 0 && (a.ldc % 8) == 0 &&
                                               ((uintptr_t)a.C % 16) == 0);
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int row0 = mb + i * 32;
    if (row0 >= a.M) break;
    if (split) {
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                              acc[i][j][4 * g + 3]};
          *reinterpret_cast<float4_t*>(area + lrow * SS::S32 + 32 * j + 8 * g + 4 * lseg) = v;
        }
    } else {
      if constexpr (ROPE) {
        if (a.rope_cos) rope_rotate<TN>(a, acc[i], row0 + lrow, nb, lseg);
      }
      uint32_t* ar = reinterpret_cast<uint32_t*>(area);
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          u32x2 v;
          v[0] = pack_f16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
          v[1] = pack_f16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          *reinterpret_cast<u32x2*>(ar + lrow * SS::S16 + 16 * j + 4 * g + 2 * lseg) = v;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (split) {
      constexpr int CPR = WN / 4;  // 16-byte chunks per row
#pragma unroll
      for (int q = 0; q < CPR / 2; q++) {
        const int c = q * 64 + lane;
        const int r = c / CPR, cc = c % CPR;
        const int m = row0 + r, n = nb + 4 * cc;
        const float4_t v = *reinterpret_cast<const float4_t*>(area + r * SS::S32 + 4 * cc);
        if (m >= a.M || n >= a.Nc) continue;
        float* w = a.ws + ((int64_t)blockIdx.z * a.M + m) * a.Nc + n;
        if (vec && n + 3 < a.Nc) {
          *reinterpret_cast<float4_t*>(w) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (n + e < a.Nc) w[e] = v[e];
        }
      }
    } else {
      constexpr int CPR = WN / 8;
      const uint32_t* ar = reinterpret_cast<const uint32_t*>(area);
#pragma unroll
      for (int q = 0; q < CPR / 2; q++) {
        const int c = q * 64 + lane;
        const int r = c / CPR, cc = c % CPR;
        const int m = row0 + r;
        int n = nb + 8 * cc;
        if constexpr (ROPE) n = a.rope_cos ? rope_col(n) : n;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ar + r * SS::S16 + 4 * cc);
        if (m >= a.M || n >= a.Nc) continue;
        _Float16* dst = a.C + (int64_t)m * a.ldc + n;
        if (vec && n + 7 < a.Nc) {
          *reinterpret_cast<u32x4*>(dst) = v;
        } else {
          const half8_t h = __builtin_bit_cast(half8_t, v);
#pragma unroll
          for (int e = 0; e < 8; e++)
            if (n + e < a.Nc) dst[e] = h[e];
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next slice
  }
}

// SwiGLU output of an unsplit warp-specialized tile (the split ones leave it to the reduce).
// The epilogue is memory-bound: one tile moves its fp16 output plus one (forward: gate) or two
// (backward: gate, up) tiles in and one more out, and every workgroup reaches it at about the
// same time.  So the producer waves, idle once their last copy has landed, issue all their
// gate/up loads right then (they land while the consumers run the last K-step); the consumers
// stage their fp16 accumulators, the whole tile at once, in the A ring and leave; the producers
// then combine and store.  One round trip per workgroup, and none of the consumers' registers.
//   forward (BWD = false): C = y (the up projection) and h = silu(gate) * y;
//   backward (BWD = true): the tile is d(hidden); gate <- d(gate), up <- d(up).
template <int BM, int BN, int CWM, int CWN, int NTP, bool BWD>
struct GluTail {
  static constexpr int WM = BM / CWM, WN = BN / CWN, TM = WM / 32, TN = WN / 32;
  using SS = StagedStore<TM, TN>;
  static constexpr int CPR = BN / 8;       // 16-byte chunks per tile row
  static constexpr int NCL = BM * CPR / NTP;  // chunks per producer lane
  static constexpr int AREA = WM * SS::S16;   // dwords of one consumer wave's staged tile
  static_assert(BM * CPR % NTP == 0, "the tile's chunks split evenly over the producers");
  // chunks in flight per lane: all of them where registers allow, else a rolling window
  static constexpr int AHEAD = NCL < (BWD ? 10 : 20) ? NCL : (BWD ? 10 : 20);
  u32x4 g[NCL];
  u32x4 u[BWD ? NCL : 1];

  // chunk k of producer lane p: tile row m, 8-column group cc (a row's chunks on adjacent lanes)
  __device__ static void chunk(int p, int k, int& m, int& cc) {
    const int q = p + k * NTP;
    m = q / CPR;
    cc = q % CPR;
  }

  __device__ __forceinline__ void load(const GemmArgs& a, int p, int m0, int n0, int k) {
    int m, cc;
    chunk(p, k, m, cc);
    const int gm = m0 + m, gn = n0 + 8 * cc;
    g[k] = (u32x4){};
    if constexpr (BWD) u[k] = (u32x4){};
    if (gm < a.M && gn < a.Nc) {  // Nc % 8 == 0: whole chunks
      const int64_t o = (int64_t)gm * a.ldc + gn;
      g[k] = *reinterpret_cast<const u32x4*>(a.glu_g + o);
      if constexpr (BWD) u[k] = *reinterpret_cast<const u32x4*>(a.glu_u + o);
    }
  }

  // the first AHEAD chunks' gate / up loads (issued before the consumers' tile is staged)
  __device__ __forceinline__ void prefetch(const GemmArgs& a, int p, int m0, int n0) {
#pragma unroll
    for (int k = 0; k < AHEAD; k++) load(a, p, m0, n0, k);
  }

  // every chunk: staged value, gate / up, SwiGLU, stores; chunk k + AHEAD is loaded once k is done
  __device__ __forceinline__ void store(const GemmArgs& a, int p, int m0, int n0,
                                        const uint32_t* staged) {
#pragma unroll
    for (int k = 0; k < NCL; k++) {
      int m, cc;
      chunk(p, k, m, cc);
      const int gm = m0 + m, gn = n0 + 8 * cc;
      if (gm < a.M && gn < a.Nc) {
        const int w = (m / WM) * CWN + (8 * cc) / WN;  // the consumer wave that staged it
        const u32x4 v = *reinterpret_cast<const u32x4*>(staged + w * AREA + (m % WM) * SS::S16 +
                                                          ((8 * cc) % WN) / 2);
        const int64_t o = (int64_t)gm * a.ldc + gn;
        const half8_t h = __builtin_bit_cast(half8_t, v);
        const half8_t gv = __builtin_bit_cast(half8_t, g[k]);
        if constexpr (BWD) {
          const half8_t uv = __builtin_bit_cast(half8_t, u[k]);
          half8_t dg, du;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            _Float16 x, y;
            swiglu_bwd((float)h[e], (float)gv[e], (float)uv[e], x, y);
            dg[e] = x;
            du[e] = y;
          }
          *reinterpret_cast<half8_t*>(a.glu_g + o) = dg;
          *reinterpret_cast<half8_t*>(a.glu_u + o) = du;
        } else {
          half8_t hh;
#pragma unroll
          for (int e = 0; e < 8; e++) hh[e] = swiglu_fwd((float)gv[e], (float)h[e]);
          *reinterpret_cast<u32x4*>(a.C + o) = v;
          *reinterpret_cast<half8_t*>(a.glu_h + o) = hh;
        }
      }
      if (k + AHEAD < NCL) load(a, p, m0, n0, k + AHEAD);
    }
  }

  // a consumer wave's accumulators as fp16, all TM row slices: row r of its tile at r * S16
  __device__ __forceinline__ static void stage(const float16_t (&acc)[TM][TN], int lane,
                                               uint32_t* area) {
    const int lrow = lane & 31, lseg = lane >> 5;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          u32x2 v;
          v[0] = pack_f16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
          v[1] = pack_f16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          *reinterpret_cast<u32x2*>(area + (i * 32 + lrow) * SS::S16 + 16 * j + 4 * q +
                                    2 * lseg) = v;
        }
  }
};

// The split-K reduce of elements e .. e + 3 (one thread).
template <int GLU>
__device__ __forceinline__ void splitk_reduce_quad(const float* __restrict__ ws, int splits,
                                                   int M, int Nc, _Float16* __restrict__ C,
                                                   int64_t ldc, _Float16* __restrict__ glu_g,
                                                   _Float16* __restrict__ glu_u,
                                                   _Float16* __restrict__ glu_h, int64_t e) {
  const int64_t plane = (int64_t)M * Nc;
  if (e >= plane) return;
  const int m = (int)(e / Nc), n = (int)(e % Nc);
  if ((Nc % 4) == 0 && (ldc % 4) == 0) {
    // loads of four splits at a time are issued before they are added (in split order)
    float4_t v = *reinterpret_cast<const float4_t*>(ws + e);
    for (int z0 = 1; z0 < splits; z0 += 4) {
      float4_t p[4];
#pragma unroll
      for (int u = 0; u < 4; u++)
        p[u] = z0 + u < splits ? *reinterpret_cast<const float4_t*>(ws + (z0 + u) * plane + e)
                               : (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (z0 + u < splits) v += p[u];
    }
    const half4_t h = __builtin_convertvector(v, half4_t);
    const int64_t o = (int64_t)m * ldc + n;
    if constexpr (GLU == 2) {  // d(hidden) -> d(gate), d(up) over gate and up (SwiGLU backward)
      const half4_t g = *reinterpret_cast<const half4_t*>(glu_g + o);
      const half4_t u = *reinterpret_cast<const half4_t*>(glu_u + o);
      half4_t dg, du;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        _Float16 x, y;
        swiglu_bwd((float)h[q], (float)g[q], (float)u[q], x, y);
        dg[q] = x;
        du[q] = y;
      }
      *reinterpret_cast<half4_t*>(glu_g + o) = dg;
      *reinterpret_cast<half4_t*>(glu_u + o) = du;
      return;
    }
    *reinterpret_cast<half4_t*>(C + o) = h;
    if constexpr (GLU == 1) {  // silu(gate) * up beside the up projection's output
      const half4_t g = *reinterpret_cast<const half4_t*>(glu_g + o);
      half4_t hh;
#pragma unroll
      for (int q = 0; q < 4; q++) hh[q] = swiglu_fwd((float)g[q], (float)h[q]);
      *reinterpret_cast<half4_t*>(glu_h + o) = hh;
    }
  } else {
    for (int q = 0; q < 4 && e + q < plane; q++) {
      const int mq = (int)((e + q) / Nc), nq = (int)((e + q) % Nc);
      float v = ws[e + q];
      for (int z = 1; z < splits; z++) v += ws[z * plane + e + q];
      const _Float16 h = (_Float16)v;
      const int64_t o = (int64_t)mq * ldc + nq;
      if constexpr (GLU == 2) {
        _Float16 x, y;
        swiglu_bwd((float)h, (float)glu_g[o], (float)glu_u[o], x, y);
        glu_g[o] = x;
        glu_u[o] = y;
        continue;
      }
      C[o] = h;
      if constexpr (GLU == 1) glu_h[o] = swiglu_fwd((float)glu_g[o], (float)h);
    }
  }
}

template <int GLU>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ ws, int splits,
                                                      int M, int Nc, _Float16* __restrict__ C,
                                                      int64_t ldc,
                                                      _Float16* __restrict__ glu_g,
                                                      _Float16* __restrict__ glu_u,
                                                      _Float16* __restrict__ glu_h) {
  splitk_reduce_quad<GLU>(ws, splits, M, Nc, C, ldc, glu_g, glu_u, glu_h,
                          ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4);
}

// The split-K reduce (no SwiGLU) and a LoRA gradient group in ONE launch: they are independent
// (the gradients read the dHs^T the GEMM wrote, not its output).  Workgroups [0, cols) are the
// gradient group's, as its own launch lays them out (same waves, so the same bits); the nred
// after them reduce quads bid - cols, + nred * blockDim.x, ...  Dispatched after the gradient
// workgroups, the reduce fills the CUs their last partial round leaves idle.
template <int CPL>
__global__ __launch_bounds__(64 * cols_max_waves<CPL>()) void k_splitk_reduce_cols(
    const float* __restrict__ ws, int splits, int Mc, int Nc, _Float16* __restrict__ C,
    int64_t ldc, ColsGroup g, int M, int ldt, int r, int nw, int nred) {
  extern __shared__ float red[];  // [nw][r][16 * CPL + 1]
  const int bid = (int)blockIdx.x, cols = g.start[g.n];
  if (bid < cols) {
    lora_cols_group_block<CPL>(g, M, ldt, r, bid, nw, red);
    return;
  }
  const int64_t quads = ((int64_t)Mc * Nc + 3) / 4;
  for (int64_t q = (int64_t)(bid - cols) * blockDim.x + threadIdx.x; q < quads;
       q += (int64_t)nred * blockDim.x)
    splitk_reduce_quad<0>(ws, splits, Mc, Nc, C, ldc, nullptr, nullptr, nullptr, 4 * q);
}

static int launch_reduce(const GemmArgs& a, int splits, hipStream_t stream) {
  const int64_t quads = ((int64_t)a.M * a.Nc + 3) / 4;
  const dim3 grid((unsigned)((quads + 255) / 256));
  if (a.glu == 1)
    hipLaunchKernelGGL(k_splitk_reduce<1>, grid, dim3(256), 0, stream, a.ws, splits, a.M, a.Nc,
                       a.C, (int64_t)a.ldc, a.glu_g, a.glu_u, a.glu_h);
  else if (a.glu == 2)
    hipLaunchKernelGGL(k_splitk_reduce<2>, grid, dim3(256), 0, stream, a.ws, splits, a.M, a.Nc,
                       a.C, (int64_t)a.ldc, a.glu_g, a.glu_u, a.glu_h);
  else
    hipLaunchKernelGGL(k_splitk_reduce<0>, grid, dim3(256), 0, stream, a.ws, splits, a.M, a.Nc,
                       a.C, (int64_t)a.ldc, a.glu_g, a.glu_u, a.glu_h);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

// LDS tables both kernels use: the byte -> (NF4[hi], NF4[lo]) pair table and the code book.
// (A 16-entry table read once per nibble has no bank conflicts, but its extra address math and
// twice the LDS instructions lengthened the producers' per-step chain: slower, measured.)
__device__ __forceinline__ void fill_tables(const GemmArgs& a, float2_t* s_pair, float* s_code,
                                            int t, int nthreads) {
  for (int i = t; i < 256; i += nthreads) {
    s_code[i] = a.code[i];
    s_pair[i] = (float2_t){kNF4[i >> 4], kNF4[i & 15]};
  }
}

// Global -> register staging and register -> LDS commit of one K-step's tiles, for NTP
// loading threads (thread index p in [0, NTP)).
//   A: BM rows x 64 fp16 (16-byte segments; rows past M clamped to the last row).
//   B forward:  item (row n, half) = 32 NF4 values of W row n, one block scale.
//   B backward: item (row group of 4 W rows, chunk of 8 output columns) = 32 values, 4 scales;
//               decoded along W's rows so LDS holds B[n'][k'] with the reduction contiguous.
// Columns past Nc are clamped to the last valid ones: they only reach outputs never stored.
template <int BM, int BN, bool BWD, int NTP>
struct Loader {
  static constexpr int A_ITEMS = BM * 8 / NTP;
  static constexpr int B_TOTAL = BWD ? (BN / 8) * (kBK / 4) : BN * 2;
  static constexpr int B_ITEMS = (B_TOTAL + NTP - 1) / NTP;
  static constexpr int NS = BWD ? 4 : 1;
  static_assert(BM * 8 % NTP == 0 && A_ITEMS >= 1, "A tile vs loading threads");
  static_assert(B_TOTAL % 64 == 0, "B items in whole waves");

  struct Stage {
    u32x4 a[A_ITEMS];
    uint32_t w[B_ITEMS][4];
    uint32_t q8[B_ITEMS][NS];
    float a2[B_ITEMS][NS];
  };

  __device__ static __forceinline__ void issue(const GemmArgs& a, Stage& S, int p, int kt, int m0,
                                               int n0) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int u = 0; u < B_ITEMS; u++) {
      const int q = p + u * NTP;
      if (q >= B_TOTAL) break;
      if (!BWD) {
        const int n = min(n0 + (q >> 1), a.Nc - 1);
        const int64_t blk = ((int64_t)n * a.Kw + k0) >> 6;
        S.q8[u][0] = a.absmax8[blk];
        S.a2[u][0] = a.absmax2[blk >> 8];
        const u32x4 w = *reinterpret_cast<const u32x4*>(
            a.packed + (int64_t)n * (a.Kw / 2) + k0 / 2 + (q & 1) * 16);
#pragma unroll
        for (int j = 0; j < 4; j++) S.w[u][j] = w[j];
      } else {
        const int chunk = q % (BN / 8);
        const int rg = q / (BN / 8);
        const int col = min(n0 + chunk * 8, a.Nc - 8);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int64_t idx = (int64_t)(k0 + rg * 4 + i) * a.Kw + col;
          S.q8[u][i] = a.absmax8[idx >> 6];
          S.a2[u][i] = a.absmax2[idx >> 14];
          S.w[u][i] = *reinterpret_cast<const uint32_t*>(a.packed + (idx >> 1));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < A_ITEMS; u++) {
      const int q = p + u * NTP;
      const int m = min(m0 + (q >> 3), a.M - 1);
      S.a[u] = *reinterpret_cast<const u32x4*>(a.A + (int64_t)m * a.lda + k0 + (q & 7) * 8);
    }
  }

  // Part `part` (0..3) of the commit: a quarter of the A segments and of the B decode.
  __device__ static __forceinline__ void commit(const Stage& S, _Float16* as, _Float16* bs, int p,
                                                int part, const float2_t* s_pair,
                                                const float* s_code, float offset) {
    constexpr int APP = (A_ITEMS + 3) / 4;
#pragma unroll
    for (int v = 0; v < APP; v++) {
      const int u = part * APP + v;
      if (u < A_ITEMS) {
        const int q = p + u * NTP;
        *reinterpret_cast<u32x4*>(as + lds_off(q >> 3, q & 7)) = S.a[u];
      }
    }
#pragma unroll
    for (int u = 0; u < B_ITEMS; u++) {
      const int q = p + u * NTP;
      if (q >= B_TOTAL) break;
      if (!BWD) {
        // dword `part`: 8 values, one LDS pair lookup per byte
        const int row = q >> 1, half = q & 1;
        const float sc = nested_scale(s_code[S.q8[u][0]], S.a2[u][0], offset);
        const uint32_t w = S.w[u][part];
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float2_t pr = s_pair[(w >> (8 * j)) & 0xffu];
          v[j] = pack_f16x2(pr[0] * sc, pr[1] * sc);
        }
        *reinterpret_cast<u32x4*>(bs + lds_off(row, half * 4 + part)) = v;
      } else {
        // byte `part` of each of the 4 rows: output columns 2*part (high nibble) and 2*part+1
        const int chunk = q % (BN / 8);
        const int rg = q / (BN / 8);
        float2_t pr[4];
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          sc[i] = nested_scale(s_code[S.q8[u][i]], S.a2[u][i], offset);
          pr[i] = s_pair[(S.w[u][i] >> (8 * part)) & 0xffu];
        }
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
          u32x2 v;
          v[0] = pack_f16x2(pr[0][cc] * sc[0], pr[1][cc] * sc[1]);
          v[1] = pack_f16x2(pr[2][cc] * sc[2], pr[3][cc] * sc[3]);
          const int row = chunk * 8 + part * 2 + cc;
          *reinterpret_cast<u32x2*>(bs + lds_off(row, rg >> 1) + (rg & 1) * 4) = v;
        }
      }
    }
  }
};

typedef short short4_t __attribute__((ext_vector_type(4)));

// Backward B tile [64][ldb]: element (k, n) in halfs.  The 16-byte unit n / 8 of row k is stored
// at unit (n / 8) ^ x(k), a permutation inside each aligned group of 4 units, so the transposing
// operand reads (4 rows x 4 units per cycle) keep their banks; x(k) = k & 3 for 20-unit rows
// (ldb 160), (k >> 2) & 3 for 12-unit rows (ldb 96).  It spreads the producers' 16-byte stores
// of one cycle over all 64 banks (without it 4 of them land on each bank).
__device__ __forceinline__ int bt_off(int k, int n, int ldb) {
  const int x = (ldb == 96 ? (k >> 2) : k) & 3;
  return k * ldb + ((((n >> 3) ^ x)) << 3) + (n & 7);
}

// All waves load, decode and multiply: K-step kt+2 is loaded while kt multiplies and kt+1 is
// committed to the other LDS buffer in four parts between the MFMA sub-steps.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool BWD>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void k_nf4_gemm(GemmArgs a) {
  using T = Tile<BM, BN, WAVES_M, WAVES_N, BWD>;
  constexpr int NTH = T::NT;
  using L = Loader<BM, BN, BWD, NTH>;
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  _Float16* As = smem;                      // [2][BM][64]
  _Float16* Bs = smem + 2 * T::LDS_A;       // [2][BN][64]
  __shared__ float2_t s_pair[256];
  __shared__ float s_code[256];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm0 = (wave / T::WAVES_N) * T::WM;
  const int wn0 = (wave % T::WAVES_N) * T::WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int n_steps = a.Kr / kBK;
  const int kt0 = ((int)blockIdx.z - a.zf) * a.steps_per_split;
  const int kt1 = min(n_steps, kt0 + a.steps_per_split);
  const int lrow = lane & 31;
  const int lseg = lane >> 5;
  fill_tables(a, s_pair, s_code, t, NTH);
  const float offset = a.offset[0];

  float16_t acc[T::TM][T::TN];

  auto mma = [&](int buf, int kk) {
    const _Float16* as = As + buf * T::LDS_A;
    const _Float16* bs = Bs + buf * T::LDS_B;
    half8_t af[T::TM], bf[T::TN];
#pragma unroll
    for (int i = 0; i < T::TM; i++)
      af[i] = *reinterpret_cast<const half8_t*>(as + lds_off(wm0 + i * 32 + lrow, 2 * kk + lseg));
#pragma unroll
    for (int j = 0; j < T::TN; j++)
      bf[j] = *reinterpret_cast<const half8_t*>(bs + lds_off(wn0 + j * 32 + lrow, 2 * kk + lseg));
#pragma unroll
    for (int i = 0; i < T::TM; i++)
#pragma unroll
      for (int j = 0; j < T::TN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[j], af[i], acc[i][j], 0, 0, 0);
  };

  // K-step kt multiplies while kt+1 is committed between the MFMA sub-steps; kt+2 is issued
  // after the commit (unconditionally, clamped) so counter waits never cover fresh loads.
  auto step = [&](int buf, int kt, const typename L::Stage& next, typename L::Stage& later) {
#pragma unroll
    for (int kk = 0; kk < kBK / 16; kk++) {
      mma(buf, kk);
      if (kt + 1 < kt1)
        L::commit(next, As + (buf ^ 1) * T::LDS_A, Bs + (buf ^ 1) * T::LDS_B, t, kk, s_pair,
                  s_code, offset);
    }
    L::issue(a, later, t, min(kt + 2, kt1 - 1), m0, n0);
    __syncthreads();
  };

  if (kt0 < kt1) {
    typename L::Stage S0, S1;
    L::issue(a, S0, t, kt0, m0, n0);
    L::issue(a, S1, t, min(kt0 + 1, kt1 - 1), m0, n0);
    // accumulator start (bias, LoRA) while the first tiles are in flight
    init_acc<T::TM, T::TN, BWD>(a, acc, m0 + wm0, n0 + wn0, lrow, lseg);
    __syncthreads();  // tables
#pragma unroll
    for (int part = 0; part < 4; part++)
      L::commit(S0, As, Bs, t, part, s_pair, s_code, offset);
    __syncthreads();
    // two K-steps per trip with a fixed register assignment for both stages; odd tail after
    int kt = kt0;
    for (; kt + 1 < kt1; kt += 2) {
      step(0, kt, S1, S0);
      step(1, kt + 1, S0, S1);
    }
    if (kt < kt1) step(0, kt, S1, S0);
  } else {
    init_acc<T::TM, T::TN, BWD>(a, acc, m0 + wm0, n0 + wn0, lrow, lseg);
  }

  epilogue<T::TM, T::TN, BWD>(a, acc, m0 + wm0, n0 + wn0, lrow, lseg);
}

// NF4 side of a forward K-step for the warp-specialized kernel's 256 producer threads.
// Item = 16 packed bytes of W row n (32 values, half of the row's block for this K-step, one
// block scale), 3 memory instructions (dwordx4, absmax8 byte, absmax2 float); a 160-row tile
// adds one 4-byte item per lane for rows 128-159, so every producer lane decodes 40 values and
// no wave does a second 16-byte round alone.  Per-lane byte offsets are computed once (setup);
// a K-step only moves the uniform base pointers, so the loads take the scalar-base address
// form and cost no per-step vector address arithmetic.  Offsets are 32-bit: the launcher only
// picks this kernel when W has fewer than 2^32 values.
template <int BN>
struct BLoad {
  static constexpr int NTP = 256;
  static constexpr int R16 = BN >= 128 ? 128 : BN;
  static constexpr int REST = BN - R16;
  static_assert(REST == 0 || REST == 32, "B tile rows: <= 128, or 128 + 32");
  static constexpr int TOTAL = R16 * 2;  // 16-byte items
  static constexpr int VMEM = REST ? 6 : 3;  // memory instructions one issue() makes per lane
  static_assert(TOTAL % 64 == 0, "B items in whole waves");

  struct Stage {
    u32x4 w;
    uint32_t q8;
    float a2;
    uint32_t w4, q8b;  // 4-byte item (REST rows)
    float a2b;
  };
  struct Src {
    uint32_t w, blk;    // packed byte offset of the item at K-step 0; its row's first block
    uint32_t w4, blk4;  // the same for the 4-byte item
  };

  __device__ static __forceinline__ Src setup(const GemmArgs& a, int p, int n0) {
    Src r;
    const int q = p;  // the caller runs only lanes with an item (p < TOTAL)
    const uint32_t n = min(n0 + (q >> 1), a.Nc - 1);
    r.w = n * (uint32_t)(a.Kw / 2) + (q & 1) * 16;
    r.blk = n * (uint32_t)(a.Kw / 64);
    const uint32_t n4 = min(n0 + R16 + (p >> 3), a.Nc - 1);
    r.w4 = n4 * (uint32_t)(a.Kw / 2) + (p & 7) * 4;
    r.blk4 = n4 * (uint32_t)(a.Kw / 64);
    return r;
  }

  __device__ static __forceinline__ void issue(const GemmArgs& a, const Src& src, Stage& S,
                                               int kt) {
    const uint8_t* pk = a.packed + kt * (kBK / 2);  // uniform
    const uint8_t* q8 = a.absmax8 + kt;             // block of row n at K-step kt: blk + kt
    S.q8 = gload_u8(q8, src.blk);
    S.a2 = gload_f32(a.absmax2, ((src.blk + kt) >> 8) * 4);
    S.w = gload_b128(pk, src.w);
    if constexpr (REST > 0) {
      S.q8b = gload_u8(q8, src.blk4);
      S.a2b = gload_f32(a.absmax2, ((src.blk4 + kt) >> 8) * 4);
      S.w4 = gload_b32(pk, src.w4);
    }
  }

  // after the wait that covers the stage's loads
  __device__ static __forceinline__ void ready(Stage& S) {
    vm_ready(S.w);
    vm_ready(S.q8);
    vm_ready(S.a2);
    if constexpr (REST > 0) {
      vm_ready(S.w4);
      vm_ready(S.q8b);
      vm_ready(S.a2b);
    }
  }

  // table lookups of one stage (issued a K-step before finish() uses them)
  struct Looked {
    float2_t pr[4][4];
    float2_t pb[4];
    float c, cb;
  };

  __device__ static __forceinline__ void lookup(const Stage& S, Looked& L, const float2_t* s_pair,
                                                const float* s_code) {
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
      for (int j = 0; j < 4; j++) L.pr[d][j] = s_pair[(S.w[d] >> (8 * j)) & 0xffu];
    L.c = s_code[S.q8];
    if constexpr (REST > 0) {
#pragma unroll
      for (int j = 0; j < 4; j++) L.pb[j] = s_pair[(S.w4 >> (8 * j)) & 0xffu];
      L.cb = s_code[S.q8b];
    }
  }

  __device__ static __forceinline__ void finish(const Stage& S, const Looked& L, _Float16* bs,
                                                int p, float offset) {
    {
      const int q = p;  // < TOTAL
      const float sc = nested_scale(L.c, S.a2, offset);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = pack_f16x2(L.pr[d][j][0] * sc, L.pr[d][j][1] * sc);
        *reinterpret_cast<u32x4*>(bs + lds_off(q >> 1, (q & 1) * 4 + d)) = v;
      }
    }
    if constexpr (REST > 0) {
      const float sc = nested_scale(L.cb, S.a2b, offset);
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = pack_f16x2(L.pb[j][0] * sc, L.pb[j][1] * sc);
      *reinterpret_cast<u32x4*>(bs + lds_off(R16 + (p >> 3), p & 7)) = v;
    }
  }
};

// NF4 side of a backward K-step for the warp-specialized kernel, with the B tile stored as W's
// rows: bt[k][n] = W[k0 + k][n0 + n] (k: reduction index = W row, n: output column), row
// stride LDB halfs (BN, or BN + 32 when BN * 2 bytes is a multiple of 256, so that the four rows
// one transposing read touches fall in different LDS banks).  Item = 16 packed bytes of one W
// row (32 columns, one block scale: n0 is a multiple of 32, so a chunk never straddles a
// block), 3 memory instructions; a 160-column tile adds one 4-byte item per lane for columns
// 128-159.  The decoded values are written as 4 contiguous 16-byte stores.
template <int BN>
struct BLoadT {
  static constexpr int NTP = 256;
  static constexpr int LDB = (BN * 2) % 256 == 0 ? BN + 32 : BN;
  static constexpr int C16 = BN >= 128 ? 128 : BN;  // columns loaded as 16-byte items
  static constexpr int REST = BN - C16;
  static_assert(REST == 0 || REST == 32, "B tile columns: <= 128, or 128 + 32");
  static constexpr int CPR = C16 / 32;               // 16-byte items per row
  static constexpr int TOTAL = kBK * CPR;
  static constexpr int VMEM = REST ? 6 : 3;
  static_assert(TOTAL % 64 == 0 && TOTAL <= NTP, "B items in whole waves, one round");
  // item q -> (row, 32-column chunk): consecutive items along the row, except with 12-unit
  // rows (BN 96), where 16 consecutive items take one chunk of 16 consecutive rows (the layout
  // under which bt_off's swizzle spreads a store cycle over all banks)
  __device__ static __forceinline__ int item_row(int q) {
    return LDB == 96 ? 16 * (q / (16 * CPR)) + (q & 15) : q / CPR;
  }
  __device__ static __forceinline__ int item_chunk(int q) {
    return LDB == 96 ? (q >> 4) % CPR : q % CPR;
  }

  struct Stage {
    u32x4 w;
    uint32_t q8;
    float a2;
    uint32_t w4, q8b;
    float a2b;
  };
  // value index of the item within its K-step's 64-row slab of W (row * Kw + col); the slab of
  // K-step kt starts at value kt * 64 * Kw (32-bit: W has fewer than 2^32 values)
  struct Src {
    uint32_t x, x4;
  };

  __device__ static __forceinline__ Src setup(const GemmArgs& a, int p, int n0) {
    Src r;
    const int q = p;  // the caller runs only lanes with an item (p < TOTAL)
    const int row = item_row(q), c = item_chunk(q);
    r.x = (uint32_t)row * a.Kw + min(n0 + 32 * c, a.Nc - 32);
    r.x4 = (uint32_t)(p >> 2) * a.Kw + min(n0 + C16 + 8 * (p & 3), a.Nc - 8);
    return r;
  }

  __device__ static __forceinline__ void issue(const GemmArgs& a, const Src& src, Stage& S,
                                               int kt) {
    const uint32_t slab = (uint32_t)kt * kBK * a.Kw;   // uniform
    const uint8_t* pk = a.packed + slab / 2;
    const uint8_t* q8 = a.absmax8 + slab / 64;
    S.q8 = gload_u8(q8, src.x >> 6);
    S.a2 = gload_f32(a.absmax2, ((slab + src.x) >> 14) * 4);
    S.w = gload_b128(pk, src.x >> 1);
    if constexpr (REST > 0) {
      S.q8b = gload_u8(q8, src.x4 >> 6);
      S.a2b = gload_f32(a.absmax2, ((slab + src.x4) >> 14) * 4);
      S.w4 = gload_b32(pk, src.x4 >> 1);
    }
  }

  __device__ static __forceinline__ void ready(Stage& S) {
    vm_ready(S.w);
    vm_ready(S.q8);
    vm_ready(S.a2);
    if constexpr (REST > 0) {
      vm_ready(S.w4);
      vm_ready(S.q8b);
      vm_ready(S.a2b);
    }
  }

  struct Looked {
    float2_t pr[4][4];
    float2_t pb[4];
    float c, cb;
  };

  __device__ static __forceinline__ void lookup(const Stage& S, Looked& L, const float2_t* s_pair,
                                                const float* s_code) {
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
      for (int j = 0; j < 4; j++) L.pr[d][j] = s_pair[(S.w[d] >> (8 * j)) & 0xffu];
    L.c = s_code[S.q8];
    if constexpr (REST > 0) {
#pragma unroll
      for (int j = 0; j < 4; j++) L.pb[j] = s_pair[(S.w4 >> (8 * j)) & 0xffu];
      L.cb = s_code[S.q8b];
    }
  }

  __device__ static __forceinline__ void finish(const Stage& S, const Looked& L, _Float16* bs,
                                                int p, float offset) {
    {
      const int q = p;  // < TOTAL
      const int row = item_row(q), c = item_chunk(q);
      const float sc = nested_scale(L.c, S.a2, offset);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = pack_f16x2(L.pr[d][j][0] * sc, L.pr[d][j][1] * sc);
        *reinterpret_cast<u32x4*>(bs + bt_off(row, 32 * c + 8 * d, LDB)) = v;
      }
    }
    if constexpr (REST > 0) {
      const int row = p >> 2, sub = p & 3;
      const float sc = nested_scale(L.cb, S.a2b, offset);
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = pack_f16x2(L.pb[j][0] * sc, L.pb[j][1] * sc);
      *reinterpret_cast<u32x4*>(bs + bt_off(row, C16 + 8 * sub, LDB)) = v;
    }
  }
};

// NF4 side of a forward K-step for 512 producer threads (tiles up to 128 columns): item = 8
// packed bytes of W row n (16 values, a quarter of the row's block for this K-step), 3 memory
// instructions; same addressing scheme as BLoad.  A 96-row tile leaves producer waves 6 and 7
// without items.  Evening out the decode per SIMD (waves 4-7 on 4-byte items) was measured and
// rejected: the 4-byte items' fixed per-item cost made those waves slower than the imbalance it
// removed.
template <int BN>
struct BLoad8 {
  static constexpr int TOTAL = BN * 4;  // 8-byte items
  static constexpr int VMEM = 3;
  static_assert(TOTAL % 64 == 0 && TOTAL <= 512, "B items in whole waves, one round");

  struct Stage {
    u32x2 w;
    uint32_t q8;
    float a2;
  };
  struct Src {
    uint32_t w, blk;
  };

  // swap: the tile's columns (W's rows) in rope_col order
  __device__ static __forceinline__ Src setup(const GemmArgs& a, int p, int n0,
                                              bool swap = false) {
    Src r;
    const int q = p;  // the caller runs only lanes with an item (p < TOTAL)
    const int c = n0 + (q >> 2);
    const uint32_t n = min(swap ? rope_col(c) : c, a.Nc - 1);
    r.w = n * (uint32_t)(a.Kw / 2) + (q & 3) * 8;
    r.blk = n * (uint32_t)(a.Kw / 64);
    return r;
  }

  __device__ static __forceinline__ void issue(const GemmArgs& a, const Src& src, Stage& S,
                                               int kt) {
    const uint8_t* pk = a.packed + kt * (kBK / 2);
    S.q8 = gload_u8(a.absmax8 + kt, src.blk);
    S.a2 = gload_f32(a.absmax2, ((src.blk + kt) >> 8) * 4);
    S.w = gload_b64(pk, src.w);
  }

  __device__ static __forceinline__ void ready(Stage& S) {
    vm_ready(S.w);
    vm_ready(S.q8);
    vm_ready(S.a2);
  }

  struct Looked {
    float2_t pr[2][4];
    float c;
  };

  __device__ static __forceinline__ void lookup(const Stage& S, Looked& L, const float2_t* s_pair,
                                                const float* s_code) {
#pragma unroll
    for (int d = 0; d < 2; d++)
#pragma unroll
      for (int j = 0; j < 4; j++) L.pr[d][j] = s_pair[(S.w[d] >> (8 * j)) & 0xffu];
    L.c = s_code[S.q8];
  }

  __device__ static __forceinline__ void finish(const Stage& S, const Looked& L, _Float16* bs,
                                                int p, float offset) {
    {
      const int q = p;  // < TOTAL
      const float sc = nested_scale(L.c, S.a2, offset);
#pragma unroll
      for (int d = 0; d < 2; d++) {
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = pack_f16x2(L.pr[d][j][0] * sc, L.pr[d][j][1] * sc);
        *reinterpret_cast<u32x4*>(bs + lds_off(q >> 2, (q & 3) * 2 + d)) = v;
      }
    }
  }
};

// NF4 side of a backward K-step for 512 producer threads (tiles up to 128 columns), B tile
// stored as W's rows like BLoadT: item = 8 packed bytes of one W row (16 columns, one block
// scale), decoded to two contiguous 16-byte stores.
template <int BN>
struct BLoadT8 {
  static constexpr int LDB = BLoadT<BN>::LDB;
  static constexpr int CPR = BN / 16;       // 8-byte items per row
  static constexpr int TOTAL = kBK * CPR;
  static constexpr int VMEM = 3;
  static_assert(BN % 16 == 0 && TOTAL % 64 == 0 && TOTAL <= 512, "B items in whole waves");
  // item -> (row, 16-column chunk), as BLoadT maps its items
  __device__ static __forceinline__ int item_row(int q) {
    return LDB == 96 ? 16 * (q / (16 * CPR)) + (q & 15) : q / CPR;
  }
  __device__ static __forceinline__ int item_chunk(int q) {
    return LDB == 96 ? (q >> 4) % CPR : q % CPR;
  }

  struct Stage {
    u32x2 w;
    uint32_t q8;
    float a2;
  };
  struct Src {
    uint32_t x;  // value index of the item within its K-step's 64-row slab of W
  };

  __device__ static __forceinline__ Src setup(const GemmArgs& a, int p, int n0) {
    Src r;
    const int q = p;  // the caller runs only lanes with an item (p < TOTAL)
    const int row = item_row(q), c = item_chunk(q);
    r.x = (uint32_t)row * a.Kw + min(n0 + 16 * c, a.Nc - 16);
    return r;
  }

  __device__ static __forceinline__ void issue(const GemmArgs& a, const Src& src, Stage& S,
                                               int kt) {
    const uint32_t slab = (uint32_t)kt * kBK * a.Kw;
    const uint8_t* pk = a.packed + slab / 2;
    S.q8 = gload_u8(a.absmax8 + slab / 64, src.x >> 6);
    S.a2 = gload_f32(a.absmax2, ((slab + src.x) >> 14) * 4);
    S.w = gload_b64(pk, src.x >> 1);
  }

  __device__ static __forceinline__ void ready(Stage& S) {
    vm_ready(S.w);
    vm_ready(S.q8);
    vm_ready(S.a2);
  }

  struct Looked {
    float2_t pr[2][4];
    float c;
  };

  __device__ static __forceinline__ void lookup(const Stage& S, Looked& L, const float2_t* s_pair,
                                                const float* s_code) {
#pragma unroll
    for (int d = 0; d < 2; d++)
#pragma unroll
      for (int j = 0; j < 4; j++) L.pr[d][j] = s_pair[(S.w[d] >> (8 * j)) & 0xffu];
    L.c = s_code[S.q8];
  }

  __device__ static __forceinline__ void finish(const Stage& S, const Looked& L, _Float16* bs,
                                                int p, float offset) {
    {
      const int q = p;  // < TOTAL
      const int row = item_row(q), c = item_chunk(q);
      const float sc = nested_scale(L.c, S.a2, offset);
#pragma unroll
      for (int d = 0; d < 2; d++) {
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = pack_f16x2(L.pr[d][j][0] * sc, L.pr[d][j][1] * sc);
        *reinterpret_cast<u32x4*>(bs + bt_off(row, 16 * c + 8 * d, LDB)) = v;
      }
    }
  }
};

// LDS halfs of the warp-specialized kernel: 3-deep A ring + 2-deep B buffer + the staged LoRA
// operands ([BM][16] and [BN][16]).
template <int BM, int BN, bool BWD>
constexpr int ws_lds_halfs() {
  return 3 * BM * kBK + 2 * (BWD ? kBK * BLoadT<BN>::LDB : BN * kBK) + (BM + BN) * 16;
}

// Direct global -> LDS copy of one K-step's A tile (BM rows x 64 fp16) by the producer waves:
// each global_load_lds_dwordx4 writes 8 rows (64 lanes x 16 B, consecutive in LDS); lane l takes
// the logical segment that the row's XOR swizzle places at its physical slot.  Producer wave pw
// of PW copies row groups pw, pw + PW, ...  Each lane's source byte offsets from the tile's
// first row are
// computed once (32-bit: the launcher checks BM * lda * 2 < 2^32); a K-step only moves the
// uniform source pointer and the ring slot, so a copy costs two scalar instructions and the
// load.
// M0 is a reserved register to the compiler; the copy below writes it on purpose (see there)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int BM, int PW>
struct ACopy {
  static constexpr int N = BM / 8 / PW;  // copies per producer wave per K-step
  static_assert(BM % (8 * PW) == 0, "whole row groups per producer wave");
  uint32_t off[N];
  const char* base;  // A row m0 (uniform)
  uint32_t lds;      // LDS byte address of this wave's first row group in ring slot 0 (uniform)

  __device__ __forceinline__ void init(const GemmArgs& a, const _Float16* as, int pw, int lane,
                                       int m0) {
#pragma unroll
    for (int i = 0; i < N; i++) {
      const int row = (pw + PW * i) * 8 + (lane >> 3);
      const int seg = ((lane & 7) ^ (row >> 1)) & 7;
      const uint32_t m = min(m0 + row, a.M - 1) - m0;
      off[i] = (m * (uint32_t)a.lda + seg * 8) * 2;
    }
    base = reinterpret_cast<const char*>(a.A + (int64_t)m0 * a.lda);
    lds = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as + pw * 8 * kBK)));
  }

  // copy K-step kt into ring slot `slot_bytes` (byte offset of the slot from slot 0)
  __device__ __forceinline__ void copy(uint32_t slot_bytes, int kt) const {
    const char* src = base + (size_t)kt * kBK * sizeof(_Float16);
#pragma unroll
    for (int i = 0; i < N; i++) {
      // Inline asm rather than __builtin_amdgcn_global_load_lds: the compiler cannot tell
      // these LDS writes from the producers' table reads and would drain every outstanding
      // load before each of those reads.  Completion is awaited explicitly (wait_vmcnt) before
      // the barrier that hands the tile over.  M0 = the LDS destination of this wave's 8 rows;
      // no other code in the kernel uses M0.
      const uint32_t dst = lds + slot_bytes + i * PW * 8 * kBK * sizeof(_Float16);
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :
                   : "s"(dst), "v"(off[i]), "s"(src)
                   : "memory", "m0");
    }
  }
};

// The A-tile copies issued by the 4 consumer waves instead (between their MFMAs, where the wave
// has issue slots to spare): wave w copies the 8-row groups w, w + 4, ... of the tile.  Under the
// segment swizzle those groups share one physical-slot assignment per lane, so a copy's source
// offset is min(row, last row) * row bytes + that lane's segment: three VALU per copy, computed
// when issued rather than held in registers the MFMA operands need.
template <int BM>
struct ACopyC {
  static constexpr int N = BM / 32;  // copies per consumer wave per K-step
  const char* base;   // A row m0 (uniform)
  uint32_t lds;       // LDS byte address of this wave's first row group in ring slot 0 (uniform)
  uint32_t rowbase;   // the lane's row within its wave's first group
  uint32_t seg16;     // byte offset of the lane's logical segment within a row
  uint32_t last;      // last valid row of the tile, relative to m0 (uniform)
  uint32_t ldab;      // bytes per A row (uniform)

  __device__ __forceinline__ void init(const GemmArgs& a, const _Float16* as, int w, int lane,
                                       int m0) {
    rowbase = w * 8 + (lane >> 3);
    seg16 = (((lane & 7) ^ (rowbase >> 1)) & 7) * 16;
    last = __builtin_amdgcn_readfirstlane((uint32_t)(min(m0 + BM, a.M) - 1 - m0));
    ldab = __builtin_amdgcn_readfirstlane((uint32_t)a.lda * 2);
    base = reinterpret_cast<const char*>(a.A + (int64_t)m0 * a.lda);
    lds = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as + w * 8 * kBK)));
  }

  // copy i (0 <= i < N) of K-step kt into ring slot `slot_bytes`
  __device__ __forceinline__ void copy(uint32_t slot_bytes, int kt, int i) const {
    copy_from(base, ldab, slot_bytes, kt, i);
  }

  // the same from another problem's A (row m0 at base_, ldab_ bytes per row; same rows)
  __device__ __forceinline__ void copy_from(const char* base_, uint32_t ldab_,
                                            uint32_t slot_bytes, int kt, int i) const {
    const char* src = base_ + (size_t)kt * kBK * sizeof(_Float16);
    const uint32_t off = min(rowbase + 32u * i, last) * ldab_ + seg16;
    const uint32_t dst = lds + slot_bytes + i * 32 * kBK * sizeof(_Float16);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(dst), "v"(off), "s"(src)
                 : "memory", "m0");
  }
};
#pragma clang diagnostic pop

// Who issues the A-tile copies of a warp-specialized kernel: the consumer waves, between their
// MFMAs, except in the 256-row tiles with 8 producer waves (12 waves per CU leave the consumers
// too few registers: the copies' offsets spill there).  Measured at 1024 tokens against the
// producers issuing them: 2-7 % faster on the gate/up forward, down_proj forward and dX and the
// 128x128 dX; 3 % slower on the 256x96 8-producer dX, which keeps them on its producers.
template <int BM, int PW>
constexpr bool consumer_copies() {
  return !(BM == 256 && PW == 8);
}

// Warp-specialized kernel: 4 consumer waves (one per SIMD, CWM x CWN over the BM x BN tile)
// read LDS fragments and issue MFMAs; PW producer waves decode the NF4 of K-step kt+1 into the
// other half of a 2-deep B buffer while the consumers multiply kt.  The A tile of kt+2 goes
// straight into a 3-deep LDS ring by direct-to-LDS copies, issued by the consumers between their
// MFMAs or by the producers (consumer_copies).  Everything issued in one K-step is waited for
// at the start of the next, and one workgroup barrier per K-step hands the buffers over.  Wave
// roles are uniform branches, so neither side's registers live through the other's code.
// One output tile (bx, by) of the warp-specialized GEMM; split index blockIdx.z - a.zf, partial
// plane blockIdx.z.
// Backward tiles whose output is the sum of up to kMaxSum problems' input gradients (autograd
// adds them for their shared input): their reductions run back to back in one K loop into one
// accumulator.  Problem q owns K-steps [end[q-1], end[q]); a[0] carries the output.
constexpr int kMaxSum = 3;
struct SumPlan {
  int n;
  int end[kMaxSum];
};

// The warp-specialized tile.  NSUM = 1: one problem `as[0]`.  NSUM > 1: the summed problems of
// `plan` (as[0 .. plan->n)): every K-step takes its operands (dY, the NF4 weight, its code
// table and offset) from its problem, and the accumulator starts from all their LoRA terms.
// The problems share M, the output width and the weight row length, LoRA rank 16 and the keep
// mask's presence; the A copies are the consumers' (consumer_copies).
// ROPE: the forward tile of a grouped launch whose problems may ask for the RoPE of attention's
// q / k (GemmArgs::rope_cos): such a tile's columns are in rope_col order and its epilogue
// rotates (rope_rotate).
template <int BM, int BN, int CWM, int CWN, bool BWD, int PW, int NS, bool GLU, int NSUM,
          bool ROPE = false>
__device__ __forceinline__ void ws_tile_impl(const GemmArgs* as, const SumPlan* plan, int bx,
                                             int by) {
  const GemmArgs& a = as[0];
  constexpr int WM = BM / CWM, WN = BN / CWN, TM = WM / 32, TN = WN / 32;
  static_assert(!ROPE || (!BWD && !GLU && NSUM == 1 && PW == 8 && TN == 2),
                "RoPE tiles: forward, 8 producer waves, two 32-column blocks per wave");
  const bool swap = ROPE && a.rope_cos != nullptr;
  constexpr int NTP = 64 * PW;  // producer threads
  static_assert(CWM * CWN == 4 && WM % 32 == 0 && WN % 32 == 0, "consumer wave tiles");
  static_assert(PW == 4 || PW == 8, "4 or 8 producer waves");
  using B = std::conditional_t<
      BWD, std::conditional_t<PW == 8, BLoadT8<BN>, BLoadT<BN>>,
      std::conditional_t<PW == 8, BLoad8<BN>, BLoad<BN>>>;
  constexpr int LDB = BWD ? BLoadT<BN>::LDB : 0;  // B tile stored [64][LDB] (backward)
  constexpr int LDS_A = BM * kBK, LDS_B = BWD ? kBK * LDB : BN * kBK;
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  _Float16* As = smem;                      // [3][BM][64]
  _Float16* Bs = smem + 3 * LDS_A;          // [2][BN][64]
  _Float16* Ls = Bs + 2 * LDS_B;            // LoRA operands: [BM][16], then [BN][16]
  // B buffer of K-step parity x: buffer 1 sits right after A-ring slot 2, so that the two
  // (both idle until K-step kt0 multiplies) can hold the staged keep mask
  auto bbuf = [&](int x) { return Bs + ((x & 1) ^ 1) * LDS_B; };
  uint8_t* Ks = reinterpret_cast<uint8_t*>(As + 2 * LDS_A);
  static_assert(BM * MaskStage<BM, BN, NTP>::KST <= (LDS_A + LDS_B) * 2, "staged keep mask fits");
  static_assert(NSUM == 1 || (BWD && !GLU && consumer_copies<BM, PW>()), "summed tiles");
  __shared__ float2_t s_pair[256];
  __shared__ float s_code[256 * NSUM];  // problem q's code book at 256 q
  __shared__ float s_off[NSUM];         // summed tiles: problem q's absmax offset
  // summed problems: their count, the problem of K-step k and its first K-step
  const int nsum = NSUM == 1 ? 1 : plan->n;
  auto prob = [&](int k) -> int {
    int q = 0;
    if constexpr (NSUM > 1) {
#pragma unroll
      for (int i = 0; i + 1 < NSUM; i++) q += (i + 1 < nsum && k >= plan->end[i]) ? 1 : 0;
    }
    return q;
  };
  auto first = [&](int q) -> int {
    if constexpr (NSUM == 1) return 0;
    else return q == 0 ? 0 : plan->end[q - 1];
  };
  // the extra LoRA operand and keep mask areas of problems 1.. (after the single-problem LDS)
  constexpr int KSTH = BM * MaskStage<BM, BN, NTP>::KST / 2;  // keep-mask halfs
  constexpr int XTRA = (BM + BN) * 16 + KSTH;
  static_assert(XTRA % 8 == 0 && ws_lds_halfs<BM, BN, BWD>() % 8 == 0, "16-byte areas");
  auto ls_of = [&](int q) -> _Float16* {
    return q == 0 ? Ls : smem + ws_lds_halfs<BM, BN, BWD>() + (q - 1) * XTRA;
  };

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int m0 = by * BM;
  const int n0 = bx * BN;
  const int n_steps = NSUM == 1 ? a.Kr / kBK : plan->end[nsum - 1];
  const int kt0 = ((int)blockIdx.z - a.zf) * a.steps_per_split;
  const int kt1 = min(n_steps, kt0 + a.steps_per_split);
  // the producers stage the LoRA operands (r = 16) and the keep mask in LDS for the consumers
  const bool lora = (int)blockIdx.z == a.zf && (a.lora_hp || a.lora_h);
  const bool lora16 = lora && a.r == 16;
  const bool kmask = BWD && lora && a.mask;
  // wave index as a scalar: the producer / consumer split below is a uniform branch, so neither
  // side's live registers are carried through the other side's code
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm0 = (wave / CWN) * WM;
  const int wn0 = (wave % CWN) * WN;
  const int lrow = lane & 31;
  const int lseg = lane >> 5;

  if (wave >= 4) {
    // ---- producers (they stay to the end: every wave takes part in every barrier) ----
    const int p = t - 256;
    const int pw = p >> 6;
    const bool run = kt0 < kt1;
    LoraStage<BM, BN, NTP> lst[NSUM];
    MaskStage<BM, BN, NTP> mst[NSUM];
    if (lora16) lst[0].issue(a, p, m0, n0, swap);  // before the tiles: one round trip for all
    if (kmask) mst[0].issue(a, p, m0, n0);
#pragma unroll
    for (int q = 1; q < NSUM; q++) {
      if (q >= nsum) break;
      if (lora16) lst[q].issue(as[q], p, m0, n0);
      if (kmask) mst[q].issue(as[q], p, m0, n0);
    }
    // the offset of K-step k's problem: a register with one problem; in a summed tile read
    // from LDS (s_off, written with the tables), not an indexed register array (which would
    // live in scratch memory and make the compiler wait for every load in flight)
    const float off0 = NSUM == 1 ? a.offset[0] : 0.0f;
    auto offset_at = [&](int k) -> float {
      if constexpr (NSUM == 1) return off0;
      else return s_off[prob(k)];
    };
    auto code_at = [&](int k) -> const float* { return s_code + 256 * prob(k); };
    auto commit_staged = [&]() {
      if (lora16) lst[0].commit(a, Ls, p);
      if (kmask) mst[0].commit(Ks, p);
#pragma unroll
      for (int q = 1; q < NSUM; q++) {
        if (q >= nsum) break;
        _Float16* lq = ls_of(q);
        if (lora16) lst[q].commit(as[q], lq, p);
        if (kmask) mst[q].commit(reinterpret_cast<uint8_t*>(lq + (BM + BN) * 16), p);
      }
    };
    // NF4 tile of K-step kt is issued NS steps ahead into register stage (kt - kt0) % NS; its
    // table lookups are issued one step ahead, right after the previous tile is finished, so
    // their LDS latency overlaps the loads and barrier of that step; it is finished (scaled,
    // converted, written to LDS) one step ahead of its multiply.  The A tile is copied two
    // steps ahead into the LDS ring.
    // Every producer wave copies its share of A.  Waves with B items decode them; whole waves
    // past the items (a 96-column tile leaves two of eight) only copy: decoding a duplicate
    // item there would take issue slots from the multiplying wave of the same SIMD.  (Handing
    // the whole A tile to those two waves instead measured slower: all copies then issue
    // from two SIMDs.)
    // Decoding wave, order within step kt: finish B(kt+1), look up B(kt+2), copy A(kt+2),
    // issue B(kt+NS), wait A(kt+1).  So in issue order A(j) comes right before B(j+NS-2), and
    // the prologue keeps that order: B(kt0) .. B(kt0+NS-3), A(kt0), B(kt0+NS-2), A(kt0+1),
    // B(kt0+NS-1).  A load of B gets NS-2 steps to land.
    // The B loads are inline asm like the copies: every wait here is counted by hand over both
    // (vmcnt counts in issue order), and the compiler adds none of its own, which, blind to the
    // copies, would drain the copy of A(kt+1) along with B(kt+2).  Every issue is unconditional
    // (steps past the end re-load the last one), so the number of memory instructions in
    // flight is a constant and each wait names exactly the group it needs.
    constexpr bool CC = consumer_copies<BM, PW>();
    using AC = ACopy<BM, PW>;
    constexpr int LA = CC ? 0 : AC::N;  // A-tile copy instructions per producer wave and step
    constexpr uint32_t SLOT = LDS_A * sizeof(_Float16);
    const int last = kt1 - 1;
    // the branch is uniform and taken once; both paths pass the same barriers
    if (B::TOTAL >= NTP || __builtin_amdgcn_readfirstlane(p) < B::TOTAL) {
      constexpr int LB = B::VMEM;
      static_assert(NS >= 4 && NS * LB + 2 * LA <= 63, "stages: at least 4; waits fit vmcnt");
      AC ac;
      if constexpr (!CC) ac.init(a, As, pw, lane, m0);
      const typename B::Src src = [&] {
        if constexpr (ROPE) return B::setup(a, p, n0, swap);
        else return B::setup(a, p, n0);
      }();
      typename B::Stage S[NS];
      typename B::Looked L;
      // B of K-step k from its problem's weight
      auto issue = [&](typename B::Stage& St, int k) {
        if constexpr (NSUM == 1) {
          B::issue(a, src, St, k);
        } else {
          const int q = prob(k);
          B::issue(as[q], src, St, k - first(q));
        }
      };
      if (run) {
#pragma unroll
        for (int u = 0; u < NS - 2; u++) issue(S[u], min(kt0 + u, last));
        if constexpr (!CC) ac.copy(0, kt0);
        issue(S[NS - 2], min(kt0 + NS - 2, last));
        if constexpr (!CC) ac.copy(SLOT, min(kt0 + 1, last));
        issue(S[NS - 1], min(kt0 + NS - 1, last));
      }
      if (lora16 || kmask) {
        if (run) wait_vmcnt<NS * LB + 2 * LA>();  // the staged loads, issued before all of those
        else wait_vmem_all();
        commit_staged();
      }
      lds_barrier();  // tables, LoRA operands
      if (run) {
        wait_vmcnt<(NS - 1) * LB + 2 * LA>();  // B(kt0)
        B::ready(S[0]);
        B::lookup(S[0], L, s_pair, code_at(kt0));
        B::finish(S[0], L, bbuf(0), p, offset_at(kt0));
        wait_vmcnt<2 * LB + LA>();  // A(kt0) and what precedes it (B(kt0+1) among them)
        B::ready(S[1]);
        B::lookup(S[1], L, s_pair, code_at(min(kt0 + 1, last)));
        lds_barrier();  // K-step kt0 ready
        // Sc = B(kt+1) (looked up in L), Sn = B(kt+2), Si = the stage of B(kt), free for B(kt+NS)
        auto step = [&](int kt, typename B::Stage& Sc, typename B::Stage& Sn,
                        typename B::Stage& Si) {
          const int r = kt - kt0;
          // Unconditional: past the end the stages hold the last K-step again and bbuf(r + 1) is
          // the buffer of step kt - 1, no longer read; branches here would only give the
          // compiler paths to merge.
          B::finish(Sc, L, bbuf(r + 1), p, offset_at(min(kt + 1, last)));
          // B(kt+2); after it A(kt+5-NS) .. A(kt+1) and B(kt+3) .. B(kt+NS-1)
          wait_vmcnt<(NS - 3) * (LA + LB)>();
          B::ready(Sn);
          B::lookup(Sn, L, s_pair, code_at(min(kt + 2, last)));
          if constexpr (!CC) ac.copy(((r + 2) % 3) * SLOT, min(kt + 2, last));
          issue(Si, min(kt + NS, last));
          // A(kt+1); after it only B(kt+NS-1), A(kt+2), B(kt+NS)
          if constexpr (!CC) wait_vmcnt<2 * LB + LA>();
          lds_barrier();
          // nothing of the next step moves above this point (its arithmetic on the next stage
          // would then sit before the copies of this step in the schedule)
          __builtin_amdgcn_sched_barrier(0);
        };
        int kt = kt0;
        for (; kt + NS <= kt1; kt += NS) {
#pragma unroll
          for (int u = 0; u < NS; u++) step(kt + u, S[(u + 1) % NS], S[(u + 2) % NS], S[u]);
        }
        // no path reaches a step without the one before it (whose wait and ready() the next
        // step's stage relies on)
#pragma unroll
        for (int u = 0; u < NS - 1; u++) {
          if (kt + u >= kt1) break;
          step(kt + u, S[(u + 1) % NS], S[(u + 2) % NS], S[u]);
        }
        wait_vmem_all();  // no copy into the A ring may still be in flight
        // The stages loaded past the end are never looked up: this use keeps their registers
        // allocated until the loads writing them have landed.
#pragma unroll
        for (int u = 0; u < NS; u++) B::ready(S[u]);
      }
    } else if constexpr (CC) {
      // no B items and no copies: the staged LoRA operands, then every barrier of the tile
      if (lora16 || kmask) {
        wait_vmem_all();  // the staged loads
        commit_staged();
      }
      lds_barrier();  // tables, LoRA operands
      if (run) {
        lds_barrier();  // K-step kt0 ready
        for (int kt = kt0; kt < kt1; kt++) lds_barrier();
      }
    } else {
      AC ac;
      ac.init(a, As, pw, lane, m0);
      if (run) {
        ac.copy(0, kt0);
        ac.copy(SLOT, min(kt0 + 1, last));
      }
      if (lora16 || kmask) {
        wait_vmem_all();  // the staged loads (issued before the copies)
        commit_staged();
      }
      lds_barrier();  // tables, LoRA operands
      if (run) {
        wait_vmcnt<LA>();  // A(kt0); after it only A(kt0+1)
        lds_barrier();     // K-step kt0 ready
        for (int kt = kt0; kt < kt1; kt++) {
          const int r = kt - kt0;
          ac.copy(((r + 2) % 3) * SLOT, min(kt + 2, last));
          wait_vmcnt<LA>();  // A(kt+1); after it only A(kt+2)
          lds_barrier();
        }
        wait_vmem_all();  // no copy into the A ring may still be in flight
      }
    }
    if constexpr (GLU) {
      // Nothing is in flight here.  This wait says so to a path-insensitive reading too, which
      // could pair the issuing prologue with a skipped main loop (the two test one `run`).
      wait_vmem_all();
      if (gridDim.z == 1) {
        GluTail<BM, BN, CWM, CWN, NTP, BWD> glu;
        glu.prefetch(a, p, m0, n0);  // in flight across both barriers
        lds_barrier();               // the A ring is free for the consumers' staged tile
        lds_barrier();               // the tile is staged
        glu.store(a, p, m0, n0, reinterpret_cast<const uint32_t*>(As));
        return;
      }
    }
    lds_barrier();  // the A ring is free for the consumers' staged epilogue
  } else {
    // ---- consumers ----
    constexpr bool CC = consumer_copies<BM, PW>();
    using AC = ACopyC<BM>;
    constexpr int LA = AC::N;
    constexpr uint32_t SLOT = LDS_A * sizeof(_Float16);
    const int lastk = kt1 - 1;
    AC ac;
    if constexpr (CC) ac.init(a, As, wave, lane, m0);
    // the summed problems' dY rows m0 and row bytes (uniform), selected per K-step by constant
    // indices (so the array stays in scalar registers)
    const char* abase[NSUM];
    uint32_t aldab[NSUM];
    if constexpr (NSUM > 1) {
#pragma unroll
      for (int q = 0; q < NSUM; q++) {
        if (q >= nsum) break;
        abase[q] = reinterpret_cast<const char*>(as[q].A + (int64_t)m0 * as[q].lda);
        aldab[q] = __builtin_amdgcn_readfirstlane((uint32_t)as[q].lda * 2);
      }
    }
    // copy i of K-step k (in a summed tile, from its problem's dY)
    auto acopy = [&](uint32_t slot, int k, int i) {
      if constexpr (NSUM == 1) {
        ac.copy(slot, k, i);
      } else {
        const int q = prob(k);
        const char* b = abase[0];
        uint32_t l = aldab[0];
#pragma unroll
        for (int j = 1; j < NSUM; j++) {
          b = q == j ? abase[j] : b;
          l = q == j ? aldab[j] : l;
        }
        ac.copy_from(b, l, slot, k - first(q), i);
      }
    };
    if constexpr (CC) {
      if (kt0 < kt1) {
#pragma unroll
        for (int i = 0; i < LA; i++) acopy(0, kt0, i);
#pragma unroll
        for (int i = 0; i < LA; i++) acopy(SLOT, min(kt0 + 1, lastk), i);
      }
    }
    AccStart<TM, TN, BWD, ROPE> start;
    start.swap = swap;
    start.load(a, n0 + wn0, lseg);  // before the tables' loads
    fill_tables(a, s_pair, s_code, t, 256);
#pragma unroll
    for (int q = 1; q < NSUM; q++) {
      if (q >= nsum) break;
      for (int i = t; i < 256; i += 256) s_code[256 * q + i] = as[q].code[i];
    }
    if constexpr (NSUM > 1) {
#pragma unroll
      for (int q = 0; q < NSUM; q++) {
        if (q >= nsum) break;
        if (t == q) s_off[q] = as[q].offset[0];
      }
    }
    float16_t acc[TM][TN];
    lds_barrier();  // tables, LoRA operands
    // accumulator start (bias, LoRA) while the producers stage K-step kt0
    if (lora16)
      start.finish_staged(a, acc, m0 + wm0, n0 + wn0, lrow, lseg, wm0, wn0, Ls, BM,
                          kmask ? Ks : nullptr, MaskStage<BM, BN, NTP>::KST);
    else
      start.finish(a, acc, m0 + wm0, n0 + wn0, lrow, lseg, wm0, wn0, nullptr, 0,
                   kmask ? Ks : nullptr, MaskStage<BM, BN, NTP>::KST);
    // the other summed problems' LoRA terms, each masked by its own keep bits, added in order
#pragma unroll
    for (int q = 1; q < NSUM; q++) {
      if (q >= nsum) break;
      float16_t part[TM][TN];
      const _Float16* lq = ls_of(q);
      start.finish_staged(as[q], part, m0 + wm0, n0 + wn0, lrow, lseg, wm0, wn0, lq, BM,
                          kmask ? reinterpret_cast<const uint8_t*>(lq + (BM + BN) * 16) : nullptr,
                          MaskStage<BM, BN, NTP>::KST);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] += part[i][j];
    }
    if (kt0 < kt1) {
      if constexpr (CC) wait_vmcnt<LA>();  // A(kt0); after it only A(kt0+1)
      lds_barrier();                        // K-step kt0 ready
      // Operand fragments of one 16-deep sub-step in two register sets.  The last sub-step of
      // each K-step is multiplied after the barrier that ends it (its fragments are read
      // before), so the reads of the next step's first fragments overlap those MFMAs instead
      // of leaving the MFMA pipe idle behind the barrier.
      half8_t fa[2][TM], fb[2][TN];
      // Per-lane fragment offsets, computed once.  Rows 32 apart share their swizzle
      // ((row >> 1) & 7 with wm0, wn0 multiples of 32; in a backward tile, bt_off's unit XOR
      // for reduction rows 16 apart and columns 32 apart), so the 32-row blocks and the
      // sub-steps of a fragment read are compile-time offsets from one register per operand
      // and sub-step, not one address register per fragment.
      const int xs = (lrow >> 1) & 7;
      int aoff[4], boff[4];  // halfs: lane's A / B (forward) fragment of sub-step kk, block 0
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const int seg = (((2 * kk + lseg) ^ xs) & 7) << 3;
        aoff[kk] = (wm0 + lrow) * kBK + seg;
        boff[kk] = (wn0 + lrow) * kBK + seg;
      }
      int btlo = 0, bthi = 0;  // backward tile: the lane's two 8-byte reads, block 0, kk 0
      if constexpr (LDB > 0) {
        const int g = lane >> 4, sl = lane & 15;
        const int kl = 8 * (g >> 1) + (sl >> 2), nl = 16 * (g & 1) + 4 * (sl & 3);
        btlo = bt_off(kl, wn0 + nl, LDB);
        bthi = bt_off(kl + 4, wn0 + nl, LDB);
      }
      typedef __attribute__((address_space(3))) short4_t lds_short4;
      auto load = [&](int set, const _Float16* as, const _Float16* bs, int kk) {
#pragma unroll
        for (int i = 0; i < TM; i++)
          fa[set][i] = *reinterpret_cast<const half8_t*>(as + aoff[kk] + i * 32 * kBK);
#pragma unroll
        for (int j = 0; j < TN; j++) {
          if constexpr (LDB > 0) {
            const _Float16* b = bs + 16 * kk * LDB + 32 * j;
            const half4_t lo = __builtin_bit_cast(
                half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(b + btlo)));
            const half4_t hi = __builtin_bit_cast(
                half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(b + bthi)));
            fb[set][j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          } else {
            fb[set][j] = *reinterpret_cast<const half8_t*>(bs + boff[kk] + j * 32 * kBK);
          }
        }
      };
      auto mma = [&](int set) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[set][j], fa[set][i],
                                                               acc[i][j], 0, 0, 0);
      };
      // Issue order of one sub-step: a fragment read of the next sub-step after each MFMA of
      // this one.  Left alone, the scheduler puts every read right before the MFMA that uses
      // it (fewer live registers) and the MFMA pipe idles through each read's latency.
      constexpr int NRD = TM + TN * (LDB > 0 ? 2 : 1);  // LDS read instructions per sub-step
      constexpr int NMF = TM * TN;                      // MFMAs per sub-step
      auto interleave = [&]() {
#pragma unroll
        for (int q = 0; q < (NRD > NMF ? NRD : NMF); q++) {
          if (q < NMF) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          if (q < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        }
      };
      load(0, As, bbuf(0), 0);
      for (int kt = kt0; kt < kt1; kt++) {
        const int r = kt - kt0;
        const _Float16* as = As + (r % 3) * LDS_A;
        const _Float16* bs = bbuf(r);
#pragma unroll
        for (int kk = 0; kk < 3; kk++) {
          load((kk + 1) & 1, as, bs, kk + 1);
          mma(kk & 1);
          interleave();
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (CC) {
            // A(kt+2) into the ring slot step kt-1 used, spread over the sub-steps
#pragma unroll
            for (int i = kk * LA / 3; i < (kk + 1) * LA / 3; i++)
              acopy(((r + 2) % 3) * SLOT, min(kt + 2, lastk), i);
          }
        }
        if constexpr (CC) wait_vmcnt<LA>();  // A(kt+1); after it only A(kt+2)
        lds_barrier();  // (its lgkmcnt(0) covers sub-step 3's fragments)
        // step kt+1's first fragments (past the end: stale slots, read and never used)
        load(0, As + ((r + 1) % 3) * LDS_A, bbuf(r + 1), 0);
        mma(1);  // sub-step 3 of step kt
        interleave();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (CC) wait_vmem_all();  // no copy into the A ring may still be in flight
    lds_barrier();  // the last copies have landed
    static_assert(4 * StagedStore<TM, TN>::AREA_DWORDS * 4 <= 3 * LDS_A * 2,
                  "staged epilogue areas fit in the A ring");
    if constexpr (GLU) {
      using G = GluTail<BM, BN, CWM, CWN, NTP, BWD>;
      static_assert(4 * G::AREA * 4 <= 3 * LDS_A * 2, "the staged tile fits in the A ring");
      if (gridDim.z == 1) {
        G::stage(acc, lane, reinterpret_cast<uint32_t*>(As) + wave * G::AREA);
        lds_barrier();  // the tile is staged for the producers
        return;
      }
    }
    epilogue_staged<TM, TN, ROPE>(a, acc, m0 + wm0, n0 + wn0, lane,
                                  reinterpret_cast<float*>(As) +
                                      wave * StagedStore<TM, TN>::AREA_DWORDS);
  }
}

template <int BM, int BN, int CWM, int CWN, bool BWD, int PW, int NS, bool GLU,
          bool ROPE = false>
__device__ __forceinline__ void ws_tile(const GemmArgs& a, int bx, int by) {
  ws_tile_impl<BM, BN, CWM, CWN, BWD, PW, NS, GLU, 1, ROPE>(&a, nullptr, bx, by);
}

template <int BM, int BN, int CWM, int CWN, bool BWD, int PW, int NS, bool GLU>
__global__ __launch_bounds__(64 * (4 + PW)) void k_nf4_gemm_ws(GemmArgs a) {
  if constexpr (BWD && BM == 128) {
    extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
    // grid rows past the GEMM's: LoRA gradient workgroups (before any barrier of the tiles).
    // Only the 128-row tiles take them (the plans that leave CUs idle); compiling the branch
    // into the others would only change their register allocation.
    const int gy = (a.M + BM - 1) / BM;
    if ((int)blockIdx.y >= gy) {
      const int id = ((int)blockIdx.y - gy) * (int)gridDim.x + (int)blockIdx.x;
      if (id < a.cols_blocks)
        lora_cols_block<kFusedColsCPL>(a.cp0, a.cp1, a.cols_cb0, a.M, a.cols_ldt, a.r, id,
                                       a.cols_nw, reinterpret_cast<float*>(smem));
      return;
    }
  }

  ws_tile<BM, BN, CWM, CWN, BWD, PW, NS, GLU>(a, (int)blockIdx.x, (int)blockIdx.y);
}

// Several forward GEMMs in one launch (the q/k/v projections of a layer read the same x):
// problem i owns workgroups [start[i], start[i+1]), its tiles in row-major order over its
// gx[i] column tiles.  Unsplit; each tile computes what the problem's own launch of this
// configuration computes.
constexpr int kMaxGemmGroup = 4;
struct GemmGroup {
  GemmArgs p[kMaxGemmGroup];
  int start[kMaxGemmGroup + 1];
  int gx[kMaxGemmGroup];
  int tiles[kMaxGemmGroup];  // the problem's tiles; in the backward its LoRA gradient
                             // workgroups (cols_blocks) follow them
  int n;
};

template <int BM, int BN, int CWM, int CWN, bool BWD, int PW, int NS, bool ROPE = false>
__global__ __launch_bounds__(64 * (4 + PW)) void k_nf4_gemm_ws_group(GemmGroup g) {
  const int bid = (int)blockIdx.x;
  int i = 0;
  while (i + 1 < g.n && bid >= g.start[i + 1]) i++;
  const int local = bid - g.start[i];
  if constexpr (BWD) {
    if (local >= g.tiles[i]) {  // before any barrier of the tiles, as in k_nf4_gemm_ws
      extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
      const GemmArgs& a = g.p[i];
      const int id = local - g.tiles[i];
      if (id < a.cols_blocks)
        lora_cols_block<kFusedColsCPL>(a.cp0, a.cp1, a.cols_cb0, a.M, a.cols_ldt, a.r, id,
                                       a.cols_nw, reinterpret_cast<float*>(smem));
      return;
    }
  }
  ws_tile<BM, BN, CWM, CWN, BWD, PW, NS, false, ROPE>(g.p[i], local % g.gx[i],
                                                     local / g.gx[i]);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, bool BWD>
static int launch_cfg(const GemmArgs& a0, int splits, hipStream_t stream) {
  using T = Tile<BM, BN, WAVES_M, WAVES_N, BWD>;
  // the all-wave kernel has neither the SwiGLU epilogue nor the gradient rows
  if (a0.glu) return MXS_ERR_SIZE;
  if (a0.cols_blocks > 0) return MXS_ERR_ARG;
  GemmArgs a = a0;
  const int n_steps = a.Kr / kBK;
  if (splits < 1) splits = 1;
  if (splits > n_steps) splits = n_steps > 0 ? n_steps : 1;
  a.steps_per_split = (n_steps + splits - 1) / splits;
  splits = n_steps > 0 ? (n_steps + a.steps_per_split - 1) / a.steps_per_split : 1;
  const dim3 grid((a.Nc + BN - 1) / BN, (a.M + BM - 1) / BM, splits);
  if (splits > 1 && !a.ws) return MXS_ERR_ARG;
  const size_t lds = (size_t)2 * (T::LDS_A + T::LDS_B) * sizeof(_Float16);
  static bool lds_set = false;  // idempotent attribute; a benign race between threads
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&k_nf4_gemm<BM, BN, WAVES_M, WAVES_N, BWD>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set = true;
  }
  hipLaunchKernelGGL((k_nf4_gemm<BM, BN, WAVES_M, WAVES_N, BWD>), grid, dim3(T::NT), lds, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  return splits > 1 ? launch_reduce(a, splits, stream) : MXS_OK;
}

template <int BM, int BN, int CWM, int CWN, bool BWD, int PW = 4, int NS = 4>
static int launch_ws(const GemmArgs& a0, int splits, hipStream_t stream) {
  // the producers' 32-bit offsets (W values and one A tile's bytes below 2^32) and the
  // backward loads' column clamp (at least one load item of output columns); otherwise the
  // all-wave kernel takes the call
  if ((int64_t)a0.Nc * a0.Kr >= (int64_t(1) << 32) || (int64_t)BM * a0.lda * 2 >= (int64_t(1) << 32) ||
      (BWD && a0.Nc < (PW == 8 ? 16 : 32))) {
    return launch_cfg<64, 128, 1, 4, BWD>(a0, splits, stream);
  }
  GemmArgs a = a0;
  const int n_steps = a.Kr / kBK;
  if (splits < 1) splits = 1;
  if (splits > n_steps) splits = n_steps > 0 ? n_steps : 1;
  a.steps_per_split = (n_steps + splits - 1) / splits;
  splits = n_steps > 0 ? (n_steps + a.steps_per_split - 1) / a.steps_per_split : 1;
  const int gx = (a.Nc + BN - 1) / BN;
  int gy = (a.M + BM - 1) / BM;
  if (a.cols_blocks > 0) {  // gradient workgroups in extra rows (unsplit backward only)
    if (!BWD || BM != 128 || splits > 1) return MXS_ERR_ARG;
    gy += (a.cols_blocks + gx - 1) / gx;
  }
  const dim3 grid(gx, gy, splits);
  if (splits > 1 && !a.ws) return MXS_ERR_ARG;
  const size_t lds = (size_t)ws_lds_halfs<BM, BN, BWD>() * sizeof(_Float16);
  // the SwiGLU output has kernels of its own, so the others keep their registers
  const void* fn =
      a.glu ? reinterpret_cast<const void*>(&k_nf4_gemm_ws<BM, BN, CWM, CWN, BWD, PW, NS, true>)
            : reinterpret_cast<const void*>(&k_nf4_gemm_ws<BM, BN, CWM, CWN, BWD, PW, NS, false>);
  static bool lds_set[2] = {false, false};  // idempotent attribute; a benign race between threads
  if (!lds_set[a.glu ? 1 : 0]) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set[a.glu ? 1 : 0] = true;
  }
  if (a.glu)
    hipLaunchKernelGGL((k_nf4_gemm_ws<BM, BN, CWM, CWN, BWD, PW, NS, true>), grid,
                       dim3(64 * (4 + PW)), lds, stream, a);
  else
    hipLaunchKernelGGL((k_nf4_gemm_ws<BM, BN, CWM, CWN, BWD, PW, NS, false>), grid,
                       dim3(64 * (4 + PW)), lds, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  return splits > 1 ? launch_reduce(a, splits, stream) : MXS_OK;
}

// Tile configurations, by id: BM x BN and the wave layout.
//   0-4: all waves load, decode and multiply (WAVES_M x WAVES_N waves)
//   6-9: warp-specialized, 4 producer + 4 consumer waves (consumers CWM x CWN)
template <bool BWD>
static int launch_by_id(int cfg, const GemmArgs& a, int splits, hipStream_t s) {
  switch (cfg) {
    case 0: return launch_cfg<256, 128, 2, 2, BWD>(a, splits, s);
    case 1: return launch_cfg<128, 128, 2, 2, BWD>(a, splits, s);
    case 2: return launch_cfg<256, 128, 4, 2, BWD>(a, splits, s);
    case 3: return launch_cfg<128, 128, 2, 4, BWD>(a, splits, s);
    case 4: return launch_cfg<64, 128, 1, 4, BWD>(a, splits, s);
    case 6: return launch_ws<256, 128, 2, 2, BWD>(a, splits, s);
    case 7: return launch_ws<256, 160, 4, 1, BWD>(a, splits, s);
    case 8: return launch_ws<128, 128, 2, 2, BWD>(a, splits, s);
    case 9: return launch_ws<256, 96, 4, 1, BWD>(a, splits, s);
    case 10: return launch_ws<128, 128, 2, 2, BWD, 8>(a, splits, s);
    case 11: return launch_ws<256, 96, 4, 1, BWD, 8, 5>(a, splits, s);
    case 12: return launch_ws<128, 64, 2, 2, BWD, 8>(a, splits, s);
    default: return MXS_ERR_ARG;
  }
}

constexpr int kNumCfg = 13;

// Compute units of the current device (queried once per device).
static int cu_count() {
  static int counts[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    counts[dev] = n > 0 ? n : -1;
  }
  return counts[dev] > 0 ? counts[dev] : 0;
}

// Tile and split choice for one GEMM (M x Nc output, Kr reduction), from measured sweeps on
// MI355X at the Qwen2.5-1.5B projection shapes (M = 1024):
//   wide outputs (Nc >= 4096): warp-specialized 256x160, one tile per CU, no split;
//   narrow outputs with a long reduction (Kr >= 4096): warp-specialized 256x96, split-K 4, with
//   4 producer waves forward (46 against 51 us for down_proj at 1024 tokens) and 8 in the
//   backward (49 against 51 us for gate/up dX); every ws configuration accumulates an output
//   element in the same order, so for one split count the choice changes no result;
//   mid outputs (Nc >= 1024): warp-specialized with 8 producer waves, no split, on 128x64 tiles
//   when those fit the CUs in one round (the 1536-wide q/o shapes up to 1024 tokens: 192 tiles,
//   13.6 against 18.9 us for 128x128 at 1024 tokens, 13.2 against 18.4 at 830), else 128x128
//   (1430 tokens: 288 tiles of 128x64 would take two rounds, 25.6 against 19.2 us);
//   small outputs: 64x128 all-wave tiles, split-K 4 when the reduction is long enough.
// Splits keep at least 6 K-steps each.
static void choose(int M, int Nc, int Kr, bool bwd, int* cfg, int* splits) {
  const int n_steps = Kr / kBK;
  int c, sp;
  if (Nc >= 4096) {
    c = 7; sp = 1;
  } else if (Kr >= 4096) {
    c = bwd ? 11 : 9; sp = 4;
  } else if (Nc >= 1024) {
    const int64_t tiles64 = (int64_t)((M + 127) / 128) * ((Nc + 63) / 64);
    const int cus = cu_count();
    c = (cus > 0 && tiles64 <= cus) ? 12 : 10;
    sp = 1;
  } else {
    c = 4; sp = Kr >= 1024 ? 4 : 1;
  }
  while (sp > 1 && n_steps / sp < 6) sp >>= 1;
  *cfg = c;
  *splits = sp;
}

// Argument checks of one GEMM problem: MXS_OK, an MXS_ERR_* code, or 1 when there is nothing
// to compute (no tokens or no output columns).
static int check_gemm(bool bwd, const GemmArgs& a) {
  if (a.M < 0 || a.Nc < 0 || a.Kr < 0) return MXS_ERR_ARG;
  if (a.M == 0 || a.Nc == 0) return 1;
  if (!a.A || !a.packed || !a.absmax8 || !a.code || !a.absmax2 || !a.offset ||
      (!a.C && a.glu != 2))
    return MXS_ERR_ARG;
  if (a.glu) {  // the SwiGLU buffers: [M, ldc] fp16, 16-byte aligned rows
    if (a.glu != (bwd ? 2 : 1)) return MXS_ERR_ARG;  // forward: silu(gate) * y; backward: adjoint
    if (!a.glu_g || (a.glu == 1 && !a.glu_h) || (a.glu == 2 && !a.glu_u)) return MXS_ERR_ARG;
    if (a.Nc % 8 != 0 || a.ldc % 8 != 0) return MXS_ERR_SIZE;
    if (((uintptr_t)a.glu_g % 16) || ((uintptr_t)a.glu_u % 16) || ((uintptr_t)a.glu_h % 16) ||
        ((uintptr_t)a.C % 16))
      return MXS_ERR_ALIGN;
  }
  if (a.Kr % kBK != 0 || a.Kw % kBK != 0) return MXS_ERR_SIZE;
  if (bwd && a.Nc % 8 != 0) return MXS_ERR_SIZE;
  if (a.lda % 8 != 0 || ((uintptr_t)a.A % 16) != 0 || ((uintptr_t)a.packed % 16) != 0 ||
      ((uintptr_t)a.mask % 4) != 0)
    return MXS_ERR_ALIGN;
  if (a.lora_h && (!a.lora_w || a.r <= 0 || a.r % 16 != 0)) return MXS_ERR_SIZE;
  if (a.lora_h && (((uintptr_t)a.lora_h % 16) != 0 || ((uintptr_t)a.lora_w % 16) != 0))
    return MXS_ERR_ALIGN;
  if (a.lora_hp) {
    if (!a.lora_w || a.r <= 0 || a.r % 16 != 0 || a.hp_slices < 1 || a.hp_slices > 4 ||
        a.ldt < a.M || a.ldt % 8 != 0)
      return MXS_ERR_SIZE;
    if (((uintptr_t)a.lora_hp % 16) != 0 || ((uintptr_t)a.lora_w % 16) != 0 ||
        ((uintptr_t)a.lora_ht % 2) != 0)
      return MXS_ERR_ALIGN;
  }
  return MXS_OK;
}

static int gemm_entry(bool bwd, const GemmArgs& a, int cfg, int splits, hipStream_t stream) {
  const int c = check_gemm(bwd, a);
  if (c != MXS_OK) return c == 1 ? MXS_OK : c;
  if (cfg < 0) choose(a.M, a.Nc, a.Kr, bwd, &cfg, &splits);
  if (cfg >= kNumCfg || cfg == 5) return MXS_ERR_ARG;
  return bwd ? launch_by_id<true>(cfg, a, splits, stream)
             : launch_by_id<false>(cfg, a, splits, stream);
}

// The backward GEMM of a projection [K -> N] at M tokens and its LoRA gradient workgroups fit
// one launch: the planned kernel is an unsplit warp-specialized one that takes the problem
// (none of its fallback conditions holds) and its tiles plus the gradient workgroups fit the
// CUs at once, so that the gradients run beside the tiles instead of after them.
static bool grads_fusable(int M, int N, int K, int r, int* cfg_out, int* nw_out) {
  if (M <= 0 || N <= 0 || K <= 0 || r <= 0 || r > 32 || N % kBK != 0 || K % kBK != 0)
    return false;
  // the gradient workgroups sum exactly as mxs_lora_grads' launch does: same columns per lane
  // and the same waves (which the GEMM's workgroup must have)
  if (cols_cpl(K + N) != kFusedColsCPL) return false;
  const int nw = cols_waves(M, r, kFusedColsCPL, cols_max_waves<kFusedColsCPL>());
  int cfg, sp;
  choose(M, K, N, true, &cfg, &sp);
  if (cfg < 6 || cfg >= kNumCfg || sp != 1) return false;
  static const int kBM[] = {256, 256, 128, 256, 128, 256, 128};  // cfg 6..12
  static const int kBN[] = {128, 160, 128, 96, 128, 96, 64};
  static const int kPW[] = {4, 4, 4, 4, 8, 8, 8};
  const int bm = kBM[cfg - 6], bn = kBN[cfg - 6], pw = kPW[cfg - 6];
  if (bm != 128) return false;  // only those kernels carry the gradient rows
  if (nw > 4 + pw) return false;
  if ((int64_t)K * N >= (int64_t(1) << 32) || (int64_t)bm * N * 2 >= (int64_t(1) << 32) ||
      K < (pw == 8 ? 16 : 32))
    return false;
  constexpr int WC = 16 * kFusedColsCPL;
  const int64_t tiles = (int64_t)((K + bn - 1) / bn) * ((M + bm - 1) / bm);
  const int64_t cols = (K + WC - 1) / WC + (N + WC - 1) / WC;
  // The 128x64 plan (chosen where its tiles alone fill the CUs once) takes the gradient
  // workgroups as a partial second round: they are short, and its tiles are (the q/o backward at
  // 1024 tokens: 192 tiles + 96 gradient workgroups).  Otherwise 128x128 tiles, where tiles and
  // gradient workgroups fit the CUs at once.
  if (cfg == 12 && tiles + cols > 2 * (int64_t)cu_count()) {
    cfg = 10;
    const int64_t tiles128 = (int64_t)((K + 127) / 128) * ((M + 127) / 128);
    if (tiles128 + cols > cu_count()) return false;
  } else if (cfg != 12 && tiles + cols > cu_count()) {
    return false;
  }
  // the gradient workgroups' cross-wave sums fit the kernel's LDS
  const size_t lds = (cfg == 12 ? ws_lds_halfs<128, 64, true>() : ws_lds_halfs<128, 128, true>()) *
                     sizeof(_Float16);
  if ((size_t)nw * r * (WC + 1) * 4 > lds) return false;
  *cfg_out = cfg;
  *nw_out = nw;
  return true;
}

// The planned kernel for a GEMM [M, Nc] over Kr takes the SwiGLU output: a warp-specialized
// configuration that none of its fallback conditions sends to the all-wave kernel.
static bool glu_plan_ok(int M, int Nc, int Kr, bool bwd) {
  if (M <= 0 || Nc <= 0 || Kr <= 0 || Nc % 8 != 0 || Kr % kBK != 0) return false;
  int cfg, sp;
  choose(M, Nc, Kr, bwd, &cfg, &sp);
  if (cfg < 6 || cfg >= kNumCfg) return false;
  static const int kBM[] = {256, 256, 128, 256, 128, 256, 128};  // cfg 6..12
  static const int kPW[] = {4, 4, 4, 4, 8, 8, 8};
  const int bm = kBM[cfg - 6], pw = kPW[cfg - 6];
  return (int64_t)Nc * Kr < (int64_t(1) << 32) && (int64_t)bm * Kr * 2 < (int64_t(1) << 32) &&
         !(bwd && Nc < (pw == 8 ? 16 : 32));
}

// The GEMMs of several problems in one launch of one warp-specialized tile configuration with 8
// producer waves, unsplit (k_nf4_gemm_ws_group): 128x128 tiles by default; in the backward each
// problem's LoRA gradient workgroups follow its tiles.  Every problem must take that kernel (its
// 32-bit offsets, the backward's column clamp).
template <bool BWD, int BN = 128, int CWM = 2, int CWN = 2, bool ROPE = false>
static int launch_ws_group(const GemmArgs* probs, int n, hipStream_t stream) {
  constexpr int BM = 128, PW = 8, NS = 4;
  if (n < 1 || n > kMaxGemmGroup) return MXS_ERR_ARG;
  GemmGroup g{};
  g.n = n;
  int total = 0;
  for (int i = 0; i < n; i++) {
    GemmArgs a = probs[i];
    if ((int64_t)a.Nc * a.Kr >= (int64_t(1) << 32) ||
        (int64_t)BM * a.lda * 2 >= (int64_t(1) << 32) || (BWD && a.Nc < 16) ||
        (!BWD && a.cols_blocks > 0))
      return MXS_ERR_SIZE;
    a.steps_per_split = a.Kr / kBK;
    g.p[i] = a;
    g.gx[i] = (a.Nc + BN - 1) / BN;
    g.tiles[i] = g.gx[i] * ((a.M + BM - 1) / BM);
    g.start[i] = total;
    total += g.tiles[i] + (BWD ? a.cols_blocks : 0);
  }
  g.start[n] = total;
  if (total == 0) return MXS_OK;
  const size_t lds = (size_t)ws_lds_halfs<BM, BN, BWD>() * sizeof(_Float16);
  static bool lds_set = false;  // idempotent attribute; a benign race between threads
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&k_nf4_gemm_ws_group<BM, BN, CWM, CWN, BWD, PW, NS, ROPE>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set = true;
  }
  hipLaunchKernelGGL((k_nf4_gemm_ws_group<BM, BN, CWM, CWN, BWD, PW, NS, ROPE>), dim3(total),
                     dim3(64 * (4 + PW)), lds, stream, g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

// The summed backward (ws_tile_impl with NSUM > 1) in one launch with each problem's LoRA
// gradient workgroups: workgroups [0, tiles) are the shared output's tiles in row-major order
// over gx column tiles, then problem q's gradient workgroups from cstart[q].
struct GemmSum {
  GemmArgs p[kMaxSum];
  SumPlan plan;
  int gx, tiles;
  int cstart[kMaxSum + 1];
};

template <int BM, int BN, int CWM, int CWN, int PW, int NS>
__global__ __launch_bounds__(64 * (4 + PW)) void k_nf4_gemm_ws_sum(GemmSum g) {
  const int bid = (int)blockIdx.x;
  if (bid >= g.tiles) {  // before any barrier of the tiles, as in k_nf4_gemm_ws
    extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
    int q = 0;
    while (q + 1 < g.plan.n && bid >= g.cstart[q + 1]) q++;
    const GemmArgs& a = g.p[q];
    const int id = bid - g.cstart[q];
    if (id < a.cols_blocks)
      lora_cols_block<kFusedColsCPL>(a.cp0, a.cp1, a.cols_cb0, a.M, a.cols_ldt, a.r, id,
                                     a.cols_nw, reinterpret_cast<float*>(smem));
    return;
  }
  ws_tile_impl<BM, BN, CWM, CWN, true, PW, NS, false, kMaxSum>(g.p, &g.plan, bid % g.gx,
                                                               bid / g.gx);
}

// LDS halfs of the summed kernel: the single-problem layout, then problems 1 and 2's staged LoRA
// operands ([BM][16] + [BN][16]) and keep bits (BM rows of MaskStage's row stride)
template <int BM, int BN>
constexpr int ws_sum_lds_halfs() {
  return ws_lds_halfs<BM, BN, true>() +
         (kMaxSum - 1) * ((BM + BN) * 16 + BM * MaskStage<BM, BN, 1>::KST / 2);
}

template <int BN>
static int launch_ws_sum(const GemmArgs* probs, int n, hipStream_t stream) {
  constexpr int BM = 128, PW = 8, NS = 4;
  if (n < 2 || n > kMaxSum) return MXS_ERR_ARG;
  GemmSum g{};
  g.plan.n = n;
  int end = 0;
  for (int q = 0; q < kMaxSum; q++) {
    if (q < n) {
      g.p[q] = probs[q];
      end += probs[q].Kr / kBK;
    }
    g.plan.end[q] = end;
  }
  const GemmArgs& a = g.p[0];
  g.p[0].steps_per_split = end;  // one split over the concatenated reduction
  g.p[0].zf = 0;
  g.gx = (a.Nc + BN - 1) / BN;
  g.tiles = g.gx * ((a.M + BM - 1) / BM);
  g.cstart[0] = g.tiles;
  for (int q = 0; q < n; q++) g.cstart[q + 1] = g.cstart[q] + g.p[q].cols_blocks;
  for (int q = n; q < kMaxSum; q++) g.cstart[q + 1] = g.cstart[q];
  const int total = g.cstart[n];
  if (total == 0) return MXS_OK;
  const size_t lds = (size_t)ws_sum_lds_halfs<BM, BN>() * sizeof(_Float16);
  static bool lds_set = false;  // idempotent attribute; a benign race between threads
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&k_nf4_gemm_ws_sum<BM, BN, 2, 2, PW, NS>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set = true;
  }
  hipLaunchKernelGGL((k_nf4_gemm_ws_sum<BM, BN, 2, 2, PW, NS>), dim3(total), dim3(64 * (4 + PW)),
                     lds, stream, g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

// Two problems of one output shape whose results are added (the gate and up projections' input
// gradients: autograd sums them for the shared input) in ONE launch of the split-K kernel:
// problem 0 owns grid z [0, sp), problem 1 [sp, 2 sp), each splitting its own reduction over
// its z range; every split writes its fp32 partial plane (the plane index is the grid z) and
// one reduce adds all 2 sp planes in order.  So neither projection's output is rounded to fp16
// on its own, and the pair costs one launch and one reduce instead of two of each.
struct GemmPair {
  GemmArgs p[2];
};

template <int BM, int BN, int CWM, int CWN, bool BWD, int PW, int NS>
__global__ __launch_bounds__(64 * (4 + PW)) void k_nf4_gemm_ws_pair(GemmPair g) {
  const int i = (int)blockIdx.z < g.p[1].zf ? 0 : 1;
  ws_tile<BM, BN, CWM, CWN, BWD, PW, NS, false>(g.p[i], (int)blockIdx.x, (int)blockIdx.y);
}

// reduce: false leaves the 2 sp planes for the caller's reduce (k_splitk_reduce_cols).
template <int BM, int BN, int CWM, int CWN, bool BWD, int PW, int NS>
static int launch_ws_pair(const GemmArgs& a0, const GemmArgs& a1, int sp, hipStream_t stream,
                          bool reduce = true) {
  if (sp < 1 || !a0.ws || a0.M != a1.M || a0.Nc != a1.Nc) return MXS_ERR_ARG;
  GemmPair g{};
  g.p[0] = a0;
  g.p[1] = a1;
  for (int i = 0; i < 2; i++) {
    GemmArgs& a = g.p[i];
    // the conditions under which launch_ws would keep this kernel; no fallback here
    if ((int64_t)a.Nc * a.Kr >= (int64_t(1) << 32) || (int64_t)BM * a.lda * 2 >= (int64_t(1) << 32) ||
        (BWD && a.Nc < (PW == 8 ? 16 : 32)) || a.glu || a.cols_blocks > 0)
      return MXS_ERR_SIZE;
    const int n_steps = a.Kr / kBK;
    a.steps_per_split = (n_steps + sp - 1) / sp;
    // every split of the z range has K-steps: its plane is written
    if (n_steps < sp || (n_steps + a.steps_per_split - 1) / a.steps_per_split != sp)
      return MXS_ERR_SIZE;
    a.zf = i * sp;
    a.ws = a0.ws;
  }
  const dim3 grid((a0.Nc + BN - 1) / BN, (a0.M + BM - 1) / BM, 2 * sp);
  const size_t lds = (size_t)ws_lds_halfs<BM, BN, BWD>() * sizeof(_Float16);
  static bool lds_set = false;  // idempotent attribute; a benign race between threads
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&k_nf4_gemm_ws_pair<BM, BN, CWM, CWN, BWD, PW, NS>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set = true;
  }
  hipLaunchKernelGGL((k_nf4_gemm_ws_pair<BM, BN, CWM, CWN, BWD, PW, NS>), grid,
                     dim3(64 * (4 + PW)), lds, stream, g);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  return reduce ? launch_reduce(g.p[0], 2 * sp, stream) : MXS_OK;
}

// Two forward projections of one shape over the same input (gate and up, solution/mlp.py:42-43),
// each unsplit, in ONE launch: grid z selects the problem.  Their 2 x 224 tiles of 256x160 at
// 1024 tokens take 1.75 rounds of the 256 CUs instead of two launches of one round each that
// leave 32 CUs idle.  Each tile runs exactly as in its own launch (the same bits).
template <int BM, int BN, int CWM, int CWN, int PW, int NS>
static int launch_ws_fwd_pair(const GemmArgs& a0, const GemmArgs& a1, hipStream_t stream) {
  if (a0.M != a1.M || a0.Nc != a1.Nc || a0.Kr != a1.Kr) return MXS_ERR_ARG;
  GemmPair g{};
  g.p[0] = a0;
  g.p[1] = a1;
  for (int i = 0; i < 2; i++) {
    GemmArgs& a = g.p[i];
    if ((int64_t)a.Nc * a.Kr >= (int64_t(1) << 32) || (int64_t)BM * a.lda * 2 >= (int64_t(1) << 32) ||
        a.glu || a.cols_blocks > 0)
      return MXS_ERR_SIZE;
    a.steps_per_split = a.Kr / kBK;
    a.zf = i;
    a.unsplit = 1;
  }
  const dim3 grid((a0.Nc + BN - 1) / BN, (a0.M + BM - 1) / BM, 2);
  const size_t lds = (size_t)ws_lds_halfs<BM, BN, false>() * sizeof(_Float16);
  static bool lds_set = false;  // idempotent attribute; a benign race between threads
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&k_nf4_gemm_ws_pair<BM, BN, CWM, CWN, false, PW, NS>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set = true;
  }
  hipLaunchKernelGGL((k_nf4_gemm_ws_pair<BM, BN, CWM, CWN, false, PW, NS>), grid,
                     dim3(64 * (4 + PW)), lds, stream, g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

// The forward pair with two tile widths in ONE launch, so that the CUs end together: 2 x 224
// tiles of 256x160 at 1024 tokens take 1.75 rounds of 256 CUs, i.e. two tile times with 64 CUs
// idle in the second.  Each projection's columns split at ncut (a multiple of 160): [0, ncut)
// in 256x160 tiles (w[i]), [ncut, N) in 256x128 tiles (n[i]: the same problem viewed from
// column ncut, its weight rows, scales, bias and lora_B rows offset, no dHs^T writes).  The
// wide tiles come first in the grid, one per CU; the narrow ones (0.86 of a wide tile's time,
// measured) fill the rest, so that a CU runs one of each or two narrow ones.  Every output
// element is computed as either tile computes it (the same K-steps, MFMAs and epilogue), so the
// results are the bits of the one-width launch.
struct GemmMixed {
  GemmArgs w[2], n[2];
  int gxw, gxn, gy, nwide;
};

template <int NS>
__global__ __launch_bounds__(64 * 8) void k_nf4_gemm_ws_pair_mixed(GemmMixed g) {
  const int bid = (int)blockIdx.x;
  if (bid < g.nwide) {
    const int per = g.gxw * g.gy, i = bid / per, l = bid % per;
    ws_tile<256, 160, 4, 1, false, 4, NS, false>(g.w[i], l % g.gxw, l / g.gxw);
  } else {
    const int b = bid - g.nwide, per = g.gxn * g.gy, i = b / per, l = b % per;
    ws_tile<256, 128, 2, 2, false, 4, NS, false>(g.n[i], l % g.gxn, l / g.gxn);
  }
}

// Time of a narrow (256x128) tile against a wide (256x160) one, measured at one round
// (1536-long reduction: 25.3 against 29.2 us).
constexpr double kNarrowTile = 0.86;

// Makespan, in wide-tile times, of W wide then Nn narrow tiles taken in that order by `cus`
// CUs, each tile by the CU that frees first.
static double list_makespan(int W, int Nn, int cus) {
  std::priority_queue<double, std::vector<double>, std::greater<double>> free_at(
      std::greater<double>(), std::vector<double>(cus, 0.0));
  double end = 0.0;
  for (int t = 0; t < W + Nn; t++) {
    const double f = free_at.top() + (t < W ? 1.0 : kNarrowTile);
    free_at.pop();
    free_at.push(f);
    end = f > end ? f : end;
  }
  return end;
}

// The column split of the mixed forward pair for two problems [K -> N] at M tokens (0: the
// one-width launch is as fast).  ncut: a multiple of 160 that leaves a multiple of 128, and a
// whole number of second-level scale groups (256 blocks of 64) before it.
static int fwd_pair_mixed_cut(int M, int N, int K) {
  const int cus = cu_count();
  if (cus <= 0 || N % 32 || (K % 64)) return 0;
  static std::mutex mu;
  static int key[3] = {-1, -1, -1}, cached = 0, cached_cus = 0;
  std::lock_guard<std::mutex> lock(mu);
  if (key[0] == M && key[1] == N && key[2] == K && cached_cus == cus) return cached;
  const int gy = (M + 255) / 256;
  const double plain = list_makespan(2 * gy * ((N + 159) / 160), 0, cus);
  double best = plain * 0.97;  // worth a second kernel only where it gains
  int cut = 0;
  for (int a = 1; 160 * a < N; a++) {
    const int rest = N - 160 * a;
    if (rest % 128 || ((int64_t)160 * a * K / 64) % 256) continue;
    const double t = list_makespan(2 * gy * a, 2 * gy * (rest / 128), cus);
    if (t < best) {
      best = t;
      cut = 160 * a;
    }
  }
  key[0] = M, key[1] = N, key[2] = K, cached = cut, cached_cus = cus;
  return cut;
}

static int launch_ws_fwd_pair_mixed(const GemmArgs& a0, const GemmArgs& a1, int ncut,
                                    hipStream_t stream) {
  constexpr int NS = 4;
  if (a0.M != a1.M || a0.Nc != a1.Nc || a0.Kr != a1.Kr || ncut <= 0 || ncut >= a0.Nc ||
      ncut % 160 || (a0.Nc - ncut) % 128)
    return MXS_ERR_ARG;
  GemmMixed g{};
  const GemmArgs* src[2] = {&a0, &a1};
  for (int i = 0; i < 2; i++) {
    GemmArgs a = *src[i];
    if ((int64_t)a.Nc * a.Kr >= (int64_t(1) << 32) || (int64_t)256 * a.lda * 2 >= (int64_t(1) << 32) ||
        a.glu || a.cols_blocks > 0 || a.rope_cos)
      return MXS_ERR_SIZE;
    const int64_t blk0 = (int64_t)ncut * a.Kw / 64;  // first scale block of the narrow view
    if (blk0 % 256) return MXS_ERR_SIZE;
    a.steps_per_split = a.Kr / kBK;
    a.zf = 0;
    a.unsplit = 0;
    GemmArgs w = a;
    w.Nc = ncut;  // the wide tiles' columns: [0, ncut) of the same buffers
    GemmArgs n = a;
    n.Nc = a.Nc - ncut;
    n.packed = a.packed + (int64_t)ncut * (a.Kw / 2);
    n.absmax8 = a.absmax8 + blk0;
    n.absmax2 = a.absmax2 + blk0 / 256;
    if (a.bias) n.bias = a.bias + ncut;
    if (a.lora_w) n.lora_w = a.lora_w + (int64_t)ncut * a.r;
    n.lora_ht = nullptr;  // the wide tiles of column 0 write dHs^T
    n.C = a.C + ncut;
    g.w[i] = w;
    g.n[i] = n;
  }
  g.gxw = ncut / 160;
  g.gxn = (a0.Nc - ncut) / 128;
  g.gy = (a0.M + 255) / 256;
  g.nwide = 2 * g.gxw * g.gy;
  const int total = g.nwide + 2 * g.gxn * g.gy;
  const size_t lds = (size_t)(ws_lds_halfs<256, 160, false>() > ws_lds_halfs<256, 128, false>()
                                  ? ws_lds_halfs<256, 160, false>()
                                  : ws_lds_halfs<256, 128, false>()) *
                     sizeof(_Float16);
  static bool lds_set = false;  // idempotent attribute; a benign race between threads
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_nf4_gemm_ws_pair_mixed<NS>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set = true;
  }
  hipLaunchKernelGGL((k_nf4_gemm_ws_pair_mixed<NS>), dim3(total), dim3(64 * 8), lds, stream, g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

// The forward pair takes two problems [K -> N] that each plan the unsplit 256x160 kernel.
static bool fwd_pair_plan_ok(int M, int N0, int N1, int K) {
  if (M <= 0 || N0 != N1 || K <= 0 || K % kBK) return false;
  int c, sp;
  choose(M, N0, K, false, &c, &sp);
  return c == 7 && sp == 1 && (int64_t)N0 * K < (int64_t(1) << 32) &&
         (int64_t)256 * K * 2 < (int64_t(1) << 32);
}

// The pair's plan: both problems must plan the 256x96 split backward kernel (cfg 11) on their
// own; the pair then splits each reduction kPairSplits ways.
constexpr int kPairSplits = 2;

static bool pair_plan_ok(int M, int N0, int N1, int K) {
  if (M <= 0 || K <= 0 || N0 <= 0 || N1 <= 0 || N0 % kBK || N1 % kBK || K % kBK) return false;
  for (int n : {N0, N1}) {
    int cfg, sp;
    choose(M, K, n, true, &cfg, &sp);
    if (cfg != 11 || sp == 1) return false;
    if ((int64_t)K * n >= (int64_t(1) << 32) || (int64_t)256 * n * 2 >= (int64_t(1) << 32))
      return false;
    const int steps = n / kBK, sps = (steps + kPairSplits - 1) / kPairSplits;
    if (steps < kPairSplits || (steps + sps - 1) / sps != kPairSplits) return false;
  }
  return true;
}

// The arguments of a dX GEMM whose launch also computes the LoRA gradients (its workgroups past
// the tiles): the gradients' checks (mxs_lora_grads); the GEMM's follow in check_gemm.
static int dx_grads_args(const void* dy, int M, int N, int K, const void* packed,
                         const void* absmax8, const float* code, const float* absmax2,
                         const float* offset, const void* lora_dh, const void* lora_at, int r,
                         const void* mask, float mask_scale, const void* dht, const void* ht,
                         int ldt, const void* x, float* da, float* db, void* dx, int nw,
                         GemmArgs& a) {
  if (r % 16 || K % 8 || N % 8 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if (((uintptr_t)x % 16) || ((uintptr_t)dht % 16) || ((uintptr_t)dy % 16) ||
      ((uintptr_t)ht % 16) || (mask && ((uintptr_t)mask % 4)))
    return MXS_ERR_ALIGN;
  a = GemmArgs{};
  a.A = static_cast<const _Float16*>(dy);
  a.lda = N;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = K;
  a.Kr = N;
  a.Kw = K;
  a.lora_h = static_cast<const _Float16*>(lora_dh);
  a.lora_w = static_cast<const _Float16*>(lora_at);
  a.r = r;
  a.mask = static_cast<const uint8_t*>(mask);
  a.mask_scale = mask_scale;
  a.C = static_cast<_Float16*>(dx);
  a.ldc = K;
  ColsProblem& pa = a.cp0;  // dA [r, K] = dHs^T . drop(X)
  pa.PT = static_cast<const _Float16*>(dht);
  pa.Q = static_cast<const _Float16*>(x);
  pa.mask = static_cast<const uint8_t*>(mask);
  pa.mscale = mask_scale;
  pa.round2 = mask && !round_once_exact(mask_scale);
  pa.Nq = K;
  pa.out = da;
  pa.out_rn = 1;
  ColsProblem& pb = a.cp1;  // dB [N, r] = dY^T . Hs
  pb.PT = static_cast<const _Float16*>(ht);
  pb.Q = static_cast<const _Float16*>(dy);
  pb.mscale = 1.0f;
  pb.round2 = 0;
  pb.Nq = N;
  pb.out = db;
  pb.out_rn = 0;
  constexpr int WC = 16 * kFusedColsCPL;
  a.cols_cb0 = (K + WC - 1) / WC;
  a.cols_blocks = a.cols_cb0 + (N + WC - 1) / WC;
  a.cols_ldt = ldt;
  a.cols_nw = nw;
  return MXS_OK;
}

// Problems the summed dX launch takes (k_nf4_gemm_ws_sum: 2..3 problems over one input of
// K >= 1024 columns, rank 16, 128-row tiles): the 32-bit offsets of the tile kernel and, with
// the LoRA gradients (grads), each problem's gradient workgroups as its fused launch would run
// them (same columns per lane and waves: up to 1152 tokens, where the sum over tokens needs at
// most the kernel's 12 waves).  *bn: 64 where the output's 128x64 tiles fit the CUs once and,
// with every gradient workgroup, twice; else 128.
static bool dx_grads_sum_ok(int n, int M, const int* N, int K, int r, bool grads, int* bn,
                            int* nw) {
  if (n < 2 || n > kMaxSum || M <= 0 || K < 1024 || K % kBK != 0 || r != 16) return false;
  *nw = grads ? cols_waves(M, r, kFusedColsCPL, cols_max_waves<kFusedColsCPL>()) : 0;
  if (*nw > 12) return false;  // the 8-producer kernel's 12 waves
  constexpr int WC = 16 * kFusedColsCPL;
  int64_t cols = 0;
  for (int i = 0; i < n; i++) {
    if (N[i] <= 0 || N[i] % kBK != 0 || (int64_t)K * N[i] >= (int64_t(1) << 32) ||
        (int64_t)128 * N[i] * 2 >= (int64_t(1) << 32))
      return false;
    // only reductions each problem's own launch runs unsplit (q, k, v): a long one (gate and up,
    // N = 8960) re-reads dY from L2 for every column tile (154 against 101 us for the split-K
    // pair at 1024 tokens)
    int cfg, sp;
    choose(M, K, N[i], true, &cfg, &sp);
    if (sp != 1) return false;
    if (grads && cols_cpl(K + N[i]) != kFusedColsCPL) return false;
    if (grads) cols += (K + WC - 1) / WC + (N[i] + WC - 1) / WC;
  }
  if ((size_t)*nw * r * (WC + 1) * 4 > (size_t)ws_sum_lds_halfs<128, 64>() * sizeof(_Float16))
    return false;
  const int64_t tiles64 = (int64_t)((M + 127) / 128) * ((K + 63) / 64);
  const int cus = cu_count();
  *bn = (cus > 0 && tiles64 <= cus && tiles64 + cols <= 2 * (int64_t)cus) ? 64 : 128;
  return true;
}

// Problems the grouped dX + LoRA-gradient launch takes: each fusable on the 128x128 tiles.
static bool dx_grads_group_ok(int n, int M, const int* N, int K, int r, int* nw) {
  if (n < 1 || n > kMaxGemmGroup) return false;
  for (int i = 0; i < n; i++) {
    int cfg;
    if (!grads_fusable(M, N[i], K, r, &cfg, &nw[i]) || (cfg != 10 && cfg != 12)) return false;
  }
  return true;
}

}  // namespace mxs

using namespace mxs;

// Split-K workspace: one fp32 partial plane per split.
int64_t mxs_nf4_gemm_workspace_bytes(int M, int Nc, int Kr, int cfg, int splits) {
  if (cfg < 0) choose(M, Nc, Kr, false, &cfg, &splits);  // both directions split alike
  if (splits <= 1) return 0;
  return (int64_t)splits * M * Nc * (int64_t)sizeof(float);
}

static void set_workspace(GemmArgs& a, void* workspace) {
  a.ws = static_cast<float*>(workspace);
}

// ---- Split-K partials for callers that cannot allocate (mxs_nf4_linear_fwd_noalloc) --------
// A file-scope device array: every GPU the library runs on holds its own copy, at its own
// address, from module load to the end of the process.  Its host-side name is only a handle:
// kernels get the device address that hipGetSymbolAddress returns for the current device,
// looked up once per device and kept.  All calls on one GPU share the array, so calls that
// overlap in time on one GPU (two streams, two threads) race on it.  Nothing needs clearing:
// each split writes its whole partial plane before the reduce reads it.
static __device__ __align__(256) unsigned char scratch[MXS_NF4_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (first call per device looks it up).
static int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return MXS_ERR_ARG;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (!p) return (int)hipErrorInvalidSymbol;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return MXS_OK;
}

// The two problems of the summed dX pair (mxs_nf4_linear_bwd_dx_hp_pair's checks): MXS_OK,
// 1 when there is nothing to compute, or an error code.
static int dx_pair_args(const void* const dy[2], int M, const int N[2], int K,
                        const void* const packed[2], const void* const absmax8[2],
                        const float* const code[2], const float* const absmax2[2],
                        const float* const offset[2], const float* const lora_dhp[2],
                        int hp_slices, int ldt, const void* const lora_at[2], int r,
                        const void* const mask[2], float mask_scale, void* const lora_dht[2],
                        void* dx, void* workspace, GemmArgs p[2]) {
  if (M < 0 || !dy || !N || !packed || !absmax8 || !code || !absmax2 || !offset || !lora_dhp ||
      !lora_at)
    return MXS_ERR_ARG;
  if (M == 0) return 1;
  if (!pair_plan_ok(M, N[0], N[1], K)) return MXS_ERR_SIZE;
  if (!workspace) return MXS_ERR_ARG;
  for (int i = 0; i < 2; i++) {
    GemmArgs a{};
    a.A = static_cast<const _Float16*>(dy[i]);
    a.lda = N[i];
    a.packed = static_cast<const uint8_t*>(packed[i]);
    a.absmax8 = static_cast<const uint8_t*>(absmax8[i]);
    a.code = code[i];
    a.absmax2 = absmax2[i];
    a.offset = offset[i];
    a.M = M;
    a.Nc = K;
    a.Kr = N[i];
    a.Kw = K;
    a.lora_hp = lora_dhp[i];
    a.hp_slices = hp_slices;
    a.ldt = ldt;
    a.lora_ht = lora_dht ? static_cast<_Float16*>(lora_dht[i]) : nullptr;
    a.lora_w = static_cast<const _Float16*>(lora_at[i]);
    a.r = r;
    a.mask = mask ? static_cast<const uint8_t*>(mask[i]) : nullptr;
    a.mask_scale = mask_scale;
    a.C = static_cast<_Float16*>(dx);
    a.ldc = K;
    set_workspace(a, workspace);
    if (!a.lora_hp) return MXS_ERR_ARG;
    const int c = check_gemm(true, a);
    if (c != MXS_OK) return c;
    p[i] = a;
  }
  return MXS_OK;
}

template <int CPL>
static int reduce_cols_launch(const GemmArgs& a, int splits, ColsGroup g, int M, int ldt, int r,
                              hipStream_t stream) {
  constexpr int WC = 16 * CPL;
  const int cols = cols_group_layout(g, CPL);
  const int nw = cols_waves(M, r, CPL, cols_max_waves<CPL>());
  const size_t lds = (size_t)nw * r * (WC + 1) * sizeof(float);
  if (lds > (size_t)kColsLds) return MXS_ERR_SIZE;
  // reduce workgroups: the CUs the gradient workgroups' last partial round leaves idle, at
  // least a quarter of the CUs
  const int cus = cu_count() > 0 ? cu_count() : 256;
  const int tail = cols % cus;
  int nred = tail == 0 ? cus : cus - tail;
  if (nred < cus / 4) nred = cus / 4;
  hipLaunchKernelGGL(k_splitk_reduce_cols<CPL>, dim3(cols + nred), dim3(64 * nw), lds, stream,
                     a.ws, splits, a.M, a.Nc, a.C, (int64_t)a.ldc, g, M, ldt, r, nw, nred);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

extern "C" {

int mxs_nf4_linear_fwd(const void* x, int M, int K, int N, const void* packed,
                       const void* absmax8, const float* code, const float* absmax2,
                       const float* offset, const void* bias, const void* lora_h,
                       const void* lora_b, int r, void* y, void* workspace, int cfg, int splits,
                       hipStream_t stream) {
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(x);
  a.lda = K;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = N;
  a.Kr = K;
  a.Kw = K;
  a.bias = static_cast<const _Float16*>(bias);
  a.lora_h = static_cast<const _Float16*>(lora_h);
  a.lora_w = static_cast<const _Float16*>(lora_b);
  a.r = r;
  a.C = static_cast<_Float16*>(y);
  a.ldc = N;
  set_workspace(a, workspace);
  return gemm_entry(false, a, cfg, splits, stream);
}

int mxs_nf4_linear_bwd_dx(const void* dy, int M, int N, int K, const void* packed,
                          const void* absmax8, const float* code, const float* absmax2,
                          const float* offset, const void* lora_dh, const void* lora_at, int r,
                          const void* mask, float mask_scale, void* dx, void* workspace, int cfg,
                          int splits, hipStream_t stream) {
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(dy);
  a.lda = N;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = K;
  a.Kr = N;
  a.Kw = K;
  a.lora_h = static_cast<const _Float16*>(lora_dh);
  a.lora_w = static_cast<const _Float16*>(lora_at);
  a.r = r;
  a.mask = static_cast<const uint8_t*>(mask);
  a.mask_scale = mask_scale;
  a.C = static_cast<_Float16*>(dx);
  a.ldc = K;
  set_workspace(a, workspace);
  return gemm_entry(true, a, cfg, splits, stream);
}

int mxs_nf4_linear_bwd_grads_fused(int M, int N, int K, int r) {
  int cfg, nw;
  return grads_fusable(M, N, K, r, &cfg, &nw) ? 1 : 0;
}

int mxs_nf4_linear_bwd_dx_grads(const void* dy, int M, int N, int K, const void* packed,
                                const void* absmax8, const float* code, const float* absmax2,
                                const float* offset, const void* lora_dh, const void* lora_at,
                                int r, const void* mask, float mask_scale, const void* dht,
                                const void* ht, int ldt, const void* x, float* da, float* db,
                                void* dx, void* workspace, hipStream_t stream) {
  if (M < 0) return MXS_ERR_ARG;
  if (M == 0)  // no tokens: dX is empty, dA and dB are empty reductions (zeros)
    return mxs_lora_grads(nullptr, nullptr, ldt, nullptr, nullptr, 0, K, N, r, nullptr,
                          mask_scale, da, db, workspace, stream);
  if (!lora_dh || !lora_at || !dht || !ht || !x || !da || !db || !dx) return MXS_ERR_ARG;
  int cfg, nw;
  if (!grads_fusable(M, N, K, r, &cfg, &nw)) {  // two launches, same results
    const int e = mxs_nf4_linear_bwd_dx(dy, M, N, K, packed, absmax8, code, absmax2, offset,
                                        lora_dh, lora_at, r, mask, mask_scale, dx, workspace,
                                        -1, 1, stream);
    if (e != MXS_OK) return e;
    return mxs_lora_grads(dht, ht, ldt, x, dy, M, K, N, r, mask, mask_scale, da, db, workspace,
                          stream);
  }
  GemmArgs a{};
  const int e = dx_grads_args(dy, M, N, K, packed, absmax8, code, absmax2, offset, lora_dh, lora_at,
                              r, mask, mask_scale, dht, ht, ldt, x, da, db, dx, nw, a);
  if (e != MXS_OK) return e;
  set_workspace(a, workspace);
  return gemm_entry(true, a, cfg, 1, stream);
}


int mxs_nf4_linear_bwd_dx_grads_group_ok(int n, int M, const int N[], int K, int r) {
  int nw[kMaxGemmGroup];
  return N && dx_grads_group_ok(n, M, N, K, r, nw) ? 1 : 0;
}

int mxs_nf4_linear_bwd_dx_grads_group(int n, const void* const dy[], int M, const int N[], int K,
                                      const void* const packed[], const void* const absmax8[],
                                      const float* const code[], const float* const absmax2[],
                                      const float* const offset[], const void* const lora_dh[],
                                      const void* const lora_at[], int r,
                                      const void* const mask[], float mask_scale,
                                      const void* const dht[], const void* const ht[], int ldt,
                                      const void* const x[], float* const da[],
                                      float* const db[], void* const dx[], hipStream_t stream) {
  if (n < 1 || n > kMaxGemmGroup || !dy || !N || !packed || !absmax8 || !code || !absmax2 ||
      !offset || !lora_dh || !lora_at || !dht || !ht || !x || !da || !db || !dx)
    return MXS_ERR_ARG;
  int nw[kMaxGemmGroup];
  if (!dx_grads_group_ok(n, M, N, K, r, nw)) return MXS_ERR_SIZE;
  GemmArgs probs[kMaxGemmGroup];
  for (int i = 0; i < n; i++) {
    if (!lora_dh[i] || !lora_at[i] || !dht[i] || !ht[i] || !x[i] || !da[i] || !db[i] || !dx[i])
      return MXS_ERR_ARG;
    const void* mk = mask ? mask[i] : nullptr;
    int e = dx_grads_args(dy[i], M, N[i], K, packed[i], absmax8[i], code[i], absmax2[i],
                          offset[i], lora_dh[i], lora_at[i], r, mk, mask_scale, dht[i], ht[i], ldt,
                          x[i], da[i], db[i], dx[i], nw[i], probs[i]);
    if (e != MXS_OK) return e;
    e = check_gemm(true, probs[i]);
    if (e != MXS_OK) return e == 1 ? MXS_ERR_SIZE : e;  // grads_fusable admits no empty problem
  }
  // 128x64 tiles where every problem plans them and all the tiles and gradient workgroups fill
  // at most two rounds of the CUs (q, k and v at 1024 tokens), as for one problem; else 128x128
  bool t64 = true;
  int64_t wgs = 0;
  for (int i = 0; i < n; i++) {
    int cfg, sp;
    choose(M, probs[i].Nc, probs[i].Kr, true, &cfg, &sp);
    t64 = t64 && cfg == 12;
    wgs += (int64_t)((M + 127) / 128) * ((probs[i].Nc + 63) / 64) + probs[i].cols_blocks;
  }
  if (t64 && wgs <= 2 * (int64_t)cu_count()) return launch_ws_group<true, 64>(probs, n, stream);
  return launch_ws_group<true>(probs, n, stream);
}

int mxs_nf4_linear_bwd_dx_grads_sum_ok(int n, int M, const int N[], int K, int r, int grads) {
  int bn, nw;
  return N && dx_grads_sum_ok(n, M, N, K, r, grads != 0, &bn, &nw) ? 1 : 0;
}

int mxs_nf4_linear_bwd_dx_grads_sum(int n, const void* const dy[], int M, const int N[], int K,
                                    const void* const packed[], const void* const absmax8[],
                                    const float* const code[], const float* const absmax2[],
                                    const float* const offset[], const void* const lora_dh[],
                                    const void* const lora_at[], int r, const void* const mask[],
                                    float mask_scale, const void* const dht[],
                                    const void* const ht[], int ldt, const void* x,
                                    float* const da[], float* const db[], void* dx,
                                    hipStream_t stream) {
  if (n < 2 || n > kMaxSum || !dy || !N || !packed || !absmax8 || !code || !absmax2 || !offset ||
      !lora_dh || !lora_at || !dx)
    return MXS_ERR_ARG;
  const bool grads = da != nullptr;  // dA and dB, or neither
  if (grads != (db != nullptr) || (grads && (!dht || !ht || !x))) return MXS_ERR_ARG;
  int bn, nw;
  if (!dx_grads_sum_ok(n, M, N, K, r, grads, &bn, &nw)) return MXS_ERR_SIZE;
  GemmArgs probs[kMaxSum];
  const bool masked = mask && mask[0];
  for (int i = 0; i < n; i++) {
    if (!lora_dh[i] || !lora_at[i] || (grads && (!dht[i] || !ht[i] || !da[i] || !db[i])))
      return MXS_ERR_ARG;
    const void* mk = mask ? mask[i] : nullptr;
    if ((mk != nullptr) != masked) return MXS_ERR_ARG;  // every problem masked, or none
    // without the gradients the LoRA-gradient operands are stand-ins (the 16-byte aligned dY)
    // that no workgroup reads: cols_blocks is zeroed below
    int e = dx_grads_args(dy[i], M, N[i], K, packed[i], absmax8[i], code[i], absmax2[i],
                          offset[i], lora_dh[i], lora_at[i], r, mk, mask_scale,
                          grads ? dht[i] : dy[i], grads ? ht[i] : dy[i], ldt, grads ? x : dy[i],
                          grads ? da[i] : nullptr, grads ? db[i] : nullptr, dx, nw, probs[i]);
    if (e != MXS_OK) return e;
    if (!grads) probs[i].cols_blocks = 0;
    e = check_gemm(true, probs[i]);
    if (e != MXS_OK) return e == 1 ? MXS_ERR_SIZE : e;
  }
  return bn == 64 ? launch_ws_sum<64>(probs, n, stream) : launch_ws_sum<128>(probs, n, stream);
}

int mxs_nf4_linear_fwd_hp(const void* x, int M, int K, int N, const void* packed,
                          const void* absmax8, const float* code, const float* absmax2,
                          const float* offset, const void* bias, const float* lora_hp,
                          int hp_slices, int ldt, const void* lora_b, int r, void* lora_ht,
                          void* y, void* workspace, int cfg, int splits, hipStream_t stream) {
  if (M < 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;  // no tokens: nothing to compute (empty partials may be NULL)
  if (!lora_hp) return MXS_ERR_ARG;
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(x);
  a.lda = K;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = N;
  a.Kr = K;
  a.Kw = K;
  a.bias = static_cast<const _Float16*>(bias);
  a.lora_hp = lora_hp;
  a.hp_slices = hp_slices;
  a.ldt = ldt;
  a.lora_ht = static_cast<_Float16*>(lora_ht);
  a.lora_w = static_cast<const _Float16*>(lora_b);
  a.r = r;
  a.C = static_cast<_Float16*>(y);
  a.ldc = N;
  set_workspace(a, workspace);
  return gemm_entry(false, a, cfg, splits, stream);
}

int mxs_nf4_linear_bwd_dx_hp(const void* dy, int M, int N, int K, const void* packed,
                             const void* absmax8, const float* code, const float* absmax2,
                             const float* offset, const float* lora_dhp, int hp_slices, int ldt,
                             const void* lora_at, int r, const void* mask, float mask_scale,
                             void* lora_dht, void* dx, void* workspace, int cfg, int splits,
                             hipStream_t stream) {
  if (M < 0) return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;  // no tokens: nothing to compute (empty partials may be NULL)
  if (!lora_dhp) return MXS_ERR_ARG;
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(dy);
  a.lda = N;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = K;
  a.Kr = N;
  a.Kw = K;
  a.lora_hp = lora_dhp;
  a.hp_slices = hp_slices;
  a.ldt = ldt;
  a.lora_ht = static_cast<_Float16*>(lora_dht);
  a.lora_w = static_cast<const _Float16*>(lora_at);
  a.r = r;
  a.mask = static_cast<const uint8_t*>(mask);
  a.mask_scale = mask_scale;
  a.C = static_cast<_Float16*>(dx);
  a.ldc = K;
  set_workspace(a, workspace);
  return gemm_entry(true, a, cfg, splits, stream);
}

int mxs_nf4_linear_fwd_pair_ok(int M, int N0, int N1, int K) {
  return fwd_pair_plan_ok(M, N0, N1, K) ? 1 : 0;
}

int mxs_nf4_linear_fwd_hp_pair(const void* x, int M, int K, const int N[2],
                               const void* const packed[2], const void* const absmax8[2],
                               const float* const code[2], const float* const absmax2[2],
                               const float* const offset[2], const void* const bias[2],
                               const float* const lora_hp[2], int hp_slices, int ldt,
                               const void* const lora_b[2], int r, void* const lora_ht[2],
                               void* const y[2], hipStream_t stream) {
  if (M < 0 || !x || !N || !packed || !absmax8 || !code || !absmax2 || !offset || !lora_hp ||
      !lora_b || !y)
    return MXS_ERR_ARG;
  if (M == 0) return MXS_OK;
  if (!fwd_pair_plan_ok(M, N[0], N[1], K)) return MXS_ERR_SIZE;
  GemmArgs p[2];
  for (int i = 0; i < 2; i++) {
    GemmArgs a{};
    a.A = static_cast<const _Float16*>(x);
    a.lda = K;
    a.packed = static_cast<const uint8_t*>(packed[i]);
    a.absmax8 = static_cast<const uint8_t*>(absmax8[i]);
    a.code = code[i];
    a.absmax2 = absmax2[i];
    a.offset = offset[i];
    a.M = M;
    a.Nc = N[i];
    a.Kr = K;
    a.Kw = K;
    a.bias = bias ? static_cast<const _Float16*>(bias[i]) : nullptr;
    a.lora_hp = lora_hp[i];
    a.hp_slices = hp_slices;
    a.ldt = ldt;
    a.lora_ht = lora_ht ? static_cast<_Float16*>(lora_ht[i]) : nullptr;
    a.lora_w = static_cast<const _Float16*>(lora_b[i]);
    a.r = r;
    a.C = static_cast<_Float16*>(y[i]);
    a.ldc = N[i];
    if (!a.lora_hp) return MXS_ERR_ARG;
    const int c = check_gemm(false, a);
    if (c != MXS_OK) return c == 1 ? MXS_OK : c;
    p[i] = a;
  }
  const int ncut = fwd_pair_mixed_cut(M, N[0], K);
  if (ncut > 0) return launch_ws_fwd_pair_mixed(p[0], p[1], ncut, stream);
  return launch_ws_fwd_pair<256, 160, 4, 1, 4, 4>(p[0], p[1], stream);
}

int mxs_nf4_linear_bwd_dx_pair_ok(int M, int N0, int N1, int K) {
  return pair_plan_ok(M, N0, N1, K) ? 1 : 0;
}

int64_t mxs_nf4_linear_bwd_dx_pair_workspace_bytes(int M, int N0, int N1, int K) {
  if (!pair_plan_ok(M, N0, N1, K)) return 0;
  return (int64_t)2 * kPairSplits * M * K * (int64_t)sizeof(float);
}

int mxs_nf4_linear_bwd_dx_hp_pair(const void* const dy[2], int M, const int N[2], int K,
                                  const void* const packed[2], const void* const absmax8[2],
                                  const float* const code[2], const float* const absmax2[2],
                                  const float* const offset[2], const float* const lora_dhp[2],
                                  int hp_slices, int ldt, const void* const lora_at[2], int r,
                                  const void* const mask[2], float mask_scale,
                                  void* const lora_dht[2], void* dx, void* workspace,
                                  hipStream_t stream) {
  GemmArgs p[2];
  const int c = dx_pair_args(dy, M, N, K, packed, absmax8, code, absmax2, offset, lora_dhp,
                             hp_slices, ldt, lora_at, r, mask, mask_scale, lora_dht, dx,
                             workspace, p);
  if (c != MXS_OK) return c == 1 ? MXS_OK : c;
  return launch_ws_pair<256, 96, 4, 1, true, 8, 5>(p[0], p[1], kPairSplits, stream);
}

int mxs_nf4_linear_bwd_dx_hp_pair_grads(
    const void* const dy[2], int M, const int N[2], int K, const void* const packed[2],
    const void* const absmax8[2], const float* const code[2], const float* const absmax2[2],
    const float* const offset[2], const float* const lora_dhp[2], int hp_slices, int ldt,
    const void* const lora_at[2], int r, const void* const mask[2], float mask_scale,
    void* const lora_dht[2], const void* const ht[2], const void* x, float* const da[2],
    float* const db[2], void* dx, void* workspace, hipStream_t stream) {
  if (!lora_dht || !ht || !x || !da || !db) return MXS_ERR_ARG;
  GemmArgs p[2];
  const int c = dx_pair_args(dy, M, N, K, packed, absmax8, code, absmax2, offset, lora_dhp,
                             hp_slices, ldt, lora_at, r, mask, mask_scale, lora_dht, dx,
                             workspace, p);
  if (c == 1) {  // no tokens: dX is empty, dA and dB are empty reductions (zeros)
    for (int i = 0; i < 2; i++) {
      const int e = mxs_lora_grads(nullptr, nullptr, ldt, nullptr, nullptr, 0, K, N[i], r,
                                   nullptr, mask_scale, da[i], db[i], nullptr, stream);
      if (e != MXS_OK) return e;
    }
    return MXS_OK;
  }
  if (c != MXS_OK) return c;
  if (r % 16) return MXS_ERR_SIZE;
  ColsGroup g{};
  g.n = 2;
  const int cpl = cols_cpl(K + N[0]);
  for (int i = 0; i < 2; i++) {
    const int e = cols_group_set(g, i, lora_dht[i], ht[i], ldt, x, dy[i], M, K, N[i],
                                 mask ? mask[i] : nullptr, mask_scale, da[i], db[i]);
    if (e != MXS_OK) return e;
    if (cols_cpl(K + N[i]) != cpl) return MXS_ERR_SIZE;
  }
  const int e = launch_ws_pair<256, 96, 4, 1, true, 8, 5>(p[0], p[1], kPairSplits, stream, false);
  if (e != MXS_OK) return e;
  if (cpl == 8) return reduce_cols_launch<8>(p[0], 2 * kPairSplits, g, M, ldt, r, stream);
  if (cpl == 4) return reduce_cols_launch<4>(p[0], 2 * kPairSplits, g, M, ldt, r, stream);
  return reduce_cols_launch<2>(p[0], 2 * kPairSplits, g, M, ldt, r, stream);
}

// The rotation the grouped forward may apply to its first n_rope problems (attention's q / k).
struct RopeSpec {
  int n_rope;
  const float* cos;
  const float* sin;
  int64_t cs_b, cs_t;
  int T;
};

static int fwd_hp_group(int n, const void* const x[], int M, int K, const int N[],
                        const void* const packed[], const void* const absmax8[],
                        const float* const code[], const float* const absmax2[],
                        const float* const offset[], const void* const bias[],
                        const float* const lora_hp[], int hp_slices, int ldt,
                        const void* const lora_b[], int r, void* const lora_ht[],
                        void* const y[], const RopeSpec& rs, hipStream_t stream) {
  if (n < 1 || n > kMaxGemmGroup || !x || !N || !packed || !absmax8 || !code || !absmax2 ||
      !offset || !y || rs.n_rope < 0 || rs.n_rope > n)
    return MXS_ERR_ARG;
  if (rs.n_rope > 0) {
    if (!rs.cos || !rs.sin || rs.T < 1 || M % rs.T != 0 || rs.cs_b < 0 || rs.cs_t < 0)
      return MXS_ERR_ARG;
    // float4 reads of cos / sin rows
    if ((uintptr_t)rs.cos % 16 || (uintptr_t)rs.sin % 16 || rs.cs_b % 4 || rs.cs_t % 4)
      return MXS_ERR_ALIGN;
    for (int i = 0; i < rs.n_rope; i++)
      if (N[i] % 128 != 0) return MXS_ERR_SIZE;  // whole 128-column heads
  }
  GemmArgs probs[kMaxGemmGroup];
  int live = 0;
  for (int i = 0; i < n; i++) {
    GemmArgs a{};
    a.A = static_cast<const _Float16*>(x[i]);
    a.lda = K;
    a.packed = static_cast<const uint8_t*>(packed[i]);
    a.absmax8 = static_cast<const uint8_t*>(absmax8[i]);
    a.code = code[i];
    a.absmax2 = absmax2[i];
    a.offset = offset[i];
    a.M = M;
    a.Nc = N[i];
    a.Kr = K;
    a.Kw = K;
    a.bias = bias ? static_cast<const _Float16*>(bias[i]) : nullptr;
    const float* hp = lora_hp ? lora_hp[i] : nullptr;
    if (hp) {
      a.lora_hp = hp;
      a.hp_slices = hp_slices;
      a.ldt = ldt;
      a.lora_ht = lora_ht ? static_cast<_Float16*>(lora_ht[i]) : nullptr;
      a.lora_w = lora_b ? static_cast<const _Float16*>(lora_b[i]) : nullptr;
      a.r = r;
    }
    a.C = static_cast<_Float16*>(y[i]);
    a.ldc = N[i];
    if (i < rs.n_rope) {
      a.rope_cos = rs.cos;
      a.rope_sin = rs.sin;
      a.rope_cs_b = rs.cs_b;
      a.rope_cs_t = rs.cs_t;
      a.rope_T = rs.T;
    }
    const int c = check_gemm(false, a);
    if (c == 1) continue;  // nothing to compute for this one
    if (c != MXS_OK) return c;
    probs[live++] = a;
  }
  if (live == 0) return MXS_OK;
  // 128x64 tiles when every problem's tiles together fit the CUs in one round (q, k and v at
  // 1024 tokens: 192 + 32 + 32 = 256 tiles), as the planner does for one problem; else 128x128.
  // With the rotation the 128x64 tiles take 4 x 1 consumer waves (each wave's two 32-column
  // blocks are one head's halves); the products, and so the bits, are those of the 2 x 2 layout.
  int64_t tiles64 = 0;
  for (int i = 0; i < live; i++)
    tiles64 += (int64_t)((M + 127) / 128) * ((probs[i].Nc + 63) / 64);
  const int cus = cu_count();
  const bool t64 = cus > 0 && tiles64 <= cus;
  if (rs.n_rope > 0)
    return t64 ? launch_ws_group<false, 64, 4, 1, true>(probs, live, stream)
               : launch_ws_group<false, 128, 2, 2, true>(probs, live, stream);
  if (t64) return launch_ws_group<false, 64>(probs, live, stream);
  return launch_ws_group<false>(probs, live, stream);
}

int mxs_nf4_linear_fwd_hp_group(int n, const void* const x[], int M, int K, const int N[],
                                const void* const packed[], const void* const absmax8[],
                                const float* const code[], const float* const absmax2[],
                                const float* const offset[], const void* const bias[],
                                const float* const lora_hp[], int hp_slices, int ldt,
                                const void* const lora_b[], int r, void* const lora_ht[],
                                void* const y[], hipStream_t stream) {
  return fwd_hp_group(n, x, M, K, N, packed, absmax8, code, absmax2, offset, bias, lora_hp,
                      hp_slices, ldt, lora_b, r, lora_ht, y, RopeSpec{}, stream);
}

int mxs_nf4_linear_fwd_hp_group_rope(int n, const void* const x[], int M, int K, const int N[],
                                     const void* const packed[], const void* const absmax8[],
                                     const float* const code[], const float* const absmax2[],
                                     const float* const offset[], const void* const bias[],
                                     const float* const lora_hp[], int hp_slices, int ldt,
                                     const void* const lora_b[], int r, void* const lora_ht[],
                                     void* const y[], int n_rope, const float* cos,
                                     const float* sin, int64_t cos_stride_b,
                                     int64_t cos_stride_t, int n_tokens, hipStream_t stream) {
  if (n_rope < 1) return MXS_ERR_ARG;
  const RopeSpec rs{n_rope, cos, sin, cos_stride_b, cos_stride_t, n_tokens};
  return fwd_hp_group(n, x, M, K, N, packed, absmax8, code, absmax2, offset, bias, lora_hp,
                      hp_slices, ldt, lora_b, r, lora_ht, y, rs, stream);
}

int mxs_nf4_linear_glu_fused(int M, int N, int K, int bwd) {
  return bwd ? (glu_plan_ok(M, K, N, true) ? 1 : 0) : (glu_plan_ok(M, N, K, false) ? 1 : 0);
}

int mxs_nf4_linear_fwd_glu(const void* x, int M, int K, int N, const void* packed,
                           const void* absmax8, const float* code, const float* absmax2,
                           const float* offset, const void* bias, const float* lora_hp,
                           int hp_slices, int ldt, const void* lora_b, int r, void* lora_ht,
                           const void* gate, void* y, void* h, void* workspace,
                           hipStream_t stream) {
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(x);
  a.lda = K;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = N;
  a.Kr = K;
  a.Kw = K;
  a.bias = static_cast<const _Float16*>(bias);
  if (lora_hp) {
    a.lora_hp = lora_hp;
    a.hp_slices = hp_slices;
    a.ldt = ldt;
    a.lora_ht = static_cast<_Float16*>(lora_ht);
    a.lora_w = static_cast<const _Float16*>(lora_b);
    a.r = r;
  }
  a.C = static_cast<_Float16*>(y);
  a.ldc = N;
  a.glu = 1;
  a.glu_g = static_cast<_Float16*>(const_cast<void*>(gate));
  a.glu_h = static_cast<_Float16*>(h);
  set_workspace(a, workspace);
  return gemm_entry(false, a, -1, 1, stream);
}

int mxs_nf4_linear_bwd_dx_glu(const void* dy, int M, int N, int K, const void* packed,
                              const void* absmax8, const float* code, const float* absmax2,
                              const float* offset, const float* lora_dhp, int hp_slices, int ldt,
                              const void* lora_at, int r, const void* mask, float mask_scale,
                              void* lora_dht, void* gate, void* up, void* workspace,
                              hipStream_t stream) {
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(dy);
  a.lda = N;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = K;
  a.Kr = N;
  a.Kw = K;
  if (lora_dhp) {
    a.lora_hp = lora_dhp;
    a.hp_slices = hp_slices;
    a.ldt = ldt;
    a.lora_ht = static_cast<_Float16*>(lora_dht);
    a.lora_w = static_cast<const _Float16*>(lora_at);
    a.r = r;
    a.mask = static_cast<const uint8_t*>(mask);
    a.mask_scale = mask_scale;
  }
  a.ldc = K;
  a.glu = 2;
  a.glu_g = static_cast<_Float16*>(gate);
  a.glu_u = static_cast<_Float16*>(up);
  set_workspace(a, workspace);
  return gemm_entry(true, a, -1, 1, stream);
}

}  // extern "C"

// mxs_nf4_linear_fwd with the split-K partial sums in the library's own device array instead of
// a caller workspace: no allocation of any kind.  Bytes the plan needs above
// MXS_NF4_SCRATCH_BYTES are refused with MXS_ERR_SIZE before anything is launched.
extern "C" int mxs_nf4_linear_fwd_noalloc(const void* x, int M, int K, int N, const void* packed,
                                          const void* absmax8, const float* code,
                                          const float* absmax2, const float* offset,
                                          const void* bias, const void* lora_h,
                                          const void* lora_b, int r, void* y, int cfg,
                                          int splits, hipStream_t stream) {
  if (M < 0 || K < 0 || N < 0) return MXS_ERR_ARG;
  if (cfg < 0) choose(M, N, K, false, &cfg, &splits);
  // the split count the launch will use (launch_cfg / launch_ws clamp it the same way)
  const int n_steps = K / kBK;
  int sp = splits < 1 ? 1 : splits;
  if (sp > n_steps) sp = n_steps > 0 ? n_steps : 1;
  const int per = (n_steps + sp - 1) / sp;
  sp = n_steps > 0 ? (n_steps + per - 1) / per : 1;
  void* ws = nullptr;
  if (sp > 1 && M > 0 && N > 0) {
    const double need = (double)sp * (double)M * (double)N * sizeof(float);
    if (need > (double)MXS_NF4_SCRATCH_BYTES) return MXS_ERR_SIZE;
    const int rc = scratch_address(&ws);
    if (rc != MXS_OK) return rc;
  }
  return mxs_nf4_linear_fwd(x, M, K, N, packed, absmax8, code, absmax2, offset, bias, lora_h,
                            lora_b, r, y, ws, cfg, sp, stream);
}
