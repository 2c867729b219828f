/*
 * mxs_nf4 — C ABI of the MI355X (gfx950) NF4 quantized-linear hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t, allocates nothing,
 * launches asynchronously on `stream`, and returns MXS_OK (0), a negative MXS_ERR_* code for a
 * rejected argument (nothing launched), or a positive hipError_t from the launch.
 *
 * Data layout (bitsandbytes' NF4 QuantState as the reference reads it,
 * solution/linear4bit.py:36-40):
 *   packed   u8  [(N*K)/2]       byte i = value 2i (high nibble) and 2i+1 (low nibble),
 *                                 values flattened row-major over W [N, K]
 *   absmax8  u8  [N*K/64]        8-bit code of each 64-value block's absmax
 *   code     f32 [256]           second-level code book (state2.code)
 *   absmax2  f32 [ceil(N*K/64/256)]  second-level scale per 256 blocks (state2.absmax)
 *   offset   f32 [1]             mean added back (state.offset), a device pointer
 *   block scale = fma(code[absmax8[b]], absmax2[b >> 8], offset); value = fp16(NF4[q] * scale)
 *
 * Dropout keep masks (every `mask` argument) are bits: u32 [M, ceil(K/32)] for a mask over
 * [M, K], bit k % 32 of word k / 32 of row m set where element (m, k) is kept, bits past K
 * zero, 4-byte aligned.  mxs_keep_pack makes them from the reference's int8 keep mask
 * (solution/dropout.py:64, `keep` [M, K], nonzero = kept).
 */
#ifndef MXS_NF4_H
#define MXS_NF4_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXS_OK 0
#define MXS_ERR_ARG (-1)    /* null pointer or negative size */
#define MXS_ERR_DTYPE (-2)  /* unsupported output dtype */
#define MXS_ERR_ALIGN (-3)  /* pointer alignment the entry point requires */
#define MXS_ERR_SIZE (-4)   /* shape outside what the kernels take */

#define MXS_DTYPE_F16 0
#define MXS_DTYPE_F32 1

/* Dense W from packed NF4.  Replaces unpack_nf4 (solution/nf4.py:138-155) with its
 * wide/one-byte dispatch (solution/nf4.py:145-154): the wide kernel when n_bytes % 32 == 0 and
 * packed/out are 16-byte aligned, else the one-byte kernel.  absmax8 != NULL selects the nested
 * (double-quantized) form with code/absmax2/offset; absmax8 == NULL takes fp32 absmax_f32
 * [n_bytes/32] (the reference's non-nested branch, solution/nf4.py:74-75).
 * out: fp16 or fp32 [2*n_bytes] (out_dtype MXS_DTYPE_F16 / MXS_DTYPE_F32). */
int mxs_nf4_dequant(const void* packed, int64_t n_bytes, const void* absmax8, const float* code,
                    const float* absmax2, const float* offset, const float* absmax_f32,
                    void* out, int out_dtype, hipStream_t stream);

/* The one-byte-per-lane kernel, launched directly: nf4_unpack_kernel (solution/nf4.py:31-51) as
 * solution/test_nf4.py:68-82 launches it.  Same arguments and result as mxs_nf4_dequant. */
int mxs_nf4_dequant_bytewise(const void* packed, int64_t n_bytes, const void* absmax8,
                             const float* code, const float* absmax2, const float* offset,
                             const float* absmax_f32, void* out, int out_dtype,
                             hipStream_t stream);

/* Several NF4 weights stored back to back, decoded by one launch to fp16 stored back to back.
 * Replaces launch_layer / nf4_layer_kernel (solution/nf4.py:158-162, 89-110).
 * Module m owns blocks [block0[m], block0[m+1]) of packed/absmax8/out, code
 * [m*256, m*256+256), absmax2 from index scale0[m], and offset[m].
 * block0: device int64 [n_modules + 1] ascending, block0[0] = 0, block0[n_modules] = n_blocks;
 * scale0: device int64 [n_modules].  packed and out must be 16-byte aligned.
 * wg_module: device int16 map from mxs_nf4_dequant_layer_plan (the counterpart of the
 * reference's per-program `module_of`, solution/stream.py:125-133) with its n_plan entries
 * (one per workgroup: ceil(n_blocks / 128), else MXS_ERR_SIZE), or NULL to look each block's
 * module up in the kernel (slower). */
int mxs_nf4_dequant_layer(const void* packed, int64_t n_blocks, const void* absmax8,
                          const float* code, const float* absmax2, const float* offset,
                          const int64_t* block0, const int64_t* scale0, int n_modules,
                          const int16_t* wg_module, int64_t n_plan, void* out,
                          hipStream_t stream);

/* Host-side plan for mxs_nf4_dequant_layer: from HOST block0 [n_modules + 1], writes the module
 * of each of the kernel's workgroups (-1 where one straddles two modules) into HOST wg_module
 * [capacity] and returns the number of workgroups; with wg_module NULL it only returns that
 * number.  Negative MXS_ERR_* on bad arguments. */
int64_t mxs_nf4_dequant_layer_plan(const int64_t* block0, int n_modules, int16_t* wg_module,
                                   int64_t capacity);

/* Workspace bytes mxs_nf4_quantize needs for n_values (device memory, 8-byte aligned). */
int mxs_nf4_quantize_workspace_bytes(int64_t n_values);

/* NF4 quantizer with double-quantized absmax (upstream of the path: it makes the packed
 * weights).  Stands in for bitsandbytes' quantize_4bit(w, blocksize=64, quant_type="nf4",
 * compress_statistics=True) as the reference calls it (solution/test_nf4.py:33,
 * tools/bench_nf4.py:30-35).  w_f16 [n_values] (16-byte aligned, n_values % 64 == 0) ->
 * packed u8 [n/2], absmax_f32 [n/64] (first level, kept for checks), absmax8 u8 [n/64],
 * absmax2 f32 [ceil(n/64/256)], offset f32 [1]; code f32 [256] is the second-level code book
 * (ascending).  Deterministic. */
int mxs_nf4_quantize(const void* w_f16, int64_t n_values, const float* code, void* packed,
                     float* absmax_f32, void* absmax8, float* absmax2, float* offset,
                     void* workspace, hipStream_t stream);

/* ---- Fused NF4 GEMMs (forward and input gradient of the frozen Linear4bit) ---------------
 * cfg: tile configuration id (0-4: all-wave kernels, 6-12: producer/consumer kernels; 5 is
 * invalid) or -1 to let the library choose tiles and split-K for the shape; splits: reduction
 * splits (used with cfg >= 0).  When the plan splits the reduction, `workspace` must hold
 * mxs_nf4_gemm_workspace_bytes(M, Nc, Kr, cfg, splits) bytes of device memory (fp32 partial
 * sums, no initial contents needed; a return of 0 means no workspace is needed) and a second
 * small kernel adds the partials in split order: results are deterministic.  Shapes:
 * in_features % 64 == 0, reduction % 64 == 0; x/dy 16-byte aligned. */
int64_t mxs_nf4_gemm_workspace_bytes(int M, int Nc, int Kr, int cfg, int splits);

/* Y[M,N] = X[M,K] . W[N,K]^T (+ bias[N]) (+ lora_h[M,r] . lora_b[N,r]^T), fp16 in/out, fp32
 * accumulation, W decoded from NF4 inside the GEMM.  Replaces NF4LinearFunction.forward
 * (solution/linear4bit.py:47-49: unpack, then F.linear) and adds peft's LoRA branch
 * (solution/attention.py:197-199) as an epilogue: lora_h = s * H from mxs_lora_h, so the added
 * term is s * B(A(drop(x))).  bias and lora_h may be NULL. */
int mxs_nf4_linear_fwd(const void* x, int M, int K, int N, const void* packed,
                       const void* absmax8, const float* code, const float* absmax2,
                       const float* offset, const void* bias, const void* lora_h,
                       const void* lora_b, int r, void* y, void* workspace, int cfg, int splits,
                       hipStream_t stream);

/* Upper bound on the split-K partial sums mxs_nf4_linear_fwd_noalloc keeps in the library's own
 * device memory (32 MiB per GPU, held from library load to process exit). */
#define MXS_NF4_SCRATCH_BYTES (32u << 20)

/* mxs_nf4_linear_fwd without the workspace argument, for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * No counterpart in the reference (its forward allocates through torch).  Nothing is allocated:
 * split-K partials go to a file-scope device array of MXS_NF4_SCRATCH_BYTES, whose address is
 * looked up once per device on the first call made with that device current.  That lookup is
 * not a stream operation: under HIP graph capture, make one call on the device before the
 * capture begins; the calls after it launch kernels only and are capturable.  A plan needing
 * more (splits * M * N * 4 bytes) returns MXS_ERR_SIZE with nothing launched.  Every call on
 * one GPU shares that array: calls that overlap in time on one GPU (other streams or threads)
 * race and must be serialized by the caller.  Same results as mxs_nf4_linear_fwd. */
int mxs_nf4_linear_fwd_noalloc(const void* x, int M, int K, int N, const void* packed,
                               const void* absmax8, const float* code, const float* absmax2,
                               const float* offset, const void* bias, const void* lora_h,
                               const void* lora_b, int r, void* y, int cfg, int splits,
                               hipStream_t stream);

/* dX[M,K] = dY[M,N] . W[N,K] (+ mask[M,K] * mask_scale * (lora_dh[M,r] . lora_at[K,r]^T)), with
 * W decoded from NF4 inside the GEMM.  Replaces NF4LinearFunction.backward
 * (solution/linear4bit.py:51-57: unpack again, then grad @ W) plus the LoRA branch's input
 * gradient through the dropout (solution/dropout.py:62-69); lora_dh = s * dY . B from
 * mxs_lora_dh, lora_at = lora_A transposed ([K, r]: the `at` output of mxs_lora_h, or
 * mxs_transpose_f16).  mask: keep bits of [M,K]
 * or NULL (no dropout); mask_scale = 1/(1-p). */
int mxs_nf4_linear_bwd_dx(const void* dy, int M, int N, int K, const void* packed,
                          const void* absmax8, const float* code, const float* absmax2,
                          const float* offset, const void* lora_dh, const void* lora_at, int r,
                          const void* mask, float mask_scale, void* dx, void* workspace, int cfg,
                          int splits, hipStream_t stream);

/* mxs_nf4_linear_bwd_dx (finished lora_dh) and mxs_lora_grads (dA = dht . drop(x) [r, K],
 * dB = dY^T . ht^T [N, r], fp32) in one launch where they fit the GPU together: the gradient
 * workgroups need nothing the dX tiles write and run on the CUs the tiles leave idle.  This is
 * the whole backward of a projection after dHs, i.e. NF4LinearFunction.backward
 * (solution/linear4bit.py:51-57) plus the input and weight gradients autograd takes through
 * peft's LoRA branch (solution/attention.py:197-199, solution/dropout.py:62-69).  Where the
 * planned dX kernel cannot take the extra workgroups (split-K, or the GPU already full) it
 * makes the same two launches as the separate entry points; results are the same either way.
 * lora_dh [M, r] and dht [r, ldt] are the outputs of one mxs_lora_dh call without a workspace;
 * ht is the forward's transposed Hs.  All outputs are required. */
int mxs_nf4_linear_bwd_dx_grads(const void* dy, int M, int N, int K, const void* packed,
                                const void* absmax8, const float* code, const float* absmax2,
                                const float* offset, const void* lora_dh, const void* lora_at,
                                int r, const void* mask, float mask_scale, const void* dht,
                                const void* ht, int ldt, const void* x, float* da, float* db,
                                void* dx, void* workspace, hipStream_t stream);

/* 1 when mxs_nf4_linear_bwd_dx_grads makes one launch for this shape (projection in_features K,
 * out_features N, M tokens, rank r) on the current device, else 0.  A caller picks the dHs
 * kernel by it: one finished launch (mxs_lora_dh) for the fused path, slice partials
 * (mxs_lora_dh_partials + mxs_nf4_linear_bwd_dx_hp) otherwise. */
int mxs_nf4_linear_bwd_grads_fused(int M, int N, int K, int r);

/* mxs_nf4_linear_fwd with the LoRA activations given as fp32 partial sums (from
 * mxs_lora_h_partials) instead of lora_h: lora_hp [hp_slices][ldt][r] (1 <= hp_slices <= 4,
 * ldt >= M, ldt % 8 == 0), already times s.  The GEMM adds the slices in order, rounds to fp16
 * and uses that as lora_h; with lora_ht != NULL it also writes that fp16 operand transposed,
 * [r, ldt] with zeros past M (the input of mxs_lora_grads' dB).  Saves the separate launch that
 * would finish lora_h. */
int mxs_nf4_linear_fwd_hp(const void* x, int M, int K, int N, const void* packed,
                          const void* absmax8, const float* code, const float* absmax2,
                          const float* offset, const void* bias, const float* lora_hp,
                          int hp_slices, int ldt, const void* lora_b, int r, void* lora_ht,
                          void* y, void* workspace, int cfg, int splits, hipStream_t stream);

/* mxs_nf4_linear_bwd_dx with s * dH given as fp32 partial sums (from mxs_lora_dh_partials),
 * [hp_slices][ldt][r]; with lora_dht != NULL it also writes fp16 s * dH transposed, [r, ldt]
 * (the input of mxs_lora_grads' dA). */
int mxs_nf4_linear_bwd_dx_hp(const void* dy, int M, int N, int K, const void* packed,
                             const void* absmax8, const float* code, const float* absmax2,
                             const float* offset, const float* lora_dhp, int hp_slices, int ldt,
                             const void* lora_at, int r, const void* mask, float mask_scale,
                             void* lora_dht, void* dx, void* workspace, int cfg, int splits,
                             hipStream_t stream);

/* The input gradient of two projections that read the same input, summed: dX = dX_0 + dX_1
 * with dX_i = dY_i . W_i + mask_i * mask_scale * (fp16(sum of lora_dhp_i) . lora_at_i^T), as
 * mxs_nf4_linear_bwd_dx_hp computes each.  These are the gate and up projections of the MLP
 * (solution/mlp.py:42-43), whose input gradients autograd adds for their shared input.  ONE
 * launch of the split-K kernel runs both reductions (each split two ways) and one reduce adds
 * the four fp32 partial planes in order, so neither dX_i is rounded to fp16 on its own; the
 * result equals the fp32 sum of the two GEMMs rounded once.  Arrays hold the per-projection
 * arguments (N[i] = out_features; mask and lora_dht may be NULL, or any entry); the two share
 * M, K, r, ldt, hp_slices and mask_scale.  workspace: at least
 * mxs_nf4_linear_bwd_dx_pair_workspace_bytes(M, N[0], N[1], K) bytes.  Only where
 * mxs_nf4_linear_bwd_dx_pair_ok(M, N[0], N[1], K) is 1 (both projections plan the narrow-output
 * split-K kernel on their own), else MXS_ERR_SIZE. */
int mxs_nf4_linear_bwd_dx_hp_pair(const void* const dy[2], int M, const int N[2], int K,
                                  const void* const packed[2], const void* const absmax8[2],
                                  const float* const code[2], const float* const absmax2[2],
                                  const float* const offset[2], const float* const lora_dhp[2],
                                  int hp_slices, int ldt, const void* const lora_at[2], int r,
                                  const void* const mask[2], float mask_scale,
                                  void* const lora_dht[2], void* dx, void* workspace,
                                  hipStream_t stream);

/* mxs_nf4_linear_bwd_dx_hp_pair and, in the same calls' stream order, both projections' LoRA
 * gradients as mxs_lora_grads_group computes them from the dHs^T the pair writes (lora_dht,
 * required here), ht[i] = Hs_i^T [r, ldt] and the shared input x [M, K] (dA_i [r, K], dB_i
 * [N[i], r], fp32): the bits of those two calls.  The backward of the gate and up projections'
 * LoRA branches (peft's lora_A / lora_B under solution/mlp.py:42-43) with their summed input
 * gradient.  Two launches instead of three: the pair GEMM, then one launch for its split-K
 * reduce and the gradients (independent of each other), the reduce's workgroups filling the
 * CUs the gradients' last partial round leaves idle.  Same conditions as
 * mxs_nf4_linear_bwd_dx_hp_pair, and the two projections share their gradients' columns per
 * lane (as mxs_lora_grads_group requires). */
int mxs_nf4_linear_bwd_dx_hp_pair_grads(
    const void* const dy[2], int M, const int N[2], int K, const void* const packed[2],
    const void* const absmax8[2], const float* const code[2], const float* const absmax2[2],
    const float* const offset[2], const float* const lora_dhp[2], int hp_slices, int ldt,
    const void* const lora_at[2], int r, const void* const mask[2], float mask_scale,
    void* const lora_dht[2], const void* const ht[2], const void* x, float* const da[2],
    float* const db[2], void* dx, void* workspace, hipStream_t stream);

/* Two projections over the same input x [M, K] (the gate and up projections of the MLP,
 * solution/mlp.py:42-43, each NF4LinearFunction.forward of solution/linear4bit.py:47-49 with
 * peft's LoRA branch) in ONE launch: y[i] and lora_ht[i] as mxs_nf4_linear_fwd_hp computes them
 * (the same bits), arrays of the per-projection arguments (bias and lora_ht may be NULL, or any
 * entry); the two share M, K, r, ldt and hp_slices.  Their tiles share the GPU's rounds: at
 * 1024 tokens 2 x 224 tiles of 256 x 160 would take 1.75 rounds of 256 CUs, so where it fills
 * the CUs better the launch cuts the columns into 256 x 160 tiles and narrower 256 x 128 ones
 * (at 1024 tokens: 192 + 320 tiles, each CU running one of each or two narrow ones).  Only
 * where mxs_nf4_linear_fwd_pair_ok(M,
 * N[0], N[1], K) is 1 (both plan the unsplit 256 x 160 kernel: N[0] == N[1] >= 4096), else
 * MXS_ERR_SIZE. */
int mxs_nf4_linear_fwd_hp_pair(const void* x, int M, int K, const int N[2],
                               const void* const packed[2], const void* const absmax8[2],
                               const float* const code[2], const float* const absmax2[2],
                               const float* const offset[2], const void* const bias[2],
                               const float* const lora_hp[2], int hp_slices, int ldt,
                               const void* const lora_b[2], int r, void* const lora_ht[2],
                               void* const y[2], hipStream_t stream);

/* 1 when mxs_nf4_linear_fwd_hp_pair takes two projections [K -> N0] and [K -> N1] at M tokens,
 * else 0. */
int mxs_nf4_linear_fwd_pair_ok(int M, int N0, int N1, int K);

/* 1 when mxs_nf4_linear_bwd_dx_hp_pair takes two projections [K -> N0] and [K -> N1] at M
 * tokens, else 0. */
int mxs_nf4_linear_bwd_dx_pair_ok(int M, int N0, int N1, int K);

/* Workspace bytes of mxs_nf4_linear_bwd_dx_hp_pair (0 where it does not apply). */
int64_t mxs_nf4_linear_bwd_dx_pair_workspace_bytes(int M, int N0, int N1, int K);

/* ---- LoRA side branch (peft lora.Linear around the 4-bit base, r % 16 == 0, r <= 128) ------
 * The transposed outputs/inputs (ht, dht) are fp16 [r, ldt] with ldt >= M, ldt % 8 == 0 (columns
 * past M hold zeros).  Results are deterministic (fixed summation order).  `workspace` may be
 * NULL: each product is then one launch that reduces inside its workgroups.  With a workspace of
 * mxs_lora_workspace_bytes(M, K, N, r) bytes (no initial contents needed; 0 means none is
 * used) and ldt = M rounded up to 8, mxs_lora_h / mxs_lora_dh split reductions of 1024 or more
 * over up to 4 slices of workgroups and add the slices in a second small launch. */
int64_t mxs_lora_workspace_bytes(int M, int K, int N, int r);

/* h = fp16(s * drop(x) . A^T) [M, r] and ht = its transpose: lora_A of peft's branch with the
 * reference's dropout (solution/dropout.py:33-35, mask: keep bits of [M,K] or NULL) and the scaling s
 * folded in.  x [M,K] fp16, lora_a [r,K] fp16, K % 32 == 0.  Side outputs for the backward
 * (each optional, NULL to skip): at [K, r] = lora_a^T (the operand mxs_nf4_linear_bwd_dx takes)
 * and bt [r, N] = lora_b^T for lora_b [N, r] (the operand mxs_lora_dh takes). */
int mxs_lora_h(const void* x, int M, int K, const void* lora_a, int r, const void* mask,
               float mask_scale, float s, void* h, void* ht, int ldt, void* at,
               const void* lora_b, int N, void* bt, void* workspace, hipStream_t stream);

/* dh = fp16(s * dY . B) [M, r] and dht = its transpose (the gradient reaching lora_B's output,
 * times s).  dy [M,N] fp16, lora_bt = lora_B transposed [r, N] fp16 (the bt output of
 * mxs_lora_h), N % 32 == 0. */
int mxs_lora_dh(const void* dy, int M, int N, const void* lora_bt, int r, float s, void* dh,
                void* dht, int ldt, void* workspace, hipStream_t stream);

/* dA[r,K] (fp32) = dh^T . drop(x): lora_A's weight gradient (autograd of peft's nn.Linear). */
int mxs_lora_grad_a(const void* dht, int ldt, const void* x, int M, int K, int r,
                    const void* mask, float mask_scale, float* da, void* workspace,
                    hipStream_t stream);

/* dB[N,r] (fp32) = dY^T . h (h = s * H): lora_B's weight gradient. */
int mxs_lora_grad_b(const void* ht, int ldt, const void* dy, int M, int N, int r, float* db,
                    void* workspace, hipStream_t stream);

/* Keep bits (the mask format of every entry point) from a byte keep mask: keep [M, K] u8,
 * nonzero = kept (the reference's int8 `keep` of PackedDropout, solution/dropout.py:47-69, drawn
 * by F.dropout at :106-119); bits u32 [M, ceil(K/32)].  One launch; reads M*K bytes, writes
 * M*K/8. */
int mxs_keep_pack(const void* keep, int M, int K, void* bits, hipStream_t stream);

/* Number of reduction slices (1..4) mxs_lora_h_partials / mxs_lora_dh_partials use for M tokens
 * and a reduction of length Kr: their partials buffer is fp32 [slices][ldt][r]. */
int mxs_lora_slices(int M, int Kr);

/* The products of mxs_lora_h as fp32 partial sums times s, one per reduction slice, for the
 * fused GEMM (mxs_nf4_linear_fwd_hp) to finish: partials [mxs_lora_slices(M, K)][ldt][r]
 * (rows past M hold zeros).  One launch; at / bt side outputs as in mxs_lora_h. */
int mxs_lora_h_partials(const void* x, int M, int K, const void* lora_a, int r, const void* mask,
                        float mask_scale, float s, int ldt, void* at, const void* lora_b, int N,
                        void* bt, float* partials, hipStream_t stream);

/* The products of mxs_lora_dh as fp32 partial sums times s, [mxs_lora_slices(M, N)][ldt][r], for
 * mxs_nf4_linear_bwd_dx_hp.  One launch. */
int mxs_lora_dh_partials(const void* dy, int M, int N, const void* lora_bt, int r, float s,
                         int ldt, float* partials, hipStream_t stream);

/* mxs_lora_h_partials for n (1..4) projections over the same M tokens in ONE launch: the q, k,
 * v (or gate, up) projections of a layer read the same activations (solution/attention.py
 * :259-266, solution/mlp.py:42-43).  Problem i: x[i] [M, K[i]], lora_a[i] [r, K[i]], mask[i]
 * (mask may be NULL, or any entry), the side outputs at[i], lora_b[i] / N[i] / bt[i] (each array
 * may be NULL), partials[i] [mxs_lora_slices(M, K[i])][ldt][r].  Each problem's workgroups run
 * as its own launch would: the partials are the same bits as n separate calls. */
int mxs_lora_h_partials_group(int n, const void* const x[], int M, const int K[],
                              const void* const lora_a[], int r, const void* const mask[],
                              float mask_scale, float s, int ldt, void* const at[],
                              const void* const lora_b[], const int N[], void* const bt[],
                              float* const partials[], hipStream_t stream);

/* mxs_lora_h_partials_group for LoRA weights kept in fp32 (peft keeps its adapter weights in
 * fp32 and casts them for each fp16 forward, solution/attention.py:197-199 under autocast):
 * lora_a[i] fp32 [r, K[i]] and lora_b[i] fp32 [N[i], r] are read in place and rounded to fp16
 * (nearest even) where used, and the fp16 operands the GEMMs and the backward take come out as
 * side outputs: at[i] = fp16(A)^T [K, r], bt[i] = fp16(B)^T [r, N], b16[i] = fp16(B) [N, r]
 * (each array, or entry, may be NULL).  The same bits as casting the weights to fp16 first and
 * calling mxs_lora_h_partials_group, without the two cast launches per projection. */
int mxs_lora_h_partials_group_w32(int n, const void* const x[], int M, const int K[],
                                  const float* const lora_a[], int r, const void* const mask[],
                                  float mask_scale, float s, int ldt, void* const at[],
                                  const float* const lora_b[], const int N[], void* const bt[],
                                  void* const b16[], float* const partials[],
                                  hipStream_t stream);

/* mxs_lora_dh_partials for n (1..4) projections in ONE launch (their output gradients arrive
 * together: q/k/v from attention's backward, gate/up from the SwiGLU's); same bits as n calls. */
int mxs_lora_dh_partials_group(int n, const void* const dy[], int M, const int N[],
                               const void* const lora_bt[], int r, float s, int ldt,
                               float* const partials[], hipStream_t stream);

/* mxs_lora_dh without a workspace (one launch per problem: finished dh [M, r] and dht [r, ldt])
 * for n (1..4) projections in ONE launch; same bits as n such calls.  The input of
 * mxs_nf4_linear_bwd_dx_grads for each. */
int mxs_lora_dh_group(int n, const void* const dy[], int M, const int N[],
                      const void* const lora_bt[], int r, float s, int ldt, void* const dh[],
                      void* const dht[], hipStream_t stream);

/* mxs_lora_grads (both dA and dB) for n (1..4) projections over the same M tokens in ONE launch
 * (gate's and up's arrive together in the MLP's backward): arrays of the per-projection
 * pointers and sizes, mask may be NULL (or any entry).  The projections must share the
 * columns-per-lane choice of their own launches (cols(K + N) equal, e.g. equal shapes; else
 * MXS_ERR_SIZE); then the results are the bits of n calls. */
int mxs_lora_grads_group(int n, const void* const dht[], const void* const ht[], int ldt,
                         const void* const x[], const void* const dy[], int M, const int K[],
                         const int N[], int r, const void* const mask[], float mask_scale,
                         float* const da[], float* const db[], hipStream_t stream);

/* The fp16 operand from such partial sums [slices][ldt][r] (1 <= slices <= 4; added in slice
 * order and rounded, the value the fused GEMMs compute from the same partials): out [M, r] (may
 * be NULL) and outT [r, ldt] with zeros past M.  Finishes dh from mxs_lora_dh_partials for
 * mxs_lora_grads while the dX GEMM runs, i.e. the tensor autograd hands to lora_B's backward
 * (solution/attention.py:197-199).  One launch. */
int mxs_lora_finish(const float* partials, int slices, int M, int r, int ldt, void* out,
                    void* outT, hipStream_t stream);

/* mxs_lora_grad_a and mxs_lora_grad_b in one launch (either output may be NULL): the two weight
 * gradients autograd computes for peft's lora_A and lora_B (solution/attention.py:197-199 under
 * torch.autograd).  M == 0 writes zero gradients. */
int mxs_lora_grads(const void* dht, const void* ht, int ldt, const void* x, const void* dy, int M,
                   int K, int N, int r, const void* mask, float mask_scale, float* da, float* db,
                   void* workspace, hipStream_t stream);

/* ---- SwiGLU of the fp16 MLP (solution/mlp.py:35-44 calls it between the projections) ------
 * fp32 arithmetic on fp16 inputs, rounded to fp16 once; sigmoid(g) = 1 / (1 + exp(-g)).
 * n = number of elements of contiguous fp16 buffers (any n; 16-byte aligned buffers take the
 * vector path). */

/* out = silu(gate) * up: silu_mul_kernel's forward (solution/silu_mul.py:26-44, called by
 * SiluMulInPlace.forward :56-63). */
int mxs_silu_mul(const void* gate, const void* up, void* out, int64_t n, hipStream_t stream);

/* In-place backward for the incoming gradient `grad`: gate <- d(gate), up <- d(up), as
 * SiluMulInPlace.backward (solution/silu_mul.py:65-71) does. */
int mxs_silu_mul_bwd(const void* grad, void* gate, void* up, int64_t n, hipStream_t stream);

/* mxs_nf4_linear_fwd_hp for n (1..4) projections of one input width K over the same M tokens in
 * ONE launch (the q, k and v projections of a layer read the same activations,
 * solution/attention.py:259-266): problem i has x[i] [M, K], out_features N[i], its NF4 weight
 * (packed[i] .. offset[i]), bias[i], LoRA partials lora_hp[i] (hp_slices, ldt, r shared),
 * lora_b[i] [N[i], r], lora_ht[i], output y[i] [M, N[i]]; the bias, lora_hp, lora_b and lora_ht
 * arrays may be NULL (or any entry: no bias / no LoRA term).  Every problem runs unsplit on
 * warp-specialized tiles with 8 producer waves, 128x64 when all the problems' tiles fit the CUs
 * in one round (q, k and v at 1024 tokens), else 128x128: the same bits as mxs_nf4_linear_fwd_hp
 * with one split for each (every warp-specialized configuration accumulates in one order; the
 * N = 256 projections alone would plan split-K tiles and a reduce). */
int mxs_nf4_linear_fwd_hp_group(int n, const void* const x[], int M, int K, const int N[],
                                const void* const packed[], const void* const absmax8[],
                                const float* const code[], const float* const absmax2[],
                                const float* const offset[], const void* const bias[],
                                const float* const lora_hp[], int hp_slices, int ldt,
                                const void* const lora_b[], int r, void* const lora_ht[],
                                void* const y[], hipStream_t stream);

/* mxs_nf4_linear_fwd_hp_group whose first n_rope (1..n) outputs are rotated as mxs_qkv_rope
 * rotates q and k (solution/attention.py:28-82, qkv_rope_kernel, on the projections' own
 * outputs; its caller solution/attention.py:259-271 projects q, k, v and then rotates): y[i]
 * for i < n_rope holds rot(the fp16 projection output), each 128-column head rotated by the
 * fp32 cos / sin row of its token (row m is token m % n_tokens of sequence m / n_tokens; rows
 * at b * cos_stride_b + t * cos_stride_t, cos_stride_b may be 0; 16-byte aligned, strides
 * multiples of 4).  The stored fp16 has the bits of mxs_nf4_linear_fwd_hp_group followed by
 * mxs_qkv_rope (forward, no LoRA term) on those outputs; the remaining outputs (v) are
 * unchanged.  N[i] of a rotated output: a multiple of 128; M a multiple of n_tokens. */
int mxs_nf4_linear_fwd_hp_group_rope(int n, const void* const x[], int M, int K, const int N[],
                                     const void* const packed[], const void* const absmax8[],
                                     const float* const code[], const float* const absmax2[],
                                     const float* const offset[], const void* const bias[],
                                     const float* const lora_hp[], int hp_slices, int ldt,
                                     const void* const lora_b[], int r, void* const lora_ht[],
                                     void* const y[], int n_rope, const float* cos,
                                     const float* sin, int64_t cos_stride_b,
                                     int64_t cos_stride_t, int n_tokens, hipStream_t stream);

/* 1 when mxs_nf4_linear_bwd_dx_grads_group takes these n (1..4) projections [K -> N[i]] at M
 * tokens: each one mxs_nf4_linear_bwd_grads_fused(M, N[i], K, r) would run as one launch on
 * 128x128 tiles. */
int mxs_nf4_linear_bwd_dx_grads_group_ok(int n, int M, const int N[], int K, int r);

/* mxs_nf4_linear_bwd_dx_grads for n (1..4) projections of one input width K in ONE launch (the
 * q, k and v projections' output gradients arrive together from attention's backward): each
 * problem's dX tiles, then its dA / dB workgroups; the same bits as the n calls.  Arrays hold
 * the per-projection pointers (mask may be NULL, or any entry); only where
 * mxs_nf4_linear_bwd_dx_grads_group_ok says so (else MXS_ERR_SIZE). */
int mxs_nf4_linear_bwd_dx_grads_group(int n, const void* const dy[], int M, const int N[], int K,
                                      const void* const packed[], const void* const absmax8[],
                                      const float* const code[], const float* const absmax2[],
                                      const float* const offset[], const void* const lora_dh[],
                                      const void* const lora_at[], int r,
                                      const void* const mask[], float mask_scale,
                                      const void* const dht[], const void* const ht[], int ldt,
                                      const void* const x[], float* const da[],
                                      float* const db[], void* const dx[], hipStream_t stream);

/* 1 when mxs_nf4_linear_bwd_dx_grads_sum takes these n (2..3) projections [K -> N[i]] of one
 * input at M tokens: rank r = 16, K >= 1024 and a multiple of 64, each N[i] a multiple of 64
 * whose own dX launch runs unsplit (q, k and v; not gate and up, whose long reductions take the
 * split-K pair); with the LoRA gradients (grads != 0) also each projection's dA / dB workgroups as
 * mxs_nf4_linear_bwd_dx_grads would run them (up to 1152 tokens). */
int mxs_nf4_linear_bwd_dx_grads_sum_ok(int n, int M, const int N[], int K, int r, int grads);

/* The q, k and v projections' backward as autograd needs it: ONE dX for their shared input x,
 *   dx = sum_i ( dy[i] . W_i + mask[i] * mask_scale * (lora_dh[i] . lora_at[i]^T) )  [M, K],
 * and every projection's dA[i] / dB[i] (as mxs_nf4_linear_bwd_dx_grads), in one launch: each
 * output tile runs the projections' reductions back to back (K-steps of dy[0] . W_0, then
 * dy[1] . W_1, ...) into one fp32 accumulator that started from all their LoRA terms (each
 * masked by its own keep bits), and is rounded to fp16 once; the gradient workgroups follow
 * the tiles.  The sum of mxs_nf4_linear_bwd_dx_grads_group's dx[i] rounded each and added in
 * fp16 differs from it by the roundings of the parts (a couple of fp16 ulps).  Every projection
 * has a keep mask or none does.  da and db NULL: the summed dX alone (dht, ht and x unused, may
 * be NULL), where mxs_nf4_linear_bwd_dx_grads_sum_ok(..., 0) says so; the caller then takes
 * dA / dB from mxs_lora_grads.  Reference: the per-projection input gradient of
 * solution/linear4bit.py:51-57 (plus peft's LoRA branch), added by autograd for the shared
 * input.  Only where mxs_nf4_linear_bwd_dx_grads_sum_ok says so (else MXS_ERR_SIZE). */
int mxs_nf4_linear_bwd_dx_grads_sum(int n, const void* const dy[], int M, const int N[], int K,
                                    const void* const packed[], const void* const absmax8[],
                                    const float* const code[], const float* const absmax2[],
                                    const float* const offset[], const void* const lora_dh[],
                                    const void* const lora_at[], int r, const void* const mask[],
                                    float mask_scale, const void* const dht[],
                                    const void* const ht[], int ldt, const void* x,
                                    float* const da[], float* const db[], void* dx,
                                    hipStream_t stream);

/* The up projection's forward with the SwiGLU after it (solution/mlp.py:42-43:
 * silu_mul(gate_proj(x), up_proj(x))): mxs_nf4_linear_fwd_hp (lora_hp may be NULL: no LoRA
 * term) writing y = up_proj(x) [M, N] and h = silu(gate) * y [M, N] from the same tile, with
 * gate [M, N] the gate projection's output.  gate, y and h are 16-byte aligned, N % 8 == 0.
 * Only where mxs_nf4_linear_glu_fused(M, N, K, 0) is 1 (else MXS_ERR_SIZE). */
int mxs_nf4_linear_fwd_glu(const void* x, int M, int K, int N, const void* packed,
                           const void* absmax8, const float* code, const float* absmax2,
                           const float* offset, const void* bias, const float* lora_hp,
                           int hp_slices, int ldt, const void* lora_b, int r, void* lora_ht,
                           const void* gate, void* y, void* h, void* workspace,
                           hipStream_t stream);

/* The down projection's input gradient followed by the SwiGLU backward
 * (SiluMulInPlace.backward, solution/silu_mul.py:65-71): mxs_nf4_linear_bwd_dx_hp whose
 * output d(hidden) [M, K] is not stored; instead gate and up [M, K] (the forward's saved
 * tensors) are overwritten with d(gate) and d(up), as the reference's in-place backward does.
 * lora_dhp may be NULL (no LoRA term).  Only where mxs_nf4_linear_glu_fused(M, N, K, 1) is 1. */
int mxs_nf4_linear_bwd_dx_glu(const void* dy, int M, int N, int K, const void* packed,
                              const void* absmax8, const float* code, const float* absmax2,
                              const float* offset, const float* lora_dhp, int hp_slices, int ldt,
                              const void* lora_at, int r, const void* mask, float mask_scale,
                              void* lora_dht, void* gate, void* up, void* workspace,
                              hipStream_t stream);

/* q, k, v of Qwen2 attention with the rotary position embedding (solution/attention.py:28-82,
 * qkv_rope_kernel; with no LoRA term and no v it is solution/rope.py:41-66, rope_kernel).
 * tensors[8] = q_a, q_b, k, v_a, v_b (inputs), q_o, k_o, v_o (outputs); each a [B, H, T, 128]
 * view with unit stride along the head and (b, h, t) element strides in strides[3 * i ..],
 * e.g. a projection's [B, T, H * 128] output has (T * H * 128, 128, H * 128).  Forward:
 * x = a (+ b * scale) in fp32, q and k rotated (y1 = x1 c1 - x2 s1, y2 = x2 c2 + x1 s2 over
 * the halves x1 = x[0:64], x2 = x[64:128] and the cos / sin row of the position), v only
 * added; backward (backward = 1) rotates by the opposite angle (dq, dk; dv copied).  cos / sin:
 * fp32 rows of 128 with strides (cos_stride_b, cos_stride_t); cos_stride_b may be 0.  q_b, v_b
 * may be NULL; v_a and v_o NULL together (no v heads).  Inputs all fp16 (in_f32 = 0) or all
 * fp32; outputs fp16 or fp32 (out_f32).  Pointers 16-byte aligned, strides multiples of
 * 16 bytes (8 fp16 or 4 fp32 elements); cos / sin strides multiples of 4. */
int mxs_qkv_rope(const void* const tensors[8], const int64_t strides[24], const float* cos,
                 const float* sin, int64_t cos_stride_b, int64_t cos_stride_t, int batch,
                 int n_tokens, int n_q, int n_kv, int in_f32, int out_f32, int backward,
                 float q_scale, float v_scale, hipStream_t stream);

/* 1 when the projection [K -> N] at M tokens takes the SwiGLU epilogue in the forward (bwd = 0)
 * or the backward (bwd = 1) on its planned kernel; else 0 (then run the GEMM and
 * mxs_silu_mul / mxs_silu_mul_bwd). */
int mxs_nf4_linear_glu_fused(int M, int N, int K, int bwd);

/* dst[cols, rows] = src[rows, cols]^T, fp16 (lora_A -> the [K, r] operand of the backward). */
int mxs_transpose_f16(const void* src, int rows, int cols, void* dst, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MXS_NF4_H */
