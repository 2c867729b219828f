// PyTorch operator library over the C ABI of libmxs_nf4.so (include/mxs_nf4.h).
//
// The host side of the NF4 + LoRA projection in C++: shape, dtype and device checks, output
// allocation from torch's caching allocator, the launch sequence on the current HIP stream, and
// the autograd nodes, so that one Python call makes a whole projection's forward and the
// autograd engine runs its backward without re-entering Python.  The ops are registered as
// torch.ops.mxs_nf4.* (TORCH_LIBRARY); the package loads this library with
// torch.ops.load_library.
//
// Device ops (HIP kernels; a Meta kernel gives fake-tensor shapes):
//   dequant           unpack_nf4 (solution/nf4.py:138-155)
//   linear_fwd        NF4LinearFunction.forward on the fused GEMM (solution/linear4bit.py:47-49)
//   linear_bwd_dx     NF4LinearFunction.backward (solution/linear4bit.py:51-57)
//   lora_fwd          base(x) + s * B(A(drop(x))) of peft's LoRA layer around the 4-bit base
//                     (solution/attention.py:193-201): LoRA row products, then the fused GEMM
//   lora_bwd          its dX, dA, dB (solution/dropout.py:62-69 for the dropout's gradient)
//   lora_fwd_group    lora_fwd for 1..4 projections reading one input (q/k/v; gate/up)
//   lora_bwd_group    lora_bwd for them, small launches shared
// Autograd ops (one node per call; backward in C++), named as the package's Python Functions
// they stand for (a node's name() says which ran):
//   linear         NF4LinearFunction
//   lora_linear    NF4LoraFunction
//   lora_siblings  NF4LoraSiblingsFunction
//
// Every result is produced by the same kernels, in the same order, as the package's Python
// path over ctypes, so the two give the same bits.

#include <ATen/ATen.h>
#include <ATen/DeviceGuard.h>
#include <c10/core/impl/LocalDispatchKeySet.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/library.h>

#include <array>
#include <optional>
#include <tuple>
#include <vector>

#include "mxs_nf4.h"

namespace {

using at::Tensor;
using at::TensorList;
using OptTensor = std::optional<Tensor>;
using OptTensorList = c10::List<std::optional<Tensor>>;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

constexpr int kMaxGroup = 4;

const char* why(int rc) {
  switch (rc) {
    case MXS_ERR_ARG: return "bad argument (null pointer or negative size)";
    case MXS_ERR_DTYPE: return "unsupported dtype";
    case MXS_ERR_ALIGN: return "pointer alignment";
    case MXS_ERR_SIZE: return "shape outside what the kernels take";
    default: return "HIP runtime error";
  }
}

void ok(int rc, const char* name) {
  TORCH_CHECK(rc == MXS_OK, name, " failed: ", why(rc), " (", rc, ")");
}

hipStream_t stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

int64_t ldt_of(int64_t M) { return (M + 7) / 8 * 8; }

template <class T = void>
T* ptr(const Tensor& t) {
  return t.defined() ? static_cast<T*>(t.data_ptr()) : nullptr;
}

int as_int(int64_t v, const char* what) {
  TORCH_CHECK(v >= 0 && v < (int64_t(1) << 31), what, " = ", v, " is outside the kernels' range");
  return static_cast<int>(v);
}

// t contiguous and 16-byte aligned (the kernels' vector loads need it; a view at an odd offset
// is copied).
Tensor aligned(const Tensor& t) {
  Tensor c = t.contiguous();
  return reinterpret_cast<uintptr_t>(c.data_ptr()) % 16 ? c.clone() : c;
}

// An activation-like operand: fp16 [rows, cols] on `dev`, contiguous and aligned.
Tensor half2d(const Tensor& t, int64_t rows, int64_t cols, const at::Device& dev,
              const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kHalf && t.dim() == 2 && t.size(1) == cols &&
                  (rows < 0 || t.size(0) == rows),
              name, " must be fp16 [", rows < 0 ? std::string("M") : std::to_string(rows), ", ",
              cols, "], got ", t.scalar_type(), " ", t.sizes());
  TORCH_CHECK(t.device() == dev, name, " must be on ", dev, ", found ", t.device());
  return aligned(t);
}

// A LoRA weight in fp16 [rows, cols] (converted from its own dtype).
Tensor lora16(const Tensor& t, int64_t rows, int64_t cols, const at::Device& dev,
              const char* name) {
  TORCH_CHECK(t.dim() == 2 && t.size(0) == rows && t.size(1) == cols, name, " must be [", rows,
              ", ", cols, "], got ", t.sizes());
  TORCH_CHECK(t.device() == dev, name, " must be on ", dev, ", found ", t.device());
  TORCH_CHECK(at::isFloatingType(t.scalar_type()), name, " must be floating point");
  return aligned(t.to(at::kHalf));
}

// The dropout keep mask as the kernels take it: keep bits, int32 [M, ceil(K/32)] (bit k % 32 of
// word k / 32 of row m set where (m, k) is kept).  A byte mask [M, K] (uint8, int8 or bool,
// nonzero = kept: the reference's int8 `keep`) is packed by one launch; bits pass through.
Tensor keep_mask(const OptTensor& keep, int64_t M, int64_t K, const at::Device& dev) {
  if (!keep.has_value() || !keep->defined()) return Tensor();
  const Tensor& k = *keep;
  TORCH_CHECK(k.device() == dev, "keep must be on ", dev);
  const int64_t kw = (K + 31) / 32;
  if (k.scalar_type() == at::kInt && k.dim() == 2 && k.size(0) == M && k.size(1) == kw)
    return k.contiguous();
  const auto t = k.scalar_type();
  TORCH_CHECK((t == at::kByte || t == at::kChar || t == at::kBool) && k.dim() == 2 &&
                  k.size(0) == M && k.size(1) == K,
              "keep must be a uint8 [", M, ", ", K, "] dropout mask or int32 [", M, ", ", kw,
              "] keep bits, got ", t, " ", k.sizes());
  const Tensor src = k.contiguous();
  Tensor bits = at::empty({M, kw}, src.options().dtype(at::kInt));
  if (src.is_meta()) return bits;  // fake tensors: the shape only
  ok(mxs_keep_pack(src.data_ptr(), as_int(M, "M"), as_int(K, "K"), bits.data_ptr(),
                   stream_of(src)),
     "mxs_keep_pack");
  return bits;
}

// keep_mask over the rows of x (a node packs once in its forward and saves the bits).
OptTensor keep_bits_for(const OptTensor& keep, const Tensor& x2) {
  const Tensor b = keep_mask(keep, x2.size(0), x2.size(1), x2.device());
  return b.defined() ? OptTensor(b) : std::nullopt;
}

Tensor bias16(const OptTensor& bias, int64_t N, const at::Device& dev) {
  if (!bias.has_value() || !bias->defined()) return Tensor();
  const Tensor& b = *bias;
  TORCH_CHECK(b.numel() == N, "bias must hold ", N, " values");
  TORCH_CHECK(b.device() == dev, "bias must be on ", dev);
  return b.to(at::kHalf).contiguous().view({N});
}

Tensor workspace(int64_t bytes, const Tensor& like) {
  if (bytes <= 0) return Tensor();
  return at::empty({bytes}, like.options().dtype(at::kByte));
}

// The NF4 operands the GEMMs read through raw pointers, checked against the weight shape
// [N, K]: packed u8 [N*K/2], absmax8 u8 [N*K/64], code fp32 [256], absmax2 fp32
// [ceil(N*K/64/256)], offset fp32, all contiguous on `dev`; N and K multiples of 64.
struct Nf4 {
  const void* packed;
  const void* absmax8;
  const float* code;
  const float* absmax2;
  const float* offset;
};

Nf4 nf4_operands(const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                 const Tensor& absmax2, const Tensor& offset, int64_t N, int64_t K,
                 const at::Device& dev) {
  TORCH_CHECK(N > 0 && K > 0 && N % 64 == 0 && K % 64 == 0,
              "the fused kernels take weights [N, K] with N and K multiples of 64, got [", N,
              ", ", K, "]");
  const int64_t blocks = N * K / 64;
  TORCH_CHECK(packed.scalar_type() == at::kByte && packed.is_contiguous() &&
                  2 * packed.numel() == N * K,
              "packed must be contiguous uint8 with ", N * K / 2, " bytes for [", N, ", ", K,
              "]");
  TORCH_CHECK(absmax8.scalar_type() == at::kByte && absmax8.is_contiguous() &&
                  absmax8.numel() == blocks,
              "absmax must be contiguous uint8 [", blocks, "]");
  TORCH_CHECK(absmax2.scalar_type() == at::kFloat && absmax2.is_contiguous() &&
                  absmax2.numel() == (blocks + 255) / 256,
              "state2.absmax must be contiguous fp32 [", (blocks + 255) / 256, "]");
  TORCH_CHECK(code.scalar_type() == at::kFloat && code.is_contiguous() && code.numel() == 256,
              "state2.code must be contiguous fp32 [256]");
  TORCH_CHECK(offset.scalar_type() == at::kFloat && offset.numel() >= 1,
              "offset must be an fp32 tensor");
  for (const Tensor* t : {&packed, &absmax8, &code, &absmax2, &offset})
    TORCH_CHECK(t->device() == dev, "NF4 operands must be on ", dev, ", found ", t->device());
  return {packed.data_ptr(), absmax8.data_ptr(), code.data_ptr<float>(),
          absmax2.data_ptr<float>(), offset.data_ptr<float>()};
}

// ---- dequant ---------------------------------------------------------------------------------

Tensor dequant_cuda(const Tensor& packed, const OptTensor& absmax8, const OptTensor& code,
                    const OptTensor& absmax2, const OptTensor& offset,
                    const OptTensor& absmax_f32, at::IntArrayRef shape, at::ScalarType dtype) {
  TORCH_CHECK(packed.is_cuda() && packed.scalar_type() == at::kByte && packed.is_contiguous(),
              "packed must be contiguous uint8 on the GPU");
  TORCH_CHECK(dtype == at::kHalf || dtype == at::kFloat, "dequant writes fp16 or fp32, not ",
              dtype);
  const at::OptionalDeviceGuard guard(at::device_of(packed));
  const at::Device dev = packed.device();
  const int64_t n_bytes = packed.numel();
  Tensor out = at::empty(shape, packed.options().dtype(dtype));
  TORCH_CHECK(out.numel() == 2 * n_bytes, "shape ", shape, " does not hold ", 2 * n_bytes,
              " values");
  const bool nested = absmax8.has_value() && absmax8->defined();
  const int64_t blocks = (n_bytes + 31) / 32;  // a trailing partial block has its own scale
  Tensor a8, cb, a2, off, af;
  if (nested) {
    TORCH_CHECK(code.has_value() && absmax2.has_value() && offset.has_value(),
                "nested absmax needs code, absmax2 and offset");
    a8 = absmax8->contiguous();
    cb = code->contiguous();
    a2 = absmax2->contiguous();
    off = offset->contiguous();
    TORCH_CHECK(a8.scalar_type() == at::kByte && a8.numel() >= blocks,
                "absmax must be uint8 with at least ", blocks, " entries");
    TORCH_CHECK(cb.scalar_type() == at::kFloat && cb.numel() == 256, "code must be fp32 [256]");
    TORCH_CHECK(a2.scalar_type() == at::kFloat && a2.numel() >= (blocks + 255) / 256,
                "absmax2 must be fp32 with at least ", (blocks + 255) / 256, " entries");
    TORCH_CHECK(off.scalar_type() == at::kFloat && off.numel() >= 1, "offset must be fp32");
    for (const Tensor* t : {&a8, &cb, &a2, &off})
      TORCH_CHECK(t->device() == dev, "NF4 operands must be on ", dev);
  } else {
    TORCH_CHECK(absmax_f32.has_value() && absmax_f32->defined(),
                "give absmax8/code/absmax2/offset or absmax_f32");
    af = absmax_f32->to(at::kFloat).contiguous();
    TORCH_CHECK(af.numel() >= blocks && af.device() == dev, "absmax must be fp32 with at least ",
                blocks, " entries on ", dev);
  }
  ok(mxs_nf4_dequant(packed.data_ptr(), n_bytes, ptr(a8), ptr<float>(cb), ptr<float>(a2),
                     ptr<float>(off), ptr<float>(af), out.data_ptr(),
                     dtype == at::kHalf ? MXS_DTYPE_F16 : MXS_DTYPE_F32, stream_of(packed)),
     "mxs_nf4_dequant");
  return out;
}

Tensor dequant_meta(const Tensor& packed, const OptTensor&, const OptTensor&, const OptTensor&,
                    const OptTensor&, const OptTensor&, at::IntArrayRef shape,
                    at::ScalarType dtype) {
  return at::empty(shape, packed.options().dtype(dtype));
}

// ---- base projection (no LoRA) -----------------------------------------------------------------

Tensor linear_fwd_cuda(const Tensor& x, const Tensor& packed, const Tensor& absmax8,
                       const Tensor& code, const Tensor& absmax2, const Tensor& offset,
                       int64_t out_features, const OptTensor& bias) {
  TORCH_CHECK(x.is_cuda(), "x must be on the GPU");
  const at::OptionalDeviceGuard guard(at::device_of(x));
  const at::Device dev = x.device();
  const int64_t N = out_features;
  TORCH_CHECK(x.dim() == 2, "x must be fp16 [M, in_features]");
  const int64_t K = x.size(1);
  const Tensor xc = half2d(x, -1, K, dev, "x");
  const int64_t M = xc.size(0);
  const Nf4 w = nf4_operands(packed, absmax8, code, absmax2, offset, N, K, dev);
  const Tensor b16 = bias16(bias, N, dev);
  Tensor y = at::empty({M, N}, xc.options());
  const int m = as_int(M, "M"), k = as_int(K, "K"), n = as_int(N, "N");
  const Tensor ws = workspace(mxs_nf4_gemm_workspace_bytes(m, n, k, -1, 1), xc);
  ok(mxs_nf4_linear_fwd(xc.data_ptr(), m, k, n, w.packed, w.absmax8, w.code, w.absmax2, w.offset,
                        ptr(b16), nullptr, nullptr, 0, y.data_ptr(), ptr(ws), -1, 1,
                        stream_of(xc)),
     "mxs_nf4_linear_fwd");
  return y;
}

Tensor linear_fwd_meta(const Tensor& x, const Tensor&, const Tensor&, const Tensor&,
                       const Tensor&, const Tensor&, int64_t out_features, const OptTensor&) {
  return at::empty({x.size(0), out_features}, x.options());
}

Tensor linear_bwd_dx_cuda(const Tensor& dy, const Tensor& packed, const Tensor& absmax8,
                          const Tensor& code, const Tensor& absmax2, const Tensor& offset,
                          int64_t in_features) {
  TORCH_CHECK(dy.is_cuda(), "dy must be on the GPU");
  const at::OptionalDeviceGuard guard(at::device_of(dy));
  const at::Device dev = dy.device();
  TORCH_CHECK(dy.dim() == 2, "dy must be fp16 [M, out_features]");
  const int64_t N = dy.size(1), K = in_features;
  const Tensor d = half2d(dy, -1, N, dev, "dy");
  const int64_t M = d.size(0);
  const Nf4 w = nf4_operands(packed, absmax8, code, absmax2, offset, N, K, dev);
  Tensor dx = at::empty({M, K}, d.options());
  const int m = as_int(M, "M"), k = as_int(K, "K"), n = as_int(N, "N");
  const Tensor ws = workspace(mxs_nf4_gemm_workspace_bytes(m, k, n, -1, 1), d);
  ok(mxs_nf4_linear_bwd_dx(d.data_ptr(), m, n, k, w.packed, w.absmax8, w.code, w.absmax2,
                           w.offset, nullptr, nullptr, 0, nullptr, 1.0f, dx.data_ptr(), ptr(ws),
                           -1, 1, stream_of(d)),
     "mxs_nf4_linear_bwd_dx");
  return dx;
}

Tensor linear_bwd_dx_meta(const Tensor& dy, const Tensor&, const Tensor&, const Tensor&,
                          const Tensor&, const Tensor&, int64_t in_features) {
  return at::empty({dy.size(0), in_features}, dy.options());
}

// ---- NF4 + LoRA projections: forward -------------------------------------------------------------

using Lists4 = std::tuple<std::vector<Tensor>, std::vector<Tensor>, std::vector<Tensor>,
                          std::vector<Tensor>>;

void check_group(size_t n, std::initializer_list<size_t> sizes) {
  TORCH_CHECK(n >= 1 && n <= kMaxGroup, "1..", kMaxGroup, " projections per group, got ", n);
  for (size_t s : sizes) TORCH_CHECK(s == n, "every per-projection list must have ", n, " entries");
}

OptTensor entry(const OptTensorList& l, size_t i) {
  if (l.size() == 0) return std::nullopt;
  std::optional<Tensor> v = l.get(i);
  return v;
}

std::vector<OptTensor> entries(const OptTensorList& l, size_t n) {
  std::vector<OptTensor> v(n);
  for (size_t i = 0; i < n && i < l.size(); ++i) v[i] = l.get(i);
  return v;
}

// A LoRA weight as the rows kernel reads it: fp32 [rows, cols] as is (w32), else fp16.
Tensor lora_w(const Tensor& t, int64_t rows, int64_t cols, const at::Device& dev,
              const char* name, bool w32) {
  if (!w32) return lora16(t, rows, cols, dev, name);
  TORCH_CHECK(t.dim() == 2 && t.size(0) == rows && t.size(1) == cols, name, " must be [", rows,
              ", ", cols, "], got ", t.sizes());
  TORCH_CHECK(t.device() == dev, name, " must be on ", dev, ", found ", t.device());
  return aligned(t);
}

// Forward of n (1..4) NF4 + LoRA projections reading x: Hs = s * drop(x) A^T of each as fp32
// slice partials, with lora_A^T, lora_B^T (the backward's operands) and, for fp32 LoRA weights,
// their fp16 B as side outputs, in one launch (mxs_lora_h_partials_group, or its _w32 form when
// every LoRA weight is fp32: no cast launches); then either one grouped GEMM launch (one_gemm:
// 128x128 tiles, mxs_nf4_linear_fwd_hp_group) or each projection's own planned GEMM
// (mxs_nf4_linear_fwd_hp), which finish Hs and compute Y = x W^T + bias + Hs B^T and write
// Hs^T.  Returns (ys, hts, ats, bts).  For one projection this is lora_fwd: the grouped rows
// launch of one problem gives the bits of mxs_lora_h_partials.
// The RoPE the grouped forward may fold into its first n_rope outputs (attention's q / k):
// cos / sin fp32 [1 or B, T, 128], one layout, unit last stride; x's rows B sequences of T.
struct RopeOperands {
  const float* cos = nullptr;
  const float* sin = nullptr;
  int64_t cs_b = 0, cs_t = 0;
  int T = 0, n_rope = 0;
};

RopeOperands rope_operands(const OptTensor& cos, const OptTensor& sin, int64_t n_rope,
                           int64_t M, size_t n, const at::Device& dev) {
  RopeOperands r;
  if (n_rope == 0) {
    TORCH_CHECK(!cos.has_value() && !sin.has_value(), "cos / sin given without n_rope");
    return r;
  }
  TORCH_CHECK(n_rope > 0 && n_rope <= (int64_t)n, "n_rope: 1 .. the number of projections");
  TORCH_CHECK(cos.has_value() && sin.has_value(), "n_rope needs cos and sin");
  const Tensor& c = *cos;
  const Tensor& sn = *sin;
  TORCH_CHECK(c.device() == dev && sn.device() == dev && c.scalar_type() == at::kFloat &&
                  sn.scalar_type() == at::kFloat && c.dim() == 3 && c.sizes() == sn.sizes() &&
                  c.strides() == sn.strides() && c.size(2) == 128 && c.stride(2) == 1,
              "cos / sin must be fp32 [1 or B, T, 128] with one layout on x's device");
  const int64_t T = c.size(1);
  TORCH_CHECK(T >= 1 && M % T == 0 && (c.size(0) == 1 || c.size(0) == M / T),
              "x's rows must be B whole sequences of cos / sin's T tokens");
  r.cos = c.data_ptr<float>();
  r.sin = sn.data_ptr<float>();
  r.cs_b = c.size(0) > 1 ? c.stride(0) : 0;
  r.cs_t = c.stride(1);
  r.T = as_int(T, "T");
  r.n_rope = static_cast<int>(n_rope);
  return r;
}

Lists4 fwd_impl(const Tensor& x, TensorList lora_a, TensorList lora_b, TensorList packed,
                TensorList absmax8, TensorList code, TensorList absmax2, TensorList offset,
                const std::vector<OptTensor>& bias, const std::vector<OptTensor>& keep,
                double mask_scale, double s, bool one_gemm, const OptTensor& cos = std::nullopt,
                const OptTensor& sin = std::nullopt, int64_t n_rope = 0) {
  const size_t n = lora_a.size();
  check_group(n, {lora_b.size(), packed.size(), absmax8.size(), code.size(), absmax2.size(),
                  offset.size(), bias.size(), keep.size()});
  TORCH_CHECK(x.is_cuda() && x.dim() == 2, "x must be fp16 [M, K] on the GPU");
  const at::OptionalDeviceGuard guard(at::device_of(x));
  const at::Device dev = x.device();
  const int64_t K = x.size(1);
  const Tensor xc = half2d(x, -1, K, dev, "x");
  const int64_t M = xc.size(0);
  TORCH_CHECK(lora_a[0].dim() == 2, "lora_a must be [r, K]");
  const int64_t r = lora_a[0].size(0);
  const int m = as_int(M, "M"), k = as_int(K, "K"), rr = as_int(r, "r");
  const int64_t ldt = ldt_of(M);
  const auto f16 = xc.options();
  const int S = mxs_lora_slices(m, k);
  bool w32 = true;
  for (size_t i = 0; i < n; ++i)
    w32 = w32 && lora_a[i].scalar_type() == at::kFloat && lora_b[i].scalar_type() == at::kFloat;
  std::vector<Tensor> aw(n), bw(n), b16(n), masks(n), biases(n), hps(n), ats(n), bts(n), ys(n),
      hts(n);
  std::array<Nf4, kMaxGroup> w{};
  std::array<int, kMaxGroup> Ns{}, Ks{};
  std::array<const void*, kMaxGroup> xs{}, pa{}, pb{}, pm{}, pbias{}, p_packed{}, p_a8{};
  std::array<const float*, kMaxGroup> p_code{}, p_a2{}, p_off{}, p_hp{};
  std::array<const void*, kMaxGroup> pbw{};
  std::array<void*, kMaxGroup> p_at{}, p_bt{}, p_b16{}, p_ht{}, p_y{};
  std::array<float*, kMaxGroup> p_hpw{};
  for (size_t i = 0; i < n; ++i) {
    TORCH_CHECK(lora_b[i].dim() == 2, "lora_b must be [N, r]");
    const int64_t N = lora_b[i].size(0);
    aw[i] = lora_w(lora_a[i], r, K, dev, "lora_a", w32);
    bw[i] = lora_w(lora_b[i], N, r, dev, "lora_b", w32);
    b16[i] = w32 ? at::empty({N, r}, f16) : bw[i];
    w[i] = nf4_operands(packed[i], absmax8[i], code[i], absmax2[i], offset[i], N, K, dev);
    masks[i] = keep_mask(keep[i], M, K, dev);
    biases[i] = bias16(bias[i], N, dev);
    hps[i] = at::empty({S, ldt, r}, f16.dtype(at::kFloat));
    ats[i] = at::empty({K, r}, f16);
    bts[i] = at::empty({r, N}, f16);
    Ns[i] = as_int(N, "N");
    Ks[i] = k;
    xs[i] = xc.data_ptr();
    pa[i] = aw[i].data_ptr();
    pb[i] = b16[i].data_ptr();
    pbw[i] = bw[i].data_ptr();
    pm[i] = ptr(masks[i]);
    pbias[i] = ptr(biases[i]);
    p_packed[i] = w[i].packed;
    p_a8[i] = w[i].absmax8;
    p_code[i] = w[i].code;
    p_a2[i] = w[i].absmax2;
    p_off[i] = w[i].offset;
    p_hpw[i] = hps[i].data_ptr<float>();
    p_hp[i] = p_hpw[i];
    p_at[i] = ats[i].data_ptr();
    p_bt[i] = bts[i].data_ptr();
    p_b16[i] = b16[i].data_ptr();
  }
  const RopeOperands rope = rope_operands(cos, sin, n_rope, M, n, dev);
  TORCH_CHECK(rope.n_rope == 0 || one_gemm, "the RoPE rides on the grouped GEMM (one_gemm)");
  const hipStream_t st = stream_of(xc);
  const float ms = static_cast<float>(mask_scale), sf = static_cast<float>(s);
  if (w32) {
    std::array<const float*, kMaxGroup> pa32{}, pb32{};
    for (size_t i = 0; i < n; ++i) {
      pa32[i] = static_cast<const float*>(pa[i]);
      pb32[i] = static_cast<const float*>(pbw[i]);
    }
    ok(mxs_lora_h_partials_group_w32((int)n, xs.data(), m, Ks.data(), pa32.data(), rr,
                                     pm.data(), ms, sf, (int)ldt, p_at.data(), pb32.data(),
                                     Ns.data(), p_bt.data(), p_b16.data(), p_hpw.data(), st),
       "mxs_lora_h_partials_group_w32");
  } else {
    ok(mxs_lora_h_partials_group((int)n, xs.data(), m, Ks.data(), pa.data(), rr, pm.data(), ms,
                                 sf, (int)ldt, p_at.data(), pb.data(), Ns.data(), p_bt.data(),
                                 p_hpw.data(), st),
       "mxs_lora_h_partials_group");
  }
  for (size_t i = 0; i < n; ++i) {
    ys[i] = at::empty({M, Ns[i]}, f16);
    hts[i] = at::empty({r, ldt}, f16);
    p_y[i] = ys[i].data_ptr();
    p_ht[i] = hts[i].data_ptr();
  }
  if (one_gemm && rope.n_rope > 0) {
    ok(mxs_nf4_linear_fwd_hp_group_rope(
           (int)n, xs.data(), m, k, Ns.data(), p_packed.data(), p_a8.data(), p_code.data(),
           p_a2.data(), p_off.data(), pbias.data(), p_hp.data(), S, (int)ldt, pb.data(), rr,
           p_ht.data(), p_y.data(), rope.n_rope, rope.cos, rope.sin, rope.cs_b, rope.cs_t,
           rope.T, st),
       "mxs_nf4_linear_fwd_hp_group_rope");
  } else if (one_gemm) {
    ok(mxs_nf4_linear_fwd_hp_group((int)n, xs.data(), m, k, Ns.data(), p_packed.data(),
                                   p_a8.data(), p_code.data(), p_a2.data(), p_off.data(),
                                   pbias.data(), p_hp.data(), S, (int)ldt, pb.data(), rr,
                                   p_ht.data(), p_y.data(), st),
       "mxs_nf4_linear_fwd_hp_group");
  } else if (n == 2 && mxs_nf4_linear_fwd_pair_ok(m, Ns[0], Ns[1], k)) {
    // gate and up: one launch, grid z selects the projection (the bits of two launches)
    ok(mxs_nf4_linear_fwd_hp_pair(xc.data_ptr(), m, k, Ns.data(), p_packed.data(), p_a8.data(),
                                  p_code.data(), p_a2.data(), p_off.data(), pbias.data(),
                                  p_hp.data(), S, (int)ldt, pb.data(), rr, p_ht.data(),
                                  p_y.data(), st),
       "mxs_nf4_linear_fwd_hp_pair");
  } else {
    int64_t need = 0;
    for (size_t i = 0; i < n; ++i)
      need = std::max(need, mxs_nf4_gemm_workspace_bytes(m, Ns[i], k, -1, 1));
    const Tensor ws = workspace(need, xc);  // reused: the GEMMs run in stream order
    for (size_t i = 0; i < n; ++i)
      ok(mxs_nf4_linear_fwd_hp(xc.data_ptr(), m, k, Ns[i], w[i].packed, w[i].absmax8, w[i].code,
                               w[i].absmax2, w[i].offset, pbias[i], p_hp[i], S, (int)ldt, pb[i],
                               rr, p_ht[i], p_y[i], ptr(ws), -1, 1, st),
         "mxs_nf4_linear_fwd_hp");
  }
  return {ys, hts, ats, bts};
}

Lists4 lora_fwd_group_cuda(const Tensor& x, TensorList lora_a, TensorList lora_b,
                           TensorList packed, TensorList absmax8, TensorList code,
                           TensorList absmax2, TensorList offset, const OptTensorList& bias,
                           const OptTensorList& keep, double mask_scale, double s,
                           bool one_gemm, const OptTensor& cos, const OptTensor& sin,
                           int64_t n_rope) {
  const size_t n = lora_a.size();
  TORCH_CHECK(bias.size() == 0 || bias.size() == n, "bias: none or one per projection");
  TORCH_CHECK(keep.size() == 0 || keep.size() == n, "keep: none or one per projection");
  return fwd_impl(x, lora_a, lora_b, packed, absmax8, code, absmax2, offset, entries(bias, n),
                  entries(keep, n), mask_scale, s, one_gemm, cos, sin, n_rope);
}

// One projection (NF4LoraFunction.forward): fwd_impl of one.  Returns (y, ht, at, bt).
std::tuple<Tensor, Tensor, Tensor, Tensor> lora_fwd_cuda(
    const Tensor& x, const Tensor& lora_a, const Tensor& lora_b, const Tensor& packed,
    const Tensor& absmax8, const Tensor& code, const Tensor& absmax2, const Tensor& offset,
    const OptTensor& bias, const OptTensor& keep, double mask_scale, double s) {
  auto [ys, hts, ats, bts] = fwd_impl(x, lora_a, lora_b, packed, absmax8, code, absmax2, offset,
                                      {bias}, {keep}, mask_scale, s, false);
  return {ys[0], hts[0], ats[0], bts[0]};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> lora_fwd_meta(
    const Tensor& x, const Tensor& lora_a, const Tensor& lora_b, const Tensor&, const Tensor&,
    const Tensor&, const Tensor&, const Tensor&, const OptTensor&, const OptTensor&, double,
    double) {
  const int64_t M = x.size(0), K = x.size(1), r = lora_a.size(0), N = lora_b.size(0);
  const auto o = x.options().dtype(at::kHalf);
  return {at::empty({M, N}, o), at::empty({r, ldt_of(M)}, o), at::empty({K, r}, o),
          at::empty({r, N}, o)};
}

// How the backward takes dHs = s * dY B for one projection: finished in one launch, for the dX
// GEMM that also computes dA and dB (where the library says that fits the GPU in one launch),
// else as slice partials that the dX GEMM finishes.
bool dh_finished(int M, int N, int K, int r, bool want_x, bool want_a, bool want_b) {
  return want_x && want_a && want_b && mxs_nf4_linear_bwd_grads_fused(M, N, K, r) != 0;
}

struct BwdOperands {  // one projection's backward inputs, checked
  Tensor dy, x, mask, ht, at, bt;
  Nf4 w;
  int M, N, K, r, ldt;
};

BwdOperands bwd_operands(const Tensor& dy, const Tensor& x, const OptTensor& keep,
                         const Tensor& ht, const Tensor& at_, const Tensor& bt,
                         const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                         const Tensor& absmax2, const Tensor& offset, const at::Device& dev) {
  TORCH_CHECK(dy.dim() == 2 && x.dim() == 2 && bt.dim() == 2, "dy [M, N], x [M, K], bt [r, N]");
  BwdOperands o;
  const int64_t M = x.size(0), K = x.size(1), N = dy.size(1), r = bt.size(0);
  o.x = half2d(x, -1, K, dev, "x");
  o.dy = half2d(dy, M, N, dev, "dy");
  o.bt = half2d(bt, r, N, dev, "bt");
  o.at = half2d(at_, K, r, dev, "at");
  const int64_t ldt = ldt_of(M);
  o.ht = half2d(ht, r, ldt, dev, "ht");
  o.mask = keep_mask(keep, M, K, dev);
  o.w = nf4_operands(packed, absmax8, code, absmax2, offset, N, K, dev);
  o.M = as_int(M, "M");
  o.N = as_int(N, "N");
  o.K = as_int(K, "K");
  o.r = as_int(r, "r");
  o.ldt = static_cast<int>(ldt);
  return o;
}

// dX through the fused dX GEMM from dHs partials (writing dHs^T when gradients follow), then dA
// and dB in one launch: the "partials" route of one projection.
void bwd_partials(const BwdOperands& o, const Tensor& dhp, float mask_scale, bool want_x,
                  bool want_a, bool want_b, Tensor& dx, Tensor& da, Tensor& db,
                  const Tensor& ws, hipStream_t st) {
  const bool want_g = want_a || want_b;
  const auto f16 = o.x.options();
  Tensor dht;
  if (want_x || want_g) {
    dx = at::empty({o.M, o.K}, f16);
    if (want_g) dht = at::empty({o.r, o.ldt}, f16);
    ok(mxs_nf4_linear_bwd_dx_hp(o.dy.data_ptr(), o.M, o.N, o.K, o.w.packed, o.w.absmax8,
                                o.w.code, o.w.absmax2, o.w.offset, dhp.data_ptr<float>(),
                                (int)dhp.size(0), o.ldt, o.at.data_ptr(), o.r, ptr(o.mask),
                                mask_scale, ptr(dht), dx.data_ptr(), ptr(ws), -1, 1, st),
       "mxs_nf4_linear_bwd_dx_hp");
  }
  if (!want_x) dx = Tensor();
  if (want_g) {
    if (want_a) da = at::empty({o.r, o.K}, f16.dtype(at::kFloat));
    if (want_b) db = at::empty({o.N, o.r}, f16.dtype(at::kFloat));
    ok(mxs_lora_grads(dht.data_ptr(), o.ht.data_ptr(), o.ldt, o.x.data_ptr(), o.dy.data_ptr(),
                      o.M, o.K, o.N, o.r, ptr(o.mask), mask_scale, ptr<float>(da),
                      ptr<float>(db), nullptr, st),
       "mxs_lora_grads");
  }
}

// The whole backward of one projection after dHs finished in one launch: dX with dA and dB.
void bwd_finished(const BwdOperands& o, const Tensor& dh, const Tensor& dht, float mask_scale,
                  Tensor& dx, Tensor& da, Tensor& db, const Tensor& ws, hipStream_t st) {
  const auto f16 = o.x.options();
  dx = at::empty({o.M, o.K}, f16);
  da = at::empty({o.r, o.K}, f16.dtype(at::kFloat));
  db = at::empty({o.N, o.r}, f16.dtype(at::kFloat));
  ok(mxs_nf4_linear_bwd_dx_grads(o.dy.data_ptr(), o.M, o.N, o.K, o.w.packed, o.w.absmax8,
                                 o.w.code, o.w.absmax2, o.w.offset, dh.data_ptr(),
                                 o.at.data_ptr(), o.r, ptr(o.mask), mask_scale, dht.data_ptr(),
                                 o.ht.data_ptr(), o.ldt, o.x.data_ptr(), da.data_ptr<float>(),
                                 db.data_ptr<float>(), dx.data_ptr(), ptr(ws), st),
     "mxs_nf4_linear_bwd_dx_grads");
}

Tensor gemm_ws_bwd(const BwdOperands& o) {
  return workspace(mxs_nf4_gemm_workspace_bytes(o.M, o.K, o.N, -1, 1), o.x);
}

// Backward of one projection: (dx, dA, dB), undefined where not wanted.  Where the dX GEMM can
// carry the weight gradients (all three wanted, dh_finished): dHs finished in one launch, then
// one launch for all three.  Otherwise dHs as partials, the dX GEMM, then dA / dB.
std::tuple<Tensor, Tensor, Tensor> lora_bwd_cuda(
    const Tensor& dy, const Tensor& x, const OptTensor& keep, const Tensor& ht, const Tensor& at_,
    const Tensor& bt, const Tensor& packed, const Tensor& absmax8, const Tensor& code,
    const Tensor& absmax2, const Tensor& offset, double mask_scale, double s, bool want_x,
    bool want_a, bool want_b) {
  TORCH_CHECK(dy.is_cuda(), "dy must be on the GPU");
  const at::OptionalDeviceGuard guard(at::device_of(dy));
  const BwdOperands o = bwd_operands(dy, x, keep, ht, at_, bt, packed, absmax8, code, absmax2,
                                     offset, dy.device());
  const hipStream_t st = stream_of(o.dy);
  const auto f16 = o.x.options();
  const float ms = static_cast<float>(mask_scale), sf = static_cast<float>(s);
  Tensor dx, da, db;
  if (dh_finished(o.M, o.N, o.K, o.r, want_x, want_a, want_b)) {
    Tensor dh = at::empty({o.M, o.r}, f16), dht = at::empty({o.r, o.ldt}, f16);
    ok(mxs_lora_dh(o.dy.data_ptr(), o.M, o.N, o.bt.data_ptr(), o.r, sf, dh.data_ptr(),
                   dht.data_ptr(), o.ldt, nullptr, st),
       "mxs_lora_dh");
    bwd_finished(o, dh, dht, ms, dx, da, db, gemm_ws_bwd(o), st);
    return {dx, da, db};
  }
  if (!(want_x || want_a || want_b)) return {dx, da, db};
  Tensor dhp = at::empty({mxs_lora_slices(o.M, o.N), o.ldt, o.r}, f16.dtype(at::kFloat));
  ok(mxs_lora_dh_partials(o.dy.data_ptr(), o.M, o.N, o.bt.data_ptr(), o.r, sf, o.ldt,
                          dhp.data_ptr<float>(), st),
     "mxs_lora_dh_partials");
  bwd_partials(o, dhp, ms, want_x, want_a, want_b, dx, da, db, gemm_ws_bwd(o), st);
  return {dx, da, db};
}

std::tuple<Tensor, Tensor, Tensor> lora_bwd_meta(
    const Tensor& dy, const Tensor& x, const OptTensor&, const Tensor&, const Tensor&,
    const Tensor& bt, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
    double, double, bool want_x, bool want_a, bool want_b) {
  const int64_t M = x.size(0), K = x.size(1), N = dy.size(1), r = bt.size(0);
  const auto o = x.options();
  return {want_x ? at::empty({M, K}, o.dtype(at::kHalf)) : Tensor(),
          want_a ? at::empty({r, K}, o.dtype(at::kFloat)) : Tensor(),
          want_b ? at::empty({N, r}, o.dtype(at::kFloat)) : Tensor()};
}

// ---- 1..4 projections over one input: shapes, backward ------------------------------------------

Lists4 lora_fwd_group_meta(const Tensor& x, TensorList lora_a, TensorList lora_b, TensorList,
                           TensorList, TensorList, TensorList, TensorList, const OptTensorList&,
                           const OptTensorList&, double, double, bool, const OptTensor&,
                           const OptTensor&, int64_t) {
  const int64_t M = x.size(0), K = x.size(1);
  const auto o = x.options().dtype(at::kHalf);
  std::vector<Tensor> ys, hts, ats, bts;
  for (size_t i = 0; i < lora_a.size(); ++i) {
    const int64_t r = lora_a[i].size(0), N = lora_b[i].size(0);
    ys.push_back(at::empty({M, N}, o));
    hts.push_back(at::empty({r, ldt_of(M)}, o));
    ats.push_back(at::empty({K, r}, o));
    bts.push_back(at::empty({r, N}, o));
  }
  return {ys, hts, ats, bts};
}

using Lists3 = std::tuple<std::vector<Tensor>, std::vector<Tensor>, std::vector<Tensor>>;

// Backward of n projections reading x whose output gradients arrive together, small launches
// shared: dHs in one launch per route (finished / partials); the dX GEMMs that carry their
// weight gradients in one launch where mxs_nf4_linear_bwd_dx_grads_group_ok allows, else each;
// the others' dX GEMMs, then their dA / dB in one launch when all are wanted and the shapes are
// equal.  wants: 3 per projection (dx, dA, dB).  Returns (dxs, das, dbs), undefined where not
// wanted; the bits of lora_bwd on each.  sum_dx: dxs[0] is the sum of the projections' input
// gradients (added in order; the others undefined), and two projections that
// mxs_nf4_linear_bwd_dx_hp_pair takes (gate and up) get it from that one summed launch.
Lists3 lora_bwd_group_cuda(TensorList dy, const Tensor& x, const OptTensorList& keep,
                           TensorList ht, TensorList at_, TensorList bt, TensorList packed,
                           TensorList absmax8, TensorList code, TensorList absmax2,
                           TensorList offset, double mask_scale, double s,
                           at::IntArrayRef wants, bool sum_dx) {
  const size_t n = dy.size();
  check_group(n, {ht.size(), at_.size(), bt.size(), packed.size(), absmax8.size(), code.size(),
                  absmax2.size(), offset.size()});
  TORCH_CHECK(keep.size() == 0 || keep.size() == n, "keep: none or one per projection");
  TORCH_CHECK(wants.size() == 3 * n, "wants: 3 flags per projection");
  TORCH_CHECK(x.is_cuda(), "x must be on the GPU");
  const at::OptionalDeviceGuard guard(at::device_of(x));
  const at::Device dev = x.device();
  std::vector<BwdOperands> o;
  o.reserve(n);
  for (size_t i = 0; i < n; ++i)
    o.push_back(bwd_operands(dy[i], x, entry(keep, i), ht[i], at_[i], bt[i], packed[i],
                             absmax8[i], code[i], absmax2[i], offset[i], dev));
  const int M = o[0].M, K = o[0].K, r = o[0].r, ldt = o[0].ldt;
  for (size_t i = 1; i < n; ++i) TORCH_CHECK(o[i].r == r, "one LoRA rank per group");
  const hipStream_t st = stream_of(o[0].x);
  const auto f16 = o[0].x.options();
  const float ms = static_cast<float>(mask_scale), sf = static_cast<float>(s);
  auto want = [&](size_t i, int j) { return wants[3 * i + j] != 0; };

  std::vector<Tensor> dxs(n), das(n), dbs(n), dh(n), dht(n), dhp(n);
  // Summed (q, k and v over one input): every flag set, one keep-mask presence, and a plan the
  // summed launch takes: dHs finished for all in one launch, then ONE launch for the summed dX
  // and every dA / dB (the sum rounded once, not each part and then added).
  if (sum_dx && n >= 2 && n <= 3) {
    bool all = true;
    std::array<int, kMaxGroup> Ns{};
    for (size_t i = 0; i < n; ++i) {
      all = all && want(i, 0) && want(i, 1) && want(i, 2) &&
            o[i].mask.defined() == o[0].mask.defined();
      Ns[i] = o[i].N;
    }
    if (all && mxs_nf4_linear_bwd_dx_grads_sum_ok((int)n, M, Ns.data(), K, r, 0)) {
      // with the gradients in the same launch up to 1152 tokens; past that the summed dX alone,
      // then dA / dB in one launch per weight height (k and v share one)
      const bool fused = mxs_nf4_linear_bwd_dx_grads_sum_ok((int)n, M, Ns.data(), K, r, 1) != 0;
      std::array<const void*, kMaxGroup> pdy{}, pbt{}, pk{}, pa8{}, pdhc{}, pat{}, pm{}, pdhtc{},
          pht{};
      std::array<void*, kMaxGroup> pdh{}, pdht{};
      std::array<const float*, kMaxGroup> pc{}, pa2{}, po{};
      std::array<float*, kMaxGroup> pda{}, pdb{};
      for (size_t i = 0; i < n; ++i) {
        const BwdOperands& q = o[i];
        dh[i] = at::empty({M, r}, f16);
        dht[i] = at::empty({r, ldt}, f16);
        das[i] = at::empty({r, K}, f16.dtype(at::kFloat));
        dbs[i] = at::empty({q.N, r}, f16.dtype(at::kFloat));
        pdy[i] = q.dy.data_ptr();
        pbt[i] = q.bt.data_ptr();
        pdh[i] = dh[i].data_ptr();
        pdht[i] = dht[i].data_ptr();
        pdhc[i] = pdh[i];
        pdhtc[i] = pdht[i];
        pk[i] = q.w.packed;
        pa8[i] = q.w.absmax8;
        pc[i] = q.w.code;
        pa2[i] = q.w.absmax2;
        po[i] = q.w.offset;
        pat[i] = q.at.data_ptr();
        pm[i] = ptr(q.mask);
        pht[i] = q.ht.data_ptr();
        pda[i] = das[i].data_ptr<float>();
        pdb[i] = dbs[i].data_ptr<float>();
      }
      ok(mxs_lora_dh_group((int)n, pdy.data(), M, Ns.data(), pbt.data(), r, sf, ldt, pdh.data(),
                           pdht.data(), st),
         "mxs_lora_dh_group");
      dxs[0] = at::empty({M, K}, f16);
      ok(mxs_nf4_linear_bwd_dx_grads_sum((int)n, pdy.data(), M, Ns.data(), K, pk.data(),
                                         pa8.data(), pc.data(), pa2.data(), po.data(),
                                         pdhc.data(), pat.data(), r, pm.data(), ms, pdhtc.data(),
                                         pht.data(), ldt, o[0].x.data_ptr(),
                                         fused ? pda.data() : nullptr,
                                         fused ? pdb.data() : nullptr, dxs[0].data_ptr(), st),
         "mxs_nf4_linear_bwd_dx_grads_sum");
      if (!fused) {
        std::vector<bool> done(n, false);
        for (size_t i = 0; i < n; ++i) {
          if (done[i]) continue;
          std::array<const void*, kMaxGroup> gdht{}, ght{}, gx{}, gdy{}, gm{};
          std::array<int, kMaxGroup> gK{}, gN{};
          std::array<float*, kMaxGroup> gda{}, gdb{};
          int cnt = 0;
          for (size_t j = i; j < n; ++j) {
            if (done[j] || o[j].N != o[i].N) continue;
            done[j] = true;
            gdht[cnt] = dht[j].data_ptr();
            ght[cnt] = o[j].ht.data_ptr();
            gx[cnt] = o[j].x.data_ptr();
            gdy[cnt] = o[j].dy.data_ptr();
            gm[cnt] = ptr(o[j].mask);
            gK[cnt] = K;
            gN[cnt] = o[j].N;
            gda[cnt] = das[j].data_ptr<float>();
            gdb[cnt] = dbs[j].data_ptr<float>();
            ++cnt;
          }
          if (cnt > 1)
            ok(mxs_lora_grads_group(cnt, gdht.data(), ght.data(), ldt, gx.data(), gdy.data(), M,
                                    gK.data(), gN.data(), r, gm.data(), ms, gda.data(),
                                    gdb.data(), st),
               "mxs_lora_grads_group");
          else
            ok(mxs_lora_grads(gdht[0], ght[0], ldt, gx[0], gdy[0], M, K, gN[0], r, gm[0], ms,
                              gda[0], gdb[0], nullptr, st),
               "mxs_lora_grads");
        }
      }
      return {dxs, das, dbs};
    }
  }
  std::vector<size_t> fin, par;
  for (size_t i = 0; i < n; ++i) {
    if (dh_finished(M, o[i].N, K, r, want(i, 0), want(i, 1), want(i, 2)))
      fin.push_back(i);
    else if (want(i, 0) || want(i, 1) || want(i, 2))
      par.push_back(i);
  }
  // dHs: one launch per route
  if (!fin.empty()) {
    std::array<const void*, kMaxGroup> pdy{}, pbt{};
    std::array<void*, kMaxGroup> pdh{}, pdht{};
    std::array<int, kMaxGroup> Ns{};
    for (size_t j = 0; j < fin.size(); ++j) {
      const size_t i = fin[j];
      dh[i] = at::empty({M, r}, f16);
      dht[i] = at::empty({r, ldt}, f16);
      pdy[j] = o[i].dy.data_ptr();
      pbt[j] = o[i].bt.data_ptr();
      pdh[j] = dh[i].data_ptr();
      pdht[j] = dht[i].data_ptr();
      Ns[j] = o[i].N;
    }
    ok(mxs_lora_dh_group((int)fin.size(), pdy.data(), M, Ns.data(), pbt.data(), r, sf, ldt,
                         pdh.data(), pdht.data(), st),
       "mxs_lora_dh_group");
  }
  if (!par.empty()) {
    std::array<const void*, kMaxGroup> pdy{}, pbt{};
    std::array<float*, kMaxGroup> pp{};
    std::array<int, kMaxGroup> Ns{};
    for (size_t j = 0; j < par.size(); ++j) {
      const size_t i = par[j];
      dhp[i] = at::empty({mxs_lora_slices(M, o[i].N), ldt, r}, f16.dtype(at::kFloat));
      pdy[j] = o[i].dy.data_ptr();
      pbt[j] = o[i].bt.data_ptr();
      pp[j] = dhp[i].data_ptr<float>();
      Ns[j] = o[i].N;
    }
    ok(mxs_lora_dh_partials_group((int)par.size(), pdy.data(), M, Ns.data(), pbt.data(), r, sf,
                                  ldt, pp.data(), st),
       "mxs_lora_dh_partials_group");
  }
  int64_t need = 0;
  for (size_t i = 0; i < n; ++i)
    need = std::max(need, mxs_nf4_gemm_workspace_bytes(M, K, o[i].N, -1, 1));
  const Tensor ws = workspace(need, o[0].x);  // reused: the GEMMs run in stream order

  // the "finished" projections: dX with dA / dB, grouped where the library takes the group
  bool grouped = false;
  if (fin.size() > 1) {
    std::array<int, kMaxGroup> Ns{};
    for (size_t j = 0; j < fin.size(); ++j) Ns[j] = o[fin[j]].N;
    if (mxs_nf4_linear_bwd_dx_grads_group_ok((int)fin.size(), M, Ns.data(), K, r)) {
      std::array<const void*, kMaxGroup> pdy{}, pk{}, pa8{}, pdh{}, pat{}, pm{}, pdht{}, pht{},
          px{};
      std::array<const float*, kMaxGroup> pc{}, pa2{}, po{};
      std::array<float*, kMaxGroup> pda{}, pdb{};
      std::array<void*, kMaxGroup> pdx{};
      for (size_t j = 0; j < fin.size(); ++j) {
        const size_t i = fin[j];
        const BwdOperands& q = o[i];
        dxs[i] = at::empty({M, K}, f16);
        das[i] = at::empty({r, K}, f16.dtype(at::kFloat));
        dbs[i] = at::empty({q.N, r}, f16.dtype(at::kFloat));
        pdy[j] = q.dy.data_ptr();
        pk[j] = q.w.packed;
        pa8[j] = q.w.absmax8;
        pc[j] = q.w.code;
        pa2[j] = q.w.absmax2;
        po[j] = q.w.offset;
        pdh[j] = dh[i].data_ptr();
        pat[j] = q.at.data_ptr();
        pm[j] = ptr(q.mask);
        pdht[j] = dht[i].data_ptr();
        pht[j] = q.ht.data_ptr();
        px[j] = q.x.data_ptr();
        pda[j] = das[i].data_ptr<float>();
        pdb[j] = dbs[i].data_ptr<float>();
        pdx[j] = dxs[i].data_ptr();
      }
      ok(mxs_nf4_linear_bwd_dx_grads_group((int)fin.size(), pdy.data(), M, Ns.data(), K,
                                           pk.data(), pa8.data(), pc.data(), pa2.data(),
                                           po.data(), pdh.data(), pat.data(), r, pm.data(), ms,
                                           pdht.data(), pht.data(), ldt, px.data(), pda.data(),
                                           pdb.data(), pdx.data(), st),
         "mxs_nf4_linear_bwd_dx_grads_group");
      grouped = true;
    }
  }
  if (!grouped)
    for (size_t i : fin) bwd_finished(o[i], dh[i], dht[i], ms, dxs[i], das[i], dbs[i], ws, st);

  // the "partials" projections: each dX GEMM (or, summed, both in one launch), then the weight
  // gradients
  std::vector<size_t> both;
  std::vector<Tensor> pend_dht(n);
  const bool pair = sum_dx && n == 2 && fin.empty() && par.size() == 2 && want(0, 0) &&
                    want(1, 0) && dhp[0].size(0) == dhp[1].size(0) &&
                    mxs_nf4_linear_bwd_dx_pair_ok(M, o[0].N, o[1].N, K) != 0;
  bool pair_grads = false;  // the pair's launches computed both projections' dA and dB
  if (pair) {
    const bool wt = want(0, 1) || want(0, 2) || want(1, 1) || want(1, 2);
    std::array<const void*, 2> pdy{}, pk{}, pa8{}, pat{}, pm{};
    std::array<const float*, 2> pc{}, pa2{}, po{}, php{};
    std::array<void*, 2> pdht{};
    std::array<int, 2> Ns{};
    for (size_t i = 0; i < 2; ++i) {
      if (wt) pend_dht[i] = at::empty({r, ldt}, f16);
      pdy[i] = o[i].dy.data_ptr();
      pk[i] = o[i].w.packed;
      pa8[i] = o[i].w.absmax8;
      pc[i] = o[i].w.code;
      pa2[i] = o[i].w.absmax2;
      po[i] = o[i].w.offset;
      php[i] = dhp[i].data_ptr<float>();
      pat[i] = o[i].at.data_ptr();
      pm[i] = ptr(o[i].mask);
      pdht[i] = ptr(pend_dht[i]);
      Ns[i] = o[i].N;
      if (want(i, 1) && want(i, 2)) both.push_back(i);
    }
    dxs[0] = at::empty({M, K}, f16);
    const Tensor pws =
        workspace(mxs_nf4_linear_bwd_dx_pair_workspace_bytes(M, Ns[0], Ns[1], K), o[0].x);
    if (both.size() == 2 && Ns[0] == Ns[1]) {
      // every weight gradient wanted: the pair's reduce and the gradients in one launch
      std::array<const void*, 2> pht{};
      std::array<float*, 2> pda{}, pdb{};
      for (size_t i = 0; i < 2; ++i) {
        das[i] = at::empty({r, K}, f16.dtype(at::kFloat));
        dbs[i] = at::empty({o[i].N, r}, f16.dtype(at::kFloat));
        pht[i] = o[i].ht.data_ptr();
        pda[i] = das[i].data_ptr<float>();
        pdb[i] = dbs[i].data_ptr<float>();
      }
      ok(mxs_nf4_linear_bwd_dx_hp_pair_grads(
             pdy.data(), M, Ns.data(), K, pk.data(), pa8.data(), pc.data(), pa2.data(),
             po.data(), php.data(), (int)dhp[0].size(0), ldt, pat.data(), r, pm.data(), ms,
             pdht.data(), pht.data(), o[0].x.data_ptr(), pda.data(), pdb.data(),
             dxs[0].data_ptr(), ptr(pws), st),
         "mxs_nf4_linear_bwd_dx_hp_pair_grads");
      both.clear();
      pair_grads = true;
    } else {
      ok(mxs_nf4_linear_bwd_dx_hp_pair(pdy.data(), M, Ns.data(), K, pk.data(), pa8.data(),
                                       pc.data(), pa2.data(), po.data(), php.data(),
                                       (int)dhp[0].size(0), ldt, pat.data(), r, pm.data(), ms,
                                       pdht.data(), dxs[0].data_ptr(), ptr(pws), st),
         "mxs_nf4_linear_bwd_dx_hp_pair");
    }
  }
  for (size_t i : par) {
    if (pair) break;
    const bool wa = want(i, 1), wb = want(i, 2), wg = wa || wb;
    dxs[i] = at::empty({M, K}, f16);
    if (wg) pend_dht[i] = at::empty({r, ldt}, f16);
    ok(mxs_nf4_linear_bwd_dx_hp(o[i].dy.data_ptr(), M, o[i].N, K, o[i].w.packed,
                                o[i].w.absmax8, o[i].w.code, o[i].w.absmax2, o[i].w.offset,
                                dhp[i].data_ptr<float>(), (int)dhp[i].size(0), ldt,
                                o[i].at.data_ptr(), r, ptr(o[i].mask), ms, ptr(pend_dht[i]),
                                dxs[i].data_ptr(), ptr(ws), -1, 1, st),
       "mxs_nf4_linear_bwd_dx_hp");
    if (!want(i, 0)) dxs[i] = Tensor();
    if (wa && wb) both.push_back(i);
  }
  bool same = both.size() > 1;
  for (size_t i : both) same = same && o[i].N == o[both[0]].N;
  if (same) {
    std::array<const void*, kMaxGroup> pdht{}, pht{}, px{}, pdy{}, pm{};
    std::array<int, kMaxGroup> Ks{}, Ns{};
    std::array<float*, kMaxGroup> pda{}, pdb{};
    for (size_t j = 0; j < both.size(); ++j) {
      const size_t i = both[j];
      das[i] = at::empty({r, K}, f16.dtype(at::kFloat));
      dbs[i] = at::empty({o[i].N, r}, f16.dtype(at::kFloat));
      pdht[j] = pend_dht[i].data_ptr();
      pht[j] = o[i].ht.data_ptr();
      px[j] = o[i].x.data_ptr();
      pdy[j] = o[i].dy.data_ptr();
      pm[j] = ptr(o[i].mask);
      Ks[j] = K;
      Ns[j] = o[i].N;
      pda[j] = das[i].data_ptr<float>();
      pdb[j] = dbs[i].data_ptr<float>();
    }
    ok(mxs_lora_grads_group((int)both.size(), pdht.data(), pht.data(), ldt, px.data(),
                            pdy.data(), M, Ks.data(), Ns.data(), r, pm.data(), ms, pda.data(),
                            pdb.data(), st),
       "mxs_lora_grads_group");
  }
  for (size_t i : par) {
    const bool wa = want(i, 1), wb = want(i, 2);
    if (!(wa || wb) || (same && wa && wb) || pair_grads) continue;
    if (wa) das[i] = at::empty({r, K}, f16.dtype(at::kFloat));
    if (wb) dbs[i] = at::empty({o[i].N, r}, f16.dtype(at::kFloat));
    ok(mxs_lora_grads(pend_dht[i].data_ptr(), o[i].ht.data_ptr(), ldt, o[i].x.data_ptr(),
                      o[i].dy.data_ptr(), M, K, o[i].N, r, ptr(o[i].mask), ms, ptr<float>(das[i]),
                      ptr<float>(dbs[i]), nullptr, st),
       "mxs_lora_grads");
  }
  if (sum_dx && !pair) {  // in order, as autograd would add them
    Tensor sum;
    for (size_t i = 0; i < n; ++i) {
      if (!dxs[i].defined()) continue;
      sum = sum.defined() ? sum.add_(dxs[i]) : dxs[i];
      dxs[i] = Tensor();
    }
    dxs[0] = sum;
  }
  return {dxs, das, dbs};
}

Lists3 lora_bwd_group_meta(TensorList dy, const Tensor& x, const OptTensorList&, TensorList,
                           TensorList, TensorList bt, TensorList, TensorList, TensorList,
                           TensorList, TensorList, double, double, at::IntArrayRef wants,
                           bool sum_dx) {
  const int64_t M = x.size(0), K = x.size(1);
  std::vector<Tensor> dxs, das, dbs;
  bool any_x = false;
  for (size_t i = 0; i < dy.size(); ++i) any_x = any_x || wants[3 * i];
  for (size_t i = 0; i < dy.size(); ++i) {
    const int64_t N = dy[i].size(1), r = bt[i].size(0);
    const bool wx = sum_dx ? (i == 0 && any_x) : wants[3 * i] != 0;
    dxs.push_back(wx ? at::empty({M, K}, x.options().dtype(at::kHalf)) : Tensor());
    das.push_back(wants[3 * i + 1] ? at::empty({r, K}, x.options().dtype(at::kFloat))
                                   : Tensor());
    dbs.push_back(wants[3 * i + 2] ? at::empty({N, r}, x.options().dtype(at::kFloat))
                                   : Tensor());
  }
  return {dxs, das, dbs};
}

// ---- autograd ----------------------------------------------------------------------------------
// The autograd ops reach the device ops through the dispatcher below the autograd keys, so that
// a fake-tensor or meta call takes their Meta kernels.

template <class Sig>
c10::TypedOperatorHandle<Sig> op(const char* name) {
  return c10::Dispatcher::singleton().findSchemaOrThrow(name, "").template typed<Sig>();
}

Tensor rows2d(const Tensor& t) { return t.reshape({-1, t.size(-1)}); }

std::vector<int64_t> out_shape(const Tensor& x, int64_t n) {
  std::vector<int64_t> s(x.sizes().begin(), x.sizes().end());
  s.back() = n;
  return s;
}

Tensor as_dtype(const Tensor& g, at::ScalarType t) {
  return g.defined() && g.scalar_type() != t ? g.to(t) : g;
}

// NF4LinearFunction (solution/linear4bit.py:43-57): Y = x W^T + bias; grad_x = grad W; no
// gradient for the frozen weight or bias.
struct NF4LinearFunction : public torch::autograd::Function<NF4LinearFunction> {
  static Tensor forward(AutogradContext* ctx, const Tensor& x, const Tensor& packed,
                        const Tensor& absmax8, const Tensor& code, const Tensor& absmax2,
                        const Tensor& offset, int64_t out_features, const OptTensor& bias) {
    static auto fwd = op<Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                const Tensor&, const Tensor&, int64_t, const OptTensor&)>(
        "mxs_nf4::linear_fwd");
    at::AutoDispatchBelowADInplaceOrView below;
    ctx->save_for_backward({packed, absmax8, code, absmax2, offset});
    ctx->saved_data["k"] = x.size(-1);
    Tensor y = fwd.call(rows2d(x), packed, absmax8, code, absmax2, offset, out_features, bias);
    return y.view(out_shape(x, out_features));
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    static auto bwd = op<Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                const Tensor&, const Tensor&, int64_t)>("mxs_nf4::linear_bwd_dx");
    const auto saved = ctx->get_saved_variables();
    const int64_t K = ctx->saved_data["k"].toInt();
    Tensor dx;
    if (ctx->needs_input_grad(0)) {
      at::AutoDispatchBelowADInplaceOrView below;
      const Tensor& g = grads[0];
      const Tensor g2 = rows2d(g.to(at::kHalf));
      dx = bwd.call(g2, saved[0], saved[1], saved[2], saved[3], saved[4], K)
               .view(out_shape(g, K));
    }
    return {dx, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Tensor linear_autograd(const Tensor& x, const Tensor& packed, const Tensor& absmax8,
                       const Tensor& code, const Tensor& absmax2, const Tensor& offset,
                       int64_t out_features, const OptTensor& bias) {
  return NF4LinearFunction::apply(x, packed, absmax8, code, absmax2, offset, out_features, bias);
}

using LoraFwdSig = std::tuple<Tensor, Tensor, Tensor, Tensor>(
    const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
    const Tensor&, const Tensor&, const OptTensor&, const OptTensor&, double, double);
using LoraBwdSig = std::tuple<Tensor, Tensor, Tensor>(
    const Tensor&, const Tensor&, const OptTensor&, const Tensor&, const Tensor&, const Tensor&,
    const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, double, double,
    bool, bool, bool);

// One NF4 + LoRA projection, y = base(x) + s * B(A(drop(x))) (NF4LoraFunction of the Python
// package).  x fp16 [..., K]; lora_a [r, K], lora_b [N, r] in any float dtype (their gradients
// come back in it); keep u8 [M, K] (M = rows of x), keep bits int32 [M, ceil(K/32)] or None;
// mask_scale = 1/(1-p).
struct NF4LoraFunction : public torch::autograd::Function<NF4LoraFunction> {
  static Tensor forward(AutogradContext* ctx, const Tensor& x, const Tensor& lora_a,
                        const Tensor& lora_b, const Tensor& packed, const Tensor& absmax8,
                        const Tensor& code, const Tensor& absmax2, const Tensor& offset,
                        const OptTensor& bias, const OptTensor& keep, double mask_scale,
                        double s) {
    static auto fwd = op<LoraFwdSig>("mxs_nf4::lora_fwd");
    at::AutoDispatchBelowADInplaceOrView below;
    const Tensor x2 = rows2d(x).contiguous();
    const OptTensor kb = keep_bits_for(keep, x2);
    auto [y, ht, at_, bt] =
        fwd.call(x2, lora_a, lora_b, packed, absmax8, code, absmax2, offset, bias, kb,
                 mask_scale, s);
    ctx->save_for_backward({x2, kb.value_or(Tensor()), ht, at_, bt, packed, absmax8, code,
                            absmax2, offset});
    ctx->saved_data["mask_scale"] = mask_scale;
    ctx->saved_data["s"] = s;
    ctx->saved_data["a_dtype"] = lora_a.scalar_type();
    ctx->saved_data["b_dtype"] = lora_b.scalar_type();
    ctx->saved_data["x_shape"] = x.sizes().vec();
    return y.view(out_shape(x, y.size(1)));
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    static auto bwd = op<LoraBwdSig>("mxs_nf4::lora_bwd");
    const auto v = ctx->get_saved_variables();
    const bool wx = ctx->needs_input_grad(0), wa = ctx->needs_input_grad(1),
               wb = ctx->needs_input_grad(2);
    Tensor dx, da, db;
    {
      at::AutoDispatchBelowADInplaceOrView below;
      const Tensor dy = rows2d(grads[0].to(at::kHalf));
      const OptTensor keep = v[1].defined() ? OptTensor(v[1]) : std::nullopt;
      std::tie(dx, da, db) = bwd.call(dy, v[0], keep, v[2], v[3], v[4], v[5], v[6], v[7], v[8],
                                      v[9], ctx->saved_data["mask_scale"].toDouble(),
                                      ctx->saved_data["s"].toDouble(), wx, wa, wb);
    }
    if (dx.defined()) dx = dx.view(ctx->saved_data["x_shape"].toIntVector());
    da = as_dtype(da, ctx->saved_data["a_dtype"].toScalarType());
    db = as_dtype(db, ctx->saved_data["b_dtype"].toScalarType());
    variable_list out(12);
    out[0] = dx;
    out[1] = da;
    out[2] = db;
    return out;
  }
};

Tensor lora_linear_autograd(const Tensor& x, const Tensor& lora_a, const Tensor& lora_b,
                            const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                            const Tensor& absmax2, const Tensor& offset, const OptTensor& bias,
                            const OptTensor& keep, double mask_scale, double s) {
  return NF4LoraFunction::apply(x, lora_a, lora_b, packed, absmax8, code, absmax2, offset, bias, keep,
                       mask_scale, s);
}

using GroupFwdSig = Lists4(const Tensor&, TensorList, TensorList, TensorList, TensorList,
                           TensorList, TensorList, TensorList, const OptTensorList&,
                           const OptTensorList&, double, double, bool, const OptTensor&,
                           const OptTensor&, int64_t);
using GroupBwdSig = Lists3(TensorList, const Tensor&, const OptTensorList&, TensorList,
                           TensorList, TensorList, TensorList, TensorList, TensorList,
                           TensorList, TensorList, double, double, at::IntArrayRef, bool);

// n NF4 + LoRA projections reading one input x fp16 [M, K] (a layer's q/k/v, or gate/up),
// their launches shared (NF4LoraSiblingsFunction of the Python package): outputs fp16 [M, N_i];
// the backward returns dx = the sum of the projections' input gradients, in order.
// With n_rope > 0 the first n_rope outputs come rotated (attention's q / k, the RoPE folded
// into the grouped GEMM) while the backward stays that of the unrotated projections: the
// caller applies the inverse rotation to their gradients first (rope.RotatedHeads).
struct NF4LoraSiblingsFunction : public torch::autograd::Function<NF4LoraSiblingsFunction> {
  static variable_list forward(AutogradContext* ctx, const Tensor& x, TensorList lora_a,
                               TensorList lora_b, TensorList packed, TensorList absmax8,
                               TensorList code, TensorList absmax2, TensorList offset,
                               const OptTensorList& bias, const OptTensorList& keep,
                               double mask_scale, double s, bool one_gemm,
                               const OptTensor& cos, const OptTensor& sin, int64_t n_rope) {
    static auto fwd = op<GroupFwdSig>("mxs_nf4::lora_fwd_group");
    at::AutoDispatchBelowADInplaceOrView below;
    const size_t n = lora_a.size();
    OptTensorList kbs;
    for (size_t i = 0; i < keep.size(); ++i) kbs.push_back(keep_bits_for(entry(keep, i), x));
    auto [ys, hts, ats, bts] = fwd.call(x, lora_a, lora_b, packed, absmax8, code, absmax2,
                                        offset, bias, kbs, mask_scale, s, one_gemm, cos, sin,
                                        n_rope);
    variable_list saved{x};
    for (const TensorList& l : {TensorList(hts), TensorList(ats), TensorList(bts), packed,
                                absmax8, code, absmax2, offset})
      saved.insert(saved.end(), l.begin(), l.end());
    for (size_t i = 0; i < n; ++i) {
      const OptTensor k = entry(kbs, i);
      saved.push_back(k.has_value() ? *k : Tensor());
    }
    ctx->save_for_backward(saved);
    ctx->saved_data["n"] = static_cast<int64_t>(n);
    ctx->saved_data["mask_scale"] = mask_scale;
    ctx->saved_data["s"] = s;
    std::vector<int64_t> ns, dts;
    for (size_t i = 0; i < n; ++i) {
      ns.push_back(lora_b[i].size(0));
      dts.push_back(static_cast<int64_t>(lora_a[i].scalar_type()));
      dts.push_back(static_cast<int64_t>(lora_b[i].scalar_type()));
    }
    ctx->saved_data["ns"] = ns;
    ctx->saved_data["dtypes"] = dts;
    return ys;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    static auto bwd = op<GroupBwdSig>("mxs_nf4::lora_bwd_group");
    const auto v = ctx->get_saved_variables();
    const int64_t n = ctx->saved_data["n"].toInt();
    const auto ns = ctx->saved_data["ns"].toIntVector();
    const auto dts = ctx->saved_data["dtypes"].toIntVector();
    const Tensor& x = v[0];
    auto slice = [&](int64_t j) {
      return std::vector<Tensor>(v.begin() + 1 + j * n, v.begin() + 1 + (j + 1) * n);
    };
    OptTensorList keep;
    for (int64_t i = 0; i < n; ++i) {
      const Tensor& k = v[1 + 8 * n + i];
      keep.push_back(k.defined() ? OptTensor(k) : std::nullopt);
    }
    std::vector<int64_t> wants;
    std::vector<Tensor> dys;
    for (int64_t i = 0; i < n; ++i) {
      wants.push_back(ctx->needs_input_grad(0));
      wants.push_back(ctx->needs_input_grad(1 + i));
      wants.push_back(ctx->needs_input_grad(1 + n + i));
      const Tensor& g = grads[i];
      dys.push_back(g.defined() ? g.to(at::kHalf).contiguous()
                                : at::zeros({x.size(0), ns[i]}, x.options()));
    }
    std::vector<Tensor> dxs, das, dbs;
    {
      at::AutoDispatchBelowADInplaceOrView below;
      std::tie(dxs, das, dbs) =
          bwd.call(dys, x, keep, slice(0), slice(1), slice(2), slice(3), slice(4), slice(5),
                   slice(6), slice(7), ctx->saved_data["mask_scale"].toDouble(),
                   ctx->saved_data["s"].toDouble(), wants, true);
    }
    variable_list out(7 * n + 9);
    if (ctx->needs_input_grad(0)) out[0] = dxs[0];
    for (int64_t i = 0; i < n; ++i) {
      out[1 + i] = as_dtype(das[i], static_cast<at::ScalarType>(dts[2 * i]));
      out[1 + n + i] = as_dtype(dbs[i], static_cast<at::ScalarType>(dts[2 * i + 1]));
    }
    return out;
  }
};

std::vector<Tensor> lora_siblings_autograd(const Tensor& x, TensorList lora_a,
                                           TensorList lora_b, TensorList packed,
                                           TensorList absmax8, TensorList code,
                                           TensorList absmax2, TensorList offset,
                                           const OptTensorList& bias, const OptTensorList& keep,
                                           double mask_scale, double s, bool one_gemm,
                                           const OptTensor& cos, const OptTensor& sin,
                                           int64_t n_rope) {
  return NF4LoraSiblingsFunction::apply(x, lora_a, lora_b, packed, absmax8, code, absmax2, offset, bias,
                           keep, mask_scale, s, one_gemm, cos, sin, n_rope);
}

// The autograd ops where no autograd key is dispatched (inference mode): the forward alone.
Tensor linear_plain(const Tensor& x, const Tensor& packed, const Tensor& absmax8,
                    const Tensor& code, const Tensor& absmax2, const Tensor& offset,
                    int64_t out_features, const OptTensor& bias) {
  static auto fwd = op<Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                              const Tensor&, const Tensor&, int64_t, const OptTensor&)>(
      "mxs_nf4::linear_fwd");
  return fwd.call(rows2d(x), packed, absmax8, code, absmax2, offset, out_features, bias)
      .view(out_shape(x, out_features));
}

Tensor lora_linear_plain(const Tensor& x, const Tensor& lora_a, const Tensor& lora_b,
                         const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                         const Tensor& absmax2, const Tensor& offset, const OptTensor& bias,
                         const OptTensor& keep, double mask_scale, double s) {
  static auto fwd = op<LoraFwdSig>("mxs_nf4::lora_fwd");
  const Tensor y = std::get<0>(fwd.call(rows2d(x).contiguous(), lora_a, lora_b, packed, absmax8,
                                        code, absmax2, offset, bias, keep, mask_scale, s));
  return y.view(out_shape(x, y.size(1)));
}

std::vector<Tensor> lora_siblings_plain(const Tensor& x, TensorList lora_a, TensorList lora_b,
                                        TensorList packed, TensorList absmax8, TensorList code,
                                        TensorList absmax2, TensorList offset,
                                        const OptTensorList& bias, const OptTensorList& keep,
                                        double mask_scale, double s, bool one_gemm,
                                        const OptTensor& cos, const OptTensor& sin,
                                        int64_t n_rope) {
  static auto fwd = op<GroupFwdSig>("mxs_nf4::lora_fwd_group");
  return std::get<0>(fwd.call(x, lora_a, lora_b, packed, absmax8, code, absmax2, offset, bias,
                              keep, mask_scale, s, one_gemm, cos, sin, n_rope));
}

}  // namespace

TORCH_LIBRARY(mxs_nf4, m) {
  m.def("dequant(Tensor packed, Tensor? absmax8, Tensor? code, Tensor? absmax2, Tensor? offset, "
        "Tensor? absmax_f32, int[] shape, ScalarType dtype) -> Tensor");
  m.def("linear_fwd(Tensor x, Tensor packed, Tensor absmax8, Tensor code, Tensor absmax2, "
        "Tensor offset, int out_features, Tensor? bias) -> Tensor");
  m.def("linear_bwd_dx(Tensor dy, Tensor packed, Tensor absmax8, Tensor code, Tensor absmax2, "
        "Tensor offset, int in_features) -> Tensor");
  m.def("lora_fwd(Tensor x, Tensor lora_a, Tensor lora_b, Tensor packed, Tensor absmax8, "
        "Tensor code, Tensor absmax2, Tensor offset, Tensor? bias, Tensor? keep, "
        "float mask_scale, float s) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("lora_bwd(Tensor dy, Tensor x, Tensor? keep, Tensor ht, Tensor at, Tensor bt, "
        "Tensor packed, Tensor absmax8, Tensor code, Tensor absmax2, Tensor offset, "
        "float mask_scale, float s, bool want_x, bool want_a, bool want_b) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("lora_fwd_group(Tensor x, Tensor[] lora_a, Tensor[] lora_b, Tensor[] packed, "
        "Tensor[] absmax8, Tensor[] code, Tensor[] absmax2, Tensor[] offset, Tensor?[] bias, "
        "Tensor?[] keep, float mask_scale, float s, bool one_gemm, Tensor? cos=None, "
        "Tensor? sin=None, int n_rope=0) -> (Tensor[], Tensor[], Tensor[], Tensor[])");
  m.def("lora_bwd_group(Tensor[] dy, Tensor x, Tensor?[] keep, Tensor[] ht, Tensor[] at, "
        "Tensor[] bt, Tensor[] packed, Tensor[] absmax8, Tensor[] code, Tensor[] absmax2, "
        "Tensor[] offset, float mask_scale, float s, int[] wants, bool sum_dx=False) "
        "-> (Tensor[], Tensor[], Tensor[])");
  m.def("linear(Tensor x, Tensor packed, Tensor absmax8, Tensor code, Tensor absmax2, "
        "Tensor offset, int out_features, Tensor? bias) -> Tensor");
  m.def("lora_linear(Tensor x, Tensor lora_a, Tensor lora_b, Tensor packed, Tensor absmax8, "
        "Tensor code, Tensor absmax2, Tensor offset, Tensor? bias, Tensor? keep, "
        "float mask_scale, float s) -> Tensor");
  m.def("lora_siblings(Tensor x, Tensor[] lora_a, Tensor[] lora_b, Tensor[] packed, "
        "Tensor[] absmax8, Tensor[] code, Tensor[] absmax2, Tensor[] offset, Tensor?[] bias, "
        "Tensor?[] keep, float mask_scale, float s, bool one_gemm, Tensor? cos=None, "
        "Tensor? sin=None, int n_rope=0) -> Tensor[]");
}

TORCH_LIBRARY_IMPL(mxs_nf4, CUDA, m) {
  m.impl("dequant", &dequant_cuda);
  m.impl("linear_fwd", &linear_fwd_cuda);
  m.impl("linear_bwd_dx", &linear_bwd_dx_cuda);
  m.impl("lora_fwd", &lora_fwd_cuda);
  m.impl("lora_bwd", &lora_bwd_cuda);
  m.impl("lora_fwd_group", &lora_fwd_group_cuda);
  m.impl("lora_bwd_group", &lora_bwd_group_cuda);
}

TORCH_LIBRARY_IMPL(mxs_nf4, Meta, m) {
  m.impl("dequant", &dequant_meta);
  m.impl("linear_fwd", &linear_fwd_meta);
  m.impl("linear_bwd_dx", &linear_bwd_dx_meta);
  m.impl("lora_fwd", &lora_fwd_meta);
  m.impl("lora_bwd", &lora_bwd_meta);
  m.impl("lora_fwd_group", &lora_fwd_group_meta);
  m.impl("lora_bwd_group", &lora_bwd_group_meta);
}

// The autograd ops: the same node with or without grad mode (without it, or with no input
// needing a gradient, apply() only runs the forward).
TORCH_LIBRARY_IMPL(mxs_nf4, Autograd, m) {
  m.impl("linear", &linear_autograd);
  m.impl("lora_linear", &lora_linear_autograd);
  m.impl("lora_siblings", &lora_siblings_autograd);
}

TORCH_LIBRARY_IMPL(mxs_nf4, CompositeExplicitAutograd, m) {
  m.impl("linear", &linear_plain);
  m.impl("lora_linear", &lora_linear_plain);
  m.impl("lora_siblings", &lora_siblings_plain);
}
