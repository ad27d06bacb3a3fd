// torch.ops.tq: the PyTorch-ROCm operator layer over the C ABI of libtq_amd.so
// (include/tq_api.h).  Each op checks its tensors, allocates its outputs with torch
// (the caching allocator, so calls are capturable into HIP graphs), and calls one
// C entry point on torch's current stream of the tensors' device.  No kernel code
// lives here: the HIP kernels are the C library's.
//
// Reference call sites these ops serve: compressors.py:99-317 (compress /
// asymmetric_attention_scores / decompress) and kernels/__init__.py:1-11 (pack_bits,
// unpack_bits, lloyd_max_quantize, lloyd_max_dequantize, asymmetric_attention_scores).
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <cstdint>
#include <tuple>

#include "tq_api.h"

namespace {

using at::Tensor;

void check_status(int st, const char* what) {
  TORCH_CHECK(st == TQ_OK, what, " failed (status ", st, "): ", tq_last_error());
}

void* stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void require_gpu(const Tensor& t, const char* what) {
  TORCH_CHECK(t.is_cuda(), what, ": expected a GPU tensor, got ", t.device());
}

int32_t dtype_code(at::ScalarType s) {
  switch (s) {
    case at::kFloat: return TQ_F32;
    case at::kHalf: return TQ_F16;
    case at::kBFloat16: return TQ_BF16;
    default: TORCH_CHECK(false, "unsupported activation dtype ", s, "; expected float32, float16 or bfloat16");
  }
  return -1;
}

// activations: float32 / float16 / bfloat16 with unit stride along the last dim
Tensor activation(const Tensor& x) {
  Tensor y = x;
  const auto s = y.scalar_type();
  if (s != at::kFloat && s != at::kHalf && s != at::kBFloat16) y = y.to(at::kFloat);
  if (y.stride(-1) != 1) y = y.contiguous();
  return y;
}

Tensor on(const Tensor& t, const Tensor& like, at::ScalarType s) {
  return t.to(like.device(), s).contiguous();
}

template <typename T>
T* ptr(const Tensor& t) {
  return reinterpret_cast<T*>(t.data_ptr());
}
template <typename T>
T* optr(const c10::optional<Tensor>& t) {
  return t.has_value() && t->defined() ? reinterpret_cast<T*>(t->data_ptr()) : nullptr;
}

int64_t out_cols(int64_t d, int64_t b) { return (d * b + 7) / 8; }

// ---------------------------------------------------------------- bit ops (kernels/bit_ops.py)
Tensor pack_bits(const Tensor& idx_in, int64_t b) {
  require_gpu(idx_in, "tq::pack_bits");
  TORCH_CHECK(idx_in.dim() == 2, "tq::pack_bits: expected [N, d] codes");
  const c10::DeviceGuard g(idx_in.device());
  Tensor idx = idx_in.to(at::kInt).contiguous();
  const int64_t n = idx.size(0), d = idx.size(1);
  Tensor out = at::empty({n, out_cols(d, b)}, idx.options().dtype(at::kByte));
  check_status(tq_pack_bits(ptr<int32_t>(idx), n, static_cast<int32_t>(d), d, static_cast<int32_t>(b),
                            ptr<uint8_t>(out), out.size(1), stream_of(out)),
               "tq::pack_bits");
  return out;
}

Tensor unpack_bits(const Tensor& packed_in, int64_t b, int64_t d) {
  require_gpu(packed_in, "tq::unpack_bits");
  TORCH_CHECK(packed_in.dim() == 2, "tq::unpack_bits: expected [N, bytes] packed rows");
  const c10::DeviceGuard g(packed_in.device());
  Tensor packed = packed_in.contiguous();
  const int64_t n = packed.size(0);
  Tensor out = at::empty({n, d}, packed.options().dtype(at::kInt));
  check_status(tq_unpack_bits(ptr<uint8_t>(packed), n, static_cast<int32_t>(d), packed.size(1),
                              static_cast<int32_t>(b), ptr<int32_t>(out), d, stream_of(out)),
               "tq::unpack_bits");
  return out;
}

// ---------------------------------------------------------------- quantize (kernels/quantize.py)
Tensor quantize_pack(const Tensor& y_in, const Tensor& bounds_in, int64_t b_eff) {
  require_gpu(y_in, "tq::quantize_pack");
  TORCH_CHECK(y_in.dim() == 2, "tq::quantize_pack: expected [N, d] rotated rows");
  const c10::DeviceGuard g(y_in.device());
  Tensor y = y_in.to(at::kFloat).contiguous();
  Tensor bounds = on(bounds_in, y, at::kFloat);
  const int64_t n = y.size(0), d = y.size(1);
  Tensor out = at::empty({n, out_cols(d, b_eff)}, y.options().dtype(at::kByte));
  check_status(tq_quantize_pack(ptr<float>(y), n, static_cast<int32_t>(d), d, ptr<float>(bounds),
                                static_cast<int32_t>(b_eff), ptr<uint8_t>(out), out.size(1), stream_of(out)),
               "tq::quantize_pack");
  return out;
}

Tensor dequantize(const Tensor& packed_in, const Tensor& cent_in, int64_t b, int64_t d) {
  require_gpu(packed_in, "tq::dequantize");
  const c10::DeviceGuard g(packed_in.device());
  Tensor packed = packed_in.contiguous();
  Tensor cent = on(cent_in, packed, at::kHalf);
  const int64_t n = packed.size(0);
  Tensor out = at::empty({n, d}, packed.options().dtype(at::kHalf));
  check_status(tq_dequantize(ptr<uint8_t>(packed), n, static_cast<int32_t>(d), packed.size(1), ptr<uint16_t>(cent),
                             static_cast<int32_t>(b), ptr<uint16_t>(out), d, stream_of(out)),
               "tq::dequantize");
  return out;
}

// ---------------------------------------------------------------- compressors (compressors.py)
std::tuple<Tensor, Tensor, Tensor, Tensor> compress_keys(const Tensor& states, const Tensor& pi_split,
                                                         const Tensor& seff_split,
                                                         const Tensor& centroids, const Tensor& bounds,
                                                         int64_t b_eff, const c10::optional<Tensor>& y_out,
                                                         const c10::optional<Tensor>& proj_out) {
  require_gpu(states, "tq::compress_keys");
  TORCH_CHECK(states.dim() == 4, "tq::compress_keys: expected [B, H, S, D] states");
  const c10::DeviceGuard g(states.device());
  Tensor x = activation(states);
  const int64_t B = x.size(0), H = x.size(1), S = x.size(2), D = x.size(3), n = B * H * S;
  auto u8 = x.options().dtype(at::kByte);
  Tensor codes = at::empty({n, out_cols(D, b_eff)}, u8);
  Tensor signs = at::empty({n, (D + 7) / 8}, u8);
  Tensor rn = at::empty({B, H, S}, x.options().dtype(at::kHalf));
  Tensor vn = at::empty({B, H, S}, x.options().dtype(at::kHalf));
  check_status(tq_compress_keys(x.data_ptr(), dtype_code(x.scalar_type()), static_cast<int32_t>(B),
                                static_cast<int32_t>(H), static_cast<int32_t>(S), static_cast<int32_t>(D),
                                x.stride(0), x.stride(1), x.stride(2), ptr<uint16_t>(pi_split),
                                ptr<uint16_t>(seff_split), ptr<float>(centroids),
                                ptr<float>(bounds), static_cast<int32_t>(b_eff), ptr<uint8_t>(codes),
                                ptr<uint8_t>(signs), ptr<uint16_t>(rn), ptr<uint16_t>(vn), optr<float>(y_out),
                                optr<float>(proj_out), stream_of(x)),
               "TurboQuantCompressorV2.compress");
  return {codes, signs, rn, vn};
}

std::tuple<Tensor, Tensor> compress_values(const Tensor& states, const Tensor& pi_split, const Tensor& bounds,
                                           int64_t bits, const c10::optional<Tensor>& y_out) {
  require_gpu(states, "tq::compress_values");
  TORCH_CHECK(states.dim() == 4, "tq::compress_values: expected [B, H, S, D] states");
  const c10::DeviceGuard g(states.device());
  Tensor x = activation(states);
  const int64_t B = x.size(0), H = x.size(1), S = x.size(2), D = x.size(3), n = B * H * S;
  Tensor codes = at::empty({n, out_cols(D, bits)}, x.options().dtype(at::kByte));
  Tensor vn = at::empty({n}, x.options().dtype(at::kHalf));
  check_status(tq_compress_values(x.data_ptr(), dtype_code(x.scalar_type()), static_cast<int32_t>(B),
                                  static_cast<int32_t>(H), static_cast<int32_t>(S), static_cast<int32_t>(D),
                                  x.stride(0), x.stride(1), x.stride(2), ptr<uint16_t>(pi_split), ptr<float>(bounds),
                                  static_cast<int32_t>(bits), ptr<uint8_t>(codes), ptr<uint16_t>(vn),
                                  optr<float>(y_out), stream_of(x)),
               "TurboQuantCompressorMSE.compress");
  return {codes, vn};
}

Tensor decompress_values(const Tensor& codes_in, const Tensor& vn_in, const Tensor& pit_split,
                         const Tensor& centroids, int64_t bits, at::IntArrayRef shape) {
  require_gpu(codes_in, "tq::decompress_values");
  TORCH_CHECK(shape.size() == 4, "tq::decompress_values: shape must be [B, H, S, D]");
  const c10::DeviceGuard g(codes_in.device());
  const int64_t n = shape[0] * shape[1] * shape[2], D = shape[3];
  Tensor codes = codes_in.reshape({n, codes_in.size(-1)}).contiguous();
  Tensor vn = vn_in.to(at::kHalf).reshape({n}).contiguous();
  Tensor out = at::empty(shape, codes.options().dtype(at::kFloat));
  check_status(tq_decompress_values(ptr<uint8_t>(codes), ptr<uint16_t>(vn), n, static_cast<int32_t>(D),
                                    ptr<uint16_t>(pit_split), ptr<float>(centroids), static_cast<int32_t>(bits),
                                    out.data_ptr(), TQ_F32, D, stream_of(out)),
               "TurboQuantCompressorMSE.decompress");
  return out;
}

std::tuple<Tensor, Tensor> query_prep(const Tensor& queries, const Tensor& pi_split, const Tensor& s_eff16) {
  require_gpu(queries, "tq::query_prep");
  TORCH_CHECK(queries.dim() == 4, "tq::query_prep: expected [B, Hq, Sq, D] queries");
  const c10::DeviceGuard g(queries.device());
  Tensor q = activation(queries);
  const int64_t B = q.size(0), Hq = q.size(1), Sq = q.size(2), D = q.size(3);
  Tensor q_rot = at::empty({B, Hq, Sq, D}, q.options().dtype(at::kHalf));
  Tensor q_proj = at::empty({B, Hq, Sq, D}, q.options().dtype(at::kFloat));
  check_status(tq_query_prep(q.data_ptr(), dtype_code(q.scalar_type()), static_cast<int32_t>(B),
                             static_cast<int32_t>(Hq), static_cast<int32_t>(Sq), static_cast<int32_t>(D), q.stride(0),
                             q.stride(1), q.stride(2), ptr<uint16_t>(pi_split), ptr<uint16_t>(s_eff16),
                             ptr<uint16_t>(q_rot), ptr<float>(q_proj), stream_of(q)),
               "prepare_queries");
  return {q_rot, q_proj};
}

// ---------------------------------------------------------------- scores and attention
Tensor scores(const Tensor& q_rot, const Tensor& q_proj, const Tensor& codes, const Tensor& signs,
              const Tensor& rn, const Tensor& vn, const Tensor& cent16, int64_t bits, int64_t hkv, int64_t sk,
              int64_t kv_stride, double coeff) {
  require_gpu(q_rot, "tq::scores");
  TORCH_CHECK(q_rot.scalar_type() == at::kHalf && q_proj.scalar_type() == at::kFloat,
              "tq::scores: q_rot must be float16 and q_proj float32 (tq::query_prep)");
  TORCH_CHECK(q_rot.is_contiguous() && q_proj.is_contiguous(), "tq::scores: prepared queries must be contiguous");
  const c10::DeviceGuard g(q_rot.device());
  const int64_t B = q_rot.size(0), Hq = q_rot.size(1), Sq = q_rot.size(2), D = q_rot.size(3);
  Tensor out = at::empty({B, Hq, Sq, sk}, q_rot.options().dtype(at::kFloat));
  check_status(tq_attention_scores_kv(ptr<uint16_t>(q_rot), ptr<float>(q_proj), ptr<uint8_t>(codes),
                                      ptr<uint8_t>(signs), ptr<uint16_t>(rn), ptr<uint16_t>(vn), ptr<uint16_t>(cent16),
                                      static_cast<int32_t>(B), static_cast<int32_t>(Hq), static_cast<int32_t>(hkv),
                                      static_cast<int32_t>(Sq), static_cast<int32_t>(sk), kv_stride,
                                      static_cast<int32_t>(D), static_cast<int32_t>(bits), static_cast<float>(coeff),
                                      ptr<float>(out), stream_of(out)),
               "asymmetric_attention_scores");
  return out;
}

// workspace: 0 = none (many-query kernels only), 1 = split-K partials allocated here from
// torch, 2 = the library's per-GPU scratch array (tq_attention_fwd_kv_noalloc)
Tensor attention(const Tensor& q_rot, const Tensor& q_proj, const Tensor& kcodes, const Tensor& ksigns,
                 const Tensor& krn, const Tensor& kvn, const Tensor& kcent16, int64_t bits, const Tensor& vcodes,
                 const Tensor& vvn, const Tensor& vcent32, int64_t val_bits, const Tensor& vpit, int64_t hkv,
                 int64_t sk, int64_t kv_stride, double coeff, double scale, bool causal,
                 const c10::optional<Tensor>& mask_in, at::ScalarType out_dtype, int64_t workspace) {
  require_gpu(q_rot, "tq::attention");
  TORCH_CHECK(q_rot.scalar_type() == at::kHalf && q_proj.scalar_type() == at::kFloat,
              "tq::attention: q_rot must be float16 and q_proj float32 (tq::query_prep)");
  TORCH_CHECK(q_rot.is_contiguous() && q_proj.is_contiguous(), "tq::attention: prepared queries must be contiguous");
  TORCH_CHECK(workspace >= 0 && workspace <= 2, "tq::attention: workspace mode must be 0, 1 or 2");
  const c10::DeviceGuard g(q_rot.device());
  const int64_t B = q_rot.size(0), Hq = q_rot.size(1), Sq = q_rot.size(2), D = q_rot.size(3);
  Tensor out = at::empty({B, Sq, Hq, D}, q_rot.options().dtype(out_dtype));
  Tensor mask;
  int64_t ms[4] = {0, 0, 0, 0};
  if (mask_in.has_value() && mask_in->defined()) {
    mask = mask_in->to(q_rot.device(), at::kFloat);
    while (mask.dim() < 4) mask = mask.unsqueeze(0);
    mask = mask.expand({B, Hq, Sq, sk});
    for (int i = 0; i < 4; ++i) ms[i] = mask.stride(i);
  }
  const float* mptr = mask.defined() ? ptr<float>(mask) : nullptr;
  void* s = stream_of(out);
  const int32_t b32 = static_cast<int32_t>(bits), B32 = static_cast<int32_t>(B), Hq32 = static_cast<int32_t>(Hq),
                Hkv32 = static_cast<int32_t>(hkv), Sq32 = static_cast<int32_t>(Sq), Sk32 = static_cast<int32_t>(sk),
                D32 = static_cast<int32_t>(D);
  if (workspace == 2) {
    check_status(tq_attention_fwd_kv_noalloc(
                     ptr<uint16_t>(q_rot), ptr<float>(q_proj), ptr<uint8_t>(kcodes), ptr<uint8_t>(ksigns),
                     ptr<uint16_t>(krn), ptr<uint16_t>(kvn), ptr<uint16_t>(kcent16), b32, ptr<uint8_t>(vcodes),
                     ptr<uint16_t>(vvn), ptr<float>(vcent32), static_cast<int32_t>(val_bits), ptr<uint16_t>(vpit), B32,
                     Hq32, Hkv32, Sq32, Sk32, kv_stride, D32, static_cast<float>(coeff), static_cast<float>(scale),
                     causal ? 1 : 0, mptr, ms[0], ms[1], ms[2], ms[3], out.data_ptr(), dtype_code(out_dtype),
                     out.stride(0), out.stride(2), out.stride(1), s),
                 "compressed_attention");
    return out;
  }
  Tensor ws;
  int64_t ws_bytes = 0;
  if (workspace == 1 && val_bits == bits) {
    ws_bytes = tq_attention_workspace_size(B32, Hq32, Hkv32, Sq32, Sk32, D32, b32);
    if (ws_bytes > 0) ws = at::empty({ws_bytes}, q_rot.options().dtype(at::kByte));
  }
  check_status(tq_attention_fwd_kv(ptr<uint16_t>(q_rot), ptr<float>(q_proj), ptr<uint8_t>(kcodes),
                                   ptr<uint8_t>(ksigns), ptr<uint16_t>(krn), ptr<uint16_t>(kvn), ptr<uint16_t>(kcent16),
                                   b32, ptr<uint8_t>(vcodes), ptr<uint16_t>(vvn), ptr<float>(vcent32),
                                   static_cast<int32_t>(val_bits), ptr<uint16_t>(vpit), B32, Hq32, Hkv32, Sq32, Sk32,
                                   kv_stride, D32, static_cast<float>(coeff), static_cast<float>(scale),
                                   causal ? 1 : 0, mptr, ms[0], ms[1], ms[2], ms[3], out.data_ptr(),
                                   dtype_code(out_dtype), out.stride(0), out.stride(2), out.stride(1),
                                   ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, s),
               "compressed_attention");
  return out;
}

int64_t workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t d, int64_t bits) {
  return tq_attention_workspace_size(static_cast<int32_t>(B), static_cast<int32_t>(Hq), static_cast<int32_t>(Hkv),
                                     static_cast<int32_t>(Sq), static_cast<int32_t>(Sk), static_cast<int32_t>(d),
                                     static_cast<int32_t>(bits));
}

}  // namespace

TORCH_LIBRARY(tq, m) {
  m.def("pack_bits(Tensor idx, int b) -> Tensor");
  m.def("unpack_bits(Tensor packed, int b, int d) -> Tensor");
  m.def("quantize_pack(Tensor y, Tensor bounds, int b_eff) -> Tensor");
  m.def("dequantize(Tensor packed, Tensor centroids, int b, int d) -> Tensor");
  m.def("compress_keys(Tensor states, Tensor pi_split, Tensor seff_split, Tensor centroids, Tensor bounds, "
        "int b_eff, Tensor? y_out=None, Tensor? proj_out=None) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("compress_values(Tensor states, Tensor pi_split, Tensor bounds, int bits, Tensor? y_out=None) "
        "-> (Tensor, Tensor)");
  m.def("decompress_values(Tensor codes, Tensor vn, Tensor pit_split, Tensor centroids, int bits, int[] shape) "
        "-> Tensor");
  m.def("query_prep(Tensor queries, Tensor pi_split, Tensor s_eff) -> (Tensor, Tensor)");
  m.def("scores(Tensor q_rot, Tensor q_proj, Tensor codes, Tensor signs, Tensor rn, Tensor vn, Tensor centroids, "
        "int bits, int hkv, int sk, int kv_stride, float coeff) -> Tensor");
  m.def("attention(Tensor q_rot, Tensor q_proj, Tensor kcodes, Tensor ksigns, Tensor krn, Tensor kvn, "
        "Tensor kcent, int bits, Tensor vcodes, Tensor vvn, Tensor vcent, int val_bits, Tensor vpit, int hkv, "
        "int sk, int kv_stride, float coeff, float scale, bool causal, Tensor? mask, ScalarType out_dtype, "
        "int workspace) -> Tensor");
  m.def("workspace_size(int B, int Hq, int Hkv, int Sq, int Sk, int d, int bits) -> int", &workspace_size);
}

TORCH_LIBRARY_IMPL(tq, CUDA, m) {
  m.impl("pack_bits", &pack_bits);
  m.impl("unpack_bits", &unpack_bits);
  m.impl("quantize_pack", &quantize_pack);
  m.impl("dequantize", &dequantize);
  m.impl("compress_keys", &compress_keys);
  m.impl("compress_values", &compress_values);
  m.impl("decompress_values", &decompress_values);
  m.impl("query_prep", &query_prep);
  m.impl("scores", &scores);
  m.impl("attention", &attention);
}
