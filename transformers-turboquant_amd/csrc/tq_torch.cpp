// torch.ops.tq: the PyTorch-ROCm operator layer over the C ABI of libtq_amd.so
// (include/tq_api.h).  Each op checks every tensor it hands to the library (device,
// dtype, contiguity, row width and the number of rows or entries the kernels will
// read), allocates its outputs with torch (the caching allocator, so calls are
// capturable into HIP graphs), and calls one C entry point on torch's current stream
// of the tensors' device.  No kernel code lives here: the HIP kernels are the C
// library's.
//
// The checks read tensor metadata only.  They are shared with a Meta kernel per op,
// which runs them and returns empty outputs of the right shapes: shape inference for
// meta / fake tensors, and the CPU-side tests of the checks themselves.
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

int32_t dtype_code(at::ScalarType s) {
  switch (s) {
    case at::kFloat: return TQ_F32;
    case at::kHalf: return TQ_F16;
    case at::kBFloat16: return TQ_BF16;
    default: TORCH_CHECK(false, "unsupported activation dtype ", s, "; expected float32, float16 or bfloat16");
  }
  return -1;
}

bool is_act(at::ScalarType s) { return s == at::kFloat || s == at::kHalf || s == at::kBFloat16; }

// activations: float32 / float16 / bfloat16 with unit stride along the last dim
Tensor activation(const Tensor& x) {
  Tensor y = x;
  if (!is_act(y.scalar_type())) y = y.to(at::kFloat);
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

// ---------------------------------------------------------------- argument checks
// A plane or table the library reads through a raw pointer: on the op's device, of the
// dtype the kernel reads, contiguous (rows are addressed by index), `width` elements per
// row when width > 1, and at least rows * width elements.
struct Checker {
  const char* op;
  c10::Device dev;

  void same_device(const Tensor& t, const char* name) const {
    TORCH_CHECK(t.defined(), op, ": ", name, " is undefined");
    TORCH_CHECK(t.device() == dev, op, ": ", name, " is on ", t.device(), ", expected ", dev);
  }
  void plane(const Tensor& t, const char* name, at::ScalarType dt, int64_t rows, int64_t width = 1) const {
    same_device(t, name);
    TORCH_CHECK(t.scalar_type() == dt, op, ": ", name, " must be ", dt, ", got ", t.scalar_type());
    TORCH_CHECK(t.is_contiguous(), op, ": ", name, " must be contiguous");
    if (width > 1)
      TORCH_CHECK(t.dim() >= 1 && t.size(-1) == width, op, ": ", name, " rows must hold ", width,
                  " elements, got shape ", t.sizes());
    TORCH_CHECK(t.numel() >= rows * width, op, ": ", name, " holds ", t.numel(), " elements, the kernels read ",
                rows * width);
  }
  void table(const Tensor& t, const char* name, at::ScalarType dt, int64_t entries) const {
    plane(t, name, dt, entries, 1);
  }
  void optional_out(const c10::optional<Tensor>& t, const char* name, int64_t n) const {
    if (t.has_value() && t->defined()) plane(*t, name, at::kFloat, n, 1);
  }
};

// rows the kernels read from B * hkv head sequences of `sk` rows that start kv_stride apart
// (0: sk, i.e. contiguous)
int64_t kv_rows(int64_t B, int64_t hkv, int64_t sk, int64_t kv_stride) {
  const int64_t stride = kv_stride > 0 ? kv_stride : sk;
  return B * hkv > 0 ? (B * hkv - 1) * stride + sk : 0;
}

// prepared queries and the key planes of tq::scores / tq::attention
void check_prepared_keys(const Checker& c, const Tensor& q_rot, const Tensor& q_proj, const Tensor& codes,
                         const Tensor& signs, const Tensor& rn, const Tensor& vn, const Tensor& cent16, int64_t bits,
                         int64_t hkv, int64_t sk, int64_t kv_stride) {
  TORCH_CHECK(q_rot.dim() == 4, c.op, ": prepared queries must be [B, Hq, Sq, D], got ", q_rot.sizes());
  TORCH_CHECK(q_rot.scalar_type() == at::kHalf && q_proj.scalar_type() == at::kFloat, c.op,
              ": q_rot must be float16 and q_proj float32 (tq::query_prep)");
  TORCH_CHECK(q_rot.is_contiguous() && q_proj.is_contiguous(), c.op, ": prepared queries must be contiguous");
  c.same_device(q_proj, "q_proj");
  TORCH_CHECK(q_proj.sizes() == q_rot.sizes(), c.op, ": q_proj ", q_proj.sizes(), " differs from q_rot ",
              q_rot.sizes());
  const int64_t B = q_rot.size(0), Hq = q_rot.size(1), D = q_rot.size(3);
  TORCH_CHECK(bits >= 2 && bits <= 9, c.op, ": key bits must be 2..9, got ", bits);
  TORCH_CHECK(hkv >= 1 && Hq % hkv == 0, c.op, ": ", Hq, " query heads are not a multiple of ", hkv, " kv heads");
  TORCH_CHECK(sk >= 0 && (kv_stride == 0 || kv_stride >= sk), c.op, ": kv_stride ", kv_stride,
              " must be 0 or at least Sk = ", sk);
  const int64_t rows = kv_rows(B, hkv, sk, kv_stride);
  c.plane(codes, "packed_key_indices", at::kByte, rows, out_cols(D, bits - 1));
  c.plane(signs, "packed_qjl_signs", at::kByte, rows, out_cols(D, 1));
  c.plane(rn, "residual_norm", at::kHalf, rows);
  c.plane(vn, "vec_norms (keys)", at::kHalf, rows);
  c.table(cent16, "key centroids", at::kHalf, int64_t{1} << (bits - 1));
}

void check_values(const Checker& c, const Tensor& q_rot, const Tensor& vcodes, const Tensor& vvn,
                  const Tensor& vcent32, int64_t val_bits, const Tensor& vpit, int64_t hkv, int64_t sk,
                  int64_t kv_stride) {
  const int64_t B = q_rot.size(0), D = q_rot.size(3);
  TORCH_CHECK(val_bits >= 1 && val_bits <= 8, c.op, ": value bits must be 1..8, got ", val_bits);
  const int64_t rows = kv_rows(B, hkv, sk, kv_stride);
  c.plane(vcodes, "packed_indices (values)", at::kByte, rows, out_cols(D, val_bits));
  c.plane(vvn, "vec_norms (values)", at::kHalf, rows);
  c.table(vcent32, "value centroids", at::kFloat, int64_t{1} << val_bits);
  c.table(vpit, "split Pi_v^T", at::kHalf, 2 * D * D);
}

// the additive mask as a float32 view broadcast to [B, Hq, Sq, Sk] (no copy when it already
// is float32 on the device)
Tensor attention_mask(const Checker& c, const c10::optional<Tensor>& mask_in, const Tensor& q_rot, int64_t sk) {
  if (!mask_in.has_value() || !mask_in->defined()) return Tensor();
  Tensor mask = *mask_in;
  TORCH_CHECK(mask.dim() <= 4, c.op, ": the mask must broadcast to [B, Hq, Sq, Sk], got ", mask.sizes());
  if (mask.device() != q_rot.device() || mask.scalar_type() != at::kFloat) mask = mask.to(q_rot.device(), at::kFloat);
  while (mask.dim() < 4) mask = mask.unsqueeze(0);
  return mask.expand({q_rot.size(0), q_rot.size(1), q_rot.size(2), sk});
}

// ---------------------------------------------------------------- bit ops (kernels/bit_ops.py)
void check_bits(const char* op, int64_t b) { TORCH_CHECK(b >= 1 && b <= 8, op, ": b must be 1..8, got ", b); }

Tensor pack_bits_meta(const Tensor& idx, int64_t b) {
  TORCH_CHECK(idx.dim() == 2, "tq::pack_bits: expected [N, d] codes");
  check_bits("tq::pack_bits", b);
  return at::empty({idx.size(0), out_cols(idx.size(1), b)}, idx.options().dtype(at::kByte));
}

Tensor pack_bits(const Tensor& idx_in, int64_t b) {
  pack_bits_meta(idx_in, b);
  const c10::DeviceGuard g(idx_in.device());
  Tensor idx = idx_in.to(at::kInt).contiguous();
  const int64_t n = idx.size(0), d = idx.size(1);
  Tensor out = at::empty({n, out_cols(d, b)}, idx.options().dtype(at::kByte));
  check_status(tq_pack_bits(ptr<int32_t>(idx), n, static_cast<int32_t>(d), d, static_cast<int32_t>(b),
                            ptr<uint8_t>(out), out.size(1), stream_of(out)),
               "tq::pack_bits");
  return out;
}

Tensor unpack_bits_meta(const Tensor& packed, int64_t b, int64_t d) {
  TORCH_CHECK(packed.dim() == 2, "tq::unpack_bits: expected [N, bytes] packed rows");
  check_bits("tq::unpack_bits", b);
  TORCH_CHECK(packed.scalar_type() == at::kByte, "tq::unpack_bits: packed rows must be uint8");
  TORCH_CHECK(packed.size(1) >= out_cols(d, b), "tq::unpack_bits: rows of ", packed.size(1), " bytes hold fewer than ",
              d, " codes of ", b, " bits");
  return at::empty({packed.size(0), d}, packed.options().dtype(at::kInt));
}

Tensor unpack_bits(const Tensor& packed_in, int64_t b, int64_t d) {
  unpack_bits_meta(packed_in, b, d);
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
Tensor quantize_pack_meta(const Tensor& y, const Tensor& bounds, int64_t b_eff) {
  TORCH_CHECK(y.dim() == 2, "tq::quantize_pack: expected [N, d] rotated rows");
  check_bits("tq::quantize_pack", b_eff);
  // the reference asserts the boundary count (quantize.py:223-227)
  TORCH_CHECK(bounds.numel() == (int64_t{1} << b_eff) - 1, "tq::quantize_pack: expected ",
              (int64_t{1} << b_eff) - 1, " boundaries for ", b_eff, " bits, got ", bounds.numel());
  return at::empty({y.size(0), out_cols(y.size(1), b_eff)}, y.options().dtype(at::kByte));
}

Tensor quantize_pack(const Tensor& y_in, const Tensor& bounds_in, int64_t b_eff) {
  quantize_pack_meta(y_in, bounds_in, b_eff);
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

Tensor dequantize_meta(const Tensor& packed, const Tensor& cent, int64_t b, int64_t d) {
  TORCH_CHECK(packed.dim() == 2 && packed.scalar_type() == at::kByte, "tq::dequantize: expected uint8 [N, bytes]");
  check_bits("tq::dequantize", b);
  TORCH_CHECK(packed.size(1) >= out_cols(d, b), "tq::dequantize: rows of ", packed.size(1), " bytes hold fewer than ",
              d, " codes of ", b, " bits");
  TORCH_CHECK(cent.numel() >= (int64_t{1} << b), "tq::dequantize: ", cent.numel(), " centroids for ", b, "-bit codes");
  return at::empty({packed.size(0), d}, packed.options().dtype(at::kHalf));
}

Tensor dequantize(const Tensor& packed_in, const Tensor& cent_in, int64_t b, int64_t d) {
  dequantize_meta(packed_in, cent_in, b, d);
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
using KeyPlanes = std::tuple<Tensor, Tensor, Tensor, Tensor>;

KeyPlanes compress_keys_meta(const Tensor& states, const Tensor& pi_split, const Tensor& seff_split,
                             const Tensor& centroids, const Tensor& bounds, int64_t b_eff,
                             const c10::optional<Tensor>& y_out, const c10::optional<Tensor>& proj_out) {
  const Checker c{"tq::compress_keys", states.device()};
  TORCH_CHECK(states.dim() == 4, c.op, ": expected [B, H, S, D] states");
  TORCH_CHECK(b_eff >= 1 && b_eff <= 8, c.op, ": key code bits must be 1..8, got ", b_eff);
  const int64_t B = states.size(0), H = states.size(1), S = states.size(2), D = states.size(3), n = B * H * S;
  c.table(pi_split, "split Pi", at::kHalf, 2 * D * D);
  c.table(seff_split, "split S_eff", at::kHalf, 2 * D * D);
  c.table(centroids, "centroids", at::kFloat, int64_t{1} << b_eff);
  c.table(bounds, "boundaries", at::kFloat, (int64_t{1} << b_eff) - 1);
  c.optional_out(y_out, "y_out", n * D);
  c.optional_out(proj_out, "proj_out", n * D);
  auto u8 = states.options().dtype(at::kByte);
  return {at::empty({n, out_cols(D, b_eff)}, u8), at::empty({n, out_cols(D, 1)}, u8),
          at::empty({B, H, S}, states.options().dtype(at::kHalf)), at::empty({B, H, S}, states.options().dtype(at::kHalf))};
}

KeyPlanes compress_keys(const Tensor& states, const Tensor& pi_split, const Tensor& seff_split, const Tensor& centroids,
                        const Tensor& bounds, int64_t b_eff, const c10::optional<Tensor>& y_out,
                        const c10::optional<Tensor>& proj_out) {
  compress_keys_meta(states, pi_split, seff_split, centroids, bounds, b_eff, y_out, proj_out);
  const c10::DeviceGuard g(states.device());
  Tensor x = activation(states);
  const int64_t B = x.size(0), H = x.size(1), S = x.size(2), D = x.size(3), n = B * H * S;
  auto u8 = x.options().dtype(at::kByte);
  Tensor codes = at::empty({n, out_cols(D, b_eff)}, u8);
  Tensor signs = at::empty({n, out_cols(D, 1)}, u8);
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

std::tuple<Tensor, Tensor> compress_values_meta(const Tensor& states, const Tensor& pi_split, const Tensor& bounds,
                                                int64_t bits, const c10::optional<Tensor>& y_out) {
  const Checker c{"tq::compress_values", states.device()};
  TORCH_CHECK(states.dim() == 4, c.op, ": expected [B, H, S, D] states");
  TORCH_CHECK(bits >= 1 && bits <= 8, c.op, ": value bits must be 1..8, got ", bits);
  const int64_t B = states.size(0), H = states.size(1), S = states.size(2), D = states.size(3), n = B * H * S;
  c.table(pi_split, "split Pi", at::kHalf, 2 * D * D);
  c.table(bounds, "boundaries", at::kFloat, (int64_t{1} << bits) - 1);
  c.optional_out(y_out, "y_out", n * D);
  return {at::empty({n, out_cols(D, bits)}, states.options().dtype(at::kByte)),
          at::empty({n}, states.options().dtype(at::kHalf))};
}

std::tuple<Tensor, Tensor> compress_values(const Tensor& states, const Tensor& pi_split, const Tensor& bounds,
                                           int64_t bits, const c10::optional<Tensor>& y_out) {
  compress_values_meta(states, pi_split, bounds, bits, y_out);
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

Tensor decompress_values_meta(const Tensor& codes, const Tensor& vn, const Tensor& pit_split, const Tensor& centroids,
                              int64_t bits, at::IntArrayRef shape) {
  const Checker c{"tq::decompress_values", codes.device()};
  TORCH_CHECK(shape.size() == 4, c.op, ": shape must be [B, H, S, D]");
  TORCH_CHECK(bits >= 1 && bits <= 8, c.op, ": value bits must be 1..8, got ", bits);
  const int64_t n = shape[0] * shape[1] * shape[2], D = shape[3];
  c.same_device(codes, "packed_indices");
  TORCH_CHECK(codes.scalar_type() == at::kByte && codes.dim() >= 1 && codes.size(-1) == out_cols(D, bits) &&
                  codes.numel() == n * out_cols(D, bits),
              c.op, ": packed_indices must be uint8 rows of ", out_cols(D, bits), " bytes for ", n, " rows, got ",
              codes.scalar_type(), " ", codes.sizes());
  c.same_device(vn, "vec_norms");
  TORCH_CHECK(vn.numel() == n, c.op, ": ", vn.numel(), " value norms for ", n, " rows");
  c.table(pit_split, "split Pi^T", at::kHalf, 2 * D * D);
  c.table(centroids, "centroids", at::kFloat, int64_t{1} << bits);
  return at::empty(shape, codes.options().dtype(at::kFloat));
}

Tensor decompress_values(const Tensor& codes_in, const Tensor& vn_in, const Tensor& pit_split,
                         const Tensor& centroids, int64_t bits, at::IntArrayRef shape) {
  decompress_values_meta(codes_in, vn_in, pit_split, centroids, bits, shape);
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

std::tuple<Tensor, Tensor> query_prep_meta(const Tensor& queries, const Tensor& pi_split, const Tensor& s_eff16) {
  const Checker c{"tq::query_prep", queries.device()};
  TORCH_CHECK(queries.dim() == 4, c.op, ": expected [B, Hq, Sq, D] queries");
  const int64_t B = queries.size(0), Hq = queries.size(1), Sq = queries.size(2), D = queries.size(3);
  c.table(pi_split, "split Pi", at::kHalf, 2 * D * D);
  c.table(s_eff16, "f16 S_eff", at::kHalf, D * D);
  return {at::empty({B, Hq, Sq, D}, queries.options().dtype(at::kHalf)),
          at::empty({B, Hq, Sq, D}, queries.options().dtype(at::kFloat))};
}

std::tuple<Tensor, Tensor> query_prep(const Tensor& queries, const Tensor& pi_split, const Tensor& s_eff16) {
  query_prep_meta(queries, pi_split, s_eff16);
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

// ---------------------------------------------------------------- compressed-cache append
// New keys / values [B, H, S, D] compressed straight into rows [pos, pos + S) of a cache's
// capacity planes ([B, H, capacity, ...], written in place), and the new queries [B, Hq, S, D]
// prepared (empty outputs when no queries are given).  No reference counterpart: the reference
// disables the KV cache (patch.py:81).
std::tuple<Tensor, Tensor> cache_append_meta(const Tensor& k, const Tensor& v, const c10::optional<Tensor>& q,
                                             const Tensor& kpi, const Tensor& kseff, const Tensor& kcent,
                                             const Tensor& kbounds, int64_t key_code_bits, const Tensor& vpi,
                                             const Tensor& vbounds, int64_t val_bits, const Tensor& kseff16,
                                             const Tensor& kcodes, const Tensor& ksigns, const Tensor& krn,
                                             const Tensor& kvn, const Tensor& vcodes, const Tensor& vvn, int64_t pos) {
  const Checker c{"tq::cache_append", k.device()};
  TORCH_CHECK(k.dim() == 4 && v.sizes() == k.sizes(), c.op, ": k and v must be [B, H, S, D] of one shape, got ",
              k.sizes(), " and ", v.sizes());
  c.same_device(v, "v");
  TORCH_CHECK(key_code_bits >= 1 && key_code_bits <= 8 && val_bits >= 1 && val_bits <= 8, c.op,
              ": bits must be 1..8");
  const int64_t B = k.size(0), H = k.size(1), S = k.size(2), D = k.size(3);
  TORCH_CHECK(kcodes.dim() == 4 && kcodes.size(0) == B && kcodes.size(1) == H, c.op,
              ": key_codes must be [B, H, capacity, width] with B, H of the new keys, got ", kcodes.sizes());
  const int64_t cap = kcodes.size(2), rows = B * H * cap;
  TORCH_CHECK(pos >= 0 && pos + S <= cap, c.op, ": rows [", pos, ", ", pos + S, ") exceed the capacity ", cap);
  c.plane(kcodes, "key_codes", at::kByte, rows, out_cols(D, key_code_bits));
  c.plane(ksigns, "key_signs", at::kByte, rows, out_cols(D, 1));
  c.plane(krn, "key residual norms", at::kHalf, rows);
  c.plane(kvn, "key norms", at::kHalf, rows);
  c.plane(vcodes, "value codes", at::kByte, rows, out_cols(D, val_bits));
  c.plane(vvn, "value norms", at::kHalf, rows);
  for (const Tensor* t : {&ksigns, &krn, &kvn, &vcodes, &vvn})
    TORCH_CHECK(t->dim() >= 3 && t->size(0) == B && t->size(1) == H && t->size(2) == cap, c.op,
                ": every cache plane must be [B, H, capacity, ...], got ", t->sizes());
  c.table(kpi, "key split Pi", at::kHalf, 2 * D * D);
  c.table(kseff, "key split S_eff", at::kHalf, 2 * D * D);
  c.table(kcent, "key centroids", at::kFloat, int64_t{1} << key_code_bits);
  c.table(kbounds, "key boundaries", at::kFloat, (int64_t{1} << key_code_bits) - 1);
  c.table(vpi, "value split Pi", at::kHalf, 2 * D * D);
  c.table(vbounds, "value boundaries", at::kFloat, (int64_t{1} << val_bits) - 1);
  if (q.has_value() && q->defined()) {
    c.same_device(*q, "q");
    TORCH_CHECK(q->dim() == 4 && q->size(0) == B && q->size(2) == S && q->size(3) == D, c.op,
                ": q must be [B, Hq, S, D] with B, S, D of the new keys, got ", q->sizes());
    c.table(kseff16, "key f16 S_eff", at::kHalf, D * D);
    return {at::empty({B, q->size(1), S, D}, q->options().dtype(at::kHalf)),
            at::empty({B, q->size(1), S, D}, q->options().dtype(at::kFloat))};
  }
  return {at::empty({0}, k.options().dtype(at::kHalf)), at::empty({0}, k.options().dtype(at::kFloat))};
}

std::tuple<Tensor, Tensor> cache_append(const Tensor& k_in, const Tensor& v_in, const c10::optional<Tensor>& q_in,
                                        const Tensor& kpi, const Tensor& kseff, const Tensor& kcent,
                                        const Tensor& kbounds, int64_t key_code_bits, const Tensor& vpi,
                                        const Tensor& vbounds, int64_t val_bits, const Tensor& kseff16,
                                        const Tensor& kcodes, const Tensor& ksigns, const Tensor& krn,
                                        const Tensor& kvn, const Tensor& vcodes, const Tensor& vvn, int64_t pos) {
  // the checks, and the q_rot / q_proj outputs they return (allocated on k's device)
  auto outs = cache_append_meta(k_in, v_in, q_in, kpi, kseff, kcent, kbounds, key_code_bits, vpi, vbounds, val_bits,
                                kseff16, kcodes, ksigns, krn, kvn, vcodes, vvn, pos);
  const c10::DeviceGuard g(k_in.device());
  Tensor k = activation(k_in);
  Tensor v = v_in.scalar_type() == k.scalar_type() && v_in.stride(-1) == 1 ? v_in : v_in.to(k.scalar_type()).contiguous();
  const bool has_q = q_in.has_value() && q_in->defined();
  Tensor q = has_q ? (q_in->scalar_type() == k.scalar_type() && q_in->stride(-1) == 1
                          ? *q_in : q_in->to(k.scalar_type()).contiguous())
                   : Tensor();
  const int64_t B = k.size(0), H = k.size(1), S = k.size(2), D = k.size(3), cap = kcodes.size(2);
  const int64_t Hq = has_q ? q.size(1) : 0;
  Tensor q_rot = std::get<0>(outs), q_proj = std::get<1>(outs);
  check_status(tq_cache_append(k.data_ptr(), v.data_ptr(), dtype_code(k.scalar_type()), static_cast<int32_t>(B),
                               static_cast<int32_t>(H), static_cast<int32_t>(S), static_cast<int32_t>(D), k.stride(0),
                               k.stride(1), k.stride(2), v.stride(0), v.stride(1), v.stride(2), ptr<uint16_t>(kpi),
                               ptr<uint16_t>(kseff), ptr<float>(kcent), ptr<float>(kbounds),
                               static_cast<int32_t>(key_code_bits), ptr<uint16_t>(vpi), ptr<float>(vbounds),
                               static_cast<int32_t>(val_bits), ptr<uint8_t>(kcodes), ptr<uint8_t>(ksigns),
                               ptr<uint16_t>(krn), ptr<uint16_t>(kvn), ptr<uint8_t>(vcodes), ptr<uint16_t>(vvn), cap,
                               pos, has_q ? q.data_ptr() : nullptr, static_cast<int32_t>(Hq),
                               has_q ? q.stride(0) : 0, has_q ? q.stride(1) : 0, has_q ? q.stride(2) : 0,
                               has_q ? ptr<uint16_t>(kseff16) : nullptr, has_q ? ptr<uint16_t>(q_rot) : nullptr,
                               has_q ? ptr<float>(q_proj) : nullptr, stream_of(k)),
               "TurboQuantCache.append");
  return {q_rot, q_proj};
}

// ---------------------------------------------------------------- scores and attention
Tensor scores_meta(const Tensor& q_rot, const Tensor& q_proj, const Tensor& codes, const Tensor& signs, const Tensor& rn,
                   const Tensor& vn, const Tensor& cent16, int64_t bits, int64_t hkv, int64_t sk, int64_t kv_stride,
                   double coeff) {
  const Checker c{"tq::scores", q_rot.device()};
  check_prepared_keys(c, q_rot, q_proj, codes, signs, rn, vn, cent16, bits, hkv, sk, kv_stride);
  return at::empty({q_rot.size(0), q_rot.size(1), q_rot.size(2), sk}, q_rot.options().dtype(at::kFloat));
}

Tensor scores(const Tensor& q_rot, const Tensor& q_proj, const Tensor& codes, const Tensor& signs,
              const Tensor& rn, const Tensor& vn, const Tensor& cent16, int64_t bits, int64_t hkv, int64_t sk,
              int64_t kv_stride, double coeff) {
  scores_meta(q_rot, q_proj, codes, signs, rn, vn, cent16, bits, hkv, sk, kv_stride, coeff);
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

Tensor attention_meta(const Tensor& q_rot, const Tensor& q_proj, const Tensor& kcodes, const Tensor& ksigns,
                      const Tensor& krn, const Tensor& kvn, const Tensor& kcent16, int64_t bits, const Tensor& vcodes,
                      const Tensor& vvn, const Tensor& vcent32, int64_t val_bits, const Tensor& vpit, int64_t hkv,
                      int64_t sk, int64_t kv_stride, double coeff, double scale, bool causal,
                      const c10::optional<Tensor>& mask_in, at::ScalarType out_dtype, int64_t workspace) {
  const Checker c{"tq::attention", q_rot.device()};
  TORCH_CHECK(workspace >= 0 && workspace <= 2, c.op, ": workspace mode must be 0, 1 or 2");
  TORCH_CHECK(is_act(out_dtype), c.op, ": out_dtype must be float32, float16 or bfloat16");
  check_prepared_keys(c, q_rot, q_proj, kcodes, ksigns, krn, kvn, kcent16, bits, hkv, sk, kv_stride);
  check_values(c, q_rot, vcodes, vvn, vcent32, val_bits, vpit, hkv, sk, kv_stride);
  attention_mask(c, mask_in, q_rot, sk);  // broadcastable to [B, Hq, Sq, Sk]
  return at::empty({q_rot.size(0), q_rot.size(2), q_rot.size(1), q_rot.size(3)}, q_rot.options().dtype(out_dtype));
}

// workspace: 0 = none (many-query kernels only), 1 = split-K partials allocated here from
// torch, 2 = the library's per-GPU scratch array (tq_attention_fwd_kv_noalloc)
Tensor attention(const Tensor& q_rot, const Tensor& q_proj, const Tensor& kcodes, const Tensor& ksigns,
                 const Tensor& krn, const Tensor& kvn, const Tensor& kcent16, int64_t bits, const Tensor& vcodes,
                 const Tensor& vvn, const Tensor& vcent32, int64_t val_bits, const Tensor& vpit, int64_t hkv,
                 int64_t sk, int64_t kv_stride, double coeff, double scale, bool causal,
                 const c10::optional<Tensor>& mask_in, at::ScalarType out_dtype, int64_t workspace) {
  // the checks, and the [B, Sq, Hq, D] output they return (allocated on q_rot's device)
  Tensor out = attention_meta(q_rot, q_proj, kcodes, ksigns, krn, kvn, kcent16, bits, vcodes, vvn, vcent32, val_bits,
                              vpit, hkv, sk, kv_stride, coeff, scale, causal, mask_in, out_dtype, workspace);
  const Checker c{"tq::attention", q_rot.device()};
  const c10::DeviceGuard g(q_rot.device());
  const int64_t B = q_rot.size(0), Hq = q_rot.size(1), Sq = q_rot.size(2), D = q_rot.size(3);
  Tensor mask = attention_mask(c, mask_in, q_rot, sk);
  int64_t ms[4] = {0, 0, 0, 0};
  if (mask.defined())
    for (int i = 0; i < 4; ++i) ms[i] = mask.stride(i);
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
  if (workspace == 1) {
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

// A cached decode step in one call: cache_append (the new keys / values into the capacity
// planes at row pos, the new queries prepared in the same launch), then attention over the
// planes' first pos + S rows.  The same two operators back to back, without the second
// crossing of the dispatcher and the Python between them (a one-token step is bound by that
// host time, not by its kernels).
Tensor cache_attend(const Tensor& k, const Tensor& v, const Tensor& q, const Tensor& kpi, const Tensor& kseff,
                    const Tensor& kcent, const Tensor& kbounds, int64_t key_code_bits, const Tensor& vpi,
                    const Tensor& vbounds, int64_t val_bits, const Tensor& kseff16, const Tensor& kcodes,
                    const Tensor& ksigns, const Tensor& krn, const Tensor& kvn, const Tensor& vcodes,
                    const Tensor& vvn, int64_t pos, const Tensor& kcent16, const Tensor& vcent32, const Tensor& vpit,
                    double coeff, double scale, bool causal, const c10::optional<Tensor>& mask,
                    at::ScalarType out_dtype, int64_t workspace) {
  auto qp = cache_append(k, v, q, kpi, kseff, kcent, kbounds, key_code_bits, vpi, vbounds, val_bits, kseff16, kcodes,
                         ksigns, krn, kvn, vcodes, vvn, pos);
  return attention(std::get<0>(qp), std::get<1>(qp), kcodes, ksigns, krn, kvn, kcent16, key_code_bits + 1, vcodes, vvn,
                   vcent32, val_bits, vpit, k.size(1), pos + k.size(2), kvn.size(-1), coeff, scale, causal, mask,
                   out_dtype, workspace);
}

Tensor cache_attend_meta(const Tensor& k, const Tensor& v, const Tensor& q, const Tensor& kpi, const Tensor& kseff,
                         const Tensor& kcent, const Tensor& kbounds, int64_t key_code_bits, const Tensor& vpi,
                         const Tensor& vbounds, int64_t val_bits, const Tensor& kseff16, const Tensor& kcodes,
                         const Tensor& ksigns, const Tensor& krn, const Tensor& kvn, const Tensor& vcodes,
                         const Tensor& vvn, int64_t pos, const Tensor& kcent16, const Tensor& vcent32,
                         const Tensor& vpit, double coeff, double scale, bool causal,
                         const c10::optional<Tensor>& mask, at::ScalarType out_dtype, int64_t workspace) {
  auto qp = cache_append_meta(k, v, q, kpi, kseff, kcent, kbounds, key_code_bits, vpi, vbounds, val_bits, kseff16,
                              kcodes, ksigns, krn, kvn, vcodes, vvn, pos);
  return attention_meta(std::get<0>(qp), std::get<1>(qp), kcodes, ksigns, krn, kvn, kcent16, key_code_bits + 1, vcodes,
                        vvn, vcent32, val_bits, vpit, k.size(1), pos + k.size(2), kvn.size(-1), coeff, scale, causal,
                        mask, out_dtype, workspace);
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
  m.def("cache_append(Tensor k, Tensor v, Tensor? q, Tensor kpi, Tensor kseff, Tensor kcent, Tensor kbounds, "
        "int key_code_bits, Tensor vpi, Tensor vbounds, int val_bits, Tensor kseff16, Tensor(a!) kcodes, "
        "Tensor(b!) ksigns, Tensor(c!) krn, Tensor(d!) kvn, Tensor(e!) vcodes, Tensor(f!) vvn, int pos) "
        "-> (Tensor, Tensor)");
  m.def("scores(Tensor q_rot, Tensor q_proj, Tensor codes, Tensor signs, Tensor rn, Tensor vn, Tensor centroids, "
        "int bits, int hkv, int sk, int kv_stride, float coeff) -> Tensor");
  m.def("attention(Tensor q_rot, Tensor q_proj, Tensor kcodes, Tensor ksigns, Tensor krn, Tensor kvn, "
        "Tensor kcent, int bits, Tensor vcodes, Tensor vvn, Tensor vcent, int val_bits, Tensor vpit, int hkv, "
        "int sk, int kv_stride, float coeff, float scale, bool causal, Tensor? mask, ScalarType out_dtype, "
        "int workspace) -> Tensor");
  m.def("cache_attend(Tensor k, Tensor v, Tensor q, Tensor kpi, Tensor kseff, Tensor kcent, Tensor kbounds, "
        "int key_code_bits, Tensor vpi, Tensor vbounds, int val_bits, Tensor kseff16, Tensor(a!) kcodes, "
        "Tensor(b!) ksigns, Tensor(c!) krn, Tensor(d!) kvn, Tensor(e!) vcodes, Tensor(f!) vvn, int pos, "
        "Tensor kcent16, Tensor vcent, Tensor vpit, float coeff, float scale, bool causal, Tensor? mask, "
        "ScalarType out_dtype, int workspace) -> Tensor");
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
  m.impl("cache_append", &cache_append);
  m.impl("scores", &scores);
  m.impl("attention", &attention);
  m.impl("cache_attend", &cache_attend);
}

// the same checks on tensor metadata, returning empty outputs of the right shapes
TORCH_LIBRARY_IMPL(tq, Meta, m) {
  m.impl("pack_bits", &pack_bits_meta);
  m.impl("unpack_bits", &unpack_bits_meta);
  m.impl("quantize_pack", &quantize_pack_meta);
  m.impl("dequantize", &dequantize_meta);
  m.impl("compress_keys", &compress_keys_meta);
  m.impl("compress_values", &compress_values_meta);
  m.impl("decompress_values", &decompress_values_meta);
  m.impl("query_prep", &query_prep_meta);
  m.impl("cache_append", &cache_append_meta);
  m.impl("scores", &scores_meta);
  m.impl("attention", &attention_meta);
  m.impl("cache_attend", &cache_attend_meta);
}
