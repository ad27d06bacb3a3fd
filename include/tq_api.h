/*
 * tq_api.h -- C ABI of the MI355X (gfx950) TurboQuant KV-compression library.
 *
 * Every entry point takes plain device pointers, element counts and strides,
 * plus the HIP stream to launch on (passed as `void*`, i.e. a hipStream_t;
 * NULL is the default stream).  Calls are asynchronous on that stream, allocate
 * no device memory, and return TQ_OK (0) or a negative error code; the message
 * for the last failure on the calling thread is returned by tq_last_error().
 *
 * Conventions shared by all entry points
 *   - "f16" buffers hold IEEE binary16 bit patterns (uint16_t), "bf16" buffers
 *     bfloat16 bit patterns.  Norm planes (rn, vn) are always f16, as in the
 *     reference's packed format.
 *   - Packed code rows use the reference bit layout: code i of a row occupies
 *     global bits [i*b, i*b+b) of the row, least-significant bit first; bit k
 *     lives in byte k/8 at bit position k%8.  A row of d b-bit codes takes
 *     ceil(d*b/8) bytes (tq_out_cols).
 *   - A compressed key record (one row = one (batch, kv-head, position)) is the
 *     four planes  codes u8[ceil(d*(bits-1)/8)], signs u8[d/8], rn f16, vn f16;
 *     a value record is codes u8[ceil(d*bits/8)], vn f16.  Planes are stored
 *     structure-of-arrays, rows contiguous in (batch, head, position) order.
 *   - A "split" d x d matrix W is f16 [2][d][d] row-major: hi = f16(1024*W),
 *     lo = f16(1024*W - hi).  The kernels run d x d products on f16 MFMA and
 *     recover f32 accuracy from the (hi, lo) pair.
 *   - Head dims d: every multiple of 8 from 8 to 256 (packed rows of d*b/8
 *     bytes, not dword aligned in general); others return TQ_EUNSUPPORTED.
 *
 * Reference: SrzStephen/transformers-turboquant, Python package
 * src/turboquant_pytorch (file:line citations below are relative to it).
 */
#ifndef TQ_API_H
#define TQ_API_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of caller-provided activations */
enum tq_dtype { TQ_F32 = 0, TQ_F16 = 1, TQ_BF16 = 2 };

/* status codes */
enum tq_status {
  TQ_OK = 0,
  TQ_EINVAL = -1,      /* bad argument (shape, bits, alignment, null pointer) */
  TQ_EUNSUPPORTED = -2,/* valid but not built (e.g. head_dim not a multiple of 8 or above 256) */
  TQ_EHIP = -3         /* HIP runtime error at launch */
};

/* Library version (major*10000 + minor*100 + patch).  Utility; no counterpart in the
 * reference (a Python package). */
int tq_version(void);

/* Message for the most recent failing call on this thread ("" if none).  Utility: the
 * reference raises Python exceptions; the bindings turn this message into one. */
const char* tq_last_error(void);

/* Bytes needed for d codes of b bits: ceil(d*b/8).
 * Replaces kernels/bit_ops.py:162-164 (_out_cols). */
int64_t tq_out_cols(int64_t d, int32_t b);

/* Pack int32 codes idx[n, d] (row stride ld_idx elements) into out[n, ld_out]
 * bytes; each code is masked to b bits (1 <= b <= 8).  Writes exactly
 * tq_out_cols(d, b) bytes per row.
 * Replaces kernels/bit_ops.py:173-204 (pack_bits; Triton kernel :56-109,
 * fallback :243-286). */
int tq_pack_bits(const int32_t* idx, int64_t n, int32_t d, int64_t ld_idx,
                 int32_t b, uint8_t* out, int64_t ld_out, void* stream);

/* Inverse of tq_pack_bits: packed[n, ld_in] -> int32 out[n, ld_out] (d codes).
 * Replaces kernels/bit_ops.py:206-235 (unpack_bits; kernel :111-155,
 * fallback :288-326). */
int tq_unpack_bits(const uint8_t* packed, int64_t n, int32_t d, int64_t ld_in,
                   int32_t b, int32_t* out, int64_t ld_out, void* stream);

/* Lloyd-Max quantize + pack: code = #{ j : bounds[j] < y } (torch.searchsorted,
 * side='left') against the 2^b_eff - 1 sorted f32 boundaries, packed with
 * b_eff bits.  y is f32 [n, ld_y].
 * Replaces kernels/quantize.py:201-247 (lloyd_max_quantize; fallback
 * :299-339). */
int tq_quantize_pack(const float* y, int64_t n, int32_t d, int64_t ld_y,
                     const float* bounds, int32_t b_eff, uint8_t* out,
                     int64_t ld_out, void* stream);

/* Unpack b-bit codes and look them up in f16 centroids[2^b] -> f16 out[n, ld_out].
 * Replaces kernels/quantize.py:249-290 (lloyd_max_dequantize; fallback
 * :341-369). */
int tq_dequantize(const uint8_t* packed, int64_t n, int32_t d, int64_t ld_in,
                  const uint16_t* centroids_f16, int32_t b, uint16_t* out_f16,
                  int64_t ld_out, void* stream);

/* Fused key compression of the n = B*H*S rows of x[B, H, S, d] (element
 * strides sxb, sxh, sxs; unit stride on d; dtype tq_dtype), rows taken in
 * (b, h, s) order:
 *   vn = ||x||, y = (x / (vn + 1e-8)) Pi^T, codes = searchsorted(bounds, y),
 *   k_mse = (f16(C)[codes] Pi) * vn, r = x - k_mse, rn = ||r||,
 *   proj = r S^T, signs = (proj >= 0),
 * writing codes u8[n, ceil(d*b_eff/8)], signs u8[n, d/8], rn f16[n], vn f16[n].
 * The residual is formed in the rotated domain, u = r Pi^T = (vn + 1e-8) y -
 * vn f16(C)[codes], so rn = ||u|| and proj = u S_eff^T with S_eff = S Pi^T: the
 * same quantities up to f32 rounding, one d x d product fewer.
 * pi_split: the rotation Pi[d,d] (row-major) as a split matrix; seff_split: the
 * split of the f32 product S_eff = S Pi^T (S the QJL matrix); centroids/bounds are
 * f32 [2^b_eff], [2^b_eff - 1].
 * y_out / proj_out (nullable) receive the f32 rotated rows and projections the
 * codes and signs were taken from.
 * Replaces compressors.py:99-138 (TurboQuantCompressorV2.compress, packed
 * branch; k_mse uses f16-rounded centroids as at :120-122). */
int tq_compress_keys(const void* x, int32_t dtype, int32_t B, int32_t H,
                     int32_t S, int32_t d, int64_t sxb, int64_t sxh, int64_t sxs,
                     const uint16_t* pi_split, const uint16_t* seff_split,
                     const float* centroids, const float* bounds, int32_t b_eff,
                     uint8_t* codes, uint8_t* signs, uint16_t* rn, uint16_t* vn,
                     float* y_out, float* proj_out, void* stream);

/* Fused value compression of x[B, H, S, d] (strides as tq_compress_keys):
 * vn = ||x||, y = (x/(vn+1e-8)) Pi^T,
 * codes = searchsorted(bounds, y) packed with b bits, vn f16.
 * Replaces compressors.py:271-287 (TurboQuantCompressorMSE.compress, packed
 * branch). */
int tq_compress_values(const void* x, int32_t dtype, int32_t B, int32_t H,
                       int32_t S, int32_t d, int64_t sxb, int64_t sxh, int64_t sxs,
                       const uint16_t* pi_split,
                       const float* bounds, int32_t b, uint8_t* codes,
                       uint16_t* vn, float* y_out, void* stream);

/* Value decompression out[n, d] (dtype tq_dtype, row stride ld_out) =
 * (centroids[codes] Pi) * vn with f32 centroids.  pit_split is Pi^T split
 * as in tq_compress_keys.
 * Replaces compressors.py:297-317 (TurboQuantCompressorMSE.decompress; the
 * reference's packed branch multiplies an f16 tensor by an f32 Pi and raises,
 * so this follows its f32 branch :311-317 on packed codes). */
int tq_decompress_values(const uint8_t* codes, const uint16_t* vn, int64_t n,
                         int32_t d, const uint16_t* pit_split,
                         const float* centroids, int32_t b, void* out,
                         int32_t out_dtype, int64_t ld_out, void* stream);

/* Query preparation for compressed-domain scoring of q[B, Hq, Sq, d]
 * (element strides sqb, sqh, sqs; unit stride on d):
 *   q_rot  = f16(q Pi^T)                      -> f16 [B, Hq, Sq, d] contiguous
 *   q_proj = q_rot S_eff^T, S_eff f16[m=d, d] -> f32 [B, Hq, Sq, d] contiguous
 * q_proj is the f32 accumulation of the exact f16 products, as the reference's
 * fp32 projection; its buffer must be 16-byte aligned for the fast path.
 * Replaces compressors.py:186-189 (q_rot, S_eff) and the per-query projection
 * of kernels/attention.py:155-167 (fallback :453). */
int tq_query_prep(const void* q, int32_t dtype, int32_t B, int32_t Hq,
                  int32_t Sq, int32_t d, int64_t sqb, int64_t sqh, int64_t sqs,
                  const uint16_t* pi_split, const uint16_t* s_eff_f16,
                  uint16_t* q_rot, float* q_proj, void* stream);

/* Materialised asymmetric scores out f32 [B, Hq, Sq, Sk] (contiguous):
 *   out = vn * <q_rot, C[codes]> + coeff * rn * <q_proj, 2*sign - 1>
 * from q_rot f16 / q_proj f32 [B, Hq, Sq, d] (tq_query_prep; q_proj enters at f32
 * grade: as 24-bit fixed point per query in the bit-plane decode kernels, as f16
 * hi + lo elsewhere) and key planes of
 * [B, Hkv, Sk] rows; query head h reads kv head h / (Hq / Hkv).
 * centroids_f16 holds the 2^(bits-1) key centroids.  bits is the total key
 * bit budget (codes use bits-1 bits), as in the reference.
 * Replaces kernels/attention.py:274-372 (asymmetric_attention_scores; fallback
 * :380-461) and compressors.py:178-200. */
int tq_attention_scores(const uint16_t* q_rot, const float* q_proj,
                        const uint8_t* key_codes, const uint8_t* key_signs,
                        const uint16_t* key_rn, const uint16_t* key_vn,
                        const uint16_t* centroids_f16, int32_t B, int32_t Hq,
                        int32_t Hkv, int32_t Sq, int32_t Sk, int32_t d,
                        int32_t bits, float coeff, float* out, void* stream);

/* Fused compressed-domain attention (one attention layer's tail).  q_proj f32 as in
 * tq_attention_scores, taken at f32 grade by every kernel:
 *   s   = (vn*<q_rot,Ck[codes]> + coeff*rn*<q_proj, 2*sign-1>) * scale
 *         (+ mask[b, h, i, j] if mask != NULL) (causal: key j > i + Sk - Sq dropped)
 *   p   = softmax_j(s)                    (f32, online)
 *   o   = (sum_j p_j * vnv_j * Cv[vcodes_j]) Pi_v    (Cv: f32 value centroids)
 * out[b, i, h, :] in out_dtype with element strides (sob, soh, sos).
 * workspace / workspace_bytes: scratch of at least tq_attention_workspace_size
 * bytes (16-byte aligned) enables the split-K paths for few-query shapes.
 * mask: f32 additive, element strides (smb, smh, smq, smk) (0 = broadcast).
 * val_pi_split: the value compressor's Pi^T split as in tq_compress_keys.
 * Replaces the family forward tail families/qwen2.py:105-117 (same in
 * llama.py:222-233, deepseek.py, gpt2.py:90-110): compress -> scores -> /sqrt(d)
 * -> +mask -> softmax -> decompress(V) -> P V. */
int tq_attention_fwd(const uint16_t* q_rot, const float* q_proj,
                     const uint8_t* key_codes, const uint8_t* key_signs,
                     const uint16_t* key_rn, const uint16_t* key_vn,
                     const uint16_t* key_centroids_f16, int32_t bits,
                     const uint8_t* val_codes, const uint16_t* val_vn,
                     const float* val_centroids, int32_t val_bits,
                     const uint16_t* val_pit_split, int32_t B, int32_t Hq,
                     int32_t Hkv, int32_t Sq, int32_t Sk, int32_t d,
                     float coeff, float scale, int32_t causal,
                     const float* mask, int64_t smb, int64_t smh, int64_t smq,
                     int64_t smk, void* out, int32_t out_dtype, int64_t sob,
                     int64_t soh, int64_t sos, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* tq_attention_scores / tq_attention_fwd over key and value planes whose
 * (batch, kv head) planes start kv_stride rows apart (kv_stride >= Sk; 0 means
 * Sk): the first Sk rows of each plane are attended.  This is the layout of a
 * compressed KV cache that preallocates kv_stride positions per head and
 * appends tokens in place.  No counterpart in the reference, which disables
 * the KV cache (patch.py:81); the tensor-level concept is
 * turboquant.py:199-286 (TurboQuantKVCache). */
int tq_attention_scores_kv(const uint16_t* q_rot, const float* q_proj,
                           const uint8_t* key_codes, const uint8_t* key_signs,
                           const uint16_t* key_rn, const uint16_t* key_vn,
                           const uint16_t* centroids_f16, int32_t B, int32_t Hq,
                           int32_t Hkv, int32_t Sq, int32_t Sk,
                           int64_t kv_stride, int32_t d, int32_t bits,
                           float coeff, float* out, void* stream);
int tq_attention_fwd_kv(const uint16_t* q_rot, const float* q_proj,
                        const uint8_t* key_codes, const uint8_t* key_signs,
                        const uint16_t* key_rn, const uint16_t* key_vn,
                        const uint16_t* key_centroids_f16, int32_t bits,
                        const uint8_t* val_codes, const uint16_t* val_vn,
                        const float* val_centroids, int32_t val_bits,
                        const uint16_t* val_pit_split, int32_t B, int32_t Hq,
                        int32_t Hkv, int32_t Sq, int32_t Sk, int64_t kv_stride,
                        int32_t d, float coeff, float scale, int32_t causal,
                        const float* mask, int64_t smb, int64_t smh, int64_t smq,
                        int64_t smk, void* out, int32_t out_dtype, int64_t sob,
                        int64_t soh, int64_t sos, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* Compressed-cache append: compress the S new keys and values of each (batch, kv head),
 * k / v [B, H, S, d] (element strides; unit stride on d), into rows [pos, pos + S) of
 * cache planes that hold `capacity` positions per (batch, kv head) -- key_codes
 * u8 [B, H, capacity, ceil(d*key_code_bits/8)], key_signs u8 [.., d/8], key_rn / key_vn
 * f16 [B, H, capacity], val_codes u8 [.., ceil(d*val_bits/8)], val_vn f16 [B, H, capacity],
 * the layout tq_attention_fwd_kv reads with kv_stride = capacity -- and, when q is not
 * NULL, prepare the S new query rows q [B, Hq, S, d] as tq_query_prep does (q_rot f16 /
 * q_proj f32 [B, Hq, S, d]).  Operands as in tq_compress_keys / tq_compress_values /
 * tq_query_prep (key_code_bits = bits - 1 for bits-bit keys); every written row equals
 * those entry points' output for the same input row bit for bit.  At head_dim 64 / 128 with
 * key_code_bits = val_bits - 1 (val_bits 2-4) the three run in one launch.
 * No counterpart in the reference, which disables the KV cache and recompresses the whole
 * sequence every step (patch.py:81); a decoding step calls this once per layer. */
int tq_cache_append(const void* k, const void* v, int32_t dtype, int32_t B,
                    int32_t H, int32_t S, int32_t d, int64_t skb, int64_t skh,
                    int64_t sks, int64_t svb, int64_t svh, int64_t svs,
                    const uint16_t* key_pi_split, const uint16_t* key_seff_split,
                    const float* key_centroids, const float* key_bounds,
                    int32_t key_code_bits, const uint16_t* val_pi_split,
                    const float* val_bounds, int32_t val_bits, uint8_t* key_codes,
                    uint8_t* key_signs, uint16_t* key_rn, uint16_t* key_vn,
                    uint8_t* val_codes, uint16_t* val_vn, int64_t capacity,
                    int64_t pos, const void* q, int32_t Hq, int64_t sqb,
                    int64_t sqh, int64_t sqs, const uint16_t* key_s_eff_f16,
                    uint16_t* q_rot, float* q_proj, void* stream);

/* Bytes of caller-provided device workspace tq_attention_fwd uses to split the keys of a
 * few-query shape: the split-K decode kernels (head_dim 64 or 128, bits 2-4, at most 16
 * (query row, query head) pairs per kv head, value bits == key bits) or, for other
 * few-query shapes whose kv head's columns fit one block (any head dim, other value
 * bits, larger groups) with at least 512 keys, the fused kernels split over keys plus a
 * merge; the larger of the two, 0 when neither applies.  With a smaller or NULL
 * workspace tq_attention_fwd runs unsplit.  No counterpart in the reference, whose
 * attention is never split over keys. */
int64_t tq_attention_workspace_size(int32_t B, int32_t Hq, int32_t Hkv,
                                    int32_t Sq, int32_t Sk, int32_t d,
                                    int32_t bits);

/* Size of the library's per-GPU scratch array used by tq_attention_fwd_kv_noalloc. */
#define TQ_NOALLOC_SCRATCH_BYTES (16LL << 20)

/* tq_attention_fwd_kv with no caller workspace and no device allocation: the split-K
 * paths keep their per-split partials in a library-owned device array of
 * TQ_NOALLOC_SCRATCH_BYTES (16 MiB) per GPU, held from the library's first use of that GPU
 * until the process ends.  Same arguments, results and error behaviour as
 * tq_attention_fwd_kv otherwise (bit-identical outputs for the same inputs).
 *   - Decode-kernel shapes whose partials need more than the array (more than 16 MiB of
 *     (batch, kv head, split) records) fail with TQ_EINVAL and a message; the other split
 *     path runs unsplit when its partials do not fit; shapes off both paths use none.
 *   - Every call on one GPU shares that GPU's array, which keeps the last call's contents:
 *     calls that overlap in time on one GPU (other streams, other host threads) race.
 *     Calls queued on one stream are ordered and safe.
 *   - Calls no hipMalloc / hipFree or other allocating routine.
 * No counterpart in the reference.  For callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid allocation. */
int tq_attention_fwd_kv_noalloc(const uint16_t* q_rot, const float* q_proj,
                                const uint8_t* key_codes, const uint8_t* key_signs,
                                const uint16_t* key_rn, const uint16_t* key_vn,
                                const uint16_t* key_centroids_f16, int32_t bits,
                                const uint8_t* val_codes, const uint16_t* val_vn,
                                const float* val_centroids, int32_t val_bits,
                                const uint16_t* val_pit_split, int32_t B, int32_t Hq,
                                int32_t Hkv, int32_t Sq, int32_t Sk, int64_t kv_stride,
                                int32_t d, float coeff, float scale, int32_t causal,
                                const float* mask, int64_t smb, int64_t smh, int64_t smq,
                                int64_t smk, void* out, int32_t out_dtype, int64_t sob,
                                int64_t soh, int64_t sos, void* stream);

/* TQ_NOALLOC_SCRATCH_BYTES as built into the library.  Utility; no reference counterpart. */
int64_t tq_noalloc_scratch_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* TQ_API_H */
