/* innerq_abi.h -- C ABI of libinnerq_hip.so, the MI355X (gfx950) InnerQ KV-cache hot path.
 *
 * The reference (mthcom/innerq) has no native FFI: its boundary is the Python
 * API of src/innerq/quant.py and src/innerq/cache.py, backed by torch ops.
 * Each entry point below replaces the torch work behind one piece of that API
 * (cited per function).  The Python package innerq_amd binds these through
 * ctypes (innerq_amd/_lib.py holds the structures and signatures).
 *
 * Conventions
 *  - All tensor arguments are device pointers (hipMalloc'd or from a torch
 *    CUDA tensor), plain sizes and element strides; no torch types.
 *  - fp16 tensors are passed as `const void*` / `void*` (IEEE binary16).
 *  - `stream` is a hipStream_t passed as `void*` (NULL = default stream).
 *    Every call is asynchronous and stream ordered.  Nothing allocates: the
 *    caller passes any workspace, sized by the matching *_workspace_bytes().
 *  - Every entry point validates its arguments on the host before any launch
 *    and returns 0 (IQ_OK) or a negative IQ_ERR_* code; iq_strerror() names it.
 *  - bits in {2,3,4} (packed-store quantize / dequantize / unpack entry
 *    points also take 1 with IQ_MODE_ASYM: the asym half of 2-bit hybrid
 *    quantization, quant.py:136); group in {32,64,128}; head_dim D in {64,128};
 *    query heads per KV head (Hq/Hkv) in {1,2,4,8}; mode IQ_MODE_ASYM or
 *    IQ_MODE_SYM (quant.py:43-56 'asymmetric' / 'symmetric'); packed stores
 *    also IQ_MODE_HYBRID ('hybrid', bits 2-4, below), which the V side of
 *    iq_av_gemv and of the decode entry points reads.
 *
 * Packed stores (layout owned by this library)
 *  K store, groups along head_dim (quant.py:75-77 channeldim):
 *     codes  uint32 [B, H, t_cap/64, D/G, 64, G*bits/32]
 *     meta   uint16 [B, H, t_cap/64, D/G, 64, M]      M = 2 (scale, zero) asym, 1 (scale) sym
 *  V store, groups along tokens (quant.py:79-81 tokendim):
 *     codes  uint32 [B, H, t_cap/G, D, G*bits/32]
 *     meta   uint16 [B, H, t_cap/G, D, M]
 *  Inside a group, code i occupies bits [bits*i, bits*i+bits) LSB first
 *  (speedtest/benchmark_quantization.cu:25-84); asym stores the code, sym
 *  sign*magnitude + 2^(bits-1) (offset binary, benchmark_quantization.cu:128).
 *  Hybrid stores (quant.py:133-176) keep one representation per group, the
 *  one the reference's mask selects, in b-bit fields and an asym-sized meta
 *  word (M = 2): flag = bit 15 of the scale half (tested as a bit, so a -0.0
 *  scale reads as flagged).  Flag clear: the group's (b-1)-bit asym code,
 *  {scale, zero}.  Flag set: the b-bit sym code (offset binary), {scale |
 *  0x8000, 0}.  The flag is the sign bit of the fp16 scale, as in the
 *  reference's hybrid attn.V proxy (speedtest/benchmark_attn_v.cu:541-636),
 *  which marks its asym groups there.
 */
#ifndef INNERQ_ABI_H
#define INNERQ_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IQ_ABI_VERSION 3
#define IQ_TOKEN_BLOCK 64

enum iq_status {
  IQ_OK = 0,
  IQ_ERR_NULL = -1,       /* a required pointer is NULL */
  IQ_ERR_BITS = -2,       /* bits not in {2,3,4} (1 allowed for asym packed stores) */
  IQ_ERR_GROUP = -3,      /* group not in {32,64,128} or does not divide the grouped axis */
  IQ_ERR_SHAPE = -4,      /* a size is negative / zero where not allowed / unsupported head_dim or GQA ratio */
  IQ_ERR_ALIGN = -5,      /* pointer or stride not aligned as the kernel needs */
  IQ_ERR_WORKSPACE = -6,  /* workspace missing or smaller than *_workspace_bytes() */
  IQ_ERR_MODE = -7,       /* mode not IQ_MODE_ASYM / IQ_MODE_SYM (/ IQ_MODE_HYBRID where taken) */
  IQ_ERR_RANGE = -8,      /* token offset + count exceeds the store capacity */
  IQ_ERR_HIP = -9         /* a HIP launch failed */
};

enum iq_mode {
  IQ_MODE_ASYM = 0,
  IQ_MODE_SYM = 1,
  IQ_MODE_HYBRID = 2,
  /* OR-ed into the mode of a quantize, dequantize, unpack or window-append
   * call (and of a store written that way): the activations - inputs, scales,
   * zero points, signs, 16-bit outputs - are bf16 instead of fp16, and every
   * rounding of the reference's ops is to bf16, as quant.py computes on a
   * bf16 model's tensors (LongBench/pred.py:240 loads the model in bf16).
   * The decode GEMVs and decode attention take fp16 only and refuse a
   * flagged store with IQ_ERR_MODE. */
  IQ_MODE_BF16 = 0x100
};

/* ABI version (IQ_ABI_VERSION) and error names. */
int iq_abi_version(void);
const char* iq_strerror(int status);

/* Byte sizes of a packed store with capacity t_cap tokens (K: t_cap % 64 == 0,
 * V: t_cap % group == 0).  Replaces the int32 code tensors and fp16
 * scale/zero tensors the reference keeps per layer (cache.py:190-210). */
int iq_k_store_bytes(int64_t B, int64_t H, int64_t t_cap, int64_t D, int group, int bits, int mode,
                     int64_t* codes_bytes, int64_t* meta_bytes);
int iq_v_store_bytes(int64_t B, int64_t H, int64_t t_cap, int64_t D, int group, int bits, int mode,
                     int64_t* codes_bytes, int64_t* meta_bytes);

/* Quantize n new tokens x[B,H,n,D] (fp16; element strides sx_b, sx_h, sx_t;
 * D contiguous) with groups along D and write them at token offset t_off of a
 * K store.  Replaces quantize_channeldim_{asym,sym} (quant.py:58-77, 95-115)
 * plus the torch.cat append of cache.py:314-339 (quantize_new_keys).
 * norm: optional fp16 [B,H,D] key-normalization factor; x is divided by it
 * in fp16 first (cache.py:121-126).  Codes are bit-exact to quant.py.
 * IQ_MODE_HYBRID (bits 2-4) quantizes each group both ways, (bits-1)-bit
 * asym and bits-bit sym, and keeps the sym codes where the asym L1 error is
 * the larger (quant.py:133-151; error sums in fp64, see iq_hybrid_mask); it
 * writes the store only (dense outputs NULL).
 * Optional dense outputs (NULL to skip), contiguous:
 *   codes_i32 int32 [B,H,n,D]   exactly quant.py's codes (INT32_MIN for NaN);
 *                               for sym the magnitude codes
 *   scale16 fp16 [B,H,n,D/G], zero16 fp16 [B,H,n,D/G] (asym only),
 *   signs16 fp16 [B,H,n,D] (sym only; torch.sign of the normalized input). */
int iq_quantize_k(const void* x, int64_t sx_b, int64_t sx_h, int64_t sx_t, const void* norm,
                  int B, int H, int n, int D, int group, int bits, int mode,
                  uint32_t* k_codes, uint16_t* k_meta, int64_t t_cap, int64_t t_off,
                  int32_t* codes_i32, void* scale16, void* zero16, void* signs16, void* stream);

/* Quantize n new tokens x[B,H,n,D] with groups along the token axis (n % group
 * == 0, t_off % group == 0) into a V store.  Replaces
 * quantize_tokendim_{asym,sym} (quant.py:79-81, 117-119) plus the append of
 * cache.py:341-365 (quantize_new_values).  Dense outputs as iq_quantize_k but
 * scale16/zero16 are [B,H,n/G,D]. */
int iq_quantize_v(const void* x, int64_t sx_b, int64_t sx_h, int64_t sx_t,
                  int B, int H, int n, int D, int group, int bits, int mode,
                  uint32_t* v_codes, uint16_t* v_meta, int64_t t_cap, int64_t t_off,
                  int32_t* codes_i32, void* scale16, void* zero16, void* signs16, void* stream);

/* Dense dequantized K [B,H,T,D] of store tokens [t0, t0+T) (fp32 c*s + z, or
 * c*s for sym, then * norm when given), written as fp16 (out16) and/or fp32
 * (out32) with element strides so_b, so_h, so_t.  Replaces
 * dequantize_channeldim_{asym,sym} (quant.py:83-87, 121-125) and the
 * unnormalize step of cache.py:241-250 (get_keys_deq).  Hybrid stores: each
 * group as its flag says, i.e. dequantize_hybrid (quant.py:153-176). */
int iq_dequant_k(const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap, const void* norm,
                 int B, int H, int t0, int T, int D, int group, int bits, int mode,
                 void* out16, float* out32, int64_t so_b, int64_t so_h, int64_t so_t, void* stream);

/* Dense dequantized V, as iq_dequant_k (quant.py:89-93, 127-131; cache.py:263-271).
 * t0 and T multiples of group. */
int iq_dequant_v(const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap,
                 int B, int H, int t0, int T, int D, int group, int bits, int mode,
                 void* out16, float* out32, int64_t so_b, int64_t so_h, int64_t so_t, void* stream);

/* Dequantize dense int32 codes (the unpacked form quant.py returns):
 * tensor [outer, n, inner] grouped along n (channeldim: inner = 1; tokendim:
 * n = tokens, inner = head_dim); scale16 fp16 [outer, n/G, inner]; zs16 is the
 * fp16 zero point [outer, n/G, inner] (asym) or the fp16 sign tensor
 * [outer, n, inner] (sym).  out is fp32 (out_f16 = 0) or fp16 (out_f16 = 1),
 * computed in that dtype with one rounding per op.  Replaces
 * dequantize_{channeldim,tokendim}_{asym,sym} (quant.py:83-93, 121-131) for
 * callers holding reference-format codes. */
int iq_dequant_dense(const int32_t* codes, const void* scale16, const void* zs16, int64_t outer, int64_t n,
                     int64_t inner, int group, int mode, int out_f16, void* out, void* stream);

/* Reference-format tensors of store tokens [t0, t0+T): int32 codes [B,H,T,D]
 * (sym: magnitudes), fp16 scale and fp16 zero point (asym) or fp16 sign
 * tensor [B,H,T,D] (sym; 0 where the code is 0, whose sign the packed form
 * does not keep), all contiguous.  K: scale/zero [B,H,T,D/G]; V (t0, T
 * multiples of group): scale/zero [B,H,T/G,D].  Backs the state attributes
 * keys_q / keys_scale_factor / keys_zp_sign (and values_*) of
 * cache.py:190-210 for callers that read them.  Hybrid stores give the raw
 * fields: codes_i32 the stored field (flagged groups: offset binary),
 * scale16 the meta scale half with its flag bit, zs16 the zero half
 * ([.., units] as asym); the caller splits them into quant.py's dicts. */
int iq_unpack_k(const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap, int B, int H, int t0, int T, int D,
                int group, int bits, int mode, int32_t* codes_i32, void* scale16, void* zs16, void* stream);
int iq_unpack_v(const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B, int H, int t0, int T, int D,
                int group, int bits, int mode, int32_t* codes_i32, void* scale16, void* zs16, void* stream);

/* Key normalization factor out16[b,h,d] = fp16(sqrt(max_t |k[b,h,t,d]|)) over
 * T tokens of k (fp16, element strides sk_b, sk_h, sk_t; D contiguous).
 * mode: 0, or IQ_MODE_BF16 for bf16 k and out16 (any other bit:
 * IQ_ERR_MODE).  Replaces key_states.abs().max(dim=-2).values.sqrt()
 * (cache.py:121-126). */
int iq_key_norm_factor(const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_t, int B, int H, int T, int D,
                       int mode, void* out16, void* stream);

/* Hybrid quantization (quant.py:133-176): per group, mask = L1 error of the
 * asym dequantization > L1 error of the sym one, i.e. use the sym codes.
 * x16: the quantizer's fp16 input [BH,T,D] (divided by norm16 [BH,D] in fp16
 * first when non-NULL, as the quantizer does); deq_a, deq_s: fp32 [BH,T,D]
 * dequantizations of the asym (bits-1) and sym (bits) codes.  axis 0: groups
 * along D, mask uint8 [BH,T,D/G]; axis 1: groups along T, mask [BH,T/G,D].
 * Error sums are accumulated in fp64 (the reference sums fp32 in torch's
 * reduction order; exact ties may resolve differently). */
int iq_hybrid_mask(const void* x16, const void* norm16, const float* deq_a, const float* deq_s, int64_t BH, int T,
                   int D, int group, int axis, int mode, uint8_t* mask, void* stream);  /* mode: 0 or IQ_MODE_BF16 */

/* out = mask ? deq_s : deq_a elementwise over [BH,T,D] (mask as produced by
 * iq_hybrid_mask), written as fp32 (out_f16 = 0), fp16 (1) or bf16 (2).
 * Replaces the torch.where of dequantize_hybrid (quant.py:153-176). */
int iq_hybrid_select(const float* deq_a, const float* deq_s, const uint8_t* mask, int64_t BH, int T, int D, int group,
                     int axis, int out_f16, void* out, void* stream);

/* Decode QK^T GEMV over a packed K store: for store tokens [t0, t0+T),
 *   out[b, h, t] = scale * sum_g ( s_g * sum_{i in g} q'[b,h,i] c[t,i] + z_g * sum_{i in g} q'[b,h,i] )
 * with KV head h / (Hq/Hkv) (repeat_kv), q' = q (or q * norm, folding the key
 * normalization of cache.py:249 into the query), fp32 accumulation.
 * q fp16 [B,Hq,D] (strides sq_b, sq_h; D contiguous); out fp32 with strides
 * so_b, so_h (token index contiguous).  Replaces matmul(q, repeat_kv(K_deq)^T)
 * * scaling (TF/models/llama/modeling_llama.py:201-204) over the quantized
 * segment, without materializing K_deq.  workspace: iq_qk_workspace_bytes(). */
int iq_qk_gemv(const void* q, int64_t sq_b, int64_t sq_h, const void* norm,
               const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap,
               int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float scale,
               float* out, int64_t so_b, int64_t so_h, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace for iq_qk_gemv: the query operand records (query pairs in the
 * unpack plan's order plus per-group sums), 16-byte aligned. */
size_t iq_qk_workspace_bytes(int B, int Hq, int D);

/* Workspace for iq_av_gemv: probability operand records plus fp32 split-T
 * partials, 16-byte aligned. */
size_t iq_av_workspace_bytes(int B, int Hq, int T, int D, int group);

/* Decode attn.V GEMV over a packed V store: for store tokens [t0, t0+T)
 * (multiples of group),
 *   out[b, h, d] = sum_g ( s[g,d] * sum_{t in g} p[b,h,t] c[t,d] + z[g,d] * sum_{t in g} p[b,h,t] )
 * p fp16 [B,Hq,T] (strides sp_b, sp_h; tokens contiguous).  Split-T partials
 * go to the workspace and an atomic-free second pass sums them.  If accumulate
 * is nonzero the result is added to out32 (fp32 [B,Hq,D], strides so_*)
 * instead of overwriting it.  out16 (fp16, same strides) optional.  Replaces
 * matmul(p, repeat_kv(V_deq)) (TF/models/llama/modeling_llama.py:210).  A
 * hybrid store (mode IQ_MODE_HYBRID) takes s = |scale| and z = zero, or
 * -2^(bits-1) |scale| for flagged groups: the single pass of
 * speedtest/benchmark_attn_v.cu:541-636 over the exact hybrid format. */
int iq_av_gemv(const void* p, int64_t sp_b, int64_t sp_h,
               const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap,
               int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode,
               float* out32, void* out16, int64_t so_b, int64_t so_h, int accumulate,
               void* workspace, size_t workspace_bytes, void* stream);

/* One K or V segment of a decode step. Segments are laid end to end in token
 * order: sink (fp16) | quantized (store) | recent (fp16), as concatenated by
 * cache.py:235-276.  An fp16 segment is x[B,Hkv,n,D] with strides
 * (s_b, s_h, s_t), D contiguous.  A quantized segment names a store and its
 * first token. */
typedef struct iq_segment {
  const void* dense;          /* fp16 (bf16) segment or NULL */
  int64_t s_b, s_h, s_t;
  int n;                      /* tokens in this segment (0 = absent) */
  const uint32_t* codes;      /* packed store (quantized segment) or NULL */
  const uint16_t* meta;
  int64_t t_cap;
  int t0;                     /* first store token of the segment (any: a sliding
                                 window starts anywhere in the store) */
  int bits, group, mode;      /* mode: the store's; of a dense segment only the
                                 IQ_MODE_BF16 bit (its rows are bf16) */
} iq_segment;

/* One role (K or V) of a layer's decode-step append: the fp16 recent window
 * lives in a caller-owned buffer, and the oldest tokens flush into the
 * layer's packed store. */
typedef struct iq_window {
  void* buf;                  /* fp16 window buffer [B,H,cap,D] (strides s_b, s_h, s_t; D contiguous) */
  int64_t s_b, s_h, s_t;
  int cap;                    /* buffer capacity in tokens */
  int start, n;               /* the window before the call: buffer tokens [start, start + n) */
  const void* x;              /* m new tokens [B,H,m,D] (strides sx_*; D contiguous) */
  int64_t sx_b, sx_h, sx_t;
  int m;                      /* written at buffer tokens start + n .. start + n + m - 1 */
  int flush;                  /* quantize the first `flush` tokens of [window | new] into the store */
  uint32_t* codes;            /* the store, written from token t_off (as iq_quantize_k / _v) */
  uint16_t* meta;
  int64_t t_cap, t_off;
  int bits, group, mode;
  int axis;                   /* 0: groups along head_dim (K store layout), 1: along tokens (V layout) */
  const void* norm;           /* axis 0: fp16 [B,H,D] key normalization factor (x / norm in fp16 first), or NULL */
  int deq_rows;               /* groups of 32 or 64: each flushed token's row of the buffer is
                                 overwritten with its dequantized values (keys: times norm), rounded once
                                 to the activation dtype: the values update() returns for it
                                 (cache.py:235-276) and the reference's attention reads.  The caller may
                                 then attend to the buffer rows before the window as dense rows (tokens
                                 packed in one role whose other role is still in its window).  0: the
                                 rows are left as they were. */
} iq_window;

/* One decode step of a layer's recent windows, both roles in one launch:
 * each role's m new tokens are written into its buffer after the window, and
 * the first `flush` tokens of [window | new] are quantized into its store,
 * bit-exact to iq_quantize_k / iq_quantize_v (asym, sym or hybrid).  The
 * caller then advances the window by `flush` tokens (start += flush, n += m -
 * flush) and the store length by `flush`.  Replaces the torch.cat / slice of
 * update_keys_recent / update_values_recent plus quantize_new_keys /
 * quantize_new_values (cache.py:283-365).  k or v may be NULL (role absent). */
int iq_window_append(const iq_window* k, const iq_window* v, int B, int H, int D, void* stream);

/* Workspace of the decode entry points (no initialization needed). */
size_t iq_decode_workspace_bytes(int B, int Hq, int T, int D);

/* Full decode attention for one layer and one new query token per sequence:
 * logits over K = [ks | kq | kr] (QK^T, scaled), fp32 softmax cast to fp16
 * (TF/models/llama/modeling_llama.py:208), then p.V over V = [vs | vq | vr].
 * k[3] / v[3] are the sink, quantized and recent segments; the token counts of
 * K and V must each sum to T.  norm: optional fp16 [B,Hkv,D] key
 * normalization factor of the quantized K segment; either quantized segment
 * may be a hybrid store (a hybrid K store with K and V of one group size
 * only, key_quantize_mode='hybrid' of cache.py:92-98; else IQ_ERR_MODE).
 * out fp16 [B,Hq,D]
 * (strides so_b, so_h).  Replaces update()'s dense read path (cache.py:278-281,
 * 395) plus the eager attention of TF/models/llama/modeling_llama.py:201-210.
 * A bf16 layer (LongBench/pred.py:240 loads the model in bf16): IQ_MODE_BF16
 * on the mode of every segment that holds tokens (its stores were written
 * with it); q, norm, the dense rows and out are then bf16, the probabilities
 * of the packed range meet V as fp16 and those of the dense tokens as fp32
 * (both finer than the reference's bf16 cast).  Segments that disagree: IQ_ERR_MODE;
 * bf16 K and V of different group sizes: IQ_ERR_MODE (fp16 only). */
int iq_decode_attention(const void* q, int64_t sq_b, int64_t sq_h, const void* norm,
                        const iq_segment* k, const iq_segment* v,
                        int B, int Hq, int Hkv, int T, int D, float scale,
                        void* out, int64_t so_b, int64_t so_h,
                        void* workspace, size_t workspace_bytes, void* stream);

/* The two stages of iq_decode_attention, for callers that schedule them
 * separately (e.g. to time or overlap the split stage); fp16 layers only
 * (_combine cannot tell a bf16 call's output type: IQ_ERR_MODE; a bf16 layer
 * takes the live stages below, whose plan records it).  _splits validates as
 * iq_decode_attention, launches every kernel up to the per-split softmax
 * statistics and unnormalized partial outputs (kept in the workspace) and
 * stores their count in *nsplit (host memory, known at return).  _combine
 * merges nsplit splits from the same workspace into out (fp16 [B,Hq,D],
 * strides so_b, so_h); T and D are those of the _splits call.  Flash-decoding
 * split + combine, atomic-free. */
int iq_decode_attention_splits(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const iq_segment* k,
                               const iq_segment* v, int B, int Hq, int Hkv, int T, int D, float scale,
                               void* workspace, size_t workspace_bytes, int* nsplit, void* stream);
int iq_decode_attention_combine(int nsplit, int B, int Hq, int T, int D, void* out, int64_t so_b, int64_t so_h,
                                void* workspace, size_t workspace_bytes, void* stream);

/* The two stages of iq_decode_attention exactly as that call launches them:
 * the fused kernel leaves a partial only in the split slots its runs own
 * (no empty statistics in the others) and the combine reads only those
 * ("live") slots, so _splits_live launches the same kernel, with the same
 * grid, as the full call (for timing and profiling the decode step's dominant
 * kernel, or for a scheduler that runs its own work between the stages).  A
 * fp16 window short enough for the full call to attend to it after the fused
 * kernel takes the dense slices here instead.  *plan (host memory, known at
 * return) describes the slots; it is opaque: pass it unchanged to
 * _combine_live with the same workspace, B, Hq, T and D. */
typedef struct iq_split_plan {
  int nsplit;   /* split slots written */
  int nsf;      /* the first nsf of them belong to the packed range */
  int grid;     /* workgroups of the fused kernel (0: not launched) */
  int nrep;     /* query heads per KV head */
  int pair_e0;  /* the fused kernel's work partition */
  int bf16;     /* the output's dtype: 1 bf16, 0 fp16 */
  int reserved[2];
} iq_split_plan;
int iq_decode_attention_splits_live(const void* q, int64_t sq_b, int64_t sq_h, const void* norm,
                                    const iq_segment* k, const iq_segment* v,
                                    int B, int Hq, int Hkv, int T, int D, float scale,
                                    void* workspace, size_t workspace_bytes, iq_split_plan* plan, void* stream);
int iq_decode_attention_combine_live(const iq_split_plan* plan, int B, int Hq, int T, int D, void* out,
                                     int64_t so_b, int64_t so_h, void* workspace, size_t workspace_bytes,
                                     void* stream);

/* iq_decode_attention without the workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc).  It has no counterpart in the
 * reference.  Arguments, results and errors are those of iq_decode_attention;
 * the workspace is a library-owned device array of
 * iq_decode_noalloc_max_bytes() bytes (64 MiB) per GPU, held until the process
 * ends, and a call whose iq_decode_workspace_bytes(B, Hq, T, D) exceeds it
 * returns IQ_ERR_WORKSPACE before any launch.  The call allocates nothing.
 * Every call on one GPU uses the same array: calls that overlap on one GPU
 * (concurrent streams, threads) race and must be serialized by the caller. */
size_t iq_decode_noalloc_max_bytes(void);
int iq_decode_attention_noalloc(const void* q, int64_t sq_b, int64_t sq_h, const void* norm,
                                const iq_segment* k, const iq_segment* v,
                                int B, int Hq, int Hkv, int T, int D, float scale,
                                void* out, int64_t so_b, int64_t so_h, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INNERQ_ABI_H */
