// Quantize-on-append and dense dequantization kernels (gfx950).
//
// Quantization restates src/innerq/quant.py op by op: every fp16 op of the
// reference (sub, division by the int level count, division by the scale) is
// an fp32 op rounded to fp16 with round-to-nearest-even (exact for + - * /
// because fp32 has more than 2*11+2 significand bits), the clamp keeps NaN,
// the rounding is half-to-even (v_rndne_f32), and NaN becomes INT32_MIN in the
// dense int32 output (0 in the packed field).  Division is IEEE (hipcc's
// default correctly rounded fp32 divide; no fast-math anywhere in this build).
//
// One thread owns one quantization group: the group's min/max (or max |x|)
// is a serial loop over G registers, which keeps the rounding order trivially
// identical to the reference and needs no cross-lane traffic.  Appends are a
// few hundred groups per decode step and prefill is a streaming pass, so this
// kernel is latency- resp. HBM-bound either way.
#include "iq_common.h"
#include "iq_device.h"

using namespace iq;

namespace {

constexpr int32_t I32_MIN = (int32_t)0x80000000u;

// groups of a K quantize call up to which it runs one lane per value
// (quant_k_lane_kernel); past it, one thread per group (~2x fewer
// instructions per value, and enough threads to fill the device)
constexpr int64_t LANE_MAX_GROUPS = 65536;

struct QuantOut {
  uint32_t* codes;     // packed store codes (or null)
  uint16_t* meta;      // packed store meta
  int64_t cap_units;   // K: t_cap/64 blocks, V: t_cap/G groups
  int64_t t_off;       // first token written in the store
  int32_t* codes_i32;  // dense outputs (optional)
  uint16_t* scale16;
  uint16_t* zero16;
  uint16_t* signs16;
};

__device__ __forceinline__ bool is_nan(float v) { return v != v; }

// clamp(y, 0, L) keeping NaN, then half-to-even round.  Returns the dense
// int32 code (INT32_MIN for NaN, as torch's float->int32 on x86).
__device__ __forceinline__ int32_t code_of(float y, float L) {
  if (is_nan(y)) return I32_MIN;
  y = fminf(fmaxf(y, 0.0f), L);
  return (int32_t)rintf(y);
}

// Group statistics and per-element codes of the two quantizers, one rounding
// to the activation dtype (fp16, or bf16 with bf) per reference op (runtime
// bit width; the templates below pass a constant).
// asym (quant.py:66-71): scale of b-bit codes from the group's min and max
__device__ __forceinline__ float asym_scale_b(float mn, float mx, int bits, bool bf = false) {
  return round_act(round_act(mx - mn, bf) / float((1 << bits) - 1), bf);    // quant.py:68
}
__device__ __forceinline__ int32_t asym_code_b(float x, float mn, float s, int bits, bool bf = false) {
  return code_of(round_act(round_act(x - mn, bf) / s, bf), float((1 << bits) - 1));  // quant.py:69-71
}
// sym (quant.py:104-109): scale of b-bit codes (one bit is the sign)
__device__ __forceinline__ float sym_scale_b(float mx, int bits, bool bf = false) {
  return round_act(mx / float((1 << (bits - 1)) - 1), bf);              // quant.py:107
}
__device__ __forceinline__ int32_t sym_code_b(float x, float s, int bits, bool bf = false) {
  return code_of(round_act(fabsf(x) / s, bf), float((1 << (bits - 1)) - 1));  // quant.py:108-109
}
__device__ __forceinline__ float sign_of(float x) { return x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f); }  // torch.sign
// stored fields: the asym code (0 for NaN); sym sign*magnitude + 2^(b-1)
__device__ __forceinline__ uint32_t asym_field_b(int32_t c, int bits) {
  return (c == I32_MIN) ? 0u : (uint32_t(c) & ((1u << bits) - 1u));
}
__device__ __forceinline__ uint32_t sym_field_b(int32_t c, float sg, int bits) {
  const int32_t sc = (c == I32_MIN) ? 0 : (sg > 0.f ? c : (sg < 0.f ? -c : 0));
  return uint32_t(sc + (1 << (bits - 1))) & ((1u << bits) - 1u);  // offset binary
}

template <int BITS, int G>
__device__ __forceinline__ void asym_params(const float* v, float& s, float& mn) {
  float mx = v[0];
  bool nan = false;
  mn = v[0];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    nan |= is_nan(v[i]);
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
  }
  if (nan) { mn = __builtin_nanf(""); mx = mn; }
  s = asym_scale_b(mn, mx, BITS);
}
template <int BITS>
__device__ __forceinline__ int32_t asym_code(float x, float mn, float s) { return asym_code_b(x, mn, s, BITS); }
template <int BITS, int G>
__device__ __forceinline__ float sym_scale(const float* v) {
  float mx = 0.f;
  bool nan = false;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    nan |= is_nan(v[i]);
    mx = fmaxf(mx, fabsf(v[i]));
  }
  if (nan) mx = __builtin_nanf("");
  return sym_scale_b(mx, BITS);
}
template <int BITS>
__device__ __forceinline__ int32_t sym_code(float x, float s) { return sym_code_b(x, s, BITS); }
template <int BITS>
__device__ __forceinline__ uint32_t asym_field(int32_t c) { return asym_field_b(c, BITS); }
template <int BITS>
__device__ __forceinline__ uint32_t sym_field(int32_t c, float sg) { return sym_field_b(c, sg, BITS); }

// x / s in fp32, rounded to nearest, for a finite x >= 0 and a finite s > 0
// that are fp16 values, given r = RN32(1 / s): q0 = RN32(x r), then one
// correction by the residual x - q0 s, which an fma gives exactly
// (Markstein's division step), so the result is RN32(x / s) and its fp16
// rounding is the reference's fp16 division.  One divide per group and three
// operations per value instead of a divide per value; checked over every
// such pair of fp16 operands (tests/test_quant_division.py).
__device__ __forceinline__ float div_rcp(float x, float s, float r) {
  const float q0 = __fmul_rn(x, r);
  return __fmaf_rn(__fmaf_rn(-q0, s, x), r, q0);
}

// Quantize G values held as fp32 copies of fp16 numbers.  fields[] receives
// the b-bit stored field, codes[] the dense reference code, sgn[] the sign.
// A group whose scale is finite and positive (every group but the constant,
// NaN and infinite ones, which divide per value) divides through its
// reciprocal: its dividends x - min (asym) and |x| (sym) are finite and >= 0.
template <int BITS, int G>
__device__ __forceinline__ void quantize_group(const float* v, bool sym, uint32_t* fields, int32_t* codes,
                                               float* sgn, float& s_out, float& z_out) {
  if (!sym) {
    float s, mn;
    asym_params<BITS, G>(v, s, mn);
    if (s > 0.f && s < INFINITY) {
      constexpr float L = float((1 << BITS) - 1);
      const float r = __fdiv_rn(1.0f, s);
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int32_t c = code_of(round_f16(div_rcp(round_f16(v[i] - mn), s, r)), L);  // quant.py:69-71
        codes[i] = c;
        fields[i] = asym_field<BITS>(c);
        sgn[i] = 0.f;
      }
    } else {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int32_t c = asym_code<BITS>(v[i], mn, s);
        codes[i] = c;
        fields[i] = asym_field<BITS>(c);
        sgn[i] = 0.f;
      }
    }
    s_out = s;
    z_out = mn;
  } else {
    const float s = sym_scale<BITS, G>(v);
    if (s > 0.f && s < INFINITY) {
      constexpr float L = float((1 << (BITS - 1)) - 1);
      const float r = __fdiv_rn(1.0f, s);
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int32_t c = code_of(round_f16(div_rcp(fabsf(v[i]), s, r)), L);  // quant.py:108-109
        const float sg = sign_of(v[i]);
        codes[i] = c;
        fields[i] = sym_field<BITS>(c, sg);
        sgn[i] = sg;
      }
    } else {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int32_t c = sym_code<BITS>(v[i], s);
        const float sg = sign_of(v[i]);
        codes[i] = c;
        fields[i] = sym_field<BITS>(c, sg);
        sgn[i] = sg;
      }
    }
    s_out = s;
    z_out = 0.f;
  }
}

// Hybrid (quant.py:133-151): the group quantized both ways, (b-1)-bit asym
// and b-bit sym; their fp32 dequantizations as the reference computes them
// (asym c*s + z, sym c*s*sign, a NaN code as INT32_MIN: quant.py:83-93,
// 121-131); the sym codes are kept iff the asym L1 error is the larger.  The
// error sums are accumulated in fp64 (as iq_hybrid_mask).  fields[] gets the
// kept b-bit fields, mw the meta dword {scale | flag << 15, zero}.
template <int BITS, int G>
__device__ __forceinline__ void quantize_group_hybrid(const float* v, uint32_t* fields, uint32_t& mw) {
  float sa, za;
  asym_params<BITS - 1, G>(v, sa, za);
  const float ss = sym_scale<BITS, G>(v);
  double ea = 0.0, es = 0.0;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const float da = __fadd_rn(__fmul_rn(float(asym_code<BITS - 1>(v[i], za, sa)), sa), za);
    const float ds = __fmul_rn(__fmul_rn(float(sym_code<BITS>(v[i], ss)), ss), sign_of(v[i]));
    ea += double(fabsf(__fsub_rn(da, v[i])));
    es += double(fabsf(__fsub_rn(ds, v[i])));
  }
  const bool sym = ea > es;
#pragma unroll
  for (int i = 0; i < G; ++i)
    fields[i] = sym ? sym_field<BITS>(sym_code<BITS>(v[i], ss), sign_of(v[i]))
                    : asym_field<BITS>(asym_code<BITS - 1>(v[i], za, sa));
  const uint32_t sh = __half_as_ushort(__float2half_rn(sym ? ss : sa));
  mw = sym ? (sh | HYB_FLAG) : ((sh & 0x7fffu) | (uint32_t(__half_as_ushort(__float2half_rn(za))) << 16));
}

template <int BITS, int G>
__device__ __forceinline__ void pack_fields(const uint32_t* f, uint32_t* w) {
  constexpr int W = G * BITS / 32;
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = 0u;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    constexpr int dummy = 0;
    (void)dummy;
    const int bit = BITS * i;
    const int wi = bit >> 5, o = bit & 31;
    w[wi] |= f[i] << o;
    if (o + BITS > 32) w[wi + 1] |= f[i] >> (32 - o);
  }
}

// one group's fields and meta into the store: W code words at unit * W;
// meta one fp16 scale (sym) or one {scale, zero} dword (asym, hybrid)
template <int BITS, int G>
__device__ __forceinline__ void store_group(const QuantOut& o, int64_t unit, const uint32_t* f, bool half_meta,
                                            uint32_t mw) {
  constexpr int W = G * BITS / 32;
  uint32_t w[W];
  pack_fields<BITS, G>(f, w);
  uint32_t* cp = o.codes + unit * W;
#pragma unroll
  for (int j = 0; j < W; ++j) cp[j] = w[j];
  if (half_meta) o.meta[unit] = uint16_t(mw);
  else reinterpret_cast<uint32_t*>(o.meta)[unit] = mw;
}

__device__ __forceinline__ uint32_t meta_word(float s, float z, bool bf = false) {
  return uint32_t(f2act(s, bf)) | (uint32_t(f2act(z, bf)) << 16);
}

template <int BITS, int G>
__device__ __forceinline__ void unpack_fields(const uint32_t* w, bool sym, int32_t* c) {
  constexpr uint32_t FMASK = (1u << BITS) - 1u;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int bit = BITS * i;
    const int wi = bit >> 5, o = bit & 31;
    uint32_t f = w[wi] >> o;
    if (o + BITS > 32) f |= w[wi + 1] << (32 - o);
    f &= FMASK;
    int32_t v = int32_t(f);
    if (sym) v -= (1 << (BITS - 1));  // offset binary
    c[i] = v;
  }
}

// ---- K: groups along head_dim, one thread per (b, h, t, g) ----------------
// HYB: a hybrid store (store only, no dense outputs)
template <int BITS, int G, bool DENSE, bool HYB = false>
__global__ __launch_bounds__(256) void quant_k_kernel(const uint16_t* __restrict__ x, int64_t sxb, int64_t sxh,
                                                      int64_t sxt, const uint16_t* __restrict__ norm, int B,
                                                      int H, int n, int D, int sym, QuantOut o) {
  const int ng = D / G;
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = int64_t(B) * H * n * ng;
  if (gid >= total) return;
  const int g = int(gid % ng);
  int64_t r = gid / ng;
  const int t = int(r % n);
  r /= n;
  const int h = int(r % H);
  const int b = int(r / H);

  const uint16_t* xp = x + b * sxb + h * sxh + t * sxt + g * G;
  float v[G];
#pragma unroll
  for (int i = 0; i < G; i += 8) {
    const uint4 u = *reinterpret_cast<const uint4*>(xp + i);
    const uint32_t uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i + 2 * j] = h2f(uint16_t(uu[j] & 0xffffu));
      v[i + 2 * j + 1] = h2f(uint16_t(uu[j] >> 16));
    }
  }
  if (norm) {  // cache.py:125  key_states / key_normalization_factor (fp16)
    const uint16_t* np_ = norm + (int64_t(b) * H + h) * D + g * G;
#pragma unroll
    for (int i = 0; i < G; ++i) v[i] = round_f16(v[i] / h2f(np_[i]));
  }
  const int64_t bh = int64_t(b) * H + h;
  const int64_t tt = o.t_off + t;
  const int64_t unit = ((bh * o.cap_units + tt / TOKEN_BLOCK) * ng + g) * TOKEN_BLOCK + tt % TOKEN_BLOCK;
  uint32_t f[G];
  if constexpr (HYB) {
    if constexpr (BITS >= 2) {
      uint32_t mw;
      quantize_group_hybrid<BITS, G>(v, f, mw);
      store_group<BITS, G>(o, unit, f, false, mw);
    }
    return;
  }
  int32_t c[G];
  float sg[G];
  float s, z;
  quantize_group<BITS, G>(v, sym != 0, f, c, sg, s, z);
  if (o.codes) store_group<BITS, G>(o, unit, f, sym != 0, meta_word(s, z));
  if constexpr (DENSE) {  // the reference-format outputs (quant.py API)
    const int64_t row_el = (bh * n + t) * D + g * G;
    if (o.codes_i32) {
#pragma unroll
      for (int i = 0; i < G; ++i) o.codes_i32[row_el + i] = c[i];
    }
    if (o.signs16) {
#pragma unroll
      for (int i = 0; i < G; ++i) o.signs16[row_el + i] = __half_as_ushort(__float2half_rn(sg[i]));
    }
    const int64_t red = (bh * n + t) * ng + g;
    if (o.scale16) o.scale16[red] = __half_as_ushort(__float2half_rn(s));
    if (o.zero16) o.zero16[red] = __half_as_ushort(__float2half_rn(z));
  }
}

// ---- one group across G lanes (small appends) ------------------------------
// The one-thread-per-group kernels run each group as one thread's chain of
// ~G * 25 dependent instructions: fine for a prompt (many groups), but a
// decode step's append is a few hundred groups, i.e. one or two workgroups
// and ~8 us of latency (a one-token K append at B=16: measured).  Here the
// G <= 64 lanes of an aligned segment of one wave hold one group, lane i its
// element i; the extremes, the NaN test and the packed words are reduced
// across the segment.  The per-value arithmetic is quantize_group's /
// quant_group_rt's, the extremes are exact and the words are ORs of disjoint
// bit fields, so the fields and meta are the same bit for bit.  Hybrid's two
// error sums are added in element order (seg_sum_ordered), as the
// one-thread path adds them.
template <int G>
__device__ __forceinline__ uint64_t seg_mask() {
  if constexpr (G == 64) {
    return ~0ull;
  } else {
    const int lane = threadIdx.x & 63;
    return ((1ull << G) - 1ull) << (lane & ~(G - 1));
  }
}
// Segment reductions (G = 32 or 64 lanes; every lane gets the result): DPP
// butterflies inside each 16-lane row (quad xor 1, quad xor 2, half-row
// mirror, row mirror: one VALU instruction each), then the rows: xor 16 by
// ds_swizzle (bit-mask mode, no address), and for G = 64 the two halves by
// readlane.  min, max and or give the same result in any order.
template <int G, typename F>
__device__ __forceinline__ uint32_t seg_reduce(uint32_t x, F op) {
  static_assert(G == 32 || G == 64, "segments of 32 or 64 lanes");
  x = op(x, uint32_t(__builtin_amdgcn_mov_dpp(int(x), 0xb1, 0xf, 0xf, true)));   // quad_perm [1,0,3,2]
  x = op(x, uint32_t(__builtin_amdgcn_mov_dpp(int(x), 0x4e, 0xf, 0xf, true)));   // quad_perm [2,3,0,1]
  x = op(x, uint32_t(__builtin_amdgcn_mov_dpp(int(x), 0x141, 0xf, 0xf, true)));  // row_half_mirror
  x = op(x, uint32_t(__builtin_amdgcn_mov_dpp(int(x), 0x140, 0xf, 0xf, true)));  // row_mirror
  x = op(x, uint32_t(__builtin_amdgcn_ds_swizzle(int(x), 0x401f)));             // lane ^ 16
  if constexpr (G == 64)
    x = op(uint32_t(__builtin_amdgcn_readlane(int(x), 0)), uint32_t(__builtin_amdgcn_readlane(int(x), 32)));
  return x;
}
template <int G>
__device__ __forceinline__ float seg_fmin(float x) {
  return __uint_as_float(seg_reduce<G>(__float_as_uint(x), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fminf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
template <int G>
__device__ __forceinline__ float seg_fmax(float x) {
  return __uint_as_float(seg_reduce<G>(__float_as_uint(x), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
template <int G>
__device__ __forceinline__ uint32_t seg_or(uint32_t x) {
  return seg_reduce<G>(x, [](uint32_t a, uint32_t b) { return a | b; });
}

// The segment's sum of x in lane (= element) order, in fp64, every lane of
// the segment getting it: ((0 + x_0) + x_1) + ..., the order of the
// one-thread-per-group loop, so the same roundings.  Lane j's value is read
// by a shuffle (two 32-bit halves).
template <int G>
__device__ __forceinline__ double seg_sum_ordered(float x) {
  const double xd = double(x);
  const int lo = __double2loint(xd), hi = __double2hiint(xd);
  const int base = int(threadIdx.x & 63) & ~(G - 1);
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < G; ++j) acc += __hiloint2double(__shfl(hi, base + j, 64), __shfl(lo, base + j, 64));
  return acc;
}

// lane i of the segment holds element v of the group; every lane of the
// segment must be active.  Writes the group's words (lane w writes word w)
// and its meta (lane 0) when `store`; returns the dense code and sets sg (the
// sign, sym) and s, z (scale; zero point, asym) for the reference outputs.
template <int G>
__device__ __forceinline__ int32_t quant_group_lanes(float v, int i, int bits, int mode, bool bf, bool store,
                                                     uint32_t* out, uint16_t* meta, int64_t unit, float& sg, float& s,
                                                     float& z, float* deq = nullptr) {
  const bool nan = (__ballot(is_nan(v)) & seg_mask<G>()) != 0ull;
  int32_t c;
  uint32_t fld;
  bool hsym = false;  // hybrid: the group keeps its sym codes
  if (mode == IQ_MODE_SYM) {
    float amx = seg_fmax<G>(fabsf(v));
    if (nan) amx = __builtin_nanf("");
    s = sym_scale_b(amx, bits, bf);
    z = 0.f;
    c = sym_code_b(v, s, bits, bf);
    sg = sign_of(v);
    fld = sym_field_b(c, sg, bits);
  } else if (mode == IQ_MODE_HYBRID) {  // quant_group_rt's hybrid choice (quant.py:133-151)
    float mn = seg_fmin<G>(v), mx = seg_fmax<G>(v), amx = seg_fmax<G>(fabsf(v));
    if (nan) { mn = __builtin_nanf(""); mx = mn; amx = mn; }
    const float sa = asym_scale_b(mn, mx, bits - 1, bf), ss = sym_scale_b(amx, bits, bf);
    const int32_t ca = asym_code_b(v, mn, sa, bits - 1, bf), cs = sym_code_b(v, ss, bits, bf);
    sg = sign_of(v);
    const float da = __fadd_rn(__fmul_rn(float(ca), sa), mn);
    const float ds = __fmul_rn(__fmul_rn(float(cs), ss), sg);
    const double ea = seg_sum_ordered<G>(fabsf(__fsub_rn(da, v)));
    const double es = seg_sum_ordered<G>(fabsf(__fsub_rn(ds, v)));
    hsym = ea > es;
    c = hsym ? cs : ca;
    s = hsym ? ss : sa;
    z = mn;
    fld = hsym ? sym_field_b(cs, sg, bits) : asym_field_b(ca, bits);
  } else {
    float mn = seg_fmin<G>(v), mx = seg_fmax<G>(v);
    if (nan) { mn = __builtin_nanf(""); mx = mn; }
    s = asym_scale_b(mn, mx, bits, bf);
    z = mn;
    c = asym_code_b(v, mn, s, bits, bf);
    sg = 0.f;
    fld = asym_field_b(c, bits);
  }
  const int bit = bits * i, wi = bit >> 5, o = bit & 31;
  const uint32_t lo = fld << o, hi = o + bits > 32 ? fld >> (32 - o) : 0u;
  const int W = (G * bits) >> 5;
#pragma unroll
  for (int w = 0; w < (G * 4) / 32; ++w) {  // up to 4-bit fields
    const uint32_t word = seg_or<G>((wi == w ? lo : 0u) | (wi + 1 == w ? hi : 0u));
    if (store && w < W && i == w) out[w] = word;
  }
  if (deq) {  // the stored field's value, as group_deq_params + dequant_k_kernel decode it (quant.py:83-93, 121-131)
    const bool symf = mode == IQ_MODE_SYM || hsym;
    const float cf = symf ? float(int(fld) - (1 << (bits - 1))) : float(fld);
    *deq = __fadd_rn(__fmul_rn(cf, s), symf ? 0.f : z);
  }
  if (store && i == 0) {
    if (mode == IQ_MODE_SYM) {
      meta[unit] = f2act(s, bf);
    } else if (mode == IQ_MODE_HYBRID) {
      const uint32_t sh = f2act(s, bf);
      reinterpret_cast<uint32_t*>(meta)[unit] = hsym ? (sh | HYB_FLAG) : ((sh & 0x7fffu) | (uint32_t(f2act(z, bf)) << 16));
    } else {
      reinterpret_cast<uint32_t*>(meta)[unit] = meta_word(s, z, bf);
    }
  }
  return c;
}

// ---- one lane per value (quant_group_lanes), either axis -------------------
// G <= 64, asym or sym, fp16 or bf16 activations; the same stores and
// reference-format outputs as quant_k_kernel (axis 0, groups along D) and
// quant_v_kernel (axis 1, groups along tokens).  Serves small K calls (a
// decode step's tokens, where one thread per group would idle the device)
// and every bf16 quantization of those formats.
struct LaneArgs {
  const uint16_t* x;
  int64_t sxb, sxh, sxt;
  const uint16_t* norm;  // axis 0 only
  int B, H, n, D, bits, mode, bf, axis;
};
template <int G>
__global__ __launch_bounds__(256) void quant_lane_kernel(LaneArgs a, QuantOut o) {
  const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t gid = e / G;
  const int i = int(e % G);
  const bool bf = a.bf != 0;
  int64_t bh, unit, xoff, el, red, row_el = 0;
  int dcol;
  if (a.axis == 0) {
    const int ng = a.D / G;
    if (gid >= int64_t(a.B) * a.H * a.n * ng) return;  // whole G-lane segments
    const int g = int(gid % ng);
    const int64_t row = gid / ng;  // bh * n + t
    const int t = int(row % a.n);
    bh = row / a.n;
    dcol = g * G + i;
    xoff = (bh / a.H) * a.sxb + (bh % a.H) * a.sxh + t * a.sxt + dcol;
    const int64_t tt = o.t_off + t;
    unit = ((bh * o.cap_units + tt / TOKEN_BLOCK) * ng + g) * TOKEN_BLOCK + tt % TOKEN_BLOCK;
    row_el = row * a.D + g * G;
    el = row_el + i;
    red = row * ng + g;
  } else {
    const int ngn = a.n / G;
    if (gid >= int64_t(a.B) * a.H * ngn * a.D) return;
    const int d = int(gid % a.D);
    const int64_t r = gid / a.D;  // bh * ngn + gi
    const int gi = int(r % ngn);
    bh = r / ngn;
    dcol = d;
    const int t = gi * G + i;
    xoff = (bh / a.H) * a.sxb + (bh % a.H) * a.sxh + int64_t(t) * a.sxt + d;
    unit = (bh * o.cap_units + o.t_off / G + gi) * a.D + d;
    el = (bh * a.n + t) * a.D + d;
    red = r * a.D + d;
  }
  float v = act2f(a.x[xoff], bf);
  if (a.norm) v = round_act(v / act2f(a.norm[bh * a.D + dcol], bf), bf);  // cache.py:125
  float sg, sc, zp;
  const int32_t c = quant_group_lanes<G>(v, i, a.bits, a.mode, bf, o.codes != nullptr,
                                         o.codes ? o.codes + unit * ((G * a.bits) >> 5) : nullptr, o.meta, unit, sg,
                                         sc, zp);
  if (o.codes_i32) o.codes_i32[el] = c;
  if (o.signs16) o.signs16[el] = f2act(sg, bf);
  if (i == 0) {
    if (o.scale16) o.scale16[red] = f2act(sc, bf);
    if (o.zero16) o.zero16[red] = f2act(zp, bf);
  }
}

// One group, quantized as quantize_group / quantize_group_hybrid do, with
// the bit width, mode and activation dtype known at run time: v[] holds the
// group's G inputs (registers; loaded together, one memory latency per group),
// the fields are stored word by word as they fill, the meta word last.
// Optional reference-format outputs (RtRef, asym or sym): element i's code and
// sign at codes[el0 + i * el_step], signs[...], the scale and zero at red.
struct RtRef {
  int32_t* codes;
  uint16_t* signs;
  uint16_t* scale;
  uint16_t* zero;
  int64_t el0, el_step, red;
};
template <int G>
__device__ __forceinline__ void quant_group_rt(const float* v, int bits, int mode, bool bf, uint32_t* out,
                                               uint16_t* meta, int64_t unit, const RtRef* ref = nullptr) {
  const int abits = mode == IQ_MODE_HYBRID ? bits - 1 : bits;
  float mn = v[0], mx = v[0], amx = 0.f;
  bool nan = false;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    nan |= is_nan(v[i]);
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
    amx = fmaxf(amx, fabsf(v[i]));
  }
  if (nan) { mn = __builtin_nanf(""); mx = mn; amx = mn; }
  const float sa = asym_scale_b(mn, mx, abits, bf), ss = sym_scale_b(amx, bits, bf);
  bool sym = mode == IQ_MODE_SYM;
  if (mode == IQ_MODE_HYBRID) {  // quantize_group_hybrid's choice
    double ea = 0.0, es = 0.0;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const float da = __fadd_rn(__fmul_rn(float(asym_code_b(v[i], mn, sa, abits, bf)), sa), mn);
      const float ds = __fmul_rn(__fmul_rn(float(sym_code_b(v[i], ss, bits, bf)), ss), sign_of(v[i]));
      ea += double(fabsf(__fsub_rn(da, v[i])));
      es += double(fabsf(__fsub_rn(ds, v[i])));
    }
    sym = ea > es;
  }
  uint64_t acc = 0;
  int pos = 0, wj = 0;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int32_t c = sym ? sym_code_b(v[i], ss, bits, bf) : asym_code_b(v[i], mn, sa, abits, bf);
    const uint32_t fld = sym ? sym_field_b(c, sign_of(v[i]), bits) : asym_field_b(c, bits);
    if (ref) {
      if (ref->codes) ref->codes[ref->el0 + i * ref->el_step] = c;
      if (ref->signs) ref->signs[ref->el0 + i * ref->el_step] = f2act(sign_of(v[i]), bf);
    }
    acc |= uint64_t(fld) << pos;
    pos += bits;
    if (pos >= 32) {
      if (out) out[wj] = uint32_t(acc);
      ++wj;
      acc >>= 32;
      pos -= 32;
    }
  }
  if (ref) {
    if (ref->scale) ref->scale[ref->red] = f2act(sym ? ss : sa, bf);
    if (ref->zero) ref->zero[ref->red] = f2act(mn, bf);
  }
  if (!out) return;
  if (mode == IQ_MODE_SYM) {
    meta[unit] = f2act(ss, bf);
  } else if (mode == IQ_MODE_HYBRID) {
    const uint32_t sh = f2act(sym ? ss : sa, bf);
    reinterpret_cast<uint32_t*>(meta)[unit] =
        sym ? (sh | HYB_FLAG) : ((sh & 0x7fffu) | (uint32_t(f2act(mn, bf)) << 16));
  } else {
    reinterpret_cast<uint32_t*>(meta)[unit] = meta_word(sa, mn, bf);
  }
}

// ---- one thread per group, bit width / mode / dtype at run time -----------
// (quant_group_rt) The bf16 formats quant_lane_kernel does not take: groups
// of 128 and hybrid stores; either axis, stores and reference outputs.
template <int G>
__global__ __launch_bounds__(256) void quant_rt_kernel(LaneArgs a, QuantOut o) {
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool bf = a.bf != 0;
  float v[G];
  int64_t bh, unit;
  RtRef ref{o.codes_i32, o.signs16, o.scale16, o.zero16, 0, 0, 0};
  if (a.axis == 0) {
    const int ng = a.D / G;
    if (gid >= int64_t(a.B) * a.H * a.n * ng) return;
    const int g = int(gid % ng);
    const int64_t row = gid / ng;  // bh * n + t
    const int t = int(row % a.n);
    bh = row / a.n;
    const uint16_t* xp = a.x + (bh / a.H) * a.sxb + (bh % a.H) * a.sxh + t * a.sxt + g * G;
#pragma unroll
    for (int i = 0; i < G; ++i) v[i] = act2f(xp[i], bf);
    if (a.norm) {  // cache.py:125
#pragma unroll
      for (int i = 0; i < G; ++i) v[i] = round_act(v[i] / act2f(a.norm[bh * a.D + g * G + i], bf), bf);
    }
    const int64_t tt = o.t_off + t;
    unit = ((bh * o.cap_units + tt / TOKEN_BLOCK) * ng + g) * TOKEN_BLOCK + tt % TOKEN_BLOCK;
    ref.el0 = row * a.D + g * G;
    ref.el_step = 1;
    ref.red = row * ng + g;
  } else {
    const int ngn = a.n / G;
    if (gid >= int64_t(a.B) * a.H * ngn * a.D) return;
    const int d = int(gid % a.D);
    const int64_t r = gid / a.D;  // bh * ngn + gi
    const int gi = int(r % ngn);
    bh = r / ngn;
    const uint16_t* xp = a.x + (bh / a.H) * a.sxb + (bh % a.H) * a.sxh + int64_t(gi) * G * a.sxt + d;
#pragma unroll
    for (int i = 0; i < G; ++i) v[i] = act2f(xp[int64_t(i) * a.sxt], bf);
    unit = (bh * o.cap_units + o.t_off / G + gi) * a.D + d;
    ref.el0 = (bh * a.n + int64_t(gi) * G) * a.D + d;
    ref.el_step = a.D;
    ref.red = r * a.D + d;
  }
  const bool any_ref = o.codes_i32 || o.signs16 || o.scale16 || o.zero16;
  quant_group_rt<G>(v, a.bits, a.mode, bf, o.codes ? o.codes + unit * ((G * a.bits) >> 5) : nullptr, o.meta, unit,
                    any_ref ? &ref : nullptr);
}

// bf16 quantization, or a small fp16 K call: one lane per value where the
// format allows (G <= 64, asym / sym), else one thread per group at run time
int launch_lane_or_rt(const LaneArgs& a, const QuantOut& o, int group, hipStream_t st) {
  const int64_t groups = a.axis == 0 ? int64_t(a.B) * a.H * a.n * (a.D / group)
                                     : int64_t(a.B) * a.H * (a.n / group) * a.D;
  if (groups == 0) return IQ_OK;
  if (group <= 64 && a.mode != IQ_MODE_HYBRID) {
    auto* kern = group == 64 ? quant_lane_kernel<64> : quant_lane_kernel<32>;
    kern<<<dim3(unsigned(ceil_div(groups * group, 256))), 256, 0, st>>>(a, o);
  } else {
    auto* kern = group == 128 ? quant_rt_kernel<128> : group == 64 ? quant_rt_kernel<64> : quant_rt_kernel<32>;
    kern<<<dim3(unsigned(ceil_div(groups, 256))), 256, 0, st>>>(a, o);
  }
  return launch_status();
}

// ---- V: groups along tokens, one thread per (b, h, token-group, d) --------
template <int BITS, int G, bool DENSE, bool HYB = false>
__global__ __launch_bounds__(256) void quant_v_kernel(const uint16_t* __restrict__ x, int64_t sxb, int64_t sxh,
                                                      int64_t sxt, int B, int H, int n, int D, int sym,
                                                      QuantOut o) {
  const int ngn = n / G;
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = int64_t(B) * H * ngn * D;
  if (gid >= total) return;
  const int d = int(gid % D);
  int64_t r = gid / D;
  const int gi = int(r % ngn);
  r /= ngn;
  const int h = int(r % H);
  const int b = int(r / H);

  const uint16_t* xp = x + b * sxb + h * sxh + int64_t(gi) * G * sxt + d;
  float v[G];
#pragma unroll
  for (int i = 0; i < G; ++i) v[i] = h2f(xp[i * sxt]);
  const int64_t bh = int64_t(b) * H + h;
  const int64_t unit = (bh * o.cap_units + o.t_off / G + gi) * D + d;
  uint32_t f[G];
  if constexpr (HYB) {
    if constexpr (BITS >= 2) {
      uint32_t mw;
      quantize_group_hybrid<BITS, G>(v, f, mw);
      store_group<BITS, G>(o, unit, f, false, mw);
    }
    return;
  }
  int32_t c[G];
  float sg[G];
  float s, z;
  quantize_group<BITS, G>(v, sym != 0, f, c, sg, s, z);
  if (o.codes) store_group<BITS, G>(o, unit, f, sym != 0, meta_word(s, z));
  if constexpr (DENSE) {  // the reference-format outputs (quant.py API)
    if (o.codes_i32 || o.signs16) {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int64_t el = (bh * n + int64_t(gi) * G + i) * D + d;
        if (o.codes_i32) o.codes_i32[el] = c[i];
        if (o.signs16) o.signs16[el] = __half_as_ushort(__float2half_rn(sg[i]));
      }
    }
    const int64_t red = (bh * ngn + gi) * D + d;
    if (o.scale16) o.scale16[red] = __half_as_ushort(__float2half_rn(s));
    if (o.zero16) o.zero16[red] = __half_as_ushort(__float2half_rn(z));
  }
}

// ---- dequantization (dense read path) --------------------------------------
struct DeqOut {
  uint16_t* out16;  // in the activation dtype
  float* out32;
  int64_t sob, soh, sot;
  int bf;           // bf16 activations: meta, norm and out16
};

__device__ __forceinline__ void put(const DeqOut& o, int64_t off, float v) {
  if (o.out16) o.out16[off] = f2act(v, o.bf != 0);
  if (o.out32) o.out32[off] = v;
}

// signed codes and {scale, zero} of one group such that value = c*s + z:
// asym {s, z}; sym offset binary, z = 0; hybrid as the group's flag says
// (quant.py:153-176: the sym codes where the mask is set)
template <int BITS, int G>
__device__ __forceinline__ void group_deq_params(const uint32_t* w, const uint16_t* meta, int64_t unit, int mode,
                                                 bool bf, int32_t* c, float& s, float& z) {
  unpack_fields<BITS, G>(w, mode == IQ_MODE_SYM, c);
  z = 0.f;
  if (mode == IQ_MODE_SYM) {
    s = act2f(meta[unit], bf);
    return;
  }
  const uint32_t mw = reinterpret_cast<const uint32_t*>(meta)[unit];
  if (mode == IQ_MODE_HYBRID && hyb_sym(mw)) {
#pragma unroll
    for (int i = 0; i < G; ++i) c[i] -= 1 << (BITS - 1);
    s = hyb_scale(mw, bf);
    return;
  }
  s = mode == IQ_MODE_HYBRID ? hyb_scale(mw, bf) : act2f(uint16_t(mw & 0xffffu), bf);
  z = act2f(uint16_t(mw >> 16), bf);
}

template <int BITS, int G>
__global__ __launch_bounds__(256) void dequant_k_kernel(const uint32_t* __restrict__ kc,
                                                        const uint16_t* __restrict__ km, int64_t cap_blocks,
                                                        const uint16_t* __restrict__ norm, int B, int H, int t0,
                                                        int T, int D, int mode, DeqOut o) {
  constexpr int W = G * BITS / 32;
  const int ng = D / G;
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = int64_t(B) * H * T * ng;
  if (gid >= total) return;
  const int g = int(gid % ng);
  int64_t r = gid / ng;
  const int t = int(r % T);
  r /= T;
  const int h = int(r % H);
  const int b = int(r / H);
  const int64_t bh = int64_t(b) * H + h;
  const int64_t tt = int64_t(t0) + t;
  const int64_t unit = ((bh * cap_blocks + tt / TOKEN_BLOCK) * ng + g) * TOKEN_BLOCK + tt % TOKEN_BLOCK;
  uint32_t w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = kc[unit * W + j];
  int32_t c[G];
  float s, z;
  group_deq_params<BITS, G>(w, km, unit, mode, o.bf != 0, c, s, z);
  const int64_t base = b * o.sob + h * o.soh + t * o.sot + g * G;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    float v = __fadd_rn(__fmul_rn(float(c[i]), s), z);       // quant.py:84-85 (c*s exact)
    if (norm) v = __fmul_rn(v, act2f(norm[bh * D + g * G + i], o.bf != 0));  // cache.py:132
    put(o, base + i, v);
  }
}

template <int BITS, int G>
__global__ __launch_bounds__(256) void dequant_v_kernel(const uint32_t* __restrict__ vc,
                                                        const uint16_t* __restrict__ vm, int64_t cap_groups,
                                                        int B, int H, int g0, int ngT, int D, int mode, DeqOut o) {
  constexpr int W = G * BITS / 32;
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = int64_t(B) * H * ngT * D;
  if (gid >= total) return;
  const int d = int(gid % D);
  int64_t r = gid / D;
  const int gi = int(r % ngT);
  r /= ngT;
  const int h = int(r % H);
  const int b = int(r / H);
  const int64_t bh = int64_t(b) * H + h;
  const int64_t unit = (bh * cap_groups + g0 + gi) * D + d;
  uint32_t w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = vc[unit * W + j];
  int32_t c[G];
  float s, z;
  group_deq_params<BITS, G>(w, vm, unit, mode, o.bf != 0, c, s, z);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const float v = __fadd_rn(__fmul_rn(float(c[i]), s), z);  // quant.py:90-91
    put(o, b * o.sob + h * o.soh + (int64_t(gi) * G + i) * o.sot + d, v);
  }
}

// ---- dense int32 codes -> values (the quant.py dequantize_* API) ----------
// tensor [outer, n, inner] grouped along n; scale/zero [outer, n/G, inner];
// signs [outer, n, inner].  op in fp32 (out_f16 = 0) or fp16 (out_f16 = 1),
// one rounding per op as torch does for that dtype (quant.py:83-93, 121-131).
__global__ __launch_bounds__(256) void dequant_dense_kernel(const int32_t* __restrict__ codes,
                                                            const uint16_t* __restrict__ scale,
                                                            const uint16_t* __restrict__ zs, int64_t outer,
                                                            int64_t n, int64_t inner, int G, int sym, int out_f16,
                                                            int bf, void* out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= outer * n * inner) return;
  const int64_t j = i % inner;
  const int64_t t = (i / inner) % n;
  const int64_t o = i / (inner * n);
  const int64_t red = (o * (n / G) + t / G) * inner + j;
  const bool b16 = bf != 0;
  const float c = float(codes[i]);
  const float s = act2f(scale[red], b16);
  float v;
  if (!out_f16) {
    v = __fmul_rn(c, s);
    v = sym ? __fmul_rn(v, act2f(zs[i], b16)) : __fadd_rn(v, act2f(zs[red], b16));
    reinterpret_cast<float*>(out)[i] = v;
  } else {  // op_dtype = the activation dtype: one rounding per op
    v = round_act(__fmul_rn(round_act(c, b16), s), b16);
    v = sym ? round_act(__fmul_rn(v, act2f(zs[i], b16)), b16) : round_act(__fadd_rn(v, act2f(zs[red], b16)), b16);
    reinterpret_cast<uint16_t*>(out)[i] = f2act(v, b16);
  }
}


// ---- packed store -> reference-format tensors (cache state attributes) -----
// codes: quant.py's int32 codes (sym: magnitudes); scale16 / zero16 as the
// quantizer returns them; signs16 (sym): the sign of the stored code (0 for a
// zero code, whose sign the packed form does not keep).
struct UnpackOut {
  int32_t* codes;
  uint16_t* scale;
  uint16_t* zs;
};

__device__ __forceinline__ void unpack_meta(const uint16_t* meta, int64_t unit, bool sym, uint16_t& s, uint16_t& z) {
  if (sym) {
    s = meta[unit];
    z = 0;
  } else {
    const uint32_t sz = reinterpret_cast<const uint32_t*>(meta)[unit];
    s = uint16_t(sz & 0xffffu);
    z = uint16_t(sz >> 16);
  }
}

__device__ __forceinline__ uint16_t sign16(int32_t c, bool bf) {  // +-1 or 0 in the activation dtype
  return c > 0 ? (bf ? 0x3f80u : 0x3c00u) : (c < 0 ? (bf ? 0xbf80u : 0xbc00u) : 0u);
}

template <int BITS, int G>
__global__ __launch_bounds__(256) void unpack_k_kernel(const uint32_t* __restrict__ kc, const uint16_t* __restrict__ km,
                                                       int64_t cap_blocks, int B, int H, int t0, int T, int D, int sym,
                                                       int bf, UnpackOut o) {
  constexpr int W = G * BITS / 32;
  const int ng = D / G;
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= int64_t(B) * H * T * ng) return;
  const int g = int(gid % ng);
  const int64_t row = gid / ng;  // (b*H + h)*T + t
  const int64_t bh = row / T;
  const int64_t tt = int64_t(t0) + row % T;
  const int64_t unit = ((bh * cap_blocks + tt / TOKEN_BLOCK) * ng + g) * TOKEN_BLOCK + tt % TOKEN_BLOCK;
  uint32_t w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = kc[unit * W + j];
  int32_t c[G];
  unpack_fields<BITS, G>(w, sym != 0, c);
  uint16_t s, z;
  unpack_meta(km, unit, sym != 0, s, z);
  o.scale[row * ng + g] = s;
  if (!sym) o.zs[row * ng + g] = z;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int64_t e = row * D + g * G + i;
    o.codes[e] = c[i] < 0 ? -c[i] : c[i];
    if (sym) o.zs[e] = sign16(c[i], bf != 0);
  }
}

template <int BITS, int G>
__global__ __launch_bounds__(256) void unpack_v_kernel(const uint32_t* __restrict__ vc, const uint16_t* __restrict__ vm,
                                                       int64_t cap_groups, int B, int H, int g0, int ngT, int D,
                                                       int sym, int bf, UnpackOut o) {
  constexpr int W = G * BITS / 32;
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= int64_t(B) * H * ngT * D) return;
  const int d = int(gid % D);
  const int64_t r = gid / D;  // (b*H + h)*ngT + gi
  const int gi = int(r % ngT);
  const int64_t bh = r / ngT;
  const int64_t unit = (bh * cap_groups + g0 + gi) * D + d;
  uint32_t w[W];
#pragma unroll
  for (int j = 0; j < W; ++j) w[j] = vc[unit * W + j];
  int32_t c[G];
  unpack_fields<BITS, G>(w, sym != 0, c);
  uint16_t s, z;
  unpack_meta(vm, unit, sym != 0, s, z);
  o.scale[r * D + d] = s;
  if (!sym) o.zs[r * D + d] = z;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int64_t e = ((bh * ngT + gi) * G + i) * D + d;
    o.codes[e] = c[i] < 0 ? -c[i] : c[i];
    if (sym) o.zs[e] = sign16(c[i], bf != 0);
  }
}

// ---- one decode step of a layer's recent windows (cache.py:283-365) ----
// Per role (K, V): the m new tokens are written after the window in its
// buffer, and the first F tokens of [window | new tokens] are quantized into
// the store, in one launch for both roles.  The quantizer here takes the bit
// width, group size and mode at run time and reads each group from memory
// once per pass (no per-group register arrays); every element goes through
// the same fp16 ops as quantize_group / quantize_group_hybrid.
struct WinRole {
  uint16_t* buf;
  int64_t sb, sh, st;
  int start, n;  // the window before the step: buffer tokens [start, start + n)
  const uint16_t* x;
  int64_t sxb, sxh, sxt;
  int m;  // new tokens, written at buffer token start + n + j
  int F;  // tokens flushed into the store: the first F of [window | new]
  uint32_t* codes;
  uint16_t* meta;
  int64_t cap_units, t_off;
  int bits, group, gsh, mode, axis;  // axis 0: groups along head_dim (K layout), 1: along tokens (V layout)
  int bf;                            // bf16 activations (mode's IQ_MODE_BF16 flag, stripped from mode)
  const uint16_t* norm;              // axis 0: fp16 [B,H,D] key normalization factor, or null
  int vec_buf, vec_x;                // rows of the buffer / of x are 16-byte aligned (base and strides)
  int deq;                           // flushed tokens' buffer rows get their dequantized values
};

struct AppendArgs {
  WinRole r[2];
  int H, D;
  // work items: copies of role 0, copies of role 1, groups of role 0, groups
  // of role 1; segment k covers [start[k], start[k] + count[k]), starts
  // aligned to the block size
  int64_t start[4], count[4];
};

// one group of the flushed tokens of role r (group item q): element i is
// token f0 + i * fstep of [window | new], column d0 + i * dstep
template <int G>
__device__ __forceinline__ void append_group(const WinRole& r, int H, int D, int64_t q) {
  int64_t bh, unit;
  int f0, fstep, d0, dstep;
  if (r.axis == 0) {
    const int ng = D / G;
    const int g = int(q % ng);
    const int64_t rest = q / ng;
    const int f = int(rest % r.F);
    bh = rest / r.F;
    const int64_t tt = r.t_off + f;
    unit = ((bh * r.cap_units + (tt >> 6)) * ng + g) * TOKEN_BLOCK + (tt & 63);
    f0 = f; fstep = 0; d0 = g * G; dstep = 1;
  } else {
    const int d = int(q % D);
    const int64_t rest = q / D;
    const int ngf = r.F / G;
    const int gi = int(rest % ngf);
    bh = rest / ngf;
    unit = (bh * r.cap_units + r.t_off / G + gi) * D + d;
    f0 = gi * G; fstep = 1; d0 = d; dstep = 0;
  }
  const int64_t b = bh / H, h = bh % H;
  float v[G];
  if (r.axis == 0 && (f0 < r.n ? r.vec_buf : r.vec_x)) {  // G contiguous fp16, 16-byte aligned rows
    const uint16_t* p = f0 < r.n ? r.buf + b * r.sb + h * r.sh + int64_t(r.start + f0) * r.st + d0
                                 : r.x + b * r.sxb + h * r.sxh + int64_t(f0 - r.n) * r.sxt + d0;
#pragma unroll
    for (int c = 0; c < G / 8; ++c) {
      const uint4 u = reinterpret_cast<const uint4*>(p)[c];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * c + 2 * j] = act2f(uint16_t(w[j] & 0xffffu), r.bf != 0);
        v[8 * c + 2 * j + 1] = act2f(uint16_t(w[j] >> 16), r.bf != 0);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int f = f0 + i * fstep, d = d0 + i * dstep;
      const uint16_t* p = f < r.n ? r.buf + b * r.sb + h * r.sh + int64_t(r.start + f) * r.st + d
                                  : r.x + b * r.sxb + h * r.sxh + int64_t(f - r.n) * r.sxt + d;
      v[i] = act2f(*p, r.bf != 0);
    }
  }
  if (r.norm) {  // cache.py:125  x / key_normalization_factor in fp16
#pragma unroll
    for (int i = 0; i < G; ++i) v[i] = round_act(v[i] / act2f(r.norm[bh * D + d0 + i * dstep], r.bf != 0), r.bf != 0);
  }
  quant_group_rt<G>(v, r.bits, r.mode, r.bf != 0, r.codes + unit * ((G * r.bits) >> 5), r.meta, unit);
}

// append_group with one lane per element (G <= 64, asym or sym): item q of
// the role's groups, element i
template <int G>
__device__ __forceinline__ void append_group_lanes(const WinRole& r, int H, int D, int64_t q, int i) {
  int64_t bh, unit;
  int f, d;
  if (r.axis == 0) {
    const int ng = D / G;
    const int g = int(q % ng);
    const int64_t rest = q / ng;
    f = int(rest % r.F);
    bh = rest / r.F;
    const int64_t tt = r.t_off + f;
    unit = ((bh * r.cap_units + (tt >> 6)) * ng + g) * TOKEN_BLOCK + (tt & 63);
    d = g * G + i;
  } else {
    d = int(q % D);
    const int64_t rest = q / D;
    const int ngf = r.F / G;
    const int gi = int(rest % ngf);
    bh = rest / ngf;
    unit = (bh * r.cap_units + r.t_off / G + gi) * D + d;
    f = gi * G + i;
  }
  const int64_t b = bh / H, h = bh % H;
  const uint16_t* p = f < r.n ? r.buf + b * r.sb + h * r.sh + int64_t(r.start + f) * r.st + d
                              : r.x + b * r.sxb + h * r.sxh + int64_t(f - r.n) * r.sxt + d;
  float v = act2f(*p, r.bf != 0);
  if (r.norm) v = round_act(v / act2f(r.norm[bh * D + d], r.bf != 0), r.bf != 0);  // cache.py:125
  float sg, sc, zp, dq;
  quant_group_lanes<G>(v, i, r.bits, r.mode, r.bf, true, r.codes + unit * ((G * r.bits) >> 5), r.meta, unit, sg, sc,
                       zp, r.deq ? &dq : nullptr);
  if (r.deq) {  // the token's buffer row (window or new token) as dequant_k_kernel gives it
    if (r.norm) dq = __fmul_rn(dq, act2f(r.norm[bh * D + d], r.bf != 0));  // cache.py:132
    r.buf[b * r.sb + h * r.sh + int64_t(r.start + f) * r.st + d] = f2act(dq, r.bf != 0);
  }
}

// lanes per group item of a role: one lane per element where quant_group_lanes
// applies (groups of up to 64; asym, sym or hybrid), else one thread per group
__host__ __device__ inline int role_lanes(int group, int mode) {
  (void)mode;
  return group <= 64 ? group : 1;
}

// element e of the new tokens (b, h, j, d) into the window buffer
__device__ __forceinline__ void window_copy(const WinRole& r, int H, int D, int64_t e) {
  const int64_t per_bh = int64_t(r.m) * D;
  const int64_t bh = e / per_bh, b = bh / H, h = bh % H;
  const int j = int((e % per_bh) / D), d = int(e % D);
  if (r.deq && r.n + j < r.F) return;  // a flushed new token: its row gets the dequantized values
  r.buf[b * r.sb + h * r.sh + int64_t(r.start + r.n + j) * r.st + d] = r.x[b * r.sxb + h * r.sxh + int64_t(j) * r.sxt + d];
}

template <int GK, int GV>
__global__ __launch_bounds__(256) void window_append_kernel(AppendArgs a) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int k = 0;
#pragma unroll
  for (int s = 1; s < 4; ++s) k = i >= a.start[s] ? s : k;
  const int64_t e = i - a.start[k];
  if (e >= a.count[k]) return;
  // (block-uniform k: each role's fields are read with a constant index)
  // (a group role's items are whole aligned G-lane segments, so a segment is
  // either all past the count or all active)
  if (k == 0) window_copy(a.r[0], a.H, a.D, e);
  else if (k == 1) window_copy(a.r[1], a.H, a.D, e);
  else if (k == 2) {
    if constexpr (GK <= 64) {
      if (role_lanes(GK, a.r[0].mode) > 1) {
        append_group_lanes<GK>(a.r[0], a.H, a.D, e / GK, int(e % GK));
        return;
      }
    }
    append_group<GK>(a.r[0], a.H, a.D, e);
  } else {
    if constexpr (GV <= 64) {
      if (role_lanes(GV, a.r[1].mode) > 1) {
        append_group_lanes<GV>(a.r[1], a.H, a.D, e / GV, int(e % GV));
        return;
      }
    }
    append_group<GV>(a.r[1], a.H, a.D, e);
  }
}

}  // namespace

// =============================================================================
// C ABI
// =============================================================================
extern "C" {

int iq_abi_version(void) { return IQ_ABI_VERSION; }

const char* iq_strerror(int status) {
  switch (status) {
    case IQ_OK: return "ok";
    case IQ_ERR_NULL: return "null pointer argument";
    case IQ_ERR_BITS: return "bits must be 2, 3 or 4 (packed stores: also 1 with asym)";
    case IQ_ERR_GROUP: return "group must be 32, 64 or 128 and divide the grouped axis";
    case IQ_ERR_SHAPE: return "unsupported or invalid shape";
    case IQ_ERR_ALIGN: return "pointer or stride misaligned";
    case IQ_ERR_WORKSPACE: return "workspace missing or too small";
    case IQ_ERR_MODE: return "mode must be IQ_MODE_ASYM or IQ_MODE_SYM";
    case IQ_ERR_RANGE: return "token range exceeds store capacity";
    case IQ_ERR_HIP: return "HIP launch failed";
    default: return "unknown status";
  }
}

int iq_k_store_bytes(int64_t B, int64_t H, int64_t t_cap, int64_t D, int group, int bits, int mode,
                     int64_t* codes_bytes, int64_t* meta_bytes) {
  IQ_CHECK(codes_bytes && meta_bytes, IQ_ERR_NULL);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && t_cap >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(D % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(t_cap % TOKEN_BLOCK == 0, IQ_ERR_ALIGN);
  *codes_bytes = B * H * t_cap * D * bits / 8;
  *meta_bytes = B * H * t_cap * (D / group) * meta_unit_bytes(mode);
  return IQ_OK;
}

int iq_v_store_bytes(int64_t B, int64_t H, int64_t t_cap, int64_t D, int group, int bits, int mode,
                     int64_t* codes_bytes, int64_t* meta_bytes) {
  IQ_CHECK(codes_bytes && meta_bytes, IQ_ERR_NULL);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && t_cap >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(t_cap % group == 0, IQ_ERR_GROUP);
  *codes_bytes = B * H * t_cap * D * bits / 8;
  *meta_bytes = B * H * (t_cap / group) * D * meta_unit_bytes(mode);
  return IQ_OK;
}

int iq_quantize_k(const void* x, int64_t sx_b, int64_t sx_h, int64_t sx_t, const void* norm, int B, int H,
                  int n, int D, int group, int bits, int mode, uint32_t* k_codes, uint16_t* k_meta,
                  int64_t t_cap, int64_t t_off, int32_t* codes_i32, void* scale16, void* zero16, void* signs16,
                  void* stream) {
  IQ_CHECK(x, IQ_ERR_NULL);
  const bool bf = act_bf16(mode);
  mode = base_mode(mode);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && n >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(D % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(aligned(x, 16) && sx_b % 8 == 0 && sx_h % 8 == 0 && sx_t % 8 == 0, IQ_ERR_ALIGN);
  IQ_CHECK((k_codes == nullptr) == (k_meta == nullptr), IQ_ERR_NULL);
  if (k_codes) {
    IQ_CHECK(t_cap % TOKEN_BLOCK == 0 && t_off >= 0, IQ_ERR_ALIGN);
    IQ_CHECK(t_off + n <= t_cap, IQ_ERR_RANGE);
    IQ_CHECK(aligned(k_codes, 4) && aligned(k_meta, 4), IQ_ERR_ALIGN);
  }
  IQ_CHECK(!(mode == IQ_MODE_SYM && zero16), IQ_ERR_MODE);
  IQ_CHECK(!(mode == IQ_MODE_ASYM && signs16), IQ_ERR_MODE);
  const bool dense = codes_i32 || scale16 || zero16 || signs16;
  IQ_CHECK(mode != IQ_MODE_HYBRID || (k_codes && !dense), IQ_ERR_MODE);
  const int64_t total = int64_t(B) * H * n * (D / group);
  if (total == 0) return IQ_OK;
  QuantOut o{k_codes, k_meta, t_cap / TOKEN_BLOCK, t_off, codes_i32, (uint16_t*)scale16, (uint16_t*)zero16,
             (uint16_t*)signs16};
  const int sym = mode == IQ_MODE_SYM;
  // a call of few groups (a decode step's tokens) takes one lane per value:
  // one thread per group would leave most of the device idle on long chains
  if (bf || (mode != IQ_MODE_HYBRID && group <= 64 && total <= LANE_MAX_GROUPS)) {
    const LaneArgs a{(const uint16_t*)x, sx_b, sx_h, sx_t, (const uint16_t*)norm, B, H, n, D, bits, mode, bf ? 1 : 0,
                     0};
    return launch_lane_or_rt(a, o, group, (hipStream_t)stream);
  }
  return dispatch_store_bits_group(bits, group, [&]<int BITS, int G>() {
    // the store-only append (no reference-format outputs) drops their registers
    auto* kern = mode == IQ_MODE_HYBRID ? quant_k_kernel<BITS, G, false, true>
                 : dense               ? quant_k_kernel<BITS, G, true>
                                       : quant_k_kernel<BITS, G, false>;
    kern<<<dim3(unsigned(ceil_div(total, 256))), 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)x, sx_b, sx_h, sx_t, (const uint16_t*)norm, B, H, n, D, sym, o);
    return launch_status();
  });
}

int iq_quantize_v(const void* x, int64_t sx_b, int64_t sx_h, int64_t sx_t, int B, int H, int n, int D,
                  int group, int bits, int mode, uint32_t* v_codes, uint16_t* v_meta, int64_t t_cap,
                  int64_t t_off, int32_t* codes_i32, void* scale16, void* zero16, void* signs16, void* stream) {
  IQ_CHECK(x, IQ_ERR_NULL);
  const bool bf = act_bf16(mode);
  mode = base_mode(mode);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && n >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(n % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(aligned(x, 2), IQ_ERR_ALIGN);
  IQ_CHECK((v_codes == nullptr) == (v_meta == nullptr), IQ_ERR_NULL);
  if (v_codes) {
    IQ_CHECK(t_cap % group == 0 && t_off % group == 0 && t_off >= 0, IQ_ERR_ALIGN);
    IQ_CHECK(t_off + n <= t_cap, IQ_ERR_RANGE);
    IQ_CHECK(aligned(v_codes, 4) && aligned(v_meta, 4), IQ_ERR_ALIGN);
  }
  IQ_CHECK(!(mode == IQ_MODE_SYM && zero16), IQ_ERR_MODE);
  IQ_CHECK(!(mode == IQ_MODE_ASYM && signs16), IQ_ERR_MODE);
  const bool dense = codes_i32 || scale16 || zero16 || signs16;
  IQ_CHECK(mode != IQ_MODE_HYBRID || (v_codes && !dense), IQ_ERR_MODE);
  const int64_t total = int64_t(B) * H * (n / group) * D;
  if (total == 0) return IQ_OK;
  QuantOut o{v_codes, v_meta, t_cap / group, t_off, codes_i32, (uint16_t*)scale16, (uint16_t*)zero16,
             (uint16_t*)signs16};
  if (bf) {
    const LaneArgs a{(const uint16_t*)x, sx_b, sx_h, sx_t, nullptr, B, H, n, D, bits, mode, 1, 1};
    return launch_lane_or_rt(a, o, group, (hipStream_t)stream);
  }
  const int sym = mode == IQ_MODE_SYM;
  return dispatch_store_bits_group(bits, group, [&]<int BITS, int G>() {
    auto* kern = mode == IQ_MODE_HYBRID ? quant_v_kernel<BITS, G, false, true>
                 : dense               ? quant_v_kernel<BITS, G, true>
                                       : quant_v_kernel<BITS, G, false>;
    kern<<<dim3(unsigned(ceil_div(total, 256))), 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)x, sx_b, sx_h, sx_t, B, H, n, D, sym, o);
    return launch_status();
  });
}

int iq_dequant_k(const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap, const void* norm, int B, int H,
                 int t0, int T, int D, int group, int bits, int mode, void* out16, float* out32, int64_t so_b,
                 int64_t so_h, int64_t so_t, void* stream) {
  IQ_CHECK(k_codes && k_meta, IQ_ERR_NULL);
  IQ_CHECK(out16 || out32, IQ_ERR_NULL);
  const bool bf = act_bf16(mode);
  mode = base_mode(mode);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && T >= 0 && t0 >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(D % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(t_cap % TOKEN_BLOCK == 0, IQ_ERR_ALIGN);
  IQ_CHECK(int64_t(t0) + T <= t_cap, IQ_ERR_RANGE);
  const int64_t total = int64_t(B) * H * T * (D / group);
  if (total == 0) return IQ_OK;
  DeqOut o{(uint16_t*)out16, out32, so_b, so_h, so_t, bf ? 1 : 0};
  return dispatch_store_bits_group(bits, group, [&]<int BITS, int G>() {
    dequant_k_kernel<BITS, G><<<dim3(unsigned(ceil_div(total, 256))), 256, 0, (hipStream_t)stream>>>(
        k_codes, k_meta, t_cap / TOKEN_BLOCK, (const uint16_t*)norm, B, H, t0, T, D, mode, o);
    return launch_status();
  });
}

int iq_dequant_v(const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B, int H, int t0, int T,
                 int D, int group, int bits, int mode, void* out16, float* out32, int64_t so_b, int64_t so_h,
                 int64_t so_t, void* stream) {
  IQ_CHECK(v_codes && v_meta, IQ_ERR_NULL);
  IQ_CHECK(out16 || out32, IQ_ERR_NULL);
  const bool bf = act_bf16(mode);
  mode = base_mode(mode);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && T >= 0 && t0 >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(T % group == 0 && t0 % group == 0 && t_cap % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(int64_t(t0) + T <= t_cap, IQ_ERR_RANGE);
  const int64_t total = int64_t(B) * H * (T / group) * D;
  if (total == 0) return IQ_OK;
  DeqOut o{(uint16_t*)out16, out32, so_b, so_h, so_t, bf ? 1 : 0};
  return dispatch_store_bits_group(bits, group, [&]<int BITS, int G>() {
    dequant_v_kernel<BITS, G><<<dim3(unsigned(ceil_div(total, 256))), 256, 0, (hipStream_t)stream>>>(
        v_codes, v_meta, t_cap / G, B, H, t0 / G, T / G, D, mode, o);
    return launch_status();
  });
}

int iq_dequant_dense(const int32_t* codes, const void* scale16, const void* zs16, int64_t outer, int64_t n,
                     int64_t inner, int group, int mode, int out_f16, void* out, void* stream) {
  IQ_CHECK(codes && scale16 && zs16 && out, IQ_ERR_NULL);
  const bool bf = act_bf16(mode);
  mode = base_mode(mode);
  IQ_CHECK(mode_ok(mode), IQ_ERR_MODE);
  IQ_CHECK(outer >= 0 && n >= 0 && inner >= 0 && (out_f16 == 0 || out_f16 == 1), IQ_ERR_SHAPE);
  IQ_CHECK(group > 0 && n % group == 0, IQ_ERR_GROUP);
  const int64_t total = outer * n * inner;
  if (total == 0) return IQ_OK;
  dequant_dense_kernel<<<dim3(unsigned(ceil_div(total, 256))), 256, 0, (hipStream_t)stream>>>(
      codes, (const uint16_t*)scale16, (const uint16_t*)zs16, outer, n, inner, group, mode == IQ_MODE_SYM, out_f16,
      bf ? 1 : 0, out);
  return launch_status();
}

namespace {
int check_window(const iq_window* w, int D) {
  if (!w) return IQ_OK;
  IQ_CHECK(w->start >= 0 && w->n >= 0 && w->m >= 0 && w->flush >= 0 && w->cap >= 0, IQ_ERR_SHAPE);
  IQ_CHECK(int64_t(w->start) + w->n + w->m <= w->cap, IQ_ERR_RANGE);
  IQ_CHECK(w->flush <= w->n + w->m, IQ_ERR_SHAPE);
  IQ_CHECK((w->n + w->m == 0 && w->flush == 0) || w->buf, IQ_ERR_NULL);
  IQ_CHECK(w->m == 0 || w->x, IQ_ERR_NULL);
  IQ_CHECK(aligned(w->buf, 2) && aligned(w->x, 2), IQ_ERR_ALIGN);
  if (w->flush == 0) return IQ_OK;
  IQ_CHECK(w->codes && w->meta, IQ_ERR_NULL);
  if (int e = check_store(w->bits, w->group, base_mode(w->mode))) return e;
  IQ_CHECK(w->axis == 0 || w->axis == 1, IQ_ERR_SHAPE);
  IQ_CHECK(!w->norm || w->axis == 0, IQ_ERR_SHAPE);
  // dequantized rows: from the lane quantizer (groups of up to 64)
  IQ_CHECK(!w->deq_rows || w->group <= 64, IQ_ERR_SHAPE);
  IQ_CHECK(w->t_off >= 0 && w->t_off + w->flush <= w->t_cap, IQ_ERR_RANGE);
  if (w->axis == 0) {
    IQ_CHECK(D % w->group == 0, IQ_ERR_GROUP);
    IQ_CHECK(w->t_cap % TOKEN_BLOCK == 0, IQ_ERR_ALIGN);
  } else {
    IQ_CHECK(w->flush % w->group == 0 && w->t_off % w->group == 0 && w->t_cap % w->group == 0, IQ_ERR_GROUP);
  }
  IQ_CHECK(aligned(w->codes, 4) && aligned(w->meta, 4), IQ_ERR_ALIGN);
  return IQ_OK;
}

WinRole to_role(const iq_window* w) {
  WinRole r{};
  if (!w) return r;
  r.buf = (uint16_t*)w->buf; r.sb = w->s_b; r.sh = w->s_h; r.st = w->s_t;
  r.start = w->start; r.n = w->n;
  r.x = (const uint16_t*)w->x; r.sxb = w->sx_b; r.sxh = w->sx_h; r.sxt = w->sx_t; r.m = w->m;
  r.F = w->flush;
  r.codes = w->codes; r.meta = w->meta; r.t_off = w->t_off;
  r.bits = w->bits; r.group = w->group; r.mode = base_mode(w->mode); r.bf = act_bf16(w->mode); r.axis = w->axis;
  r.gsh = w->group > 0 ? __builtin_ctz(unsigned(w->group)) : 0;
  r.cap_units = w->flush ? (w->axis == 0 ? w->t_cap / TOKEN_BLOCK : w->t_cap / w->group) : 0;
  r.norm = (const uint16_t*)w->norm;
  r.vec_buf = aligned(w->buf, 16) && w->s_b % 8 == 0 && w->s_h % 8 == 0 && w->s_t % 8 == 0;
  r.vec_x = aligned(w->x, 16) && w->sx_b % 8 == 0 && w->sx_h % 8 == 0 && w->sx_t % 8 == 0;
  r.deq = w->flush ? w->deq_rows : 0;
  return r;
}
}  // namespace

int iq_window_append(const iq_window* k, const iq_window* v, int B, int H, int D, void* stream) {
  IQ_CHECK(B >= 0 && H >= 0 && D > 0, IQ_ERR_SHAPE);
  if (int e = check_window(k, D)) return e;
  if (int e = check_window(v, D)) return e;
  AppendArgs a{};
  a.r[0] = to_role(k);
  a.r[1] = to_role(v);
  a.H = H; a.D = D;
  const int64_t bh = int64_t(B) * H;
  for (int r = 0; r < 2; ++r) {
    const WinRole& w = a.r[r];
    a.count[r] = bh * w.m * D;
    a.count[2 + r] = w.F == 0 ? 0 : (w.axis == 0 ? bh * w.F * (D / w.group) : bh * (w.F / w.group) * D) *
                                        role_lanes(w.group, w.mode);
  }
  int64_t at = 0;
  for (int s = 0; s < 4; ++s) {
    a.start[s] = at;
    at += ceil_div(a.count[s], 256) * 256;
  }
  if (at == 0) return IQ_OK;
  auto go = [&]<int GK>(int gv) {
    auto* kern = gv == 128 ? window_append_kernel<GK, 128> : gv == 64 ? window_append_kernel<GK, 64>
                                                                      : window_append_kernel<GK, 32>;
    kern<<<dim3(unsigned(at / 256)), 256, 0, (hipStream_t)stream>>>(a);
  };
  const int gk = a.r[0].F ? a.r[0].group : 32, gv = a.r[1].F ? a.r[1].group : 32;
  if (gk == 128) go.template operator()<128>(gv);
  else if (gk == 64) go.template operator()<64>(gv);
  else go.template operator()<32>(gv);
  return launch_status();
}

int iq_unpack_k(const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap, int B, int H, int t0, int T, int D,
                int group, int bits, int mode, int32_t* codes_i32, void* scale16, void* zs16, void* stream) {
  IQ_CHECK(k_codes && k_meta && codes_i32 && scale16 && zs16, IQ_ERR_NULL);
  const bool bf = act_bf16(mode);
  mode = base_mode(mode);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && T >= 0 && t0 >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(D % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(t_cap % TOKEN_BLOCK == 0, IQ_ERR_ALIGN);
  IQ_CHECK(int64_t(t0) + T <= t_cap, IQ_ERR_RANGE);
  const int64_t total = int64_t(B) * H * T * (D / group);
  if (total == 0) return IQ_OK;
  const UnpackOut o{codes_i32, (uint16_t*)scale16, (uint16_t*)zs16};
  return dispatch_store_bits_group(bits, group, [&]<int BITS, int G>() {
    unpack_k_kernel<BITS, G><<<dim3(unsigned(ceil_div(total, 256))), 256, 0, (hipStream_t)stream>>>(
        k_codes, k_meta, t_cap / TOKEN_BLOCK, B, H, t0, T, D, mode == IQ_MODE_SYM, bf ? 1 : 0, o);
    return launch_status();
  });
}

int iq_unpack_v(const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B, int H, int t0, int T, int D,
                int group, int bits, int mode, int32_t* codes_i32, void* scale16, void* zs16, void* stream) {
  IQ_CHECK(v_codes && v_meta && codes_i32 && scale16 && zs16, IQ_ERR_NULL);
  const bool bf = act_bf16(mode);
  mode = base_mode(mode);
  if (int e = check_store(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && H >= 0 && T >= 0 && t0 >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(T % group == 0 && t0 % group == 0 && t_cap % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(int64_t(t0) + T <= t_cap, IQ_ERR_RANGE);
  const int64_t total = int64_t(B) * H * (T / group) * D;
  if (total == 0) return IQ_OK;
  const UnpackOut o{codes_i32, (uint16_t*)scale16, (uint16_t*)zs16};
  return dispatch_store_bits_group(bits, group, [&]<int BITS, int G>() {
    unpack_v_kernel<BITS, G><<<dim3(unsigned(ceil_div(total, 256))), 256, 0, (hipStream_t)stream>>>(
        v_codes, v_meta, t_cap / G, B, H, t0 / G, T / G, D, mode == IQ_MODE_SYM, bf ? 1 : 0, o);
    return launch_status();
  });
}

}  // extern "C"
