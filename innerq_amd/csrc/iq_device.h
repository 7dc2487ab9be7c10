// Device-side building blocks for the InnerQ gfx950 kernels.
//
// Packed group format (one quantization group of G codes, b bits each):
// code i sits at bits [b*i, b*i+b) of a little-endian bit string stored as
// G*b/32 32-bit words, LSB first (the convention of the reference's speedtest
// kernels, speedtest/benchmark_quantization.cu:25-84).  Asym codes are the
// unsigned field; sym codes are offset binary, u = sign*magnitude + 2^(b-1)
// (the speedtest's sym packing, benchmark_quantization.cu:128 and 161).
//
// In-register unpack ("pair plans").  A GEMV never converts codes one by one.
// A window of the group's bit string (a word, a shifted word, or an alignbit
// of two words) is masked and OR-ed with an fp16 exponent pattern in one
// v_and_or_b32, which yields two fp16 values {bias_a + c_a, bias_b + c_b}
// exactly (field LSB weight 1, bias 2^(10-p) for a field at in-half bit p).
// The fused decode kernel feeds these biased pairs to the matrix cores as
// they are and starts each accumulation from -sum(operand * bias) (exact
// powers of two, summed once per operand record), so the bias costs no VALU;
// the unfused kernels remove it with one v_pk_add_f16 per pair (exact: both
// operands are integers below 2048).  The plans keep every field at p >= 10 -
// b - 4 or so, i.e. bias / code unit <= 256 (4-bit), 64 (2-bit), 128 (3-bit):
// the fp32 partial sums stay within ~2^8 of the result, a relative error of a
// few 1e-6 per 128-code dot product.  Sym codes are offset binary
// (u = signed + 2^(b-1)), so sum(q*signed) = sum(q*u) - 2^(b-1)*sum(q),
// folded into the zero term: sym and asym unpack alike.
//
// Plans (found by exhaustive search for the fewest windows under that bias
// bound; S = window start bit, word-aligned windows are free):
//   4-bit, per word (8 codes):   pairs (i, i+4); S = -6, 0, 6, 6  (2 shifts)
//   2-bit, per word (16 codes):  pairs (i, i+8); S = -6,-6, 0,0,0, 6,6,6
//   3-bit, per 3 words (32 codes): 16 pairs over 11 windows, 8 of them
//          shifts or alignbits (24 VALU per 32 codes).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace iq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

constexpr int TOKEN_BLOCK = 64;

// ---------------------------------------------------------------------------
// pair plans
// ---------------------------------------------------------------------------
template <int BITS> struct Plan;

template <> struct Plan<4> {
  static constexpr int WORDS = 1, CODES = 8, NPAIR = 4;
  static constexpr int S[NPAIR] = {-6, 0, 6, 6};
  static constexpr int A[NPAIR] = {0, 1, 2, 3};
  static constexpr int C[NPAIR] = {4, 5, 6, 7};
};
template <> struct Plan<2> {
  static constexpr int WORDS = 1, CODES = 16, NPAIR = 8;
  static constexpr int S[NPAIR] = {-6, -6, 0, 0, 0, 6, 6, 6};
  static constexpr int A[NPAIR] = {0, 1, 2, 3, 4, 5, 6, 7};
  static constexpr int C[NPAIR] = {8, 9, 10, 11, 12, 13, 14, 15};
};
template <> struct Plan<3> {
  static constexpr int WORDS = 3, CODES = 32, NPAIR = 16;
  static constexpr int S[NPAIR] = {-4, -4, 0, 5, 5, 26, 26, 32, 32, 35, 53, 58, 61, 64, 71, 71};
  static constexpr int A[NPAIR] = {0, 1, 2, 3, 4, 10, 11, 12, 13, 14, 20, 21, 22, 23, 25, 26};
  static constexpr int C[NPAIR] = {5, 6, 7, 8, 9, 15, 16, 17, 18, 19, 24, 27, 28, 29, 30, 31};
};

template <int BITS> __host__ __device__ constexpr int pa_of(int k) { return BITS * Plan<BITS>::A[k] - Plan<BITS>::S[k]; }
template <int BITS> __host__ __device__ constexpr int pc_of(int k) { return BITS * Plan<BITS>::C[k] - Plan<BITS>::S[k] - 16; }
template <int BITS> __host__ __device__ constexpr uint32_t mask_of(int k) {
  return (((1u << BITS) - 1u) << pa_of<BITS>(k)) | (((1u << BITS) - 1u) << (16 + pc_of<BITS>(k)));
}
template <int BITS> __host__ __device__ constexpr uint32_t magic_of(int k) {
  return (uint32_t(25 - pa_of<BITS>(k)) << 10) | (uint32_t(25 - pc_of<BITS>(k)) << 26);
}
template <int BITS> __host__ __device__ constexpr float bias_a(int k) { return float(1 << (10 - pa_of<BITS>(k))); }
template <int BITS> __host__ __device__ constexpr float bias_c(int k) { return float(1 << (10 - pc_of<BITS>(k))); }

// A plan is valid when its pairs cover every code of the super-block once,
// every field lies inside its half's 10-bit mantissa at p >= 2 (bias <= 256
// code units), and every window is one the window() helper can form.
template <int BITS>
constexpr bool plan_valid() {
  using P = Plan<BITS>;
  int seen[P::CODES] = {};
  for (int k = 0; k < P::NPAIR; ++k) {
    const int pa = pa_of<BITS>(k), pc = pc_of<BITS>(k);
    if (pa < 2 || pa > 10 - BITS || pc < 2 || pc > 10 - BITS) return false;
    if (P::S[k] < -9 || P::S[k] >= 32 * P::WORDS) return false;
    ++seen[P::A[k]];
    ++seen[P::C[k]];
  }
  for (int i = 0; i < P::CODES; ++i)
    if (seen[i] != 1) return false;
  return P::CODES * BITS == 32 * P::WORDS;
}
static_assert(plan_valid<2>() && plan_valid<3>() && plan_valid<4>(), "pair plans");

// window of the super-block's bit string starting at bit S (S may be -1..-9:
// a left shift of word 0; windows past the end are zero-filled).
template <int BITS, int S>
__device__ __forceinline__ uint32_t window(const uint32_t* w) {
  constexpr int NW = Plan<BITS>::WORDS;
  if constexpr (S < 0) {
    return w[0] << (-S);
  } else if constexpr ((S & 31) == 0) {
    return w[S >> 5];
  } else if constexpr ((S >> 5) + 1 < NW) {
    return __builtin_amdgcn_alignbit(w[(S >> 5) + 1], w[S >> 5], S & 31);
  } else {
    return w[S >> 5] >> (S & 31);
  }
}

// A constant held in a VGPR and opaque to constant folding.  The asm is not
// volatile, so identical constants are CSE'd and hoisted out of loops.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
  asm("" : "+v"(c));
  return c;
}

// (x & m) | c is one v_and_or_b32.  gfx9 VOP3 has no literal operand, so the
// mask and the exponent pattern live in VGPRs (PlanRegs, materialized once
// per kernel); with literal operands the compiler would split it into
// v_and_b32 + v_or_b32.  The instruction itself must come from the compiler,
// not from inline asm: its result feeds MFMA source operands, and the
// required VALU write -> MFMA read wait states are only inserted for
// instructions the compiler's hazard recognizer can see.

// The distinct (mask, exponent pattern) pairs of a plan (4 for 4-bit, 5 for
// 2- and 3-bit) and which one each code pair uses.
template <int BITS>
struct PlanConsts {
  static constexpr int N = Plan<BITS>::NPAIR;
  int idx[N] = {};
  int nd = 0;
  uint32_t mask[N] = {}, magic[N] = {};
  constexpr PlanConsts() {
    for (int k = 0; k < N; ++k) {
      const uint32_t m = mask_of<BITS>(k), c = magic_of<BITS>(k);
      int j = 0;
      while (j < nd && !(mask[j] == m && magic[j] == c)) ++j;
      if (j == nd) {
        mask[nd] = m;
        magic[nd] = c;
        ++nd;
      }
      idx[k] = j;
    }
  }
};

// A plan's constants held in VGPRs, materialized once per kernel (the VGPR
// operands of v_and_or_b32).
template <int BITS>
struct PlanRegs {
  static constexpr PlanConsts<BITS> PC{};
  uint32_t m[PC.nd], c[PC.nd];
  __device__ __forceinline__ PlanRegs() {
#pragma unroll
    for (int j = 0; j < PC.nd; ++j) {
      m[j] = vgpr_const(PC.mask[j]);
      c[j] = vgpr_const(PC.magic[j]);
    }
  }
};

template <int BITS, int K>
__device__ __forceinline__ h2_t extract_pair(const uint32_t* w, const PlanRegs<BITS>& pr) {
  constexpr int S = Plan<BITS>::S[K];
  constexpr int J = PlanRegs<BITS>::PC.idx[K];
  const uint32_t x = (window<BITS, S>(w) & pr.m[J]) | pr.c[J];  // one v_and_or_b32
  return __builtin_bit_cast(h2_t, x);
}

// The pair's two codes as exact fp16 integers (bias removed).
template <int BITS, int K>
__device__ __forceinline__ h2_t extract_codes(const uint32_t* w, const PlanRegs<BITS>& pr) {
  constexpr h2_t bias = {_Float16(bias_a<BITS>(K)), _Float16(bias_c<BITS>(K))};
  return extract_pair<BITS, K>(w, pr) - bias;
}

__device__ __forceinline__ h2_t h2_from_halves(__half a, __half b) {
  h2_t r;
  r.x = __builtin_bit_cast(_Float16, a);
  r.y = __builtin_bit_cast(_Float16, b);
  return r;
}

__device__ __forceinline__ float h2f(uint16_t bits) {
  return __half2float(__ushort_as_half(bits));
}

// fp16 result of an fp32 value, round to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ float round_f16(float x) {
  return __half2float(__float2half_rn(x));
}

// bf16 activations (IQ_MODE_BF16): the same ops with bf16 in place of fp16
// at every rounding and storage point, as torch computes bf16 tensor ops (in
// fp32, rounded to nearest even; NaN becomes 0x7fc0).
__device__ __forceinline__ float bf2f(uint16_t bits) { return __uint_as_float(uint32_t(bits) << 16); }
__device__ __forceinline__ uint16_t f2bf(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
// the activation dtype's value of 16 stored bits, rounding, and bits
__device__ __forceinline__ float act2f(uint16_t bits, bool bf) { return bf ? bf2f(bits) : h2f(bits); }
__device__ __forceinline__ float round_act(float x, bool bf) { return bf ? bf2f(f2bf(x)) : round_f16(x); }
__device__ __forceinline__ uint16_t f2act(float x, bool bf) {
  return bf ? f2bf(x) : __half_as_ushort(__float2half_rn(x));
}

// Hybrid stores: a group's meta dword is {scale | flag << 15, zero}; the flag
// (bit 15, tested as a bit: a -0.0 scale is flagged) marks b-bit sym codes in
// offset binary, else the field holds the (b-1)-bit asym code.  (bf16 and fp16
// both keep their sign in bit 15.)
constexpr uint32_t HYB_FLAG = 0x8000u;
__device__ __forceinline__ bool hyb_sym(uint32_t mw) { return (mw & HYB_FLAG) != 0u; }
__device__ __forceinline__ float hyb_scale(uint32_t mw, bool bf = false) {
  return act2f(uint16_t(mw & 0x7fffu), bf);
}

// the reference's value of one field of a hybrid group (quant.py:153-176):
// asym u*s + z (fp32, c*s exact), sym (u - 2^(b-1))*s (exact)
__device__ __forceinline__ float hyb_value(uint32_t u, int bits, uint32_t mw, bool bf = false) {
  const float s = hyb_scale(mw, bf);
  if (hyb_sym(mw)) return __fmul_rn(float(int(u) - (1 << (bits - 1))), s);
  return __fadd_rn(__fmul_rn(float(u), s), act2f(uint16_t(mw >> 16), bf));
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
// Wave reductions with six DPP steps (no LDS traffic): pairs (quad_perm
// 1,0,3,2), quads (2,3,0,1), 8 lanes (row_half_mirror), rows of 16
// (row_mirror), then row_bcast:15 and row_bcast:31 fold rows 0-1 and 2-3 so
// that lane 63 holds the result, which is returned to every lane.  Every step
// runs on all four rows (rows without a broadcast source read 0); only lane
// 63 is meaningful after the broadcasts, and every lane it depends on has a
// source.  N independent reductions advance together, so the operands of
// each DPP step are ready without wait states, and each step is one DPP VALU
// instruction.
template <int CTRL, int N>
__device__ __forceinline__ void sum_step(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i)
    v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), CTRL, 0xf, 0xf,
                                                                  true));
}
template <int CTRL, int N>
__device__ __forceinline__ void max_step(int (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = max(v[i], __builtin_amdgcn_update_dpp(0, v[i], CTRL, 0xf, 0xf, true));
}

// float <-> int with the same order (for non-NaN values): negative floats
// have their magnitude bits reversed.  The map is its own inverse.
__device__ __forceinline__ int f2ord(float f) {
  const int i = __builtin_bit_cast(int, f);
  return i ^ ((i >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float ord2f(int i) { return __builtin_bit_cast(float, i ^ ((i >> 31) & 0x7fffffff)); }

template <int N>
__device__ __forceinline__ void wave_sum_dpp(float (&v)[N]) {
  sum_step<0xb1>(v);
  sum_step<0x4e>(v);
  sum_step<0x141>(v);
  sum_step<0x140>(v);
  sum_step<0x142>(v);
  sum_step<0x143>(v);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[i]), 63));
}
// max of non-NaN values (-inf allowed)
template <int N>
__device__ __forceinline__ void wave_max_dpp(float (&v)[N]) {
  int o[N];
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = f2ord(v[i]);
  max_step<0xb1>(o);
  max_step<0x4e>(o);
  max_step<0x141>(o);
  max_step<0x140>(o);
  max_step<0x142>(o);
  max_step<0x143>(o);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = ord2f(__builtin_amdgcn_readlane(o[i], 63));
}

// Orders one wave's LDS accesses around a point where lanes read what other
// lanes of the same wave wrote: a wave's LDS instructions execute in order,
// so only the compiler has to be kept from moving them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// wave64 reductions through the compiler's shuffle lowering
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace iq
