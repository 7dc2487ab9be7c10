// Shared pieces of the decode GEMV kernels (gfx950).
//
// Operand records.  Both GEMVs multiply unpacked code pairs by pairs of an
// fp16 operand that is the same for every lane of a wave: the query (QK^T,
// lane = token) or the attention probabilities (attn.V, lane = head_dim
// column).  That operand is laid out once per (batch, KV head, group) as a
// record
//     pairs [n_rep][G/2]  uint32 = {x[a_k], x[c_k]} in the unpack plan's pair order
//     beta  [n_rep]       f32    = sum_k x[a_k]*bias_a(k) + x[c_k]*bias_c(k)
//     osum  [n_rep]       f32    = sum_i x[i]
// and read with scalar loads (s_load_dwordx16) into SGPRs, so that every
// v_dot2_f32_f16 takes its operand pair straight from the scalar register
// file: no LDS traffic and no VGPRs for the operand.  A head's pairs are
// contiguous, so a chunk of 16 pairs of one head is one s_load_dwordx16 and
// only that chunk is live in SGPRs.
#pragma once

#include <utility>

#include "iq_common.h"
#include "iq_device.h"

namespace iq {

typedef const __attribute__((address_space(4))) uint32_t* cptr_u32;

constexpr int NWAVES = 4;
constexpr int WG = NWAVES * 64;

template <int G, int NREP>
__host__ __device__ constexpr int rec_dwords() {
  return NREP * (G / 2 + 2);
}

__host__ __device__ constexpr int rec_dwords_rt(int G, int nrep) { return nrep * (G / 2 + 2); }

template <int N>
__device__ __forceinline__ void load_words(const uint32_t* __restrict__ p, uint32_t* w) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int j = 0; j < N; j += 4) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + j);
      w[j] = u.x; w[j + 1] = u.y; w[j + 2] = u.z; w[j + 3] = u.w;
    }
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int j = 0; j < N; j += 2) {
      const uint2 u = *reinterpret_cast<const uint2*>(p + j);
      w[j] = u.x; w[j + 1] = u.y;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) w[j] = p[j];
  }
}

// code index of the first / second half of pair k of a group
template <int BITS>
__host__ __device__ constexpr int pair_code_a(int k) {
  return (k / Plan<BITS>::NPAIR) * Plan<BITS>::CODES + Plan<BITS>::A[k % Plan<BITS>::NPAIR];
}
template <int BITS>
__host__ __device__ constexpr int pair_code_c(int k) {
  return (k / Plan<BITS>::NPAIR) * Plan<BITS>::CODES + Plan<BITS>::C[k % Plan<BITS>::NPAIR];
}

template <int BITS, int NP>
struct PairTable {
  int a[NP], c[NP];
  float ba[NP], bc[NP];
  constexpr PairTable() : a(), c(), ba(), bc() {
    for (int k = 0; k < NP; ++k) {
      a[k] = pair_code_a<BITS>(k);
      c[k] = pair_code_c<BITS>(k);
      ba[k] = bias_a<BITS>(k % Plan<BITS>::NPAIR);
      bc[k] = bias_c<BITS>(k % Plan<BITS>::NPAIR);
    }
  }
};

// Pair k (any k < 64, any group size) of the unpack plan for runtime bits:
// code indices a, c inside the group and the fp16 biases of the two halves.
template <int BITS>
__device__ __forceinline__ void plan_pair_t(int k, int& a, int& c, float& ba, float& bc) {
  constexpr PairTable<BITS, 64> PT{};
  a = PT.a[k];
  c = PT.c[k];
  ba = PT.ba[k];
  bc = PT.bc[k];
}
__device__ __forceinline__ void plan_pair(int bits, int k, int& a, int& c, float& ba, float& bc) {
  if (bits == 2) plan_pair_t<2>(k, a, c, ba, bc);
  else if (bits == 3) plan_pair_t<3>(k, a, c, ba, bc);
  else plan_pair_t<4>(k, a, c, ba, bc);
}

template <int BITS>
__device__ __forceinline__ void to_offset_binary(uint32_t* w, int nw) {
  constexpr int SBW = Plan<BITS>::WORDS;
#pragma unroll
  for (int j = 0; j < nw; ++j) w[j] ^= Plan<BITS>::SIGN[j % SBW];
}

// The value of p, unknown to the optimizer until `after` has been computed.
// Constant-address loads count as invariant, so without this the compiler
// hoists every group's / chunk's scalar loads to the top of the kernel and
// spills SGPRs; tying the base pointer to the previous chunk's accumulator
// keeps at most one chunk of operand SGPRs live.
__device__ __forceinline__ cptr_u32 launder(cptr_u32 p, float after) {
  asm volatile("" : "+s"(p) : "v"(after));
  return p;
}

template <int OFF, int... I>
constexpr std::integer_sequence<int, (OFF + I)...> offset_seq(std::integer_sequence<int, I...>) {
  return {};
}

// Extract pairs [K0, K0+CH) of NB code-word sets into VGPRs, then for each
// head read that head's CH operand pairs (one scalar load) and accumulate.
template <int BITS, int W, int NREP, int NB, int NP, int K0, int... K>
__device__ __forceinline__ void chunk_dot(const uint32_t (&w)[NB][W], cptr_u32 rec, float (&dv)[NB][NREP],
                                          std::integer_sequence<int, K...>) {
  constexpr int NPS = Plan<BITS>::NPAIR;
  constexpr int SBW = Plan<BITS>::WORDS;
  constexpr int CH = sizeof...(K);
  h2_t x[CH][NB];
  (
      [&] {
#pragma unroll
        for (int j = 0; j < NB; ++j) x[K][j] = extract_pair<BITS, (K0 + K) % NPS>(&w[j][((K0 + K) / NPS) * SBW]);
      }(),
      ...);
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    // head h's pairs may load once head h-2 is done: two heads of operands
    // (32 SGPRs) in flight, so the scalar-load latency overlaps head h-1's dots
    const cptr_u32 r = launder(rec + h * NP + K0, dv[0][h < 2 ? 0 : h - 2]);
    (
        [&] {
          const h2_t op = __builtin_bit_cast(h2_t, r[K]);
#pragma unroll
          for (int j = 0; j < NB; ++j) dv[j][h] = dot2(op, x[K][j], dv[j][h]);
        }(),
        ...);
  }
}

template <int BITS, int G, int NREP, int NB, int C, int NCH>
__device__ __forceinline__ void chunks_from(const uint32_t (&w)[NB][G * BITS / 32], cptr_u32 rec,
                                           float (&dv)[NB][NREP]) {
  if constexpr (C < NCH) {
    constexpr int NP = G / 2;
    constexpr int CH = NP / NCH;
    chunk_dot<BITS, G * BITS / 32, NREP, NB, NP, C * CH>(w, rec, dv, std::make_integer_sequence<int, CH>{});
    chunks_from<BITS, G, NREP, NB, C + 1, NCH>(w, rec, dv);
  }
}

// One group: NB code-word sets (tokens for QK^T, columns for attn.V) against
// one operand record.  dv must be pre-initialized (to -beta).  Pairs are
// handled 16 at a time so the extracted pairs stay within 16*NB VGPRs.
template <int BITS, int G, int NREP, int NB>
__device__ __forceinline__ void group_dot_rec(const uint32_t (&w)[NB][G * BITS / 32], cptr_u32 rec,
                                              float (&dv)[NB][NREP]) {
  constexpr int NP = G / 2;
  constexpr int NCH = NP <= 16 ? 1 : NP / 16;
  chunks_from<BITS, G, NREP, NB, 0, NCH>(w, rec, dv);
}

__device__ __forceinline__ float rec_f32(cptr_u32 rec, int i) { return __builtin_bit_cast(float, rec[i]); }

// ---------------------------------------------------------------------------
// Matrix-core group dot (v_mfma_f32_4x4x4_16b_f16).
//
// The instruction runs 16 independent 4x4x4 products; block b = lane / 4,
// and lane 4b+i supplies row i of A and column i of B (the four fp16 of its
// operand, k = element index) and receives column i of D, rows 0..3 in its
// four result registers (verified on gfx950 with lane-coded operands).  With
// B = four unpacked codes of the lane's own token / column and A = the
// operand pairs of head 4q + (lane & 3), one instruction gives every lane the
// dot products of four heads over four codes: 8 instructions cover a 32-code
// group, and the VALU only unpacks codes and applies scale / zero point.
//
// The B operand is the code pair itself, not the biased magic-number pair:
// with a bias of up to 1024 per code, partial sums reach ~1e4 and cancel
// back to ~1, and the MFMA's fp32 accumulation loses ~1e-3 of the result at
// G = 128.  Subtracting the bias pair first (one v_pk_add_f16, exact because
// both operands are integers below 2048) keeps every partial sum small.
// ---------------------------------------------------------------------------
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4_t mfma4(h4_t a, h4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h4_t cat_h2(h2_t lo, h2_t hi) { return __builtin_shufflevector(lo, hi, 0, 1, 2, 3); }

template <int BITS, int W, int NREP, int NB, int K0, int... K>
__device__ __forceinline__ void mfma_chunk(const uint32_t (&w)[NB][W], const uint32_t* __restrict__ rec, int NP,
                                           int hl, f4_t (&dv)[NB][(NREP + 3) / 4],
                                           std::integer_sequence<int, K...>) {
  constexpr int NPS = Plan<BITS>::NPAIR;
  constexpr int SBW = Plan<BITS>::WORDS;
  constexpr int CH = sizeof...(K);
  constexpr int NQ = (NREP + 3) / 4;
  // A rows: pairs [K0, K0+CH) of head 4q + hl (heads past NREP read as zero)
  uint32_t av[NQ][CH];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int h = 4 * q + hl;
    if constexpr (NREP % 4 == 0) {
      load_words<CH>(rec + h * NP + K0, av[q]);
    } else {
      load_words<CH>(rec + min(h, NREP - 1) * NP + K0, av[q]);
#pragma unroll
      for (int k = 0; k < CH; ++k) av[q][k] = h < NREP ? av[q][k] : 0u;
    }
  }
  h2_t x[NB][CH];
  (
      [&] {
#pragma unroll
        for (int j = 0; j < NB; ++j) x[j][K] = extract_codes<BITS, (K0 + K) % NPS>(&w[j][((K0 + K) / NPS) * SBW]);
      }(),
      ...);
#pragma unroll
  for (int st = 0; st < CH / 2; ++st) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const h4_t a4 = cat_h2(__builtin_bit_cast(h2_t, av[q][2 * st]), __builtin_bit_cast(h2_t, av[q][2 * st + 1]));
#pragma unroll
      for (int j = 0; j < NB; ++j) dv[j][q] = mfma4(a4, cat_h2(x[j][2 * st], x[j][2 * st + 1]), dv[j][q]);
    }
  }
}

template <int BITS, int G, int NREP, int NB, int C, int NCH>
__device__ __forceinline__ void mfma_chunks(const uint32_t (&w)[NB][G * BITS / 32], const uint32_t* __restrict__ rec,
                                            int hl, f4_t (&dv)[NB][(NREP + 3) / 4]) {
  if constexpr (C < NCH) {
    constexpr int CH = (G / 2) / NCH;
    mfma_chunk<BITS, G * BITS / 32, NREP, NB, C * CH>(w, rec, G / 2, hl, dv, std::make_integer_sequence<int, CH>{});
    mfma_chunks<BITS, G, NREP, NB, C + 1, NCH>(w, rec, hl, dv);
  }
}

// dv[j][q][i] += sum over the group's pairs of opnd(head 4q+i) . codes(set j)
// (unbiased codes: no -beta start value),
// rec = this group's operand record (vector-loaded per lane: row = hl).
template <int BITS, int G, int NREP, int NB>
__device__ __forceinline__ void group_mfma(const uint32_t (&w)[NB][G * BITS / 32], const uint32_t* __restrict__ rec,
                                           int hl, f4_t (&dv)[NB][(NREP + 3) / 4]) {
  constexpr int NP = G / 2;
  constexpr int NCH = NP <= 16 ? 1 : NP / 16;
  mfma_chunks<BITS, G, NREP, NB, 0, NCH>(w, rec, hl, dv);
}

// ---- host-side launchers shared between translation units -----------------
namespace detail {
int qk_record_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, int B, int Hq, int Hkv, int D,
                     int group, int bits, uint32_t* rec, hipStream_t stream);
int qk_main_launch(const uint32_t* rec, const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap, int B,
                   int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float scale, float* out,
                   int64_t so_b, int64_t so_h, hipStream_t stream);
// Flash-decoding split size (tokens per QK^T workgroup) and the QK^T launch
// that, instead of logits, writes per-split softmax statistics (m, l) and the
// attn.V operand records of the split's probabilities exp(logit - m).
int flash_split_tokens();
struct FlashOut {
  float* ml;          // [nsplit][B*Hq][2]  (max, sum) of each split
  uint32_t* vrec;     // attn.V operand records [B*Hkv][T/vgroup]
  int vbits, vgroup;  // V store format (records follow its unpack plan)
};
int qk_flash_launch(const uint32_t* rec, const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap, int B,
                    int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float scale,
                    const FlashOut& f, hipStream_t stream);
int av_flash_launch(const uint32_t* rec, const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B,
                    int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float* part,
                    hipStream_t stream);
int av_record_launch(const void* p, int64_t sp_b, int64_t sp_h, int B, int Hq, int Hkv, int T, int group, int bits,
                     uint32_t* rec, hipStream_t stream);
struct OutPair {
  float* out32;
  int64_t s32b, s32h;
  uint16_t* out16;
  int64_t s16b, s16h;
};
int av_splits(int B, int Hkv, int T, int group);
int av_main_launch(const uint32_t* rec, const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B,
                   int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float* part,
                   hipStream_t stream);
int av_combine_launch(const float* part, int nsplit, int B, int Hq, int D, const OutPair& o, int accumulate,
                      hipStream_t stream);
size_t qk_record_bytes(int B, int Hq, int D);
size_t av_record_bytes(int B, int Hq, int T, int group);
size_t av_part_bytes(int B, int Hq, int T, int D, int group);
int num_cus();
}  // namespace detail

template <typename F>
int dispatch_shape(int bits, int group, int D, int nrep, int sym, F&& f) {
  return dispatch_bits_group(bits, group, [&]<int BITS, int G>() -> int {
    auto d2 = [&]<int DD>() -> int {
      if constexpr (G > DD) {
        return IQ_ERR_GROUP;
      } else {
        auto r2 = [&]<int R>() -> int {
          if (sym) return f.template operator()<BITS, G, DD, R, true>();
          return f.template operator()<BITS, G, DD, R, false>();
        };
        switch (nrep) {
          case 1: return r2.template operator()<1>();
          case 2: return r2.template operator()<2>();
          case 4: return r2.template operator()<4>();
          case 8: return r2.template operator()<8>();
          default: return IQ_ERR_SHAPE;
        }
      }
    };
    if (D == 64) return d2.template operator()<64>();
    if (D == 128) return d2.template operator()<128>();
    return IQ_ERR_SHAPE;
  });
}

template <typename F>
int dispatch_rec(int bits, int group, int nrep, F&& f) {
  return dispatch_bits_group(bits, group, [&]<int BITS, int G>() -> int {
    switch (nrep) {
      case 1: return f.template operator()<BITS, G, 1>();
      case 2: return f.template operator()<BITS, G, 2>();
      case 4: return f.template operator()<BITS, G, 4>();
      case 8: return f.template operator()<BITS, G, 8>();
      default: return IQ_ERR_SHAPE;
    }
  });
}

}  // namespace iq
