// Shared pieces of the decode GEMV kernels (gfx950).
//
// Operand records.  Both GEMVs multiply unpacked codes by an fp16 operand
// that is shared by every lane of a wave: the query (QK^T, lane = token) or
// the attention probabilities (attn.V, lane = head_dim column).  That operand
// is laid out once per (batch, KV head, group) as a record
//     pairs [n_rep][G/2]  uint32 = {x[a_k], x[c_k]} in the unpack plan's pair order
//     osum  [n_rep]       f32    = sum_i x[i]
// A head's pairs are contiguous, so the matrix-core A operand of a 16-pair
// chunk is four 16-byte loads per lane (from global memory or LDS), and osum
// (needed for the zero-point term) is a scalar load.
//
// Matrix-core group dot (v_mfma_f32_4x4x4_16b_f16).  The instruction runs 16
// independent 4x4x4 products; block b = lane / 4, and lane 4b+i supplies row
// i of A and column i of B (the four fp16 of its operand, k = element index)
// and receives column i of D, rows 0..3 in its four result registers
// (verified on gfx950 with lane-coded operands).  With B = four unpacked codes
// of the lane's own token / column and A = the operand pairs of head
// 4q + (lane & 3), one instruction gives every lane the dot products of four
// heads over four codes: 8 instructions cover a 32-code group, and the VALU
// only unpacks codes and applies scale and zero point.
//
// The B operand is either the code pair itself (unfused kernels: the bias
// pair is subtracted with one v_pk_add_f16) or the biased magic-number pair
// (fused kernel: each accumulation starts from -sum(opnd * bias) instead of
// 0, taken from the operand record).  The pair plans keep the biases within
// 2^8 code units (iq_device.h), so the fp32 partial sums stay small.
#pragma once

#include <atomic>
#include <utility>

#include "iq_common.h"
#include "iq_device.h"

// 64-token K blocks per wave in a flash-decoding split (split = 4 waves x
// this x 64 tokens) and code pairs unpacked per matrix-core chunk.
#ifndef IQ_FLASH_BPW
#define IQ_FLASH_BPW 1
#endif
#ifndef IQ_MFMA_CH
#define IQ_MFMA_CH 8
#endif

namespace iq {

typedef const __attribute__((address_space(4))) uint32_t* cptr_u32;

constexpr int NWAVES = 4;
constexpr int WG = NWAVES * 64;

// record stride: padded to 4 dwords so every head's pairs start 16-byte aligned
__host__ __device__ constexpr int rec_dwords_rt(int G, int nrep) { return (nrep * (G / 2 + 1) + 3) & ~3; }

template <int G, int NREP>
__host__ __device__ constexpr int rec_dwords() {
  return rec_dwords_rt(G, NREP);
}

// bound on the record bytes of n_heads query heads (n_heads / n_rep records of
// n_rep heads each) over n_groups groups of G: at most G/2 + 4 dwords per head
__host__ __device__ constexpr size_t rec_bytes_bound(int64_t n_heads, int64_t n_groups, int G) {
  return size_t(n_heads) * size_t(n_groups) * size_t(G / 2 + 4) * 4;
}

template <int N, typename P>
__device__ __forceinline__ void load_words(P p, uint32_t* w) {
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
  constexpr PairTable() : a(), c() {
    for (int k = 0; k < NP; ++k) {
      a[k] = pair_code_a<BITS>(k);
      c[k] = pair_code_c<BITS>(k);
    }
  }
};

// Pair k (any k < 64, any group size) of the unpack plan for runtime bits:
// the code indices a, c of its two halves inside the group.
template <int BITS>
__device__ __forceinline__ void plan_pair_t(int k, int& a, int& c) {
  constexpr PairTable<BITS, 64> PT{};
  a = PT.a[k];
  c = PT.c[k];
}
__device__ __forceinline__ void plan_pair(int bits, int k, int& a, int& c) {
  if (bits == 2) plan_pair_t<2>(k, a, c);
  else if (bits == 3) plan_pair_t<3>(k, a, c);
  else plan_pair_t<4>(k, a, c);
}


__device__ __forceinline__ float rec_f32(cptr_u32 rec, int i) { return __builtin_bit_cast(float, rec[i]); }

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4_t mfma4(h4_t a, h4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h4_t cat_h2(h2_t lo, h2_t hi) { return __builtin_shufflevector(lo, hi, 0, 1, 2, 3); }

// The sum operand of the attn.V products.  In v_mfma_f32_4x4x4f16 each 4-lane
// block computes D[i][c] = sum_k A[i][k] B[k][c], with A row i from lane i of
// the block (the record row of head 4q + i) and B column c from lane c.  B
// column 0 of ones and column 1 of the four fields' code biases (the fields
// of pairs 2st and 2st + 1 of the plan) make the same A, already loaded for
// the code products, give sum(p) and sum(p * bias) of every head over the
// group in lanes hl = 0 and hl = 1 (columns 2 and 3 are zero): one matrix-core
// instruction per step instead of a 64-lane reduction per head.  One h4 per
// step of a plan period, lane constants built once per kernel.
template <int BITS>
struct SumRegs {
  static constexpr int NS = Plan<BITS>::NPAIR / 2;  // steps per plan period
  h4_t b[NS];
  __device__ __forceinline__ explicit SumRegs(int hl) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const uint32_t ones = 0x3c003c00u;
      const uint32_t b0 = uint32_t(__half_as_ushort(__float2half_rn(bias_a<BITS>(2 * st)))) |
                          (uint32_t(__half_as_ushort(__float2half_rn(bias_c<BITS>(2 * st)))) << 16);
      const uint32_t b1 = uint32_t(__half_as_ushort(__float2half_rn(bias_a<BITS>(2 * st + 1)))) |
                          (uint32_t(__half_as_ushort(__float2half_rn(bias_c<BITS>(2 * st + 1)))) << 16);
      uint32_t lo = hl == 0 ? ones : hl == 1 ? b0 : 0u;
      uint32_t hi = hl == 0 ? ones : hl == 1 ? b1 : 0u;
      asm("" : "+v"(lo), "+v"(hi));  // kept in VGPRs, not rebuilt in the loops
      b[st] = cat_h2(__builtin_bit_cast(h2_t, lo), __builtin_bit_cast(h2_t, hi));
    }
  }
};

// Pairs [K0, K0+CH) of one group: A rows from the record (head 4q + hl; heads
// past NREP read as zero), B from the NB code-word sets; with SUMS also the
// sums of the A rows (SumRegs) into dsum.
template <int BITS, int W, int NREP, int NB, int K0, bool BIASED, bool SUMS, typename P, int... K>
__device__ __forceinline__ void mfma_chunk(const uint32_t (&w)[NB][W], P rec, int NP, int hl,
                                           const PlanRegs<BITS>& pr, f4_t (&dv)[NB][(NREP + 3) / 4],
                                           const SumRegs<BITS>* sr, f4_t* dsum, std::integer_sequence<int, K...>) {
  constexpr int NPS = Plan<BITS>::NPAIR;
  constexpr int SBW = Plan<BITS>::WORDS;
  constexpr int CH = sizeof...(K);
  constexpr int NQ = (NREP + 3) / 4;
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
        for (int j = 0; j < NB; ++j) {
          if constexpr (BIASED) x[j][K] = extract_pair<BITS, (K0 + K) % NPS>(&w[j][((K0 + K) / NPS) * SBW], pr);
          else x[j][K] = extract_codes<BITS, (K0 + K) % NPS>(&w[j][((K0 + K) / NPS) * SBW], pr);
        }
      }(),
      ...);
#pragma unroll
  for (int st = 0; st < CH / 2; ++st) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const h4_t a4 = cat_h2(__builtin_bit_cast(h2_t, av[q][2 * st]), __builtin_bit_cast(h2_t, av[q][2 * st + 1]));
#pragma unroll
      for (int j = 0; j < NB; ++j) dv[j][q] = mfma4(a4, cat_h2(x[j][2 * st], x[j][2 * st + 1]), dv[j][q]);
      if constexpr (SUMS) dsum[q] = mfma4(a4, sr->b[((K0 + 2 * st) % NPS) / 2], dsum[q]);
    }
  }
}

// (RS: the dwords from one record row to the next, G / 2 unless padded)
template <int BITS, int G, int NREP, int NB, int C, int NCH, bool BIASED, bool SUMS = false, int RS = G / 2,
          typename P>
__device__ __forceinline__ void mfma_chunks(const uint32_t (&w)[NB][G * BITS / 32], P rec, int hl,
                                            const PlanRegs<BITS>& pr, f4_t (&dv)[NB][(NREP + 3) / 4],
                                            const SumRegs<BITS>* sr = nullptr, f4_t* dsum = nullptr) {
  if constexpr (C < NCH) {
    constexpr int CH = (G / 2) / NCH;
    static_assert(!SUMS || (CH % 2 == 0 && (C * CH) % 2 == 0), "sum steps cover whole pairs of pairs");
    mfma_chunk<BITS, G * BITS / 32, NREP, NB, C * CH, BIASED, SUMS>(w, rec, RS, hl, pr, dv, sr, dsum,
                                                                    std::make_integer_sequence<int, CH>{});
    mfma_chunks<BITS, G, NREP, NB, C + 1, NCH, BIASED, SUMS, RS>(w, rec, hl, pr, dv, sr, dsum);
  }
}

// Query operand record (QK^T) of one group:
//     pairs [2*n_rep][G/2]  rows h < n_rep: fp16 query pairs, or with key
//                           normalization the high parts hi = fp16(q*n);
//                           rows n_rep + h: the low parts lo = fp16(q*n - hi)
//                           (key normalization only)
//     osum  [n_rep]  f32    sum_i q_i (times n_i)
//     nbsum [2*n_rep] f32   -sum_i x[i] * bias(i) of every row (hi and lo),
//                           16-byte aligned: the initial accumulators of the
//                           fused kernel's biased matrix-core products (built
//                           by the fused kernel only)
// q*n is exact in fp32 and hi + lo holds it to 2^-22, so folding the key
// normalization into the query costs no precision (rounding q*n to one fp16
// moves the logits by ~1e-4 relative, which exp() turns into ~1e-3 of the
// attention output).
template <int G, int NREP>
__host__ __device__ constexpr int qrec_osum() {
  return NREP * G;
}
template <int G, int NREP>
__host__ __device__ constexpr int qrec_nbsum() {
  return (NREP * G + NREP + 3) & ~3;
}
template <int G, int NREP>
__host__ __device__ constexpr int qrec_dwords() {
  return (qrec_nbsum<G, NREP>() + 2 * NREP + 3) & ~3;
}

// pair (ia, ic) of query row qrow (and norm row nrow, or null): writes the hi
// pair to *hi and, with a norm, the lo pair to *lo; adds the pair to sum.
// the same from already loaded fp16 values (na, nc ignored without a norm)
__device__ __forceinline__ void qrec_pair_vals(uint16_t ua, uint16_t uc, uint16_t na, uint16_t nc, bool norm,
                                               uint32_t* hi, uint32_t* lo, float& sum) {
  if (!norm) {
    *hi = uint32_t(ua) | (uint32_t(uc) << 16);
    sum += h2f(ua) + h2f(uc);
    return;
  }
  const float qa = h2f(ua) * h2f(na), qc = h2f(uc) * h2f(nc);  // exact
  const uint16_t ha = __half_as_ushort(__float2half_rn(qa)), hc = __half_as_ushort(__float2half_rn(qc));
  *hi = uint32_t(ha) | (uint32_t(hc) << 16);
  *lo = uint32_t(__half_as_ushort(__float2half_rn(qa - h2f(ha)))) |
        (uint32_t(__half_as_ushort(__float2half_rn(qc - h2f(hc)))) << 16);
  sum += qa + qc;
}
// the same for bf16 query (and factor) values: q * n is exact in fp32 (8-bit
// significands), and its hi/lo fp16 parts hold it to 2^-22 (no factor: n = 1)
__device__ __forceinline__ void qrec_pair_vals_bf(uint16_t ua, uint16_t uc, uint16_t na, uint16_t nc, bool norm,
                                                  uint32_t* hi, uint32_t* lo, float& sum) {
  const float qa = bf2f(ua) * (norm ? bf2f(na) : 1.f), qc = bf2f(uc) * (norm ? bf2f(nc) : 1.f);
  const uint16_t ha = __half_as_ushort(__float2half_rn(qa)), hc = __half_as_ushort(__float2half_rn(qc));
  *hi = uint32_t(ha) | (uint32_t(hc) << 16);
  *lo = uint32_t(__half_as_ushort(__float2half_rn(qa - h2f(ha)))) |
        (uint32_t(__half_as_ushort(__float2half_rn(qc - h2f(hc)))) << 16);
  sum += qa + qc;
}
__device__ __forceinline__ void qrec_pair(const uint16_t* qrow, const uint16_t* nrow, int ia, int ic, uint32_t* hi,
                                          uint32_t* lo, float& sum) {
  qrec_pair_vals(qrow[ia], qrow[ic], nrow ? nrow[ia] : uint16_t(0), nrow ? nrow[ic] : uint16_t(0), nrow != nullptr,
                 hi, lo, sum);
}

// dv[j][q][i] = sum over the group's pairs of opnd(head 4q+i) . codes(set j),
// rec = this group's operand record (global memory or LDS; each lane loads
// the row of head 4q + hl).  Pairs go IQ_MFMA_CH at a time so the extracted
// codes stay within IQ_MFMA_CH*NB VGPRs.
template <int BITS, int G, int NREP, int NB, typename P>
__device__ __forceinline__ void group_mfma(const uint32_t (&w)[NB][G * BITS / 32], P rec, int hl,
                                           const PlanRegs<BITS>& pr, f4_t (&dv)[NB][(NREP + 3) / 4]) {
  constexpr int NP = G / 2;
  constexpr int NCH = NP <= IQ_MFMA_CH ? 1 : NP / IQ_MFMA_CH;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int q = 0; q < (NREP + 3) / 4; ++q) dv[j][q] = f4_t{0.f, 0.f, 0.f, 0.f};
  mfma_chunks<BITS, G, NREP, NB, 0, NCH, false>(w, rec, hl, pr, dv);
}

// The same over biased code pairs: dv[j][q] starts at init[q] (rows 4q..4q+3:
// -sum(opnd * bias) of the record's rows), which removes the biases exactly
// in the accumulation.
template <int BITS, int G, int NREP, int NB, typename P>
__device__ __forceinline__ void group_mfma_biased(const uint32_t (&w)[NB][G * BITS / 32], P rec, int hl,
                                                  const PlanRegs<BITS>& pr, const f4_t (&init)[(NREP + 3) / 4],
                                                  f4_t (&dv)[NB][(NREP + 3) / 4]) {
  constexpr int NP = G / 2;
  constexpr int NCH = NP <= IQ_MFMA_CH ? 1 : NP / IQ_MFMA_CH;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int q = 0; q < (NREP + 3) / 4; ++q) dv[j][q] = init[q];
  mfma_chunks<BITS, G, NREP, NB, 0, NCH, true>(w, rec, hl, pr, dv);
}

// group_mfma_biased from zero accumulators, plus the record rows' sums:
// dsum[q] element i holds, in the lanes with hl = 0, sum(p) of head 4q + i
// over the group and, in the lanes with hl = 1, sum(p * bias) (SumRegs).
template <int BITS, int G, int NREP, int NB, int RS = G / 2, typename P>
__device__ __forceinline__ void group_mfma_biased_sums(const uint32_t (&w)[NB][G * BITS / 32], P rec, int hl,
                                                       const PlanRegs<BITS>& pr, const SumRegs<BITS>& sr,
                                                       f4_t (&dv)[NB][(NREP + 3) / 4], f4_t (&dsum)[(NREP + 3) / 4]) {
  constexpr int NP = G / 2;
  constexpr int NCH = NP <= IQ_MFMA_CH ? 1 : NP / IQ_MFMA_CH;
#pragma unroll
  for (int q = 0; q < (NREP + 3) / 4; ++q) {
    dsum[q] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NB; ++j) dv[j][q] = f4_t{0.f, 0.f, 0.f, 0.f};
  }
  mfma_chunks<BITS, G, NREP, NB, 0, NCH, true, true, RS>(w, rec, hl, pr, dv, &sr, &dsum[0]);
}

// Query dot products of NB code sets: d[j][h] = sum_i q'[h,i] c_j[i] over the
// group, from the hi rows or, when split, hi + lo rows of the query record.
template <int BITS, int G, int NREP, int NB, typename P>
__device__ __forceinline__ void qk_group_dot(const uint32_t (&w)[NB][G * BITS / 32], P rec, int hl, bool split,
                                             const PlanRegs<BITS>& pr, float (&d)[NB][NREP]) {
  if (split) {
    f4_t dv[NB][(2 * NREP + 3) / 4];
    group_mfma<BITS, G, 2 * NREP, NB>(w, rec, hl, pr, dv);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int h = 0; h < NREP; ++h) d[j][h] = dv[j][h / 4][h % 4] + dv[j][(NREP + h) / 4][(NREP + h) % 4];
  } else {
    f4_t dv[NB][(NREP + 3) / 4];
    group_mfma<BITS, G, NREP, NB>(w, rec, hl, pr, dv);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int h = 0; h < NREP; ++h) d[j][h] = dv[j][h / 4][h % 4];
  }
}

// qk_group_dot over biased code pairs; rec is a query record in LDS (its
// nbsum rows seed the accumulators)
template <int BITS, int G, int NREP, int NB>
__device__ __forceinline__ void qk_group_dot_biased(const uint32_t (&w)[NB][G * BITS / 32], const uint32_t* rec, int hl,
                                                    bool split, const PlanRegs<BITS>& pr, float (&d)[NB][NREP]) {
  const f4_t* nb = reinterpret_cast<const f4_t*>(rec + qrec_nbsum<G, NREP>());
  if (split) {
    constexpr int NQ = (2 * NREP + 3) / 4;
    f4_t init[NQ], dv[NB][NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) init[q] = nb[q];
    group_mfma_biased<BITS, G, 2 * NREP, NB>(w, rec, hl, pr, init, dv);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int h = 0; h < NREP; ++h) d[j][h] = dv[j][h / 4][h % 4] + dv[j][(NREP + h) / 4][(NREP + h) % 4];
  } else {
    constexpr int NQ = (NREP + 3) / 4;
    f4_t init[NQ], dv[NB][NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) init[q] = nb[q];
    group_mfma_biased<BITS, G, NREP, NB>(w, rec, hl, pr, init, dv);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int h = 0; h < NREP; ++h) d[j][h] = dv[j][h / 4][h % 4];
  }
}

// ---- host-side launchers shared between translation units -----------------
namespace detail {
int qk_record_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, int B, int Hq, int Hkv, int D,
                     int group, int bits, uint32_t* rec, hipStream_t stream);
// split: the records carry hi/lo query rows (built with a key normalization)
int qk_main_launch(const uint32_t* rec, int split, const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap,
                   int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float scale, float* out,
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
int qk_flash_launch(const uint32_t* rec, int split, const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap,
                    int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float scale,
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
// grid > 0: the partials of the persistent kernel's runs (slots [0, runs of
// the (batch, KV head)) of nsplit per (batch, KV head), a grid of `grid`
// workgroups); grid = 0: every one of the nsplit slots
int av_combine_launch(const float* part, int nsplit, int B, int Hq, int D, const OutPair& o, int accumulate,
                      hipStream_t stream, int grid = 0, int nrep = 1);
// The fused flash-decoding kernel (QK^T + softmax + attn.V, persistent) for
// K and V stores of the same group size (any bit widths); writes split
// statistics and partials that the same combine merges as the unfused path's.
struct FusedStore {
  const uint32_t* codes;
  const uint16_t* meta;
  int64_t t_cap;
  int t0;  // first store token of the range
  int bits, group, mode;
};
// the fused kernel reads each (batch, KV head) slice through 32-bit buffer offsets
bool flash_fused_supported(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const FusedStore& k,
                           const FusedStore& v, int Hq, int Hkv, int D);
// launch = false: only *grid (the workgroup count the launch would take) is
// set, nothing is launched
int flash_fused_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const FusedStore& k,
                       const FusedStore& v, int B, int Hq, int Hkv, int T, int D, float scale, float* ml,
                       float* part, int* grid, hipStream_t stream, bool launch = true);
// Work partition of the persistent fused kernel: which splits of the
// (batch, KV head)-major split list each workgroup streams, and in which
// split slot each of its runs (maximal pieces of one (batch, KV head))
// leaves its partial.  The kernel and both combine kernels derive it from
// (grid, heads, splits per head) alone.  Workgroups are dealt to the XCDs
// round robin (workgroup b runs on XCD b % 8).
//
// plain:  one list (every head's splits in order), one equal contiguous share
//         per workgroup; share (b % 8) * (grid / 8) + b / 8 for workgroup b, so
//         XCD x streams the x-th contiguous eighth of the list.  The runs of a
//         head come from the consecutive shares holding its splits and take
//         slots [0, nr) in share order.
// paired: each head's splits are cut at e0: [0, e0) belong to side 0, [e0,
//         nsplit) to side 1.  Side s's parts of all heads, in head order,
//         form list s; the even XCDs (side 0) and the odd XCDs (side 1) each
//         take their list in equal contiguous shares, XCD 2k / 2k + 1 the k-th
//         quarter, so an XCD pair streams the two parts of the same heads.
//         Used where shares and head parts align (workgroups per side a
//         multiple of the heads, kk shares per part, or the other way round,
//         whole parts per share): a run of side s in share sh takes slot
//         s * kk + sh % kk of its head's 2 kk.
//         The cut is e0_num / 128 of a head (fused_pair_e0: which kernels
//         use it, and where).
struct ShareMap {
  static constexpr int XCDS = 8;  // accelerator complex dies of an MI355X
  static constexpr int E0_DEN = 128;
  int grid, nhead, nsplit;
  int e0;      // splits of a head on side 0 (plain: nsplit)
  int paired;  // 1: two sides
  int kk;      // paired: shares per head part (1: whole parts per share)

  // e0_num > 0 asks for the paired partition: used wherever the grid deals
  // evenly over the XCDs, a head has at least four splits, a workgroup
  // streams at least eight splits on average, and shares align with head
  // parts; plain otherwise
  __host__ __device__ static ShareMap make(int grid, int nhead, int nsplit, int e0_num) {
    ShareMap m{grid, nhead, nsplit, nsplit, 0, 1};
    const int w = grid / 2;
    if (e0_num > 0 && grid >= 2 * XCDS && grid % XCDS == 0 && nsplit >= 4 && nhead > 0 &&
        int64_t(nhead) * nsplit >= int64_t(8) * grid && (w % nhead == 0 || nhead % w == 0)) {
      m.paired = 1;
      m.kk = w >= nhead ? w / nhead : 1;
      m.e0 = (nsplit * e0_num + E0_DEN / 2) / E0_DEN;
      m.e0 = m.e0 < m.kk ? m.kk : m.e0 > nsplit - m.kk ? nsplit - m.kk : m.e0;
    }
    return m;
  }
  __host__ __device__ int len(int side) const { return side ? nsplit - e0 : e0; }
  __host__ __device__ int first(int side) const { return side ? e0 : 0; }  // a head's first split of the side
  __host__ __device__ int width() const { return paired ? grid / 2 : grid; }  // workgroups per side
  __host__ __device__ int64_t items(int side) const { return int64_t(nhead) * len(side); }
  // side and side-local share of workgroup b
  __host__ __device__ void share(int b, int& side, int& sh) const {
    if (grid % XCDS) {
      side = 0;
      sh = b;
      return;
    }
    const int x = b % XCDS, r = b / XCDS, per = grid / XCDS;
    side = paired ? x & 1 : 0;
    sh = (paired ? x >> 1 : x) * per + r;
  }
  // first list position of share sh of a side (sh = width(): the list's end)
  __host__ __device__ int64_t begin(int side, int sh) const { return int64_t(sh) * items(side) / width(); }
  // plain: the share holding list position j
  __host__ __device__ int share_of(int64_t j) const { return int(((j + 1) * grid + items(0) - 1) / items(0)) - 1; }
  // runs (= partial slots) of head h
  __host__ __device__ int nruns(int h) const {
    if (paired) return 2 * kk;
    return share_of(int64_t(h + 1) * nsplit - 1) - share_of(int64_t(h) * nsplit) + 1;
  }
  // paired: the slot of every run in share sh of a side
  __host__ __device__ int paired_slot(int side, int sh) const { return side * kk + sh % kk; }
  // split slot of head h's run in share sh of a side
  __host__ __device__ int slot(int side, int sh, int h) const {
    return paired ? paired_slot(side, sh) : sh - share_of(int64_t(h) * nsplit);
  }
};

// The decode kernel's partition per store format: 4-bit K and V take the
// paired partition with a 68/128 cut (ShareMap e0_num), every other format
// the plain one.  Per-workgroup end times of the 4/4-bit kernel at the
// headline shape showed the odd XCDs of an MI355X finishing ~3 us after the
// even ones on every launch of equal shares (two boxes); cuts of 66-68 / 128
// measured 1.1-1.9 us faster per launch there (four boxes, same-box A/B).
// The same A/B at the other formats measured: 2-bit K / 4-bit V (config-4
// layer) equal at 66 and 0.5-1.5 us slower at 64 and 68-70, 3-bit sym K and V
// 0.7 us slower at 66-68, attn.V only (2-bit, G = 64) 1.1-2.4 us slower.
__host__ __device__ inline int fused_pair_e0(int kbits, int vbits, bool hybrid_v) {
  return kbits == 4 && vbits == 4 && !hybrid_v ? 68 : 0;
}

// the fused kernel's arguments (filled by flash_fused_launch)
struct FusedArgs {
  const uint16_t* q;
  int64_t sqb, sqh;
  const uint16_t* norm;  // [B*Hkv][D] or null
  const uint32_t* kc;
  const uint16_t* km;
  int64_t k_cap_blocks;
  int kblk0, ksym;
  const uint32_t* vc;
  const uint16_t* vm;
  int64_t v_cap_groups;
  int vg0, vsym;
  int Hkv, T;          // T: tokens of the range, a multiple of G
  int nsplit, nitems;  // splits per (batch, KV head); nsplit * B * Hkv
  uint32_t k_code_bytes, k_meta_bytes, v_code_bytes, v_meta_bytes, q_bytes, norm_bytes;
  float scale_log2;    // scale * log2(e)
  float* ml;           // [nsplit][B*Hq][2]
  float* part;         // [nsplit][B*Hq][D]
  int64_t sob, soh;    // QK^T only: strides of the logits output (part)
  // 1: empty statistics in the split slots past a (batch, KV head)'s run
  // partials (a combine that scans every slot needs them; one told the
  // launch's workgroup count reads only the run slots)
  int empty_stats;
  int pair_e0;  // the partition (ShareMap e0_num; 0: plain)
  int khyb;     // 1: a hybrid K store (meta as asym, the group's flag picks sym)
};
// its launch per K bit width (iq_flash_k{2,3,4}.hip)
int flash_fused_launch_k2(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                          hipStream_t stream, bool launch);
int flash_fused_launch_k3(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                          hipStream_t stream, bool launch);
int flash_fused_launch_k4(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                          hipStream_t stream, bool launch);
// for a bf16 layer (iq_flash_bf_k{2,3,4}.hip, iq_flash_bf_vh_k{2,3,4}.hip: hybrid V)
int flash_fused_launch_bf_k2(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                             hipStream_t stream, bool launch);
int flash_fused_launch_bf_k3(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                             hipStream_t stream, bool launch);
int flash_fused_launch_bf_k4(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                             hipStream_t stream, bool launch);
int flash_fused_launch_bf_vh_k2(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                                hipStream_t stream, bool launch);
int flash_fused_launch_bf_vh_k3(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                                hipStream_t stream, bool launch);
int flash_fused_launch_bf_vh_k4(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                                hipStream_t stream, bool launch);
// and for a hybrid V store (iq_flash_vh_k{2,3,4}.hip)
int flash_fused_launch_vh_k2(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                             hipStream_t stream, bool launch);
int flash_fused_launch_vh_k3(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                             hipStream_t stream, bool launch);
int flash_fused_launch_vh_k4(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                             hipStream_t stream, bool launch);
size_t qk_record_bytes(int B, int Hq, int D);
size_t av_record_bytes(int B, int Hq, int T, int group);
size_t av_part_bytes(int B, int Hq, int T, int D, int group);
// Per-device facts, looked up once per device (a process may drive several
// GPUs): the current device's index (0 if it cannot be read) and its CU count
constexpr int MAX_DEVICES = 64;
int device_index();
int num_cus();
// workgroups of `kern` (nt threads) resident per CU at once on the current
// device, queried once per device and kernel (`cache`: one per kernel)
struct OccCache {
  std::atomic<int> n[MAX_DEVICES];
};
template <typename K>
int blocks_per_cu(K kern, int nt, OccCache& cache) {
  std::atomic<int>& slot = cache.n[device_index()];
  int v = slot.load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kern, nt, 0) != hipSuccess || v <= 0) v = 1;
    slot.store(v, std::memory_order_relaxed);
  }
  return v;
}
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
