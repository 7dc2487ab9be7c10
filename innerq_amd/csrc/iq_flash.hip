// Fused flash-decoding split (gfx950): QK^T, softmax and attn.V of one
// (batch, KV head) over FSPLIT consecutive tokens in one workgroup, for K and
// V stores that share bit width and group size.
//
// Each of the four waves owns a sub-split of FBPW*64 consecutive tokens
// (lane = token for QK^T) and runs the whole pipeline on it alone; the waves
// meet only at the start (query records) and at the end (merge):
//   start  query operand records of the D/G head_dim groups, built in LDS
//          while every wave's first K group is in flight (a key
//          normalization, which the reference applies to the dequantized
//          keys, cache.py:128-133 and 249, is folded into q as hi/lo fp16
//          parts of q*n);
//   QK^T   the wave walks the head_dim groups with the next group's code words
//          and {scale, zero} prefetched, eight v_mfma_f32_4x4x4f16 per 32
//          codes and four query heads (iq_gemv.h); its V groups' loads are
//          issued when the last K group has arrived;
//   softmax  max m_w over the sub-split per head (DPP reduction), p =
//          exp(logit - m_w); each lane writes its fp16 p straight into its
//          slot of the wave's attn.V operand records (the inverse of the
//          unpack plan), and the wave sums l_w = sum p (fp32);
//   attn.V lane = head_dim column d = lane + 64 e over the wave's V groups
//          (G divides the sub-split);
//   merge  m = max_w m_w; each wave's output is rescaled by exp(m_w - m) and
//          the four are summed in LDS in wave order; the split's (m, l) and
//          unnormalized output go to the split statistics and partials.
// The probabilities never leave LDS, nothing is exchanged between waves in
// the middle of the pipeline (so the waves of a CU drift apart and one's
// arithmetic overlaps another's loads), and one launch replaces the
// query-record, QK^T and attn.V launches of the unfused path.  A combine
// kernel (iq_decode.hip) merges the splits.
//
// The store formats follow the unfused kernels: K codes [B,H,t_cap/64,D/G,64,W],
// V codes [B,H,t_cap/G,D,W]; sym or asym per store is a runtime flag (a
// uniform branch), so the kernel is instantiated per (bits, G, D, n_rep) only.
#include "iq_gemv.h"

using namespace iq;

namespace {

constexpr int FBPW = IQ_FLASH_BPW;                   // 64-token K blocks per wave
constexpr int WTOK = FBPW * TOKEN_BLOCK;             // tokens per wave (sub-split)
constexpr int FSPLIT = NWAVES * WTOK;                // tokens per workgroup

// V units loaded into each K group's slots as soon as QK^T has read them (1),
// or all after QK^T (0).
#ifndef IQ_FLASH_VSTREAM
#define IQ_FLASH_VSTREAM 0
#endif

// Fully unrolled group loops (1) or runtime loops (0).
#ifndef IQ_FLASH_UNROLL
#define IQ_FLASH_UNROLL 0
#endif
#if IQ_FLASH_UNROLL
#define IQ_GROUP_LOOP _Pragma("unroll")
#else
#define IQ_GROUP_LOOP _Pragma("unroll 1")
#endif

// Pair k of a group's unpack plan: code index of its first and second half.
template <int BITS>
__host__ __device__ constexpr int plan_a(int k) {
  if constexpr (BITS == 4) {
    return 8 * (k >> 2) + (k & 3);
  } else if constexpr (BITS == 2) {
    return 16 * (k >> 3) + (k & 7);
  } else {
    const int kk = k & 15;
    return 32 * (k >> 4) + (kk < 5 ? kk : kk < 10 ? kk + 5 : kk + 10);
  }
}
template <int BITS>
__host__ __device__ constexpr int plan_c(int k) {
  if constexpr (BITS == 4) return plan_a<4>(k) + 4;
  else if constexpr (BITS == 2) return plan_a<2>(k) + 8;
  else return plan_a<3>(k) + ((k & 15) < 10 ? 5 : 6);
}
template <int BITS>
constexpr bool plan_formula_ok() {
  for (int k = 0; k < 64; ++k)
    if (plan_a<BITS>(k) != pair_code_a<BITS>(k) || plan_c<BITS>(k) != pair_code_c<BITS>(k)) return false;
  return true;
}
static_assert(plan_formula_ok<2>() && plan_formula_ok<3>() && plan_formula_ok<4>(), "plan formula");

// Inverse of the plan: code i of a group sits in pair k, half hi (0: low).
template <int BITS>
__host__ __device__ constexpr void plan_inv(int i, int& k, int& hi) {
  if constexpr (BITS == 4) {
    const int r = i & 7;
    k = 4 * (i >> 3) + (r & 3);
    hi = r >> 2;
  } else if constexpr (BITS == 2) {
    const int r = i & 15;
    k = 8 * (i >> 4) + (r & 7);
    hi = r >> 3;
  } else {
    const int r = i & 31, sb = 16 * (i >> 5);
    if (r < 5) { k = sb + r; hi = 0; }
    else if (r < 10) { k = sb + r - 5; hi = 1; }
    else if (r < 15) { k = sb + r - 5; hi = 0; }
    else if (r < 20) { k = sb + r - 10; hi = 1; }
    else if (r < 26) { k = sb + r - 10; hi = 0; }
    else { k = sb + r - 16; hi = 1; }
  }
}
template <int BITS>
constexpr bool plan_inv_ok() {
  for (int i = 0; i < 128; ++i) {
    int k = 0, hi = 0;
    plan_inv<BITS>(i, k, hi);
    if ((hi ? plan_c<BITS>(k) : plan_a<BITS>(k)) != i) return false;
  }
  return true;
}
static_assert(plan_inv_ok<2>() && plan_inv_ok<3>() && plan_inv_ok<4>(), "plan inverse");

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
  int Hkv, T;  // T: tokens of the range, a multiple of G
  float scale;
  float* ml;    // [nsplit][B*Hq][2]
  float* part;  // [nsplit][B*Hq][D]
};

// Staging of packed data in LDS.  A "unit" is the data of 64 lanes for one
// (K block, head_dim group) or one (V group, 64-column set): 64 x W code words
// in chunks of CW words per lane ([chunk][lane][CW] words, one direct
// global->LDS load per chunk) followed by 256 bytes of {scale, zero} (asym:
// one dword per lane; sym: the 128 bytes of 64 fp16 scales, loaded as 32
// dwords).  Each wave stages its own units in a private region: all of its K
// units at kernel start, then, once its QK^T is done, its V units in the same
// place.  Loads land in LDS without occupying VGPRs, so a wave has every byte
// of its sub-split in flight at once.
template <int W>
struct Stage {
  static constexpr int CW = W % 4 == 0 ? 4 : 1;  // words per lane per load (16- or 4-byte loads)
  static constexpr int NCHK = W / CW;
  static constexpr int META = W * 256;              // byte offset of the meta block
  static constexpr int UNIT = (W + 1) * 256;        // bytes per unit
};

// Records use the padded stride rec_dwords(): each head's pairs start 16-byte
// aligned, as the 16-byte LDS reads of the matrix-core operand require.
template <int BITS, int G, int D, int NREP>
struct FusedSmem {
  static constexpr int W = G * BITS / 32;
  static constexpr int NUNITS = (D / G) * FBPW;  // = (WTOK / G) * (D / 64)
  static constexpr int QDW = NREP * D / 2;                 // query dwords (fp16 pairs)
  static constexpr int QDW_PAD = (QDW + 63) / 64 * 64;     // whole 64-lane loads
  alignas(16) uint32_t qrec[D / G][qrec_dwords<G, NREP>()];
  alignas(16) uint32_t vrec[NWAVES][WTOK / G][rec_dwords<G, NREP>()];
  alignas(16) uint32_t qraw[QDW_PAD];  // q rows of the n_rep heads, [h][D] fp16
  alignas(16) uint32_t nraw[64];       // key normalization row, D fp16
  union alignas(16) {
    unsigned char stage[NWAVES][NUNITS * Stage<W>::UNIT];  // until attn.V ends
    float red[NWAVES - 1][NREP][D];                         // merge
  };
  float m[NWAVES][NREP];
  float l[NWAVES][NREP];
};

// Direct global->LDS load of BYTES per lane (4 or 16); lane i's data lands
// at lds + i * BYTES.
template <int BYTES>
__device__ __forceinline__ void dma_t(const void* src, void* lds) {
  auto* l = (__attribute__((address_space(3))) void*)lds;
  if constexpr (BYTES == 16) __builtin_amdgcn_global_load_lds(src, l, 16, 0, 0);
  else if constexpr (BYTES == 4) __builtin_amdgcn_global_load_lds(src, l, 4, 0, 0);
  else static_assert(BYTES == 4, "direct LDS loads of 4 or 16 bytes per lane");
}

// The compiler does not order LDS reads after direct LDS loads: every read
// of a stage region is preceded by an explicit wait for the loads.
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_lgkm_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier for data exchanged through LDS only.  __syncthreads()
// would also wait for every outstanding global load, direct LDS loads
// included, i.e. for the wave's whole stage stream; the stage regions are
// wave-private, so only the LDS writes need to be complete.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// issue the loads of one unit: codes at src (this lane's first word) and meta
template <int W>
__device__ __forceinline__ void stage_unit(unsigned char* unit, const uint32_t* codes, const uint16_t* meta_unit0,
                                           int lane, int sym) {
  using S = Stage<W>;
#pragma unroll
  for (int c = 0; c < S::NCHK; ++c) dma_t<S::CW * 4>(codes + c * S::CW, unit + c * 64 * S::CW * 4);
  // asym: one {scale, zero} dword per lane; sym: 64 fp16 scales = 32 dwords,
  // lanes 32-63 re-load them into the unused upper half of the meta block
  const uint32_t* m32 = reinterpret_cast<const uint32_t*>(meta_unit0);
  dma_t<4>(m32 + (sym ? (lane & 31) : lane), unit + S::META);
}

// read back this lane's words and meta of one unit
template <int W>
__device__ __forceinline__ void read_unit(const unsigned char* unit, int lane, int sym, uint32_t (&w)[W],
                                          uint32_t& meta) {
  using S = Stage<W>;
#pragma unroll
  for (int c = 0; c < S::NCHK; ++c) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(unit + (c * 64 + lane) * S::CW * 4);
    if constexpr (S::CW == 4) {
      const uint4 u = *reinterpret_cast<const uint4*>(p);
      w[4 * c] = u.x; w[4 * c + 1] = u.y; w[4 * c + 2] = u.z; w[4 * c + 3] = u.w;
    } else {
#pragma unroll
      for (int x = 0; x < S::CW; ++x) w[c * S::CW + x] = p[x];
    }
  }
  if (sym) meta = reinterpret_cast<const uint16_t*>(unit + S::META)[lane];
  else meta = reinterpret_cast<const uint32_t*>(unit + S::META)[lane];
}

template <int BITS, int G, int D, int NREP>
__global__ __launch_bounds__(WG) void flash_fused_kernel(FusedArgs a) {
  constexpr int NG = D / G;
  constexpr int W = G * BITS / 32;
  constexpr int NP = G / 2;
  constexpr int VPW = WTOK / G;  // V groups per wave
  constexpr int RD = rec_dwords<G, NREP>();
  constexpr int DPL = D / 64;
  constexpr int UB = Stage<W>::UNIT;
  constexpr float ZS = -float(1 << (BITS - 1));
  static_assert(WTOK % G == 0, "a V group lies inside one wave's tokens");
  __shared__ FusedSmem<BITS, G, D, NREP> sm;

  const int bh = blockIdx.y;
  const int split = blockIdx.x;
  const int b = bh / a.Hkv, kvh = bh % a.Hkv;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hl = lane & 3;
  const int wt0 = (split * NWAVES + wave) * WTOK;  // first token of the wave's sub-split
  unsigned char* stage = sm.stage[wave];

  // ---- q rows (and the norm row) into LDS, issued ahead of the K stream ----
  // Direct LDS loads complete in order with the stage loads issued after
  // them; a wait for "all but the K loads" then covers exactly these.
  using SM = FusedSmem<BITS, G, D, NREP>;
  constexpr int QLOADS = SM::QDW_PAD / 64;  // 64-dword loads over the workgroup
  constexpr int QLPW = (QLOADS + NWAVES - 1) / NWAVES;
  const bool qsplit = a.norm != nullptr;
  {
    const uint16_t* qb = a.q + b * a.sqb + int64_t(kvh * NREP) * a.sqh;
#pragma unroll
    for (int r = 0; r < QLPW; ++r) {
      const int c = min(wave + NWAVES * r, QLOADS - 1);  // waves past the loads repeat the last one
      const int i = min(c * 64 + lane, SM::QDW - 1);      // dword: head i / (D/2), pair i % (D/2)
      const int h = i / (D / 2), dd = i % (D / 2);
      dma_t<4>(qb + h * a.sqh + 2 * dd, &sm.qraw[c * 64]);
    }
    const uint16_t* nb = a.norm ? a.norm + int64_t(bh) * D : qb;  // the q row itself when unused
    dma_t<4>(nb + 2 * min(lane, D / 2 - 1), &sm.nraw[0]);
  }
  // ---- every K unit of the wave into its stage region ----
  // blocks past the range (tail waves) re-read its last block: in-bounds
  // loads whose tokens are masked out
  {
    const int nblk = (a.T + TOKEN_BLOCK - 1) / TOKEN_BLOCK;
    const int64_t kbase = int64_t(bh) * a.k_cap_blocks + a.kblk0;
    const uint32_t* kcb = a.kc + kbase * (NG * TOKEN_BLOCK * W);
    const uint16_t* kmb = a.km + kbase * (NG * TOKEN_BLOCK * (a.ksym ? 1 : 2));
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int j = 0; j < FBPW; ++j) {
        const int blk = min(wt0 / TOKEN_BLOCK + j, nblk - 1);
        const int64_t unit0 = (int64_t(blk) * NG + g) * TOKEN_BLOCK;
        stage_unit<W>(stage + (g * FBPW + j) * UB, kcb + (unit0 + lane) * W,
                      kmb + unit0 * (a.ksym ? 1 : 2), lane, a.ksym);
      }
  }

  // ---- query records (the only workgroup-wide step before the merge) ----
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NG * FBPW * (Stage<W>::NCHK + 1)) : "memory");
  lds_barrier();
  {
    const uint16_t* qh = reinterpret_cast<const uint16_t*>(sm.qraw);
    const uint16_t* nh = reinterpret_cast<const uint16_t*>(sm.nraw);
    for (int i = tid; i < NG * NREP * NP; i += WG) {
      const int k = i % NP, h = (i / NP) % NREP, g = i / (NP * NREP);
      const int ia = g * G + plan_a<BITS>(k), ic = g * G + plan_c<BITS>(k);
      float unused = 0.f;
      qrec_pair_vals(qh[h * D + ia], qh[h * D + ic], nh[ia], nh[ic], qsplit, &sm.qrec[g][h * NP + k],
                     &sm.qrec[g][(NREP + h) * NP + k], unused);
    }
    lds_barrier();
    if (tid < NG * NREP) {
      const int g = tid / NREP, h = tid % NREP;
      float s = 0.f;
      for (int k = 0; k < NP; ++k) {
        const uint32_t u = sm.qrec[g][h * NP + k];
        s += h2f(uint16_t(u & 0xffffu)) + h2f(uint16_t(u >> 16));
        if (qsplit) {
          const uint32_t v = sm.qrec[g][(NREP + h) * NP + k];
          s += h2f(uint16_t(v & 0xffffu)) + h2f(uint16_t(v >> 16));
        }
      }
      sm.qrec[g][qrec_osum<G, NREP>() + h] = __float_as_uint(s);
    }
    lds_barrier();
  }

  // ---- QK^T over the wave's tokens, from the stage; V streams in behind ----
  // Group g's K units occupy slots [g*FBPW, (g+1)*FBPW); once they are read,
  // the V units of the same slots are loaded there (slot = V group * DPL +
  // column set).  Every wave loads every V unit (groups past the range
  // re-read the range's last group), so the load counts are compile-time:
  // before group g, the outstanding loads are the K loads of groups > g plus
  // the V loads of groups < g, NG - 1 groups' worth in all.
  constexpr int KPG = FBPW * (Stage<W>::NCHK + 1);  // loads per group of slots
  const int vg_last = a.T / G - 1;                  // T is a multiple of G
  const int64_t vbase = int64_t(bh) * a.v_cap_groups + a.vg0;
  auto stage_v = [&](int slot0) {
#pragma unroll
    for (int j = 0; j < FBPW; ++j) {
      const int slot = slot0 + j, u = slot / DPL, e = slot % DPL;
      const int64_t unit0 = (vbase + min(wt0 / G + u, vg_last)) * D + 64 * e;
      stage_unit<W>(stage + slot * UB, a.vc + (unit0 + lane) * W, a.vm + unit0 * (a.vsym ? 1 : 2), lane, a.vsym);
    }
  };
  const PlanRegs<BITS> pr;
  float acc[FBPW][NREP];
#pragma unroll
  for (int j = 0; j < FBPW; ++j)
#pragma unroll
    for (int h = 0; h < NREP; ++h) acc[j][h] = 0.f;
  IQ_GROUP_LOOP
  for (int g = 0; g < NG; ++g) {
#if IQ_FLASH_VSTREAM
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(KPG * (NG - 1)) : "memory");
#else
    if (g == 0) wait_vm_all();
#endif
    uint32_t cw[FBPW][W], cm[FBPW];
#pragma unroll
    for (int j = 0; j < FBPW; ++j) read_unit<W>(stage + (g * FBPW + j) * UB, lane, a.ksym, cw[j], cm[j]);
#if IQ_FLASH_VSTREAM
    wait_lgkm_all();
    stage_v(g * FBPW);
#endif
    if (a.ksym) {
#pragma unroll
      for (int j = 0; j < FBPW; ++j) to_offset_binary<BITS>(cw[j], W);
    }
    float d[FBPW][NREP];
    qk_group_dot<BITS, G, NREP, FBPW>(cw, &sm.qrec[g][0], hl, qsplit, pr, d);
#pragma unroll
    for (int j = 0; j < FBPW; ++j) {
      const float s = h2f(uint16_t(cm[j] & 0xffffu));
      const float z = a.ksym ? ZS * s : h2f(uint16_t(cm[j] >> 16));
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        const float qs = __uint_as_float(sm.qrec[g][qrec_osum<G, NREP>() + h]);
        acc[j][h] = fmaf(s, d[j][h], fmaf(z, qs, acc[j][h]));
      }
    }
  }
#if !IQ_FLASH_VSTREAM
  wait_lgkm_all();
  for (int g = 0; g < NG; ++g) stage_v(g * FBPW);
#endif
  const int vcnt = max(0, min(VPW, (a.T - wt0) / G));  // the wave's V groups inside the range

  // ---- softmax over the wave's tokens; fp16 p straight into the V records ----
  uint32_t (&vrec)[VPW][RD] = sm.vrec[wave];
  float mw[NREP], lw[NREP];
#pragma unroll
  for (int j = 0; j < FBPW; ++j) {
    const bool live = wt0 + j * TOKEN_BLOCK + lane < a.T;
#pragma unroll
    for (int h = 0; h < NREP; ++h) acc[j][h] = live ? acc[j][h] * a.scale : -INFINITY;
  }
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    mw[h] = acc[0][h];
#pragma unroll
    for (int j = 1; j < FBPW; ++j) mw[h] = fmaxf(mw[h], acc[j][h]);
  }
  wave_max_dpp(mw);
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    lw[h] = 0.f;
#pragma unroll
    for (int j = 0; j < FBPW; ++j) {
      const float p = acc[j][h] == -INFINITY ? 0.f : __expf(acc[j][h] - mw[h]);
      lw[h] += p;
      const int tl = j * TOKEN_BLOCK + lane;  // token within the wave
      int k = 0, hi = 0;
      plan_inv<BITS>(tl % G, k, hi);
      reinterpret_cast<uint16_t*>(&vrec[tl / G][h * NP + k])[hi] = __half_as_ushort(__float2half_rn(p));
    }
  }
  wave_sum_dpp(lw);
  wave_lds_sync();
  // per (V group, head): sum of the fp16 probabilities (zero-point term)
  if (lane < VPW * NREP) {
    const int u = lane / NREP, h = lane % NREP;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NP; k += 4) {
      const uint4 w4 = *reinterpret_cast<const uint4*>(&vrec[u][h * NP + k]);
      const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
      for (int y = 0; y < 4; ++y) s += h2f(uint16_t(ww[y] & 0xffffu)) + h2f(uint16_t(ww[y] >> 16));
    }
    vrec[u][NP * NREP + h] = __float_as_uint(s);
  }
  wave_lds_sync();

  // ---- attn.V over the wave's V groups, from the stage ----
  wait_vm_all();
  float o[NREP][DPL];
#pragma unroll
  for (int h = 0; h < NREP; ++h)
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[h][e] = 0.f;
  IQ_GROUP_LOOP
  for (int u = 0; u < VPW; ++u) {
    if (u >= vcnt) break;
    uint32_t cw[DPL][W], cm[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) read_unit<W>(stage + (u * DPL + e) * UB, lane, a.vsym, cw[e], cm[e]);
    if (a.vsym) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) to_offset_binary<BITS>(cw[e], W);
    }
    f4_t dv[DPL][(NREP + 3) / 4];
    group_mfma<BITS, G, NREP, DPL>(cw, &vrec[u][0], hl, pr, dv);
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const float s = h2f(uint16_t(cm[e] & 0xffffu));
      const float z = a.vsym ? ZS * s : h2f(uint16_t(cm[e] >> 16));
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        const float ps = __uint_as_float(vrec[u][NP * NREP + h]);
        o[h][e] = fmaf(s, dv[e][h / 4][h % 4], fmaf(z, ps, o[h][e]));
      }
    }
  }

  // ---- merge the four waves ----
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      sm.m[wave][h] = mw[h];
      sm.l[wave][h] = lw[h];
    }
  }
  lds_barrier();  // also: every wave is done with its stage (red aliases it)
  float mt[NREP];
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    mt[h] = fmaxf(fmaxf(sm.m[0][h], sm.m[1][h]), fmaxf(sm.m[2][h], sm.m[3][h]));
    const float sc = mw[h] == -INFINITY ? 0.f : __expf(mw[h] - mt[h]);
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[h][e] *= sc;
  }
  if (wave > 0) {
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < DPL; ++e) sm.red[wave - 1][h][lane + 64 * e] = o[h][e];
  }
  lds_barrier();
  const int64_t rows = int64_t(gridDim.y) * NREP;
  if (wave == 0) {
    float* dst = a.part + (int64_t(split) * rows + int64_t(bh) * NREP) * D;
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        float v = o[h][e];
#pragma unroll
        for (int r = 0; r < NWAVES - 1; ++r) v += sm.red[r][h][lane + 64 * e];
        dst[h * D + lane + 64 * e] = v;
      }
    if (lane < NREP) {  // split statistics of head `lane`
      const int h = lane;
      const float m = fmaxf(fmaxf(sm.m[0][h], sm.m[1][h]), fmaxf(sm.m[2][h], sm.m[3][h]));
      float l = 0.f;
#pragma unroll
      for (int w = 0; w < NWAVES; ++w) l += sm.m[w][h] == -INFINITY ? 0.f : sm.l[w][h] * __expf(sm.m[w][h] - m);
      float* ml = a.ml + (int64_t(split) * rows + int64_t(bh) * NREP + h) * 2;
      ml[0] = m;
      ml[1] = l;
    }
  }
}

}  // namespace

namespace iq::detail {

// q rows (and the norm row) are read as fp16 pairs: 4-byte aligned rows
bool flash_fused_supported(const void* q, int64_t sq_b, int64_t sq_h, const void* norm) {
  return aligned(q, 4) && sq_b % 2 == 0 && sq_h % 2 == 0 && (!norm || aligned(norm, 4));
}

int flash_fused_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const FusedStore& k,
                       const FusedStore& v, int B, int Hq, int Hkv, int T, int D, float scale, float* ml,
                       float* part, hipStream_t stream) {
  if (B == 0 || T == 0) return IQ_OK;
  if (k.bits != v.bits || k.group != v.group) return IQ_ERR_GROUP;
  if (T % k.group || FSPLIT != flash_split_tokens()) return IQ_ERR_GROUP;
  if (k.t0 % TOKEN_BLOCK || v.t0 % v.group) return IQ_ERR_ALIGN;
  if (!flash_fused_supported(q, sq_b, sq_h, norm)) return IQ_ERR_ALIGN;
  FusedArgs a{};
  a.q = (const uint16_t*)q; a.sqb = sq_b; a.sqh = sq_h; a.norm = (const uint16_t*)norm;
  a.kc = k.codes; a.km = k.meta; a.k_cap_blocks = k.t_cap / TOKEN_BLOCK; a.kblk0 = k.t0 / TOKEN_BLOCK;
  a.ksym = k.mode == IQ_MODE_SYM;
  a.vc = v.codes; a.vm = v.meta; a.v_cap_groups = v.t_cap / v.group; a.vg0 = v.t0 / v.group;
  a.vsym = v.mode == IQ_MODE_SYM;
  a.Hkv = Hkv; a.T = T; a.scale = scale; a.ml = ml; a.part = part;
  const int nsplit = int(ceil_div(T, FSPLIT));
  return dispatch_shape(k.bits, k.group, D, Hq / Hkv, 0, [&]<int BITS, int G, int DD, int R, bool S>() {
    flash_fused_kernel<BITS, G, DD, R><<<dim3(nsplit, B * Hkv), WG, 0, stream>>>(a);
    return launch_status();
  });
}

}  // namespace iq::detail
