// attn.V GEMV by column slices (gfx950): the main path of iq_av_gemv where
// its workgroups fill the device.  This header holds the kernel template and
// its launch for one V bit width; iq_av_cols_k{2,3,4}.hip instantiate it (one
// translation unit per bit width, compiled in parallel).
#pragma once

#include "iq_flash.h"

using namespace iq;

namespace {

// ---- attn.V by column slices ------------------------------------------------
// The main path of iq_av_gemv where the launch fills the device: a workgroup
// owns AVC_CW output columns of one (batch, KV head) over the whole token
// range, so it writes its columns of the output itself: no split-T partials
// and no second launch.  The four slices of a head read the same
// probabilities; they are dealt to one XCD (workgroup b runs on XCD b % 8),
// so the repeats are served by that XCD's L2.
//
// A wave step covers GPS V groups: lanes [LPG*i, LPG*i + LPG) take group i of
// the step, lane = column cl (plus LPG * j for its SPL column sets), and load
// that (group, column)'s codes and meta word (16 B + 4 B at 2-bit, G = 64).
// The step's probabilities come in as plan periods (CODES consecutive tokens
// of one head and group, one per lane): the lane forms the period's code-pair
// order with byte permutes and writes it into the wave's operand records in
// LDS, which the matrix-core products read as the fused kernel's attn.V does
// (B = biased code pairs, A = the record row of head 4q + lane % 4, and one
// more product per step for sum(p) and sum(p * bias), SumRegs).  The loads
// run a step ahead; every step issues the same loads (a group past the range
// reads zeros through the buffer bounds), so the memory-counter waits stay
// exact.  The probabilities keep the default cache policy (each is read by
// the four slices of its head: -2.5 us per config-2 call against
// non-temporal loads), the codes and metadata stream non-temporally.  At the
// end the waves' sums go through LDS in a fixed order.
constexpr int AVC_CW = 32;  // output columns per workgroup
constexpr int AVC_NW = 16;  // waves per workgroup (one workgroup per CU), at most
// column sets per lane: 2 (16 lanes per group, four groups per wave step);
// one set measured 1.3 us slower at config 2, four spill registers
#ifndef IQ_AVC_SPL
#define IQ_AVC_SPL 2
#endif
// cache policy of the probability loads: default (0), kept in L2 for the
// other slices of the head
#ifndef IQ_AVC_PPOL
#define IQ_AVC_PPOL 0
#endif

template <int VB, int G, int NREP, int SPL>
struct AvcShape {
  static constexpr int LPG = AVC_CW / SPL;                       // lanes per group
  static constexpr int GPS = 64 / LPG;                           // groups per wave step
  static constexpr int VW = G * VB / 32;                         // code words per (group, column)
  static constexpr int NP = G / 2;                               // code pairs per group
  static constexpr int CODES = Plan<VB>::CODES, NPAIR = Plan<VB>::NPAIR;
  static constexpr int PPG = G / CODES;                          // plan periods per group
  static constexpr int NU = GPS * NREP * PPG;                    // probability periods per step
  static constexpr int UPL = (NU + 63) / 64;                     // periods per lane
  static constexpr int UW = CODES / 2;                           // dwords of a period
  // Record layout in LDS: a head's row of NP pairs padded to RS dwords and a
  // group slot's rows to SS = 16 (mod 64) dwords, so that the 16 rows one
  // operand read touches (four group slots x four heads) start in 16
  // different 4-bank blocks of the 64 banks (unpadded, rows 128 B apart share
  // their banks: up to 8-way conflicts)
  static constexpr int RS = NP + 4;
  static constexpr int SS = NREP * RS + ((16 - (NREP * RS) % 64) + 64) % 64;
  static_assert(LPG % 4 == 0, "a matrix-core block's four lanes share their group");
  static_assert(UW % 4 == 0, "a period loads in 16-byte pieces");
};
// waves per workgroup: 16 (four per SIMD, 128 VGPRs each), or 8 where a
// wave's registers need more (8 query heads per KV head, 3- and 4-bit groups
// of 128)
template <int VB, int G, int NREP>
constexpr int avc_waves() { return NREP >= 8 || (G == 128 && VB >= 3) ? 8 : AVC_NW; }

// steps whose loads are in flight ahead of the one computed: one (two
// measured 0.7-1.2 us slower at config 2, three 1.3-2 us: more registers per
// wave, the same bytes in flight per CU)
template <int VB, int G, int NREP, int SPL>
constexpr int avc_prefetch() {
#ifdef IQ_AVC_PF
  return IQ_AVC_PF;
#else
  return 1;
#endif
}

struct AVCArgs {
  const uint16_t* p;  // probabilities [B][Hq][T], element strides spb, sph
  int64_t spb, sph;
  const uint32_t* vc;
  const uint16_t* vm;
  int64_t cap_groups;
  int g0, Hkv, ngroups, vsym, nslice, nitems;
  uint32_t p_bytes, v_code_bytes, v_meta_bytes;
  float* out32;
  uint16_t* out16;
  int64_t sob, soh;  // output strides (elements) per batch and query head
  int accumulate;
};

template <int VB, int G, int D, int NREP, int SPL, bool VH>
__global__ __launch_bounds__((avc_waves<VB, G, NREP>() * 64)) void av_cols_kernel(AVCArgs a) {
  using S = AvcShape<VB, G, NREP, SPL>;
  constexpr int NW = avc_waves<VB, G, NREP>(), NT = NW * 64;
  constexpr int LPG = S::LPG, GPS = S::GPS, VW = S::VW, NP = S::NP, PPG = S::PPG, UPL = S::UPL, UW = S::UW;
  constexpr int NQ = (NREP + 3) / 4;
  constexpr int PF = avc_prefetch<VB, G, NREP, SPL>();
  constexpr int RS = S::RS, SS = S::SS;
  constexpr int REC = GPS * SS;                    // dwords of a wave's records
  constexpr int RED = GPS * NREP * AVC_CW;         // floats of a wave's sums
  constexpr int WSM = REC > RED ? REC : RED;
  __shared__ uint32_t smem[NW][WSM];               // records, then (after the loop) the waves' sums

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hl = lane & 3;
  const int gs = lane / LPG, cl = lane % LPG;
  // workgroup -> (batch, KV head, slice): the slices of a head on one XCD
  int item = int(blockIdx.x);
  if (gridDim.x % 8 == 0) item = int(blockIdx.x % 8) * int(gridDim.x / 8) + int(blockIdx.x / 8);
  const int bh = item / a.nslice, slice = item - bh * a.nslice;
  const int b = bh / a.Hkv, kvh = bh - b * a.Hkv;
  const int col0 = slice * AVC_CW + cl;  // the lane's column of set 0 (set j: + LPG * j)

  const int ms = a.vsym ? 2 : 4;  // meta bytes per (group, column)
  const int64_t gbase = int64_t(bh) * a.cap_groups + a.g0;
  const rsrc_t rc = make_rsrc(a.vc + gbase * (D * VW), a.v_code_bytes);
  const rsrc_t rm = make_rsrc(a.vm + gbase * (D * (ms / 2)), a.v_meta_bytes);
  const rsrc_t rp = make_rsrc(a.p + b * a.spb + int64_t(kvh * NREP) * a.sph, a.p_bytes);
  uint32_t moff[SPL], msh[SPL];
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    const int c = col0 + LPG * j;
    moff[j] = a.vsym ? uint32_t(c & ~1) * 2 : uint32_t(c) * 4;
    msh[j] = a.vsym ? uint32_t(c & 1) * 16 : 0u;
  }

  struct Buf {
    uint32_t w[SPL][VW];
    uint32_t m[SPL];
    uint32_t pu[UPL][UW];
  };
  constexpr uint32_t OOB = 0x80000000u;  // an offset past every buffer: the load returns zeros
  auto load = [&](int step, Buf& bf) {
    const int g = step * GPS + gs;  // the lane's group (past the range: zeros)
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      const uint32_t unit = uint32_t(g) * D + uint32_t(col0 + LPG * j);
      bload_words<VW>(rc, unit * (VW * 4), 0, bf.w[j]);
      bf.m[j] = bload_u32(rm, uint32_t(g) * (D * ms) + moff[j], 0);
    }
#pragma unroll
    for (int u = 0; u < UPL; ++u) {
      const int id = lane + 64 * u;  // period (group slot, head, period of the group)
      const int slot = id / (NREP * PPG), hh = (id / PPG) % NREP, pp = id % PPG;
      const int gg = step * GPS + slot;
      const uint32_t off = id < S::NU && gg < a.ngroups
                               ? uint32_t((int64_t(hh) * a.sph + int64_t(gg) * G + pp * S::CODES) * 2)
                               : OOB;
      bload_words<UW, IQ_AVC_PPOL>(rp, off, 0, bf.pu[u]);
    }
  };
  // the periods' probabilities in code-pair order into the wave's records
  uint32_t* rec = &smem[wave][0];
  auto build = [&](const Buf& bf) {
#pragma unroll
    for (int u = 0; u < UPL; ++u) {
      const int id = lane + 64 * u;
      if (S::NU % 64 == 0 || id < S::NU) {
        const int slot = id / (NREP * PPG), hh = (id / PPG) % NREP, pp = id % PPG;
        uint32_t pr[S::NPAIR];
#pragma unroll
        for (int x = 0; x < S::NPAIR; ++x) {
          const int ca = Plan<VB>::A[x], cc = Plan<VB>::C[x];
          const uint32_t sel = uint32_t(2 * (ca & 1)) | (uint32_t(2 * (ca & 1) + 1) << 8) |
                               (uint32_t(4 + 2 * (cc & 1)) << 16) | (uint32_t(5 + 2 * (cc & 1)) << 24);
          pr[x] = __builtin_amdgcn_perm(bf.pu[u][cc >> 1], bf.pu[u][ca >> 1], sel);
        }
        uint32_t* dst = rec + slot * SS + hh * RS + pp * S::NPAIR;
#pragma unroll
        for (int x = 0; x < S::NPAIR; x += 4)
          *reinterpret_cast<uint4*>(dst + x) = make_uint4(pr[x], pr[x + 1], pr[x + 2], pr[x + 3]);
      }
    }
  };

  const PlanRegs<VB> prv;
  const SumRegs<VB> srv(hl);
  float o[NREP][SPL];
#pragma unroll
  for (int h = 0; h < NREP; ++h)
#pragma unroll
    for (int j = 0; j < SPL; ++j) o[h][j] = 0.f;
  auto compute = [&](const Buf& bf) {
    f4_t dv[SPL][NQ], dsum[NQ];
    group_mfma_biased_sums<VB, G, NREP, SPL, RS>(bf.w, rec + gs * SS, hl, prv, srv, dv, dsum);
    float ps[NREP], pbs[NREP];  // sum(p), sum(p * bias) of the lane's group: lanes hl = 0, 1 of each block
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      const int d = __float_as_int(float(dsum[h / 4][h % 4]));
      ps[h] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(d, 0x00, 0xf, 0xf, true));
      pbs[h] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(d, 0x55, 0xf, 0xf, true));
    }
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      float s, z;
      if constexpr (VH) meta_sz_hyb<VB>(bf.m[j], s, z);
      else meta_sz<VB>(bf.m[j], msh[j], a.vsym, s, z);
#pragma unroll
      for (int h = 0; h < NREP; ++h) o[h][j] = fmaf(s, dv[j][h / 4][h % 4] - pbs[h], fmaf(z, ps[h], o[h][j]));
    }
  };

  // the wave's steps: wave, wave + NW, ...
  const int nsteps = (a.ngroups + GPS - 1) / GPS;
  const int nst = (nsteps - wave + NW - 1) / NW;  // this wave's step count (may be 0)
  Buf bufs[PF + 1];
#pragma unroll
  for (int i = 0; i < PF; ++i) load(wave + NW * i, bufs[i]);
  for (int i0 = 0; i0 < nst; i0 += PF + 1) {
#pragma unroll
    for (int j = 0; j <= PF; ++j) {
      load(wave + NW * (i0 + j + PF), bufs[(j + PF) % (PF + 1)]);
      if (i0 + j < nst) {
        wave_lds_sync();  // the previous step's record reads are issued
        build(bufs[j]);
        wave_lds_sync();
        compute(bufs[j]);
      }
    }
  }

  // ---- the waves' sums, in a fixed order: wave, then group slot ----
  __syncthreads();  // every record read is done
  float* red = reinterpret_cast<float*>(&smem[wave][0]);
#pragma unroll
  for (int h = 0; h < NREP; ++h)
#pragma unroll
    for (int j = 0; j < SPL; ++j) red[(gs * NREP + h) * AVC_CW + cl + LPG * j] = o[h][j];
  __syncthreads();
  for (int r = tid; r < NREP * AVC_CW; r += NT) {
    const int h = r / AVC_CW, c = r % AVC_CW;
    float v = 0.f;
    for (int w = 0; w < NW; ++w) {
      const float* rw = reinterpret_cast<const float*>(&smem[w][0]);
#pragma unroll
      for (int s = 0; s < GPS; ++s) v += rw[(s * NREP + h) * AVC_CW + c];
    }
    const int64_t off = b * a.sob + int64_t(kvh * NREP + h) * a.soh + slice * AVC_CW + c;
    if (a.accumulate) v += a.out32[off];
    if (a.out32) a.out32[off] = v;
    if (a.out16) a.out16[off] = __half_as_ushort(__float2half_rn(v));
  }
}


// Launch for V bit width VB (a.nitems workgroups of AVC_NW waves).
template <int VB>
int av_cols_launch_vb(const AVCArgs& a, int group, int D, int nrep, bool hybrid, hipStream_t stream) {
  auto go = [&]<int G, int DD, int R>() -> int {
    auto* kern = hybrid ? av_cols_kernel<VB, G, DD, R, IQ_AVC_SPL, true> : av_cols_kernel<VB, G, DD, R, IQ_AVC_SPL, false>;
    kern<<<dim3(unsigned(a.nitems)), avc_waves<VB, G, R>() * 64, 0, stream>>>(a);
    return launch_status();
  };
  auto by_r = [&]<int G, int DD>() -> int {
    switch (nrep) {
      case 1: return go.template operator()<G, DD, 1>();
      case 2: return go.template operator()<G, DD, 2>();
      case 4: return go.template operator()<G, DD, 4>();
      case 8: return go.template operator()<G, DD, 8>();
      default: return IQ_ERR_SHAPE;
    }
  };
  auto by_d = [&]<int G>() -> int {
    if (D == 128) return by_r.template operator()<G, 128>();
    if constexpr (G <= 64) {
      if (D == 64) return by_r.template operator()<G, 64>();
    }
    return IQ_ERR_SHAPE;
  };
  switch (group) {
    case 32: return by_d.template operator()<32>();
    case 64: return by_d.template operator()<64>();
    case 128: return by_d.template operator()<128>();
    default: return IQ_ERR_GROUP;
  }
}

}  // namespace
