// Fused flash-decoding kernel (gfx950): QK^T, softmax and attn.V over the
// packed range of every (batch, KV head), for K and V stores that share their
// group size (bit widths may differ: KB for K, VB for V).  Its output is one
// partial (m, l, unnormalized o) per run in the split slots of the decode
// workspace; the combine kernel (iq_decode.hip) merges the slots.
//
// This header holds the kernel template and its launch for one K bit width;
// iq_flash_k{2,3,4}.hip instantiate it (one translation unit per K width, so
// the instantiations compile in parallel) and iq_flash.hip holds the entry.
//
// Persistent and software pipelined.  One workgroup per CU (waves per SIMD:
// fused_waves_per_simd) takes an equal contiguous share of a list of
// FSPLIT-token splits (detail::ShareMap: the (batch, KV head)-major list, or
// for 4-bit K and V each head's splits cut 68:60 between the even and the
// odd XCDs, whose workgroups measured ~3 us slower), loaded with the
// non-temporal cache policy, and processes it as
// runs, the maximal pieces of one (batch, KV head).  Inside a run the waves
// claim wave blocks of WTOK tokens (lane = token for QK^T) from a counter in
// LDS, so they finish the run together, and each wave keeps a running
// softmax state (m, l, o) over its blocks.  A wave streams its packed data
// straight into VGPRs with raw buffer loads:
//   at the top of a block: K codes and {scale, zero} of its NEXT block (kept
//          in flight through the whole block);
//   after attn.V: V codes and {scale, zero} of the next block (lane = head_dim
//          column);
// and computes on data loaded one block earlier:
//   QK^T   per head_dim group eight v_mfma_f32_4x4x4f16 per 32 codes and four
//          query heads (iq_gemv.h): B = biased code pairs, A = the run's query
//          records in LDS, accumulators seeded with -sum(q * bias);
//   softmax  against the wave's running max (log2 domain, DPP reductions);
//          each lane writes its fp16 p straight into its slot of the wave's
//          attn.V operand record (the inverse of the unpack plan); the
//          per-V-group sums of p (zero-point term, l) and of -p * bias (seed
//          of attn.V) by DPP;
//   attn.V lane = column d = lane + 64 e over the block's V groups.
// At the end of a run the waves merge (rescale by exp2(m_w - m), sum in LDS)
// and write the run's partial into split slot k for the k-th run of its
// (batch, KV head); the slots past the last run's get empty statistics.  Each
// run starts by building its query records from q loaded at that point (a key
// normalization, which the reference applies to the dequantized keys,
// cache.py:128-133 and 249, is folded into q as hi/lo fp16 parts of q*n).
//
// The store formats follow the unfused kernels: K codes [B,H,t_cap/64,D/G,64,W],
// V codes [B,H,t_cap/G,D,W]; sym or asym per store is a runtime flag (a
// uniform branch), so the kernel is instantiated per (K bits, V bits, G, D,
// n_rep, hi/lo query rows) only.
#pragma once
#include <algorithm>
#include <type_traits>

#include "iq_gemv.h"

using namespace iq;

namespace {

constexpr int FSPLIT = NWAVES * IQ_FLASH_BPW * TOKEN_BLOCK;  // tokens per split (= flash_split_tokens())


// Pair k of a group's unpack plan: code index of its first and second half.
template <int BITS>
__host__ __device__ constexpr int plan_a(int k) { return pair_code_a<BITS>(k); }
template <int BITS>
__host__ __device__ constexpr int plan_c(int k) { return pair_code_c<BITS>(k); }

// Inverse of the plan: code i of a group sits in pair k, half hi (0: low),
// with bias 2^(10 - p) (p = the field's bit position in its half).
template <int BITS>
__host__ __device__ constexpr void plan_inv(int i, int& k, int& hi, float& bias) {
  using P = Plan<BITS>;
  const int sb = i / P::CODES, r = i % P::CODES;
  k = 0;
  hi = 0;
  bias = 0.f;
  for (int x = 0; x < P::NPAIR; ++x) {
    if (P::A[x] == r) { k = sb * P::NPAIR + x; hi = 0; bias = bias_a<BITS>(x); }
    if (P::C[x] == r) { k = sb * P::NPAIR + x; hi = 1; bias = bias_c<BITS>(x); }
  }
}
template <int BITS>
constexpr bool plan_inv_ok() {
  for (int i = 0; i < 128; ++i) {
    int k = 0, hi = 0;
    float b = 0.f;
    plan_inv<BITS>(i, k, hi, b);
    if ((hi ? plan_c<BITS>(k) : plan_a<BITS>(k)) != i) return false;
  }
  return true;
}
static_assert(plan_inv_ok<2>() && plan_inv_ok<3>() && plan_inv_ok<4>(), "plan inverse");

using detail::FusedArgs;

// waves per SIMD: one for G-token waves (G > 64); for 64-token waves two,
// and four in attn.V-only mode (AVO).  Three fit the registers of up to 4
// query heads per KV head, but measured slower for the decode step (~1.5 us
// at the headline): each wave keeps one block's loads in flight (10 KB at
// 4-bit), and the memory system streams the cache faster with fewer requests
// in flight per CU (the same trend as load-only probes).  An attn.V-only
// block is 3 KB (2-bit, G = 64) and its waves need <= 104 VGPRs: four per
// SIMD measured ~0.6 us faster than three, three ~1 us faster than two.
template <int G, int NREP, bool QS, bool AVO = false>
constexpr int fused_waves_per_simd() {
  return G > TOKEN_BLOCK ? 1 : AVO && NREP <= 4 && !QS ? 4 : 2;
}

// Workgroup shape: one workgroup per CU, filling every SIMD to the register
// allocation's occupancy; a wave processes blocks of WTOK consecutive tokens
// (lane = token for QK^T), so that a V group of G tokens lies inside a block.
template <int G, int NREP, bool QS, bool AVO = false>
struct FusedShape {
  static constexpr int WTOK = G > TOKEN_BLOCK ? G : TOKEN_BLOCK;
  static constexpr int FBPW = WTOK / TOKEN_BLOCK;                // 64-token K blocks per wave block
  static constexpr int NW = 4 * fused_waves_per_simd<G, NREP, QS, AVO>();  // waves per workgroup
  static constexpr int NT = NW * 64;
  static constexpr int VPW = WTOK / G;                           // V groups per wave block
  static_assert(FSPLIT % WTOK == 0, "a split holds whole wave blocks");
};

template <int G, int D, int NREP, bool QS, bool AVO>
struct FusedSmem {
  using FS = FusedShape<G, NREP, QS, AVO>;
  alignas(16) uint32_t qrec[D / G][qrec_dwords<G, NREP>()];         // query records of the current split
  alignas(16) uint32_t vrec[FS::NW][FS::VPW][rec_dwords<G, NREP>()];  // per wave: fp16 p pairs
  alignas(16) float red[FS::NW][NREP][D];                            // merge of the waves' outputs
  float m[FS::NW][NREP];
  float l[FS::NW][NREP];
  int next_block;  // the current run's next unclaimed wave block
};

// ---- raw buffer loads -------------------------------------------------------
// A block reads its (batch, KV head) slice of a store through a buffer
// resource: a byte offset per lane (VGPR) plus a uniform offset (SGPR).  A
// resource with zero records turns every load into a zero fill that moves no
// data; the prefetch past a wave's last block uses that, so every iteration
// issues the same loads and the compiler's memory counter waits stay exact.
//
// The cache's codes and metadata (and attn.V's probabilities) are read once:
// their loads carry the non-temporal cache policy (`nt`), which measured -5 us
// per headline step (67.8 -> 62.8 us, A/B over five rounds; sc0 / sc1 on top
// of it changed nothing).  The query, reused by every workgroup of a head,
// keeps the default policy.
constexpr int STREAM = 2;  // cache policy bits of a streaming load: nt
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}
template <int N, int POLICY = STREAM>
__device__ __forceinline__ void bload_words(rsrc_t r, uint32_t voff, uint32_t soff, uint32_t (&w)[N]) {
#pragma unroll
  for (int c = 0; c < N / 4; ++c) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16 * c, soff, POLICY);
    w[4 * c] = v[0]; w[4 * c + 1] = v[1]; w[4 * c + 2] = v[2]; w[4 * c + 3] = v[3];
  }
  constexpr int R = N % 4, C0 = N - N % 4;
  if constexpr (R == 3) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, voff + 4 * C0, soff, POLICY);
    w[C0] = v[0]; w[C0 + 1] = v[1]; w[C0 + 2] = v[2];
  } else if constexpr (R == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 4 * C0, soff, POLICY);
    w[C0] = v[0]; w[C0 + 1] = v[1];
  } else if constexpr (R == 1) {
    w[C0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff + 4 * C0, soff, POLICY);
  }
}
__device__ __forceinline__ uint32_t bload_u32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, STREAM);
}
template <int POLICY = 0>
__device__ __forceinline__ uint16_t bload_u16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, POLICY);
}

// {scale, zero} of a lane's token (K) or column (V) from its meta dword: asym
// meta is one {scale, zero} dword per lane; sym meta is one fp16 scale per
// lane, read as the dword holding the scales of lanes 2i and 2i + 1.  sh is
// the lane's shift to its scale: 0 for asym, 16 * (lane & 1) for sym (fixed
// per store), so both modes take one shift, two conversions, one multiply and
// one select.
__device__ __forceinline__ uint32_t meta_voff(int lane, int sym) { return sym ? uint32_t(lane & ~1) * 2 : uint32_t(lane) * 4; }
__device__ __forceinline__ uint32_t meta_shift(int lane, int sym) { return sym ? uint32_t(lane & 1) * 16 : 0u; }
// (BF: the meta halves hold bf16 values, a bf16 layer's store)
template <int BITS, bool BF = false>
__device__ __forceinline__ void meta_sz(uint32_t mw, uint32_t sh, int sym, float& s, float& z) {
  s = act2f(uint16_t(mw >> sh), BF);
  const float zh = act2f(uint16_t(mw >> 16), BF);
  z = sym ? -float(1 << (BITS - 1)) * s : zh;  // offset-binary sym codes: signed = u - 2^(b-1)
}

// {scale, zero} of a hybrid V group-column from its meta dword: the flag bit
// (bit 15, tested as a bit) marks b-bit sym codes (offset binary, zero
// -2^(b-1) |scale|), else (b-1)-bit asym codes with the stored zero.
template <int BITS, bool BF = false>
__device__ __forceinline__ void meta_sz_hyb(uint32_t mw, float& s, float& z) {
  s = hyb_scale(mw, BF);
  const float zh = act2f(uint16_t(mw >> 16), BF);
  z = hyb_sym(mw) ? -float(1 << (BITS - 1)) * s : zh;
}

// {scale, zero} of a K token-group whose store form is known only at run
// time (asym, sym or hybrid): the group is read as sym where its scale's
// float class is in `cls` (meta_sym_classes: every class for a sym store,
// none for asym, the negative ones for hybrid, whose flag is the scale's sign
// bit, -0.0 included) and the scale is taken as |scale| (asym and sym scales
// are never negative).  One compare more than meta_sz, no branch.
template <int BITS, bool BF = false>
__device__ __forceinline__ void meta_sz_rt(uint32_t mw, uint32_t sh, uint32_t cls, float& s, float& z) {
  const float sr = act2f(uint16_t(mw >> sh), BF);
  s = fabsf(sr);
  const float zh = act2f(uint16_t(mw >> 16), BF);
  z = __builtin_amdgcn_classf(sr, int(cls)) ? -float(1 << (BITS - 1)) * s : zh;
}
// float classes of v_cmp_class: bit 0 signaling NaN, 1 quiet NaN, 2 -inf,
// 3 -normal, 4 -denormal, 5 -0, 6 +0, 7 +denormal, 8 +normal, 9 +inf
__host__ __device__ constexpr uint32_t meta_sym_classes(int sym, int hyb) {
  return hyb ? 0x3Cu : sym ? 0x3FFu : 0u;
}

// Workgroup barrier for data exchanged through LDS.  __syncthreads() would
// also wait for every outstanding global load, i.e. for the next split's
// prefetch; only the LDS writes need to be complete.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// sum over aligned segments of N lanes (every lane gets its segment's sum)
template <int N>
__device__ __forceinline__ float seg_sum(float v) {
#pragma unroll
  for (int o = 1; o < N; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// AVO (attn.V only, the standalone GEMV of iq_av.hip): no K, no softmax; the
// fp16 probabilities p [B, Hq, T] come in through the q fields of the
// arguments (q, sqb, sqh, q_bytes), are loaded one block ahead in place of K
// and written into the attn.V operand records as they are; the runs' partials
// are plain sums (no statistics are written).
// QKO (QK^T only, the standalone logits GEMV of iq_qk.hip): no V, no
// softmax; each block's scaled logits (scale_log2 holds the plain scale) go to
// the fp32 output at part (element strides sob, soh per batch and query head,
// 1 per token).
// VH: the V store is hybrid (per-group flag in its meta, meta_sz_hyb).  A
// hybrid K store (a.khyb: meta laid out as asym, the flag per group) is read
// by the SM = 0 instances.
// BF: a bf16 layer (query, key normalization factor, scales and zero points
// in bf16): the query (times the factor, exact in fp32) goes into the hi/lo
// fp16 query rows (QS) and the metadata decodes as bf16; the probabilities
// meet V as fp16, finer than the reference's bf16 cast of the softmax.
// SM: the stores' modes known at compile time (1: K and V asym, 2: both sym;
// 0: the arguments' ksym / vsym).  A known mode drops the meta word's shift
// and the zero point's select from every group's decode: -0.3 us per
// headline launch and -0.7 to -1.3 us per 3-bit sym launch (same-box A/B).
template <int KB, int VB, int G, int D, int NREP, bool QS, bool AVO = false, bool QKO = false, bool VH = false,
          bool BF = false, int SM = 0>
__global__ __launch_bounds__((FusedShape<G, NREP, QS, AVO>::NT), (fused_waves_per_simd<G, NREP, QS, AVO>())) void flash_fused_kernel(FusedArgs a) {
  using FS = FusedShape<G, NREP, QS, AVO>;
  constexpr int NW = FS::NW, NT = FS::NT, WTOK = FS::WTOK, FBPW = FS::FBPW, VPW = FS::VPW;
  constexpr int BPS = FSPLIT / WTOK;  // wave blocks per split
  constexpr int NG = D / G;
  constexpr int KW = G * KB / 32, VW = G * VB / 32;  // code words per unit of K, V
  constexpr int NP = G / 2;
  constexpr int DPL = D / 64;
  constexpr int NPAIRS = NG * NREP * NP;  // query pairs of a split's records
  constexpr int NPT = (NPAIRS + NT - 1) / NT;
  constexpr int QOS = qrec_osum<G, NREP>();
  constexpr int QNB = qrec_nbsum<G, NREP>();
  constexpr int NQ = (NREP + 3) / 4;
  __shared__ FusedSmem<G, D, NREP, QS, AVO> sm;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hl = lane & 3;
  constexpr bool qsplit = QS;  // key normalization: hi/lo query rows
  const int ksym = SM == 0 ? a.ksym : int(SM == 2), vsym = SM == 0 ? a.vsym : int(SM == 2);
  const int kms = ksym ? 2 : 4, vms = vsym ? 2 : 4;  // meta bytes per token / column
  const uint32_t kmv = meta_voff(lane, ksym), vmv = meta_voff(lane, vsym);
  const uint32_t ksh = meta_shift(lane, ksym), vsh = meta_shift(lane, vsym);
  const uint32_t kcls = meta_sym_classes(ksym, a.khyb);  // SM == 0: the K groups read as sym
  const int64_t rows = int64_t(a.nitems / a.nsplit) * NREP;

  struct KRegs { uint32_t w[NG][FBPW][KW]; uint32_t m[NG][FBPW]; };
  struct VRegs { uint32_t w[VPW][DPL][VW]; uint32_t m[VPW][DPL]; };
  struct QRegs { uint16_t a[NPT], c[NPT], na[NPT], nc[NPT]; };
  struct PRegs { uint32_t p[FBPW][NREP]; };  // attn.V only: a block's fp16 probabilities
  using XRegs = std::conditional_t<AVO, PRegs, KRegs>;  // what is loaded one block ahead

  // ---- loads of wave block blk (tokens [blk*WTOK, +WTOK) of the range) of
  // (batch, KV head) bh into registers; real = false: zero fill ----
  auto load_k = [&](int bh, int blk, bool real, KRegs& k) {
    const int64_t blk0 = int64_t(bh) * a.k_cap_blocks + a.kblk0;
    const rsrc_t rc = make_rsrc(a.kc + blk0 * (NG * TOKEN_BLOCK * KW), real ? a.k_code_bytes : 0u);
    const rsrc_t rm = make_rsrc(a.km + blk0 * (NG * TOKEN_BLOCK * (kms / 2)), real ? a.k_meta_bytes : 0u);
    const int b0 = blk * FBPW;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int j = 0; j < FBPW; ++j) {
        const uint32_t u = uint32_t((b0 + j) * NG + g) * TOKEN_BLOCK;  // first token slot of the unit
        bload_words<KW>(rc, uint32_t(lane) * (KW * 4), u * (KW * 4), k.w[g][j]);
        k.m[g][j] = bload_u32(rm, kmv, u * kms);
      }
  };
  auto load_v = [&](int bh, int blk, bool real, VRegs& v) {
    const int64_t g0 = int64_t(bh) * a.v_cap_groups + a.vg0;
    const rsrc_t rc = make_rsrc(a.vc + g0 * (D * VW), real ? a.v_code_bytes : 0u);
    const rsrc_t rm = make_rsrc(a.vm + g0 * (D * (vms / 2)), real ? a.v_meta_bytes : 0u);
    const int vgw = blk * WTOK / G;  // the block's first V group
#pragma unroll
    for (int u = 0; u < VPW; ++u)
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const uint32_t c0 = uint32_t((vgw + u) * D + 64 * e);  // first column slot of the unit
        bload_words<VW>(rc, uint32_t(lane) * (VW * 4), c0 * (VW * 4), v.w[u][e]);
        v.m[u][e] = bload_u32(rm, vmv, c0 * vms);
      }
  };
  // attn.V only: the probabilities of block blk, lane = token, one row per head
  auto load_p = [&](int bh, int blk, bool real, PRegs& pp) {
    const int b = bh / a.Hkv, kvh = bh - b * a.Hkv;
    const rsrc_t rp = make_rsrc(a.q + b * a.sqb + int64_t(kvh * NREP) * a.sqh, real ? a.q_bytes : 0u);
#pragma unroll
    for (int j = 0; j < FBPW; ++j)
#pragma unroll
      for (int h = 0; h < NREP; ++h)
        pp.p[j][h] = bload_u16<STREAM>(rp, uint32_t(h * a.sqh + blk * WTOK + j * TOKEN_BLOCK + lane) * 2, 0);
  };
  auto load_x = [&](int bh, int blk, bool real, XRegs& x) {
    if constexpr (AVO) load_p(bh, blk, real, x);
    else load_k(bh, blk, real, x);
  };
  auto load_q = [&](int bh, bool real, QRegs& qq) {
    const int b = bh / a.Hkv, kvh = bh - b * a.Hkv;
    const rsrc_t rq = make_rsrc(a.q + b * a.sqb + int64_t(kvh * NREP) * a.sqh, real ? a.q_bytes : 0u);
    const rsrc_t rn = make_rsrc(a.norm ? a.norm + int64_t(bh) * D : a.q, real ? a.norm_bytes : 0u);
#pragma unroll
    for (int r = 0; r < NPT; ++r) {
      const int i = min(tid + r * NT, NPAIRS - 1);
      const int k = i % NP, h = (i / NP) % NREP, g = i / (NP * NREP);
      const int ia = g * G + plan_a<KB>(k), ic = g * G + plan_c<KB>(k);
      qq.a[r] = bload_u16(rq, uint32_t(h * a.sqh + ia) * 2, 0);
      qq.c[r] = bload_u16(rq, uint32_t(h * a.sqh + ic) * 2, 0);
      qq.na[r] = bload_u16(rn, uint32_t(ia) * 2, 0);
      qq.nc[r] = bload_u16(rn, uint32_t(ic) * 2, 0);
    }
  };
  // query records of a split from its loaded q (and norm) values; osum by
  // shuffles inside the NP lanes of each (group, head)
  auto build_records = [&](const QRegs& qq) {
#pragma unroll
    for (int r = 0; r < NPT; ++r) {
      const int i0 = tid + r * NT;
      const int i = min(i0, NPAIRS - 1);
      const int k = i % NP, h = (i / NP) % NREP, g = i / (NP * NREP);
      uint32_t hi = 0, lo = 0;
      float s = 0.f;
      if constexpr (BF) qrec_pair_vals_bf(qq.a[r], qq.c[r], qq.na[r], qq.nc[r], a.norm != nullptr, &hi, &lo, s);
      else qrec_pair_vals(qq.a[r], qq.c[r], qq.na[r], qq.nc[r], qsplit, &hi, &lo, s);
      // -sum(x * bias) of the hi and lo rows (exact products: the biases are powers of two)
      const float ba = bias_a<KB>(k % Plan<KB>::NPAIR), bc = bias_c<KB>(k % Plan<KB>::NPAIR);
      float bh = -(h2f(uint16_t(hi & 0xffffu)) * ba + h2f(uint16_t(hi >> 16)) * bc);
      float bl = -(h2f(uint16_t(lo & 0xffffu)) * ba + h2f(uint16_t(lo >> 16)) * bc);
      s = seg_sum<NP>(s);
      bh = seg_sum<NP>(bh);
      bl = seg_sum<NP>(bl);
      if (i0 < NPAIRS) {
        sm.qrec[g][h * NP + k] = hi;
        if (qsplit) sm.qrec[g][(NREP + h) * NP + k] = lo;
        if (k == 0) {
          sm.qrec[g][QOS + h] = __float_as_uint(s);
          sm.qrec[g][QNB + h] = __float_as_uint(bh);
          sm.qrec[g][QNB + NREP + h] = __float_as_uint(bl);
        }
      }
    }
  };

  const PlanRegs<KB> prk;
  const PlanRegs<VB> prv;
  const SumRegs<VB> srv(hl);
  // ---- work: this workgroup's share [i0, i1) of its side's list of splits
  // (detail::ShareMap: contiguous, equal shares, one workgroup per CU; each
  // XCD, or each XCD pair, streams a contiguous part of the cache), processed
  // as runs, the maximal pieces of one (batch, KV head).  Inside a run the
  // waves claim wave blocks from a counter in LDS (the first two per wave are
  // fixed), so they all finish the run within about one block of each other
  // whatever the issue arbitration favours. ----
  const detail::ShareMap smap = detail::ShareMap::make(int(gridDim.x), a.nitems / a.nsplit, a.nsplit, a.pair_e0);
  int side, sh;
  smap.share(int(blockIdx.x), side, sh);
  const int plen = smap.len(side), pfirst = smap.first(side);  // a head's splits on this side
  const int i0 = int(smap.begin(side, sh));
  const int i1 = int(smap.begin(side, sh + 1));
  if (i0 >= i1) return;  // uniform over the workgroup, before any barrier
  struct Run {
    int bh, split0, nsplit, nb;  // (batch, KV head), first split, splits, wave blocks
  };
  auto run_at = [&](int s0) {  // the run at list position s0
    Run r;
    r.bh = s0 / plen;
    r.split0 = pfirst + (s0 - r.bh * plen);
    r.nsplit = min(i1, (r.bh + 1) * plen) - s0;
    r.nb = r.nsplit * BPS;
    return r;
  };
  // wave block (within the (batch, KV head)) of run-relative index idx
  auto block_of = [&](const Run& r, int idx) { return r.split0 * BPS + idx; };
  // A (batch, KV head)'s runs come from consecutive shares of each side, one
  // run per share: they write their partials into split slots [0, nr) in
  // share order, side 0 first, so the combine finds them without a search;
  // the slots [nr, nsplit) carry empty statistics, each written by the run
  // whose splits hold it.
  // paired: one slot for every run of the share and a fixed run count
  // (computed here, so that only two values stay live through the loop)
  const int fslot = smap.paired ? smap.paired_slot(side, sh) : -1, fnr = 2 * smap.kk;
  auto run_slots = [&](const Run& r, int& slot, int& nr) {
    if (fslot >= 0) {
      slot = fslot;
      nr = fnr;
      return;
    }
    // plain: the shares holding the head's first and last split
    auto share_of = [&](int s) { return int(((int64_t(s) + 1) * gridDim.x + a.nitems - 1) / a.nitems) - 1; };
    const int c0 = share_of(r.bh * a.nsplit);
    slot = sh - c0;
    nr = share_of((r.bh + 1) * a.nsplit - 1) - c0 + 1;
  };

  // running softmax state of the wave over the current run (log2 domain)
  // Lazy running max: the reference max only has to bound a block's logits,
  // so it is raised (a wave reduction and a rescale) only when one exceeds it
  // by more than LAZY_MAX (log2 units): p <= 2^LAZY_MAX, well inside fp16, and
  // softmax does not depend on the reference.  m_thr = m_run + LAZY_MAX.
  constexpr float LAZY_MAX = 8.f;
  float m_run[NREP], m_thr[NREP], l_run[NREP], o_run[NREP][DPL];
  auto reset_run = [&]() {
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      m_run[h] = -INFINITY;
      m_thr[h] = -INFINITY;
      l_run[h] = 0.f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) o_run[h][e] = 0.f;
    }
  };
  // merge the waves' run states and write the run's partial into split slot
  // `slot` (every wave is past its last QK^T of the run afterwards)
  auto flush_run = [&](int bh, int slot) {
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        sm.m[wave][h] = m_run[h];
        sm.l[wave][h] = l_run[h];
      }
    }
    lds_barrier();
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      float mt = sm.m[0][h];
#pragma unroll
      for (int w = 1; w < NW; ++w) mt = fmaxf(mt, sm.m[w][h]);
      const float sc = AVO ? 1.f : m_run[h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[h] - mt);
#pragma unroll
      for (int e = 0; e < DPL; ++e) sm.red[wave][h][lane + 64 * e] = o_run[h][e] * sc;
    }
    float mls = 0.f, lls = 0.f;  // run statistics of head tid (m in natural-log units)
    if (tid < NREP) {
      const int h = tid;
      float mt = sm.m[0][h];
#pragma unroll
      for (int w = 1; w < NW; ++w) mt = fmaxf(mt, sm.m[w][h]);
#pragma unroll
      for (int w = 0; w < NW; ++w) lls += sm.m[w][h] == -INFINITY ? 0.f : sm.l[w][h] * __builtin_amdgcn_exp2f(sm.m[w][h] - mt);
      mls = mt * 0.69314718055994531f;
    }
    // every read of the statistics is done: a wave that runs ahead into its
    // next run may overwrite them after this barrier
    lds_barrier();
    float* dst = a.part + (int64_t(slot) * rows + int64_t(bh) * NREP) * D;
#pragma unroll
    for (int r = tid; r < NREP * D; r += NT) {
      const int h = r / D, dd = r % D;
      float val = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) val += sm.red[w][h][dd];
      dst[r] = val;
    }
    if (!AVO && tid < NREP) {
      float* ml = a.ml + (int64_t(slot) * rows + int64_t(bh) * NREP + tid) * 2;
      ml[0] = mls;
      ml[1] = lls;
    }
  };

  // the lane's tokens' slots in the attn.V operand records
  int tk[FBPW], thi[FBPW];
#pragma unroll
  for (int j = 0; j < FBPW; ++j) {
    float tb;
    plan_inv<VB>((j * TOKEN_BLOCK + lane) % G, tk[j], thi[j], tb);
  }

  Run run = run_at(i0);
  int rs2 = i0 + run.nsplit;                // first split of the next run (i1: none)
  Run run2 = run_at(min(rs2, i1 - 1));
  int cur = wave < run.nb ? wave : -1;           // the wave's current block (index in the run)
  int nxt = NW + wave < run.nb ? NW + wave : -1;  // the block whose data it loads next
  QRegs qq;
  VRegs v;
  // ---- one wave block: K in kc and V in v (loaded during the previous
  // block); loads the next block's K into kn at the top and its V into v
  // after attn.V; the wave's last block of a run ends in the run merge ----
  auto step = [&](XRegs& kc, XRegs& kn) -> bool {
    const bool have = cur >= 0;
    const bool ends = nxt < 0;  // the wave's last block of the run
    const bool nrun = rs2 < i1;
    // the block loaded during this one: nxt, or the wave's first block of the next run
    const int lbh = ends ? run2.bh : run.bh;
    const int lblk = ends ? block_of(run2, wave) : block_of(run, max(nxt, 0));
    const bool lreal = ends ? nrun && wave < run2.nb : true;
    load_x(lbh, lblk, lreal, kn);  // in flight through this whole block
    int nn = 0;
    if (!ends && lane == 0) nn = atomicAdd(&sm.next_block, 1);
    if (have) {
      const int wt0 = block_of(run, cur) * WTOK;  // first token of the block
      // ---- QK^T over the wave's tokens, from registers ----
      float acc[FBPW][NREP];
#pragma unroll
      for (int j = 0; j < FBPW; ++j)
#pragma unroll
        for (int h = 0; h < NREP; ++h) acc[j][h] = 0.f;
      if constexpr (!AVO) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          float d[FBPW][NREP];
          qk_group_dot_biased<KB, G, NREP, FBPW>(kc.w[g], &sm.qrec[g][0], hl, qsplit, prk, d);
#pragma unroll
          for (int j = 0; j < FBPW; ++j) {
            float s, z;
            if constexpr (SM == 0) meta_sz_rt<KB, BF>(kc.m[g][j], ksh, kcls, s, z);
            else meta_sz<KB, BF>(kc.m[g][j], ksh, ksym, s, z);
#pragma unroll
            for (int h = 0; h < NREP; ++h) {
              const float qs = __uint_as_float(sm.qrec[g][QOS + h]);
              acc[j][h] = fmaf(s, d[j][h], fmaf(z, qs, acc[j][h]));
            }
          }
        }
      }

      if constexpr (QKO) {
        // ---- the block's logits, lane = token ----
        const int b = run.bh / a.Hkv, kvh = run.bh - b * a.Hkv;
        float* o = a.part + b * a.sob + int64_t(kvh * NREP) * a.soh;
#pragma unroll
        for (int j = 0; j < FBPW; ++j) {
          const int t = wt0 + j * TOKEN_BLOCK + lane;
          if (t < a.T) {
#pragma unroll
            for (int h = 0; h < NREP; ++h) o[h * a.soh + t] = acc[j][h] * a.scale_log2;
          }
        }
      } else {
      // ---- softmax against the running max (log2 domain); fp16 p straight
      // into the V records ----
      auto& vrec = sm.vrec[wave];
      float mw[NREP], alpha[NREP];
      bool rescale = false;  // the running max moved: the run state is rescaled by alpha
      if constexpr (!AVO) {
        // Each comparison with the lazy threshold is its own ballot (a lane
        // mask ORed by the scalar unit): one compare per logit.
#pragma unroll
        for (int j = 0; j < FBPW; ++j)
#pragma unroll
          for (int h = 0; h < NREP; ++h) acc[j][h] *= a.scale_log2;
        if (wt0 + WTOK > a.T) {  // only a run's last block reaches past the range
          asm volatile("");      // a real branch: the masking costs nothing in full blocks
#pragma unroll
          for (int j = 0; j < FBPW; ++j) {
            const bool live = wt0 + j * TOKEN_BLOCK + lane < a.T;
#pragma unroll
            for (int h = 0; h < NREP; ++h) acc[j][h] = live ? acc[j][h] : -INFINITY;
          }
        }
        unsigned long long need = 0;
#pragma unroll
        for (int j = 0; j < FBPW; ++j)
#pragma unroll
          for (int h = 0; h < NREP; ++h) need |= __builtin_amdgcn_ballot_w64(acc[j][h] > m_thr[h]);
        rescale = need != 0;
        if (rescale) {
          asm volatile("");  // a real branch: keeps the compiler from flattening it into selects
#pragma unroll
          for (int h = 0; h < NREP; ++h) {
            mw[h] = acc[0][h];
#pragma unroll
            for (int j = 1; j < FBPW; ++j) mw[h] = fmaxf(mw[h], acc[j][h]);
          }
          wave_max_dpp(mw);
#pragma unroll
          for (int h = 0; h < NREP; ++h) {
            const float mn = fmaxf(m_run[h], mw[h]);
            alpha[h] = m_run[h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[h] - mn);
            m_run[h] = mn;
            m_thr[h] = mn + LAZY_MAX;
          }
        }
      }
      // p into the wave's attn.V operand records, as the fp16 the matrix
      // cores see (the zero-point term and l are sums of the same values)
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
#pragma unroll
        for (int j = 0; j < FBPW; ++j) {
          uint16_t p16;
          if constexpr (AVO) {
            p16 = uint16_t(kc.p[j][h]);  // the given probability, as it is
          } else {
            // the running max is finite from the run's first block on (a block
            // holds at least one token of the range), so a masked logit's
            // exp2(-inf) is 0 without a test
            const float p = __builtin_amdgcn_exp2f(acc[j][h] - m_run[h]);
            p16 = __half_as_ushort(__float2half_rn(p));
          }
          const int tl = j * TOKEN_BLOCK + lane;  // token within the wave
          reinterpret_cast<uint16_t*>(&vrec[tl / G][h * NP + tk[j]])[thi[j]] = p16;
        }
      }
      if constexpr (!AVO) {
        if (rescale) {
          asm volatile("");
#pragma unroll
          for (int h = 0; h < NREP; ++h) {
            l_run[h] *= alpha[h];
#pragma unroll
            for (int e = 0; e < DPL; ++e) o_run[h][e] *= alpha[h];
          }
        }
      }
      wave_lds_sync();

      // ---- attn.V over the wave's V groups, from registers; the same
      // matrix-core products sum p and p * bias per (group, head) ----
      const int vcnt = max(0, min(VPW, (a.T - wt0) / G));  // the wave's V groups inside the range
#pragma unroll
      for (int u = 0; u < VPW; ++u) {
        if (u < vcnt) {
          f4_t dv[DPL][NQ], dsum[NQ];
          group_mfma_biased_sums<VB, G, NREP, DPL>(v.w[u], &vrec[u][0], hl, prv, srv, dv, dsum);
          float ps[NREP], pbs[NREP];  // sum(p), sum(p * bias): lanes hl = 0, 1 of every 4-lane block
#pragma unroll
          for (int h = 0; h < NREP; ++h) {
            // (a float first: __builtin_bit_cast of a vector element reads element 0)
            const int d = __float_as_int(float(dsum[h / 4][h % 4]));
            // quad broadcasts; every source lane is valid, so no old value
            // (update_dpp with an old value cost a v_mov per broadcast)
            ps[h] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(d, 0x00, 0xf, 0xf, true));
            pbs[h] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(d, 0x55, 0xf, 0xf, true));
          }
          if constexpr (!AVO) {
#pragma unroll
            for (int h = 0; h < NREP; ++h) l_run[h] += ps[h];
          }
#pragma unroll
          for (int e = 0; e < DPL; ++e) {
            float s, z;
            if constexpr (VH) meta_sz_hyb<VB, BF>(v.m[u][e], s, z);
            else meta_sz<VB, BF>(v.m[u][e], vsh, vsym, s, z);
#pragma unroll
            for (int h = 0; h < NREP; ++h)  // codes = biased codes - bias
              o_run[h][e] = fmaf(s, dv[e][h / 4][h % 4] - pbs[h], fmaf(z, ps[h], o_run[h][e]));
          }
        }
      }
      }
    }
    if constexpr (!QKO) load_v(lbh, lblk, lreal, v);  // streams in during the next block's QK^T
    if (!ends) {
      nn = __builtin_amdgcn_readlane(nn, 0);
      cur = nxt;
      nxt = nn < run.nb ? nn : -1;
      return true;
    }
    // ---- run end: merge the waves; empty statistics in the slots past the
    // (batch, KV head)'s partials that lie among this run's splits (the
    // combine skips them) ----
    int slot, nr;
    run_slots(run, slot, nr);
    if constexpr (QKO) lds_barrier();  // every wave is past its last QK^T of the run
    else flush_run(run.bh, slot);
    if (!AVO && !QKO && a.empty_stats && wave == 0 && lane < NREP) {
      for (int sp = max(run.split0, nr); sp < run.split0 + run.nsplit; ++sp) {
        float* ml = a.ml + (int64_t(sp) * rows + int64_t(run.bh) * NREP + lane) * 2;
        ml[0] = -INFINITY;
        ml[1] = 0.f;
      }
    }
    if (!nrun) return false;
    reset_run();
    run = run2;
    rs2 += run.nsplit;
    run2 = run_at(min(rs2, i1 - 1));
    // the new (batch, KV head)'s query records.  The query is loaded here and
    // not prefetched during the previous run: registers with loads pending
    // across the block loop made the compiler wait for every outstanding load
    // at the loop's back edge
    if constexpr (!AVO) {
      load_q(run.bh, true, qq);
      build_records(qq);
    }
    if (tid == 0) sm.next_block = 2 * NW;
    lds_barrier();
    cur = wave < run.nb ? wave : -1;
    nxt = NW + wave < run.nb ? NW + wave : -1;
    return true;
  };

  XRegs ka, kb;
  reset_run();
  load_x(run.bh, block_of(run, max(cur, 0)), cur >= 0, ka);
  if constexpr (!QKO) load_v(run.bh, block_of(run, max(cur, 0)), cur >= 0, v);
  if constexpr (!AVO) {
    load_q(run.bh, true, qq);
    build_records(qq);
  }
  if (tid == 0) sm.next_block = 2 * NW;
  lds_barrier();
  while (step(ka, kb) && step(kb, ka)) {
  }
}

// Launch of the fused kernel for K bit width KB (the arguments filled by
// flash_fused_launch): persistent grid, one workgroup per CU.  VH: hybrid V;
// BF: a bf16 layer (hi/lo query rows whether or not keys are normalized).
// launch = false: only the grid is computed.
template <int KB, bool VH = false, bool BF = false>
int fused_launch_kb(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid_out,
                    hipStream_t stream, bool launch) {
  return dispatch_shape(vbits, group, D, nrep, 0, [&]<int VB, int G, int DD, int R, bool S>() {
    // store modes known at compile time for groups of 32 at head_dim 128 (fp16
    // layers, K and V both asym or both sym): instance sm, else 0
    int sm = 0;
    if constexpr (G == 32 && DD == 128 && !BF && !VH) sm = a.ksym == a.vsym && !a.khyb ? 1 + (a.ksym != 0) : 0;
    auto pick = [&]<int M>() {
      return BF     ? flash_fused_kernel<KB, VB, G, DD, R, true, false, false, VH, true>
             : norm ? flash_fused_kernel<KB, VB, G, DD, R, true, false, false, VH, false, M>
                    : flash_fused_kernel<KB, VB, G, DD, R, false, false, false, VH, false, M>;
    };
    auto* kern = pick.template operator()<0>();
    if constexpr (G == 32 && DD == 128 && !BF && !VH) {
      if (sm == 1) kern = pick.template operator()<1>();
      if (sm == 2) kern = pick.template operator()<2>();
    }
    const bool qs = BF || norm;
    const int nt = qs ? FusedShape<G, R, true>::NT : FusedShape<G, R, false>::NT;
    // as many workgroups as fit at once on the device (per instance)
    static detail::OccCache occ[6];
    const int pc = detail::blocks_per_cu(kern, nt, occ[(qs ? 1 : 0) + 2 * sm]);
    const int grid = int(std::min<int64_t>(a.nitems, int64_t(pc) * detail::num_cus()));
    if (grid_out) *grid_out = grid;
    if (!launch) return int(IQ_OK);
    kern<<<dim3(grid), nt, 0, stream>>>(a);
    return launch_status();
  });
}

}  // namespace
