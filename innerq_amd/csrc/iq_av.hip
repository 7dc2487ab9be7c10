// Decode attn.V GEMV over a packed V store (gfx950).
//
// out[b, h, d] = sum_g ( s[g,d] * sum_{t in g} p[h,t] c[t,d] + z[g,d] * sum_{t in g} p[h,t] )
//
// Mapping: a workgroup of four waves owns a contiguous range of token groups
// of one (batch, KV head) (split-T); wave w takes every fourth group of the
// range, two groups per step with the next two prefetched.  Lane = head_dim
// column d = lane + 64 e (two columns at D=128), so each wave load covers 64
// consecutive (group, column) units.  The dot products run on the matrix
// cores: eight v_mfma_f32_4x4x4f16 per group and column set, B = four unpacked
// codes of the lane's column, A = four probabilities of head 4q + lane%4 from
// the probability operand record (iq_gemv.h); the VALU unpacks codes and
// applies scale and zero point.
// The four waves' partial sums are reduced in LDS in a fixed order, each
// workgroup writes one fp32 partial per split, and a second kernel sums the
// splits in split order: no atomics, deterministic results.
//
// iq_av_gemv takes this path only where the persistent kernel cannot run (a
// slice beyond 32-bit buffer offsets).  Its main path is the column-slice
// kernel (iq_av_cols.h: a workgroup per (batch, KV head, 32 output columns)
// over the whole token range, no partials, no combine) wherever that grid
// fills the device; else the fused decode kernel in attn.V-only mode
// (iq_flash.h): one workgroup per CU streams V and the probabilities of its
// share of the token range (read straight into the operand records, no record
// kernel), one partial per run, then the same combine over each (batch, KV
// head)'s run slots.
#include "iq_av_cols.h"

using namespace iq;

namespace {

// one thread per (b, kvh, g, h): probability pairs in plan order and their sum
template <int BITS, int G, int NREP>
__global__ __launch_bounds__(256) void av_record_kernel(const uint16_t* __restrict__ p, int64_t spb, int64_t sph,
                                                        int B, int Hkv, int ngroups, uint32_t* __restrict__ rec) {
  constexpr int NP = G / 2;
  constexpr int RD = rec_dwords<G, NREP>();
  constexpr PairTable<BITS, NP> PT{};
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(B) * Hkv * ngroups * NREP) return;
  const int h = int(i % NREP);
  const int64_t g = (i / NREP) % ngroups;
  const int64_t bh = i / (int64_t(NREP) * ngroups);
  const int b = int(bh / Hkv), kvh = int(bh % Hkv);
  const uint16_t* pr = p + b * spb + (kvh * NREP + h) * sph + g * G;
  uint32_t* r = rec + (bh * ngroups + g) * RD;
  float sum = 0.f;
  for (int k = 0; k < NP; ++k) {
    const uint16_t ua = pr[PT.a[k]], uc = pr[PT.c[k]];
    r[h * NP + k] = uint32_t(ua) | (uint32_t(uc) << 16);
    sum += h2f(ua) + h2f(uc);
  }
  r[NP * NREP + h] = __float_as_uint(sum);
}

struct AVArgs {
  const uint32_t* rec;   // records of the range's groups, [B*Hkv][ngroups]
  const uint32_t* vc;
  const uint16_t* vm;
  int64_t cap_groups;
  int Hkv, g0, ngroups, gpw;
  float* part;           // [nsplit][B*Hq][D]
  int hyb;               // hybrid store (per-group flag in the meta dword)
};

template <int BITS, int G, int D, int NREP, bool SYM>
__global__ __launch_bounds__(WG) void av_kernel(AVArgs a) {
  constexpr int W = G * BITS / 32;
  constexpr int NP = G / 2;
  constexpr int M = SYM ? 1 : 2;
  constexpr int DPL = D / 64;
  constexpr int RD = rec_dwords<G, NREP>();
  constexpr int NB = 2;  // groups per step
  __shared__ float red[NWAVES - 1][NREP][D];

  const int bh = blockIdx.y;
  const int split = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int gl0 = split * a.gpw;
  const int ng = min(a.gpw, a.ngroups - gl0);
  const int cnt = ng > wave ? (ng - wave + NWAVES - 1) / NWAVES : 0;
  const int64_t gbase = int64_t(bh) * a.cap_groups + a.g0 + gl0;
  const cptr_u32 recb = (cptr_u32)(a.rec) + (int64_t(bh) * a.ngroups + gl0) * RD;

  float acc[NREP][DPL];
#pragma unroll
  for (int h = 0; h < NREP; ++h)
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[h][e] = 0.f;

  uint32_t w[NB][DPL][W];
  uint32_t m[NB][DPL];
  // column d = lane + 64 e: every wave load is 64 consecutive (group, d) units
  auto load = [&](int i0) {
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (i0 + u < cnt) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          const int64_t unit = (gbase + wave + NWAVES * (i0 + u)) * D + lane + 64 * e;
          load_words<W>(a.vc + unit * W, w[u][e]);
          if constexpr (SYM) m[u][e] = a.vm[unit];
          else m[u][e] = reinterpret_cast<const uint32_t*>(a.vm)[unit];
        }
      }
    }
  };
  const PlanRegs<BITS> pr;
  if (cnt > 0) load(0);
  for (int i = 0; i < cnt; i += NB) {
    uint32_t cw[NB][DPL][W];
    uint32_t cm[NB][DPL];
#pragma unroll
    for (int u = 0; u < NB; ++u)
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        cm[u][e] = m[u][e];
#pragma unroll
        for (int x = 0; x < W; ++x) cw[u][e][x] = w[u][e][x];
      }
    if (i + NB < cnt) load(i + NB);  // prefetch the next step
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (i + u < cnt) {
        const cptr_u32 rec = recb + (wave + NWAVES * (i + u)) * RD;
        f4_t dv[DPL][(NREP + 3) / 4];
        group_mfma<BITS, G, NREP, DPL>(cw[u], a.rec + (int64_t(bh) * a.ngroups + gl0 + wave + NWAVES * (i + u)) * RD,
                                       lane & 3, pr, dv);
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          float s = h2f(uint16_t(cm[u][e] & 0xffffu));
          float z = SYM ? -float(1 << (BITS - 1)) * s : h2f(uint16_t(cm[u][e] >> 16));
          if (!SYM && a.hyb) meta_sz_hyb<BITS>(cm[u][e], s, z);
#pragma unroll
          for (int h = 0; h < NREP; ++h) {
            const float ps = rec_f32(rec, NP * NREP + h);
            acc[h][e] = fmaf(s, dv[e][h / 4][h % 4], fmaf(z, ps, acc[h][e]));
          }
        }
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < DPL; ++e) red[wave - 1][h][lane + 64 * e] = acc[h][e];
  }
  __syncthreads();
  if (wave == 0) {
    float* dst = a.part + (int64_t(split) * gridDim.y * NREP + int64_t(bh) * NREP) * D;
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        float v = acc[h][e];
#pragma unroll
        for (int r = 0; r < NWAVES - 1; ++r) v += red[r][h][lane + 64 * e];
        dst[h * D + lane + 64 * e] = v;
      }
  }
}

template <int AB>
__global__ __launch_bounds__(256) void av_combine_kernel(const float* __restrict__ part, int nsplit, int Hq, int D,
                                                         int64_t rows, detail::OutPair o, int accumulate, int grid,
                                                         int nrep) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * D) return;
  const int64_t bq = i / D;
  const int d = int(i % D);
  int n = nsplit;
  if (grid > 0)  // the runs of the (batch, KV head) in the persistent kernel's shares
    n = detail::ShareMap::make(grid, int(rows / nrep), nsplit, 0).nruns(int(bq / nrep));  // plain partition
  // the slots in order, their loads AB at a time (indices clamped so that a
  // round's loads are all in flight at once; the sum order is the slot order)
  float v = 0.f;
  for (int s0 = 0; s0 < n; s0 += AB) {
    float x[AB];
#pragma unroll
    for (int u = 0; u < AB; ++u) x[u] = part[(int64_t(min(s0 + u, n - 1)) * rows + bq) * D + d];
#pragma unroll
    for (int u = 0; u < AB; ++u)
      if (s0 + u < n) v += x[u];
  }
  const int64_t off32 = (bq / Hq) * o.s32b + (bq % Hq) * o.s32h + d;
  if (accumulate) v += o.out32[off32];
  if (o.out32) o.out32[off32] = v;
  if (o.out16) o.out16[(bq / Hq) * o.s16b + (bq % Hq) * o.s16h + d] = __half_as_ushort(__float2half_rn(v));
}

// groups per workgroup for a range of ngroups groups: about four workgroups
// per CU over the whole launch, at least two groups per wave
int groups_per_wg(int B, int Hkv, int ngroups) {
  const int64_t target = int64_t(detail::num_cus()) * 4;
  const int64_t bhs = std::max<int64_t>(1, int64_t(B) * Hkv);
  const int64_t splits = std::max<int64_t>(1, target / bhs);
  int gpw = int(ceil_div(ngroups, splits));
  gpw = std::max(gpw, std::min(ngroups, 2 * NWAVES));
  gpw = int(ceil_div(gpw, NWAVES) * NWAVES);
  return std::max(gpw, 1);
}

int check_av(const void* p, const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B, int Hq, int Hkv,
             int t0, int T, int D, int group, int bits, int mode) {
  IQ_CHECK(p && v_codes && v_meta, IQ_ERR_NULL);
  if (int e = check_v_common(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && T >= 0 && t0 >= 0 && Hkv > 0 && Hq > 0, IQ_ERR_SHAPE);
  IQ_CHECK(d_ok(D) && Hq % Hkv == 0 && nrep_ok(Hq / Hkv), IQ_ERR_SHAPE);
  IQ_CHECK(T % group == 0 && t0 % group == 0 && t_cap % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(int64_t(t0) + T <= t_cap, IQ_ERR_RANGE);
  IQ_CHECK(aligned(v_codes, 16) && aligned(v_meta, 8), IQ_ERR_ALIGN);
  return IQ_OK;
}

}  // namespace

namespace iq::detail {

int av_cols_launch_k2(const void* args, int group, int D, int nrep, bool hybrid, hipStream_t stream);
int av_cols_launch_k3(const void* args, int group, int D, int nrep, bool hybrid, hipStream_t stream);
int av_cols_launch_k4(const void* args, int group, int D, int nrep, bool hybrid, hipStream_t stream);

// The column-slice kernel, where it applies: its B * Hkv * D/32 workgroups
// fill the device, the probability rows are 16-byte aligned, and every
// buffer offset (a head's V slice, the steps read past its end, a KV head's
// probability rows) fits 32 bits.  *launched = false: nothing launched.
int av_cols_launch(const void* p, int64_t sp_b, int64_t sp_h, const uint32_t* v_codes, const uint16_t* v_meta,
                   int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode,
                   const OutPair& o, int accumulate, bool* launched, hipStream_t stream) {
  *launched = false;
  const int nrep = Hq / Hkv;
  const int nslice = D / AVC_CW;
  const int64_t items = int64_t(B) * Hkv * nslice;
  const int64_t lim = int64_t(1) << 31;
  const int ngroups = T / group;
  const int64_t vw = int64_t(group) * bits / 32;
  // groups a launch may address past the range (the prefetches past a
  // wave's last step)
  const int64_t slack = int64_t(AVC_NW) * 6 * 8 + 8;
  if (items < num_cus() || ngroups <= 0 || items > int64_t(1) << 30) return IQ_OK;
  if (!aligned(p, 16) || sp_b % 8 || sp_h % 8 || sp_h < 0 || sp_b < 0) return IQ_OK;
  if ((int64_t(nrep - 1) * sp_h + T) * 2 >= lim || (ngroups + slack) * D * vw * 4 >= lim ||
      (ngroups + slack) * D * 4 >= lim || t_cap * D * bits / 8 >= lim)
    return IQ_OK;
  if (o.out32 && o.out16 && (o.s32b != o.s16b || o.s32h != o.s16h)) return IQ_OK;
  AVCArgs a{};
  a.p = (const uint16_t*)p; a.spb = sp_b; a.sph = sp_h;
  a.vc = v_codes; a.vm = v_meta; a.cap_groups = t_cap / group; a.g0 = t0 / group;
  a.Hkv = Hkv; a.ngroups = ngroups; a.vsym = mode == IQ_MODE_SYM;
  a.nslice = nslice; a.nitems = int(items);
  a.p_bytes = uint32_t((int64_t(nrep - 1) * sp_h + T) * 2);
  a.v_code_bytes = uint32_t(int64_t(ngroups) * D * vw * 4);
  a.v_meta_bytes = uint32_t(int64_t(ngroups) * D * meta_unit_bytes(mode));
  a.out32 = o.out32; a.out16 = o.out16;
  a.sob = o.out32 ? o.s32b : o.s16b;
  a.soh = o.out32 ? o.s32h : o.s16h;
  a.accumulate = accumulate;
  const bool hyb = mode == IQ_MODE_HYBRID;
  int e = IQ_ERR_BITS;
  switch (bits) {
    case 2: e = av_cols_launch_k2(&a, group, D, nrep, hyb, stream); break;
    case 3: e = av_cols_launch_k3(&a, group, D, nrep, hyb, stream); break;
    case 4: e = av_cols_launch_k4(&a, group, D, nrep, hyb, stream); break;
  }
  *launched = e == IQ_OK;
  return e;
}

int av_splits(int B, int Hkv, int T, int group) {
  const int ng = T / group;
  if (ng <= 0) return 0;
  return int(ceil_div(ng, groups_per_wg(B, Hkv, ng)));
}

size_t av_record_bytes(int B, int Hq, int T, int group) {
  return (rec_bytes_bound(int64_t(B) * Hq, T / group, group) + 255) & ~size_t(255);
}

size_t av_part_bytes(int B, int Hq, int T, int D, int group) {
  // Bound on the split count of any range of at most T tokens and any Hkv:
  // groups_per_wg() gives gpw >= ceil(ng / S) with S <= 4*CUs/B (Hkv = 1), and
  // gpw >= min(ng, 8), so nsplit <= min(S, ceil(ng / 8)) (and >= 1).  The
  // persistent kernel writes at most one slot per FSPLIT tokens.
  const int64_t ng = T / group;
  const int64_t s_max = std::max<int64_t>(1, int64_t(num_cus()) * 4 / std::max(B, 1));
  const int64_t bound = std::max<int64_t>({1, std::min<int64_t>(s_max, ceil_div(ng, 2 * NWAVES)), ceil_div(T, FSPLIT)});
  return ((size_t(bound) * B * Hq * D * 4) + 255) & ~size_t(255);
}

int av_record_launch(const void* p, int64_t sp_b, int64_t sp_h, int B, int Hq, int Hkv, int T, int group, int bits,
                     uint32_t* rec, hipStream_t stream) {
  const int ng = T / group;
  const int64_t n = int64_t(B) * Hq * ng;
  if (n == 0) return IQ_OK;
  return dispatch_rec(bits, group, Hq / Hkv, [&]<int BITS, int G, int R>() {
    av_record_kernel<BITS, G, R><<<dim3(unsigned(ceil_div(n, 256))), 256, 0, stream>>>(
        (const uint16_t*)p, sp_b, sp_h, B, Hkv, ng, rec);
    return launch_status();
  });
}

int av_launch_gpw(const uint32_t* rec, const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B, int Hq,
                  int Hkv, int t0, int T, int D, int group, int bits, int mode, float* part, int gpw,
                  hipStream_t stream) {
  const int ng = T / group;
  const int nsplit = int(ceil_div(ng, gpw));
  AVArgs a{rec, v_codes, v_meta, t_cap / group, Hkv, t0 / group, ng, gpw, part, mode == IQ_MODE_HYBRID};
  return dispatch_shape(bits, group, D, Hq / Hkv, mode == IQ_MODE_SYM, [&]<int BITS, int G, int DD, int R, bool S>() {
    av_kernel<BITS, G, DD, R, S><<<dim3(nsplit, B * Hkv), WG, 0, stream>>>(a);
    return launch_status();
  });
}

int av_main_launch(const uint32_t* rec, const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B,
                   int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float* part,
                   hipStream_t stream) {
  return av_launch_gpw(rec, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, part,
                       groups_per_wg(B, Hkv, T / group), stream);
}

// attn.V over the flash-decoding splits: one workgroup per QK^T split
int av_flash_launch(const uint32_t* rec, const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B,
                    int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float* part,
                    hipStream_t stream) {
  return av_launch_gpw(rec, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, part,
                       flash_split_tokens() / group, stream);
}

int av_combine_launch(const float* part, int nsplit, int B, int Hq, int D, const OutPair& o, int accumulate,
                      hipStream_t stream, int grid, int nrep) {
  const int64_t rows = int64_t(B) * Hq;
  if (rows == 0) return IQ_OK;
  // loads per round: 8, or 32 where a head can have more than eight runs (the
  // persistent kernel's workgroups over few (batch, KV head)s, or every split
  // slot without its workgroup count)
  const int64_t heads = std::max<int64_t>(1, rows / std::max(nrep, 1));
  const int64_t runs = grid > 0 ? std::min<int64_t>(nsplit, ceil_div(grid, heads) + 1) : nsplit;
  const dim3 g{unsigned(ceil_div(rows * D, 256))};
  if (runs > 8) av_combine_kernel<32><<<g, 256, 0, stream>>>(part, nsplit, Hq, D, rows, o, accumulate, grid, nrep);
  else av_combine_kernel<8><<<g, 256, 0, stream>>>(part, nsplit, Hq, D, rows, o, accumulate, grid, nrep);
  return launch_status();
}

// attn.V over the persistent fused kernel in attn.V-only mode; *grid = its
// workgroup count (0: the slices exceed its 32-bit buffer offsets, nothing
// launched)
int av_fused_launch(const void* p, int64_t sp_b, int64_t sp_h, const uint32_t* v_codes, const uint16_t* v_meta,
                    int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode,
                    float* part, int* grid, hipStream_t stream) {
  *grid = 0;
  const int nrep = Hq / Hkv;
  const int64_t lim = int64_t(1) << 31;
  if (sp_h < 0 || (int64_t(nrep - 1) * sp_h + T) * 2 >= lim || t_cap * D * bits / 8 >= lim ||
      t_cap * D * 4 / group >= lim)
    return IQ_OK;
  FusedArgs a{};
  a.q = (const uint16_t*)p; a.sqb = sp_b; a.sqh = sp_h;
  a.vc = v_codes; a.vm = v_meta; a.v_cap_groups = t_cap / group; a.vg0 = t0 / group;
  a.vsym = mode == IQ_MODE_SYM;
  a.Hkv = Hkv; a.T = T;
  a.nsplit = int(ceil_div(T, FSPLIT));
  a.nitems = a.nsplit * B * Hkv;
  a.v_code_bytes = uint32_t(int64_t(T) * D * bits / 8);
  a.v_meta_bytes = uint32_t(int64_t(T / group) * D * (a.vsym ? 2 : 4));
  a.q_bytes = uint32_t((int64_t(nrep - 1) * sp_h + T) * 2);
  a.part = part;
  const bool hyb = mode == IQ_MODE_HYBRID;
  return dispatch_shape(bits, group, D, nrep, 0, [&]<int VB, int G, int DD, int R, bool S>() {
    auto* kern = hyb ? flash_fused_kernel<VB, VB, G, DD, R, false, true, false, true>
                     : flash_fused_kernel<VB, VB, G, DD, R, false, true>;
    const int nt = FusedShape<G, R, false, true>::NT;
    static OccCache occ[2];  // workgroups per CU at once
    const int pc = blocks_per_cu(kern, nt, occ[hyb ? 1 : 0]);
    *grid = int(std::min<int64_t>(a.nitems, int64_t(pc) * num_cus()));
    kern<<<dim3(*grid), nt, 0, stream>>>(a);
    return launch_status();
  });
}

}  // namespace iq::detail

extern "C" {

size_t iq_av_workspace_bytes(int B, int Hq, int T, int D, int group) {
  if (B <= 0 || Hq <= 0 || T <= 0 || !group_ok(group) || !d_ok(D) || T % group) return 0;
  return detail::av_record_bytes(B, Hq, T, group) + detail::av_part_bytes(B, Hq, T, D, group);
}

int iq_av_gemv(const void* p, int64_t sp_b, int64_t sp_h, const uint32_t* v_codes, const uint16_t* v_meta,
               int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode,
               float* out32, void* out16, int64_t so_b, int64_t so_h, int accumulate, void* workspace,
               size_t workspace_bytes, void* stream) {
  if (int e = check_av(p, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode)) return e;
  IQ_CHECK(out32 || out16, IQ_ERR_NULL);
  IQ_CHECK(!accumulate || out32, IQ_ERR_NULL);
  IQ_CHECK(aligned(p, 2), IQ_ERR_ALIGN);
  hipStream_t st = (hipStream_t)stream;
  const detail::OutPair o{out32, so_b, so_h, (uint16_t*)out16, so_b, so_h};
  if (B == 0) return IQ_OK;
  if (T == 0) return accumulate ? detail::av_combine_launch(nullptr, 0, B, Hq, D, o, 1, st) : IQ_ERR_SHAPE;
  const size_t rb = detail::av_record_bytes(B, Hq, T, group);
  IQ_CHECK(workspace && workspace_bytes >= rb + detail::av_part_bytes(B, Hq, T, D, group), IQ_ERR_WORKSPACE);
  IQ_CHECK(aligned(workspace, 16), IQ_ERR_ALIGN);
  uint32_t* rec = (uint32_t*)workspace;
  float* part = (float*)((char*)workspace + rb);
  bool cols = false;
  if (int e = detail::av_cols_launch(p, sp_b, sp_h, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode,
                                     o, accumulate, &cols, st))
    return e;
  if (cols) return IQ_OK;
  int grid = 0;
  if (int e = detail::av_fused_launch(p, sp_b, sp_h, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode,
                                      part, &grid, st))
    return e;
  if (grid > 0)
    return detail::av_combine_launch(part, int(ceil_div(T, FSPLIT)), B, Hq, D, o, accumulate, st, grid, Hq / Hkv);
  if (int e = detail::av_record_launch(p, sp_b, sp_h, B, Hq, Hkv, T, group, bits, rec, st)) return e;
  if (int e = detail::av_main_launch(rec, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, part, st))
    return e;
  return detail::av_combine_launch(part, detail::av_splits(B, Hkv, T, group), B, Hq, D, o, accumulate, st);
}

}  // extern "C"
