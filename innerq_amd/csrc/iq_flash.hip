// Fused flash-decoding split (gfx950): QK^T, softmax within the split and
// attn.V of one (batch, KV head) over FSPLIT consecutive tokens, in one
// workgroup, for K and V stores that share bit width and group size.
//
// Phases of a workgroup (four waves):
//   0  query operand records of the D/G head_dim groups, built in LDS from q
//      while the first K group's loads are in flight (a key normalization,
//      which the reference applies to the dequantized keys, cache.py:128-133
//      and 249, is folded into q as hi/lo fp16 parts of q*n);
//   1  QK^T: wave w owns 64-token blocks 2w, 2w+1 of the split, lane = token;
//      it walks the head_dim groups with the next group's code words and
//      {scale, zero} prefetched, eight v_mfma_f32_4x4x4f16 per 32 codes and
//      four query heads (iq_gemv.h);
//   2  softmax within the split: max m and sum l of exp(logit - m) per head
//      go to the split statistics, the probabilities exp(logit - m), rounded
//      to fp16, to LDS.  The first V groups' loads are issued first, so they
//      overlap this phase and the next;
//   3  probability operand records of the split's V groups, built in LDS;
//   4  attn.V: wave w takes V groups w, w+4, ...; lane = head_dim column
//      d = lane + 64 e; the waves' partial sums are reduced in LDS in a fixed
//      order and the split's unnormalized output goes to the partials.
// Nothing but the split statistics and partials leaves the workgroup: the
// logits and probabilities never touch HBM, and one launch replaces the
// query-record, QK^T and attn.V launches of the unfused path.  A combine
// kernel (iq_decode.hip) merges the splits.
//
// The store formats follow the unfused kernels: K codes [B,H,t_cap/64,D/G,64,W],
// V codes [B,H,t_cap/G,D,W]; sym or asym per store is a runtime flag (a
// uniform branch), so the kernel is instantiated per (bits, G, D, n_rep) only.
#include "iq_gemv.h"

using namespace iq;

namespace {

constexpr int FBPW = IQ_FLASH_BPW;                     // 64-token K blocks per wave
constexpr int FSPLIT = NWAVES * FBPW * TOKEN_BLOCK;    // tokens per workgroup


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

// Records use the padded stride rec_dwords(): each head's pairs start 16-byte
// aligned, as the 16-byte LDS reads of the matrix-core operand require.
template <int G, int D, int NREP>
struct FusedSmem {
  alignas(16) uint32_t qrec[D / G][qrec_dwords<G, NREP>()];
  alignas(16) uint32_t vrec[FSPLIT / G][rec_dwords<G, NREP>()];
  union alignas(16) {
    uint16_t p[NREP][FSPLIT];        // phases 2-3
    float red[NWAVES - 1][NREP][D];  // after phase 4
  };
  float m[NWAVES][NREP];
  float l[NWAVES][NREP];
};

__device__ __forceinline__ uint32_t load_meta(const uint16_t* meta, int64_t unit, int sym) {
  if (sym) return meta[unit];
  return reinterpret_cast<const uint32_t*>(meta)[unit];
}

template <int BITS, int G, int D, int NREP>
__global__ __launch_bounds__(WG) void flash_fused_kernel(FusedArgs a) {
  constexpr int NG = D / G;
  constexpr int W = G * BITS / 32;
  constexpr int NP = G / 2;
  constexpr int GPS = FSPLIT / G;  // V groups per split
  constexpr int DPL = D / 64;
  constexpr int VNB = 2;           // V groups per step
  constexpr float ZS = -float(1 << (BITS - 1));
  __shared__ FusedSmem<G, D, NREP> sm;

  const int bh = blockIdx.y;
  const int split = blockIdx.x;
  const int b = bh / a.Hkv, kvh = bh % a.Hkv;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hl = lane & 3;

  // ---- K loads of group 0 (in flight during phase 0) ----
  // blocks past the range (tail waves) re-read its last block: in-bounds
  // loads whose tokens are masked out
  const int nblk = (a.T + TOKEN_BLOCK - 1) / TOKEN_BLOCK;
  const int wblk = (split * NWAVES + wave) * FBPW;
  const int64_t kbase = int64_t(bh) * a.k_cap_blocks + a.kblk0;
  const uint32_t* kcb = a.kc + kbase * (NG * TOKEN_BLOCK * W);
  const uint16_t* kmb = a.km + kbase * (NG * TOKEN_BLOCK * (a.ksym ? 1 : 2));
  uint32_t kw[FBPW][W], kmv[FBPW];
  auto load_k = [&](int g) {
#pragma unroll
    for (int j = 0; j < FBPW; ++j) {
      const int blk = min(wblk + j, nblk - 1);
      const int64_t unit = (int64_t(blk) * NG + g) * TOKEN_BLOCK + lane;
      load_words<W>(kcb + unit * W, kw[j]);
      kmv[j] = load_meta(kmb, unit, a.ksym);
    }
  };
  load_k(0);

  // V groups of the split: wave w takes groups w, w+4, ..., VNB per step
  const int ngs = min(GPS, a.T / G - split * GPS);  // >= 1: T and FSPLIT are multiples of G
  const int vcnt = ngs > wave ? (ngs - wave + NWAVES - 1) / NWAVES : 0;
  const int64_t vbase = int64_t(bh) * a.v_cap_groups + a.vg0 + int64_t(split) * GPS;
  uint32_t vw[VNB][DPL][W], vmv[VNB][DPL];
  auto load_v = [&](int i0) {
#pragma unroll
    for (int u = 0; u < VNB; ++u) {
      if (i0 + u < vcnt) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          const int64_t unit = (vbase + wave + NWAVES * (i0 + u)) * D + lane + 64 * e;
          load_words<W>(a.vc + unit * W, vw[u][e]);
          vmv[u][e] = load_meta(a.vm, unit, a.vsym);
        }
      }
    }
  };

  // ---- phase 0: query records ----
  const bool qsplit = a.norm != nullptr;
  {
    const uint16_t* qb = a.q + b * a.sqb + int64_t(kvh * NREP) * a.sqh;
    const uint16_t* nb = a.norm ? a.norm + int64_t(bh) * D : nullptr;
    for (int i = tid; i < NG * NREP * NP; i += WG) {
      const int k = i % NP, h = (i / NP) % NREP, g = i / (NP * NREP);
      float unused = 0.f;
      qrec_pair(qb + h * a.sqh + g * G, nb ? nb + g * G : nullptr, plan_a<BITS>(k), plan_c<BITS>(k),
                &sm.qrec[g][h * NP + k], &sm.qrec[g][(NREP + h) * NP + k], unused);
    }
    __syncthreads();
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
    __syncthreads();
  }

  // ---- phase 1: QK^T ----
  float acc[FBPW][NREP];
#pragma unroll
  for (int j = 0; j < FBPW; ++j)
#pragma unroll
    for (int h = 0; h < NREP; ++h) acc[j][h] = 0.f;
#pragma unroll 1
  for (int g = 0; g < NG; ++g) {
    uint32_t cw[FBPW][W], cm[FBPW];
#pragma unroll
    for (int j = 0; j < FBPW; ++j) {
      cm[j] = kmv[j];
#pragma unroll
      for (int x = 0; x < W; ++x) cw[j][x] = kw[j][x];
    }
    if (g + 1 < NG) load_k(g + 1);
    if (a.ksym) {
#pragma unroll
      for (int j = 0; j < FBPW; ++j) to_offset_binary<BITS>(cw[j], W);
    }
    float d[FBPW][NREP];
    qk_group_dot<BITS, G, NREP, FBPW>(cw, &sm.qrec[g][0], hl, qsplit, d);
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
  if (vcnt > 0) load_v(0);  // in flight during phases 2 and 3

  // ---- phase 2: softmax within the split ----
  float lg[FBPW][NREP];
#pragma unroll
  for (int j = 0; j < FBPW; ++j) {
    const int t = (wblk + j) * TOKEN_BLOCK + lane;
#pragma unroll
    for (int h = 0; h < NREP; ++h) lg[j][h] = (t < a.T) ? acc[j][h] * a.scale : -INFINITY;
  }
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    float mx = lg[0][h];
#pragma unroll
    for (int j = 1; j < FBPW; ++j) mx = fmaxf(mx, lg[j][h]);
    mx = wave_max(mx);
    if (lane == 0) sm.m[wave][h] = mx;
  }
  __syncthreads();
  float mh[NREP];
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    mh[h] = fmaxf(fmaxf(sm.m[0][h], sm.m[1][h]), fmaxf(sm.m[2][h], sm.m[3][h]));
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < FBPW; ++j) {
      const float p = lg[j][h] == -INFINITY ? 0.f : __expf(lg[j][h] - mh[h]);
      ls += p;
      sm.p[h][(wave * FBPW + j) * TOKEN_BLOCK + lane] = __half_as_ushort(__float2half_rn(p));
    }
    ls = wave_sum(ls);
    if (lane == 0) sm.l[wave][h] = ls;
  }
  __syncthreads();
  const int64_t rows = int64_t(gridDim.y) * NREP;
  if (tid < NREP) {
    float* dst = a.ml + (int64_t(split) * rows + int64_t(bh) * NREP + tid) * 2;
    dst[0] = mh[tid];
    dst[1] = (sm.l[0][tid] + sm.l[1][tid]) + (sm.l[2][tid] + sm.l[3][tid]);
  }

  // ---- phase 3: probability records of the split's V groups ----
  for (int i = tid; i < GPS * NREP * NP; i += WG) {
    const int k = i % NP, h = (i / NP) % NREP, gl = i / (NP * NREP);
    const uint16_t* pp = &sm.p[h][gl * G];
    sm.vrec[gl][h * NP + k] = uint32_t(pp[plan_a<BITS>(k)]) | (uint32_t(pp[plan_c<BITS>(k)]) << 16);
  }
  if (tid < GPS * NREP) {
    const int gl = tid / NREP, h = tid % NREP;
    const uint4* pp = reinterpret_cast<const uint4*>(&sm.p[h][gl * G]);
    float s = 0.f;
#pragma unroll
    for (int x = 0; x < G / 8; ++x) {
      const uint4 u = pp[x];
      const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int y = 0; y < 4; ++y) s += h2f(uint16_t(uw[y] & 0xffffu)) + h2f(uint16_t(uw[y] >> 16));
    }
    sm.vrec[gl][NP * NREP + h] = __float_as_uint(s);
  }
  __syncthreads();

  // ---- phase 4: attn.V ----
  float o[NREP][DPL];
#pragma unroll
  for (int h = 0; h < NREP; ++h)
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[h][e] = 0.f;
  for (int i = 0; i < vcnt; i += VNB) {
    uint32_t cw[VNB][DPL][W], cm[VNB][DPL];
#pragma unroll
    for (int u = 0; u < VNB; ++u)
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        cm[u][e] = vmv[u][e];
#pragma unroll
        for (int x = 0; x < W; ++x) cw[u][e][x] = vw[u][e][x];
      }
    if (i + VNB < vcnt) load_v(i + VNB);
#pragma unroll
    for (int u = 0; u < VNB; ++u) {
      if (i + u < vcnt) {
        const int gl = wave + NWAVES * (i + u);
        if (a.vsym) {
#pragma unroll
          for (int e = 0; e < DPL; ++e) to_offset_binary<BITS>(cw[u][e], W);
        }
        f4_t dv[DPL][(NREP + 3) / 4];
        group_mfma<BITS, G, NREP, DPL>(cw[u], &sm.vrec[gl][0], hl, dv);
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          const float s = h2f(uint16_t(cm[u][e] & 0xffffu));
          const float z = a.vsym ? ZS * s : h2f(uint16_t(cm[u][e] >> 16));
#pragma unroll
          for (int h = 0; h < NREP; ++h) {
            const float ps = __uint_as_float(sm.vrec[gl][NP * NREP + h]);
            o[h][e] = fmaf(s, dv[e][h / 4][h % 4], fmaf(z, ps, o[h][e]));
          }
        }
      }
    }
  }
  // sm.p is dead (every wave passed the barrier after phase 3): reuse it
  if (wave > 0) {
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < DPL; ++e) sm.red[wave - 1][h][lane + 64 * e] = o[h][e];
  }
  __syncthreads();
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
  }
}

}  // namespace

namespace iq::detail {

int flash_fused_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const FusedStore& k,
                       const FusedStore& v, int B, int Hq, int Hkv, int T, int D, float scale, float* ml,
                       float* part, hipStream_t stream) {
  if (B == 0 || T == 0) return IQ_OK;
  if (k.bits != v.bits || k.group != v.group) return IQ_ERR_GROUP;
  if (T % k.group || FSPLIT != flash_split_tokens()) return IQ_ERR_GROUP;
  if (k.t0 % TOKEN_BLOCK || v.t0 % v.group) return IQ_ERR_ALIGN;
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
