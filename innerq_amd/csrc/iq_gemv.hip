// Decode GEMVs over packed KV stores (gfx950): QK^T, attn.V, softmax and the
// decode-attention driver.
//
// QK^T  (K grouped along head_dim)
//   One wave64 owns 64 consecutive tokens of one (batch, KV head): lane = token.
//   For every group g the lane reads its token's G*b/32 code words (one
//   16-byte load for 4-bit G=32; a wave reads 1 KiB contiguous because the K
//   store keeps the 64 tokens of a block group-major) and the {scale, zero}
//   dword.  The n_rep = Hq/Hkv query heads that share the KV head are served
//   from the same unpacked pairs: v_dot2_f32_f16 against query pairs that are
//   pre-permuted into the unpack plan's pair order in LDS (broadcast reads).
//   Per group and head:  logit += s * (sum q*c) + z * sum(q).
//
// attn.V (V grouped along tokens)
//   A workgroup owns a token range of one (batch, KV head) (split-T).  The
//   probability rows of its n_rep heads are staged into LDS in pair order,
//   with per-group sums of p and the bias constants.  Lane = head_dim column
//   (2 columns per lane at D=128): per group the lane reads its columns'
//   code words (a wave reads the group's D*G*b/8 bytes contiguously) and
//   accumulates  s[g,d] * sum p*c + z[g,d] * sum p.  The four waves' partial
//   sums are reduced in LDS, the workgroup writes one fp32 partial per split,
//   and a second kernel sums the splits in a fixed order (no atomics).
#include "iq_common.h"
#include "iq_device.h"

#include <utility>

using namespace iq;

namespace {

constexpr int NWAVES = 4;
constexpr int WG = NWAVES * 64;

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

// index of the first / second code of pair k of a group (super-block aware)
template <int BITS>
__host__ __device__ constexpr int pair_code_a(int k) {
  return (k / Plan<BITS>::NPAIR) * Plan<BITS>::CODES + Plan<BITS>::A[k % Plan<BITS>::NPAIR];
}
template <int BITS>
__host__ __device__ constexpr int pair_code_c(int k) {
  return (k / Plan<BITS>::NPAIR) * Plan<BITS>::CODES + Plan<BITS>::C[k % Plan<BITS>::NPAIR];
}
template <int BITS>
__host__ __device__ constexpr float pair_bias_a(int k) { return bias_a<BITS>(k % Plan<BITS>::NPAIR); }
template <int BITS>
__host__ __device__ constexpr float pair_bias_c(int k) { return bias_c<BITS>(k % Plan<BITS>::NPAIR); }

// Runtime lookup of the constexpr pair tables (used only while staging).
template <int BITS, int NP>
struct PairTable {
  int a[NP], c[NP];
  float ba[NP], bc[NP];
  constexpr PairTable() : a(), c(), ba(), bc() {
    for (int k = 0; k < NP; ++k) {
      a[k] = pair_code_a<BITS>(k);
      c[k] = pair_code_c<BITS>(k);
      ba[k] = pair_bias_a<BITS>(k);
      bc[k] = pair_bias_c<BITS>(k);
    }
  }
};

// Accumulate one group's pairs: acc[h] += dot2(op[k][h], pair_k(words)).
template <int BITS, int NSB, int NREP, typename OpFn, int... K>
__device__ __forceinline__ void group_dot_impl(const uint32_t* w, float* acc, OpFn op,
                                               std::integer_sequence<int, K...>) {
  constexpr int NPS = Plan<BITS>::NPAIR;
  constexpr int SBW = Plan<BITS>::WORDS;
  (
      [&] {
        constexpr int sb = K / NPS;
        constexpr int kk = K % NPS;
        const h2_t x = extract_pair<BITS, kk>(w + sb * SBW);
#pragma unroll
        for (int h = 0; h < NREP; ++h) acc[h] = dot2(op(K, h), x, acc[h]);
      }(),
      ...);
}

template <int BITS, int G, int NREP, typename OpFn>
__device__ __forceinline__ void group_dot(const uint32_t* w, float* acc, OpFn op) {
  constexpr int NP = G / 2;
  constexpr int NSB = (G * BITS / 32) / Plan<BITS>::WORDS;
  group_dot_impl<BITS, NSB, NREP>(w, acc, op, std::make_integer_sequence<int, NP>{});
}

template <int BITS>
__device__ __forceinline__ void to_offset_binary(uint32_t* w, int nw) {
  constexpr int SBW = Plan<BITS>::WORDS;
#pragma unroll
  for (int j = 0; j < nw; ++j) w[j] ^= Plan<BITS>::SIGN[j % SBW];
}

// ============================================================================
// QK^T
// ============================================================================
struct QKArgs {
  const uint16_t* q;
  int64_t sqb, sqh;
  const uint16_t* norm;
  const uint32_t* kc;
  const uint16_t* km;
  int64_t cap_blocks;
  int Hkv, blk0, T;
  float scale;
  float* out;
  int64_t sob, soh;
  int bpw;  // token blocks per wave
};

template <int BITS, int G, int D, int NREP, bool SYM>
__global__ __launch_bounds__(WG) void qk_kernel(QKArgs a) {
  constexpr int NG = D / G;
  constexpr int W = G * BITS / 32;
  constexpr int NP = G / 2;
  constexpr int M = SYM ? 1 : 2;
  constexpr PairTable<BITS, NP> PT{};
  __shared__ h2_t qp[NG][NP][NREP];
  __shared__ float beta[NG][NREP];
  __shared__ float qsum[NG][NREP];

  const int bh = blockIdx.y;
  const int b = bh / a.Hkv, kvh = bh % a.Hkv;

  // stage q' (optionally q * norm, rounded to fp16) in pair order
  for (int i = threadIdx.x; i < NG * NP * NREP; i += WG) {
    const int h = i % NREP, k = (i / NREP) % NP, g = i / (NREP * NP);
    const int ia = g * G + PT.a[k], ic = g * G + PT.c[k];
    const uint16_t* qrow = a.q + b * a.sqb + (kvh * NREP + h) * a.sqh;
    float qa = h2f(qrow[ia]), qc = h2f(qrow[ic]);
    if (a.norm) {
      const uint16_t* nr = a.norm + int64_t(bh) * D;
      qa *= h2f(nr[ia]);
      qc *= h2f(nr[ic]);
    }
    qp[g][k][h] = h2_from_halves(__float2half_rn(qa), __float2half_rn(qc));
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NG * NREP; i += WG) {
    const int h = i % NREP, g = i / NREP;
    float bs = 0.f, sm = 0.f;
    for (int k = 0; k < NP; ++k) {
      const float xa = float(qp[g][k][h].x), xc = float(qp[g][k][h].y);
      bs += xa * PT.ba[k] + xc * PT.bc[k];
      sm += xa + xc;
    }
    beta[g][h] = bs;
    qsum[g][h] = sm;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nblk = (a.T + TOKEN_BLOCK - 1) / TOKEN_BLOCK;
  const int first = (blockIdx.x * NWAVES + wave) * a.bpw;
  const int last = min(first + a.bpw, nblk);
  const uint32_t* kcb = a.kc + (int64_t(bh) * a.cap_blocks + a.blk0) * (NG * TOKEN_BLOCK * W);
  const uint16_t* kmb = a.km + (int64_t(bh) * a.cap_blocks + a.blk0) * (NG * TOKEN_BLOCK * M);
  float* outb = a.out + int64_t(b) * a.sob + int64_t(kvh * NREP) * a.soh;

  uint32_t w[NG][W];
  uint32_t m[NG];
  auto load_block = [&](int blk) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int64_t unit = (int64_t(blk) * NG + g) * TOKEN_BLOCK + lane;
      load_words<W>(kcb + unit * W, w[g]);
      if constexpr (SYM) m[g] = kmb[unit];
      else m[g] = reinterpret_cast<const uint32_t*>(kmb)[unit];
    }
  };
  if (first < last) load_block(first);
  for (int blk = first; blk < last; ++blk) {
    uint32_t cw[NG][W];
    uint32_t cm[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      cm[g] = m[g];
#pragma unroll
      for (int j = 0; j < W; ++j) cw[g][j] = w[g][j];
    }
    if (blk + 1 < last) load_block(blk + 1);  // prefetch the next block
    // Re-read the LDS query pairs every block: hoisting all NG*NP*NREP of them
    // out of the loop would need hundreds of VGPRs.
    asm volatile("" ::: "memory");

    float acc[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) acc[h] = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if constexpr (SYM) to_offset_binary<BITS>(cw[g], W);
      float dv[NREP];
#pragma unroll
      for (int h = 0; h < NREP; ++h) dv[h] = -beta[g][h];
      group_dot<BITS, G, NREP>(cw[g], dv, [&](int k, int h) { return qp[g][k][h]; });
      const float s = h2f(uint16_t(cm[g] & 0xffffu));
      const float z = SYM ? -float(1 << (BITS - 1)) * s : h2f(uint16_t(cm[g] >> 16));
#pragma unroll
      for (int h = 0; h < NREP; ++h) acc[h] = fmaf(s, dv[h], fmaf(z, qsum[g][h], acc[h]));
    }
    const int t = blk * TOKEN_BLOCK + lane;
    if (t < a.T) {
#pragma unroll
      for (int h = 0; h < NREP; ++h) outb[h * a.soh + t] = acc[h] * a.scale;
    }
  }
}

// ============================================================================
// attn.V
// ============================================================================
constexpr int AV_MAX_TOK = 2048;  // tokens per workgroup (LDS staging bound)

struct AVArgs {
  const uint16_t* p;
  int64_t spb, sph;
  const uint32_t* vc;
  const uint16_t* vm;
  int64_t cap_groups;
  int Hkv, g0, ngroups;  // store group offset, groups in the range
  int gpw;               // groups per workgroup
  float* part;           // [nsplit][B*Hq][D]
  int Hq;
};

template <int BITS, int G, int D, int NREP, bool SYM>
__global__ __launch_bounds__(WG) void av_kernel(AVArgs a) {
  constexpr int W = G * BITS / 32;
  constexpr int NP = G / 2;
  constexpr int M = SYM ? 1 : 2;
  constexpr int DPL = D / 64;
  constexpr int MAXG = AV_MAX_TOK / G;
  constexpr PairTable<BITS, NP> PT{};
  __shared__ h2_t pp[MAXG][NP][NREP];
  __shared__ float beta[MAXG][NREP];
  __shared__ float psum[MAXG][NREP];
  __shared__ float red[NWAVES - 1][NREP][D];

  const int bh = blockIdx.y;
  const int b = bh / a.Hkv, kvh = bh % a.Hkv;
  const int split = blockIdx.x;
  const int gl0 = split * a.gpw;
  const int ng = min(a.gpw, a.ngroups - gl0);
  const uint16_t* prow0 = a.p + b * a.spb + int64_t(kvh * NREP) * a.sph + int64_t(gl0) * G;

  for (int i = threadIdx.x; i < ng * NP * NREP; i += WG) {
    const int h = i % NREP, k = (i / NREP) % NP, g = i / (NREP * NP);
    const uint16_t* pr = prow0 + h * a.sph + g * G;
    pp[g][k][h] = h2_from_halves(__ushort_as_half(pr[PT.a[k]]), __ushort_as_half(pr[PT.c[k]]));
  }
  __syncthreads();
  for (int i = threadIdx.x; i < ng * NREP; i += WG) {
    const int h = i % NREP, g = i / NREP;
    float bs = 0.f, sm = 0.f;
    for (int k = 0; k < NP; ++k) {
      const float xa = float(pp[g][k][h].x), xc = float(pp[g][k][h].y);
      bs += xa * PT.ba[k] + xc * PT.bc[k];
      sm += xa + xc;
    }
    beta[g][h] = bs;
    psum[g][h] = sm;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d0 = lane * DPL;
  const int64_t gbase = int64_t(bh) * a.cap_groups + a.g0 + gl0;
  float acc[NREP][DPL];
#pragma unroll
  for (int h = 0; h < NREP; ++h)
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[h][e] = 0.f;

  uint32_t w[DPL][W];
  uint32_t m[DPL];
  auto load_group = [&](int g) {
    const int64_t unit = (gbase + g) * D + d0;
    load_words<DPL * W>(a.vc + unit * W, &w[0][0]);
    if constexpr (SYM) {
      if constexpr (DPL == 2) {
        const uint32_t mm = reinterpret_cast<const uint32_t*>(a.vm + unit)[0];
        m[0] = mm & 0xffffu;
        m[1] = mm >> 16;
      } else {
        m[0] = a.vm[unit];
      }
    } else {
      if constexpr (DPL == 2) {
        const uint2 mm = reinterpret_cast<const uint2*>(a.vm + unit * 2)[0];
        m[0] = mm.x;
        m[1] = mm.y;
      } else {
        m[0] = reinterpret_cast<const uint32_t*>(a.vm)[unit];
      }
    }
  };
  int g = wave;
  if (g < ng) load_group(g);
  for (; g < ng; g += NWAVES) {
    uint32_t cw[DPL][W];
    uint32_t cm[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      cm[e] = m[e];
#pragma unroll
      for (int j = 0; j < W; ++j) cw[e][j] = w[e][j];
    }
    if (g + NWAVES < ng) load_group(g + NWAVES);
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      if constexpr (SYM) to_offset_binary<BITS>(cw[e], W);
      float dv[NREP];
#pragma unroll
      for (int h = 0; h < NREP; ++h) dv[h] = -beta[g][h];
      group_dot<BITS, G, NREP>(cw[e], dv, [&](int k, int h) { return pp[g][k][h]; });
      const float s = h2f(uint16_t(cm[e] & 0xffffu));
      const float z = SYM ? -float(1 << (BITS - 1)) * s : h2f(uint16_t(cm[e] >> 16));
#pragma unroll
      for (int h = 0; h < NREP; ++h) acc[h][e] = fmaf(s, dv[h], fmaf(z, psum[g][h], acc[h][e]));
    }
  }
  // reduce the four waves' partial sums (fixed order) and write this split
  if (wave > 0) {
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int e = 0; e < DPL; ++e) red[wave - 1][h][d0 + e] = acc[h][e];
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
        for (int r = 0; r < NWAVES - 1; ++r) v += red[r][h][d0 + e];
        dst[h * D + d0 + e] = v;
      }
  }
}

// out[bq][d] (+)= sum_split part[split][bq][d]
struct OutPair {
  float* out32;
  int64_t s32b, s32h;
  uint16_t* out16;
  int64_t s16b, s16h;
};
__global__ __launch_bounds__(256) void av_combine_kernel(const float* __restrict__ part, int nsplit, int Hq, int D,
                                                         int64_t rows, OutPair o, int accumulate) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * D) return;
  const int64_t bq = i / D;
  const int d = int(i % D);
  float v = 0.f;
  for (int s = 0; s < nsplit; ++s) v += part[(int64_t(s) * rows + bq) * D + d];
  const int64_t off32 = (bq / Hq) * o.s32b + (bq % Hq) * o.s32h + d;
  if (accumulate) v += o.out32[off32];
  if (o.out32) o.out32[off32] = v;
  if (o.out16) o.out16[(bq / Hq) * o.s16b + (bq % Hq) * o.s16h + d] = __half_as_ushort(__float2half_rn(v));
}

// ============================================================================
// fp16 (sink / recent) segments, softmax
// ============================================================================
// logits[b, hq, t0 + t] = scale * q . K[b, kvh, t]    one thread per (b, hq, t)
__global__ __launch_bounds__(256) void dense_qk_kernel(const uint16_t* __restrict__ q, int64_t sqb, int64_t sqh,
                                                       const uint16_t* __restrict__ k, int64_t skb, int64_t skh,
                                                       int64_t skt, int B, int Hq, int Hkv, int n, int D,
                                                       float scale, float* out, int64_t sob, int64_t soh,
                                                       int t_out0) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(B) * Hq * n) return;
  const int t = int(i % n);
  const int hq = int((i / n) % Hq);
  const int b = int(i / (int64_t(n) * Hq));
  const int kvh = hq / (Hq / Hkv);
  const uint16_t* qr = q + b * sqb + hq * sqh;
  const uint16_t* kr = k + b * skb + kvh * skh + t * skt;
  float s = 0.f;
  for (int d = 0; d < D; ++d) s = fmaf(h2f(qr[d]), h2f(kr[d]), s);
  out[b * sob + hq * soh + t_out0 + t] = s * scale;
}

// out32[b, hq, d] = sum over two fp16 V segments of p[b, hq, tp + t] * V[b, kvh, t, d]
struct DenseSeg {
  const uint16_t* v;
  int64_t sb, sh, st;
  int n, tp;
};
__global__ __launch_bounds__(256) void dense_av_kernel(const uint16_t* __restrict__ p, int64_t spb, int64_t sph,
                                                       DenseSeg s0, DenseSeg s1, int B, int Hq, int Hkv, int D,
                                                       float* out32, int64_t sob, int64_t soh) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(B) * Hq * D) return;
  const int d = int(i % D);
  const int hq = int((i / D) % Hq);
  const int b = int(i / (int64_t(D) * Hq));
  const int kvh = hq / (Hq / Hkv);
  const uint16_t* pr = p + b * spb + hq * sph;
  float acc = 0.f;
  for (int t = 0; t < s0.n; ++t) acc = fmaf(h2f(pr[s0.tp + t]), h2f(s0.v[b * s0.sb + kvh * s0.sh + t * s0.st + d]), acc);
  for (int t = 0; t < s1.n; ++t) acc = fmaf(h2f(pr[s1.tp + t]), h2f(s1.v[b * s1.sb + kvh * s1.sh + t * s1.st + d]), acc);
  out32[b * sob + hq * soh + d] = acc;
}

// p = fp16( softmax_fp32(logits row) ), one workgroup per row
__global__ __launch_bounds__(256) void softmax_kernel(const float* __restrict__ x, int T, uint16_t* __restrict__ p) {
  __shared__ float sh[256 / 64];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * T;
  uint16_t* pr = p + row * T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float m = -INFINITY;
  for (int t = threadIdx.x; t < T; t += 256) m = fmaxf(m, xr[t]);
  m = wave_max(m);
  if (lane == 0) sh[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  __syncthreads();
  float l = 0.f;
  for (int t = threadIdx.x; t < T; t += 256) l += __expf(xr[t] - m);
  l = wave_sum(l);
  if (lane == 0) sh[wave] = l;
  __syncthreads();
  l = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  for (int t = threadIdx.x; t < T; t += 256) pr[t] = __half_as_ushort(__float2half_rn(__expf(xr[t] - m) / l));
}

// ---------------------------------------------------------------------------
// host-side launch helpers
// ---------------------------------------------------------------------------
int g_num_cus = 0;
int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        g_num_cus <= 0)
      g_num_cus = 256;
  }
  return g_num_cus;
}

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

int check_qk(const void* q, const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap, int B, int Hq, int Hkv,
             int t0, int T, int D, int group, int bits, int mode, const float* out) {
  IQ_CHECK(q && k_codes && k_meta && out, IQ_ERR_NULL);
  if (int e = check_common(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && T >= 0 && t0 >= 0 && Hkv > 0 && Hq > 0, IQ_ERR_SHAPE);
  IQ_CHECK(d_ok(D) && Hq % Hkv == 0 && nrep_ok(Hq / Hkv), IQ_ERR_SHAPE);
  IQ_CHECK(D % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(t_cap % TOKEN_BLOCK == 0 && t0 % TOKEN_BLOCK == 0, IQ_ERR_ALIGN);
  IQ_CHECK(int64_t(t0) + T <= t_cap, IQ_ERR_RANGE);
  IQ_CHECK(aligned(k_codes, 16) && aligned(k_meta, 4), IQ_ERR_ALIGN);
  return IQ_OK;
}

int launch_qk(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const uint32_t* k_codes,
              const uint16_t* k_meta, int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group,
              int bits, int mode, float scale, float* out, int64_t so_b, int64_t so_h, hipStream_t stream) {
  if (B == 0 || T == 0) return IQ_OK;
  const int nblk = int(ceil_div(T, TOKEN_BLOCK));
  const int64_t units = int64_t(B) * Hkv * nblk;
  // enough waves to fill the chip (~8 per CU), at most 8 blocks per wave
  const int64_t target_waves = int64_t(num_cus()) * 8;
  int bpw = int(std::max<int64_t>(1, std::min<int64_t>(8, units / std::max<int64_t>(1, target_waves))));
  const int wgx = int(ceil_div(nblk, int64_t(bpw) * NWAVES));
  QKArgs a{(const uint16_t*)q, sq_b, sq_h, (const uint16_t*)norm, k_codes, k_meta, t_cap / TOKEN_BLOCK, Hkv,
           t0 / TOKEN_BLOCK, T, scale, out, so_b, so_h, bpw};
  return dispatch_shape(bits, group, D, Hq / Hkv, mode == IQ_MODE_SYM, [&]<int BITS, int G, int DD, int R, bool S>() {
    qk_kernel<BITS, G, DD, R, S><<<dim3(wgx, B * Hkv), WG, 0, stream>>>(a);
    return launch_status();
  });
}

// split-T plan for attn.V: groups per workgroup
int av_groups_per_wg(int B, int Hkv, int T, int group) {
  const int ngroups = T / group;
  const int maxg = AV_MAX_TOK / group;
  const int64_t target_wgs = int64_t(num_cus()) * 4;
  const int64_t bhs = std::max<int64_t>(1, int64_t(B) * Hkv);
  int64_t splits = std::max<int64_t>(1, target_wgs / bhs);
  int gpw = int(ceil_div(ngroups, splits));
  gpw = std::max(gpw, std::min(ngroups, 4 * NWAVES));  // at least 4 groups per wave when possible
  gpw = std::min(std::max(gpw, 1), maxg);
  return gpw;
}

size_t av_ws_bytes(int B, int Hq, int T, int D, int group, int Hkv_hint) {
  // the split count depends on Hkv only through B*Hkv; use Hkv = Hq (largest split count bound)
  if (T <= 0 || group <= 0) return 0;
  const int ngroups = T / group;
  const int maxg_min = 1;
  (void)maxg_min;
  const int gpw = av_groups_per_wg(B, Hkv_hint, T, group);
  const int64_t nsplit = ceil_div(ngroups, gpw);
  return size_t(nsplit) * size_t(B) * size_t(Hq) * size_t(D) * sizeof(float);
}

int check_av(const void* p, const uint32_t* v_codes, const uint16_t* v_meta, int64_t t_cap, int B, int Hq, int Hkv,
             int t0, int T, int D, int group, int bits, int mode) {
  IQ_CHECK(p && v_codes && v_meta, IQ_ERR_NULL);
  if (int e = check_common(bits, group, mode)) return e;
  IQ_CHECK(B >= 0 && T >= 0 && t0 >= 0 && Hkv > 0 && Hq > 0, IQ_ERR_SHAPE);
  IQ_CHECK(d_ok(D) && Hq % Hkv == 0 && nrep_ok(Hq / Hkv), IQ_ERR_SHAPE);
  IQ_CHECK(T % group == 0 && t0 % group == 0 && t_cap % group == 0, IQ_ERR_GROUP);
  IQ_CHECK(int64_t(t0) + T <= t_cap, IQ_ERR_RANGE);
  IQ_CHECK(aligned(v_codes, 16) && aligned(v_meta, 8), IQ_ERR_ALIGN);
  return IQ_OK;
}

int launch_av(const void* p, int64_t sp_b, int64_t sp_h, const uint32_t* v_codes, const uint16_t* v_meta,
              int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode,
              const OutPair& o, int accumulate, float* ws, size_t ws_bytes, hipStream_t stream) {
  if (B == 0) return IQ_OK;
  const int64_t rows = int64_t(B) * Hq;
  if (T == 0) {
    if (accumulate) {
      av_combine_kernel<<<dim3(unsigned(ceil_div(rows * D, 256))), 256, 0, stream>>>(ws, 0, Hq, D, rows, o, 1);
      return launch_status();
    }
    return IQ_ERR_SHAPE;
  }
  const int ngroups = T / group;
  const int gpw = av_groups_per_wg(B, Hkv, T, group);
  const int nsplit = int(ceil_div(ngroups, gpw));
  IQ_CHECK(ws && ws_bytes >= size_t(nsplit) * size_t(rows) * size_t(D) * sizeof(float), IQ_ERR_WORKSPACE);
  AVArgs a{(const uint16_t*)p, sp_b, sp_h, v_codes, v_meta, t_cap / group, Hkv, t0 / group, ngroups, gpw, ws, Hq};
  int st = dispatch_shape(bits, group, D, Hq / Hkv, mode == IQ_MODE_SYM, [&]<int BITS, int G, int DD, int R, bool S>() {
    av_kernel<BITS, G, DD, R, S><<<dim3(nsplit, B * Hkv), WG, 0, stream>>>(a);
    return launch_status();
  });
  if (st) return st;
  av_combine_kernel<<<dim3(unsigned(ceil_div(rows * D, 256))), 256, 0, stream>>>(ws, nsplit, Hq, D, rows, o,
                                                                                  accumulate);
  return launch_status();
}

}  // namespace

// =============================================================================
// C ABI
// =============================================================================
extern "C" {

int iq_qk_gemv(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const uint32_t* k_codes,
               const uint16_t* k_meta, int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group,
               int bits, int mode, float scale, float* out, int64_t so_b, int64_t so_h, void* stream) {
  if (int e = check_qk(q, k_codes, k_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, out)) return e;
  IQ_CHECK(aligned(q, 2), IQ_ERR_ALIGN);
  return launch_qk(q, sq_b, sq_h, norm, k_codes, k_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, scale, out,
                   so_b, so_h, (hipStream_t)stream);
}

size_t iq_av_workspace_bytes(int B, int Hq, int T, int D, int group) {
  if (B <= 0 || Hq <= 0 || T <= 0 || !group_ok(group) || !d_ok(D)) return 0;
  // bound over every Hkv dividing Hq (smaller B*Hkv -> more splits)
  size_t best = 0;
  for (int hkv = 1; hkv <= Hq; ++hkv)
    if (Hq % hkv == 0) best = std::max(best, av_ws_bytes(B, Hq, T, D, group, hkv));
  return best;
}

int iq_av_gemv(const void* p, int64_t sp_b, int64_t sp_h, const uint32_t* v_codes, const uint16_t* v_meta,
               int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode,
               float* out32, void* out16, int64_t so_b, int64_t so_h, int accumulate, void* workspace,
               size_t workspace_bytes, void* stream) {
  if (int e = check_av(p, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode)) return e;
  IQ_CHECK(out32 || out16, IQ_ERR_NULL);
  IQ_CHECK(!accumulate || out32, IQ_ERR_NULL);
  IQ_CHECK(T > 0 || accumulate, IQ_ERR_SHAPE);
  const OutPair o{out32, so_b, so_h, (uint16_t*)out16, so_b, so_h};
  return launch_av(p, sp_b, sp_h, v_codes, v_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, o, accumulate,
                   (float*)workspace, workspace_bytes, (hipStream_t)stream);
}

size_t iq_decode_workspace_bytes(int B, int Hq, int T, int D) {
  if (B <= 0 || Hq <= 0 || T <= 0 || !d_ok(D)) return 0;
  const size_t rows = size_t(B) * Hq;
  size_t logits = rows * T * sizeof(float);
  size_t p = ((rows * T * sizeof(uint16_t)) + 255) & ~size_t(255);
  size_t out32 = rows * D * sizeof(float);
  size_t av = 0;
  for (int g : {32, 64, 128}) av = std::max(av, iq_av_workspace_bytes(B, Hq, T, D, g));
  return ((logits + 255) & ~size_t(255)) + p + ((out32 + 255) & ~size_t(255)) + av;
}

int iq_decode_attention(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const iq_segment* k,
                        const iq_segment* v, int B, int Hq, int Hkv, int T, int D, float scale, void* out,
                        int64_t so_b, int64_t so_h, void* workspace, size_t workspace_bytes, void* stream) {
  IQ_CHECK(q && k && v && out, IQ_ERR_NULL);
  IQ_CHECK(B >= 0 && T > 0 && Hkv > 0 && Hq > 0, IQ_ERR_SHAPE);
  IQ_CHECK(d_ok(D) && Hq % Hkv == 0 && nrep_ok(Hq / Hkv), IQ_ERR_SHAPE);
  IQ_CHECK(k[0].n >= 0 && k[1].n >= 0 && k[2].n >= 0 && v[0].n >= 0 && v[1].n >= 0 && v[2].n >= 0, IQ_ERR_SHAPE);
  IQ_CHECK(k[0].n + k[1].n + k[2].n == T && v[0].n + v[1].n + v[2].n == T, IQ_ERR_SHAPE);
  for (int s : {0, 2}) {
    IQ_CHECK(k[s].n == 0 || k[s].dense, IQ_ERR_NULL);
    IQ_CHECK(v[s].n == 0 || v[s].dense, IQ_ERR_NULL);
  }
  if (k[1].n) {
    if (int e = check_qk(q, k[1].codes, k[1].meta, k[1].t_cap, B, Hq, Hkv, k[1].t0, k[1].n, D, k[1].group,
                         k[1].bits, k[1].mode, (const float*)workspace))
      return e;
  }
  if (v[1].n) {
    if (int e = check_av(q, v[1].codes, v[1].meta, v[1].t_cap, B, Hq, Hkv, v[1].t0, v[1].n, D, v[1].group,
                         v[1].bits, v[1].mode))
      return e;
  }
  const size_t need = iq_decode_workspace_bytes(B, Hq, T, D);
  IQ_CHECK(workspace && workspace_bytes >= need, IQ_ERR_WORKSPACE);
  if (B == 0) return IQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const size_t rows = size_t(B) * Hq;
  char* ws = (char*)workspace;
  float* logits = (float*)ws;
  ws += (rows * T * sizeof(float) + 255) & ~size_t(255);
  uint16_t* p = (uint16_t*)ws;
  ws += (rows * T * sizeof(uint16_t) + 255) & ~size_t(255);
  float* out32 = (float*)ws;
  ws += (rows * D * sizeof(float) + 255) & ~size_t(255);
  float* avws = (float*)ws;
  const size_t avws_bytes = workspace_bytes - size_t(ws - (char*)workspace);
  const int64_t lb = int64_t(Hq) * T, lh = T;

  // 1) logits: sink | quantized | recent
  int tk = 0;
  for (int s = 0; s < 3; ++s) {
    const iq_segment& g = k[s];
    if (g.n == 0) continue;
    if (s == 1) {
      int e = launch_qk(q, sq_b, sq_h, norm, g.codes, g.meta, g.t_cap, B, Hq, Hkv, g.t0, g.n, D, g.group, g.bits,
                        g.mode, scale, logits + tk, lb, lh, st);
      if (e) return e;
    } else {
      const int64_t n = int64_t(B) * Hq * g.n;
      dense_qk_kernel<<<dim3(unsigned(ceil_div(n, 256))), 256, 0, st>>>(
          (const uint16_t*)q, sq_b, sq_h, (const uint16_t*)g.dense, g.s_b, g.s_h, g.s_t, B, Hq, Hkv, g.n, D, scale,
          logits, lb, lh, tk);
      if (int e = launch_status()) return e;
    }
    tk += g.n;
  }
  // 2) p = fp16(softmax_fp32(logits))
  softmax_kernel<<<dim3(unsigned(rows)), 256, 0, st>>>(logits, T, p);
  if (int e = launch_status()) return e;
  // 3) fp16 V segments -> out32, then the quantized V segment accumulates and writes fp16 out
  DenseSeg s0{(const uint16_t*)v[0].dense, v[0].s_b, v[0].s_h, v[0].s_t, v[0].n, 0};
  DenseSeg s2{(const uint16_t*)v[2].dense, v[2].s_b, v[2].s_h, v[2].s_t, v[2].n, v[0].n + v[1].n};
  dense_av_kernel<<<dim3(unsigned(ceil_div(int64_t(rows) * D, 256))), 256, 0, st>>>(
      p, lb, lh, s0, s2, B, Hq, Hkv, D, out32, int64_t(Hq) * D, D);
  if (int e = launch_status()) return e;
  const iq_segment& g = v[1];
  const OutPair o{out32, int64_t(Hq) * D, D, (uint16_t*)out, so_b, so_h};
  if (g.n) {
    return launch_av(p + v[0].n, lb, lh, g.codes, g.meta, g.t_cap, B, Hq, Hkv, g.t0, g.n, D, g.group, g.bits, g.mode,
                     o, 1, avws, avws_bytes, st);
  }
  av_combine_kernel<<<dim3(unsigned(ceil_div(int64_t(rows) * D, 256))), 256, 0, st>>>(avws, 0, Hq, D,
                                                                                     int64_t(rows), o, 1);
  return launch_status();
}

}  // extern "C"
