// Cache-side helpers of the drop-in layer (gfx950): the key normalization
// factor and the hybrid (asym / sym per group) selection.  Both run once per
// prefill or flush, never in the decode GEMVs.
#include "iq_common.h"
#include "iq_device.h"

using namespace iq;

namespace {

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// out[bh, d] = fp16(sqrt(max_t |k[bh, t, d]|)): cache.py:121-126 computes
// key_states.abs().max(dim=-2).values.sqrt() in the activation dtype, i.e.
// the correctly rounded fp32 square root of an fp16 (bf16) value, rounded to
// fp16 (bf16).
__global__ __launch_bounds__(256) void key_norm_kernel(const uint16_t* __restrict__ k, int64_t skb, int64_t skh,
                                                       int64_t skt, int H, int T, int D, int64_t n, int bf,
                                                       uint16_t* __restrict__ out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int d = int(i % D);
  const int64_t bh = i / D;
  const uint16_t* p = k + (bh / H) * skb + (bh % H) * skh + d;
  uint32_t mx = 0u;  // |x| as its bit pattern (below): a NaN propagates
  for (int t = 0; t < T; ++t) mx = max(mx, uint32_t(p[int64_t(t) * skt] & 0x7fffu));
  out[i] = f2act(__fsqrt_rn(act2f(uint16_t(mx), bf != 0)), bf != 0);
}

// The same factor for head_dim 64 and 128 (the prompt lengths of a prefill):
// one 1024-thread workgroup per (batch, head); thread (token lane tl,
// 8-channel group cg) reads 16 bytes of every TL-th row, so a wave reads
// whole rows.  |x| of fp16 and bf16 values orders like its bit pattern with
// the sign bit cleared (a NaN above every number, as torch's max propagates
// it), so the maximum is a packed 16-bit integer max, exact in any order;
// the token lanes' maxima meet in LDS.  One thread per channel walked the
// tokens one row at a time: 13.2 ms for a 32k-token prompt of 8 x 8 heads.
template <int D>
__global__ __launch_bounds__(1024) void key_norm_rows_kernel(const uint16_t* __restrict__ k, int64_t skb,
                                                             int64_t skh, int64_t skt, int H, int T, int bf,
                                                             int vec, uint16_t* __restrict__ out) {
  constexpr int CG = D / 8, TL = 1024 / CG;
  __shared__ uint4 red[TL][CG];
  const int bh = blockIdx.x, tid = threadIdx.x, cg = tid % CG, tl = tid / CG;
  const uint16_t* p = k + int64_t(bh / H) * skb + int64_t(bh % H) * skh + cg * 8;
  uint32_t m[4] = {0u, 0u, 0u, 0u};  // |x| bit patterns, two channels per dword
  auto fold = [&](const uint32_t (&w)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = w[j] & 0x7fff7fffu;
      m[j] = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, m[j]),
                                                                     __builtin_bit_cast(u16x2_t, a)));
    }
  };
  if (vec) {
    int t = tl;
    for (; t + 3 * TL < T; t += 4 * TL) {  // four rows in flight per thread
      uint4 r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = *reinterpret_cast<const uint4*>(p + int64_t(t + u * TL) * skt);
#pragma unroll
      for (int u = 0; u < 4; ++u) fold({r[u].x, r[u].y, r[u].z, r[u].w});
    }
    for (; t < T; t += TL) {
      const uint4 r = *reinterpret_cast<const uint4*>(p + int64_t(t) * skt);
      fold({r.x, r.y, r.z, r.w});
    }
  } else {
    for (int t = tl; t < T; t += TL) {
      const uint16_t* q = p + int64_t(t) * skt;
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = uint32_t(q[2 * j]) | (uint32_t(q[2 * j + 1]) << 16);
      fold(w);
    }
  }
  red[tl][cg] = make_uint4(m[0], m[1], m[2], m[3]);
  __syncthreads();
  if (tid < D) {  // channel d = tid: its token lanes' maxima
    const int c = tid / 8, j = (tid % 8) / 2, hi = tid % 2;
    uint32_t mx = 0u;
    for (int r = 0; r < TL; ++r) {
      const uint4 v = red[r][c];
      const uint32_t w = j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
      mx = max(mx, hi ? w >> 16 : w & 0xffffu);
    }
    out[int64_t(bh) * D + tid] = f2act(__fsqrt_rn(act2f(uint16_t(mx), bf != 0)), bf != 0);
  }
}

// Hybrid selection mask (quant.py:133-151): per group, the L1 error of the
// asym dequantization exceeds that of the sym one.  x fp16 [BH, T, D] (the
// quantizer's input; divided by norm [BH, D] in fp16 first when given, as
// the quantizer does), deq_a / deq_s fp32 [BH, T, D] contiguous.  Groups along D
// (axis 0, mask [BH, T, D/G]) or along T (axis 1, mask [BH, T/G, D]).  The
// differences are fp32 like the reference's; the sums are accumulated in
// fp64, which the oracle uses and which reproduced the reference's traces.
__global__ __launch_bounds__(256) void hybrid_mask_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ norm,
                                                          const float* __restrict__ da, const float* __restrict__ ds,
                                                          int T, int D, int group, int axis, int64_t n, int bf,
                                                          uint8_t* __restrict__ mask) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t bh, e0, step;
  int dcol;  // a column of the group (for the norm)
  if (axis == 0) {
    const int ng = D / group;
    const int64_t row = i / ng;  // bh * T + t
    const int g = int(i % ng);
    bh = row / T;
    e0 = row * D + int64_t(g) * group;
    step = 1;
    dcol = g * group;
  } else {
    const int d = int(i % D);
    const int64_t r = i / D;  // bh * (T / G) + gi
    const int ngT = T / group;
    bh = r / ngT;
    e0 = (bh * T + (r % ngT) * group) * D + d;
    step = D;
    dcol = d;
  }
  double ea = 0.0, es = 0.0;
  for (int j = 0; j < group; ++j) {
    const int64_t e = e0 + j * step;
    float v = act2f(x[e], bf != 0);
    if (norm) v = round_act(v / act2f(norm[bh * D + dcol + (axis == 0 ? j : 0)], bf != 0), bf != 0);
    ea += double(fabsf(__fsub_rn(da[e], v)));
    es += double(fabsf(__fsub_rn(ds[e], v)));
  }
  mask[i] = ea > es ? 1 : 0;
}

// out = mask ? deq_s : deq_a (quant.py:153-176 dequantize_hybrid), fp32, fp16
// (out_f16 = 1) or bf16 (out_f16 = 2).
__global__ __launch_bounds__(256) void hybrid_select_kernel(const float* __restrict__ da,
                                                            const float* __restrict__ ds,
                                                            const uint8_t* __restrict__ mask, int T, int D,
                                                            int group, int axis, int64_t n, int out_f16,
                                                            void* __restrict__ out) {
  const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int d = int(e % D);
  const int64_t row = e / D;  // bh * T + t
  int64_t mi;
  if (axis == 0) {
    mi = row * (D / group) + d / group;
  } else {
    const int64_t bh = row / T;
    const int t = int(row % T);
    mi = (bh * (T / group) + t / group) * D + d;
  }
  const float v = mask[mi] ? ds[e] : da[e];
  if (out_f16) static_cast<uint16_t*>(out)[e] = f2act(v, out_f16 == 2);
  else static_cast<float*>(out)[e] = v;
}

int check_hybrid(int64_t BH, int T, int D, int group, int axis) {
  IQ_CHECK(BH >= 0 && T >= 0 && D > 0, IQ_ERR_SHAPE);
  IQ_CHECK(group > 0 && (axis == 0 || axis == 1), IQ_ERR_SHAPE);
  IQ_CHECK(axis == 0 ? D % group == 0 : T % group == 0, IQ_ERR_GROUP);
  return IQ_OK;
}

}  // namespace

extern "C" {

int iq_key_norm_factor(const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_t, int B, int H, int T, int D,
                       int mode, void* out16, void* stream) {
  IQ_CHECK(k && out16, IQ_ERR_NULL);
  IQ_CHECK(base_mode(mode) == 0, IQ_ERR_MODE);  // only the dtype flag
  IQ_CHECK(B >= 0 && H >= 0 && T > 0 && D > 0, IQ_ERR_SHAPE);
  const int64_t n = int64_t(B) * H * D;
  if (n == 0) return IQ_OK;
  const int bf = act_bf16(mode) ? 1 : 0;
  if (D == 64 || D == 128) {
    // 16-byte row loads where every row's channels start 16-byte aligned
    const int vec = aligned(k, 16) && sk_b % 8 == 0 && sk_h % 8 == 0 && sk_t % 8 == 0;
    const dim3 grid{unsigned(int64_t(B) * H)};
    if (D == 128)
      key_norm_rows_kernel<128><<<grid, 1024, 0, (hipStream_t)stream>>>((const uint16_t*)k, sk_b, sk_h, sk_t, H, T,
                                                                         bf, vec, (uint16_t*)out16);
    else
      key_norm_rows_kernel<64><<<grid, 1024, 0, (hipStream_t)stream>>>((const uint16_t*)k, sk_b, sk_h, sk_t, H, T,
                                                                        bf, vec, (uint16_t*)out16);
    return launch_status();
  }
  key_norm_kernel<<<dim3(unsigned(ceil_div(n, 256))), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)k, sk_b, sk_h, sk_t, H, T, D, n, bf, (uint16_t*)out16);
  return launch_status();
}

int iq_hybrid_mask(const void* x16, const void* norm16, const float* deq_a, const float* deq_s, int64_t BH, int T,
                   int D, int group, int axis, int mode, uint8_t* mask, void* stream) {
  IQ_CHECK(x16 && deq_a && deq_s && mask, IQ_ERR_NULL);
  IQ_CHECK(base_mode(mode) == 0, IQ_ERR_MODE);  // only the dtype flag
  if (int e = check_hybrid(BH, T, D, group, axis)) return e;
  const int64_t n = axis == 0 ? BH * T * (D / group) : BH * (T / group) * D;
  if (n == 0) return IQ_OK;
  hybrid_mask_kernel<<<dim3(unsigned(ceil_div(n, 256))), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x16, (const uint16_t*)norm16, deq_a, deq_s, T, D, group, axis, n, act_bf16(mode) ? 1 : 0, mask);
  return launch_status();
}

int iq_hybrid_select(const float* deq_a, const float* deq_s, const uint8_t* mask, int64_t BH, int T, int D, int group,
                     int axis, int out_f16, void* out, void* stream) {
  IQ_CHECK(deq_a && deq_s && mask && out, IQ_ERR_NULL);
  IQ_CHECK(out_f16 >= 0 && out_f16 <= 2, IQ_ERR_SHAPE);
  if (int e = check_hybrid(BH, T, D, group, axis)) return e;
  const int64_t n = BH * T * int64_t(D);
  if (n == 0) return IQ_OK;
  hybrid_select_kernel<<<dim3(unsigned(ceil_div(n, 256))), 256, 0, (hipStream_t)stream>>>(
      deq_a, deq_s, mask, T, D, group, axis, n, out_f16, out);
  return launch_status();
}

}  // extern "C"
