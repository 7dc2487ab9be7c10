// Decode QK^T GEMV over a packed K store (gfx950).
//
// logit[b, h, t] = scale * sum_g ( s[t,g] * sum_{i in g} q'[h,i] c[t,i] + z[t,g] * sum_{i in g} q'[h,i] )
//
// Mapping: one wave64 owns QK_BPW consecutive 64-token blocks of one
// (batch, KV head); lane = token.  The wave walks the head_dim groups; for
// group g it holds the code words and {scale, zero} dword of its blocks (the
// K store keeps a block's 64 tokens contiguous per group, so every load is a
// 1 KiB coalesced wave access for 4-bit G=32) while group g+1's are in
// flight.  The n_rep query heads sharing the KV head use the same unpacked
// codes: each group is eight v_mfma_f32_4x4x4f16 per four heads, B = four
// unpacked codes of the lane's token, A = four query values of head
// 4q + lane%4 from the query operand record (iq_gemv.h), so the VALU only
// unpacks codes and applies scale and zero point.  A workgroup (four waves)
// covers one split of 4*QK_BPW*64 tokens.
//
// Epilogue, chosen per launch:
//   logits  write scale * logit (fp32) for every token;
//   flash   softmax within the split (flash decoding): the workgroup's max m
//           and sum l of exp(logit - m) per head go to (m, l) statistics, and
//           the probabilities exp(logit - m), rounded to fp16, are written
//           straight into attn.V operand records for the V store's unpack
//           plan, so no logits or probabilities round-trip through HBM.
#include "iq_flash.h"

using namespace iq;

namespace {

constexpr int QK_BPW = IQ_FLASH_BPW;
constexpr int SPLIT = NWAVES * QK_BPW * TOKEN_BLOCK;  // tokens per workgroup

// one thread per (b, kvh, g, h): query pairs in plan order (hi/lo with a key
// normalization folded in, cache.py:128-133) and their sum
template <int BITS, int G, int NREP>
__global__ __launch_bounds__(256) void qk_record_kernel(const uint16_t* __restrict__ q, int64_t sqb, int64_t sqh,
                                                        const uint16_t* __restrict__ norm, int B, int Hkv, int D,
                                                        uint32_t* __restrict__ rec) {
  constexpr int NP = G / 2;
  constexpr int RD = qrec_dwords<G, NREP>();
  constexpr PairTable<BITS, NP> PT{};
  const int ng = D / G;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(B) * Hkv * ng * NREP) return;
  const int h = int(i % NREP);
  const int g = int((i / NREP) % ng);
  const int64_t bh = i / (int64_t(NREP) * ng);
  const int b = int(bh / Hkv), kvh = int(bh % Hkv);
  const uint16_t* qr = q + b * sqb + (kvh * NREP + h) * sqh + g * G;
  const uint16_t* nr = norm ? norm + bh * D + g * G : nullptr;
  uint32_t* r = rec + (bh * ng + g) * RD;
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < NP; ++k) qrec_pair(qr, nr, PT.a[k], PT.c[k], &r[h * NP + k], &r[(NREP + h) * NP + k], sum);
  r[qrec_osum<G, NREP>() + h] = __float_as_uint(sum);
}

struct QKArgs {
  const uint32_t* rec;
  const uint32_t* kc;
  const uint16_t* km;
  int64_t cap_blocks;
  int Hkv, blk0, T, nblk;
  float scale;
  int split;   // hi/lo query rows
  float* out;  // logits epilogue
  int64_t sob, soh;
  int flash;   // flash epilogue
  detail::FlashOut f;
  int ngv;     // V groups covered by the records (T / vgroup)
};

template <int NREP>
struct FlashSmem {
  float m[NWAVES][NREP];
  float l[NWAVES][NREP];
  uint16_t p[NREP][SPLIT];
};

template <int BITS, int G, int D, int NREP, bool SYM>
__global__ __launch_bounds__(WG) void qk_kernel(QKArgs a) {
  constexpr int NG = D / G;
  constexpr int W = G * BITS / 32;
  constexpr int NP = G / 2;
  constexpr int M = SYM ? 1 : 2;
  constexpr int RD = qrec_dwords<G, NREP>();
  constexpr int BPW = QK_BPW;
  __shared__ FlashSmem<NREP> sm;

  const int bh = blockIdx.y;
  const int b = bh / a.Hkv, kvh = bh % a.Hkv;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wblk = (blockIdx.x * NWAVES + wave) * BPW;
  if (wblk >= a.nblk && !a.flash) return;  // the flash epilogue needs every wave at its barriers
  const int nb = max(0, min(BPW, a.nblk - wblk));

  const int64_t blkbase = int64_t(bh) * a.cap_blocks + a.blk0;
  const uint32_t* kcb = a.kc + blkbase * (NG * TOKEN_BLOCK * W);
  const uint16_t* kmb = a.km + blkbase * (NG * TOKEN_BLOCK * M);

  // words of group g for the wave's blocks; the next group's are prefetched
  uint32_t w[BPW][W];
  uint32_t m[BPW];
  // Blocks past the end of the range (tail waves) re-read the range's last
  // block: in-bounds loads whose results are masked out, and no branches.
  auto load = [&](int g) {
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int blk = min(wblk + j, a.nblk - 1);
      const int64_t unit = (int64_t(blk) * NG + g) * TOKEN_BLOCK + lane;
      load_words<W>(kcb + unit * W, w[j]);
      if constexpr (SYM) m[j] = kmb[unit];
      else m[j] = reinterpret_cast<const uint32_t*>(kmb)[unit];
    }
  };
  load(0);

  const cptr_u32 recb = (cptr_u32)(a.rec) + int64_t(bh) * NG * RD;
  float acc[BPW][NREP];
#pragma unroll
  for (int j = 0; j < BPW; ++j)
#pragma unroll
    for (int h = 0; h < NREP; ++h) acc[j][h] = 0.f;

  const PlanRegs<BITS> pr;
  // A runtime loop: each group's operand records are loaded inside its own
  // iteration, so at most one chunk of them occupies SGPRs.
#pragma unroll 1
  for (int g = 0; g < NG; ++g) {
    uint32_t cw[BPW][W];
    uint32_t cm[BPW];
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      cm[j] = m[j];
#pragma unroll
      for (int x = 0; x < W; ++x) cw[j][x] = w[j][x];
    }
    if (g + 1 < NG) load(g + 1);
    const cptr_u32 rec = recb + g * RD;
    float d[BPW][NREP];
    qk_group_dot<BITS, G, NREP, BPW>(cw, a.rec + (int64_t(bh) * NG + g) * RD, lane & 3, a.split, pr, d);
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const float s = h2f(uint16_t(cm[j] & 0xffffu));
      const float z = SYM ? -float(1 << (BITS - 1)) * s : h2f(uint16_t(cm[j] >> 16));
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        const float qs = rec_f32(rec, qrec_osum<G, NREP>() + h);
        acc[j][h] = fmaf(s, d[j][h], fmaf(z, qs, acc[j][h]));
      }
    }
  }

  if (!a.flash) {
    float* outb = a.out + int64_t(b) * a.sob + int64_t(kvh * NREP) * a.soh;
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int t = (wblk + j) * TOKEN_BLOCK + lane;
      if (j < nb && t < a.T) {
#pragma unroll
        for (int h = 0; h < NREP; ++h) outb[h * a.soh + t] = acc[j][h] * a.scale;
      }
    }
    return;
  }

  // ---- flash epilogue: softmax statistics of this split + attn.V records ----
  float lg[BPW][NREP];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int t = (wblk + j) * TOKEN_BLOCK + lane;
#pragma unroll
    for (int h = 0; h < NREP; ++h) lg[j][h] = (j < nb && t < a.T) ? acc[j][h] * a.scale : -INFINITY;
  }
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    float mx = lg[0][h];
#pragma unroll
    for (int j = 1; j < BPW; ++j) mx = fmaxf(mx, lg[j][h]);
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
    for (int j = 0; j < BPW; ++j) {
      const float p = lg[j][h] == -INFINITY ? 0.f : __expf(lg[j][h] - mh[h]);
      ls += p;
      sm.p[h][(wave * BPW + j) * TOKEN_BLOCK + lane] = __half_as_ushort(__float2half_rn(p));
    }
    ls = wave_sum(ls);
    if (lane == 0) sm.l[wave][h] = ls;
  }
  __syncthreads();
  const int split = blockIdx.x;
  const int64_t rows = int64_t(gridDim.y) * NREP;
  if (threadIdx.x < NREP) {
    const int h = threadIdx.x;
    float* dst = a.f.ml + (int64_t(split) * rows + int64_t(bh) * NREP + h) * 2;
    dst[0] = mh[h];
    dst[1] = (sm.l[0][h] + sm.l[1][h]) + (sm.l[2][h] + sm.l[3][h]);
  }
  // records: one thread per (V group of this split, head)
  const int vg = a.f.vgroup, vnp = vg / 2, vrd = rec_dwords_rt(vg, NREP);
  const int gps = SPLIT / vg;
  for (int i = threadIdx.x; i < gps * NREP; i += WG) {
    const int gl = i / NREP, h = i % NREP;
    const int gabs = split * gps + gl;
    if (gabs >= a.ngv) continue;
    uint32_t* r = a.f.vrec + (int64_t(bh) * a.ngv + gabs) * vrd;
    const uint16_t* pp = &sm.p[h][gl * vg];
    float sum = 0.f;
    for (int k = 0; k < vnp; ++k) {
      int ia, ic;
      plan_pair(a.f.vbits, k, ia, ic);
      const uint16_t ua = pp[ia], uc = pp[ic];
      r[h * vnp + k] = uint32_t(ua) | (uint32_t(uc) << 16);
      sum += h2f(ua) + h2f(uc);
    }
    r[vnp * NREP + h] = __float_as_uint(sum);
  }
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
  IQ_CHECK(aligned(k_codes, 16) && aligned(k_meta, 4) && aligned(q, 2), IQ_ERR_ALIGN);
  return IQ_OK;
}

int launch(const QKArgs& a, int B, int Hq, int Hkv, int D, int group, int bits, int mode, hipStream_t stream) {
  const int wgx = int(ceil_div(a.nblk, int64_t(QK_BPW) * NWAVES));
  return dispatch_shape(bits, group, D, Hq / Hkv, mode == IQ_MODE_SYM, [&]<int BITS, int G, int DD, int R, bool S>() {
    qk_kernel<BITS, G, DD, R, S><<<dim3(wgx, B * Hkv), WG, 0, stream>>>(a);
    return launch_status();
  });
}

}  // namespace

namespace iq::detail {

int device_index() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) dev = 0;
  return dev;
}

// CU count per device (MI355X: 256), read once per device
std::atomic<int> g_num_cus[MAX_DEVICES];
int num_cus() {
  const int dev = device_index();
  int n = g_num_cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_num_cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int flash_split_tokens() { return SPLIT; }

size_t qk_record_bytes(int B, int Hq, int D) {
  // largest record set over the supported groups: D/G records per n_rep query
  // heads, at most G + 3 dwords per head (pairs, osum, nbsum) and 9 of
  // alignment padding per record
  size_t best = 0;
  for (int g : {32, 64, 128})
    if (D % g == 0) best = std::max(best, size_t(B) * Hq * (D / g) * size_t(g + 12) * 4);
  return (best + 255) & ~size_t(255);
}

int qk_record_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, int B, int Hq, int Hkv, int D,
                     int group, int bits, uint32_t* rec, hipStream_t stream) {
  const int64_t n = int64_t(B) * Hq * (D / group);
  if (n == 0) return IQ_OK;
  return dispatch_rec(bits, group, Hq / Hkv, [&]<int BITS, int G, int R>() {
    qk_record_kernel<BITS, G, R><<<dim3(unsigned(ceil_div(n, 256))), 256, 0, stream>>>(
        (const uint16_t*)q, sq_b, sq_h, (const uint16_t*)norm, B, Hkv, D, rec);
    return launch_status();
  });
}

int qk_main_launch(const uint32_t* rec, int split, const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap,
                   int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float scale, float* out,
                   int64_t so_b, int64_t so_h, hipStream_t stream) {
  if (B == 0 || T == 0) return IQ_OK;
  QKArgs a{};
  a.rec = rec; a.split = split; a.kc = k_codes; a.km = k_meta; a.cap_blocks = t_cap / TOKEN_BLOCK; a.Hkv = Hkv;
  a.blk0 = t0 / TOKEN_BLOCK; a.T = T; a.nblk = int(ceil_div(T, TOKEN_BLOCK)); a.scale = scale;
  a.out = out; a.sob = so_b; a.soh = so_h; a.flash = 0;
  return launch(a, B, Hq, Hkv, D, group, bits, mode, stream);
}

int qk_flash_launch(const uint32_t* rec, int split, const uint32_t* k_codes, const uint16_t* k_meta, int64_t t_cap,
                    int B, int Hq, int Hkv, int t0, int T, int D, int group, int bits, int mode, float scale,
                    const FlashOut& f, hipStream_t stream) {
  if (B == 0 || T == 0) return IQ_OK;
  if (SPLIT % f.vgroup || T % f.vgroup) return IQ_ERR_GROUP;
  QKArgs a{};
  a.rec = rec; a.split = split; a.kc = k_codes; a.km = k_meta; a.cap_blocks = t_cap / TOKEN_BLOCK; a.Hkv = Hkv;
  a.blk0 = t0 / TOKEN_BLOCK; a.T = T; a.nblk = int(ceil_div(T, TOKEN_BLOCK)); a.scale = scale;
  a.flash = 1; a.f = f; a.ngv = T / f.vgroup;
  return launch(a, B, Hq, Hkv, D, group, bits, mode, stream);
}

}  // namespace iq::detail

namespace {

// QK^T through the persistent fused kernel in QK^T-only mode (query records
// built in LDS by each workgroup, no record kernel); returns 1 if launched, 0
// if a slice exceeds its 32-bit buffer offsets
int qk_fused_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const uint32_t* k_codes,
                    const uint16_t* k_meta, int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group,
                    int bits, int mode, float scale, float* out, int64_t so_b, int64_t so_h, hipStream_t stream,
                    int* status) {
  const int nrep = Hq / Hkv;
  const int64_t lim = int64_t(1) << 31;
  if (sq_h < 0 || (int64_t(nrep - 1) * sq_h + D) * 2 >= lim || t_cap * D * bits / 8 >= lim ||
      t_cap * D * 4 / group >= lim)
    return 0;
  detail::FusedArgs a{};
  a.q = (const uint16_t*)q; a.sqb = sq_b; a.sqh = sq_h; a.norm = (const uint16_t*)norm;
  a.kc = k_codes; a.km = k_meta; a.k_cap_blocks = t_cap / TOKEN_BLOCK; a.kblk0 = t0 / TOKEN_BLOCK;
  a.ksym = mode == IQ_MODE_SYM;
  a.Hkv = Hkv; a.T = T;
  a.nsplit = int(ceil_div(T, FSPLIT));
  a.nitems = a.nsplit * B * Hkv;
  const int64_t nblk = ceil_div(T, TOKEN_BLOCK);
  a.k_code_bytes = uint32_t(nblk * TOKEN_BLOCK * D * bits / 8);
  a.k_meta_bytes = uint32_t(nblk * TOKEN_BLOCK * (D / group) * (a.ksym ? 2 : 4));
  a.q_bytes = uint32_t((int64_t(nrep - 1) * sq_h + D) * 2);
  a.norm_bytes = norm ? uint32_t(D * 2) : 0u;
  a.scale_log2 = scale;  // QK^T only: the plain scale of the logits
  a.part = out; a.sob = so_b; a.soh = so_h;
  *status = dispatch_shape(bits, group, D, nrep, 0, [&]<int KB, int G, int DD, int R, bool S>() {
    auto* kern = norm ? flash_fused_kernel<KB, KB, G, DD, R, true, false, true>
                      : flash_fused_kernel<KB, KB, G, DD, R, false, false, true>;
    const int nt = norm ? FusedShape<G, R, true>::NT : FusedShape<G, R, false>::NT;
    static detail::OccCache occ[2];  // workgroups per CU at once
    const int pc = detail::blocks_per_cu(kern, nt, occ[norm ? 1 : 0]);
    const int grid = int(std::min<int64_t>(a.nitems, int64_t(pc) * detail::num_cus()));
    kern<<<dim3(grid), nt, 0, stream>>>(a);
    return launch_status();
  });
  return 1;
}

}  // namespace

extern "C" {

size_t iq_qk_workspace_bytes(int B, int Hq, int D) {
  if (B <= 0 || Hq <= 0 || !d_ok(D)) return 0;
  return detail::qk_record_bytes(B, Hq, D);
}

int iq_qk_gemv(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const uint32_t* k_codes,
               const uint16_t* k_meta, int64_t t_cap, int B, int Hq, int Hkv, int t0, int T, int D, int group,
               int bits, int mode, float scale, float* out, int64_t so_b, int64_t so_h, void* workspace,
               size_t workspace_bytes, void* stream) {
  if (int e = check_qk(q, k_codes, k_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, out)) return e;
  IQ_CHECK(workspace && workspace_bytes >= detail::qk_record_bytes(B, Hq, D), IQ_ERR_WORKSPACE);
  IQ_CHECK(aligned(workspace, 16), IQ_ERR_ALIGN);
  hipStream_t st = (hipStream_t)stream;
  if (B == 0 || T == 0) return IQ_OK;
  int status = IQ_OK;
  if (qk_fused_launch(q, sq_b, sq_h, norm, k_codes, k_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, scale, out,
                      so_b, so_h, st, &status))
    return status;
  uint32_t* rec = (uint32_t*)workspace;
  if (int e = detail::qk_record_launch(q, sq_b, sq_h, norm, B, Hq, Hkv, D, group, bits, rec, st)) return e;
  return detail::qk_main_launch(rec, norm != nullptr, k_codes, k_meta, t_cap, B, Hq, Hkv, t0, T, D, group, bits, mode, scale, out,
                                so_b, so_h, st);
}

}  // extern "C"
