// One decode step of attention over [sink | packed | recent] K and V (gfx950),
// flash-decoding style.
//
// The token axis is cut into
//   * the fused range: tokens packed in both the K and the V store (the
//     middle segment of cache.py:235-276 for both), in splits of
//     flash_split_tokens() tokens.  When K and V share their group size (bit
//     widths may differ), one persistent kernel runs QK^T, the softmax and
//     attn.V over every split (iq_flash.h) and writes one partial per run of
//     splits.  Otherwise QK^T runs with its flash epilogue (per split max m,
//     sum l and fp16 probabilities written as attn.V operand records), then
//     attn.V writes one unnormalized partial output per split;
//   * the dense tokens: everything else (fp16 sinks and recent windows, plus
//     packed tokens of only one of K/V, which are dequantized element by
//     element), in up to NSD_MAX slices, each an extra split: one workgroup
//     per (slice, batch, KV head) runs an online softmax over its tokens for
//     the KV head's query heads.
// A combine kernel rescales the splits by exp(m_s - max m) and divides by the
// total sum: softmax(q K^T * scale) V in fp32, written as fp16
// (TF/models/llama/modeling_llama.py:201-210).  The probabilities that meet V
// are rounded to fp16 as the reference rounds its softmax output.
#include <mutex>

#include "iq_gemv.h"

using namespace iq;

namespace {

constexpr int DT = 64;        // dense tokens per chunk
constexpr int NSD_MAX = 4;    // split slots of the dense tokens, at most
constexpr int DSLICE = 32;    // dense tokens per split slot, at least
constexpr int MERGE_RUNS_MAX = 4;  // fused runs per (batch, KV head) the merging dense kernel preloads
// 256-thread sections of the merging dense kernel: three where the window
// holds packed rows (32 sinks, a 96-token recent window and the <= 31 packed
// keys short of a V group, 129-159 tokens that two sections take in two
// chunks each: 13.9 us against 15.2 us per call), two for fp16 windows of up
// to two chunks (configs 3 and 4: 7.5 us against 8.2 us); fp16 windows
// longer than that take three (merge_sections_dense)
// (bf16 layers: two, whose fp32 tiles fill the LDS; eight query heads per KV
// head: two, whose fp16 accumulators would not fit three sections' registers)
constexpr int merge_sections(bool pk, bool bf, int nrep) { return pk && !bf && nrep <= 4 ? 3 : 2; }
constexpr int merge_sections_dense(int n_dense, int nrep) { return nrep <= 4 && n_dense > 2 * DT ? 3 : 2; }

struct Seg {
  const uint16_t* dense;
  int64_t sb, sh, st;
  int n, start;  // token count, first token of the segment in the step
  int vec;       // dense rows 16-byte aligned (base and strides): vector loads
  const uint32_t* codes;
  const uint16_t* meta;
  int64_t t_cap;
  int t0, bits, group, mode;
  int gsh;            // log2(group)
  int64_t cap_groups;  // t_cap / group
};

// {scale, zero} of a packed unit from its meta (mw: the unit's dword, or
// its fp16 scale for sym) with value = u * s + z for its b-bit field u (exact
// in fp32: sym offset binary folds into z = -2^(b-1) s; a hybrid unit as its
// flag says)
// (bf: the halves hold bf16 values, a bf16 layer's store)
__device__ __forceinline__ void unit_sz(uint32_t mw, int mode, int bits, float& s, float& z, bool bf = false) {
  if (mode == IQ_MODE_SYM) {
    s = act2f(uint16_t(mw), bf);
    z = -float(1 << (bits - 1)) * s;
  } else if (mode == IQ_MODE_HYBRID) {
    s = hyb_scale(mw, bf);
    z = hyb_sym(mw) ? -float(1 << (bits - 1)) * s : act2f(uint16_t(mw >> 16), bf);
  } else {
    s = act2f(uint16_t(mw & 0xffffu), bf);
    z = act2f(uint16_t(mw >> 16), bf);
  }
}

typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
// c + a.x * b.x + a.y * b.y over two 16-bit pairs of the activation type
// (v_dot2_f32_f16 / v_dot2_f32_bf16: exact products, fp32 accumulation)
template <bool BF>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (BF)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2_t, a), __builtin_bit_cast(bf2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}
template <bool BF>
__device__ __forceinline__ uint32_t to_act(float x) {
  if constexpr (BF) return f2bf(x);
  else return __half_as_ushort(__float2half_rn(x));
}

__device__ __forceinline__ uint32_t unit_meta(const Seg& g, int64_t unit) {
  return g.mode == IQ_MODE_SYM ? uint32_t(g.meta[unit]) : reinterpret_cast<const uint32_t*>(g.meta)[unit];
}

// fp16 elements [d0, d0 + N) of token t's row (a K or V segment list), as N/2
// dwords; a token outside every dense segment gives zeros.  Dense rows load
// as 16-byte vectors where aligned.  Returns whether the token lies in the
// list's packed segment (its row is decoded by packed_to_lds instead).
template <int N>
__device__ __forceinline__ bool gather_row(const Seg* s, int64_t b, int64_t kvh, int t, int d0,
                                           uint32_t (&out)[N / 2]) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) out[i] = 0u;
  // The lane's segment, chosen by value: every segment's fields are read with
  // a constant index (uniform, scalar loads of the kernel arguments) and the
  // lane selects its row pointer; a per-lane pointer to the segment would turn
  // every field into a dependent load through memory.
  const uint16_t* row = nullptr;
  bool vec = false, packed = false;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const bool in = t >= s[i].start && t < s[i].start + s[i].n;
    if (in && s[i].dense) {
      row = s[i].dense + b * s[i].sb + kvh * s[i].sh + int64_t(t - s[i].start) * s[i].st + d0;
      vec = s[i].vec != 0;
    } else if (in) {
      packed = true;
    }
  }
  if (row) {
    if (vec) {
#pragma unroll
      for (int c = 0; c < N / 8; ++c) {
        const uint4 x = reinterpret_cast<const uint4*>(row)[c];
        out[4 * c] = x.x; out[4 * c + 1] = x.y; out[4 * c + 2] = x.z; out[4 * c + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < N / 2; ++j) out[j] = uint32_t(row[2 * j]) | (uint32_t(row[2 * j + 1]) << 16);
    }
  }
  return packed;
}

struct DenseArgs {
  const uint16_t* q;
  int64_t sqb, sqh;
  const uint16_t* norm;
  Seg k[3], v[3];
  int lo0, hi0, lo1, hi1;  // dense tokens: [lo0, hi0) and [lo1, hi1)
  int Hq, Hkv;
  float scale;
  float* ml;  // the dense split slots' statistics: slot s at ml + s * rows * 2
  float* o;   // and partial outputs: slot s at o + s * rows * D
  // merging instance (after the fused kernel): its run partials (slots
  // [0, nruns) of the workspace, ShareMap(fgrid, B * Hkv, fnsf, fpair_e0))
  // and the output, fp16 [B, Hq, D] at b * sob + hq * soh
  const float* fml;
  const float* fpart;
  int fgrid, fnsf, fpair_e0;
  uint16_t* out;
  int64_t sob, soh;
};

// ---- packed rows of a dense chunk (kernels with packed segments) ----
// Tokens in the quantized segment of a list (the middle one: sinks and recent
// windows are fp16) that fall in the dense range are dequantized into the
// chunk's fp16 tiles.  A chunk's rows form at most two runs of consecutive
// tokens (one per dense range).  Each thread decodes 32 consecutive fields of
// one unit straight from global memory into registers (the unit's `bits`
// words and its meta word, one round trip, then compile-time shifts): a
// 32-token piece of one V column (groups along tokens), or 32 columns of one
// K row (groups along head_dim), and writes their fp16 values into the tile.
// (Staging the units in LDS and decoding element by element from LDS was
// LDS-bound: 21 us for a 128-token window at the presets' shape.)

// fields i = 0..31 of the first BITS words of w: value u * s + z, as the
// reference computes it (exact u * s in fp32, one rounding of the sum)
template <int BITS>
__device__ __forceinline__ void decode32(const uint32_t (&w)[4], float s, float z, float (&out)[32]) {
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    constexpr uint32_t M = (1u << BITS) - 1u;
    const int bit = BITS * i, wi = bit >> 5, sh = bit & 31;
    uint32_t f = w[wi] >> sh;
    if (sh + BITS > 32) f |= w[wi + 1] << (32 - sh);
    out[i] = __fadd_rn(__fmul_rn(float(f & M), s), z);
  }
}

// the `bits` words of a unit's 32-field piece and the unit's meta word
struct Piece {
  uint32_t w[4];
  uint32_t m;
};
__device__ __forceinline__ void load_piece(const Seg& g, int64_t u, int piece, Piece& p) {
  const int W = (g.bits << g.gsh) >> 5;  // words per unit
  const uint32_t* wp = g.codes + u * W + piece * g.bits;
  p.w[0] = wp[0];
  p.w[1] = wp[1];
  p.w[2] = g.bits > 2 ? wp[2] : 0u;
  p.w[3] = g.bits > 3 ? wp[3] : 0u;
  p.m = unit_meta(g, u);
}
template <bool BF>
__device__ __forceinline__ void decode_piece(const Seg& g, const Piece& p, float (&out)[32]) {
  float s, z;
  unit_sz(p.m, g.mode, g.bits, s, z, BF);
  switch (g.bits) {
    case 2: decode32<2>(p.w, s, z, out); break;
    case 3: decode32<3>(p.w, s, z, out); break;
    default: decode32<4>(p.w, s, z, out); break;
  }
}

// one run of the chunk: rows [r0, r1) hold tokens base + r.  Decodes its
// packed rows into the tiles (row strides kld, vld in dwords; fp16 pairs, or
// fp32 values in a bf16 layer's tiles) and leaves the workgroup synchronized.  Run by
// 256 threads (a workgroup, or one section of a merging workgroup: ALLB,
// whose sections share the barrier, so all of them always take it).  A
// thread decodes K pieces (32 columns of a row), then V pieces (32 tokens of
// a column), one at a time: loading every piece of the thread first measured
// no faster and needed more registers than three sections of a merging
// workgroup hold.
template <int D, bool ALLB = false, bool BF = false>
__device__ __forceinline__ void packed_run(const Seg& K, const Seg& V, const uint16_t* norm, int64_t bh, int base,
                                           int r0, int r1, uint32_t* ktile, int kld, uint32_t* vtile, int vld) {
  constexpr int NC = D / 32;  // K pieces per row
  const int tid = int(threadIdx.x) & 255;
  // the run's packed rows per list: [ka, kb) and [va, vb)
  const int ka = max(r0, K.start - base), kb = K.dense ? ka : min(r1, K.start + K.n - base);
  const int va = max(r0, V.start - base), vb = V.dense ? va : min(r1, V.start + V.n - base);
  const bool kon = kb > ka, von = vb > va;
  if (!ALLB && !kon && !von) return;  // uniform
  const int kcnt = kon ? (kb - ka) * NC : 0;
  for (int it = tid; it < kcnt; it += 256) {
    const int r = ka + it / NC, c = it % NC;
    const int st = K.t0 + (base + r - K.start);  // the store token
    const int g = (32 * c) >> K.gsh, piece = ((32 * c) & (K.group - 1)) >> 5;
    const int64_t u = ((bh * (K.t_cap >> 6) + (st >> 6)) * (D >> K.gsh) + g) * TOKEN_BLOCK + (st & 63);
    Piece p;
    load_piece(K, u, piece, p);
    float v[32];
    decode_piece<BF>(K, p, v);
    if (norm) {  // the key normalization factor, times the dequantized value (cache.py:128-133)
      const uint32_t* nr = reinterpret_cast<const uint32_t*>(norm + bh * D + 32 * c);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t x = nr[j];
        v[2 * j] = __fmul_rn(v[2 * j], act2f(uint16_t(x), BF));
        v[2 * j + 1] = __fmul_rn(v[2 * j + 1], act2f(uint16_t(x >> 16), BF));
      }
    }
    if constexpr (BF) {  // fp32 tile: the dequantized values as they are
      uint32_t* dst = ktile + r * kld + 32 * c;
#pragma unroll
      for (int j = 0; j < 32; ++j) dst[j] = __float_as_uint(v[j]);
    } else {
      uint32_t* dst = ktile + r * kld + 16 * c;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        dst[j] = uint32_t(__half_as_ushort(__float2half_rn(v[2 * j]))) |
                 (uint32_t(__half_as_ushort(__float2half_rn(v[2 * j + 1]))) << 16);
    }
  }
  const int sa = V.t0 + (base + va - V.start), sb = sa + (vb - va);  // V store tokens [sa, sb)
  const int p0 = sa >> 5, vcnt = von ? (((sb + 31) >> 5) - p0) * D : 0;
  for (int it = tid; it < vcnt; it += 256) {
    const int pc = p0 + it / D, d = it % D;
    const int g = (32 * pc) >> V.gsh, piece = ((32 * pc) & (V.group - 1)) >> 5;
    Piece p;
    load_piece(V, (bh * V.cap_groups + g) * D + d, piece, p);
    float v[32];
    decode_piece<BF>(V, p, v);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int st = 32 * pc + j;
      if (st >= sa && st < sb) {
        if constexpr (BF) vtile[(va + st - sa) * vld + d] = __float_as_uint(v[j]);
        else reinterpret_cast<uint16_t*>(vtile)[(va + st - sa) * 2 * vld + d] = __half_as_ushort(__float2half_rn(v[j]));
      }
    }
  }
  __syncthreads();
}

// Online softmax over the dense tokens (fp16 sinks and recent windows, and
// tokens packed in only one of K and V).  Workgroup (s, b * Hkv + kvh) takes
// slice s of the dense tokens for the NREP query heads of KV head kvh, in
// chunks of DT tokens: the chunk's K and V rows are gathered as fp16 into
// LDS (the next chunk's rows are loaded into registers meanwhile); the logits
// come from the four waves' quarters of head_dim (lane = token, every head),
// wave w keeps the running (m, l) of heads w, w + 4, ..., and wave w
// accumulates the output of every head over a quarter of the chunk's tokens
// (lane = column pair), so a section reads its K and V tiles once per chunk
// (per query head, when a wave took one head: 7.45 -> 7.01 us per merging
// call at config 4's shape, 13.94 -> 13.33 us with packed rows, traced).  The
// probability that meets V is rounded to fp16, as the reference rounds its
// softmax output; logits, sums and outputs are fp32.
// MERGE (launched after the fused kernel, one workgroup of merge_sections
// 256-thread sections per (batch, KV head)): each section takes its share of
// the dense tokens as its slice, side by side, and the workgroup then merges
// the sections' states with the fused kernel's run partials of the head and
// writes the output, in place of the dense slots and the combine launch.
// BF: a bf16 layer (query, rows, factor, metadata and output in bf16).  Its
// tiles hold fp32 values (bf16 rows convert exactly, packed rows keep their
// fp32 dequantized values) and the logits and p.V are fp32 products with the
// unrounded probabilities: rounding the window's rows and probabilities to
// bf16 put a window-heavy step at 1.005e-3 of fp32 attention.  Its waves take
// one head each for the logits and thread (head, column pair) accumulates
// the output.
template <int D, int NREP, bool PK, bool MERGE = false, bool BF = false, int NS = merge_sections(PK, BF, NREP)>
__global__ __launch_bounds__(MERGE ? 256 * NS : 256) void dense_attn_kernel(DenseArgs a) {
  constexpr int NH = MERGE ? NS : 1;  // slices per workgroup (256-thread sections)
  constexpr int NTH = 256 * NH;
  constexpr int TW = BF ? D : D / 2;          // dwords of a row's values: fp32, or fp16 pairs
  constexpr int KS = TW + 1;                  // K tile row stride in dwords (odd: no bank conflicts)
  constexpr int VS = BF ? D + 2 : D / 2 + 1;  // V tile row stride (fp16: odd, the gather writes a row's
                                              // quarter per thread and at D / 2 the rows shared their
                                              // banks; fp32: even, for column-pair reads)
  constexpr int HPW = (NREP + 3) / 4;         // heads per wave
  constexpr int NPR = D / 2;                  // column pairs per head
  constexpr int OPT = (NREP * NPR + 255) / 256;  // (head, pair) items per thread
  constexpr int RE = D / 4;                   // row elements per gathering thread
  // fp16: each section reads its K and V tiles once, not once per query head.
  // For the logits wave w sums its quarter of head_dim (QW pair-dwords) for
  // every head, lane = token, and the quarters meet in LDS (lgp); for attn.V
  // wave w takes a quarter of the chunk's tokens for every head, lane =
  // (column pair, token subgroup), and the waves' partial outputs are summed
  // once, after the last chunk.
  constexpr int QW = TW / 4;
  constexpr int PPL = NPR < 64 ? NPR : 64;  // column pairs across a wave's lanes
  constexpr int TSUB = 64 / PPL;            // token subgroups of a wave (D = 64: two)
  constexpr int TPS = DT / 4 / TSUB;        // attn.V tokens per lane and chunk
  static_assert(BF || (QW % 4 == 0 && TSUB <= 2 && TPS % 2 == 0 && 4 * NREP * D <= DT * KS), "fp16 split");
  __shared__ uint32_t kts[NH][DT][KS];
  __shared__ __align__(8) uint32_t vts[NH][DT][VS];
  __shared__ __align__(16) uint32_t qs2[NREP][TW];  // the query heads' fp16 pairs (fp32 values: BF)
  __shared__ float lgps[BF ? 1 : NH][BF ? 1 : 4][BF ? 1 : NREP][BF ? 1 : DT];  // fp16: logits per head_dim quarter
  __shared__ __align__(4) uint16_t pss[NH][NREP][BF ? 2 * DT : DT];  // probabilities: fp16 (fp32: BF)
  __shared__ float als[NH][NREP];
  const int half = MERGE ? int(threadIdx.x >> 8) : 0;
  auto& kt = kts[half];
  auto& vt = vts[half];
  auto& ps = pss[half];
  float* psf = reinterpret_cast<float*>(&pss[half][0][0]);  // BF: [NREP][DT] fp32
  auto& al = als[half];
  auto& lgp = lgps[BF ? 0 : half];
  const int tid = int(threadIdx.x) & 255, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave within the section
  const int bh = blockIdx.y, b = bh / a.Hkv, kvh = bh % a.Hkv;
  const int n0 = a.hi0 - a.lo0, n = n0 + (a.hi1 - a.lo1);
  const int nsl = MERGE ? NH : int(gridDim.x), sl = MERGE ? half : int(blockIdx.x);  // slices, this one
  const int i0 = int(int64_t(sl) * n / nsl), i1 = int(int64_t(sl + 1) * n / nsl);
  // chunks: the same count in every section (their barriers are shared)
  const int nch = MERGE ? ((n + NH - 1) / NH + DT - 1) / DT : (i1 - i0 + DT - 1) / DT;
  const int64_t rows = int64_t(gridDim.y) * NREP;

  // gathering: thread = (row tid / 4, quarter tid % 4 of the row)
  const int gr = tid >> 2, gq = tid & 3;
  // (zero until the first gather: a section with no token stages zero rows)
  uint32_t kr[RE / 2] = {}, vr[RE / 2] = {};
  bool kpk = false, vpk = false;  // the thread's row is in the packed K / V segment
  auto gather = [&](int c0) {
    const int i = c0 + gr;
    const int t = i < i1 ? (i < n0 ? a.lo0 + i : a.lo1 + (i - n0)) : -1;
    kpk = gather_row<RE>(a.k, b, kvh, t, gq * RE, kr);
    vpk = gather_row<RE>(a.v, b, kvh, t, gq * RE, vr);
  };
  // the first chunk's rows and the query are loaded together (one round trip);
  // MERGE: so are the fused runs' statistics and partials of the thread's
  // first output element (up to NRPRE runs; more are read at the merge)
  constexpr int NRPRE = MERGE_RUNS_MAX;
  float pm[NRPRE], pl[NRPRE], po[NRPRE];
  int nr = 0;
  if constexpr (MERGE) {
    nr = detail::ShareMap::make(a.fgrid, int(gridDim.y), a.fnsf, a.fpair_e0).nruns(bh);
    const int r = int(threadIdx.x);
    const int64_t row = int64_t(bh) * NREP + min(r / D, NREP - 1);
#pragma unroll
    for (int sp = 0; sp < NRPRE; ++sp) {
      const int64_t sr = int64_t(min(sp, nr - 1)) * rows + row;  // clamped: every load issued at once
      pm[sp] = a.fml[sr * 2];
      pl[sp] = a.fml[sr * 2 + 1];
      po[sp] = a.fpart[sr * D + r % D];
    }
  }
  if (i0 < i1) gather(i0);
  for (int i = int(threadIdx.x); i < NREP * TW; i += NTH) {
    const int h = i / TW, c = i % TW;
    if constexpr (BF) {
      qs2[h][c] = __float_as_uint(bf2f(a.q[b * a.sqb + (kvh * NREP + h) * a.sqh + c]));
    } else {
      const uint16_t* qr = a.q + b * a.sqb + (kvh * NREP + h) * a.sqh + 2 * c;
      qs2[h][c] = uint32_t(qr[0]) | (uint32_t(qr[1]) << 16);
    }
  }
  float m[HPW], l[HPW];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) { m[hh] = -INFINITY; l[hh] = 0.f; }
  float o[OPT][2];  // BF: thread = (head, column pair) items
#pragma unroll
  for (int it = 0; it < OPT; ++it) o[it][0] = o[it][1] = 0.f;
  float ov[NREP][2];  // fp16: columns 2 pr, 2 pr + 1 of every head over the lane's tokens
#pragma unroll
  for (int h = 0; h < NREP; ++h) ov[h][0] = ov[h][1] = 0.f;
  const int pr = lane % PPL, tl0 = wave * (DT / 4) + (lane / PPL) * TPS;  // fp16 attn.V: pair, first token

  for (int ci = 0; ci < nch; ++ci) {
    // a chunk past the slice's tokens (MERGE: a shorter section) has no live
    // token: its logits are -inf and no V row is read
    const int c0 = i0 + ci * DT;
    // the fp16 rows from registers; packed rows are decoded into the tiles
    // (disjoint rows: no ordering needed between the two)
    if (!kpk) {
#pragma unroll
      for (int j = 0; j < RE / 2; ++j) {
        if constexpr (BF) {
          kt[gr][gq * RE + 2 * j] = kr[j] << 16;             // bf16 -> fp32: exact
          kt[gr][gq * RE + 2 * j + 1] = kr[j] & 0xffff0000u;
        } else {
          kt[gr][gq * (RE / 2) + j] = kr[j];
        }
      }
    }
    if (!vpk) {
#pragma unroll
      for (int j = 0; j < RE / 2; ++j) {
        if constexpr (BF) {
          vt[gr][gq * RE + 2 * j] = vr[j] << 16;
          vt[gr][gq * RE + 2 * j + 1] = vr[j] & 0xffff0000u;
        } else {
          vt[gr][gq * (RE / 2) + j] = vr[j];
        }
      }
    }
    if constexpr (PK) {  // runs: dense range 0 (rows < n0 - c0), then range 1
      const int64_t bh64 = int64_t(b) * a.Hkv + kvh;
      const int rend = min(DT, i1 - c0), rs = min(max(n0 - c0, 0), rend);
      packed_run<D, MERGE, BF>(a.k[1], a.v[1], a.norm, bh64, a.lo0 + c0, 0, rs, &kt[0][0], KS, &vt[0][0], VS);
      packed_run<D, MERGE, BF>(a.k[1], a.v[1], a.norm, bh64, a.lo1 + c0 - n0, rs, rend, &kt[0][0], KS, &vt[0][0],
                               VS);
    }
    __syncthreads();
    if (c0 + DT < i1) gather(c0 + DT);  // in flight through this chunk
    // ---- logits and running softmax: wave w, heads w + 4 hh, lane = token ----
    float dot[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) dot[hh] = 0.f;
    if constexpr (BF) {
      // no per-iteration guard on the head (a wave-uniform branch in the loop
      // serialized it on LDS latency): heads past NREP read the last head's
      // query and their logits are dropped below; one fp32 fma per column
#pragma unroll 16
      for (int i = 0; i < TW; ++i) {
        const uint32_t k2 = kt[lane][i];
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
          const int h = min(wave + 4 * hh, NREP - 1);
          dot[hh] = fmaf(__uint_as_float(k2), __uint_as_float(qs2[h][i]), dot[hh]);
        }
      }
    } else {
      // wave w: its quarter of head_dim for every head, four of the row's
      // pairs per step against each head's four query pairs (one broadcast
      // read); one v_dot2_f32_f16 per (head, column pair): both products
      // exact, accumulated in fp32.  The quarters are summed in wave order.
      float dq[NREP];
#pragma unroll
      for (int h = 0; h < NREP; ++h) dq[h] = 0.f;
      const uint32_t* krow = &kt[lane][wave * QW];
#pragma unroll
      for (int i = 0; i < QW; i += 4) {
        const uint32_t k0 = krow[i], k1 = krow[i + 1], k2 = krow[i + 2], k3 = krow[i + 3];
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
          const uint4 qv = *reinterpret_cast<const uint4*>(&qs2[h][wave * QW + i]);
          dq[h] = dot2<false>(k3, qv.w, dot2<false>(k2, qv.z, dot2<false>(k1, qv.y, dot2<false>(k0, qv.x, dq[h]))));
        }
      }
#pragma unroll
      for (int h = 0; h < NREP; ++h) lgp[wave][h][lane] = dq[h];
      __syncthreads();
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        const int h = min(wave + 4 * hh, NREP - 1);
        dot[hh] = ((lgp[0][h][lane] + lgp[1][h][lane]) + lgp[2][h][lane]) + lgp[3][h][lane];
      }
    }
    const bool live = c0 + lane < i1;
    {  // DPP reductions over the wave's heads at once
      float x[HPW], mx[HPW], cs[HPW];
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        x[hh] = live && wave + 4 * hh < NREP ? dot[hh] * a.scale : -INFINITY;
        mx[hh] = x[hh];
      }
      wave_max_dpp(mx);
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        mx[hh] = fmaxf(m[hh], mx[hh]);
        cs[hh] = x[hh] == -INFINITY ? 0.f : __expf(x[hh] - mx[hh]);
        x[hh] = cs[hh];
      }
      wave_sum_dpp(cs);
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        const int h = wave + 4 * hh;
        if (h < NREP) {
          if constexpr (BF) psf[h * DT + lane] = x[hh];
          else ps[h][lane] = __half_as_ushort(__float2half_rn(x[hh]));
          const float alpha = m[hh] == -INFINITY ? 0.f : __expf(m[hh] - mx[hh]);
          l[hh] = fmaf(l[hh], alpha, cs[hh]);
          m[hh] = mx[hh];
          if (lane == 0) al[h] = alpha;
        }
      }
    }
    __syncthreads();
    if constexpr (BF) {
      // ---- attn.V: thread = (head, column pair), eight tokens per step in
      // two accumulation chains (the tile rows past the chunk's tokens are
      // zero and their p is 0, so the chunk is read in whole steps); fp32
      // values and probabilities ----
      const int cnt8 = (min(DT, i1 - c0) + 7) & ~7;
#pragma unroll
      for (int it = 0; it < OPT; ++it) {
        const int idx = tid + 256 * it;
        if (idx < NREP * NPR) {
          const int h = idx / NPR, dp = idx % NPR;
          float o0 = o[it][0] * al[h], o1 = o[it][1] * al[h], e0 = 0.f, e1 = 0.f;
          for (int j = 0; j < cnt8; j += 8) {
#pragma unroll
            for (int u = 0; u < 8; u += 4) {  // columns 2 dp, 2 dp + 1 of four tokens
              const float* pf = psf + h * DT + j + u;
              const float2 va = *reinterpret_cast<const float2*>(&vt[j + u][2 * dp]);
              const float2 vb = *reinterpret_cast<const float2*>(&vt[j + u + 1][2 * dp]);
              const float2 vc = *reinterpret_cast<const float2*>(&vt[j + u + 2][2 * dp]);
              const float2 vd = *reinterpret_cast<const float2*>(&vt[j + u + 3][2 * dp]);
              o0 = fmaf(vb.x, pf[1], fmaf(va.x, pf[0], o0));
              o1 = fmaf(vb.y, pf[1], fmaf(va.y, pf[0], o1));
              e0 = fmaf(vd.x, pf[3], fmaf(vc.x, pf[2], e0));
              e1 = fmaf(vd.y, pf[3], fmaf(vc.y, pf[2], e1));
            }
          }
          o[it][0] = o0 + e0;
          o[it][1] = o1 + e1;
        }
      }
    } else {
      // ---- attn.V: wave w takes tokens [DT/4 w, DT/4 (w+1)) of the chunk
      // for every head, lane = (column pair pr, token subgroup); per two
      // tokens and column a v_dot2_f32_f16 of (v_j, v_j+1) (one v_perm_b32
      // from the two rows' pairs) and each head's fp16 (p_j, p_j+1).  Every
      // row is read: rows past the chunk's tokens hold zeros (or, in a
      // section with fewer chunks, its last chunk's rows) and have p = 0 ----
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        ov[h][0] *= al[h];
        ov[h][1] *= al[h];
      }
#pragma unroll
      for (int j = 0; j < TPS; j += 2) {
        const uint32_t va = vt[tl0 + j][pr], vb = vt[tl0 + j + 1][pr];
        const uint32_t lo = __builtin_amdgcn_perm(vb, va, 0x05040100u);  // column 2 pr of tokens j, j + 1
        const uint32_t hi = __builtin_amdgcn_perm(vb, va, 0x07060302u);  // column 2 pr + 1
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
          const uint32_t pp = *reinterpret_cast<const uint32_t*>(&ps[h][tl0 + j]);
          ov[h][0] = dot2<false>(lo, pp, ov[h][0]);
          ov[h][1] = dot2<false>(hi, pp, ov[h][1]);
        }
      }
    }
    __syncthreads();
  }
  // fp16: the waves' partial outputs go into the K tile (every wave is past
  // its last read of it), [wave][head][column]; D = 64: lanes l and l + 32
  // (the two token subgroups) first
  if constexpr (!BF) {
    float* opart = reinterpret_cast<float*>(&kt[0][0]);
    if constexpr (TSUB == 2) {
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        ov[h][0] += __shfl_xor(ov[h][0], 32, 64);
        ov[h][1] += __shfl_xor(ov[h][1], 32, 64);
      }
    }
    if (lane < PPL) {
#pragma unroll
      for (int h = 0; h < NREP; ++h) {
        opart[(wave * NREP + h) * D + 2 * pr] = ov[h][0];
        opart[(wave * NREP + h) * D + 2 * pr + 1] = ov[h][1];
      }
    }
  }
  // the section's output column dd of head h: its waves' partials in wave order
  auto sec_out = [&](int hf, int h, int dd) {
    const float* op = reinterpret_cast<const float*>(&kts[hf][0][0]) + h * D + dd;
    return ((op[0] + op[NREP * D]) + op[2 * NREP * D]) + op[3 * NREP * D];
  };
  if constexpr (MERGE) {
    // ---- merge: the sections' states and the fused runs' partials ----
    __shared__ float mh[NH][NREP], lh[NH][NREP];
    __shared__ float oh[BF ? NH : 1][BF ? NREP : 1][BF ? D : 1];  // BF: the sections' outputs
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      const int h = wave + 4 * hh;
      if (h < NREP && lane == 0) {
        mh[half][h] = m[hh];
        lh[half][h] = l[hh];
      }
    }
    if constexpr (BF) {
#pragma unroll
      for (int it = 0; it < OPT; ++it) {
        const int idx = tid + 256 * it;
        if (idx < NREP * NPR) {
          const int h = idx / NPR, dp = idx % NPR;
          oh[half][h][2 * dp] = o[it][0];
          oh[half][h][2 * dp + 1] = o[it][1];
        }
      }
    }
    __syncthreads();
    for (int r = int(threadIdx.x); r < NREP * D; r += NTH) {
      const int h = r / D, dd = r % D;
      const int64_t row = int64_t(bh) * NREP + h;
      const bool pre = r < NTH;  // the preloaded element (registers indexed by constants only)
      float M = -INFINITY;
#pragma unroll
      for (int hf = 0; hf < NH; ++hf) M = fmaxf(M, mh[hf][h]);
#pragma unroll
      for (int sp = 0; sp < NRPRE; ++sp)
        if (sp < nr) M = fmaxf(M, pre ? pm[sp] : a.fml[(int64_t(sp) * rows + row) * 2]);
      for (int sp = NRPRE; sp < nr; ++sp) M = fmaxf(M, a.fml[(int64_t(sp) * rows + row) * 2]);
      float L = 0.f, acc = 0.f;
      auto add_run = [&](float ms, float ls, float pv) {  // the runs in slot order, then the sections
        const float w = ms == -INFINITY ? 0.f : __expf(ms - M);
        L = fmaf(w, ls, L);
        acc = w != 0.f ? fmaf(w, pv, acc) : acc;
      };
#pragma unroll
      for (int sp = 0; sp < NRPRE; ++sp) {
        if (sp < nr) {
          const int64_t sr = int64_t(sp) * rows + row;
          if (pre) add_run(pm[sp], pl[sp], po[sp]);
          else add_run(a.fml[sr * 2], a.fml[sr * 2 + 1], a.fpart[sr * D + dd]);
        }
      }
      for (int sp = NRPRE; sp < nr; ++sp) {
        const int64_t sr = int64_t(sp) * rows + row;
        add_run(a.fml[sr * 2], a.fml[sr * 2 + 1], a.fpart[sr * D + dd]);
      }
#pragma unroll
      for (int hf = 0; hf < NH; ++hf) {
        const float w = mh[hf][h] == -INFINITY ? 0.f : __expf(mh[hf][h] - M);
        L = fmaf(w, lh[hf][h], L);
        if constexpr (BF) acc = fmaf(w, oh[hf][h][dd], acc);
        else acc = fmaf(w, sec_out(hf, h, dd), acc);
      }
      a.out[b * a.sob + (int64_t(kvh) * NREP + h) * a.soh + dd] = uint16_t(to_act<BF>(acc / L));
    }
    return;
  }
  // ---- this slice's statistics and unnormalized output (an empty slice:
  // m = -inf, which the combine skips) ----
  float* mls = a.ml + int64_t(blockIdx.x) * rows * 2;
  float* os = a.o + int64_t(blockIdx.x) * rows * D;
  const int64_t row0 = int64_t(b) * a.Hq + int64_t(kvh) * NREP;
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    const int h = wave + 4 * hh;
    if (h < NREP && lane == 0) {
      mls[(row0 + h) * 2] = m[hh];
      mls[(row0 + h) * 2 + 1] = l[hh];
    }
  }
  if constexpr (BF) {
#pragma unroll
    for (int it = 0; it < OPT; ++it) {
      const int idx = tid + 256 * it;
      if (idx < NREP * NPR) {
        const int h = idx / NPR, dp = idx % NPR;
        float* dst = os + (row0 + h) * D + 2 * dp;
        dst[0] = o[it][0];
        dst[1] = o[it][1];
      }
    }
  } else {
    __syncthreads();  // the waves' partials are in the K tile
    for (int r = tid; r < NREP * D; r += 256) os[(row0 + r / D) * D + r % D] = sec_out(half, r / D, r % D);
  }
}

// out[bq, d] = sum_s e^{m_s - M} o_s[bq, d] / sum_s e^{m_s - M} l_s
// One wave per row bq, lane = head_dim columns DPL*lane .. DPL*lane+DPL-1,
// over the row's live split slots, listed in slot order: the fused kernel's
// run partials of the row's (batch, KV head), slots 0 .. nr-1, then the dense
// slices' slots nsf .. nsplit-1.  With the fused kernel's workgroup count
// (grid > 0) nr follows from its share arithmetic (detail::ShareMap): the
// runs of a (batch, KV head) come from the shares that hold its splits, one
// run each.
// Without it (grid = 0: the unfused path, which writes every slot, or a
// caller of the split stage alone, whose fused kernel wrote empty statistics
// in the slots past the runs) every slot 0 .. nsplit-1 is read.  One round of
// loads - the live slots' (m, l) and, unconditionally, the partials of the
// first CSPEC listed slots (indices clamped so that every load is issued at
// once) - covers up to CSPEC live slots; a slot is used only if its weight is
// nonzero (a select: an unwritten partial cannot reach the sum).  Further
// live slots are listed in LDS and read CREST at a time.
constexpr int MAXSPLIT = 1024;  // split slots of one step, at most
// live slots past the first CSPEC (8, or 32 where a head has more than eight
// runs) are read CREST per round of loads (a head
// spread over many workgroups, e.g. one (batch, KV head) over a long context,
// has a run per workgroup: 248 further slots took 31 dependent rounds of 8)
constexpr int CREST = 32;
template <int DPL, int E, int CSPEC>
__global__ __launch_bounds__(64) void flash_combine_kernel(const float* __restrict__ ml, const float* __restrict__ part,
                                                           int nsplit, int nsf, int grid, int pair_e0, int nrep,
                                                           int64_t rows, int Hq, uint16_t* __restrict__ out,
                                                           int64_t sob, int64_t soh, int bf) {
  using Vec = float __attribute__((ext_vector_type(DPL)));
  constexpr int D = 64 * DPL;
  __shared__ int sidx[64 * E];
  __shared__ float swgt[64 * E];
  const int64_t bq = blockIdx.x;
  const int lane = threadIdx.x;
  int nr = nsf;
  if (grid > 0)  // the runs of the (batch, KV head) in the fused kernel's shares
    nr = detail::ShareMap::make(grid, int(rows / nrep), nsf, pair_e0).nruns(int(bq / nrep));
  const int n = nr + (nsplit - nsf);                                   // live slots
  auto slot = [&](int i) { return i < nr ? i : nsf + (i - nr); };     // i-th live slot
  const float2* st = reinterpret_cast<const float2*>(ml) + bq;         // slot s: st[s * rows]
  const Vec* pr = reinterpret_cast<const Vec*>(part + bq * D) + lane;  // slot s: pr[s * rows * 64]
  const int64_t pstride = rows * 64;
  // ---- one round: statistics of the live slots, partials of the first CSPEC ----
  float2 sl[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = e * 64 + lane;
    sl[e] = i < n ? st[int64_t(slot(i)) * rows] : make_float2(-INFINITY, 0.f);
  }
  Vec pv[CSPEC];
#pragma unroll
  for (int j = 0; j < CSPEC; ++j) pv[j] = pr[int64_t(slot(min(j, n - 1))) * pstride];
  float Mv[1] = {-INFINITY};
#pragma unroll
  for (int e = 0; e < E; ++e) Mv[0] = fmaxf(Mv[0], sl[e].x);
  wave_max_dpp(Mv);
  const float M = Mv[0];
  float Lv[1] = {0.f}, w[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    w[e] = sl[e].x == -INFINITY ? 0.f : __expf(sl[e].x - M);
    Lv[0] = fmaf(w[e], sl[e].y, Lv[0]);
  }
  wave_sum_dpp(Lv);
  const float L = Lv[0];
  Vec acc = 0.f;
#pragma unroll
  for (int j = 0; j < CSPEC; ++j) {
    const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[0]), j));  // live slot j: lane j
    if (wj != 0.f) acc += wj * pv[j];
  }
  // ---- the rest: nonempty live slots past the first CSPEC ----
  int m = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (e * 64 >= n) break;
    const int i = e * 64 + lane;
    const bool take = w[e] != 0.f && i >= CSPEC;
    const unsigned long long bal = __ballot(take);
    if (take) {
      const int k = m + __popcll(bal & ((1ull << lane) - 1ull));
      sidx[k] = slot(i);
      swgt[k] = w[e];
    }
    m += __popcll(bal);
  }
  if (m) {
    __syncthreads();
    for (int k0 = 0; k0 < m; k0 += CREST) {
      Vec v[CREST];
#pragma unroll
      for (int u = 0; u < CREST; ++u) v[u] = pr[int64_t(sidx[min(k0 + u, m - 1)]) * pstride];
#pragma unroll
      for (int u = 0; u < CREST; ++u)
        if (k0 + u < m) acc += swgt[k0 + u] * v[u];
    }
  }
  uint16_t* o = out + (bq / Hq) * sob + (bq % Hq) * soh + DPL * lane;
#pragma unroll
  for (int i = 0; i < DPL; ++i) o[i] = uint16_t(bf ? f2bf(acc[i] / L) : __half_as_ushort(__float2half_rn(acc[i] / L)));
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int nsplit_max(int T) { return int(ceil_div(T, detail::flash_split_tokens())); }

Seg to_seg(const iq_segment& s, int start) {
  Seg g{};
  g.dense = (const uint16_t*)s.dense;
  g.sb = s.s_b; g.sh = s.s_h; g.st = s.s_t;
  g.n = s.n; g.start = start;
  g.codes = s.codes; g.meta = s.meta; g.t_cap = s.t_cap; g.t0 = s.t0;
  g.bits = s.bits; g.group = s.group; g.mode = base_mode(s.mode);
  g.gsh = s.group > 0 ? __builtin_ctz(unsigned(s.group)) : 0;
  g.cap_groups = s.group > 0 ? s.t_cap / s.group : 0;
  if (s.n && s.codes) g.dense = nullptr;
  g.vec = g.dense && aligned(g.dense, 16) && s.s_b % 8 == 0 && s.s_h % 8 == 0 && s.s_t % 8 == 0;
  return g;
}

}  // namespace

namespace {

struct Workspace {
  uint32_t* qrec;  // query operand records (unfused path)
  uint32_t* vrec;  // probability operand records (unfused path)
  float* ml;       // [nsplit][B*Hq][2] split (max, sum)
  float* part;     // [nsplit][B*Hq][D] unnormalized split outputs
};

Workspace carve(void* workspace, int B, int Hq, int T, int D) {
  const size_t rows = size_t(B) * Hq;
  char* ws = (char*)workspace;
  Workspace w{};
  w.qrec = (uint32_t*)ws;
  ws += detail::qk_record_bytes(B, Hq, D);
  size_t vrec_bytes = 0;
  for (int g : {32, 64, 128}) vrec_bytes = std::max(vrec_bytes, rec_bytes_bound(int64_t(B) * Hq, T / g, g));
  w.vrec = (uint32_t*)ws;
  ws += align256(vrec_bytes);
  const size_t ns_cap = size_t(nsplit_max(T)) + NSD_MAX;
  w.ml = (float*)ws;
  ws += align256(ns_cap * rows * 2 * 4);
  w.part = (float*)ws;
  return w;
}

// 1: bf16 activations (IQ_MODE_BF16 on every segment holding tokens), 0:
// fp16 (on none), -1: mixed
int decode_act(const iq_segment* k, const iq_segment* v) {
  int act = -1;
  for (int s = 0; s < 3; ++s)
    for (const iq_segment* g : {&k[s], &v[s]}) {
      if (!g->n) continue;
      const int a = act_bf16(g->mode) ? 1 : 0;
      if (act >= 0 && a != act) return -1;
      act = a;
    }
  return act < 0 ? 0 : act;
}

int check_decode(const void* q, const iq_segment* k, const iq_segment* v, int B, int Hq, int Hkv, int T, int D,
                 const void* workspace, size_t workspace_bytes) {
  IQ_CHECK(q && k && v, IQ_ERR_NULL);
  IQ_CHECK(B >= 0 && T > 0 && Hkv > 0 && Hq > 0, IQ_ERR_SHAPE);
  IQ_CHECK(d_ok(D) && Hq % Hkv == 0 && nrep_ok(Hq / Hkv), IQ_ERR_SHAPE);
  for (int s = 0; s < 3; ++s) IQ_CHECK(k[s].n >= 0 && v[s].n >= 0, IQ_ERR_SHAPE);
  IQ_CHECK(k[0].n + k[1].n + k[2].n == T && v[0].n + v[1].n + v[2].n == T, IQ_ERR_SHAPE);
  for (int s : {0, 2}) {
    IQ_CHECK(k[s].n == 0 || k[s].dense, IQ_ERR_NULL);
    IQ_CHECK(v[s].n == 0 || v[s].dense, IQ_ERR_NULL);
  }
  // the call's activation dtype: IQ_MODE_BF16 on every segment that holds
  // tokens or on none (a dense segment's mode carries only that bit)
  if (decode_act(k, v) < 0) return IQ_ERR_MODE;
  for (int s : {0, 2})
    IQ_CHECK((k[s].n == 0 || base_mode(k[s].mode) == 0) && (v[s].n == 0 || base_mode(v[s].mode) == 0), IQ_ERR_MODE);
  if (k[1].n) {
    const iq_segment& g = k[1];
    IQ_CHECK(g.codes && g.meta, IQ_ERR_NULL);
    if (int e = check_v_common(g.bits, g.group, base_mode(g.mode))) return e;  // asym, sym or hybrid
    IQ_CHECK(D % g.group == 0, IQ_ERR_GROUP);
    // any store token may start the segment (a sliding window's start): the
    // fused range begins at the first token where K blocks and V groups align,
    // the tokens before it are decoded by the dense kernel
    IQ_CHECK(g.t_cap % TOKEN_BLOCK == 0 && g.t0 >= 0, IQ_ERR_ALIGN);
    IQ_CHECK(int64_t(g.t0) + g.n <= g.t_cap, IQ_ERR_RANGE);
    IQ_CHECK(aligned(g.codes, 16) && aligned(g.meta, 4), IQ_ERR_ALIGN);
  }
  if (v[1].n) {
    const iq_segment& g = v[1];
    IQ_CHECK(g.codes && g.meta, IQ_ERR_NULL);
    if (int e = check_v_common(g.bits, g.group, base_mode(g.mode))) return e;
    IQ_CHECK(g.t0 >= 0 && g.t_cap % g.group == 0, IQ_ERR_GROUP);
    IQ_CHECK(int64_t(g.t0) + g.n <= g.t_cap, IQ_ERR_RANGE);
    IQ_CHECK(aligned(g.codes, 16) && aligned(g.meta, 8), IQ_ERR_ALIGN);
  }
  IQ_CHECK(workspace && workspace_bytes >= iq_decode_workspace_bytes(B, Hq, T, D), IQ_ERR_WORKSPACE);
  IQ_CHECK(aligned(workspace, 256), IQ_ERR_ALIGN);
  return IQ_OK;
}

// What the split stage launched: nsplit split slots, nsf of them for the
// packed range (the rest are dense slices); grid = the fused kernel's
// workgroup count (0: it did not run, or it wrote empty statistics for a
// combine that scans every slot).
struct SplitPlan {
  int nsplit = 0, nsf = 0, grid = 0, nrep = 1;
  int bf = 0;           // bf16 activations (the output's dtype)
  int pair_e0 = 0;      // the fused kernel's partition (detail::ShareMap)
  bool merged = false;  // the output is written (dense window and merge after the fused kernel)
};

// The output of a full decode call (what the merging dense kernel writes)
struct MergeOut {
  void* out;
  int64_t so_b, so_h;
};
// dense tokens per (batch, KV head), at most, that the merging dense kernel
// takes (its sections' chunks: at most two per section); longer windows take
// the slices
constexpr int MERGE_DENSE_MAX = 4 * DT;

// Launches everything up to the split statistics and partials.  `live`: the
// combine will be told the fused kernel's workgroup count and read only the
// live slots (the fused kernel then writes no empty statistics).  `mo` (a full
// call): where the output goes when a short fp16 window is attended after the
// fused kernel by the merging dense kernel, which also writes the output
// (plan->merged: no combine launch).
int launch_splits(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const iq_segment* k,
                  const iq_segment* v, int B, int Hq, int Hkv, int T, int D, float scale, const Workspace& w,
                  SplitPlan* plan, bool live, hipStream_t st, const MergeOut* mo = nullptr) {
  *plan = SplitPlan{};
  plan->nrep = Hq / Hkv;
  const bool bf = decode_act(k, v) == 1;
  plan->bf = bf;
  const int64_t rows = int64_t(B) * Hq;
  // fused range: packed in both K and V, aligned to K blocks and V groups
  const int ks = k[0].n, vs = v[0].n;
  const int lo = std::max(ks, vs), hi = std::min(ks + k[1].n, vs + v[1].n);
  int a0 = -1, c = 0;
  if (k[1].n && v[1].n && hi > lo) {
    const int vg = v[1].group;
    for (int t = lo; t < std::min(hi, lo + TOKEN_BLOCK * vg); ++t)
      if ((k[1].t0 + t - ks) % TOKEN_BLOCK == 0 && (v[1].t0 + t - vs) % vg == 0) {
        a0 = t;
        break;
      }
    if (a0 >= 0) {
      c = hi - a0;
      c -= c % vg;
      if (detail::flash_split_tokens() % vg) c = 0;
    }
  }
  if (c <= 0) { a0 = 0; c = 0; }
  const int nsf = c ? int(ceil_div(c, detail::flash_split_tokens())) : 0;

  const detail::FusedStore fk{k[1].codes, k[1].meta, k[1].t_cap, k[1].t0 + (a0 - ks), k[1].bits, k[1].group,
                              k[1].mode};
  const detail::FusedStore fv{v[1].codes, v[1].meta, v[1].t_cap, v[1].t0 + (a0 - vs), v[1].bits, v[1].group,
                              v[1].mode};
  const bool fused =
      c && k[1].group == v[1].group && detail::flash_fused_supported(q, sq_b, sq_h, norm, fk, fv, Hq, Hkv, D);
  // A combine that reads every split slot (the unfused kernels write one per
  // split; the split stage alone leaves empty statistics in the slots past
  // the fused runs) holds at most MAXSPLIT of them: checked before any launch.
  // A full call on the fused path reads only the live slots (a head's fused
  // runs, at most one per workgroup, and the dense slices), so the context
  // length is bounded by the workspace alone.
  if (c && !(fused && live) && nsf + NSD_MAX > MAXSPLIT) return IQ_ERR_SHAPE;
  // bf16 layers: the fused kernel (K and V of one group size) and the dense
  // kernels; the unfused packed kernels take fp16 only
  if (c && !fused && bf) return IQ_ERR_MODE;
  // hybrid K: the fused kernel (K and V of one group size) and the dense kernels
  if (c && !fused && base_mode(k[1].mode) == IQ_MODE_HYBRID) return IQ_ERR_MODE;
  // The live slots of a row: at most one fused run per workgroup, then the
  // slices.  The fused kernel's grid (one workgroup per CU: far below the
  // limit) is worked out and checked before anything is launched.
  int fgrid = 0;
  if (fused && live) {
    if (int e = detail::flash_fused_launch(q, sq_b, sq_h, norm, fk, fv, B, Hq, Hkv, c, D, scale, w.ml, w.part,
                                           &fgrid, st, false))
      return e;
    if (fgrid + NSD_MAX > MAXSPLIT) return IQ_ERR_SHAPE;
  }

  // dense tokens -> split slots nsf, nsf + 1, ...: up to two workgroups per
  // CU (a workgroup's chunks run one after another, each a chain of memory
  // round trips), at least DSLICE tokens each
  DenseArgs da{};
  da.q = (const uint16_t*)q; da.sqb = sq_b; da.sqh = sq_h; da.norm = (const uint16_t*)norm;
  int start = 0;
  for (int s = 0; s < 3; ++s) { da.k[s] = to_seg(k[s], start); start += k[s].n; }
  start = 0;
  for (int s = 0; s < 3; ++s) { da.v[s] = to_seg(v[s], start); start += v[s].n; }
  da.lo0 = 0; da.hi0 = c ? a0 : T;
  da.lo1 = c ? a0 + c : T; da.hi1 = T;
  da.Hq = Hq; da.Hkv = Hkv; da.scale = scale;
  da.ml = w.ml + int64_t(nsf) * rows * 2;
  da.o = w.part + int64_t(nsf) * rows * D;
  const int n_dense = (da.hi0 - da.lo0) + (da.hi1 - da.lo1);
  const int64_t bhs = int64_t(B) * Hkv;
  // any packed segment (tokens packed in only one of K and V) needs the
  // general gather; a dense-only step takes the short kernel
  auto packed_in_range = [&](const Seg& g) {
    auto meets = [&](int lo, int hi) { return lo < hi && g.start < hi && lo < g.start + g.n; };
    return g.n > 0 && !g.dense && (meets(da.lo0, da.hi0) || meets(da.lo1, da.hi1));
  };
  bool pk = false;
  for (int s = 0; s < 3; ++s) pk |= packed_in_range(da.k[s]) || packed_in_range(da.v[s]);
  // The dense slices: split slots nsf .. nsf + nsd - 1, read by the combine
  int nsd = 0;
  auto launch_slices = [&]() -> int {
    nsd = int(std::min<int64_t>({NSD_MAX, ceil_div(n_dense, DSLICE), std::max<int64_t>(1, ceil_div(2 * detail::num_cus(), bhs))}));
    const dim3 grid{unsigned(nsd), unsigned(bhs), 1u};
    auto go = [&]<int DD, int R>() {
      if (bf) {
        if (pk) dense_attn_kernel<DD, R, true, false, true><<<grid, 256, 0, st>>>(da);
        else dense_attn_kernel<DD, R, false, false, true><<<grid, 256, 0, st>>>(da);
      } else {
        if (pk) dense_attn_kernel<DD, R, true><<<grid, 256, 0, st>>>(da);
        else dense_attn_kernel<DD, R, false><<<grid, 256, 0, st>>>(da);
      }
    };
    auto by_r = [&]<int DD>() {
      switch (Hq / Hkv) {
        case 1: go.template operator()<DD, 1>(); break;
        case 2: go.template operator()<DD, 2>(); break;
        case 4: go.template operator()<DD, 4>(); break;
        default: go.template operator()<DD, 8>(); break;
      }
    };
    if (D == 128) by_r.template operator()<128>();
    else by_r.template operator()<64>();
    return launch_status();
  };
  // A short window next to the fused kernel (fp16 tokens and tokens packed in
  // only one of K and V) may be attended after the fused kernel by the merging
  // dense kernel, which also merges the fused runs and writes the output (no
  // dense slots, no combine): chosen once the fused kernel's workgroup count
  // is known, if no (batch, KV head) has more fused runs than that kernel
  // preloads.  Heads spread over more workgroups (a small batch over a long
  // context) take the slices and the combine, which reads every slot in one
  // round of loads.
  const bool merge_cand = mo && live && fused && n_dense > 0 && n_dense <= MERGE_DENSE_MAX;
  if (n_dense > 0 && !merge_cand)
    if (int e = launch_slices()) return e;

  if (fused) {
    int grid = 0;
    if (int e = detail::flash_fused_launch(q, sq_b, sq_h, norm, fk, fv, B, Hq, Hkv, c, D, scale, w.ml, w.part,
                                           live ? &grid : nullptr, st))
      return e;
    plan->grid = grid;
    plan->pair_e0 = detail::fused_pair_e0(k[1].bits, v[1].bits, base_mode(v[1].mode) == IQ_MODE_HYBRID);
    bool merge_dense = merge_cand;
    if (merge_cand) {
      const detail::ShareMap sm = detail::ShareMap::make(grid, int(bhs), nsf, plan->pair_e0);
      for (int h = 0; h < int(bhs) && merge_dense; ++h) merge_dense = sm.nruns(h) <= MERGE_RUNS_MAX;
      if (!merge_dense)
        if (int e = launch_slices()) return e;
    }
    if (merge_dense) {
      da.fml = w.ml;
      da.fpart = w.part;
      da.fgrid = grid;
      da.fnsf = nsf;
      da.fpair_e0 = plan->pair_e0;
      da.out = (uint16_t*)mo->out;
      da.sob = mo->so_b;
      da.soh = mo->so_h;
      const dim3 mgrid{1u, unsigned(bhs), 1u};
      auto go = [&]<int DD, int R>() {
        if (bf) {
          if (pk) dense_attn_kernel<DD, R, true, true, true><<<mgrid, 256 * merge_sections(true, true, R), 0, st>>>(da);
          else dense_attn_kernel<DD, R, false, true, true><<<mgrid, 256 * merge_sections(false, true, R), 0, st>>>(da);
        } else {
          if (pk) {
            dense_attn_kernel<DD, R, true, true><<<mgrid, 256 * merge_sections(true, false, R), 0, st>>>(da);
          } else if (merge_sections_dense(n_dense, R) == 3) {
            if constexpr (R <= 4) dense_attn_kernel<DD, R, false, true, false, 3><<<mgrid, 768, 0, st>>>(da);
          } else {
            dense_attn_kernel<DD, R, false, true><<<mgrid, 256 * merge_sections(false, false, R), 0, st>>>(da);
          }
        }
      };
      auto by_r = [&]<int DD>() {
        switch (Hq / Hkv) {
          case 1: go.template operator()<DD, 1>(); break;
          case 2: go.template operator()<DD, 2>(); break;
          case 4: go.template operator()<DD, 4>(); break;
          default: go.template operator()<DD, 8>(); break;
        }
      };
      if (D == 128) by_r.template operator()<128>();
      else by_r.template operator()<64>();
      if (int e = launch_status()) return e;
      plan->merged = true;
    }
  } else if (c) {
    const iq_segment& kg = k[1];
    const iq_segment& vg = v[1];
    if (int e = detail::qk_record_launch(q, sq_b, sq_h, norm, B, Hq, Hkv, D, kg.group, kg.bits, w.qrec, st))
      return e;
    const detail::FlashOut f{w.ml, w.vrec, vg.bits, vg.group};
    if (int e = detail::qk_flash_launch(w.qrec, norm != nullptr, kg.codes, kg.meta, kg.t_cap, B, Hq, Hkv,
                                        kg.t0 + (a0 - ks), c, D, kg.group, kg.bits, kg.mode, scale, f, st))
      return e;
    if (int e = detail::av_flash_launch(w.vrec, vg.codes, vg.meta, vg.t_cap, B, Hq, Hkv, vg.t0 + (a0 - vs), c, D,
                                        vg.group, vg.bits, vg.mode, w.part, st))
      return e;
  }
  plan->nsplit = nsf + nsd;
  plan->nsf = nsf;
  return IQ_OK;
}

int launch_combine(const Workspace& w, const SplitPlan& plan, int B, int Hq, int D, void* out, int64_t so_b,
                   int64_t so_h, hipStream_t st) {
  const int64_t rows = int64_t(B) * Hq;
  const int nsplit = plan.nsplit;
  // slots a row reads, at most: with the fused kernel's workgroup count, the
  // most runs of any (batch, KV head) (the share arithmetic the kernel uses)
  // and the dense slices; else every slot
  int nlive = nsplit;
  if (plan.grid > 0) {
    const int heads = int(rows / std::max(plan.nrep, 1));
    const detail::ShareMap sm = detail::ShareMap::make(plan.grid, heads, plan.nsf, plan.pair_e0);
    int maxr = 0;
    for (int h = 0; h < heads; ++h) maxr = std::max(maxr, sm.nruns(h));
    nlive = std::min(nsplit, maxr + (nsplit - plan.nsf));
  }
  // statistics registers per lane: the smallest power of two with 64 E >= nlive
  auto go = [&]<int DPL, int E>() {
    auto* kern = nlive > 8 ? flash_combine_kernel<DPL, E, 32> : flash_combine_kernel<DPL, E, 8>;
    kern<<<dim3(unsigned(rows)), 64, 0, st>>>(w.ml, w.part, nsplit, plan.nsf, plan.grid,
                                                                      plan.pair_e0, plan.nrep, rows, Hq,
                                                                      (uint16_t*)out, so_b, so_h, plan.bf);
  };
  auto by_e = [&]<int DPL>() {
    if (nlive <= 64) go.template operator()<DPL, 1>();
    else if (nlive <= 128) go.template operator()<DPL, 2>();
    else if (nlive <= 256) go.template operator()<DPL, 4>();
    else if (nlive <= 512) go.template operator()<DPL, 8>();
    else go.template operator()<DPL, 16>();
  };
  static_assert(MAXSPLIT == 64 * 16, "combine variants");
  if (D == 128) by_e.template operator()<2>();
  else by_e.template operator()<1>();
  return launch_status();
}

// ---- scratch of the no-allocation entry point ----
// The decode workspace (records, split statistics, partials) of
// iq_decode_attention_noalloc lives in this file-scope device array: each GPU
// the library runs on holds its own copy, at its own address, until the
// process ends.  Nothing in it has to start at zero: every split slot the
// combine reads is written by the split stage of the same call.  Calls that
// overlap on one GPU share the array and race.
constexpr size_t SCRATCH_BYTES = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// The device address of `scratch` on the current device, looked up once per
// device with that device current (the array's name is a host-side stand-in,
// never a device address).
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return IQ_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return IQ_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return IQ_OK;
}

}  // namespace

extern "C" {

size_t iq_decode_noalloc_max_bytes(void) { return SCRATCH_BYTES; }

int iq_decode_attention_noalloc(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const iq_segment* k,
                                const iq_segment* v, int B, int Hq, int Hkv, int T, int D, float scale, void* out,
                                int64_t so_b, int64_t so_h, void* stream) {
  IQ_CHECK(out, IQ_ERR_NULL);
  // every check of iq_decode_attention, host only, with the scratch's size as
  // the workspace size: a call whose workspace would exceed SCRATCH_BYTES
  // returns IQ_ERR_WORKSPACE before any HIP call (the stand-in pointer is only
  // tested for being non-null and aligned, never used)
  if (int e = check_decode(q, k, v, B, Hq, Hkv, T, D, reinterpret_cast<void*>(256), SCRATCH_BYTES)) return e;
  if (B == 0) return IQ_OK;
  void* ws = nullptr;
  if (int e = scratch_address(&ws)) return e;
  const Workspace w = carve(ws, B, Hq, T, D);
  SplitPlan plan;
  const MergeOut mo{out, so_b, so_h};
  if (int e = launch_splits(q, sq_b, sq_h, norm, k, v, B, Hq, Hkv, T, D, scale, w, &plan, true, (hipStream_t)stream,
                            &mo))
    return e;
  if (plan.merged) return IQ_OK;
  return launch_combine(w, plan, B, Hq, D, out, so_b, so_h, (hipStream_t)stream);
}

size_t iq_decode_workspace_bytes(int B, int Hq, int T, int D) {
  if (B <= 0 || Hq <= 0 || T <= 0 || !d_ok(D)) return 0;
  const size_t rows = size_t(B) * Hq;
  size_t vrec = 0;
  for (int g : {32, 64, 128}) vrec = std::max(vrec, rec_bytes_bound(int64_t(B) * Hq, T / g, g));
  const size_t ns = size_t(nsplit_max(T)) + NSD_MAX;
  return detail::qk_record_bytes(B, Hq, D) + align256(vrec) + align256(ns * rows * 2 * 4) +
         align256(ns * rows * D * 4);
}

int iq_decode_attention_splits(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const iq_segment* k,
                               const iq_segment* v, int B, int Hq, int Hkv, int T, int D, float scale,
                               void* workspace, size_t workspace_bytes, int* nsplit, void* stream) {
  IQ_CHECK(nsplit, IQ_ERR_NULL);
  if (int e = check_decode(q, k, v, B, Hq, Hkv, T, D, workspace, workspace_bytes)) return e;
  IQ_CHECK(nsplit_max(T) + NSD_MAX <= MAXSPLIT, IQ_ERR_SHAPE);  // its combine reads every slot
  IQ_CHECK(decode_act(k, v) == 0, IQ_ERR_MODE);  // its combine writes fp16 (bf16: the live stages)
  *nsplit = 0;
  if (B == 0) return IQ_OK;
  SplitPlan plan;
  // the split stage alone: empty statistics for a combine that scans every slot
  const int e = launch_splits(q, sq_b, sq_h, norm, k, v, B, Hq, Hkv, T, D, scale, carve(workspace, B, Hq, T, D),
                              &plan, false, (hipStream_t)stream);
  *nsplit = plan.nsplit;
  return e;
}

int iq_decode_attention_splits_live(const void* q, int64_t sq_b, int64_t sq_h, const void* norm,
                                    const iq_segment* k, const iq_segment* v, int B, int Hq, int Hkv, int T, int D,
                                    float scale, void* workspace, size_t workspace_bytes, iq_split_plan* plan,
                                    void* stream) {
  IQ_CHECK(plan, IQ_ERR_NULL);
  if (int e = check_decode(q, k, v, B, Hq, Hkv, T, D, workspace, workspace_bytes)) return e;
  *plan = iq_split_plan{};
  if (B == 0) return IQ_OK;
  SplitPlan sp;
  // the launches of iq_decode_attention with live slots; a short fp16 window
  // takes the slices (there is no output to merge into here)
  const int e = launch_splits(q, sq_b, sq_h, norm, k, v, B, Hq, Hkv, T, D, scale, carve(workspace, B, Hq, T, D), &sp,
                              true, (hipStream_t)stream);
  plan->nsplit = sp.nsplit;
  plan->nsf = sp.nsf;
  plan->grid = sp.grid;
  plan->nrep = sp.nrep;
  plan->pair_e0 = sp.pair_e0;
  plan->bf16 = sp.bf;
  return e;
}

int iq_decode_attention_combine_live(const iq_split_plan* plan, int B, int Hq, int T, int D, void* out, int64_t so_b,
                                     int64_t so_h, void* workspace, size_t workspace_bytes, void* stream) {
  IQ_CHECK(plan && out && workspace, IQ_ERR_NULL);
  IQ_CHECK(B >= 0 && Hq > 0 && T > 0 && d_ok(D), IQ_ERR_SHAPE);
  const iq_split_plan& p = *plan;
  IQ_CHECK(nrep_ok(p.nrep) && Hq % p.nrep == 0, IQ_ERR_SHAPE);
  IQ_CHECK(p.nsplit >= 1 && p.nsplit <= nsplit_max(T) + NSD_MAX && p.nsf >= 0 && p.nsf <= p.nsplit, IQ_ERR_SHAPE);
  IQ_CHECK(p.nsplit - p.nsf <= NSD_MAX && p.pair_e0 >= 0 && p.pair_e0 < detail::ShareMap::E0_DEN, IQ_ERR_SHAPE);
  // a grid the plan's slots cannot hold (every run covers at least one split)
  const int64_t heads = int64_t(B) * (Hq / p.nrep);
  IQ_CHECK(p.grid >= 0 && p.grid + NSD_MAX <= MAXSPLIT && (p.grid == 0 || p.grid <= int64_t(p.nsf) * heads),
           IQ_ERR_SHAPE);
  IQ_CHECK(p.grid > 0 || p.nsplit <= MAXSPLIT, IQ_ERR_SHAPE);  // without a grid every slot is read
  IQ_CHECK(workspace_bytes >= iq_decode_workspace_bytes(B, Hq, T, D), IQ_ERR_WORKSPACE);
  IQ_CHECK(aligned(workspace, 256), IQ_ERR_ALIGN);
  if (B == 0) return IQ_OK;
  SplitPlan sp;
  sp.nsplit = p.nsplit;
  sp.nsf = p.nsf;
  sp.grid = p.grid;
  sp.nrep = p.nrep;
  sp.pair_e0 = p.pair_e0;
  sp.bf = p.bf16 != 0;
  return launch_combine(carve(workspace, B, Hq, T, D), sp, B, Hq, D, out, so_b, so_h, (hipStream_t)stream);
}

int iq_decode_attention_combine(int nsplit, int B, int Hq, int T, int D, void* out, int64_t so_b, int64_t so_h,
                                void* workspace, size_t workspace_bytes, void* stream) {
  IQ_CHECK(out && workspace, IQ_ERR_NULL);
  IQ_CHECK(B >= 0 && Hq > 0 && T > 0 && d_ok(D), IQ_ERR_SHAPE);
  IQ_CHECK(nsplit >= 1 && nsplit <= nsplit_max(T) + NSD_MAX && nsplit <= MAXSPLIT, IQ_ERR_SHAPE);
  IQ_CHECK(workspace_bytes >= iq_decode_workspace_bytes(B, Hq, T, D), IQ_ERR_WORKSPACE);
  IQ_CHECK(aligned(workspace, 256), IQ_ERR_ALIGN);
  if (B == 0) return IQ_OK;
  SplitPlan plan;
  plan.nsplit = plan.nsf = nsplit;  // every slot
  return launch_combine(carve(workspace, B, Hq, T, D), plan, B, Hq, D, out, so_b, so_h, (hipStream_t)stream);
}

int iq_decode_attention(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const iq_segment* k,
                        const iq_segment* v, int B, int Hq, int Hkv, int T, int D, float scale, void* out,
                        int64_t so_b, int64_t so_h, void* workspace, size_t workspace_bytes, void* stream) {
  IQ_CHECK(out, IQ_ERR_NULL);
  if (int e = check_decode(q, k, v, B, Hq, Hkv, T, D, workspace, workspace_bytes)) return e;
  if (B == 0) return IQ_OK;
  const Workspace w = carve(workspace, B, Hq, T, D);
  SplitPlan plan;
  const MergeOut mo{out, so_b, so_h};
  if (int e = launch_splits(q, sq_b, sq_h, norm, k, v, B, Hq, Hkv, T, D, scale, w, &plan, true, (hipStream_t)stream,
                            &mo))
    return e;
  if (plan.merged) return IQ_OK;
  return launch_combine(w, plan, B, Hq, D, out, so_b, so_h, (hipStream_t)stream);
}

}  // extern "C"
