// Host entry of the fused flash-decoding kernel (iq_flash.h): argument
// checks, the kernel's argument block, and the launch for the K bit width.
#include <algorithm>

#include "iq_gemv.h"

using namespace iq;

namespace {
constexpr int FSPLIT = NWAVES * IQ_FLASH_BPW * TOKEN_BLOCK;  // tokens per split (= flash_split_tokens())
}  // namespace

namespace iq::detail {

// the buffer offsets of a split are 32-bit: every (batch, KV head) slice of
// the stores and the q rows of one KV head must stay below 2 GiB
bool flash_fused_supported(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const FusedStore& k,
                           const FusedStore& v, int Hq, int Hkv, int D) {
  (void)q; (void)sq_b; (void)norm;
  const int64_t lim = int64_t(1) << 31;
  const int nrep = Hkv > 0 ? Hq / Hkv : 1;
  return sq_h >= 0 && (int64_t(nrep - 1) * sq_h + D) * 2 < lim && k.t_cap * D * k.bits / 8 < lim &&
         k.t_cap * D * 4 / std::max(k.group, 1) < lim && v.t_cap * D * v.bits / 8 < lim &&
         v.t_cap * D * 4 / std::max(v.group, 1) < lim;
}

int flash_fused_launch(const void* q, int64_t sq_b, int64_t sq_h, const void* norm, const FusedStore& k,
                       const FusedStore& v, int B, int Hq, int Hkv, int T, int D, float scale, float* ml,
                       float* part, int* grid, hipStream_t stream, bool launch) {
  if (B == 0 || T == 0) return IQ_OK;
  if (k.group != v.group) return IQ_ERR_GROUP;
  // a bf16 layer: IQ_MODE_BF16 on both stores (the query, factor and metadata in bf16)
  const bool bf = act_bf16(k.mode);
  if (bf != act_bf16(v.mode)) return IQ_ERR_MODE;
  const int kmode = base_mode(k.mode), vmode = base_mode(v.mode);
  if (T % k.group || FSPLIT != flash_split_tokens()) return IQ_ERR_GROUP;
  if (k.t0 % TOKEN_BLOCK || v.t0 % v.group) return IQ_ERR_ALIGN;
  if (!flash_fused_supported(q, sq_b, sq_h, norm, k, v, Hq, Hkv, D)) return IQ_ERR_SHAPE;
  FusedArgs a{};
  a.q = (const uint16_t*)q; a.sqb = sq_b; a.sqh = sq_h; a.norm = (const uint16_t*)norm;
  a.kc = k.codes; a.km = k.meta; a.k_cap_blocks = k.t_cap / TOKEN_BLOCK; a.kblk0 = k.t0 / TOKEN_BLOCK;
  a.ksym = kmode == IQ_MODE_SYM;
  a.khyb = kmode == IQ_MODE_HYBRID;  // meta as asym ({scale | flag << 15, zero})
  a.vc = v.codes; a.vm = v.meta; a.v_cap_groups = v.t_cap / v.group; a.vg0 = v.t0 / v.group;
  a.vsym = vmode == IQ_MODE_SYM;
  a.Hkv = Hkv; a.T = T;
  a.nsplit = int(ceil_div(T, FSPLIT));
  a.nitems = a.nsplit * B * Hkv;
  const int64_t nblk = ceil_div(T, TOKEN_BLOCK);
  a.k_code_bytes = uint32_t(nblk * TOKEN_BLOCK * D * k.bits / 8);
  a.k_meta_bytes = uint32_t(nblk * TOKEN_BLOCK * (D / k.group) * (a.ksym ? 2 : 4));
  a.v_code_bytes = uint32_t(int64_t(T) * D * v.bits / 8);
  a.v_meta_bytes = uint32_t(int64_t(T / v.group) * D * (a.vsym ? 2 : 4));
  a.q_bytes = uint32_t((int64_t(Hq / Hkv - 1) * sq_h + D) * 2);
  a.norm_bytes = norm ? uint32_t(D * 2) : 0u;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.ml = ml; a.part = part;
  a.empty_stats = grid ? 0 : 1;  // a caller that takes the workgroup count reads only the run slots
  a.pair_e0 = fused_pair_e0(k.bits, v.bits, vmode == IQ_MODE_HYBRID);
  const bool nm = norm != nullptr;
  if (bf) {
    const bool vh = vmode == IQ_MODE_HYBRID;
    switch (k.bits) {
      case 2: return vh ? flash_fused_launch_bf_vh_k2(a, v.bits, k.group, D, Hq / Hkv, nm, grid, stream, launch)
                        : flash_fused_launch_bf_k2(a, v.bits, k.group, D, Hq / Hkv, nm, grid, stream, launch);
      case 3: return vh ? flash_fused_launch_bf_vh_k3(a, v.bits, k.group, D, Hq / Hkv, nm, grid, stream, launch)
                        : flash_fused_launch_bf_k3(a, v.bits, k.group, D, Hq / Hkv, nm, grid, stream, launch);
      case 4: return vh ? flash_fused_launch_bf_vh_k4(a, v.bits, k.group, D, Hq / Hkv, nm, grid, stream, launch)
                        : flash_fused_launch_bf_k4(a, v.bits, k.group, D, Hq / Hkv, nm, grid, stream, launch);
      default: return IQ_ERR_BITS;
    }
  }
  if (vmode == IQ_MODE_HYBRID) {
    switch (k.bits) {
      case 2: return flash_fused_launch_vh_k2(a, v.bits, k.group, D, Hq / Hkv, norm != nullptr, grid, stream, launch);
      case 3: return flash_fused_launch_vh_k3(a, v.bits, k.group, D, Hq / Hkv, norm != nullptr, grid, stream, launch);
      case 4: return flash_fused_launch_vh_k4(a, v.bits, k.group, D, Hq / Hkv, norm != nullptr, grid, stream, launch);
      default: return IQ_ERR_BITS;
    }
  }
  switch (k.bits) {
    case 2: return flash_fused_launch_k2(a, v.bits, k.group, D, Hq / Hkv, norm != nullptr, grid, stream, launch);
    case 3: return flash_fused_launch_k3(a, v.bits, k.group, D, Hq / Hkv, norm != nullptr, grid, stream, launch);
    case 4: return flash_fused_launch_k4(a, v.bits, k.group, D, Hq / Hkv, norm != nullptr, grid, stream, launch);
    default: return IQ_ERR_BITS;
  }
}

}  // namespace iq::detail
