// Host-side helpers shared by the C-ABI entry points: argument validation
// (done before any launch, so every error path is testable without a GPU),
// compile-time dispatch over (bits, group, head_dim, GQA ratio).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/innerq_abi.h"

namespace iq {

inline bool bits_ok(int bits) { return bits == 2 || bits == 3 || bits == 4; }
inline bool group_ok(int g) { return g == 32 || g == 64 || g == 128; }
inline bool mode_ok(int m) { return m == IQ_MODE_ASYM || m == IQ_MODE_SYM; }
// a mode argument's activation flag: bf16 instead of fp16 inputs, scales,
// zero points, signs and outputs (entry points that take it strip it first;
// everywhere else a flagged mode fails mode_ok)
inline bool act_bf16(int m) { return (m & IQ_MODE_BF16) != 0; }
inline int base_mode(int m) { return m & ~int(IQ_MODE_BF16); }
inline bool store_mode_ok(int m) { return mode_ok(m) || m == IQ_MODE_HYBRID; }
inline bool d_ok(int d) { return d == 64 || d == 128; }
inline bool nrep_ok(int r) { return r == 1 || r == 2 || r == 4 || r == 8; }
inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

#define IQ_CHECK(cond, err) \
  do {                      \
    if (!(cond)) return (err); \
  } while (0)

inline int check_common(int bits, int group, int mode) {
  IQ_CHECK(bits_ok(bits), IQ_ERR_BITS);
  IQ_CHECK(group_ok(group), IQ_ERR_GROUP);
  IQ_CHECK(mode_ok(mode), IQ_ERR_MODE);
  return IQ_OK;
}

// Packed stores also hold 1-bit asym codes (the asym half of 2-bit hybrid
// quantization, quant.py:136) and hybrid groups (bits 2-4).  The GEMVs take
// 2-4 bits only.
inline int check_store(int bits, int group, int mode) {
  IQ_CHECK(bits_ok(bits) || bits == 1, IQ_ERR_BITS);
  IQ_CHECK(group_ok(group), IQ_ERR_GROUP);
  IQ_CHECK(store_mode_ok(mode), IQ_ERR_MODE);
  IQ_CHECK(bits != 1 || mode == IQ_MODE_ASYM, IQ_ERR_BITS);
  return IQ_OK;
}

// a V store read by the attn.V GEMV / decode, or a K store read by the
// decode: asym, sym or hybrid
inline int check_v_common(int bits, int group, int mode) {
  IQ_CHECK(bits_ok(bits), IQ_ERR_BITS);
  IQ_CHECK(group_ok(group), IQ_ERR_GROUP);
  IQ_CHECK(store_mode_ok(mode), IQ_ERR_MODE);
  return IQ_OK;
}

// meta bytes per unit (K token-group, V group-column): sym stores keep the
// scale only, asym and hybrid {scale, zero}
inline int meta_unit_bytes(int mode) { return mode == IQ_MODE_SYM ? 2 : 4; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? IQ_OK : IQ_ERR_HIP;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Dispatch helpers: call f.template operator()<BITS, G>() for runtime (bits, group).
template <typename F>
int dispatch_bits_group(int bits, int group, F&& f) {
#define IQ_CASE(B_, G_) \
  if (bits == B_ && group == G_) return f.template operator()<B_, G_>();
  IQ_CASE(2, 32) IQ_CASE(2, 64) IQ_CASE(2, 128)
  IQ_CASE(3, 32) IQ_CASE(3, 64) IQ_CASE(3, 128)
  IQ_CASE(4, 32) IQ_CASE(4, 64) IQ_CASE(4, 128)
#undef IQ_CASE
  return IQ_ERR_BITS;
}

// dispatch_bits_group plus 1-bit (packed-store kernels only)
template <typename F>
int dispatch_store_bits_group(int bits, int group, F&& f) {
  if (bits == 1) {
    if (group == 32) return f.template operator()<1, 32>();
    if (group == 64) return f.template operator()<1, 64>();
    if (group == 128) return f.template operator()<1, 128>();
    return IQ_ERR_GROUP;
  }
  return dispatch_bits_group(bits, group, f);
}

}  // namespace iq
