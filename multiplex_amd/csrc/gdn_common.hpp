// Shared device helpers and host-side status handling for libgdn (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "../../include/gdn.h"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
// Native 128-bit integer vector: plain loads/stores, unlike HIP's uint4
// struct, whose copies lower to memcpy and keep values out of registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- dtypes

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN): gfx950's
// v_cvt_pk_bf16_f32, one instruction, no branches.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two floats -> packed bf16 pair (low half = a), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

// Two floats -> packed f16 pair (low half = a).
__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), f16x2_t));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Scalar load of a runtime-typed element (gates, per-head parameters).  Two
// unconditional 16-bit loads -- the halves of an fp32 element, or the 16-bit
// element twice -- combined by selects: a per-dtype branch around the load
// would force a wait for it (and for every load issued before it) right there.
__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  const bool f32 = dt == GDN_DTYPE_F32;
  const uint16_t* e = static_cast<const uint16_t*>(p) + (f32 ? 2 * i : i);
  const uint16_t lo = e[0];
  const uint16_t hi = e[f32 ? 1 : 0];
  const float as_f32 = __uint_as_float((static_cast<uint32_t>(hi) << 16) | lo);
  const float as_16 = dt == GDN_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
  return f32 ? as_f32 : as_16;
}

// Compile-time typed I/O for q/k/v/y: DT is one of the GDN_DTYPE_* codes.
template <int DT>
struct IO;

// raw4 / raw1: the loaded bits before conversion (load4_raw, cvt4), for a
// caller that issues many loads before it uses any of them.
template <>
struct IO<GDN_DTYPE_F32> {
  using elem = float;
  using raw4 = f32x4;
  using raw1 = float;
  __device__ __forceinline__ static raw4 load4_raw(const void* p, int64_t i) {
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  }
  __device__ __forceinline__ static f32x4 cvt4(raw4 h) { return h; }
  __device__ __forceinline__ static raw1 load1_raw(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
  __device__ __forceinline__ static float cvt1(raw1 h) { return h; }
  __device__ __forceinline__ static f32x4 load4(const void* p, int64_t i) {
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  }
  __device__ __forceinline__ static float load1(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
  __device__ __forceinline__ static void store1(void* p, int64_t i, float x) {
    static_cast<float*>(p)[i] = x;
  }
  __device__ __forceinline__ static void store2(void* p, int64_t i, float x0, float x1) {
    f32x2 v = {x0, x1};
    *reinterpret_cast<f32x2*>(static_cast<float*>(p) + i) = v;
  }
  __device__ __forceinline__ static f32x2 load2(const void* p, int64_t i) {
    return *reinterpret_cast<const f32x2*>(static_cast<const float*>(p) + i);
  }
};

template <>
struct IO<GDN_DTYPE_BF16> {
  using elem = uint16_t;
  using raw4 = u16x4;
  using raw1 = uint16_t;
  __device__ __forceinline__ static raw4 load4_raw(const void* p, int64_t i) {
    return *reinterpret_cast<const u16x4*>(static_cast<const uint16_t*>(p) + i);
  }
  __device__ __forceinline__ static f32x4 cvt4(raw4 h) {
    return f32x4{bf16_to_f32(h.x), bf16_to_f32(h.y), bf16_to_f32(h.z), bf16_to_f32(h.w)};
  }
  __device__ __forceinline__ static raw1 load1_raw(const void* p, int64_t i) {
    return static_cast<const uint16_t*>(p)[i];
  }
  __device__ __forceinline__ static float cvt1(raw1 h) { return bf16_to_f32(h); }
  __device__ __forceinline__ static f32x4 load4(const void* p, int64_t i) {
    u16x4 h = *reinterpret_cast<const u16x4*>(static_cast<const uint16_t*>(p) + i);
    return f32x4{bf16_to_f32(h.x), bf16_to_f32(h.y), bf16_to_f32(h.z), bf16_to_f32(h.w)};
  }
  __device__ __forceinline__ static float load1(const void* p, int64_t i) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ __forceinline__ static void store1(void* p, int64_t i, float x) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(x);
  }
  __device__ __forceinline__ static void store2(void* p, int64_t i, float x0, float x1) {
    u16x2 h = {f32_to_bf16(x0), f32_to_bf16(x1)};
    *reinterpret_cast<u16x2*>(static_cast<uint16_t*>(p) + i) = h;
  }
  __device__ __forceinline__ static f32x2 load2(const void* p, int64_t i) {
    u16x2 h = *reinterpret_cast<const u16x2*>(static_cast<const uint16_t*>(p) + i);
    return f32x2{bf16_to_f32(h.x), bf16_to_f32(h.y)};
  }
};

template <>
struct IO<GDN_DTYPE_F16> {
  using elem = uint16_t;
  using raw4 = u16x4;
  using raw1 = uint16_t;
  __device__ __forceinline__ static raw4 load4_raw(const void* p, int64_t i) {
    return *reinterpret_cast<const u16x4*>(static_cast<const uint16_t*>(p) + i);
  }
  __device__ __forceinline__ static f32x4 cvt4(raw4 h) {
    return f32x4{f16_to_f32(h.x), f16_to_f32(h.y), f16_to_f32(h.z), f16_to_f32(h.w)};
  }
  __device__ __forceinline__ static raw1 load1_raw(const void* p, int64_t i) {
    return static_cast<const uint16_t*>(p)[i];
  }
  __device__ __forceinline__ static float cvt1(raw1 h) { return f16_to_f32(h); }
  __device__ __forceinline__ static f32x4 load4(const void* p, int64_t i) {
    u16x4 h = *reinterpret_cast<const u16x4*>(static_cast<const uint16_t*>(p) + i);
    return f32x4{f16_to_f32(h.x), f16_to_f32(h.y), f16_to_f32(h.z), f16_to_f32(h.w)};
  }
  __device__ __forceinline__ static float load1(const void* p, int64_t i) {
    return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ __forceinline__ static void store1(void* p, int64_t i, float x) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16(x);
  }
  __device__ __forceinline__ static void store2(void* p, int64_t i, float x0, float x1) {
    u16x2 h = {f32_to_f16(x0), f32_to_f16(x1)};
    *reinterpret_cast<u16x2*>(static_cast<uint16_t*>(p) + i) = h;
  }
  __device__ __forceinline__ static f32x2 load2(const void* p, int64_t i) {
    u16x2 h = *reinterpret_cast<const u16x2*>(static_cast<const uint16_t*>(p) + i);
    return f32x2{f16_to_f32(h.x), f16_to_f32(h.y)};
  }
};

// ------------------------------------------------------------ gate math

// The gates are transformed once per (token, head) and wave, where the
// library's correctly rounded expf / log1pf and IEEE division cost ~150
// instructions: the hardware exp2, log2 and reciprocal (v_exp_f32,
// v_log_f32, v_rcp_f32, each within ~1 ulp) do it in ~20.  e^x = 2^(x log2 e)
// has a relative error of ~|x| 2^-24, so g keeps ~1e-6 relative accuracy
// wherever it is not negligibly small, and beta ~1e-7.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// softplus(x) = log(1 + e^x) = max(x, 0) + log1p(u), u = e^-|x| in (0, 1],
// stable for all x.  log1p(u) = log(w) u / (w - 1) with w = 1 + u rounded
// (Goldberg's correction of the rounding in w; u itself when w == 1).
__device__ __forceinline__ float softplus_f(float x) {
  const float u = exp_fast(-fabsf(x));
  const float w = 1.0f + u;
  const float lp = __builtin_amdgcn_logf(w) * 0.693147180559945309f * (u * __builtin_amdgcn_rcpf(w - 1.0f));
  return fmaxf(x, 0.0f) + (w == 1.0f ? u : lp);
}

__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_fast(-x)); }

// Gate encodings.  GF_ANY reads runtime dtypes (and GDN_GATES_PRE); the
// typed formats cover the usual layouts with plain typed loads, which keeps
// the loads free of per-dtype branches (and of the waits those force).
enum GateFormat : int {
  GF_ANY = 0,     // any dtypes, raw or pre-transformed gates
  GF_IO_F32 = 1,  // raw: a, b in the q/k/v dtype; A_log, dt_bias fp32
  GF_IO_IO = 2,   // raw: a, b, A_log, dt_bias all in the q/k/v dtype
};

struct GateArgs {
  const void* gx;  // a or g
  const void* gy;  // b or beta
  const void* A_log;
  const void* dt_bias;
  int64_t ld;      // elements from one token's gate row to the next (Hv when packed)
  int mode, gdt, pdt;
};

// Raw gate inputs of token index gi (= token * Hv + hv).
template <int GF, int DT>
__device__ __forceinline__ void gate_load(const GateArgs& ga, int64_t gi, float& x, float& y) {
  if constexpr (GF == GF_ANY) {
    x = load_any(ga.gx, ga.gdt, gi);
    y = load_any(ga.gy, ga.gdt, gi);
  } else {
    x = IO<DT>::load1(ga.gx, gi);
    y = IO<DT>::load1(ga.gy, gi);
  }
}

// Per-head parameters (raw mode): A_log[hv] (0 for pre-transformed gates)
// and dt_bias[hv], loads only.  The caller applies exp(A_log) at its use, so
// nothing waits here for the loads while it issues more.
template <int GF, int DT>
__device__ __forceinline__ void param_load_raw(const GateArgs& ga, int hv, float& al, float& db) {
  if (GF == GF_ANY && ga.mode == GDN_GATES_PRE) {  // typed formats are raw gates
    al = 0.0f;
    db = 0.0f;
    return;
  }
  if constexpr (GF == GF_ANY) {
    al = load_any(ga.A_log, ga.pdt, hv);
    db = load_any(ga.dt_bias, ga.pdt, hv);
  } else if constexpr (GF == GF_IO_F32) {
    al = static_cast<const float*>(ga.A_log)[hv];
    db = static_cast<const float*>(ga.dt_bias)[hv];
  } else {
    al = IO<DT>::load1(ga.A_log, hv);
    db = IO<DT>::load1(ga.dt_bias, hv);
  }
}

// g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b)  (raw mode).
template <int GF>
__device__ __forceinline__ void gate_transform(int mode, float x, float y, float ea, float db, float& g,
                                               float& beta) {
  if (GF == GF_ANY && mode == GDN_GATES_PRE) {
    g = x;
    beta = y;
  } else {
    g = exp_fast(-ea * softplus_f(x + db));
    beta = sigmoid_f(y);
  }
}

// Raw gate inputs of one token, loads only: the 16-bit halves of a (or g),
// b (or beta) and the head's A_log and dt_bias, as load_any reads them.  Every
// load is unconditional (pre-transformed gates read gx in place of the
// absent parameters) and nothing is converted here, so a caller can issue
// more loads before anything waits for these.
struct GateRaw {
  uint32_t lo[4], hi[4];  // 16-bit halves, one per register (no packing, which would wait)
};
__device__ __forceinline__ void load_raw_any(const void* p, int dt, int64_t i, uint32_t& lo, uint32_t& hi) {
  const bool f32 = dt == GDN_DTYPE_F32;
  const uint16_t* e = static_cast<const uint16_t*>(p) + (f32 ? 2 * i : i);
  lo = e[0];
  hi = e[f32 ? 1 : 0];
}
__device__ __forceinline__ float raw_any_value(int dt, uint32_t lo, uint32_t hi) {
  const float as_f32 = __uint_as_float((hi << 16) | lo);
  const uint16_t h = static_cast<uint16_t>(lo);
  const float as_16 = dt == GDN_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
  return dt == GDN_DTYPE_F32 ? as_f32 : as_16;
}
__device__ __forceinline__ GateRaw load_gate_raw(const GateArgs& ga, int64_t gi, int hv) {
  const bool raw = ga.mode != GDN_GATES_PRE;
  GateRaw r;
  load_raw_any(ga.gx, ga.gdt, gi, r.lo[0], r.hi[0]);
  load_raw_any(ga.gy, ga.gdt, gi, r.lo[1], r.hi[1]);
  load_raw_any(raw ? ga.A_log : ga.gx, raw ? ga.pdt : ga.gdt, raw ? hv : gi, r.lo[2], r.hi[2]);
  load_raw_any(raw ? ga.dt_bias : ga.gx, raw ? ga.pdt : ga.gdt, raw ? hv : gi, r.lo[3], r.hi[3]);
  return r;
}

// Log decay (chunked prefill): -exp(A_log) softplus(a + dt_bias), or log g.
__device__ __forceinline__ void log_gates(const GateArgs& ga, const GateRaw& r, float& logg, float& beta) {
  const float x = raw_any_value(ga.gdt, r.lo[0], r.hi[0]);
  const float y = raw_any_value(ga.gdt, r.lo[1], r.hi[1]);
  if (ga.mode == GDN_GATES_PRE) {
    logg = logf(x);
    beta = y;
  } else {
    const float al = raw_any_value(ga.pdt, r.lo[2], r.hi[2]);
    const float db = raw_any_value(ga.pdt, r.lo[3], r.hi[3]);
    logg = -exp_fast(al) * softplus_f(x + db);
    beta = sigmoid_f(y);
  }
}

// ------------------------------------------------------------- unrolling

// static_for<N>(f) calls f(std::integral_constant<int, i>) for i = 0..N-1.
// Indexing register-staged arrays with these constants keeps them in VGPRs:
// the alloca promotion pass runs before loop unrolling, and a loop index
// would make it move such arrays to LDS or scratch.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_impl(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_impl<I + 1, N>(f);
  }
}

template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<0, N>(f);
}

// ------------------------------------------------------- cross-lane sums

// DPP lane permutations inside a 16-lane row (gfx9 encodings).
#define GDN_DPP_QUAD_XOR1 0xB1  // quad_perm [1,0,3,2]
#define GDN_DPP_QUAD_XOR2 0x4E  // quad_perm [2,3,0,1]
#define GDN_DPP_HALF_MIRROR 0x141
#define GDN_DPP_ROW_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of 8 lanes; every lane of the group gets the sum.
__device__ __forceinline__ float sum8(float x) {
  x += dpp_f<GDN_DPP_QUAD_XOR1>(x);
  x += dpp_f<GDN_DPP_QUAD_XOR2>(x);
  x += dpp_f<GDN_DPP_HALF_MIRROR>(x);
  return x;
}

// Sum over aligned groups of 16 lanes.
__device__ __forceinline__ float sum16(float x) {
  x = sum8(x);
  x += dpp_f<GDN_DPP_ROW_MIRROR>(x);
  return x;
}

// Sum over the whole 64-lane wavefront; every lane gets the sum.
__device__ __forceinline__ float wave_sum(float x) {
  x = sum16(x);
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

// ------------------------------------------- 8-element row slices

constexpr int CPL = 8;  // channels per lane

// Raw 8-channel slice of a row as loaded (converted at its use, so the loads
// of a whole run can be in flight at once).
template <int DT>
struct Raw8 {
  u32x4 v;  // 8 x 16-bit
};
template <>
struct Raw8<GDN_DTYPE_F32> {
  f32x4 a, b;
};

template <int DT>
__device__ __forceinline__ Raw8<DT> load_raw8(const void* base, int64_t i) {
  Raw8<DT> r;
  if constexpr (DT == GDN_DTYPE_F32) {
    r.a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + i);
    r.b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + i + 4);
  } else {
    r.v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
  }
  return r;
}

template <int DT>
__device__ __forceinline__ void unpack8(const Raw8<DT>& r, float (&x)[CPL]) {
  if constexpr (DT == GDN_DTYPE_F32) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[k] = r.a[k];
      x[4 + k] = r.b[k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == GDN_DTYPE_BF16) {
        x[2 * k] = __uint_as_float(r.v[k] << 16);
        x[2 * k + 1] = __uint_as_float(r.v[k] & 0xffff0000u);
      } else {
        x[2 * k] = f16_to_f32(static_cast<uint16_t>(r.v[k] & 0xffffu));
        x[2 * k + 1] = f16_to_f32(static_cast<uint16_t>(r.v[k] >> 16));
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t i, const float (&x)[CPL]) {
  if constexpr (DT == GDN_DTYPE_F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(base) + i) = f32x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<f32x4*>(static_cast<float*>(base) + i + 4) = f32x4{x[4], x[5], x[6], x[7]};
  } else {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      v[k] = DT == GDN_DTYPE_BF16 ? pk_bf16(x[2 * k], x[2 * k + 1]) : pk_f16(x[2 * k], x[2 * k + 1]);
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + i) = v;
  }
}

// Sum over the LPH lanes of a row (aligned lane groups of 8, 16 or 32).
template <int LPH>
__device__ __forceinline__ float head_sum(float x) {
  if constexpr (LPH == 8) {
    return sum8(x);
  } else if constexpr (LPH == 16) {
    return sum16(x);
  } else {
    x = sum16(x);
    return x + __shfl_xor(x, 16, 64);
  }
}

// SiLU x * sigmoid(x) = x / (1 + 2^(-x log2 e)) on the hardware exp2 and
// reciprocal (about 1 ulp each; the result is rounded to the io dtype).  For
// x -> -inf the denominator overflows to inf and the result is -0.
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// ------------------------------------------- causal conv on bf16 pairs
//
// With bf16 inputs and bf16 taps the 4-tap causal conv runs on packed pairs:
// for channel c at token t, p(t) = (x_{t-1}[c], x_t[c]) (earlier token in the
// low half), and
//   acc = dot(w23, p(t)) + dot(w01, p(t - 2)),   w01 = (w0, w1), w23 = (w2, w3)
// on v_dot2c_f32_bf16 (exact bf16 products, fp32 accumulation).  One byte
// permute forms a pair from two rows and serves two tokens' dots, the taps
// are used as loaded, and nothing is unpacked to fp32 before the conv.

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// A row slice (8 16-bit channels) or zeros: a masked or absent row.  Component
// by component (a ternary on the whole vector would be lowered through memory).
__device__ __forceinline__ u32x4 row_or_zero(bool keep, const u32x4& r) {
  return u32x4{keep ? r.x : 0u, keep ? r.y : 0u, keep ? r.z : 0u, keep ? r.w : 0u};
}

// pr[c] = (prev[c], cur[c]) for the 8 channels of two consecutive rows.
// v_perm_b32 selects bytes of {cur, prev} (prev = bytes 0-3, cur = 4-7).
__device__ __forceinline__ void row_pairs(const u32x4& prev, const u32x4& cur, uint32_t (&pr)[CPL]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    pr[2 * k] = __builtin_amdgcn_perm(cur[k], prev[k], 0x05040100u);      // low halves
    pr[2 * k + 1] = __builtin_amdgcn_perm(cur[k], prev[k], 0x07060302u);  // high halves
  }
}

// The conv of one channel from its taps (w01, w23 as loaded: 4 consecutive
// bf16 taps per channel) and the pairs p(t - 2), p(t).
__device__ __forceinline__ float conv_pairs(uint32_t w01, uint32_t w23, uint32_t p_m2, uint32_t p_0) {
  const float a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w23), __builtin_bit_cast(bf16x2_t, p_0),
                                                  0.0f, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w01), __builtin_bit_cast(bf16x2_t, p_m2), a,
                                         false);
}

}  // namespace gdn

// ----------------------------------------------------- host-side status

namespace gdn_host {

// Records a message for gdn_last_error() and returns the status code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch.
int check_launch(const char* what);

inline bool dtype_ok(int dt) {
  return dt == GDN_DTYPE_F32 || dt == GDN_DTYPE_BF16 || dt == GDN_DTYPE_F16;
}

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

}  // namespace gdn_host
