// Shared device helpers and host-side argument checks for the gfx950 GSA
// kernels.  Wave64 throughout: a "row group" is one DPP row of 16 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gsa_hip.h"

// Every product and sum rounds on its own (torch's rounding points); fused
// multiply-adds are written explicitly where wanted.
#pragma clang fp contract(off)

namespace gsa {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Never apply __builtin_bit_cast to one element of a vector (`v[i]` of a
// u32x4): this compiler reads element 0 for every i -- for a loop over
// `__builtin_bit_cast(bf16x2, v[i])` it loads a single dword.  Copy the
// element into a scalar first, or bit-cast whole vectors and arrays.

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// bf16 <-> fp32.  Rounding is round-to-nearest-even, the rounding torch uses
// when an fp32 intermediate is stored as bf16, done by the hardware convert
// (v_cvt_pk_bf16_f32; two values per instruction in pack_bf16); NaN stays
// NaN.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(f32_to_bf16_bits(f) << 16);
}
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Storage-type traits: how one 16-lane head slice of 8 elements is held.
template <typename T> struct Elem;
template <> struct Elem<uint16_t> {          // bf16 storage
  static constexpr bool kBf16 = true;
  __device__ static float rnd(float f) { return round_bf16(f); }
};
template <> struct Elem<float> {
  static constexpr bool kBf16 = false;
  __device__ static float rnd(float f) { return f; }
};

// Load / store 8 consecutive elements as fp32.
__device__ __forceinline__ void load8(const uint16_t* p, float (&x)[8]) {
  u32x4 r = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) { x[2 * i] = bf16lo(r[i]); x[2 * i + 1] = bf16hi(r[i]); }
}
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
  floatx4 a = *reinterpret_cast<const floatx4*>(p);
  floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) { x[i] = a[i]; x[4 + i] = b[i]; }
}
__device__ __forceinline__ void store8(uint16_t* p, const float (&x)[8]) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16(x[2 * i], x[2 * i + 1]);
  *reinterpret_cast<u32x4*>(p) = r;
}
__device__ __forceinline__ void store8(float* p, const float (&x)[8]) {
  floatx4 a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) { a[i] = x[i]; b[i] = x[4 + i]; }
  *reinterpret_cast<floatx4*>(p) = a;
  *reinterpret_cast<floatx4*>(p + 4) = b;
}

// sigmoid(x) = 1 / (1 + 2^(-x*log2 e)), hardware exp2 and reciprocal
// (about 1 ulp each).  exp2 overflow gives +inf and the reciprocal 0, the
// correct limit.
__device__ __forceinline__ float sigmoidf_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// ---------------------------------------------------------------------------
// Cross-lane helpers (DPP within a 16-lane row; ballots over the wave).
// ---------------------------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
// row_ror:n is DPP control 0x120 + n.  Rotations make every lane of the row
// hold the full reduction.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0x128>(v);
  v += dpp<0x124>(v);
  v += dpp<0x122>(v);
  v += dpp<0x121>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0x128>(v));
  v = fmaxf(v, dpp<0x124>(v));
  v = fmaxf(v, dpp<0x122>(v));
  v = fmaxf(v, dpp<0x121>(v));
  return v;
}
// Value of lane (i + 8) mod 16 within the row.
__device__ __forceinline__ float row16_swap8(float v) { return dpp<0x128>(v); }

__device__ __forceinline__ int lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}
__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }
// Number of set bits of `mask` below the calling lane.
__device__ __forceinline__ int count_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// RoPE on one lane's 8 elements: x*cos + rotate_half(x)*sin, where
// rotate_half takes element i+64 (negated) for i < 64 and element i-64 for
// i >= 64 -- the value held by lane (li +/- 8) of the same 16-lane row.
template <typename T>
__device__ __forceinline__ void rope8(float (&x)[8], const float (&c)[8], const float (&s)[8], int li) {
  float partner[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) partner[i] = row16_swap8(x[i]);
  const float sign = li < 8 ? -1.f : 1.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = Elem<T>::rnd(x[i] * c[i]);
    const float r = Elem<T>::rnd((sign * partner[i]) * s[i]);
    x[i] = Elem<T>::rnd(a + r);
  }
}

// Monotone map of an fp32 score to uint32: a > b  <=>  key(a) > key(b).
// -inf is first replaced by -1e9 (the selector's fill value) and every NaN
// ranks above +inf, as torch.topk orders them.
__device__ __forceinline__ uint32_t score_key(float s) {
  if (s == -__builtin_inff()) s = -1e9f;
  uint32_t u = __float_as_uint(s);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

}  // namespace gsa

// ---------------------------------------------------------------------------
// Host-side checks shared by the entry points.
// ---------------------------------------------------------------------------
namespace gsa_host {

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline int dtype_size(int dtype) {
  return dtype == GSA_DTYPE_BF16 ? 2 : (dtype == GSA_DTYPE_F32 ? 4 : 0);
}
// A [.., T, H*d] tensor read 16 bytes at a time: base and strides must keep
// every 8-element (bf16) or 4-element (fp32) group 16-byte aligned.
inline bool vec_ok(const void* p, int64_t sb, int64_t st, int dtype) {
  const int64_t grp = dtype == GSA_DTYPE_BF16 ? 8 : 4;
  return aligned(p, 16) && (sb % grp) == 0 && (st % grp) == 0;
}
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? GSA_OK : -static_cast<int>(e);
}

// Variance-based per-row k from per-row variances var[0..n) (indexer.hip):
// k = min(clamp(floor(k_base * max(mean(var),1e-6) / max(var,1e-6)), k_min, k_max), k_cap).
// One launch on `stream`; returns launch_status().
int launch_adaptive_k(const float* var, int n, int k_base, int k_min, int k_max, int k_cap, int32_t* k_rows,
                      hipStream_t stream);

}  // namespace gsa_host
