// Internal helpers shared by the libparoquant_hip.so translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/paroquant_hip.h"

namespace pq {

// Records the message returned by pq_last_error() (thread-local).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline bool aligned_to(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int dtype_size(int dt) {
  switch (dt) {
    case PQ_F32: return 4;
    case PQ_F16: return 2;
    case PQ_BF16: return 2;
    default: return 0;
  }
}

// Checks hipGetLastError() after a launch.
int launch_status(const char* what);

}  // namespace pq

#define PQ_REQUIRE(cond, code, ...)       \
  do {                                    \
    if (!(cond)) {                        \
      ::pq::set_error(__VA_ARGS__);       \
      return (code);                      \
    }                                     \
  } while (0)

// ---------------------------------------------------------------------------
// Device-side scalar conversions (gfx950 has native f16 and bf16 converts).
// ---------------------------------------------------------------------------

__device__ __forceinline__ float pq_bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bfloat16 bits (NaN stays NaN): one
// v_cvt_pk_bf16_f32 instead of the five-instruction integer rounding.
__device__ __forceinline__ uint16_t pq_f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float pq_f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return static_cast<float>(v);
}

// Round-to-nearest-even float -> fp16 bits.
__device__ __forceinline__ uint16_t pq_f32_to_f16(float f) {
  _Float16 v = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, v);
}

__device__ __forceinline__ float pq_round_f16(float f) { return pq_f16_to_f32(pq_f32_to_f16(f)); }

template <int DT>
__device__ __forceinline__ float pq_load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == PQ_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == PQ_F16) return pq_f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return pq_bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// Split form of pq_load_as_f32: the raw bits now, the conversion later (so a
// barrier can sit between issuing a load and consuming it).
template <int DT>
__device__ __forceinline__ uint32_t pq_load_raw(const void* p, int64_t i) {
  if constexpr (DT == PQ_F32) return static_cast<const uint32_t*>(p)[i];
  else return static_cast<const uint16_t*>(p)[i];
}

template <int DT>
__device__ __forceinline__ float pq_raw_to_f32(uint32_t r) {
  if constexpr (DT == PQ_F32) return __uint_as_float(r);
  else if constexpr (DT == PQ_F16) return pq_f16_to_f32(static_cast<uint16_t>(r));
  else return pq_bf16_to_f32(static_cast<uint16_t>(r));
}

template <int DT>
__device__ __forceinline__ void pq_store_from_f32(void* p, int64_t i, float v) {
  if constexpr (DT == PQ_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (DT == PQ_F16) static_cast<uint16_t*>(p)[i] = pq_f32_to_f16(v);
  else static_cast<uint16_t*>(p)[i] = pq_f32_to_bf16(v);
}

__device__ __forceinline__ float pq_load_dyn(const void* p, int dt, int64_t i) {
  if (dt == PQ_F32) return static_cast<const float*>(p)[i];
  if (dt == PQ_F16) return pq_f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return pq_bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ void pq_store_dyn(void* p, int dt, int64_t i, float v) {
  if (dt == PQ_F32) static_cast<float*>(p)[i] = v;
  else if (dt == PQ_F16) static_cast<uint16_t*>(p)[i] = pq_f32_to_f16(v);
  else static_cast<uint16_t*>(p)[i] = pq_f32_to_bf16(v);
}

// Wave64 maximum of unsigned integers, or of non-negative, non-NaN floats (an
// absmax: their bit patterns order like unsigned integers), the same in every
// lane.  Six v_max_u32 with DPP operands -- lane pairs and quads, mirrored
// half rows and rows of 16, then lane 15 of rows 0 / 2 into rows 1 / 3 and
// lane 31 into rows 2 / 3 -- leave the maximum in lane 63.  Lanes a step does
// not write take 0, which changes no maximum here.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t pq_dpp_umax(uint32_t u) {
  const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), CTRL, ROW_MASK, 0xf, false));
  return u > o ? u : o;
}
__device__ __forceinline__ uint32_t pq_wave_umax(uint32_t u) {
  u = pq_dpp_umax<0xb1, 0xf>(u);    // quad_perm [1, 0, 3, 2]
  u = pq_dpp_umax<0x4e, 0xf>(u);    // quad_perm [2, 3, 0, 1]
  u = pq_dpp_umax<0x141, 0xf>(u);   // row_half_mirror
  u = pq_dpp_umax<0x140, 0xf>(u);   // row_mirror
  u = pq_dpp_umax<0x142, 0xa>(u);   // row_bcast:15
  u = pq_dpp_umax<0x143, 0xc>(u);   // row_bcast:31
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 63));
}
__device__ __forceinline__ float pq_wave_max_nonneg(float v) { return __uint_as_float(pq_wave_umax(__float_as_uint(v))); }
// The same for N values, each step applied to all N before the next: the
// independent DPP operations fill each other's wait states.
template <int N>
__device__ __forceinline__ void pq_wave_umax_n(uint32_t (&u)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = pq_dpp_umax<0xb1, 0xf>(u[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = pq_dpp_umax<0x4e, 0xf>(u[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = pq_dpp_umax<0x141, 0xf>(u[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = pq_dpp_umax<0x140, 0xf>(u[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = pq_dpp_umax<0x142, 0xa>(u[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = pq_dpp_umax<0x143, 0xc>(u[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u[i]), 63));
}
