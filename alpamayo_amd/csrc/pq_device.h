// Device helpers shared by the rotation, quantization and GEMM kernels.
#pragma once

#include "pq_common.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace pqd {

// ---------------------------------------------------------------------------
// int8 quantization: q = saturate(rne(v * inv)), inv = 127/absmax (0 for a zero row)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t quant1(float v, float inv) {
  float r = __builtin_rintf(v * inv);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return static_cast<uint32_t>(static_cast<int>(r)) & 0xffu;
}

__device__ __forceinline__ uint32_t quant4(float a, float b, float c, float d, float inv) {
  return quant1(a, inv) | (quant1(b, inv) << 8) | (quant1(c, inv) << 16) | (quant1(d, inv) << 24);
}

__device__ __forceinline__ float inv_scale(float absmax) { return absmax > 0.0f ? 127.0f / absmax : 0.0f; }

// ---------------------------------------------------------------------------
// int4 weight unpacking (layout in pq_gemm.hip): a dword of 8 codes -> two
// dwords of 4 signed bytes (q - z).  Every byte stays in [113, 143] before the
// xor, so no carry crosses a byte; the xor maps 128 + d to two's complement d.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t zero_bias(uint32_t z) { return 0x80808080u - z * 0x01010101u; }

__device__ __forceinline__ int unpack_lo(uint32_t w, uint32_t zb) {
  return static_cast<int>(((w & 0x0f0f0f0fu) + zb) ^ 0x80808080u);
}
__device__ __forceinline__ int unpack_hi(uint32_t w, uint32_t zb) {
  return static_cast<int>((((w >> 4) & 0x0f0f0f0fu) + zb) ^ 0x80808080u);
}

// 8 bytes of codes (16 consecutive k) -> 16 signed bytes in k order.
__device__ __forceinline__ v4i unpack16(uint32_t w0, uint32_t w1, uint32_t zb) {
  v4i r;
  r.x = unpack_lo(w0, zb);
  r.y = unpack_hi(w0, zb);
  r.z = unpack_lo(w1, zb);
  r.w = unpack_hi(w1, zb);
  return r;
}

__device__ __forceinline__ float meta_scale(uint32_t meta) {
  return pq_f16_to_f32(static_cast<uint16_t>(meta & 0xffffu));
}
__device__ __forceinline__ uint32_t meta_zero_bias(uint32_t meta) { return zero_bias((meta >> 16) & 0xfu); }

__device__ __forceinline__ float epilogue(float acc, float xscale, const void* bias, int bias_dtype, int n) {
  float v = acc * xscale;
  if (bias != nullptr) v = v + pq_load_dyn(bias, bias_dtype, n);
  return v;
}

// One Givens update in the fixed float32 form of the rotation kernels.
__device__ __forceinline__ void givens(float xi, float xj, float c, float s, float& ni, float& nj) {
  ni = fmaf(xi, c, xj * s);
  nj = fmaf(xj, c, -(xi * s));
}

}  // namespace pqd
