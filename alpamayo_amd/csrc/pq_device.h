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

// The code in the low byte of the result (the other bytes are not part of
// it), from a product p = v * inv that is already formed.  Every caller
// scales by 127 / absmax of the very values it quantizes, so p lies in
// [-127, 127] up to two roundings; adding 1.5 * 2^23 lands in [2^23, 2^24),
// where float32 spacing is 1, so the sum is rne(p) + 1.5 * 2^23 and its low
// byte is rne(p) in two's complement -- the code of rne, clamp and convert,
// in two instructions.  The max keeps the clamp's answer for a NaN product
// (code -128).
__device__ __forceinline__ uint32_t quant_scaled(float p) {
  return __float_as_uint(fmaxf(p, -128.0f) + 12582912.0f);
}

// Low bytes of four codes, a in byte 0: three byte permutes.
__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

__device__ __forceinline__ uint32_t quant4(float a, float b, float c, float d, float inv) {
  return pack4(quant_scaled(a * inv), quant_scaled(b * inv), quant_scaled(c * inv), quant_scaled(d * inv));
}

// Four codes from two dwords of fp16 values.  fma(h, inv, +0) differs from
// h * inv only in the sign of a zero product, which rounds to the same code;
// the form lets the fp16 -> float32 conversion ride in v_fma_mix_f32.
__device__ __forceinline__ float mul_f16(uint32_t w, bool hi, float inv) {
  const _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? w >> 16 : w & 0xffffu));
  return __builtin_fmaf(static_cast<float>(h), inv, 0.0f);
}

__device__ __forceinline__ uint32_t quant4_f16(uint32_t w01, uint32_t w23, float inv) {
  return pack4(quant_scaled(mul_f16(w01, false, inv)), quant_scaled(mul_f16(w01, true, inv)),
               quant_scaled(mul_f16(w23, false, inv)), quant_scaled(mul_f16(w23, true, inv)));
}

__device__ __forceinline__ float inv_scale(float absmax) { return absmax > 0.0f ? 127.0f / absmax : 0.0f; }

// -0.0f that the compiler cannot see through (it would fold an fma with a
// constant -0 addend back into a multiply).
__device__ __forceinline__ float opaque_neg_zero() {
  float nz;
  asm volatile("s_mov_b32 %0, 0x80000000" : "=s"(nz));
  return nz;
}

// v rounded to fp16, times s: one v_cvt_f16_f32 and one v_fma_mix_f32.
// fma(h, s, -0) equals the product h * s bit for bit (adding -0 changes no
// rounded product, a -0 product included); nz is opaque_neg_zero().
__device__ __forceinline__ float f16_scaled(float v, float s, float nz) {
  return __builtin_fmaf(static_cast<float>(static_cast<_Float16>(v)), s, nz);
}

// Two floats -> a dword of two fp16 (a in the low half), rounded to nearest
// even: one v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const f2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
}

// A dword of two fp16 taken from an array of fp16 pairs: number i0 in the low
// half, number i1 in the high half (fp16 number i of d is half i & 1 of
// d[i >> 1]).  One byte permute when i0, i1 are known at compile time.
template <int N>
__device__ __forceinline__ uint32_t f16_pair(const uint32_t (&d)[N], int i0, int i1) {
  const uint32_t sel = ((i0 & 1) ? 0x0302u : 0x0100u) | ((i1 & 1) ? 0x07060000u : 0x05040000u);
  return __builtin_amdgcn_perm(d[i1 >> 1], d[i0 >> 1], sel);
}

// N floats -> N fp16 stored side by side at p (aligned to 2 N bytes).
template <int N>
__device__ __forceinline__ void store_f16xn(uint16_t* p, const float (&v)[N]) {
  static_assert(N >= 1 && N <= 8 && N != 5 && N != 7, "1, 2, 3, 4, 6 or 8 values");
  if constexpr (N == 1) {
    *p = pq_f32_to_f16(v[0]);
  } else if constexpr (N == 3) {   // 2-byte aligned
    p[0] = pq_f32_to_f16(v[0]);
    p[1] = pq_f32_to_f16(v[1]);
    p[2] = pq_f32_to_f16(v[2]);
  } else if constexpr (N == 6) {   // 4-byte aligned
    uint32_t* q = reinterpret_cast<uint32_t*>(p);
    q[0] = pk_f16(v[0], v[1]);
    q[1] = pk_f16(v[2], v[3]);
    q[2] = pk_f16(v[4], v[5]);
  } else {
    uint32_t w[N / 2];
#pragma unroll
    for (int q = 0; q < N / 2; ++q) w[q] = pk_f16(v[2 * q], v[2 * q + 1]);
    if constexpr (N == 2) *reinterpret_cast<uint32_t*>(p) = w[0];
    else if constexpr (N == 4) *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---------------------------------------------------------------------------
// int4 weight unpacking (layout in pq_gemm.hip): a dword of 8 codes -> two
// dwords of 4 signed bytes (q - z).  Every byte stays in [113, 143] before the
// xor, so no carry crosses a byte; the xor maps 128 + d to two's complement d.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t zero_bias(uint32_t z) {
  return __builtin_amdgcn_perm(0u, 0x80u - z, 0u);   // 0x80 - z in every byte (= 0x80808080 - z * 0x01010101)
}

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

// 8 bytes of codes (16 consecutive k) -> 16 unsigned bytes q in k order (the
// zero point is applied separately, see meta_neg_zero4).
__device__ __forceinline__ v4i nibbles16(uint32_t w0, uint32_t w1) {
  v4i r;
  r.x = static_cast<int>(w0 & 0x0f0f0f0fu);
  r.y = static_cast<int>((w0 >> 4) & 0x0f0f0f0fu);
  r.z = static_cast<int>(w1 & 0x0f0f0f0fu);
  r.w = static_cast<int>((w1 >> 4) & 0x0f0f0f0fu);
  return r;
}

// Four bytes of -z (z = the zero point in meta bits 16..19): as an MFMA B
// operand it adds -z * sum_k a[m, k] to a column's accumulator, which turns
// sum_k a * q into sum_k a * (q - z) exactly.
__device__ __forceinline__ uint32_t meta_neg_zero4(uint32_t meta) {
  const uint32_t nz = 0u - ((meta >> 16) & 0xfu);   // byte 0 = (256 - z) mod 256
  return __builtin_amdgcn_perm(0u, nz, 0u);          // replicate byte 0
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

// ---------------------------------------------------------------------------
// Register-chain rotation of one 128-channel group by one wave (operands
// built by pq_rotation_pack):
//   rot_idx [G][64][KP/2] uint32: word 0 = Af | Bf << 8 | init << 16,
//                                 byte 4 + r = src | flag << 7 (layer r)
//   rot_cs  [G][64][KP][2] float: (cos, +-sin) of the lane's pair in layer r
// Lane l loads channels l and l+64 into slots (a, b), swapped when init is
// set.  Before layer r it fetches slot a of lane src (ds_bpermute) and puts
// the value into slot a when flag is set (else into slot b), keeping its old
// slot b in the other slot; then a' = fma(a, c, b*s), b' = fma(b, c, -(a*s)).
// After the last layer slot a holds channel Af and slot b channel Bf.
// ---------------------------------------------------------------------------
template <int KP>
struct RotLane {
  uint32_t w[KP / 2];
  float cs[2 * KP];
};

// g is wave-uniform.  SADDR: the group's base address is scalar and the
// lane's part a 32-bit offset, so the loads take the saddr + voffset form with
// no per-lane 64-bit address arithmetic (the compiler keeps the two offsets
// in four VGPRs); otherwise the per-lane address is formed at each call (the
// row kernel, whose six-row instance must stay within 128 VGPRs to keep two
// workgroups per CU).
template <int KP, bool SADDR = true>
__device__ __forceinline__ void load_rot_lane(const uint32_t* __restrict__ rot_idx, const float* __restrict__ rot_cs,
                                              int g, int lane, RotLane<KP>& p) {
  const int64_t o = static_cast<int64_t>(g) * 64 + lane;
  const uint32_t* gi = rot_idx + static_cast<int64_t>(g) * 64 * (KP / 2);
  const float* gc = rot_cs + static_cast<int64_t>(g) * 64 * (2 * KP);
  const uint4* wi = SADDR ? reinterpret_cast<const uint4*>(gi + lane * (KP / 2))
                          : reinterpret_cast<const uint4*>(rot_idx + o * (KP / 2));
#pragma unroll
  for (int q = 0; q < KP / 8; ++q) {
    const uint4 v = wi[q];
    p.w[4 * q] = v.x;
    p.w[4 * q + 1] = v.y;
    p.w[4 * q + 2] = v.z;
    p.w[4 * q + 3] = v.w;
  }
  const float4* c = SADDR ? reinterpret_cast<const float4*>(gc + lane * (2 * KP))
                          : reinterpret_cast<const float4*>(rot_cs + o * (2 * KP));
#pragma unroll
  for (int q = 0; q < KP / 2; ++q) {
    const float4 v = c[q];
    p.cs[4 * q] = v.x;
    p.cs[4 * q + 1] = v.y;
    p.cs[4 * q + 2] = v.z;
    p.cs[4 * q + 3] = v.w;
  }
}

// Ties the lane's operands to this point of the program: the compiler
// otherwise sinks the load of a layer's cos/sin into that layer's
// `layer < krot` branch, where it costs a round trip of its own.
template <int KP>
__device__ __forceinline__ void pin_rot_lane(RotLane<KP>& p) {
#pragma unroll
  for (int i = 0; i < 2 * KP; ++i) asm volatile("" : "+v"(p.cs[i]));
#pragma unroll
  for (int i = 0; i < KP / 2; ++i) asm volatile("" : "+v"(p.w[i]));
}

template <int KP>
__device__ __forceinline__ bool rot_init_swapped(const RotLane<KP>& p) { return (p.w[0] >> 16) & 1u; }
template <int KP>
__device__ __forceinline__ int rot_final_a(const RotLane<KP>& p) { return p.w[0] & 127u; }
template <int KP>
__device__ __forceinline__ int rot_final_b(const RotLane<KP>& p) { return (p.w[0] >> 8) & 127u; }

// Layer r (compile-time after unrolling) for N value pairs sharing the lane's operands.
template <int KP, int N>
__device__ __forceinline__ void rot_layer(const RotLane<KP>& p, int r, float (&a)[N], float (&b)[N]) {
  const uint32_t st = (p.w[(4 + r) >> 2] >> (8 * ((4 + r) & 3))) & 0xffu;
  const int addr = static_cast<int>(st & 63u) << 2;
  const bool fl = (st & 128u) != 0;
#pragma unroll
  for (int n = 0; n < N; ++n) {
    const float recv = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(a[n])));
    const float keep = b[n];
    a[n] = fl ? recv : keep;
    b[n] = fl ? keep : recv;
  }
  const float c = p.cs[2 * r], s = p.cs[2 * r + 1];
#pragma unroll
  for (int n = 0; n < N; ++n) {
    float na, nb;
    givens(a[n], b[n], c, s, na, nb);
    a[n] = na;
    b[n] = nb;
  }
}

// All Givens layers of one group.  With krot == KP (the usual KROT) the
// layers run as one straight-line block; with fewer, each layer sits behind
// a uniform branch on its index, whose condition the compiler evaluates with
// VALU instructions in every layer (6-9 % of the row kernel's time).
template <int KP, int N>
__device__ __forceinline__ void rot_layers(const RotLane<KP>& p, int krot, float (&a)[N], float (&b)[N]) {
  if (krot == KP) {
#pragma unroll
    for (int k = 0; k < KP; ++k) rot_layer<KP, N>(p, k, a, b);
  } else {
#pragma unroll
    for (int k = 0; k < KP; ++k)
      if (k < krot) rot_layer<KP, N>(p, k, a, b);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm prologue (reference: Qwen3VLTextRMSNorm.forward,
// src/alpamayo_r1/models/qwen3_vl/modeling_qwen3_vl.py:354-359):
//   s = x (+ res), rounded to the activation dtype;
//   h = round(w * round(s * rsqrt(mean(s^2) + eps))).
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float round_to_dt(float v) {
  if constexpr (DT == PQ_F16) return pq_round_f16(v);
  else if constexpr (DT == PQ_BF16) return pq_bf16_to_f32(pq_f32_to_bf16(v));
  else return v;
}

// Eight consecutive elements of a row as raw bits: one 16-byte load (two for
// float32).
template <int DT>
struct Raw8 {
  uint4 a;
  uint4 b;   // float32 only
};

template <int DT>
__device__ __forceinline__ Raw8<DT> load8_raw(const void* base, int64_t elem) {
  Raw8<DT> r;
  if constexpr (DT == PQ_F32) {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(base) + elem);
    r.a = p[0];
    r.b = p[1];
  } else {
    r.a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem);
    r.b = make_uint4(0u, 0u, 0u, 0u);
  }
  return r;
}

template <int DT>
__device__ __forceinline__ void unpack8(const Raw8<DT>& r, float f[8]) {
  if constexpr (DT == PQ_F32) {
    f[0] = __uint_as_float(r.a.x); f[1] = __uint_as_float(r.a.y); f[2] = __uint_as_float(r.a.z);
    f[3] = __uint_as_float(r.a.w); f[4] = __uint_as_float(r.b.x); f[5] = __uint_as_float(r.b.y);
    f[6] = __uint_as_float(r.b.z); f[7] = __uint_as_float(r.b.w);
  } else {
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = pq_raw_to_f32<DT>(w[e] & 0xffffu);
      f[2 * e + 1] = pq_raw_to_f32<DT>(w[e] >> 16);
    }
  }
}

template <int DT>
__device__ __forceinline__ void load8_as_f32(const void* base, int64_t elem, float f[8]) {
  unpack8<DT>(load8_raw<DT>(base, elem), f);
}

// Wave64 sum through xor butterflies: every lane ends with the same value
// (the same additions in the same association, only commuted).  (A DPP
// version gathers the sum in another association; against the float64
// RMSNorm oracle it moved one normalized element of the tests by 2 bf16 ulps,
// so the sum keeps this order.)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The RMSNorm sum of squares of one row (h % 8 == 0), s = x (+ res) rounded
// to DT, in one fixed association that every kernel uses: lane l's 8-element
// chunks k (elements 8l + 512k .. 8l + 512k + 7) fall into kSumClasses = 8
// classes k mod 8; P_w adds the squares of class w's chunks in ascending k,
// each chunk's eight in order (one float32 chain); the lane's total is
// ((P_0 + P_1) + ...) + P_7, and the xor butterfly adds the lanes.  One wave
// can form all eight partials (row_sumsq), or the waves of a workgroup a few
// each, exchanged through LDS (row_sumsq_part, row_sumsq_total): the same
// bits either way.
// Loads use indices clamped into the row, so they stay unconditional (the
// residual's from x when there is none): a load under a branch made the
// compiler wait for every load at the join.
constexpr int kSumClasses = 8;

// acc + the eight squares of one chunk, in order.
template <int DT>
__device__ __forceinline__ float add_sq8(const Raw8<DT>& xv, const Raw8<DT>& rv, bool has_res, float acc) {
  float f[8];
  unpack8<DT>(xv, f);
  if (has_res) {
    float r[8];
    unpack8<DT>(rv, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = round_to_dt<DT>(f[e] + r[e]);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = acc + f[e] * f[e];
  return acc;
}

// The partials of lane l for the NC classes w, w + cs, ..., w + (NC - 1) cs
// of one row: acc[j] is class w + j cs.  Each step requests kQ chunks of
// every class.
template <int DT, int NC, int kQ>
__device__ __forceinline__ void row_sumsq_part(const void* __restrict__ x, const void* __restrict__ res,
                                               int64_t row_off, int h, int lane, int w, int cs, float (&acc)[NC]) {
  const void* rs = res != nullptr ? res : x;
#pragma unroll
  for (int j = 0; j < NC; ++j) acc[j] = 0.0f;
  // class w is the first: once its chunk is past the row, so are the others'
  for (int k0 = w; lane * 8 + 512 * k0 < h; k0 += kQ * kSumClasses) {
    Raw8<DT> xv[NC][kQ], rv[NC][kQ];
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        const int c8 = min(lane * 8 + 512 * (k0 + j * cs + q * kSumClasses), h - 8);
        xv[j][q] = load8_raw<DT>(x, row_off + c8);
        rv[j][q] = load8_raw<DT>(rs, row_off + c8);
      }
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int q = 0; q < kQ; ++q)
        if (lane * 8 + 512 * (k0 + j * cs + q * kSumClasses) < h)
          acc[j] = add_sq8<DT>(xv[j][q], rv[j][q], res != nullptr, acc[j]);
  }
}

// The row's total from the lane's eight partials (P[w] = class w).
__device__ __forceinline__ float row_sumsq_total(const float (&p)[kSumClasses]) {
  float t = p[0];
#pragma unroll
  for (int w = 1; w < kSumClasses; ++w) t = t + p[w];
  return wave_sum(t);
}

// All eight partials by one wave: the chunks of kB consecutive classes
// requested together, each added to its own class's chain.
template <int DT, int kB = kSumClasses>
__device__ __forceinline__ float row_sumsq(const void* __restrict__ x, const void* __restrict__ res, int64_t row_off,
                                           int h, int lane) {
  static_assert(kSumClasses % kB == 0, "batches of whole class sets");
  const void* rs = res != nullptr ? res : x;
  float p[kSumClasses];
#pragma unroll
  for (int w = 0; w < kSumClasses; ++w) p[w] = 0.0f;
  for (int k0 = 0; lane * 8 + 512 * k0 < h; k0 += kSumClasses) {
#pragma unroll
    for (int w0 = 0; w0 < kSumClasses; w0 += kB) {
      Raw8<DT> xv[kB], rv[kB];
#pragma unroll
      for (int q = 0; q < kB; ++q) {
        const int c8 = min(lane * 8 + 512 * (k0 + w0 + q), h - 8);
        xv[q] = load8_raw<DT>(x, row_off + c8);
        rv[q] = load8_raw<DT>(rs, row_off + c8);
      }
#pragma unroll
      for (int q = 0; q < kB; ++q)
        if (lane * 8 + 512 * (k0 + w0 + q) < h) p[w0 + q] = add_sq8<DT>(xv[q], rv[q], res != nullptr, p[w0 + q]);
    }
  }
  return row_sumsq_total(p);
}

// rsqrt(mean + eps) as two correctly rounded float32 operations.
__device__ __forceinline__ float rms_inv(float sumsq, int h, float eps) {
  return 1.0f / __builtin_sqrtf(sumsq / static_cast<float>(h) + eps);
}

// The normalized value of one element (s already rounded to DT).
template <int DT>
__device__ __forceinline__ float rms_apply(float s, float r, float w) {
  return round_to_dt<DT>(w * round_to_dt<DT>(s * r));
}

// A gated MLP's activation in the module's rounding: round(round(silu(g)) * u),
// silu(g) = g / (1 + exp(-g)) in float32.
template <int DT>
__device__ __forceinline__ float swiglu(float g, float u) {
  const float a = round_to_dt<DT>(g / (1.0f + expf(-g)));
  return round_to_dt<DT>(a * u);
}

// One wave rotates 128-channel group g of the first min(M, MR) rows: channel
// scale, the krot register-chain layers, then the rotated values go to xr
// (fp16 when MAT16, else fp32; row stride h) and each row's absmax over the
// group to gmax[m * (h / 128) + g].  With PQ_RQ_INPUT_FP16 the scaled input
// is first rounded through fp16.  Rows past M repeat row M-1 and store
// nothing.
//
// With NORM the group's rows first go through the prologue of `mode`
// (PQ_PRO_*): RMSNORM computes each row's RMSNorm factor over the whole row
// (every wave of the launch gets the same bits; rinv >= 0 passes it in,
// summed by the caller in the same association) and normalizes, ADD adds the
// residual, SWIGLU forms silu(x) * up; the wave rotates the result and, when
// h_out / s_out are set, writes it (h) or the residual sum s for the group's
// channels.
template <int DT, int KP, bool MAT16, int MR, bool NORM = false>
__device__ __forceinline__ void rotate_group_rows(const void* __restrict__ x, const uint32_t* __restrict__ rot_idx,
                                                  const float* __restrict__ rot_cs, const float* __restrict__ scales,
                                                  void* __restrict__ xr, float* __restrict__ gmax, int M, int h,
                                                  int krot, unsigned flags, int g, int lane,
                                                  const void* __restrict__ nres = nullptr,
                                                  const void* __restrict__ nw = nullptr,
                                                  void* __restrict__ h_out = nullptr,
                                                  void* __restrict__ s_out = nullptr, float eps = 0.0f,
                                                  int mode = PQ_PRO_RMSNORM, float rinv = -1.0f) {
  const int G = h >> 7;
  const bool in16 = (flags & PQ_RQ_INPUT_FP16) != 0;
  const bool has_scales = scales != nullptr;
  // unconditional scale loads (from rot_cs when there are no scales): a
  // branch around them would make the compiler wait for them early
  const float* sp = has_scales ? scales : rot_cs;
  const int smask = has_scales ? 0x7fffffff : 0;

  RotLane<KP> p;
  load_rot_lane<KP>(rot_idx, rot_cs, g, lane, p);
  uint32_t xa[MR], xb[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int mm = m < M ? m : M - 1;
    xa[m] = pq_load_raw<DT>(x, static_cast<int64_t>(mm) * h + g * 128 + lane);
    xb[m] = pq_load_raw<DT>(x, static_cast<int64_t>(mm) * h + g * 128 + 64 + lane);
  }
  const float s0r = sp[(g * 128 + lane) & smask];
  const float s1r = sp[(g * 128 + 64 + lane) & smask];
  const float s0 = has_scales ? s0r : 1.0f, s1 = has_scales ? s1r : 1.0f;
  pin_rot_lane<KP>(p);
  const bool sw = rot_init_swapped(p);
  float a[MR], b[MR];
  float xlo[MR], xhi[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    xlo[m] = pq_raw_to_f32<DT>(xa[m]);
    xhi[m] = pq_raw_to_f32<DT>(xb[m]);
  }
  if constexpr (NORM) {
    // the second operand of the group (residual or up projection), loaded
    // unconditionally (from x when there is none) so that no load waits
    // behind a branch
    const void* np = nres != nullptr ? nres : x;
    float nlo[MR], nhi[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const int mm = m < M ? m : M - 1;
      const int64_t ro = static_cast<int64_t>(mm) * h;
      nlo[m] = pq_load_as_f32<DT>(np, ro + g * 128 + lane);
      nhi[m] = pq_load_as_f32<DT>(np, ro + g * 128 + 64 + lane);
    }
    if (mode == PQ_PRO_SWIGLU) {
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const int mm = m < M ? m : M - 1;
        const int64_t ro = static_cast<int64_t>(mm) * h;
        xlo[m] = swiglu<DT>(xlo[m], nlo[m]);
        xhi[m] = swiglu<DT>(xhi[m], nhi[m]);
        if (m < M && h_out != nullptr) {
          pq_store_from_f32<DT>(h_out, ro + g * 128 + lane, xlo[m]);
          pq_store_from_f32<DT>(h_out, ro + g * 128 + 64 + lane, xhi[m]);
        }
      }
    } else {
      const bool norm = mode == PQ_PRO_RMSNORM;
      const void* nwp = norm ? nw : x;   // ADD has no weight: a harmless stand-in, unused
      const float w0 = pq_load_as_f32<DT>(nwp, g * 128 + lane), w1 = pq_load_as_f32<DT>(nwp, g * 128 + 64 + lane);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const int mm = m < M ? m : M - 1;
        const int64_t ro = static_cast<int64_t>(mm) * h;
        const float r = !norm         ? 1.0f
                        : rinv >= 0.0f ? rinv
                                       : rms_inv(row_sumsq<DT, MR <= 4 ? 8 : 4>(x, nres, ro, h, lane), h, eps);
        if (nres != nullptr) {
          xlo[m] = round_to_dt<DT>(xlo[m] + nlo[m]);
          xhi[m] = round_to_dt<DT>(xhi[m] + nhi[m]);
        }
        if (m < M && s_out != nullptr) {
          pq_store_from_f32<DT>(s_out, ro + g * 128 + lane, xlo[m]);
          pq_store_from_f32<DT>(s_out, ro + g * 128 + 64 + lane, xhi[m]);
        }
        if (norm) {
          xlo[m] = rms_apply<DT>(xlo[m], r, w0);
          xhi[m] = rms_apply<DT>(xhi[m], r, w1);
          if (m < M && h_out != nullptr) {
            pq_store_from_f32<DT>(h_out, ro + g * 128 + lane, xlo[m]);
            pq_store_from_f32<DT>(h_out, ro + g * 128 + 64 + lane, xhi[m]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float lo = xlo[m], hi = xhi[m];
    lo = (in16 ? pq_round_f16(lo) : lo) * s0;
    hi = (in16 ? pq_round_f16(hi) : hi) * s1;
    a[m] = sw ? hi : lo;
    b[m] = sw ? lo : hi;
  }
  rot_layers<KP, MR>(p, krot, a, b);
  const int fa = g * 128 + rot_final_a(p), fb = g * 128 + rot_final_b(p);
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const float va = a[m], vb = b[m];
    if (m < M) {
      if constexpr (MAT16) {
        static_cast<uint16_t*>(xr)[static_cast<int64_t>(m) * h + fa] = pq_f32_to_f16(va);
        static_cast<uint16_t*>(xr)[static_cast<int64_t>(m) * h + fb] = pq_f32_to_f16(vb);
      } else {
        static_cast<float*>(xr)[static_cast<int64_t>(m) * h + fa] = va;
        static_cast<float*>(xr)[static_cast<int64_t>(m) * h + fb] = vb;
      }
    }
    // the group's absmax of the stored rows: rounding to fp16 is monotonic,
    // so it is the float32 absmax rounded once
    float mx = pq_wave_max_nonneg(fmaxf(fabsf(va), fabsf(vb)));
    if constexpr (MAT16) mx = pq_round_f16(mx);
    if (m < M && lane == 0) gmax[static_cast<int64_t>(m) * G + g] = mx;
  }
}


// ---------------------------------------------------------------------------
// LDS staging shared by the GEMM kernels
// ---------------------------------------------------------------------------
// Barrier for LDS hand-offs only: the wave's LDS operations complete, then
// s_barrier.  Unlike __syncthreads() it does not wait for the wave's global
// stores (vmcnt), which may stay in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16-byte chunk swizzle of a 128-byte LDS row (row-dependent XOR).
__device__ __forceinline__ int pf_swz(int line) { return (line >> 1) & 7; }

// Global -> LDS copies of 16 (4) bytes per lane: lane l's bytes land at LDS
// address lds + 16*l (4*l).  Written as inline asm on purpose: the compiler
// would otherwise treat every later LDS read as possibly aliasing the copy
// and wait for all outstanding loads (vmcnt(0)) before it, which serializes
// the stage ring.  The kernels wait for these loads explicitly (wait_vmcnt).
// M0 is used only here.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}
__device__ __forceinline__ void lds_copy16(const void* gsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(gsrc) : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void* gsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(gsrc) : "memory", "m0");
}

// s_waitcnt with vmcnt(n), any lgkmcnt/expcnt (gfx9 immediate encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ---------------------------------------------------------------------------
// OCP MX (v1.0) MXFP4: blocks of 32 elements share an E8M0 scale 2^e with
// e = floor(log2(amax)) - 2 (2 = the largest exponent of E2M1), clamped to
// [-127, 127]; each element v / 2^e goes to the E2M1 grid {0, 0.5, 1, 1.5,
// 2, 3, 4, 6} by round-to-nearest-even, saturating at 6, sign kept (NaN
// elements: code 0; their block's scale byte is 0xFF).
// ---------------------------------------------------------------------------
// Shared exponent of a block from its absmax (0, subnormal: -127; Inf: 126).
__device__ __forceinline__ int mx_shared_exp(float amax) {
  const int ef = static_cast<int>((__float_as_uint(amax) >> 23) & 0xffu);   // biased exponent
  const int e = ef - 127 - 2;                                               // ef = 0 gives e < -127
  return e < -127 ? -127 : e;
}
// 2^-e as a float (e in [-127, 126]).
__device__ __forceinline__ float mx_inv_scale(int e) { return __uint_as_float(static_cast<uint32_t>(127 - e) << 23); }
// E2M1 code of y = v / 2^e: magnitude index = number of grid midpoints below
// |y|, a midpoint counting when passed (>) or, for the ties that round up to
// an even code (0.75, 1.75, 3.5), when reached (>=).
__device__ __forceinline__ uint32_t mx_e2m1(float y) {
  const float a = fabsf(y);
  const uint32_t c = static_cast<uint32_t>(a > 0.25f) + static_cast<uint32_t>(a >= 0.75f) +
                     static_cast<uint32_t>(a > 1.25f) + static_cast<uint32_t>(a >= 1.75f) +
                     static_cast<uint32_t>(a > 2.5f) + static_cast<uint32_t>(a >= 3.5f) +
                     static_cast<uint32_t>(a > 5.0f);
  const uint32_t sign = (__float_as_uint(y) >> 28) & 8u;
  return c | (y == y ? sign : 0u);   // a NaN element is code 0 (its block's scale is NaN)
}

}  // namespace pqd
